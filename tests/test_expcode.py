"""Exponent-coded blocks on the CPU: the oracle pinned by known answers, and the library's encoder
(host code, no GPU) byte for byte against the oracle.

Known answers are written out by hand from the format: a three-word block with an odd tail byte, a
block with two escaped exponents, and the table's tie rule. Round trips cover bf16 weights, every
class of bf16 value and arbitrary bytes; the decoder refuses escape lists that do not match the codes.
"""

from __future__ import annotations

import ctypes
import struct

import numpy as np
import pytest
import torch

from oracle import expcode as X


def _bf16(n_words: int, seed: int, std: float = 0.02) -> np.ndarray:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n_words, generator=g) * std).to(torch.bfloat16).view(torch.uint8).numpy().copy()


def _words(*ws: int) -> np.ndarray:
    return np.array(ws, dtype="<u2").view(np.uint8)


def test_known_answer_three_words_and_a_tail():
    # 1.0 (exp 127), -2.0 (exp 128), 1.0078125 (exp 127, mantissa 1), then an odd byte 0xAB
    raw = np.concatenate([_words(0x3F80, 0xC000, 0x3F81), np.array([0xAB], np.uint8)])
    enc = X.encode(raw)
    assert enc.size == 1808 == X.encoded_size(raw) == X.sections(1, 0)[4]
    head = struct.pack("<4sIQQQQ", b"FTXE", 1, 7, 3, 1, 0) + bytes([127, 128] + [0] * 14) + bytes([0xAB]) + bytes(7)
    assert bytes(enc[:64]) == head and not enc[64:256].any()
    assert list(enc[256:259]) == [0x00, 0x80, 0x01] and not enc[259:1280].any()  # sign << 7 | mantissa
    assert list(enc[1280:1282]) == [0x10, 0x00] and not enc[1282:1792].any()  # codes 0, 1 | 0 (low nibble first)
    assert not enc[1792:1808].any()  # S = [0, 0], padded to 16 bytes
    assert X.decode(enc) == raw.tobytes()


def test_known_answer_escapes():
    # exponents 1..17, exponent e written 18 - e times: 1..15 fill the table, 16 and 17 escape
    ws = [e << 7 | (e & 0x7F) for e in range(1, 18) for _ in range(18 - e)]
    raw = _words(*ws)
    enc = X.encode(raw)
    h = X.parse_header(enc)
    assert h["table"] == list(range(1, 16)) + [0] and h["escapes"] == 3 and h["groups"] == 1
    pos16 = ws.index(16 << 7 | 16)
    want_x = [(pos16 << 8) | 16, ((pos16 + 1) << 8) | 16, ((pos16 + 2) << 8) | 17]
    assert list(enc[h["off_s"]: h["off_s"] + 8].view("<u4")) == [0, 3]
    assert list(enc[h["off_x"]: h["off_x"] + 12].view("<u4")) == want_x
    nib = np.empty(2 * 512, np.uint8)
    b = enc[h["off_b"]: h["off_b"] + 512]
    nib[0::2], nib[1::2] = b & 15, b >> 4
    assert list(nib[pos16: pos16 + 3]) == [15, 15, 15] and nib[0] == 0 and nib[pos16 - 1] == 14
    assert X.decode(enc) == raw.tobytes()


def test_table_ties_go_to_the_smaller_exponent():
    raw = _words(*([5 << 7] * 3 + [9 << 7] * 3 + [7 << 7] * 4))
    assert X.parse_header(X.encode(raw))["table"][:3] == [7, 5, 9]


@pytest.mark.parametrize("n", [0, 1, 2, 3, 2046, 2048, 2049, 6145, 1 << 16])
def test_round_trips(n):
    rng = np.random.default_rng(n)
    for raw in (_bf16(n // 2 + 1, n)[:n], rng.integers(0, 256, n, dtype=np.uint8),
                (rng.integers(0, 4, n, dtype=np.uint8) * 0x7F)):
        enc = X.encode(raw)
        assert enc.size == X.encoded_size(raw)
        assert X.decode(enc) == raw.tobytes()


def test_every_bf16_class_round_trips():
    words = np.arange(1 << 16, dtype=np.uint32)  # every bit pattern: zeros, subnormals, normals, inf, NaN
    raw = words.astype("<u2").view(np.uint8)
    assert X.decode(X.encode(raw)) == raw.tobytes()


def test_bf16_weights_encode_to_three_quarters():
    raw = _bf16(1 << 20, 7)
    enc = X.encode(raw)
    h = X.parse_header(enc)
    assert h["escapes"] < 1e-3 * h["n_words"]
    assert 0.75 < enc.size / raw.size < 0.753


def test_decoder_refuses_inconsistent_escapes():
    raw = _words(*([1 << 7] * 20 + list(range(2 << 7, 20 << 7, 1 << 7))))
    enc = X.encode(raw)
    h = X.parse_header(enc)
    assert h["escapes"] > 0
    bad = enc.copy()
    bad[h["off_x"] + 1] ^= 0x01  # an escape moved to another word
    with pytest.raises(ValueError):
        X.decode(bad)
    bad = enc.copy()
    bad[h["off_s"] + 4] += 1  # S[G] no longer E
    with pytest.raises(ValueError):
        X.decode(bad)
    with pytest.raises(ValueError):
        X.decode(enc[: h["total"] - 4])


# ---- the library's encoder (host code: runs without a GPU) ----------------------------------------


def _lib_encode(raw: np.ndarray) -> np.ndarray:
    from flextensor_amd import _native as nat

    raw = np.ascontiguousarray(raw)
    size = ctypes.c_size_t(0)
    ptr = raw.ctypes.data if raw.size else None
    nat.call("ftx_expcode_encode", ptr, raw.size, None, 0, ctypes.byref(size))
    out = np.full(size.value + 8, 0xEE, dtype=np.uint8)
    got = ctypes.c_size_t(0)
    nat.call("ftx_expcode_encode", ptr, raw.size, out.ctypes.data, out.size, ctypes.byref(got))
    assert got.value == size.value
    assert np.all(out[size.value:] == 0xEE)  # nothing written past the encoded size
    return out[: size.value]


@pytest.mark.parametrize("n", [0, 1, 2, 5, 2047, 2048, 2050, 10001, (1 << 21) + 3])
def test_library_encoder_matches_the_oracle(n):
    rng = np.random.default_rng(n + 1)
    for raw in (_bf16(n // 2 + 1, n)[:n], rng.integers(0, 256, n, dtype=np.uint8)):
        assert np.array_equal(_lib_encode(raw), X.encode(raw))


def test_library_encoder_on_a_multithreaded_block():
    raw = _bf16(3 << 20, 11)  # 6 MiB: large enough for the encoder's host threads
    raw[1000:1064] = np.random.default_rng(3).integers(0, 256, 64, dtype=np.uint8)  # a few escapes
    assert np.array_equal(_lib_encode(raw), X.encode(raw))


def test_library_encoder_refusals_and_header_reader():
    from flextensor_amd import _native as nat

    raw = _bf16(4096, 1)
    size = ctypes.c_size_t(0)
    nat.call("ftx_expcode_encode", raw.ctypes.data, raw.size, None, 0, ctypes.byref(size))
    small = np.zeros(size.value - 1, np.uint8)
    with pytest.raises(nat.FtxError) as err:
        nat.call("ftx_expcode_encode", raw.ctypes.data, raw.size, small.ctypes.data, small.size, ctypes.byref(size))
    assert err.value.code == nat.FTX_ERR_INVALID
    with pytest.raises(nat.FtxError):  # out overlapping raw
        nat.call("ftx_expcode_encode", raw.ctypes.data, raw.size, raw.ctypes.data + 8, raw.size, ctypes.byref(size))
    with pytest.raises(nat.FtxError):
        nat.call("ftx_expcode_encode", raw.ctypes.data, raw.size, None, 0, None)
    enc = _lib_encode(raw)
    got = ctypes.c_size_t(0)
    nat.call("ftx_expcode_raw_bytes", enc.ctypes.data, enc.size, ctypes.byref(got))
    assert got.value == raw.size
    bad = enc.copy()
    bad[4] = 2  # version
    with pytest.raises(nat.FtxError):
        nat.call("ftx_expcode_raw_bytes", bad.ctypes.data, bad.size, ctypes.byref(got))
    with pytest.raises(nat.FtxError):  # truncated
        nat.call("ftx_expcode_raw_bytes", enc.ctypes.data, enc.size - 1, ctypes.byref(got))


def test_config_needs_the_allocation_block_controller():
    from flextensor_amd.config import OffloadConfig

    assert OffloadConfig(encode_streamed_blocks=True).encode_streamed_blocks
    with pytest.raises(ValueError, match="encode_streamed_blocks"):
        OffloadConfig(encode_streamed_blocks=True, transfer_mode="raw_block_transfer")


def test_encoding_follows_its_own_pass_rule():
    """Encoded transfers stay on while the profiled compute is under 0.9 of the raw transfer time, also
    where the ring already keeps SDMA (compute at 0.4 of the transfers or more); at 0.9 and above they are
    off. No link measurement, or none that profiled the pass, keeps them on."""
    import types

    from flextensor_amd.link_model import ENCODE_COMPUTE_SHARE, encoding_pays, is_link_bound
    from flextensor_amd.manager import OffloadManager

    assert ENCODE_COMPUTE_SHARE == 0.9
    assert encoding_pays(35.0, 113.0) and is_link_bound(35.0, 113.0)
    assert encoding_pays(68.0, 84.7) and not is_link_bound(68.0, 84.7)  # between the two rules
    assert not encoding_pays(90.0, 100.0) and not encoding_pays(1.0, 0.0)
    mgr = OffloadManager(name="encode-rule")
    for link, off in ((None, False), (types.SimpleNamespace(pass_compute_ms=None, pass_transfer_ms=None), False),
                      (types.SimpleNamespace(pass_compute_ms=68.0, pass_transfer_ms=84.7), False),
                      (types.SimpleNamespace(pass_compute_ms=95.0, pass_transfer_ms=100.0), True)):
        mgr.link = link
        assert mgr._measured_compute_bound() == off


# ---- the dense format (version 2) of units kept encoded in HBM ---------------------------------------

from oracle import expcode_dense as D  # noqa: E402


def test_dense_known_answer_with_both_escape_levels():
    # exponents 1..24, exponent e written 25 - e times: 1..7 are primary, 8..22 secondary, 23 and 24 listed
    ws = [e << 7 | (e & 0x7F) for e in range(1, 25) for _ in range(25 - e)]
    raw = _words(*ws)
    enc = D.encode(raw)
    h = D.parse_header(enc)
    assert h["t1"] == list(range(1, 8)) + [0] and h["t2"] == list(range(8, 23)) + [0]
    n8 = sum(25 - e for e in range(1, 8))  # words before the first primary escape
    assert h["e1"] == len(ws) - n8 and h["e2"] == 2 + 1 and h["groups"] == 1
    assert enc.size == D.sections(1, h["e1"], 3)["total"]
    codes = np.zeros(1024, np.uint8)
    planes = enc[h["off_p"]: h["off_p"] + 384].reshape(3, 64, 2)  # [plane, lane l, run h]: words 512 h + 8 l + b
    for k in range(3):
        codes |= (np.unpackbits(planes[k].T.reshape(-1), bitorder="little") << k).astype(np.uint8)
    assert list(codes[:3]) == [0] * 3 and codes[n8 - 1] == 6 and codes[n8] == 7 and not codes[len(ws):].any()
    y = enc[h["off_y"]: h["off_y"] + 2]
    assert y[0] == 0x00 and list(enc[h["off_s1"]: h["off_s1"] + 8].view("<u4")) == [0, h["e1"]]
    p23 = ws.index(23 << 7 | 23)
    assert list(enc[h["off_x"]: h["off_x"] + 12].view("<u4")) == [p23 << 8 | 23, (p23 + 1) << 8 | 23, (p23 + 2) << 8 | 24]
    assert D.decode(enc) == raw.tobytes()


@pytest.mark.parametrize("n", [0, 1, 2, 3, 2046, 2048, 2049, 6145, 1 << 16])
def test_dense_round_trips(n):
    rng = np.random.default_rng(n + 5)
    for raw in (_bf16(n // 2 + 1, n)[:n], rng.integers(0, 256, n, dtype=np.uint8)):
        enc = D.encode(raw)
        assert enc.size == D.encoded_size(raw)
        assert D.decode(enc) == raw.tobytes()


def test_dense_every_bf16_pattern_and_density():
    words = np.arange(1 << 16, dtype=np.uint32).astype("<u2").view(np.uint8)
    assert D.decode(D.encode(words)) == words.tobytes()
    raw = _bf16(1 << 20, 7)
    assert 0.69 < D.encoded_size(raw) / raw.size < 0.70 < 0.75 < X.encoded_size(raw) / raw.size


def test_dense_decoder_refuses_inconsistent_blocks():
    raw = _words(*[e << 7 for e in range(1, 30) for _ in range(31 - e)])
    enc = D.encode(raw)
    h = D.parse_header(enc)
    bad = enc.copy()
    bad[h["off_s1"] + 4] += 1  # S1[G] no longer E1
    with pytest.raises(ValueError):
        D.decode(bad)
    bad = enc.copy()
    bad[h["off_x"] + 1] ^= 0x01  # a listed word moved
    with pytest.raises(ValueError):
        D.decode(bad)
    bad = enc.copy()
    for k in range(3):
        bad[h["off_p"] + 128 * k] |= 0x01  # word 0's primary code made an escape: one more than S1 counts
    with pytest.raises(ValueError):
        D.decode(bad)
    with pytest.raises(ValueError):
        D.decode(enc[: h["total"] - 1])


def _lib_encode_dense(raw: np.ndarray) -> np.ndarray:
    from flextensor_amd import _native as nat

    raw = np.ascontiguousarray(raw)
    size = ctypes.c_size_t(0)
    ptr = raw.ctypes.data if raw.size else None
    nat.call("ftx_expcode_encode_dense", ptr, raw.size, None, 0, ctypes.byref(size))
    out = np.full(size.value + 8, 0xEE, dtype=np.uint8)
    got = ctypes.c_size_t(0)
    nat.call("ftx_expcode_encode_dense", ptr, raw.size, out.ctypes.data, out.size, ctypes.byref(got))
    assert got.value == size.value and np.all(out[size.value:] == 0xEE)
    return out[: size.value]


@pytest.mark.parametrize("n", [0, 1, 2, 5, 2047, 2048, 2050, 10001, (1 << 21) + 3])
def test_library_dense_encoder_matches_the_oracle(n):
    rng = np.random.default_rng(n + 2)
    for raw in (_bf16(n // 2 + 1, n)[:n], rng.integers(0, 256, n, dtype=np.uint8)):
        assert np.array_equal(_lib_encode_dense(raw), D.encode(raw))


def test_library_dense_encoder_on_threaded_blocks_with_shared_nibble_bytes():
    """Blocks large enough for the encoder's threads: with escapes in every group, the nibble bytes at the
    edges of one thread's range hold a nibble of the next (an odd count of escapes before them)."""
    for seed in range(3):
        raw = _bf16(3 << 20, 20 + seed, std=0.02 * (1 + seed))
        rng = np.random.default_rng(seed)
        idx = rng.integers(0, raw.size // 2, 5000) * 2 + 1  # high bytes: exponents off the tables
        raw[idx] = rng.integers(0, 256, idx.size, dtype=np.uint8)
        assert np.array_equal(_lib_encode_dense(raw), D.encode(raw))
