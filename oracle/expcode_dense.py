"""Dense exponent-coded blocks (``FTXE`` v2): the lossless format of units kept encoded in HBM, in numpy.

TEST INFRASTRUCTURE ONLY (see the package docstring). No reference counterpart: the reference keeps the
units it does not stream as raw tensors on the GPU (tensor_processors.py:685-742). The format is this
build's own, and this module is its definition; ``flextensor_amd`` encodes with a host routine in the C
library and decodes from device memory with a GPU kernel, and both are checked against this module.

Like v1 (``oracle.expcode``), a raw block of N bytes is read as W = N // 2 little-endian 16-bit words
(bf16 bit patterns: sign bit 15, exponent bits 14..7, mantissa bits 6..0), an odd last byte kept
verbatim, in G = ceil(W / 1024) groups of 1024 words. The exponents are ranked by frequency, most
frequent first, ties to the smaller exponent: table T1 holds the first 7, table T2 the next 15. A word
whose exponent is T1[c] has primary code c < 7; any other word has primary code 7 (a primary escape)
and a secondary code: c2 < 15 where its exponent is T2[c2], else 15 (a secondary escape). The encoded
block is:

* header, 80 bytes, then zeros up to byte 256: ``b"FTXE"``, u32 version 2, u64 N, u64 W, u64 G,
  u64 E1 (primary escapes), u64 E2 (secondary escapes), T1 in 8 bytes, T2 in 16 bytes (unused entries
  zero), u8 tail byte (the odd last byte, else 0), 7 zero bytes;
* plane A at 256, G * 1024 bytes: byte w = sign(w) << 7 | mantissa(w); zero past W;
* plane P at 256 + 1024 G, 384 bytes per group: for group g, three bit planes of 128 bytes; bit k of
  the primary code of word 1024 g + 512 h + 8 l + b (h < 2, l < 64, b < 8) is bit b of byte 2 l + h of
  plane k, so the 16 words a decoder lane takes (two runs of 8) have their code bits in one 16-bit
  value per plane; zero past W;
* S1 at 256 + 1408 G: G + 1 u32, primary escapes in groups before g (S1[G] = E1);
* S2 at S1 + align16(4 (G + 1)): G + 1 u32, secondary escapes in groups before g (S2[G] = E2);
* Y at S2 + align16(4 (G + 1)): one nibble per primary escape in word order, the r-th in the low
  nibble of byte r // 2 for even r and the high nibble for odd r: its secondary code;
* X at Y + align16(ceil(E1 / 2)): E2 u32, one per secondary escape in word order,
  (w % 1024) << 8 | exponent.

The encoded size is 256 + 1408 G + 2 align16(4 (G + 1)) + align16(ceil(E1 / 2)) + 4 E2 bytes: about
0.695 of the raw size for bf16 weights drawn from one distribution (7 exponents cover 98% of their
words, 22 all but one in a million), against 0.752 for v1. A decoder needs each primary escape's rank
in word order to find its nibble: the prefix count S1 of its group plus the escapes before it inside
the group.
"""

from __future__ import annotations

import struct

import numpy as np

MAGIC = b"FTXE"
VERSION = 2
HEADER_BYTES = 256
GROUP_WORDS = 1024
PLANE_BYTES = 384  # per group: three bit planes of 128 bytes
PRIMARY = 7
SECONDARY = 15
_HEAD = struct.Struct("<4sIQQQQQ8s16sB7x")  # 80 bytes


def _align16(x: int) -> int:
    return (x + 15) // 16 * 16


def sections(n_groups: int, e1: int, e2: int) -> dict[str, int]:
    """Byte offsets of every section and the total size."""
    off_a = HEADER_BYTES
    off_p = off_a + GROUP_WORDS * n_groups
    off_s1 = off_p + PLANE_BYTES * n_groups
    off_s2 = off_s1 + _align16(4 * (n_groups + 1))
    off_y = off_s2 + _align16(4 * (n_groups + 1))
    off_x = off_y + _align16((e1 + 1) // 2)
    return dict(off_a=off_a, off_p=off_p, off_s1=off_s1, off_s2=off_s2, off_y=off_y, off_x=off_x,
                total=off_x + 4 * e2)


def tables_of(exponents: np.ndarray) -> tuple[list[int], list[int]]:
    """T1 (the 7 most frequent exponents) and T2 (the next 15), ties to the smaller exponent."""
    hist = np.bincount(exponents.astype(np.int64), minlength=256)
    ranked = sorted((e for e in range(256) if hist[e] > 0), key=lambda e: (-int(hist[e]), e))
    return ranked[:PRIMARY], ranked[PRIMARY: PRIMARY + SECONDARY]


def _bytes_of(raw) -> np.ndarray:
    return np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw.view(np.uint8)


def _codes(exp: np.ndarray, t1: list[int], t2: list[int]) -> tuple[np.ndarray, np.ndarray]:
    c1_of = np.full(256, PRIMARY, dtype=np.uint8)
    for c, e in enumerate(t1):
        c1_of[e] = c
    c2_of = np.full(256, SECONDARY, dtype=np.uint8)
    for c, e in enumerate(t2):
        c2_of[e] = c
    return c1_of[exp], c2_of[exp]


def encoded_size(raw) -> int:
    b = _bytes_of(raw)
    w = b[: b.size // 2 * 2].view("<u2")
    exp = ((w >> 7) & 0xFF).astype(np.int64)
    t1, t2 = tables_of(exp)
    c1, c2 = _codes(exp, t1, t2)
    esc1 = c1 == PRIMARY
    e1 = int(np.count_nonzero(esc1))
    e2 = int(np.count_nonzero(esc1 & (c2 == SECONDARY)))
    g = (w.size + GROUP_WORDS - 1) // GROUP_WORDS
    return sections(g, e1, e2)["total"]


def encode(raw) -> np.ndarray:
    """Encode ``raw`` (bytes or a uint8 array); returns the encoded block as a uint8 array."""
    b = _bytes_of(raw)
    n = int(b.size)
    n_words = n // 2
    words = b[: 2 * n_words].view("<u2").astype(np.uint32)
    exp = ((words >> 7) & 0xFF).astype(np.int64)
    t1, t2 = tables_of(exp)
    c1, c2 = _codes(exp, t1, t2)
    g = (n_words + GROUP_WORDS - 1) // GROUP_WORDS
    esc1 = np.nonzero(c1 == PRIMARY)[0]
    esc2 = esc1[c2[esc1] == SECONDARY]
    sec = sections(g, int(esc1.size), int(esc2.size))
    out = np.zeros(sec["total"], dtype=np.uint8)
    tail = int(b[-1]) if n % 2 else 0
    head = _HEAD.pack(MAGIC, VERSION, n, n_words, g, int(esc1.size), int(esc2.size),
                      bytes(t1) + bytes(8 - len(t1)), bytes(t2) + bytes(16 - len(t2)), tail)
    out[: len(head)] = np.frombuffer(head, dtype=np.uint8)
    out[sec["off_a"]: sec["off_a"] + n_words] = (((words >> 8) & 0x80) | (words & 0x7F)).astype(np.uint8)
    codes = np.zeros(g * GROUP_WORDS, dtype=np.uint8)
    codes[:n_words] = c1
    bits = codes.reshape(g, GROUP_WORDS // 8, 8)  # [group, word // 8 = 64 h + l, bit]
    weights = (1 << np.arange(8)).astype(np.uint16)
    planes = np.stack([(((bits >> k) & 1).astype(np.uint16) * weights).sum(-1).astype(np.uint8) for k in range(3)],
                      axis=1)  # [group, plane, 64 h + l]
    planes = planes.reshape(g, 3, 2, 64).transpose(0, 1, 3, 2)  # [group, plane, l, h]: byte 2 l + h
    out[sec["off_p"]: sec["off_p"] + PLANE_BYTES * g] = planes.reshape(-1)
    for key, esc in (("off_s1", esc1), ("off_s2", esc2)):
        counts = np.bincount(esc // GROUP_WORDS, minlength=g) if g else np.zeros(0, dtype=np.int64)
        s = np.zeros(g + 1, dtype="<u4")
        s[1:] = np.cumsum(counts)
        out[sec[key]: sec[key] + 4 * (g + 1)] = s.view(np.uint8)
    nib = np.zeros(2 * ((esc1.size + 1) // 2), dtype=np.uint8)
    nib[: esc1.size] = c2[esc1]
    out[sec["off_y"]: sec["off_y"] + nib.size // 2] = nib[0::2] | (nib[1::2] << 4)
    x = (((esc2 % GROUP_WORDS) << 8) | exp[esc2]).astype("<u4")
    out[sec["off_x"]: sec["off_x"] + 4 * esc2.size] = x.view(np.uint8)
    return out


def parse_header(buf: np.ndarray) -> dict:
    magic, version, n, n_words, g, e1, e2, t1, t2, tail = _HEAD.unpack(bytes(buf[: _HEAD.size]))
    if magic != MAGIC or version != VERSION:
        raise ValueError("not a dense exponent-coded block")
    if n_words != n // 2 or g != (n_words + GROUP_WORDS - 1) // GROUP_WORDS or e2 > e1:
        raise ValueError("inconsistent header")
    sec = sections(g, e1, e2)
    if sec["total"] > buf.size:
        raise ValueError("truncated block")
    return dict(n=n, n_words=n_words, groups=g, e1=e1, e2=e2, t1=list(t1), t2=list(t2), tail=tail, **sec)


def decode(buf: np.ndarray) -> bytes:
    """Decode a dense encoded block; raises ValueError on inconsistent escape counts or lists."""
    buf = np.asarray(buf, dtype=np.uint8)
    h = parse_header(buf)
    n, n_words, g, e1, e2 = h["n"], h["n_words"], h["groups"], h["e1"], h["e2"]
    a = buf[h["off_a"]: h["off_a"] + n_words].astype(np.uint32)
    planes = buf[h["off_p"]: h["off_p"] + PLANE_BYTES * g].reshape(g, 3, 64, 2).transpose(0, 1, 3, 2)
    planes = planes.reshape(g, 3, GROUP_WORDS // 8)  # back to [group, plane, word // 8]
    c1 = np.zeros((g, GROUP_WORDS // 8, 8), dtype=np.uint8)
    for k in range(3):
        c1 |= (((planes[:, k, :, None] >> np.arange(8)) & 1) << k).astype(np.uint8)
    c1 = c1.reshape(-1)[:n_words]
    s1 = buf[h["off_s1"]: h["off_s1"] + 4 * (g + 1)].view("<u4").astype(np.int64)
    s2 = buf[h["off_s2"]: h["off_s2"] + 4 * (g + 1)].view("<u4").astype(np.int64)
    esc1 = np.nonzero(c1 == PRIMARY)[0]
    for s, e in ((s1, e1), (s2, e2)):
        if s[0] != 0 or s[-1] != e or np.any(np.diff(s) < 0):
            raise ValueError("inconsistent escape counts")
    if esc1.size != e1 or not np.array_equal(np.bincount(esc1 // GROUP_WORDS, minlength=g), np.diff(s1)):
        raise ValueError("primary escapes do not match their counts")
    packed = buf[h["off_y"]: h["off_y"] + (e1 + 1) // 2]
    nib = np.empty(2 * packed.size, dtype=np.uint8)
    nib[0::2], nib[1::2] = packed & 0x0F, packed >> 4
    c2 = nib[:e1]
    t1 = np.array(h["t1"][:PRIMARY] + [0], dtype=np.uint32)
    t2 = np.array(h["t2"][:SECONDARY] + [0], dtype=np.uint32)
    exp = t1[c1]
    exp[esc1] = t2[c2]
    esc2 = esc1[c2 == SECONDARY]
    x = buf[h["off_x"]: h["off_x"] + 4 * e2].view("<u4").astype(np.int64)
    group = np.repeat(np.arange(g, dtype=np.int64), np.diff(s2))
    w = group * GROUP_WORDS + (x >> 8)
    if w.size != esc2.size or not np.array_equal(np.sort(w), esc2):
        raise ValueError("secondary escape list does not match the secondary codes")
    exp[w] = (x & 0xFF).astype(np.uint32)
    words = ((a & 0x80) << 8) | (exp << 7) | (a & 0x7F)
    out = words.astype("<u2").tobytes()
    if n % 2:
        out += bytes([h["tail"]])
    return out
