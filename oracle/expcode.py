"""Exponent-coded blocks: the lossless byte format of compressed streamed blocks, restated in numpy.

TEST INFRASTRUCTURE ONLY (see the package docstring). No reference counterpart: the reference streams
each label's packed block as raw bytes (allocation_block.py:104-106). The format is this build's own,
and this module is its definition; ``flextensor_amd`` encodes with a host routine in the C library and
decodes with a zero-copy GPU kernel, and both are checked against this module.

A raw block of N bytes is read as W = N // 2 little-endian 16-bit words (the bit patterns of bf16
values: sign bit 15, exponent bits 14..7, mantissa bits 6..0); an odd last byte is kept verbatim.
Words are grouped in groups of 1024 (G = ceil(W / 1024) groups). The encoded block is:

* header, 64 bytes, then zeros up to byte 256:
  ``b"FTXE"``, u32 version 1, u64 N, u64 W, u64 G, u64 E (escapes), 16 table bytes, u8 tail byte
  (the odd last byte, else 0), 7 zero bytes;
* plane A at 256, G * 1024 bytes: byte w = sign(w) << 7 | mantissa(w); zero past W;
* plane B at 256 + 1024 G, G * 512 bytes: the 4-bit code of word w, in the low nibble of byte w // 2
  for even w and the high nibble for odd w; zero past W. Code c < 15 stands for exponent table[c];
  code 15 is an escape;
* S at 256 + 1536 G: G + 1 u32, S[g] = escapes in groups before g (S[G] = E);
* X at S + align16(4 (G + 1)): E u32, one per escaped word in word order, (w % 1024) << 8 | exponent.

The table holds the block's 15 most frequent exponents, most frequent first, ties to the smaller
exponent; a block with fewer distinct exponents leaves the rest of the table zero (codes that never
occur). The encoded size is 256 + 1536 G + align16(4 (G + 1)) + 4 E bytes: about 0.75 of the raw
size when escapes are rare (bf16 weights drawn from one distribution have 2-3 bits of exponent
entropy, so 15 exponents cover nearly every word).
"""

from __future__ import annotations

import struct

import numpy as np

MAGIC = b"FTXE"
VERSION = 1
HEADER_BYTES = 256
GROUP_WORDS = 1024
ESCAPE = 15
_HEAD = struct.Struct("<4sIQQQQ16sB7x")  # 64 bytes


def _align16(x: int) -> int:
    return (x + 15) // 16 * 16


def sections(n_groups: int, n_escapes: int) -> tuple[int, int, int, int, int]:
    """Byte offsets of planes A and B, S and X, and the total size."""
    off_a = HEADER_BYTES
    off_b = off_a + GROUP_WORDS * n_groups
    off_s = off_b + GROUP_WORDS // 2 * n_groups
    off_x = off_s + _align16(4 * (n_groups + 1))
    return off_a, off_b, off_s, off_x, off_x + 4 * n_escapes


def table_of(exponents: np.ndarray) -> list[int]:
    """The 15 most frequent exponents, most frequent first, ties to the smaller exponent."""
    hist = np.bincount(exponents.astype(np.int64), minlength=256)
    ranked = sorted((e for e in range(256) if hist[e] > 0), key=lambda e: (-int(hist[e]), e))
    return ranked[:ESCAPE]


def encoded_size(raw: bytes | np.ndarray) -> int:
    b = np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw.view(np.uint8)
    w = b[: b.size // 2 * 2].view("<u2")
    exp = (w >> 7) & 0xFF
    table = set(table_of(exp))
    escapes = int(np.count_nonzero(~np.isin(exp, list(table)))) if table else int(w.size)
    g = (w.size + GROUP_WORDS - 1) // GROUP_WORDS
    return sections(g, escapes)[4]


def encode(raw: bytes | np.ndarray) -> np.ndarray:
    """Encode ``raw`` (bytes or a uint8 array); returns the encoded block as a uint8 array."""
    b = np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw.view(np.uint8)
    n = int(b.size)
    n_words = n // 2
    words = b[: 2 * n_words].view("<u2").astype(np.uint32)
    exp = (words >> 7) & 0xFF
    table = table_of(exp)
    code_of = np.full(256, ESCAPE, dtype=np.uint8)
    for c, e in enumerate(table):
        code_of[e] = c
    codes = code_of[exp]
    g = (n_words + GROUP_WORDS - 1) // GROUP_WORDS
    esc = np.nonzero(codes == ESCAPE)[0]
    off_a, off_b, off_s, off_x, total = sections(g, int(esc.size))
    out = np.zeros(total, dtype=np.uint8)
    tab = bytes(table) + bytes(16 - len(table))
    tail = int(b[-1]) if n % 2 else 0
    out[:64] = np.frombuffer(_HEAD.pack(MAGIC, VERSION, n, n_words, g, int(esc.size), tab, tail), dtype=np.uint8)
    out[off_a: off_a + n_words] = (((words >> 8) & 0x80) | (words & 0x7F)).astype(np.uint8)
    nib = np.zeros(g * GROUP_WORDS, dtype=np.uint8)
    nib[:n_words] = codes
    out[off_b: off_b + g * GROUP_WORDS // 2] = nib[0::2] | (nib[1::2] << 4)
    counts = np.bincount(esc // GROUP_WORDS, minlength=g) if g else np.zeros(0, dtype=np.int64)
    s = np.zeros(g + 1, dtype="<u4")
    s[1:] = np.cumsum(counts)
    out[off_s: off_s + 4 * (g + 1)] = s.view(np.uint8)
    x = (((esc % GROUP_WORDS) << 8) | exp[esc]).astype("<u4")
    out[off_x: off_x + 4 * esc.size] = x.view(np.uint8)
    return out


def parse_header(buf: np.ndarray) -> dict:
    magic, version, n, n_words, g, e, tab, tail = _HEAD.unpack(bytes(buf[:64]))
    if magic != MAGIC or version != VERSION:
        raise ValueError("not an exponent-coded block")
    if n_words != n // 2 or g != (n_words + GROUP_WORDS - 1) // GROUP_WORDS:
        raise ValueError("inconsistent header")
    off_a, off_b, off_s, off_x, total = sections(g, e)
    if total > buf.size:
        raise ValueError("truncated block")
    return dict(n=n, n_words=n_words, groups=g, escapes=e, table=list(tab), tail=tail, off_a=off_a,
                off_b=off_b, off_s=off_s, off_x=off_x, total=total)


def decode(buf: np.ndarray) -> bytes:
    """Decode an encoded block; raises ValueError on an inconsistent escape list."""
    buf = np.asarray(buf, dtype=np.uint8)
    h = parse_header(buf)
    n, n_words, g, e = h["n"], h["n_words"], h["groups"], h["escapes"]
    a = buf[h["off_a"]: h["off_a"] + n_words].astype(np.uint32)
    packed = buf[h["off_b"]: h["off_b"] + g * GROUP_WORDS // 2]
    nib = np.empty(g * GROUP_WORDS, dtype=np.uint8)
    nib[0::2] = packed & 0x0F
    nib[1::2] = packed >> 4
    codes = nib[:n_words]
    table = np.array(h["table"][:ESCAPE] + [0], dtype=np.uint32)
    exp = table[codes]
    s = buf[h["off_s"]: h["off_s"] + 4 * (g + 1)].view("<u4").astype(np.int64)
    x = buf[h["off_x"]: h["off_x"] + 4 * e].view("<u4").astype(np.int64)
    if s[0] != 0 or s[-1] != e or np.any(np.diff(s) < 0):
        raise ValueError("inconsistent escape counts")
    group = np.repeat(np.arange(g, dtype=np.int64), np.diff(s))
    w = group * GROUP_WORDS + (x >> 8)
    escaped = np.nonzero(codes == ESCAPE)[0]
    if w.size != escaped.size or not np.array_equal(np.sort(w), escaped):
        raise ValueError("escape list does not match the escape codes")
    exp[w] = (x & 0xFF).astype(np.uint32)
    words = ((a & 0x80) << 8) | (exp << 7) | (a & 0x7F)
    out = words.astype("<u2").tobytes()
    if n % 2:
        out += bytes([h["tail"]])
    return out
