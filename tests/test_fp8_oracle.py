"""The fp8 oracle pinned by the format's closed forms, by brute force and by torch's own decoding."""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle import fp8


def test_e4m3fn_closed_forms():
    v = fp8.e4m3fn_value
    assert v(0x00) == 0.0 and math.copysign(1.0, v(0x80)) == -1.0 and v(0x80) == 0.0
    assert v(0x38) == 1.0 and v(0xB8) == -1.0  # exponent field 7 = bias
    assert v(0x7E) == 448.0 and v(0xFE) == -448.0  # largest finite
    assert v(0x01) == 2.0 ** -9  # smallest subnormal
    assert v(0x07) == 7 * 2.0 ** -9  # largest subnormal
    assert v(0x08) == 2.0 ** -6  # smallest normal
    assert math.isnan(v(0x7F)) and math.isnan(v(0xFF))
    assert v(0x78) == 256.0  # exponent 15 with mantissa < 7 is finite: no infinities


def test_e4m3fn_ordering_and_symmetry():
    pos = fp8.E4M3FN_TABLE[:0x7F]
    assert np.all(np.diff(pos) > 0)  # byte order is value order for positive codes
    assert np.array_equal(fp8.E4M3FN_TABLE[0x80:0xFF], -pos)
    # consecutive normals within one binade are 1/8 of the binade apart
    assert np.allclose(np.diff(pos[8:16]), 2.0 ** -6 / 8)


def test_e4m3fn_agrees_with_torch_for_every_byte():
    got = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    want = fp8.E4M3FN_TABLE
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])


def test_fp8_linear_matches_brute_force():
    rng = np.random.default_rng(0)
    w_raw = rng.integers(0, 256, size=(5, 7), dtype=np.uint8)
    w_raw[(w_raw & 0x7F) == 0x7F] = 0x38  # no NaN codes
    x = rng.standard_normal((3, 7))
    scale = rng.standard_normal(5)
    got = fp8.fp8_linear(x, w_raw, scale)
    for i in range(3):
        for j in range(5):
            s = sum(x[i, k] * fp8.e4m3fn_value(int(w_raw[j, k])) for k in range(7))
            assert math.isclose(got[i, j], s * scale[j], rel_tol=1e-12, abs_tol=1e-12)
