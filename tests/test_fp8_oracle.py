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


def test_bf16_round_closed_forms_and_torch():
    """Round to nearest bf16, ties to even: known answers a dropped tie rule or a truncation fails, and
    agreement with torch's own float32 -> bfloat16 conversion on random and edge values."""
    r = fp8.bf16_round
    assert r(1.0) == 1.0 and r(-2.5) == -2.5
    assert r(1.0 + 2.0 ** -8) == 1.0  # tie below an even mantissa: stays
    assert r(1.0 + 3 * 2.0 ** -8) == 1.0 + 2.0 ** -6  # tie above an odd mantissa: up to even
    assert r(1.0 + 2.0 ** -8 + 2.0 ** -20) == 1.0 + 2.0 ** -7  # past the tie: up
    assert r(1.0 + 2.0 ** -9) == 1.0  # below the tie: truncates
    assert math.isnan(float(r(float("nan")))) and r(3.5e38) == float("inf")
    rng = np.random.default_rng(3)
    vals = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-30, 30, 20000),
                           [0.0, -0.0, 1e-40, -1e-40, 3.3895e38]]).astype(np.float32)
    want = torch.from_numpy(vals).to(torch.bfloat16).double().numpy()
    assert np.array_equal(r(vals), want)


def test_swiglu_and_residual_restate_the_separate_operations():
    """The epilogue oracles equal the separate bf16 operations as PyTorch runs them on the CPU (linear,
    silu, product, add), up to the float32 rounding of silu (1 bf16 ulp at most, in a small share)."""
    rng = np.random.default_rng(9)
    m, n, k = 6, 40, 64
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
    codes = rng.integers(0, 256, size=(2, n, k), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x38
    scales = torch.from_numpy(rng.random((2, n)).astype(np.float32) / 8 + 0.01).to(torch.bfloat16)
    xs = x.double().numpy()
    gate, up = (fp8.bf16_round(fp8.fp8_linear(xs, codes[i], scales[i].double().numpy())) for i in range(2))
    g, u = torch.from_numpy(gate).to(torch.bfloat16), torch.from_numpy(up).to(torch.bfloat16)
    want = (torch.nn.functional.silu(g) * u).double().numpy()
    got = fp8.fp8_linear_swiglu(xs, codes[0], scales[0].double().numpy(), codes[1], scales[1].double().numpy())
    ulp = np.abs(want) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - want) <= ulp)
    # any output that differs has silu(g) next to a bf16 rounding midpoint (torch evaluates silu in float32)
    with np.errstate(over="ignore"):
        a = np.abs(gate / (1.0 + np.exp(-gate)))
    at = np.power(2.0, np.floor(np.log2(np.maximum(a, 1e-300))) - 7)
    near = np.abs((a / at) % 1.0 - 0.5) < 2.0 ** -10
    assert not np.any((got != want) & ~near)
    # gates far below zero: exp(-g) overflows float32, and silu is a signed zero, as torch gives
    big = np.array([-90.5, -200.0, -88.0, 88.0])
    one_codes = np.full((4, 1), 0x38, dtype=np.uint8)  # weights of 1.0: the gate is its scale
    far = torch.tensor(big, dtype=torch.bfloat16)
    torch_act = torch.nn.functional.silu(far).double().numpy()
    got_far = fp8.fp8_linear_swiglu(np.ones((1, 1)), one_codes, big, one_codes, np.ones(4))[0]
    assert np.array_equal(got_far, torch_act) and np.signbit(got_far[0]) and got_far[0] == 0.0
    resid = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(torch.bfloat16)
    want_r = (resid + g).double().numpy()
    got_r = fp8.fp8_linear_residual(xs, codes[0], scales[0].double().numpy(), resid.double().numpy())
    assert np.array_equal(got_r, want_r)
