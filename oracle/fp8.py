"""Oracle: float8 e4m3fn decoding and the fp8-weight linear layer, in float64.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference streams whatever weights the user's model holds and has no fp8
code of its own; the fp8 workload's layer is ``F.linear(x, w.to(bf16)) *
scale``. This module restates the OCP 8-bit floating-point format (OFP8,
E4M3 variant: 1 sign, 4 exponent bits with bias 7, 3 mantissa bits,
subnormals, no infinities, NaN = S.1111.111, largest finite 448) and the layer
``y[i, j] = scale[j] * sum_k x[i, k] * w[j, k]`` in exact float64 arithmetic.
"""

from __future__ import annotations

import numpy as np


def e4m3fn_value(byte: int) -> float:
    """Value of one e4m3fn byte from the format definition."""
    if not 0 <= byte <= 255:
        raise ValueError(f"not a byte: {byte}")
    sign = -1.0 if byte & 0x80 else 1.0
    exp = (byte >> 3) & 0xF
    man = byte & 0x7
    if exp == 0xF and man == 0x7:
        return float("nan")
    if exp == 0:
        return sign * (man / 8.0) * 2.0 ** (1 - 7)
    return sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)


E4M3FN_TABLE = np.array([e4m3fn_value(b) for b in range(256)], dtype=np.float64)


def decode_e4m3fn(raw: np.ndarray) -> np.ndarray:
    """float64 values of an array of e4m3fn bytes (uint8)."""
    return E4M3FN_TABLE[np.asarray(raw, dtype=np.uint8)]


def fp8_linear(x: np.ndarray, w_raw: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """float64 ``scale[j] * sum_k x[i, k] * w[j, k]``; x and scale as float64-convertible arrays."""
    w = decode_e4m3fn(w_raw)
    return (np.asarray(x, dtype=np.float64) @ w.T) * np.asarray(scale, dtype=np.float64)[None, :]


FLOAT32_MAX = float(np.finfo(np.float32).max)


def bf16_round(a) -> np.ndarray:
    """float64 values rounded to the nearest bfloat16 (ties to even), the rounding of every bf16 tensor
    operation: to float32 first (exact for float32 inputs), then the low 16 bits of the float32 pattern
    rounded away. NaN stays NaN; values past the largest bf16 round to infinity."""
    with np.errstate(over="ignore"):  # beyond float32's range is beyond bf16's: infinity either way
        f = np.asarray(a, dtype=np.float64).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = rounded.astype(np.uint32).view(np.float32).astype(np.float64)
    return np.where(np.isnan(f), np.nan, out)


def fp8_linear_swiglu(x: np.ndarray, wg_raw: np.ndarray, sg: np.ndarray, wu_raw: np.ndarray,
                      su: np.ndarray) -> np.ndarray:
    """``F.silu(g) * u`` of two bf16 fp8 linears, each operation rounded to bf16 as the separate PyTorch
    operations round it: g = bf16(gate), u = bf16(up), a = bf16(g / (1 + exp(-g))), then bf16(a * u).
    The arithmetic between roundings is float64, with one float32 trait kept: PyTorch evaluates a bf16
    silu in float32, where exp(-g) overflows to infinity once it passes float32's largest value (g below
    about -88.72), and the quotient is then a zero of g's sign."""
    g = bf16_round(fp8_linear(x, wg_raw, sg))
    u = bf16_round(fp8_linear(x, wu_raw, su))
    with np.errstate(over="ignore"):
        e = np.exp(-g)
    e = np.where(e > FLOAT32_MAX, np.inf, e)
    act = bf16_round(g / (1.0 + e))
    return bf16_round(act * u)


def fp8_linear_residual(x: np.ndarray, w_raw: np.ndarray, scale: np.ndarray, residual: np.ndarray) -> np.ndarray:
    """``residual + F.linear(...)`` in bf16: bf16(residual + bf16(linear)), the add exact in float64."""
    return bf16_round(np.asarray(residual, dtype=np.float64) + bf16_round(fp8_linear(x, w_raw, scale)))
