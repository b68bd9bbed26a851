"""OCP FP8 E4M3 decoding and per-output-channel dequantisation — TEST INFRASTRUCTURE.

The reference has no fp8 path; its fp8 configuration is defined as the
reference layer (pure_torch_mlx/model.py:41-102) run on the dequantised weights
W = decode(q) * s. This module restates that decoding from the OCP 8-bit
floating point specification (E4M3: 1 sign bit, 4 exponent bits with bias 7,
3 mantissa bits, no infinities, S.1111.111 = NaN, exponent 0 = subnormals
m * 2^-9), independently of the product's e4m3 conversion.
"""
from __future__ import annotations

import numpy as np


def decode(codes) -> np.ndarray:
    """float64 values of uint8 E4M3 codes (any shape)."""
    b = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 0x7
    normal = (1.0 + m / 8.0) * np.power(2.0, e - 7)
    sub = (m / 8.0) * 2.0 ** -6
    v = sign * np.where(e == 0, sub, normal)
    return np.where((e == 15) & (m == 7), np.nan, v)


def dequantize(codes, scale, name: str) -> np.ndarray:
    """float64 weight of `name` from its codes and per-output-channel scales:
    U_in (d_in, r3) with scales (r3,), core (r1, r3, r2) with (r1, r2),
    U_out (r2, d_out) with (d_out,). A channel whose scale is zero is zero,
    whatever its codes (NaN codes included): the C ABI's fp8 contract (tmoe.h,
    tmoe_pack_weights_fp8), which a plain decode(q) * s would break for NaN codes."""
    v = decode(codes)
    s = np.asarray(scale, dtype=np.float64)
    if name == "core":
        s = s[:, None, :]
    elif name in ("U_in", "U_out"):
        s = s[None, :]
    else:
        raise ValueError(f"no fp8 layout for {name!r}")
    return np.where(s == 0, 0.0, v * s)
