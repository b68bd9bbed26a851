"""Seeded synthetic parameters and tokens for the workloads in config.py.

Every tensor comes from its own numpy PCG64 stream keyed on (seed, tensor id),
drawn as float32 standard normals and scaled; values are then rounded to the
workload dtype (round to nearest even for bf16). The same seed gives the same
bits on every machine with this numpy, which is what lets the GPU box rebuild
the exact inputs the committed fixtures were made from.

Initialisation (std of a zero-mean normal), following the reference's own test
precedent (pre-train/test_cpmoe.py:385-388) and BASELINE's N(0, 1/fan_in):
  router.weight N(0, 1/d_in) (or router_std)   U_in N(0, 1/d_in)
  U_expert N(0, 1)   core N(0, 1/(r1*r3))   U_out N(0, 1/r2)   x N(0, 1)
  inner_norm.weight = 1, bias = 0 by default; `affine="random"` draws
  gain 1 + 0.1 N(0,1) and bias 0.1 N(0,1) so that tests exercise both.
"""
from __future__ import annotations

import hashlib
from typing import Dict

import numpy as np
import torch

from . import fp8
from .config import FfnWorkload, Workload

PARAM_KEYS = ("router.weight", "U_in", "inner_norm.weight", "U_expert", "core", "U_out", "bias")
_IDS = {k: i + 1 for i, k in enumerate(PARAM_KEYS)}
_X_ID = 100


def _normal(seed: int, tid: int, shape, std: float) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64([seed, tid]))
    return rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std)


def round_to(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Rounds float32 values to `dtype` (kept in `dtype`)."""
    return t.to(dtype)


def make_params(w: Workload, affine: str = "unit", dtype: torch.dtype = None) -> Dict[str, torch.Tensor]:
    """CPU tensors keyed like TuckerMoE.state_dict(), in `dtype` (default: the workload's)."""
    dtype = w.dtype if dtype is None else dtype
    E, d_in, d_out, r1, r2, r3 = w.E, w.d_in, w.d_out, w.r1, w.r2, w.r3
    rstd = w.router_std if w.router_std is not None else (1.0 / d_in) ** 0.5
    p = {
        "router.weight": _normal(w.seed, _IDS["router.weight"], (E, d_in), rstd),
        "U_in": _normal(w.seed, _IDS["U_in"], (d_in, r3), (1.0 / d_in) ** 0.5),
        "U_expert": _normal(w.seed, _IDS["U_expert"], (E, r1), 1.0),
        "core": _normal(w.seed, _IDS["core"], (r1, r3, r2), (1.0 / (r1 * r3)) ** 0.5),
        "U_out": _normal(w.seed, _IDS["U_out"], (r2, d_out), (1.0 / r2) ** 0.5),
    }
    if affine == "unit":
        p["inner_norm.weight"] = np.ones((r3,), np.float32)
        p["bias"] = np.zeros((d_out,), np.float32)
    elif affine == "random":
        p["inner_norm.weight"] = 1.0 + _normal(w.seed, _IDS["inner_norm.weight"], (r3,), 0.1)
        p["bias"] = _normal(w.seed, _IDS["bias"], (d_out,), 0.1)
    else:
        raise ValueError(f"affine={affine!r}: 'unit' or 'random'")
    return {k: round_to(torch.from_numpy(np.ascontiguousarray(p[k])), dtype) for k in PARAM_KEYS}


def make_fp8_params(w: Workload, affine: str = "unit"):
    """fp8-weight variant of make_params (the C5 format).

    The float32 draws of make_params are quantised per output channel (fp8.py):
    U_in, core and U_out become e4m3 codes + fp32 scales; router.weight,
    U_expert, inner_norm.weight and bias are rounded to bf16. Returns
    (params, codes, reference):
      params     bf16 state_dict for the module (dequantised weights rounded to bf16)
      codes      {U_in_q, U_in_scale, core_q, core_scale, U_out_q, U_out_scale}
      reference  float32 state_dict of the layer actually computed: the bf16
                 values above and the exactly dequantised q * s weights
    """
    p32 = make_params(w, affine=affine, dtype=torch.float32)
    codes = fp8.quantize_params(p32)
    ref = {k: v.to(torch.bfloat16).float() for k, v in p32.items()}
    for k in fp8.FP8_KEYS:
        ref[k] = fp8.dequantize(codes[f"{k}_q"], codes[f"{k}_scale"], k)
    params = {k: v.to(torch.bfloat16) for k, v in ref.items()}
    return params, codes, ref


def make_x(w: Workload, T: int = None, dtype: torch.dtype = None, stream: int = 0) -> torch.Tensor:
    """(T, d_in) CPU tokens ~ N(0, 1) in `dtype`; `stream` selects an independent draw."""
    T = w.T if T is None else T
    dtype = w.dtype if dtype is None else dtype
    x = _normal(w.seed, _X_ID + stream, (T, w.d_in), 1.0)
    return round_to(torch.from_numpy(x), dtype)


_FFN_NORM_ID, _FFN_GAMMA_ID = 200, 201


def make_ffn_params(f: FfnWorkload, affine: str = "random",
                    dtype: torch.dtype = None) -> Dict[str, torch.Tensor]:
    """CPU tensors keyed like TransformerBlock.state_dict() restricted to the FFN
    sub-block: norm_ffn.weight, ffn_gate.*, ffn_up.*, ffn_down.*, ls_ffn.gamma.
    Each TuckerMoE comes from make_params of f.layer(name); norm_ffn.weight and
    ls_ffn.gamma are 1 + 0.1 N(0, 1) ("random") or ones ("unit")."""
    dtype = f.dtype if dtype is None else dtype
    p = {}
    for name in ("ffn_gate", "ffn_up", "ffn_down"):
        for k, v in make_params(f.layer(name), affine=affine, dtype=dtype).items():
            p[f"{name}.{k}"] = v
    for key, tid in (("norm_ffn.weight", _FFN_NORM_ID), ("ls_ffn.gamma", _FFN_GAMMA_ID)):
        v = (1.0 + _normal(f.seed, tid, (f.d,), 0.1) if affine == "random"
             else np.ones((f.d,), np.float32))
        p[key] = round_to(torch.from_numpy(np.ascontiguousarray(v)), dtype)
    return p


def make_ffn_x(f: FfnWorkload, T: int = None, dtype: torch.dtype = None) -> torch.Tensor:
    """(T, d) CPU residual-stream rows ~ N(0, 1) in `dtype`."""
    T = f.T if T is None else T
    dtype = f.dtype if dtype is None else dtype
    return round_to(torch.from_numpy(_normal(f.seed, _X_ID, (T, f.d), 1.0)), dtype)


def sha256(t: torch.Tensor) -> str:
    """Digest of a CPU tensor's bytes (dtype-exact)."""
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    elif t.dtype == torch.float8_e4m3fn:
        t = t.view(torch.uint8)
    return hashlib.sha256(t.numpy().tobytes()).hexdigest()
