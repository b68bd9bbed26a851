"""fp8 (OCP e4m3) weights with one fp32 scale per output channel.

The reference has no quantised path; this is the weight format of the fp8
configuration. A projection weight W is stored as q = e4m3(W / s) with
s = max|W| / 448 over each output channel (448 is the largest e4m3 value), and
the layer computed is the reference TuckerMoE (pure_torch_mlx/model.py:41-102)
with the dequantised weights q * s. Output channels:
  U_in  (d_in, r3)       one scale per column j            -> scale (r3,)
  core  (r1, r3, r2)     one per (r, q): a column of the (r3, r1*r2) view
                                                            -> scale (r1, r2)
  U_out (r2, d_out)      one per column n                  -> scale (d_out,)
A channel whose weights are all zero gets scale 0 and zero codes.
"""
from __future__ import annotations

from typing import Dict, Tuple

import torch

E4M3_MAX = 448.0
FP8_KEYS = ("U_in", "core", "U_out")
# reduction dims of each weight's per-output-channel amax
_REDUCE = {"U_in": (0,), "core": (1,), "U_out": (0,)}


def quantize(w: torch.Tensor, name: str) -> Tuple[torch.Tensor, torch.Tensor]:
    """Returns (codes as torch.float8_e4m3fn, fp32 scales) of weight `name`."""
    if name not in _REDUCE:
        raise ValueError(f"no fp8 layout for {name!r}; expected one of {FP8_KEYS}")
    w32 = w.detach().float()
    dims = _REDUCE[name]
    amax = w32.abs().amax(dim=dims, keepdim=True)
    scale = amax / E4M3_MAX
    safe = torch.where(scale > 0, scale, torch.ones_like(scale))
    q = (w32 / safe).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q.contiguous(), scale.squeeze(dims).contiguous()


def dequantize(q: torch.Tensor, scale: torch.Tensor, name: str) -> torch.Tensor:
    """fp32 weight q * s of `name` (q as float8_e4m3fn or its uint8 bits); a
    channel whose scale is zero is zero whatever its codes (NaN codes included),
    as the packed weights hold it."""
    if q.dtype == torch.uint8:
        q = q.view(torch.float8_e4m3fn)
    s = scale.float()
    if name == "core":
        s = s.unsqueeze(1)          # (r1, 1, r2)
    elif name in ("U_in", "U_out"):
        s = s.unsqueeze(0)          # (1, cols)
    else:
        raise ValueError(f"no fp8 layout for {name!r}")
    return torch.where(s == 0, torch.zeros((), dtype=torch.float32, device=q.device), q.float() * s)


def quantize_params(params: Dict[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
    """{U_in_q, U_in_scale, core_q, core_scale, U_out_q, U_out_scale} of a
    state_dict-like mapping."""
    out = {}
    for k in FP8_KEYS:
        q, s = quantize(params[k], k)
        out[f"{k}_q"], out[f"{k}_scale"] = q, s
    return out
