"""PyTorch CPU restatement of the reference TransformerBlock FFN sub-block — TEST
INFRASTRUCTURE (only tests/, __graft_entry__.smoke() and bench.py's CPU baseline
use it).

Follows pure_torch_mlx/model.py:337-341 op for op:
  x_f   = norm_ffn(x_res)                    RMSNorm          model.py:25-27
  gate  = ffn_gate(x_f)                      TuckerMoE        model.py:68-102
  up    = ffn_up(x_f)                        TuckerMoE
  dn    = ffn_down(F.silu(gate) * up)        TuckerMoE
  x_res = x_res + ls_ffn(dn)                 LayerScale       model.py:35-36

Rounding: with compute_dtype=float32 on bf16 parameters ("oracle mode"), every
sub-module computes in fp32 on bf16-valued inputs and its result is rounded to
the module dtype, as the module's own output is: x_f, gate, up, silu(gate),
silu(gate) * up, dn, gamma * dn and the sum each round once. Without
compute_dtype the same op sequence runs in the parameters' dtype (the reference
module on the CPU).
"""
from __future__ import annotations

from typing import Dict, Optional

import torch
import torch.nn.functional as F

from . import tucker_moe_torch as tm

LAYERS = ("ffn_gate", "ffn_up", "ffn_down")


def layer_params(params: Dict[str, torch.Tensor], name: str) -> Dict[str, torch.Tensor]:
    """The TuckerMoE state_dict of sub-module `name` out of the block's."""
    pre = name + "."
    return {k[len(pre):]: v for k, v in params.items() if k.startswith(pre)}


def _residual(x, scaled):
    """x_res + ls_ffn(dn), model.py:341."""
    return x + scaled


STAGES = {"rmsnorm": tm.rmsnorm, "silu": F.silu, "residual": _residual}


def ffn_forward(x_res: torch.Tensor, params: Dict[str, torch.Tensor], top_k: int,
                eps: float = 1e-5, compute_dtype: Optional[torch.dtype] = None,
                chunk: int = 512, intermediates: bool = False, router=None,
                stages: Optional[dict] = None):
    """The FFN sub-block (model.py:337-341) on the CPU.

    x_res: (..., d). params: keyed like the block's state_dict restricted to the
    sub-block (norm_ffn.weight, ffn_gate.*, ffn_up.*, ffn_down.*, ls_ffn.gamma).
    Returns the new x_res (..., d) in the parameters' dtype or, with
    intermediates=True, a dict with x_f, gate, up, h (= silu(gate) * up), dn and
    out, each (T, .), and idx {layer: (T, k) selected experts}. `stages` replaces the functions of STAGES by name (the
    tests' planted mistakes)."""
    st = dict(STAGES)
    if stages:
        st.update(stages)
    dt = params["norm_ffn.weight"].dtype
    cd = compute_dtype or dt

    def rnd(v):
        return v.to(dt).to(cd)

    *batch, d = x_res.shape
    x = x_res.detach().to("cpu", cd).reshape(-1, d)
    g = params["norm_ffn.weight"].detach().to("cpu", cd)
    gamma = params["ls_ffn.gamma"].detach().to("cpu", cd)
    x_f = rnd(st["rmsnorm"](x, g, eps))

    idx = {}

    def layer(name, inp):
        r = tm.forward(inp, layer_params(params, name), top_k, eps, chunk=chunk,
                       compute_dtype=cd, router=router, intermediates=intermediates)
        if not intermediates:
            return rnd(r)
        idx[name] = r["idx"]
        return rnd(r["out"])

    gate = layer("ffn_gate", x_f)
    up = layer("ffn_up", x_f)
    h = rnd(rnd(st["silu"](gate)) * up)
    dn = layer("ffn_down", h)
    out = rnd(st["residual"](x, rnd(gamma * dn)))
    out = out.to(dt).reshape(*batch, d)
    if not intermediates:
        return out
    return {"x_f": x_f, "gate": gate, "up": up, "h": h, "dn": dn, "out": out, "idx": idx}
