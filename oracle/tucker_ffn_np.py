"""float64 numpy formulation of the TransformerBlock FFN sub-block — TEST
INFRASTRUCTURE.

An independent statement of pure_torch_mlx/model.py:337-341 written from the
mathematics, used to pin the torch restatement (tucker_ffn_torch.py):
  x_f = x / sqrt(mean(x^2) + eps) * g_norm                model.py:337, :25-27
  h   = silu(TMoE_gate(x_f)) * TMoE_up(x_f),  silu(u) = u / (1 + e^-u)   :338-340
  out = x + gamma * TMoE_down(h)                          model.py:341, :35-36
with each TMoE the float64 layer of tucker_moe_np.forward_f64, and no rounding.
Returns the per-layer router logits too, so that a test can tell a routing
flip (a top-k gap within rounding) from a mistake.
"""
from __future__ import annotations

from typing import Dict

import numpy as np

from . import tucker_moe_np as tnp


def _layer(params: Dict, name: str) -> Dict:
    pre = name + "."
    return {k[len(pre):]: v for k, v in params.items() if k.startswith(pre)}


def _f64(v) -> np.ndarray:
    if hasattr(v, "detach"):
        v = v.detach().cpu().double().numpy()
    return np.asarray(v, np.float64)


def ffn_forward_f64(x_res, params: Dict, top_k: int, eps: float = 1e-5, router=None) -> Dict:
    """dict(x_f, gate, up, h, dn, out) in float64, and per layer {name: ...} the
    router logits (T, E), scores and selected experts idx (T, k)."""
    X = _f64(x_res)
    X = X.reshape(-1, X.shape[-1])
    g = _f64(params["norm_ffn.weight"])
    gamma = _f64(params["ls_ffn.gamma"])
    x_f = X / np.sqrt(np.mean(X * X, axis=1, keepdims=True) + eps) * g
    rg = tnp.forward_f64(x_f, _layer(params, "ffn_gate"), top_k, eps, router=router)
    ru = tnp.forward_f64(x_f, _layer(params, "ffn_up"), top_k, eps, router=router)
    gate, up = rg["out"], ru["out"]
    h = gate / (1.0 + np.exp(-gate)) * up
    rd = tnp.forward_f64(h, _layer(params, "ffn_down"), top_k, eps, router=router)
    dn = rd["out"]
    out = X + gamma * dn
    return {"x_f": x_f, "gate": gate, "up": up, "h": h, "dn": dn, "out": out,
            "logits": {"ffn_gate": rg["logits"], "ffn_up": ru["logits"],
                       "ffn_down": rd["logits"]},
            "scores": {"ffn_gate": rg["scores"], "ffn_up": ru["scores"],
                       "ffn_down": rd["scores"]},
            "idx": {"ffn_gate": rg["idx"], "ffn_up": ru["idx"], "ffn_down": rd["idx"]}}
