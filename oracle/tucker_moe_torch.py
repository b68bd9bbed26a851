"""PyTorch CPU restatement of the reference Tucker-MoE forward — TEST INFRASTRUCTURE.

Follows pure_torch_mlx/model.py op for op, on purpose (same torch ops in the same
order, so that it rounds like the reference module does on the same torch):
  rmsnorm      model.py:25-27   x.pow(2).mean(-1, keepdim).add(eps).sqrt(); (x / rms) * w
  forward      model.py:68-102  router linear -> topk -> softmax over the k
                                -> x @ U_in -> RMSNorm -> per-slot einsum/bmm
                                accumulation -> @ U_out + bias

Differences from the reference module, none of which changes a row's result:
  - rows are processed in chunks of `chunk` tokens (rows are independent; the
    reference materialises a (T, r3, r2) tensor per slot, 17 GB fp32 at T=16384);
  - parameters come in as a dict keyed like TuckerMoE.state_dict();
  - `compute_dtype` lets a caller run the same op sequence in float32 on
    bf16-valued inputs ("oracle mode": fp32 router logits, as the bf16
    workloads require), or in the inputs' own dtype (the CPU baseline).
"""
from __future__ import annotations

from typing import Dict, Optional

import torch
import torch.nn.functional as F


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """model.py:25-27."""
    rms = x.pow(2).mean(-1, keepdim=True).add(eps).sqrt()
    return (x / rms) * weight


def route(xf: torch.Tensor, router_w: torch.Tensor, top_k: int):
    """model.py:75-77: logits, top-k (values, indices), softmax over the k values."""
    scores = F.linear(xf, router_w)
    topk_v, topk_idx = torch.topk(scores, top_k, dim=-1)
    return scores, topk_idx, F.softmax(topk_v, dim=-1)


def tanh_approx(x: torch.Tensor) -> torch.Tensor:
    """mamba3_mlx/mlx_model/ops.py:9-10: 2 sigmoid(2x) - 1."""
    return 2.0 * torch.sigmoid(2.0 * x) - 1.0


def route_capped(xf: torch.Tensor, router_w: torch.Tensor, top_k: int, scale: float,
                 temperature: float):
    """The trained checkpoints' router, mamba3_mlx/mlx_model/tucker_moe.py:107-114 (with
    ops.py:13-14 scaled_tanh): raw logits in fp32, capped = tanh_approx(raw / scale) *
    scale, scores = capped / temperature, probs = softmax over all E, top-k of the
    scores (torch.topk order: descending, as sft_cot_bundle/scripts/model.py:327),
    weights = probs at the selected experts / (their sum + 1e-6). Returns the raw
    logits, the indices and the weights."""
    raw = F.linear(xf, router_w)
    capped = tanh_approx(raw.float() * (1.0 / scale)) * scale
    scores = capped / temperature
    probs = torch.softmax(scores, dim=-1)
    _, topk_idx = torch.topk(scores, top_k, dim=-1)
    top = probs.gather(-1, topk_idx)
    return raw, topk_idx, (top / (top.sum(-1, keepdim=True) + 1e-6)).to(raw.dtype)


def project_in(xf, U_in, inner_w, eps):
    """model.py:80-81."""
    return rmsnorm(xf @ U_in, inner_w, eps)


def core_contract(z, topk_idx, topk_w, U_expert, core):
    """model.py:87-98: sum over slots j of w_j * z (U_expert[e_j] . core)."""
    acc = z.new_zeros(z.shape[0], core.shape[2])
    for j in range(topk_idx.shape[1]):
        g = U_expert[topk_idx[:, j]]
        G = torch.einsum("br,rst->bst", g, core)
        acc.add_(topk_w[:, j:j + 1] * torch.bmm(z.unsqueeze(1), G).squeeze(1))
    return acc


def project_out(mid, U_out, bias):
    """model.py:101."""
    return mid @ U_out + bias


STAGES = {"route": route, "project_in": project_in, "core_contract": core_contract,
          "project_out": project_out}


def forward(x: torch.Tensor, params: Dict[str, torch.Tensor], top_k: int, eps: float = 1e-5,
            chunk: int = 512, compute_dtype: Optional[torch.dtype] = None,
            intermediates: bool = False, stages: Optional[dict] = None, router=None):
    """TuckerMoE.forward (model.py:68-102) on the CPU.

    x: (..., d_in). params: state_dict-keyed tensors. Returns out (..., d_out) in
    compute_dtype (default: the parameters' dtype) or, with intermediates=True,
    a dict with logits (T, E), idx (T, k) int64, w (T, k), z (T, r3),
    mid (T, r2) and out.
    `stages` replaces stage functions by name (used by the tests' planted
    mistakes). `router` = ("capped", scale, temperature) selects route_capped
    instead of the reference module's route."""
    st = dict(STAGES)
    if stages:
        st.update(stages)
    cd = compute_dtype or params["U_in"].dtype
    p = {k: v.detach().to("cpu", cd) for k, v in params.items()}
    *batch, d_in = x.shape
    xf_all = x.detach().to("cpu", cd).reshape(-1, d_in)
    T = xf_all.shape[0]
    keep = {"logits": [], "idx": [], "w": [], "z": [], "mid": [], "out": []}
    for s in range(0, max(T, 1), chunk):
        xf = xf_all[s:s + chunk]
        if xf.shape[0] == 0:
            break
        if router is not None and router[0] == "capped":
            logits, idx, w = route_capped(xf, p["router.weight"], top_k, router[1], router[2])
        else:
            logits, idx, w = st["route"](xf, p["router.weight"], top_k)
        z = st["project_in"](xf, p["U_in"], p["inner_norm.weight"], eps)
        mid = st["core_contract"](z, idx, w, p["U_expert"], p["core"])
        out = st["project_out"](mid, p["U_out"], p["bias"])
        keep["out"].append(out)
        if intermediates:
            for k_, v_ in (("logits", logits), ("idx", idx), ("w", w), ("z", z), ("mid", mid)):
                keep[k_].append(v_)
    d_out = p["U_out"].shape[1]
    out = torch.cat(keep["out"]) if keep["out"] else xf_all.new_zeros(0, d_out)
    out = out.reshape(*batch, d_out)
    if not intermediates:
        return out
    res = {k: torch.cat(v) for k, v in keep.items() if k != "out" and v}
    res["out"] = out
    return res
