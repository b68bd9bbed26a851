"""The training module's latent expert contraction on MI355X (gfx950), with backward.

FusedLatentMoE mirrors the reference's autograd function
(sft_cot_bundle/scripts/model.py:225-289, called by TritonTuckerMoE.forward :336-338):

    x_core = FusedLatentMoE.apply(x_shared, G_experts, top_k_indices, top_k_probs)

x_shared (B, r3) and G_experts (E, r3, r2) in bfloat16 or float32, top_k_indices
(B, k) int64, top_k_probs (B, k) (converted to x_shared's dtype; its gradient is
returned in its own dtype). The forward and backward run tmoe_latent_forward /
tmoe_latent_backward of libtmoe.so (HIP devices only, no fallback):

    out[b]   = sum_j p[b,j] x[b] G[idx[b,j]]
    dx[b]    = sum_j p[b,j] dout[b] G[idx[b,j]]^T
    dp[b,j]  = dout[b] . (x[b] G[idx[b,j]])
    dG[e]    = sum_{b,j: idx[b,j] = e} p[b,j] x[b]^T dout[b]

Indices get no gradient (as in the reference).
"""
from __future__ import annotations

import torch

from . import _lib


def _ws(nbytes: int, dev) -> torch.Tensor:
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)


def _check(x, G, idx, p):
    if x.device.type != "cuda":
        raise RuntimeError(f"FusedLatentMoE runs on HIP devices only; input is on {x.device}")
    if G.dtype != x.dtype:
        raise RuntimeError(f"FusedLatentMoE: G_experts dtype {G.dtype} != x_shared dtype {x.dtype}")
    if x.dim() != 2 or G.dim() != 3 or G.shape[1] != x.shape[1]:
        raise RuntimeError(f"FusedLatentMoE: x_shared {tuple(x.shape)} and G_experts "
                           f"{tuple(G.shape)} do not match (B, r3) and (E, r3, r2)")
    if idx.shape != p.shape or idx.shape[0] != x.shape[0] or idx.dtype != torch.int64:
        raise RuntimeError("FusedLatentMoE: top_k_indices (B, k) int64 and top_k_probs (B, k) "
                           "expected")


class FusedLatentMoE(torch.autograd.Function):
    """HIP forward and backward of the reference's FusedLatentMoE."""

    @staticmethod
    def forward(ctx, x_shared, G_experts, top_k_indices, top_k_probs):
        _check(x_shared, G_experts, top_k_indices, top_k_probs)
        x = x_shared.contiguous()
        G = G_experts.contiguous()
        idx = top_k_indices.contiguous()
        p = top_k_probs.to(x.dtype).contiguous()
        B, r3 = x.shape
        E, _, r2 = G.shape
        k = idx.shape[1]
        dt = _lib.dtype_code(x.dtype)
        L = _lib.lib()
        out = torch.empty(B, r2, dtype=x.dtype, device=x.device)
        nws = L.tmoe_latent_workspace_bytes(B, E, r3, r2, dt, 0)
        ws = _ws(nws, x.device)
        with torch.cuda.device(x.device):
            _lib.check(L.tmoe_latent_forward(
                x.data_ptr(), G.data_ptr(), idx.data_ptr(), p.data_ptr(), B, E, k, r3, r2, dt,
                out.data_ptr(), ws.data_ptr(), nws,
                torch.cuda.current_stream(x.device).cuda_stream))
        ctx.save_for_backward(x, G, idx, p)
        ctx.p_dtype = top_k_probs.dtype
        return out

    @staticmethod
    def backward(ctx, dout):
        x, G, idx, p = ctx.saved_tensors
        B, r3 = x.shape
        E, _, r2 = G.shape
        k = idx.shape[1]
        d = dout.to(x.dtype).contiguous()
        dt = _lib.dtype_code(x.dtype)
        L = _lib.lib()
        dx = torch.empty_like(x)
        dG = torch.empty_like(G)
        dp = torch.empty(B, k, dtype=x.dtype, device=x.device)
        nws = L.tmoe_latent_workspace_bytes(B, E, r3, r2, dt, 1)
        ws = _ws(nws, x.device)
        with torch.cuda.device(x.device):
            _lib.check(L.tmoe_latent_backward(
                x.data_ptr(), G.data_ptr(), idx.data_ptr(), p.data_ptr(), d.data_ptr(), B, E, k,
                r3, r2, dt, dx.data_ptr(), dG.data_ptr(), dp.data_ptr(), ws.data_ptr(), nws,
                torch.cuda.current_stream(x.device).cuda_stream))
        return dx, dG, None, dp.to(ctx.p_dtype)


def fused_latent_moe(x_shared, G_experts, top_k_indices, top_k_probs):
    """FusedLatentMoE.apply(...)."""
    return FusedLatentMoE.apply(x_shared, G_experts, top_k_indices, top_k_probs)
