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
        # the reference's kernels read the probabilities in their own dtype
        # (model.py:160-174, :196-219): fp32 ones reach the kernels unrounded, others
        # in x's dtype
        p_f32 = top_k_probs.dtype == torch.float32 and x.dtype != torch.float32
        p = top_k_probs.to(torch.float32 if p_f32 else x.dtype).contiguous()
        B, r3 = x.shape
        E, _, r2 = G.shape
        k = idx.shape[1]
        dt = _lib.dtype_code(x.dtype) | (_lib.TMOE_LATENT_P_F32 if p_f32 else 0)
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
        p_f32 = p.dtype == torch.float32 and x.dtype != torch.float32
        dt = _lib.dtype_code(x.dtype) | (_lib.TMOE_LATENT_P_F32 if p_f32 else 0)
        L = _lib.lib()
        dx = torch.empty_like(x)
        dG = torch.empty_like(G)
        dp = torch.empty(B, k, dtype=p.dtype, device=x.device)
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


def router_temperature(step, warmup: int = 500, total: int = 10000, t_start: float = 2.0,
                       t_end: float = 0.5):
    """The reference's router temperature schedule (model.py:114-120): t_end before
    any step is given, else a cosine from t_start to t_end over steps warmup .. total."""
    if step is None:
        return t_end
    s = torch.as_tensor(step, dtype=torch.float32)
    progress = torch.clamp((s - warmup) / max(1, total - warmup), min=0.0, max=1.0)
    return t_end + 0.5 * (t_start - t_end) * (1.0 + torch.cos(torch.pi * progress))


def scaled_tanh(x: torch.Tensor, scale: float = 10.0) -> torch.Tensor:
    """scale * tanh(x / scale) as 2 sigmoid(2u) - 1 (the reference's fast_scaled_tanh,
    model.py:22-64; its backward dy (1 - t^2) is the autograd of this expression)."""
    return scale * (2.0 * torch.sigmoid(2.0 * x / scale) - 1.0)


class TuckerMoETrain(torch.nn.Module):
    """The reference's training layer TritonTuckerMoE (model.py:292-340): the same
    constructor, parameters (router.weight, U_expert, U_in, U_out, core, bias,
    inner_norm.weight) and forward(x, step) -> (out, lb_loss, z_loss). The latent
    expert contraction and its backward run on FusedLatentMoE (HIP); the router,
    projections and losses are the reference's torch expressions."""

    def __init__(self, dim_in, dim_out, num_experts=8, top_k=2, r1=4, r2=1024, r3=256):
        super().__init__()
        self.num_experts = num_experts
        self.top_k = min(top_k, num_experts)
        self.router = torch.nn.Linear(dim_in, num_experts, bias=False)
        torch.nn.init.normal_(self.router.weight, mean=0.0, std=0.02)
        self.U_expert = torch.nn.Parameter(torch.empty(num_experts, r1))
        self.U_in = torch.nn.Parameter(torch.empty(dim_in, r3))
        self.U_out = torch.nn.Parameter(torch.empty(r2, dim_out))
        self.core = torch.nn.Parameter(torch.empty(r1, r3, r2))
        self.bias = torch.nn.Parameter(torch.zeros(dim_out))
        self.inner_norm = torch.nn.RMSNorm(r3, eps=1e-5)
        torch.nn.init.orthogonal_(self.U_in)
        torch.nn.init.orthogonal_(self.U_out)
        torch.nn.init.xavier_uniform_(self.U_expert)
        torch.nn.init.xavier_uniform_(self.core)

    def forward(self, x, step=None):
        orig = x.shape
        xf = x.reshape(-1, orig[-1])
        temperature = router_temperature(step)
        raw = self.router(xf)
        capped = scaled_tanh(raw, 10.0)
        z_loss = torch.mean(torch.logsumexp(capped, dim=-1) ** 2) if self.training else 0.0
        logits = capped / temperature
        probs = torch.softmax(logits, dim=-1)
        _, idx = torch.topk(logits, self.top_k, dim=-1)
        top = probs.gather(-1, idx)
        top_p = top / (top.sum(-1, keepdim=True) + 1e-6)
        if self.training:
            mask = torch.zeros_like(logits).scatter_(1, idx, 1.0)
            lb_loss = self.num_experts * torch.sum(mask.mean(0) * probs.float().mean(0))
        else:
            lb_loss = 0.0
        xs = self.inner_norm(torch.matmul(xf, self.U_in))
        G = torch.einsum("er,rst->est", self.U_expert, self.core)
        core = FusedLatentMoE.apply(xs, G, idx, top_p).to(x.dtype)
        out = torch.matmul(core, self.U_out).reshape(*orig[:-1], -1)
        return out + self.bias, lb_loss, z_loss
