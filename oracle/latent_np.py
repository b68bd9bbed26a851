"""float64 formulation of the training module's latent expert contraction and its
backward — TEST INFRASTRUCTURE.

The reference (sft_cot_bundle/scripts/model.py) computes, for x = x_shared (B, r3),
G = G_experts (E, r3, r2), selected experts idx (B, k) and probabilities p (B, k):
  forward (_fused_latent_moe_fwd, :160-174):  out[b] = sum_j p[b,j] x[b] @ G[idx[b,j]]
  backward (FusedLatentMoE.backward, :240-289, dG kernel :196-219):
    dx[b]    = sum_j p[b,j] dout[b] @ G[idx[b,j]]^T
    dp[b,j]  = dout[b] . (x[b] @ G[idx[b,j]])
    dG[e]    = sum_{b,j: idx[b,j] = e} p[b,j] outer(x[b], dout[b])
Here they are stated per token and per slot with numpy in float64. tests pin them
against torch autograd of the forward (float64) and a finite-difference check.
"""
from __future__ import annotations

import numpy as np


def _f64(v):
    if hasattr(v, "detach"):
        v = v.detach().cpu()
        if v.dtype.is_floating_point:
            v = v.double()
        return v.numpy()
    return np.asarray(v)


def forward(x, G, idx, p) -> np.ndarray:
    X, Gm, I, P = _f64(x).astype(np.float64), _f64(G).astype(np.float64), _f64(idx), _f64(p)
    out = np.zeros((X.shape[0], Gm.shape[2]))
    for j in range(I.shape[1]):
        out += P[:, j:j + 1] * np.einsum("bs,bsq->bq", X, Gm[I[:, j]])
    return out


def backward(x, G, idx, p, dout):
    """(dx (B, r3), dG (E, r3, r2), dp (B, k)) in float64."""
    X, Gm, I, P = _f64(x).astype(np.float64), _f64(G).astype(np.float64), _f64(idx), _f64(p)
    D = _f64(dout).astype(np.float64)
    B, k = I.shape
    dx = np.zeros_like(X)
    dp = np.zeros((B, k))
    dG = np.zeros_like(Gm)
    for j in range(k):
        Ge = Gm[I[:, j]]                                   # (B, r3, r2)
        dx += P[:, j:j + 1] * np.einsum("bq,bsq->bs", D, Ge)
        dp[:, j] = np.einsum("bq,bs,bsq->b", D, X, Ge)
        np.add.at(dG, I[:, j], P[:, j, None, None] * np.einsum("bs,bq->bsq", X, D))
    return dx, dG, dp
