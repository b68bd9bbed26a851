"""float64 numpy formulation of the Tucker-MoE forward — TEST INFRASTRUCTURE.

An independent statement of pure_torch_mlx/model.py:68-102, written from the
mathematics rather than the reference's op sequence, used to pin the torch
restatement (tucker_moe_torch.py) and, at full sizes, the GPU results:
  logits = X W_r^T                                        model.py:75
  top-k by a stable argsort of -logits (ties: lower index) model.py:76
  w = exp(v - v_0) / sum exp(v - v_0)                     model.py:77
  z = RMSNorm(X U_in) * g                                 model.py:80-81, :25-27
  c = sum_j w_j U_expert[e_j]             (T, r1)         model.py:91-93 regrouped
  mid[t] = sum_r c[t, r] * (z[t] @ core[r])               model.py:95-98 regrouped
  out = mid U_out + bias                                  model.py:101

brute_force() restates the same layer with pure-Python loops, in the
reference's own grouping (per slot, G_j = sum_r g_jr core[r]), for tiny shapes.

router=("capped", scale, temperature) states the trained checkpoints' router
(mamba3_mlx/mlx_model/tucker_moe.py:107-114) from its definition: scores =
scale * tanh(logits / scale) / temperature (tanh itself, which the reference's
2 sigmoid(2u) - 1 equals), top-k of the scores, P = softmax(scores) over all E,
w = P[top-k] / (sum P[top-k] + 1e-6).
"""
from __future__ import annotations

import math
from typing import Dict

import numpy as np


def _np(p):
    return {k: np.asarray(v.detach().cpu().double().numpy() if hasattr(v, "detach") else v,
                          dtype=np.float64) for k, v in p.items()}


def forward_f64(x, params: Dict, top_k: int, eps: float = 1e-5, chunk: int = 4096,
                router=None) -> Dict:
    """Returns dict(logits, scores, idx (int64), w, z, c, mid, out) in float64
    (scores: what top-k ranks; the logits unless router is "capped").

    x: (T, d_in) array or tensor; params: state_dict-keyed arrays or tensors."""
    p = _np(params)
    X = np.asarray(x.detach().cpu().float().numpy() if hasattr(x, "detach") else x, np.float64)
    X = X.reshape(-1, X.shape[-1])
    Wr, U_in, g = p["router.weight"], p["U_in"], p["inner_norm.weight"]
    U_exp, core, U_out, bias = p["U_expert"], p["core"], p["U_out"], p["bias"]
    r1, r3, r2 = core.shape
    P = core.transpose(1, 0, 2).reshape(r3, r1 * r2)     # z @ P = [z @ core[r]]_r
    res = {k: [] for k in ("logits", "scores", "idx", "w", "z", "c", "mid", "out")}
    capped = router is not None and router[0] == "capped"
    for s in range(0, X.shape[0], chunk):
        Xc = X[s:s + chunk]
        S = Xc @ Wr.T
        L = router[1] * np.tanh(S / router[1]) / router[2] if capped else S
        idx = np.argsort(-L, axis=1, kind="stable")[:, :top_k]
        if capped:
            prob = np.exp(L - L.max(axis=1, keepdims=True))
            prob /= prob.sum(axis=1, keepdims=True)
            top = np.take_along_axis(prob, idx, axis=1)
            w = top / (top.sum(axis=1, keepdims=True) + 1e-6)
        else:
            v = np.take_along_axis(S, idx, axis=1)
            e = np.exp(v - v[:, :1])
            w = e / e.sum(axis=1, keepdims=True)
        zr = Xc @ U_in
        rms = np.sqrt(np.mean(zr * zr, axis=1, keepdims=True) + eps)
        z = zr / rms * g
        c = np.einsum("tj,tjr->tr", w, U_exp[idx])
        Y = (z @ P).reshape(-1, r1, r2)
        mid = np.einsum("tr,trj->tj", c, Y)
        out = mid @ U_out + bias
        for k_, v_ in (("logits", S), ("scores", L), ("idx", idx), ("w", w), ("z", z), ("c", c),
                       ("mid", mid), ("out", out)):
            res[k_].append(v_)
    return {k: (np.concatenate(v) if v else None) for k, v in res.items()}


def topk_gap(logits: np.ndarray, top_k: int) -> np.ndarray:
    """Per row, the gap between the k-th and (k+1)-th largest logit (inf if k == E).

    A GPU/CPU routing difference can only come from a row whose gap is within
    the two sides' fp32 summation error."""
    if top_k >= logits.shape[1]:
        return np.full(logits.shape[0], np.inf)
    srt = -np.sort(-logits, axis=1)
    return srt[:, top_k - 1] - srt[:, top_k]


def brute_force(x, params: Dict, top_k: int, eps: float = 1e-5):
    """Pure-Python loops, per token, in the reference's per-slot grouping.
    Tiny shapes only. Returns out as a (T, d_out) float list of lists."""
    p = _np(params)
    X = np.asarray(x.detach().cpu().float().numpy() if hasattr(x, "detach") else x, np.float64)
    Wr, U_in, g = p["router.weight"].tolist(), p["U_in"].tolist(), p["inner_norm.weight"].tolist()
    U_exp, core = p["U_expert"].tolist(), p["core"].tolist()
    U_out, bias = p["U_out"].tolist(), p["bias"].tolist()
    E, d_in = len(Wr), len(Wr[0])
    r1, r3, r2 = len(core), len(core[0]), len(core[0][0])
    d_out = len(bias)
    outs = []
    for xt in X.reshape(-1, d_in).tolist():
        s = [sum(xt[i] * Wr[e][i] for i in range(d_in)) for e in range(E)]
        order = sorted(range(E), key=lambda e: (-s[e], e))[:top_k]
        m = s[order[0]]
        ex = [math.exp(s[e] - m) for e in order]
        tot = sum(ex)
        wts = [v / tot for v in ex]
        zr = [sum(xt[i] * U_in[i][q] for i in range(d_in)) for q in range(r3)]
        rms = math.sqrt(sum(v * v for v in zr) / r3 + eps)
        z = [zr[q] / rms * g[q] for q in range(r3)]
        mid = [0.0] * r2
        for j, e in enumerate(order):
            G = [[sum(U_exp[e][r] * core[r][q][t] for r in range(r1)) for t in range(r2)]
                 for q in range(r3)]
            for t in range(r2):
                mid[t] += wts[j] * sum(z[q] * G[q][t] for q in range(r3))
        outs.append([sum(mid[t] * U_out[t][o] for t in range(r2)) + bias[o] for o in range(d_out)])
    return outs


def rel_l2(a, b) -> float:
    """||a - b|| / ||b|| in float64."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))
