"""float64 restatement of the reference training layer's router, temperature
schedule and auxiliary losses — TEST INFRASTRUCTURE.

The reference trains with TritonTuckerMoE (sft_cot_bundle/scripts/model.py:292-340):
  get_router_temperature(step)            model.py:114-120 (cosine from t_start to
                                          t_end over steps warmup .. total; t_end
                                          when no step is given)
  capped   = fast_scaled_tanh(raw, 10)    model.py:318-319 (10 tanh(raw / 10))
  z_loss   = mean(logsumexp(capped)^2)    model.py:321 (training only, else 0)
  logits   = capped / temperature         model.py:323
  probs    = softmax(logits)              model.py:324
  idx      = topk(logits, k)              model.py:326
  top_p    = probs[idx] / (sum + 1e-6)    model.py:327-328
  lb_loss  = E sum_e mean_b(mask)[e] mean_b(float32(probs))[e]   model.py:330-332
                                          (training only)
  x_shared = RMSNorm(x U_in)              model.py:336-337
  G        = einsum(U_expert, core)       model.py:339
  out      = FusedLatentMoE(x_shared, G, idx, top_p) U_out + bias   model.py:340-344
This module restates those expressions in numpy float64 (top-k by a stable sort:
larger first, the lower index on ties) with the latent contraction of
oracle/latent_np.py. Only tests import it.
"""
from __future__ import annotations

import numpy as np

from . import latent_np


def temperature(step, warmup: int = 500, total: int = 10000, t_start: float = 2.0,
                t_end: float = 0.5) -> float:
    """model.py:114-120, in float32 arithmetic as there (the step becomes a float32
    tensor, model.py:116); t_end itself when no step is given."""
    if step is None:
        return t_end
    f = np.float32
    s = f(step)
    progress = np.clip((s - f(warmup)) / f(max(1, total - warmup)), f(0.0), f(1.0))
    return float(f(t_end) + f(0.5 * (t_start - t_end)) * (f(1.0) + np.cos(f(np.pi) * progress)))


def scaled_tanh(x, scale: float = 10.0) -> np.ndarray:
    """scale * tanh(x / scale) (model.py:22-64's fast_scaled_tanh, as a function)."""
    return scale * np.tanh(np.asarray(x, np.float64) / scale)


def _logsumexp(a: np.ndarray) -> np.ndarray:
    m = a.max(-1, keepdims=True)
    return (m + np.log(np.exp(a - m).sum(-1, keepdims=True)))[..., 0]


def route(raw, k: int, temp: float, training: bool):
    """The router of model.py:318-332 on raw logits (B, E): dict of capped, probs,
    idx (B, k) (descending logit, lower index on ties), top_p (B, k), lb_loss and
    z_loss (0.0 when not training)."""
    raw = np.asarray(raw, np.float64)
    B, E = raw.shape
    capped = scaled_tanh(raw, 10.0)
    z_loss = float(np.mean(_logsumexp(capped) ** 2)) if training else 0.0
    logits = capped / temp
    e = np.exp(logits - logits.max(-1, keepdims=True))
    probs = e / e.sum(-1, keepdims=True)
    idx = np.argsort(-logits, axis=-1, kind="stable")[:, :k]
    top = np.take_along_axis(probs, idx, -1)
    top_p = top / (top.sum(-1, keepdims=True) + 1e-6)
    lb_loss = 0.0
    if training:
        mask = np.zeros((B, E))
        np.put_along_axis(mask, idx, 1.0, -1)
        # the reference averages router_probs.float(): the probabilities cast to
        # float32 whatever the module's dtype (model.py:331)
        lb_loss = float(E * np.sum(mask.mean(0) * probs.astype(np.float32).astype(np.float64).mean(0)))
    return {"capped": capped, "probs": probs, "idx": idx, "top_p": top_p,
            "lb_loss": lb_loss, "z_loss": z_loss}


def layer_forward(x, params, k: int, step=None, training: bool = True, eps: float = 1e-5):
    """(out, lb_loss, z_loss) of TritonTuckerMoE.forward (model.py:313-344) in float64.
    params: router.weight (E, d_in), U_in (d_in, r3), inner_norm.weight (r3),
    U_expert (E, r1), core (r1, r3, r2), U_out (r2, d_out), bias (d_out)."""
    P = {n: np.asarray(v.detach().double().numpy() if hasattr(v, "detach") else v, np.float64)
         for n, v in params.items()}
    X = np.asarray(x.detach().double().numpy() if hasattr(x, "detach") else x, np.float64)
    lead = X.shape[:-1]
    xf = X.reshape(-1, X.shape[-1])
    r = route(xf @ P["router.weight"].T, k, temperature(step), training)
    xs = xf @ P["U_in"]
    xs = xs / np.sqrt(np.mean(xs * xs, -1, keepdims=True) + eps) * P["inner_norm.weight"]
    G = np.einsum("er,rst->est", P["U_expert"], P["core"])
    core = latent_np.forward(xs, G, r["idx"], r["top_p"])
    out = (core @ P["U_out"]).reshape(*lead, -1) + P["bias"]
    return out, r["lb_loss"], r["z_loss"]


def route_bruteforce(raw, k: int, temp: float):
    """Pure-Python loops of the same router (small cases): (idx, top_p, lb, z)."""
    raw = [[float(v) for v in row] for row in np.asarray(raw, np.float64)]
    B, E = len(raw), len(raw[0])
    import math
    idx, top_p, lse2, mask_cnt, prob_sum = [], [], 0.0, [0.0] * E, [0.0] * E
    for row in raw:
        cap = [10.0 * math.tanh(v / 10.0) for v in row]
        mx = max(cap)
        lse2 += (mx + math.log(sum(math.exp(c - mx) for c in cap))) ** 2
        lg = [c / temp for c in cap]
        m2 = max(lg)
        ex = [math.exp(v - m2) for v in lg]
        s = sum(ex)
        pr = [v / s for v in ex]
        order = sorted(range(E), key=lambda e: (-lg[e], e))[:k]
        tot = sum(pr[e] for e in order)
        idx.append(order)
        top_p.append([pr[e] / (tot + 1e-6) for e in order])
        for e in order:
            mask_cnt[e] += 1.0
        for e in range(E):
            prob_sum[e] += pr[e]
    lb = E * sum((mask_cnt[e] / B) * (prob_sum[e] / B) for e in range(E))
    return np.array(idx), np.array(top_p), lb, lse2 / B
