"""The training layer's router, temperature schedule and lb / z losses
(sft_cot_bundle/scripts/model.py:114-120, :313-344): the float64 oracle
(oracle/train_router_np.py) pinned by closed forms, a pure-Python brute force and
planted mistakes; then the product's TuckerMoETrain expressions (latent.py) checked
against the oracle on the CPU (the latent contraction as a torch expression)."""
import math

import numpy as np
import pytest
import torch

from oracle import train_router_np as tr


# ---- the oracle, pinned --------------------------------------------------------

def test_temperature_endpoints():
    assert tr.temperature(None) == 0.5                 # no step: t_end
    assert tr.temperature(0) == pytest.approx(2.0)     # before warmup: t_start
    assert tr.temperature(500) == pytest.approx(2.0)
    assert tr.temperature(10000) == pytest.approx(0.5)
    assert tr.temperature(10 ** 6) == pytest.approx(0.5)
    assert tr.temperature((500 + 10000) / 2) == pytest.approx(1.25)   # cos(pi/2) = 0
    ts = [tr.temperature(s) for s in range(0, 12000, 250)]
    assert all(a >= b for a, b in zip(ts, ts[1:]))     # monotone cooling


def test_scaled_tanh_closed_forms():
    x = np.linspace(-200, 200, 4001)
    y = tr.scaled_tanh(x)
    assert np.allclose(y, -tr.scaled_tanh(-x)) and tr.scaled_tanh(0.0) == 0.0
    h = 1e-6
    assert (tr.scaled_tanh(h) - tr.scaled_tanh(-h)) / (2 * h) == pytest.approx(1.0, rel=1e-9)
    assert np.all(np.abs(y) <= 10.0) and tr.scaled_tanh(200.0) == pytest.approx(10.0, rel=1e-12)
    assert np.all(np.abs(tr.scaled_tanh(np.linspace(-50, 50, 101))) < 10.0)


@pytest.mark.parametrize("E,k", [(8, 1), (8, 2), (16, 3)])
def test_uniform_router_closed_forms(E, k):
    """Equal logits: uniform probabilities, the k lowest indices selected, each top
    probability (1/E) / (k/E + 1e-6), lb = E * k * (1/E) = k; zero logits give
    z = log(E)^2."""
    raw = np.zeros((5, E))
    r = tr.route(raw, k, 0.5, training=True)
    assert np.allclose(r["probs"], 1.0 / E)
    assert np.array_equal(r["idx"], np.tile(np.arange(k), (5, 1)))
    assert np.allclose(r["top_p"], (1.0 / E) / (k / E + 1e-6))
    assert r["lb_loss"] == pytest.approx(k)
    assert r["z_loss"] == pytest.approx(math.log(E) ** 2)


def test_all_experts_selected_closed_forms():
    """k = E: every expert selected, lb = E whatever the logits, top_p = probs /
    (1 + 1e-6)."""
    g = np.random.default_rng(4)
    raw = g.normal(size=(40, 6)) * 5
    r = tr.route(raw, 6, 0.7, training=True)
    assert r["lb_loss"] == pytest.approx(6.0)
    got = np.take_along_axis(r["top_p"], np.argsort(r["idx"], -1), -1)
    assert np.allclose(got, r["probs"] / (1 + 1e-6))


def test_eval_mode_has_no_losses():
    r = tr.route(np.random.default_rng(1).normal(size=(7, 8)), 2, 0.5, training=False)
    assert r["lb_loss"] == 0.0 and r["z_loss"] == 0.0


def test_route_matches_bruteforce():
    g = np.random.default_rng(11)
    for E, k, temp in ((8, 2, 0.5), (12, 3, 1.7), (5, 5, 2.0)):
        raw = g.normal(size=(23, E)) * 8
        r = tr.route(raw, k, temp, training=True)
        idx, top_p, lb, z = tr.route_bruteforce(raw, k, temp)
        assert np.array_equal(r["idx"], idx)
        assert np.allclose(r["top_p"], top_p, rtol=1e-12, atol=0)
        assert r["lb_loss"] == pytest.approx(lb, rel=1e-6)   # float32-cast probabilities
        assert r["z_loss"] == pytest.approx(z, rel=1e-12)


def _mutants():
    """Plausible mistakes in the router, each a function like tr.route."""
    def no_E(raw, k, t, training):
        r = tr.route(raw, k, t, training)
        r["lb_loss"] /= raw.shape[1]
        return r

    def z_no_square(raw, k, t, training):
        r = tr.route(raw, k, t, training)
        r["z_loss"] = float(np.mean(tr._logsumexp(tr.scaled_tanh(raw))))
        return r

    def temp_inside_cap(raw, k, t, training):
        return tr.route(np.asarray(raw) / t * 1.0, k, 1.0, training) if t != 1.0 else None

    def no_eps(raw, k, t, training):
        r = tr.route(raw, k, t, training)
        top = r["top_p"] * (r["top_p"].sum(-1, keepdims=True) * 0 + 1)
        r["top_p"] = top / top.sum(-1, keepdims=True)
        return r

    def softmax_over_topk(raw, k, t, training):
        r = tr.route(raw, k, t, training)
        lg = tr.scaled_tanh(raw) / t
        v = np.take_along_axis(lg, r["idx"], -1)
        e = np.exp(v - v.max(-1, keepdims=True))
        r["top_p"] = e / e.sum(-1, keepdims=True)
        return r

    def lb_on_logits(raw, k, t, training):
        r = tr.route(raw, k, t, training)
        mask = np.zeros_like(r["probs"])
        np.put_along_axis(mask, r["idx"], 1.0, -1)
        r["lb_loss"] = float(raw.shape[1] * np.sum(mask.mean(0) * (tr.scaled_tanh(raw) / t).mean(0)))
        return r
    return [no_E, z_no_square, temp_inside_cap, no_eps, softmax_over_topk, lb_on_logits]


@pytest.mark.parametrize("mut", _mutants(), ids=lambda f: f.__name__)
def test_planted_mistakes_are_caught(mut):
    """Each mistake fails the closed forms or the brute force."""
    g = np.random.default_rng(2)
    failed = False
    for E, k, temp in ((8, 2, 0.5), (6, 6, 0.7)):
        raw = g.normal(size=(19, E)) * 6
        r = mut(raw, k, temp, True)
        idx, top_p, lb, z = tr.route_bruteforce(raw, k, temp)
        failed |= (not np.array_equal(r["idx"], idx) or not np.allclose(r["top_p"], top_p, rtol=1e-9)
                   or abs(r["lb_loss"] - lb) > 1e-6 * abs(lb) or abs(r["z_loss"] - z) > 1e-9 * abs(z))
    raw0 = np.zeros((4, 8))
    r = mut(raw0, 2, 0.5, True)
    failed |= abs(r["lb_loss"] - 2.0) > 1e-6 or abs(r["z_loss"] - math.log(8) ** 2) > 1e-9
    assert failed


# ---- the product's expressions against the oracle ------------------------------

def _latent_torch(xs, G, idx, p):
    out = 0
    for j in range(idx.shape[1]):
        out = out + p[:, j:j + 1] * torch.einsum("bs,bsq->bq", xs, G[idx[:, j]])
    return out


@pytest.mark.parametrize("step", [None, 0, 700, 5250, 20000])
@pytest.mark.parametrize("training", [True, False])
def test_training_layer_matches_oracle(pkg, step, training):
    import mamba_tuckermoe_amd.latent as lat
    torch.manual_seed(3)
    m = pkg.TuckerMoETrain(64, 48, num_experts=8, top_k=2, r1=4, r2=64, r3=64).double()
    with torch.no_grad():
        m.router.weight.mul_(300.0)        # logits of tens: the cap saturates for some
        m.inner_norm.weight.copy_(1 + 0.1 * torch.randn(64, dtype=torch.float64))
        m.bias.copy_(0.1 * torch.randn(48, dtype=torch.float64))
    m.train(training)
    x = torch.randn(3, 17, 64, dtype=torch.float64)
    orig = lat.FusedLatentMoE.apply
    lat.FusedLatentMoE.apply = staticmethod(_latent_torch)
    try:
        with torch.no_grad():
            out, lb, zl = m(x, step=step)
    finally:
        lat.FusedLatentMoE.apply = orig
    params = dict(m.state_dict())
    ref, lb_r, z_r = tr.layer_forward(x, params, 2, step=step, training=training)
    # the temperature is float32 in both (model.py:116): float32 cos may differ by an ulp
    assert np.allclose(out.numpy(), ref, rtol=1e-6, atol=1e-9)
    # lb averages float32-cast probabilities (model.py:331): float32 summation order
    assert float(lb) == pytest.approx(lb_r, rel=1e-6, abs=0)
    assert float(zl) == pytest.approx(z_r, rel=1e-12, abs=0)   # before the temperature
    assert float(pkg.latent.router_temperature(step)) == pytest.approx(tr.temperature(step), rel=1e-6)
    v = torch.linspace(-300, 300, 601, dtype=torch.float64)
    assert np.allclose(pkg.latent.scaled_tanh(v).numpy(), tr.scaled_tanh(v.numpy()), rtol=1e-12,
                       atol=1e-12)
