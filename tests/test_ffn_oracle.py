"""Pins the FFN sub-block oracle (oracle/tucker_ffn_torch.py) on the CPU.

The reference ships no vectors for TransformerBlock's FFN (model.py:337-341), so
the torch restatement is pinned by: the float64 formulation written from the
mathematics (oracle/tucker_ffn_np.py); torch's own RMSNorm and SiLU routines;
closed forms that hold when the TuckerMoE cores are zero (each layer's output is
then exactly its bias); the LayerScale identity gamma = 0; and planted
mistakes, each of which at least one check must catch.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import tucker_ffn_np as fnp
from oracle import tucker_ffn_torch as ft
from oracle import tucker_moe_np as onp
from oracle import tucker_moe_torch as tm


@pytest.fixture(scope="module")
def f0(pkg):
    f = pkg.FFN_WORKLOADS["F0"]
    return f, pkg.synth.make_ffn_params(f), pkg.synth.make_ffn_x(f, 48)


def _routing_stable(ref64, k, bound=1e-3):
    """Rows whose top-k is separated by more than `bound` times the logits'
    standard deviation in every layer. bf16 rounding of a layer input moves a
    logit by about 1e-3 of that deviation, so bf16 checks use bound = 1e-2."""
    keep = None
    for lg in ref64["logits"].values():
        ok = onp.topk_gap(lg, k) > bound * lg.std()
        keep = ok if keep is None else keep & ok
    return keep


def check_suite(forward, f, p, x):
    """(name, passed) for each pinning check of an FFN forward(x, params, k)."""
    res = []
    ref = fnp.ffn_forward_f64(x, p, f.k)
    out = forward(x, p, f.k)
    keep = _routing_stable(ref, f.k)
    res.append(("routing-stable rows", keep.mean() > 0.9))
    res.append(("f64 agreement", onp.rel_l2(out.double().numpy()[keep], ref["out"][keep]) < 1e-5))
    # zero cores: every TuckerMoE returns its bias exactly, so
    #   h = silu(b_gate) * b_up and out = x + gamma * b_down
    pz = dict(p)
    for name in ("ffn_gate", "ffn_up", "ffn_down"):
        pz[f"{name}.core"] = torch.zeros_like(p[f"{name}.core"])
    oz = forward(x, pz, f.k).double()
    bg, bu, bd = (p[f"{n}.bias"].double() for n in ("ffn_gate", "ffn_up", "ffn_down"))
    g64 = p["ls_ffn.gamma"].double()
    closed = x.double() + g64 * bd
    res.append(("zero-core closed form", onp.rel_l2(oz, closed) < 1e-6))
    # gamma = 0: the sub-block is the identity (exactly)
    p0 = dict(p)
    p0["ls_ffn.gamma"] = torch.zeros_like(p["ls_ffn.gamma"])
    res.append(("gamma = 0 identity", torch.equal(forward(x, p0, f.k), x.to(out.dtype))))
    return res


def test_oracle_pinned(f0):
    f, p, x = f0
    fwd = lambda x_, p_, k: ft.ffn_forward(x_, p_, k)
    for name, ok in check_suite(fwd, f, p, x):
        assert ok, name


def test_oracle_intermediates_closed_form(f0):
    """With zero gate/up cores, h is silu(b_gate) * b_up, stated through torch's
    sigmoid (x * sigmoid(x)) rather than F.silu."""
    f, p, x = f0
    pz = dict(p)
    for name in ("ffn_gate", "ffn_up"):
        pz[f"{name}.core"] = torch.zeros_like(p[f"{name}.core"])
    r = ft.ffn_forward(x, pz, f.k, intermediates=True)
    bg, bu = p["ffn_gate.bias"].double(), p["ffn_up.bias"].double()
    h = (bg * torch.sigmoid(bg) * bu).expand(x.shape[0], -1)
    assert onp.rel_l2(r["h"].double(), h) < 1e-6
    assert torch.equal(r["gate"], p["ffn_gate.bias"].expand(x.shape[0], -1))


def test_rmsnorm_matches_torch_routine(f0):
    f, p, x = f0
    w = p["norm_ffn.weight"]
    ours = tm.rmsnorm(x, w, 1e-5)
    lib = F.rms_norm(x, (x.shape[-1],), w, 1e-5)
    assert (ours - lib).abs().max() < 1e-5
    # a constant row c * 1 normalises to sign(c) * w (eps = 0)
    c = torch.full((1, x.shape[-1]), -3.0)
    assert torch.allclose(tm.rmsnorm(c, w, 0.0)[0], -w, atol=1e-6)


PLANTED = {
    "no silu": dict(stages={"silu": lambda v: v}),
    "no residual": dict(stages={"residual": lambda x, s: s}),
    "no norm": dict(stages={"rmsnorm": lambda x, w, eps: x * w}),
    "gate/up swapped": dict(swap=True),
    "gamma dropped": dict(gamma_one=True),
    "sigmoid for silu": dict(stages={"silu": torch.sigmoid}),
}


@pytest.mark.parametrize("name", list(PLANTED))
def test_planted_mistake_is_caught(f0, name):
    f, p, x = f0
    spec = PLANTED[name]

    def fwd(x_, p_, k):
        q = dict(p_)
        if spec.get("swap"):
            for key in [kk for kk in p_ if kk.startswith("ffn_gate.")]:
                up = "ffn_up." + key[len("ffn_gate."):]
                q[key], q[up] = p_[up], p_[key]
        if spec.get("gamma_one"):
            q["ls_ffn.gamma"] = torch.ones_like(p_["ls_ffn.gamma"])
        return ft.ffn_forward(x_, q, k, stages=spec.get("stages"))

    failed = [n for n, ok in check_suite(fwd, f, p, x) if not ok]
    assert failed, f"planted mistake {name!r} passed every check"


def test_bf16_oracle_mode_rounds_at_module_outputs(pkg):
    """bf16 parameters, fp32 compute: every intermediate holds bf16 values and
    the result is within the bf16 bar of the float64 formulation."""
    f = pkg.FFN_WORKLOADS["F0"]
    p = pkg.synth.make_ffn_params(f, dtype=torch.bfloat16)
    x = pkg.synth.make_ffn_x(f, 32, dtype=torch.bfloat16)
    r = ft.ffn_forward(x, p, f.k, compute_dtype=torch.float32, intermediates=True)
    for key in ("x_f", "gate", "up", "h", "dn"):
        v = r[key]
        assert torch.equal(v, v.to(torch.bfloat16).float()), key
    ref = fnp.ffn_forward_f64(x, p, f.k)
    keep = _routing_stable(ref, f.k, bound=1e-2)
    assert keep.mean() > 0.8
    assert onp.rel_l2(r["out"].double().numpy()[keep], ref["out"][keep]) < 1e-2
