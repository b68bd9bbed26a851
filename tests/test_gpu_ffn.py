"""Parity of the FFN sub-block path (TuckerFFN / TuckerOutProj: tmoe_rmsnorm_rows
and tmoe_forward_epi's fused epilogues) with the CPU oracle.

Each stage is checked on the GPU's own input to that stage, so a routing
decision is compared on identical inputs (bit-exact, as for the layer):
  x_f = RMSNorm(x)                          vs float64
  gate = ffn_gate(x_f)                      vs float64 layer on the GPU's x_f
  h = silu(gate) * ffn_up(x_f)              vs float64 on the GPU's x_f
  out = x + gamma * ffn_down(h)             vs float64 on the GPU's h
plus the end-to-end result against oracle/tucker_ffn_np (unrounded float64) on
the rows routed alike in all three layers; a row routed differently must be a
near-tie there, and such rows at most 3% (or 2 rows). Bars: rel-L2 <= 1e-5 (fp32) and
<= 1e-2 (bf16); the residual increment out - x alone within twice that (bf16).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import tucker_ffn_np as fnp
from oracle import tucker_ffn_torch as ft
from oracle import tucker_moe_np as onp

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}
LAYERS = ("ffn_gate", "ffn_up", "ffn_down")


def _ffn(pkg, dev, f, params):
    m = pkg.TuckerFFN(f.d, f.cfg()).to(dev, f.dtype)
    m.load_state_dict({k: v.to(dev) for k, v in params.items()})
    return m


def _f64(t):
    return t.detach().double().cpu().numpy()


def _layer_check(m, name, inp, params, k, dtype, label):
    """The GPU layer's routing on `inp` equals the float64 oracle's; returns the
    oracle's output for `inp`."""
    sub = ft.layer_params(params, name)
    ref = onp.forward_f64(inp.float().cpu(), sub, k)
    with torch.no_grad():
        _, idx, _, _ = getattr(m, name).forward_with_routing(inp)
    idx = idx.cpu().numpy()
    mism = np.nonzero((idx != ref["idx"]).any(1))[0]
    gaps = onp.topk_gap(ref["logits"], k)
    assert len(mism) == 0, f"{label}/{name}: routing rows {mism[:8]} gaps {gaps[mism[:8]]}"
    return ref["out"], idx


def _check_ffn(pkg, dev, f, T, affine="random", label=""):
    params = pkg.synth.make_ffn_params(f, affine=affine)
    x = pkg.synth.make_ffn_x(f, T).to(dev)
    m = _ffn(pkg, dev, f, params)
    with torch.no_grad():
        st = m.stages(x)
        y = m(x)
    torch.cuda.synchronize()
    tol = TOL[f.dtype]
    X = _f64(x)
    g = _f64(params["norm_ffn.weight"])
    gamma = _f64(params["ls_ffn.gamma"])
    xf64 = X / np.sqrt(np.mean(X * X, axis=1, keepdims=True) + 1e-5) * g
    errs = {"x_f": onp.rel_l2(_f64(st["x_f"]), xf64)}
    gate64, i_gate = _layer_check(m, "ffn_gate", st["x_f"], params, f.k, f.dtype, label)
    up64, i_up = _layer_check(m, "ffn_up", st["x_f"], params, f.k, f.dtype, label)
    errs["gate"] = onp.rel_l2(_f64(st["gate"]), gate64)
    errs["h"] = onp.rel_l2(_f64(st["h"]), gate64 / (1 + np.exp(-gate64)) * up64)
    dn64, i_down = _layer_check(m, "ffn_down", st["h"], params, f.k, f.dtype, label)
    errs["out"] = onp.rel_l2(_f64(st["out"]), X + gamma * dn64)
    # the residual increment alone (out - x), so that x does not mask it
    errs["increment"] = onp.rel_l2(_f64(st["out"]) - X, gamma * dn64)
    # End to end against the unrounded float64 sub-block. The GPU's layer inputs
    # (x_f; h) differ from the float64 ones by the dtype's rounding, which moves
    # the router logits by d_in = (input_gpu - input_f64) @ W_r^T. A row may route
    # differently only where the float64 top-k gap is within 2 max|d_in| of the
    # row (both sides of the gap move); such rows must also be few. The rest meet
    # the bar.
    ref = fnp.ffn_forward_f64(x.float().cpu(), params, f.k)
    flip = np.zeros(T, bool)
    near = np.zeros(T, bool)
    for name, got_idx, inp in (("ffn_gate", i_gate, "x_f"), ("ffn_up", i_up, "x_f"),
                               ("ffn_down", i_down, "h")):
        lg = ref["logits"][name]
        moved = (_f64(st[inp]) - ref[inp]) @ _f64(params[f"{name}.router.weight"]).T
        # the selected set (an order swap inside the top-k changes no output)
        flip |= (np.sort(got_idx, 1) != np.sort(ref["idx"][name], 1)).any(1)
        near |= onp.topk_gap(lg, f.k) <= 2 * np.abs(moved).max(1) + 1e-5 * lg.std()
    keep = ~flip
    errs["end_to_end"] = onp.rel_l2(_f64(y)[keep], ref["out"][keep])
    print(f"{label} T={T} flipped={flip.sum()} near_ties={near.sum()} " +
          " ".join(f"{k}={v:.3e}" for k, v in errs.items()), flush=True)
    assert torch.equal(y, st["out"]), "forward() and stages() differ"
    assert not (flip & ~near).any(), f"rows routed differently without a near-tie: " \
                                     f"{np.nonzero(flip & ~near)[0][:8]}"
    assert flip.sum() <= max(2, 0.03 * T), flip.sum()   # measured: ~1.5% of rows (bf16)
    inc_tol = tol if f.dtype == torch.float32 else 2 * tol
    for k_, v in errs.items():
        assert v <= (inc_tol if k_ == "increment" else tol), (label, k_, v)


@pytest.mark.parametrize("T", [64, 300])
def test_ffn_fp32(pkg, dev, T):
    """fp32: T = 64 takes the small-T kernels (epilogue in k_sk_out), T = 300
    the tiled out-projection (epilogue in its LDS flush)."""
    _check_ffn(pkg, dev, pkg.FFN_WORKLOADS["F0"], T, label="F0")


@pytest.mark.parametrize("T", [100, 1024])
@pytest.mark.parametrize("name", ["F1", "F2"])
def test_ffn_bf16_reference_dims(pkg, dev, name, T):
    """The reference block's dims (d 768, d_ff 4608, E 8, k 2, r2 512, r3 256)
    with r1 = 32 (F1) and r1 = 4 (F2, the persistent core)."""
    _check_ffn(pkg, dev, pkg.FFN_WORKLOADS[name], T, label=name)


def test_ffn_full_size(pkg, dev):
    """F2 at its full T = 4096 (the persistent out-projection's staged flush)."""
    f = pkg.FFN_WORKLOADS["F2"]
    _check_ffn(pkg, dev, f, f.T, affine="unit", label="F2/full")


@pytest.mark.parametrize("T", [1, 37, 257])
def test_ffn_ragged(pkg, dev, T):
    _check_ffn(pkg, dev, pkg.FFN_WORKLOADS["F2"], T, label="F2/ragged")


@pytest.mark.parametrize("name,T", [("F0", 64), ("F0", 300), ("F2", 100), ("F2", 600)])
def test_gamma_zero_is_identity_and_inplace(pkg, dev, name, T):
    """gamma = 0 returns x exactly (the residual path adds an exact zero), and
    inplace=True gives the out-of-place result bit for bit."""
    f = pkg.FFN_WORKLOADS[name]
    params = pkg.synth.make_ffn_params(f)
    x = pkg.synth.make_ffn_x(f, T).to(dev)
    m = _ffn(pkg, dev, f, params)
    with torch.no_grad():
        y = m(x)
        x2 = x.clone()
        r = m(x2, inplace=True)
        assert r.data_ptr() == x2.data_ptr() and torch.equal(x2, y)
        m.ls_ffn.gamma.zero_()
        assert torch.equal(m(x), x)


@pytest.mark.parametrize("name,T", [("F0", 64), ("F0", 300), ("F2", 100), ("F2", 600)])
def test_zero_core_closed_form(pkg, dev, name, T):
    """Zero cores: each TuckerMoE returns its bias, so h = R(R(silu(b_gate)) * b_up)
    (torch's silu on the CPU, rounded like the kernel) and out = R(x + R(gamma * b_down)).
    The kernel's silu (g / (1 + expf(-g))) and torch's differ by a few fp32
    units in the last place: after rounding to bf16 at most one bf16 unit, on at
    most 2% of the elements; in fp32 at most 8 units."""
    f = pkg.FFN_WORKLOADS[name]
    params = pkg.synth.make_ffn_params(f)
    for n in LAYERS:
        params[f"{n}.core"] = torch.zeros_like(params[f"{n}.core"])
    x = pkg.synth.make_ffn_x(f, T)
    m = _ffn(pkg, dev, f, params)
    with torch.no_grad():
        st = m.stages(x.to(dev))
    dt = f.dtype
    R = lambda v: v.to(dt).float()
    bg, bu, bd = (params[f"{n}.bias"].float() for n in LAYERS)
    h = R(R(F.silu(bg)) * bu).expand(T, -1)
    out = R(x.float() + R(params["ls_ffn.gamma"].float() * bd))
    assert torch.equal(st["gate"].cpu(), params["ffn_gate.bias"].expand(T, -1))
    assert torch.equal(st["out"].cpu().float(), out)

    def ulps(a, b):
        if dt == torch.bfloat16:
            ai, bi = a.to(dt).view(torch.int16).int(), b.to(dt).view(torch.int16).int()
        else:
            ai, bi = a.view(torch.int32).long(), b.view(torch.int32).long()
        return (ai - bi).abs()

    d = ulps(st["h"].cpu().float(), h)
    if dt == torch.bfloat16:
        assert d.max() <= 1 and (d > 0).float().mean() <= 0.02, (d.max(), (d > 0).float().mean())
    else:
        assert d.max() <= 8, d.max()


@pytest.mark.parametrize("d", [200, 768, 4096, 4104])
@pytest.mark.parametrize("T", [64, 301])
def test_rmsnorm_rows(pkg, dev, T, d):
    """tmoe_rmsnorm_rows against float64, in both dtypes: rows held in registers
    (16-byte multiples up to 8 KB) and the general path (d = 200 in bf16,
    d = 4104)."""
    for dt in (torch.float32, torch.bfloat16):
        g = torch.Generator().manual_seed(T)
        x = (torch.randn(T, d, generator=g) * 3).to(dt)
        w = (1 + 0.1 * torch.randn(d, generator=g)).to(dt)
        n = pkg.RMSNorm(d, eps=1e-5).to(dev, dt)
        with torch.no_grad():
            n.weight.copy_(w.to(dev))
            y = n(x.to(dev)).cpu()
        X, W = x.double(), w.double()
        ref = X / torch.sqrt((X * X).mean(-1, keepdim=True) + 1e-5) * W
        err = onp.rel_l2(y.double().numpy(), ref.numpy())
        assert err <= (1e-6 if dt == torch.float32 else 4e-3), (dt, err)


@pytest.mark.parametrize("T", [100, 600])
def test_outproj_subblock(pkg, dev, T):
    """Mamba3Block's out = mid + ls_out_proj(out_proj(norm_out_proj(mid)))
    (model.py:258-260), square d -> d TuckerMoE, against float64."""
    f = pkg.FFN_WORKLOADS["F2"]
    w = pkg.Workload("outproj", T, f.d, f.d, f.E, f.k, f.r1, f.r3, f.r2, torch.bfloat16, 31)
    lp = pkg.synth.make_params(w, affine="random")
    g = torch.Generator().manual_seed(5)
    nw = (1 + 0.1 * torch.randn(f.d, generator=g)).to(torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn(f.d, generator=g)).to(torch.bfloat16)
    sd = {f"out_proj.{k}": v for k, v in lp.items()}
    sd["norm_out_proj.weight"] = nw
    sd["ls_out_proj.gamma"] = gamma
    m = pkg.TuckerOutProj(f.d, w.cfg()).to(dev, torch.bfloat16)
    m.load_state_dict({k: v.to(dev) for k, v in sd.items()})
    x = pkg.synth.make_x(w, T).to(dev)
    with torch.no_grad():
        xn = m.norm_out_proj(x)
        y = m(x)
        x2 = x.clone()
        m(x2, inplace=True)
    assert torch.equal(x2, y)
    ref = onp.forward_f64(xn.float().cpu(), lp, f.k)
    with torch.no_grad():
        _, idx, _, _ = m.out_proj.forward_with_routing(xn)
    assert np.array_equal(idx.cpu().numpy(), ref["idx"])
    X = _f64(x)
    err = onp.rel_l2(_f64(y) - X, _f64(gamma) * ref["out"])
    assert err <= 2e-2, err
    assert onp.rel_l2(_f64(y), X + _f64(gamma) * ref["out"]) <= 1e-2


@pytest.mark.parametrize("T", [100, 2048, 4096])
@pytest.mark.parametrize("same_plan", [True, False])
@pytest.mark.parametrize("d_ff", [None, 512], ids=["F2", "folded"])
def test_glu_pair_equals_two_calls(pkg, dev, T, same_plan, d_ff):
    """tmoe_forward_glu (both fronts in one launch) gives, bit for bit, tmoe_forward of
    the gate then tmoe_forward_epi(GLU) of the up; layers whose plans differ (here r1)
    take the two-call path inside glu_pair. d_ff = 512 makes the same-rank plans take
    the folded form (W = core U_out: 1024 x 512 against 4 x 256 x 512 + 512 x 512)."""
    f = pkg.FFN_WORKLOADS["F2"]
    dff = d_ff or f.d_ff
    wg = pkg.Workload("g", T, f.d, dff, f.E, f.k, f.r1, f.r3, f.r2, torch.bfloat16, 41)
    wu = pkg.Workload("u", T, f.d, dff, f.E, f.k, f.r1 if same_plan else 2 * f.r1, f.r3,
                      f.r2, torch.bfloat16, 42)
    mods = []
    for w in (wg, wu):
        m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg()).to(dev, torch.bfloat16)
        m.load_state_dict({k: v.to(dev) for k, v in pkg.synth.make_params(w).items()})
        mods.append(m)
    x = pkg.synth.make_x(wg, T).to(dev)
    with torch.no_grad():
        h = pkg.block.glu_pair(mods[0], mods[1], x)
        g = mods[0](x)
        ref = mods[1].forward_raw(x, epi=pkg._lib.TMOE_EPI_GLU, epi_a=g)[0]
    torch.cuda.synchronize()
    assert mods[0].plan().folded() == (d_ff is not None)
    assert torch.equal(h, ref)
