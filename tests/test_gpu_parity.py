"""Parity of the gfx950 path (through the C ABI) with the CPU oracle.

Bar (north star): top-k indices bit-exact; outputs within rel-L2 <= 1e-5 (fp32)
and <= 1e-2 (bf16) of the reference's PyTorch path. For bf16 workloads the
reference path is run in float32 on the bf16-valued inputs (fp32 router logits),
which is oracle/tucker_moe_torch.forward(compute_dtype=float32).
"""
import dataclasses

import numpy as np
import pytest
import torch

from oracle import e4m3
from oracle import tucker_moe_np as onp
from oracle import tucker_moe_torch as ot

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def _module(pkg, dev, w, params, fold=True):
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg()).to(dev, w.dtype)
    m.load_state_dict({k: v.to(dev) for k, v in params.items()})
    return m.set_fold(fold)


def _run(m, x, dev):
    with torch.no_grad():
        out, idx, wts, lg = m.forward_with_routing(x.to(dev), logits=True)
    torch.cuda.synchronize()
    return out.float().cpu(), idx.cpu(), wts.cpu(), lg.cpu()


def _check(w, got, ref64, label, torch_ref=None):
    out, idx, wts, lg = got
    T = out.shape[0]
    gaps = onp.topk_gap(ref64["logits"][:T], w.k)
    mism = np.nonzero((idx.numpy() != ref64["idx"][:T]).any(1))[0]
    lg_err = onp.rel_l2(lg.numpy(), ref64["logits"][:T])
    err64 = onp.rel_l2(out.numpy(), ref64["out"][:T])
    msg = (f"{label}: T={T} rel_l2(out, f64)={err64:.3e} rel_l2(logits)={lg_err:.3e} "
           f"min_topk_gap={gaps.min():.3e} routing_mismatch_rows={len(mism)}")
    if torch_ref is not None:
        n = torch_ref["out"].shape[0]
        err_t = onp.rel_l2(out[:n].numpy(), torch_ref["out"].double().numpy())
        same_t = torch.equal(idx[:n], torch_ref["idx"])
        msg += f" rel_l2(out, torch fp32 ref)={err_t:.3e} routing_equal_torch={same_t}"
    print(msg, flush=True)
    assert len(mism) == 0, f"{msg}; rows {mism[:8]} gaps {gaps[mism[:8]]}"
    assert lg_err < (1e-6 if w.dtype == torch.float32 else 1e-5), msg
    assert np.abs(wts.numpy() - ref64["w"][:T]).max() < 1e-5, msg
    assert err64 <= TOL[w.dtype], msg
    if torch_ref is not None:
        assert same_t and err_t <= TOL[w.dtype], msg


# fold=False keeps the core and the out-projection as two GEMMs (TMOE_FLAG_NO_FOLD);
# the default lets the library fold them (bf16 plans of these shapes at T > 256)
@pytest.mark.parametrize("fold", [True, False], ids=["fold", "nofold"])
@pytest.mark.parametrize("name,T", [("C1", 64), ("C2", 32), ("C3", 1024), ("C4", 512)])
@pytest.mark.parametrize("affine", ["unit", "random"])
def test_workload_parity(pkg, dev, name, T, affine, fold):
    w = pkg.WORKLOADS[name]
    params = pkg.synth.make_params(w, affine=affine)
    x = pkg.synth.make_x(w, T)
    got = _run(_module(pkg, dev, w, params, fold), x, dev)
    ref64 = onp.forward_f64(x, params, w.k)
    tref = ot.forward(x, params, w.k, compute_dtype=torch.float32, intermediates=True)
    _check(w, got, ref64, f"{name}/{affine}/fold={fold}", tref)


@pytest.mark.parametrize("fold", [True, False], ids=["fold", "nofold"])
@pytest.mark.parametrize("name", ["C3", "C4"])
def test_full_size(pkg, dev, name, fold):
    """BASELINE's full T, against the float64 oracle on every token and the
    torch fp32 restatement on the first 512."""
    w = pkg.WORKLOADS[name]
    params = pkg.synth.make_params(w)
    x = pkg.synth.make_x(w)
    m = _module(pkg, dev, w, params, fold)
    got = _run(m, x, dev)
    assert m.plan().folded() == fold
    ref64 = onp.forward_f64(x, params, w.k)
    tref = ot.forward(x[:512], params, w.k, compute_dtype=torch.float32, intermediates=True)
    _check(w, got, ref64, f"{name}/full/fold={fold}", tref)


# The 256 x 288-tile out-projection (k_outproj_wide) runs when its tiles number at
# least one per compute unit: a ragged last row tile (whose stores the next tile
# waits for in full), d_out = 2 column tiles, and both forms.
@pytest.mark.parametrize("fold", [True, False], ids=["fold", "nofold"])
@pytest.mark.parametrize("T", [12345, 16284])
def test_wide_outproj_ragged(pkg, dev, T, fold):
    w = pkg.WORKLOADS["C3"]
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w, T, stream=5)
    m = _module(pkg, dev, w, params, fold)
    got = _run(m, x, dev)
    _check(w, got, onp.forward_f64(x, params, w.k), f"C3/T={T}/fold={fold}")


# The register-weight front (k_front_ks: bf16, r3 = 256, E_pad = 32, T past one round
# of 32-token tiles): E = 24, k = 3, d_in of 17 K tiles (the K loop's ring tail), a
# ragged last tile, both forms.
@pytest.mark.parametrize("fold", [True, False], ids=["fold", "nofold"])
def test_register_weight_front(pkg, dev, fold):
    w = pkg.Workload("custom", 9000 - 7, 1088, 288, 24, 3, 4, 256, 256, torch.bfloat16, 81)
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w)
    m = _module(pkg, dev, w, params, fold)
    got = _run(m, x, dev)
    _check(w, got, onp.forward_f64(x, params, w.k), f"ks-front/fold={fold}")


# Mid-size T: the 128 x 144-tile out-projection (k_outproj_mid, T <= 2048 at the C3
# shapes) and the 128 x 288 tiles of k_outproj_wide<1> (2048 < T <= 4096): ragged
# last row tiles, a K of 256 and two column tiles.
@pytest.mark.parametrize("fold", [True, False], ids=["fold", "nofold"])
@pytest.mark.parametrize("T", [257, 777, 2000, 2048, 3001, 4096])
def test_mid_outproj_ragged(pkg, dev, T, fold):
    w = pkg.WORKLOADS["C3"]
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w, T, stream=6)
    got = _run(_module(pkg, dev, w, params, fold), x, dev)
    _check(w, got, onp.forward_f64(x, params, w.k), f"C3/T={T}/fold={fold}")


@pytest.mark.parametrize("fold", [True, False], ids=["fold", "nofold"])
def test_mid_outproj_narrow(pkg, dev, fold):
    w = pkg.Workload("custom", 1500, 256, 288, 8, 2, 2, 128, 256, torch.bfloat16, 79)
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w)
    got = _run(_module(pkg, dev, w, params, fold), x, dev)
    _check(w, got, onp.forward_f64(x, params, w.k), f"mid narrow/fold={fold}")


@pytest.mark.parametrize("r2", [64, 128])
def test_mid_outproj_short_k(pkg, dev, r2):
    # the unfolded out-projection's K = r2: at 128, k_outproj_mid with two K tiles of
    # 64 (its prologue's short case: every tile in flight before the first wait); at
    # 64 the plan's core is k_core and its out-projection k_outproj_pp
    w = pkg.Workload("custom", 1000, 256, 288, 8, 2, 2, 128, r2, torch.bfloat16, 81)
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w)
    got = _run(_module(pkg, dev, w, params, False), x, dev)
    _check(w, got, onp.forward_f64(x, params, w.k), f"mid short K={r2}")


@pytest.mark.parametrize("fold", [True, False], ids=["fold", "nofold"])
def test_wide_outproj_narrow(pkg, dev, fold):
    # (E, k, r1, r3, r2, d_in, d_out): K = 256 either way, 2 column tiles of 288
    w = pkg.Workload("custom", 32768 - 200, 256, 576, 8, 2, 2, 128, 256, torch.bfloat16, 78)
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w)
    got = _run(_module(pkg, dev, w, params, fold), x, dev)
    _check(w, got, onp.forward_f64(x, params, w.k), f"narrow/fold={fold}")


@pytest.mark.parametrize("T", [1, 3, 63, 65, 255, 257, 1000])
@pytest.mark.parametrize("name", ["C1", "C2"])
def test_ragged_tokens(pkg, dev, name, T):
    w = pkg.WORKLOADS[name]
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w, T, stream=3)
    got = _run(_module(pkg, dev, w, params), x, dev)
    _check(w, got, onp.forward_f64(x, params, w.k), f"{name}/T={T}")


SHAPES = [
    # (E, k, r1, r3, r2, d_in, d_out)
    (1, 1, 4, 128, 256, 256, 512),      # E = k = 1: dense chain
    (16, 16, 4, 256, 512, 512, 256),    # k = E: every expert
    (32, 3, 2, 64, 128, 128, 96),       # r3 = 64, E_pad 32
    (100, 5, 8, 128, 192, 320, 160),    # E_pad 128, odd k
    (64, 4, 1, 256, 64, 64, 64),        # r1 = 1, tiny r2
    (16, 2, 1, 128, 512, 256, 128),     # r1 = 1 on the persistent core (r1 * r2 = 512)
    (8, 2, 32, 256, 512, 768, 4608),    # the reference's default ranks (config.py:20-24)
    (8, 2, 8, 128, 192, 256, 256),      # r1 = 8: persistent core in 2 rank groups
    (16, 2, 12, 256, 320, 512, 256),    # r1 = 12: 3 rank groups, 5 channel tiles
    (8, 2, 64, 64, 128, 128, 128),      # r1 = 64, E = 8: the expert form (E ranks)
    (64, 2, 64, 64, 128, 128, 128),     # r1 = 64: 16 rank groups, r3 = 64
    (4, 2, 6, 128, 192, 256, 256),      # E < r1: expert form on the persistent core (bf16)
    (3, 2, 8, 128, 192, 256, 256),      # E = 3 < r1 = 8: bf16 keeps r1 (rank groups), fp32 E
]


# T = 200 takes the small-T kernels, T = 600 the large-tile ones
@pytest.mark.parametrize("T", [200, 600])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "E%d_k%d_r%d-%d-%d_%dx%d" % s)
def test_shapes(pkg, dev, shape, dtype, T):
    E, k, r1, r3, r2, d_in, d_out = shape
    w = pkg.Workload("custom", T, d_in, d_out, E, k, r1, r3, r2, dtype, 77)
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w)
    got = _run(_module(pkg, dev, w, params), x, dev)
    _check(w, got, onp.forward_f64(x, params, w.k), f"shape {shape} {dtype}")


@pytest.mark.parametrize("fold", [True, False], ids=["fold", "nofold"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "E%d_k%d_r%d-%d-%d_%dx%d" % s)
def test_shapes_fold_choice(pkg, dev, shape, fold):
    """Large-T bf16 with the fold allowed or forbidden: the folded form where the
    library picks it (fewer multiply-adds), the two-GEMM form otherwise."""
    E, k, r1, r3, r2, d_in, d_out = shape
    w = pkg.Workload("custom", 600, d_in, d_out, E, k, r1, r3, r2, torch.bfloat16, 78)
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w)
    m = _module(pkg, dev, w, params, fold)
    got = _run(m, x, dev)
    rk = m.plan().core_rank()
    assert m.plan().folded() == (fold and rk * r3 * d_out < rk * r3 * r2 + r2 * d_out)
    _check(w, got, onp.forward_f64(x, params, w.k), f"shape {shape} fold={m.plan().folded()}")


def test_deterministic_and_batch_dims(pkg, dev):
    w = pkg.WORKLOADS["C2"]
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w, 60).to(dev)
    m = _module(pkg, dev, w, params)
    with torch.no_grad():
        a = m(x)
        b = m(x.reshape(3, 4, 5, w.d_in))
        c = m(x)
    assert b.shape == (3, 4, 5, w.d_out)
    assert torch.equal(a, c) and torch.equal(a, b.reshape(60, w.d_out))


def test_repack_after_parameter_update(pkg, dev):
    w = pkg.WORKLOADS["C1"]
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w, 16)
    m = _module(pkg, dev, w, params)
    with torch.no_grad():
        m(x.to(dev))
        m.bias.add_(1.0)      # moves the version counter: repacked automatically
        out = m(x.to(dev)).cpu()
    p2 = dict(params)
    p2["bias"] = params["bias"] + 1.0
    assert onp.rel_l2(out.numpy(), onp.forward_f64(x, p2, w.k)["out"]) < 1e-5
    m.U_out.data.mul_(0.0)    # a .data write: the tracked parameter forces a re-pack
    with torch.no_grad():
        out = m(x.to(dev)).cpu()
    assert torch.allclose(out, p2["bias"].expand_as(out))


def _load_tucker_ref_style(moe, w, pfx):
    """The reference loader's write pattern (pure_torch_mlx/weights.py:74-81):
    every weight through `param.data.copy_`, no refresh call."""
    moe.router.weight.data.copy_(w[f"{pfx}.router.weight"])
    moe.U_in.data.copy_(w[f"{pfx}.U_in"])
    moe.inner_norm.weight.data.copy_(w[f"{pfx}.inner_norm.weight"])
    moe.U_expert.data.copy_(w[f"{pfx}.U_expert"])
    moe.core.data.copy_(w[f"{pfx}.core"])
    moe.U_out.data.copy_(w[f"{pfx}.U_out"])
    moe.bias.data.copy_(w[f"{pfx}.bias"])


@pytest.mark.parametrize("name,tol", [("C1", 1e-5), ("C2", 1e-2)])
def test_reference_loader_after_forward(pkg, dev, name, tol):
    """forward, reload new weights the way the reference loader does, forward
    again: the second output is the new layer's (no stale packed weights)."""
    w = pkg.WORKLOADS[name]
    p1 = pkg.synth.make_params(w, affine="random")
    p2 = pkg.synth.make_params(dataclasses.replace(w, seed=w.seed + 17), affine="random")
    x = pkg.synth.make_x(w, 24)
    m = _module(pkg, dev, w, p1)
    with torch.no_grad():
        out1 = m(x.to(dev)).float().cpu()
        _load_tucker_ref_style(m, {f"L.{k}": v.to(dev, w.dtype) for k, v in p2.items()}, "L")
        out2, idx2, _, _ = m.forward_with_routing(x.to(dev))
    r1, r2 = onp.forward_f64(x, p1, w.k), onp.forward_f64(x, p2, w.k)
    assert onp.rel_l2(out1.numpy(), r1["out"]) < tol
    assert onp.rel_l2(out2.float().cpu().numpy(), r2["out"]) < tol
    assert np.array_equal(idx2.cpu().numpy(), r2["idx"])


def test_side_stream(pkg, dev):
    w = pkg.WORKLOADS["C2"]
    params = pkg.synth.make_params(w)
    x = pkg.synth.make_x(w, 40).to(dev)
    m = _module(pkg, dev, w, params)
    with torch.no_grad():
        ref = m(x)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            out = m(x)
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_signal_workspace_reuse_and_graph_replay(pkg, dev):
    """The E_pad = 256 front signals between its work-groups (the z work-groups wait
    for the router work-groups' c through flag words in the workspace). The result
    does not depend on what the workspace held before (0xFF bytes, random bytes, the
    flags a previous forward left), and replays of a captured graph (the same epoch
    each time) equal the eager forward."""
    w = pkg.WORKLOADS["C4"]
    T = 600
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w, T, stream=7).to(dev)
    m = _module(pkg, dev, w, params, True)
    plan, packed = m.plan(), m.packed()
    L = pkg._lib.lib()
    with torch.no_grad():
        ref = m(x)
    ws_bytes = plan.workspace_bytes(T)
    g = torch.Generator(device=dev).manual_seed(3)
    fills = [torch.full((ws_bytes,), 255, dtype=torch.uint8, device=dev),
             torch.randint(0, 256, (ws_bytes,), dtype=torch.uint8, device=dev, generator=g)]
    for ws in fills:
        for _ in range(2):   # the second call finds the first one's flags
            out = torch.empty_like(ref)
            pkg._lib.check(L.tmoe_forward(plan.ptr, x.data_ptr(), T, packed.data_ptr(),
                                          out.data_ptr(), None, None, None, ws.data_ptr(),
                                          ws_bytes, torch.cuda.current_stream().cuda_stream))
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    out_g = torch.empty_like(ref)
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(graph, stream=s):
        m.forward_raw(x, out=out_g)
    torch.cuda.synchronize()
    for _ in range(3):
        out_g.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, ref)
        with torch.no_grad():
            assert torch.equal(m(x), ref)   # eager work between the replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("T", [1, 17, 32, 64])
def test_decode_one_launch_workspace_and_graph(pkg, dev, T):
    """Decode-sized folded forwards run as one launch whose out-projection
    work-groups wait for the front's work-groups (flags in the workspace). Against
    the float64 oracle on workspaces pre-filled with 0xFF and random bytes (twice
    each, the second call finding the first one's flags, all bit-equal); under graph
    capture the library takes the two-launch path, whose replays match the oracle
    and route identically."""
    w = pkg.WORKLOADS["C2"]
    params = pkg.synth.make_params(w, affine="random")
    x_cpu = pkg.synth.make_x(w, T, stream=11)
    x = x_cpu.to(dev)
    m = _module(pkg, dev, w, params, True)
    plan, packed = m.plan(), m.packed()
    assert plan.folded()
    L = pkg._lib.lib()
    ref64 = onp.forward_f64(x_cpu, params, w.k)
    ws_bytes = plan.workspace_bytes(T)
    g = torch.Generator(device=dev).manual_seed(5)
    fills = [torch.full((ws_bytes,), 255, dtype=torch.uint8, device=dev),
             torch.randint(0, 256, (ws_bytes,), dtype=torch.uint8, device=dev, generator=g)]
    first = None
    for ws in fills:
        for _ in range(2):
            out = torch.empty(T, w.d_out, dtype=w.dtype, device=dev)
            idx = torch.empty(T, w.k, dtype=torch.int32, device=dev)
            pkg._lib.check(L.tmoe_forward(plan.ptr, x.data_ptr(), T, packed.data_ptr(),
                                          out.data_ptr(), idx.data_ptr(), None, None,
                                          ws.data_ptr(), ws_bytes,
                                          torch.cuda.current_stream().cuda_stream))
            torch.cuda.synchronize()
            if first is None:
                first = out.clone()
                assert (idx.cpu().numpy() == ref64["idx"]).all()
                assert onp.rel_l2(out.float().cpu().numpy(), ref64["out"]) <= TOL[w.dtype]
            assert torch.equal(out, first)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    out_g = torch.empty(T, w.d_out, dtype=w.dtype, device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(graph, stream=s):
        _, idx_g, _, _ = m.forward_raw(x, routing=True, out=out_g)
    torch.cuda.synchronize()
    for _ in range(3):
        out_g.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert (idx_g.cpu().numpy() == ref64["idx"]).all()
        assert onp.rel_l2(out_g.float().cpu().numpy(), ref64["out"]) <= TOL[w.dtype]
        with torch.no_grad():
            assert torch.equal(m(x), first)   # eager (one launch) between the replays
        torch.cuda.synchronize()


def _fp8_reference(params, codes):
    """float64 state_dict of the fp8 layer: bf16 router / U_expert / gain / bias
    and the oracle's dequantisation of the e4m3 weights."""
    ref = {k: v.double() for k, v in params.items()}
    for k in ("U_in", "core", "U_out"):
        q = codes[f"{k}_q"]
        q = q.view(torch.uint8) if q.dtype == torch.float8_e4m3fn else q
        ref[k] = torch.from_numpy(e4m3.dequantize(q.numpy(), codes[f"{k}_scale"].double().numpy(), k))
    return ref


def _fp8_module(pkg, dev, w, params, codes, fold=True):
    m = _module(pkg, dev, w, params, fold)
    m.load_fp8(*[codes[k].to(dev) for k in ("U_in_q", "U_in_scale", "core_q", "core_scale",
                                              "U_out_q", "U_out_scale")])
    return m


@pytest.mark.parametrize("fold", [True, False], ids=["fold", "nofold"])
@pytest.mark.parametrize("affine", ["unit", "random"])
def test_fp8_weights_parity(pkg, dev, affine, fold):
    """C5: e4m3 U_in / core / U_out with per-output-channel scales, against the
    oracle run on the dequantised weights (bf16 bar); folded, W is formed from the
    dequantised core and U_out."""
    w = pkg.WORKLOADS["C5"]
    params, codes, _ = pkg.synth.make_fp8_params(w, affine=affine)
    ref = _fp8_reference(params, codes)
    x = pkg.synth.make_x(w, 1024)
    got = _run(_fp8_module(pkg, dev, w, params, codes, fold), x, dev)
    ref64 = onp.forward_f64(x, ref, w.k)
    ref32 = {k: v.float() for k, v in ref.items()}
    tref = ot.forward(x, ref32, w.k, compute_dtype=torch.float32, intermediates=True)
    _check(w, got, ref64, f"C5/{affine}", tref)


def test_fp8_decode(pkg, dev):
    """C5's shapes at a decode-sized batch (small-T kernels)."""
    w = pkg.WORKLOADS["C5"].with_T(32)
    params, codes, _ = pkg.synth.make_fp8_params(w, affine="random")
    ref = _fp8_reference(params, codes)
    x = pkg.synth.make_x(w)
    got = _run(_fp8_module(pkg, dev, w, params, codes), x, dev)
    _check(w, got, onp.forward_f64(x, ref, w.k), "C5/T=32")


def test_fp8_full_size(pkg, dev):
    w = pkg.WORKLOADS["C5"]
    params, codes, _ = pkg.synth.make_fp8_params(w)
    ref = _fp8_reference(params, codes)
    x = pkg.synth.make_x(w)
    got = _run(_fp8_module(pkg, dev, w, params, codes), x, dev)
    ref64 = onp.forward_f64(x, ref, w.k)
    ref32 = {k: v.float() for k, v in ref.items()}
    tref = ot.forward(x[:512], ref32, w.k, compute_dtype=torch.float32, intermediates=True)
    _check(w, got, ref64, "C5/full", tref)


@pytest.mark.parametrize("r1,r2", [(3, 320), (4, 256)])
@pytest.mark.parametrize("T", [40, 300])
@pytest.mark.parametrize("fold", [True, False], ids=["fold", "nofold"])
def test_fp8_every_code_and_zero_scales(pkg, dev, T, r1, r2, fold):
    """Every finite e4m3 code appears in each weight, with some channels' scales
    zero (and, for core, a zero scale between non-zero ones of the same column);
    the zero-scaled channels also hold NaN codes, which they must not propagate.
    r1 = 3 with r2 = 320 runs the rank-rescaling core on a partial last tile,
    r1 = 4 with r2 = 256 the persistent core (scales in its epilogue); T = 40 takes
    the small-T kernels, T = 300 the large-tile ones."""
    w = pkg.Workload("fp8-codes", T, 256, 192, 8, 2, r1, 128, r2, torch.bfloat16, 91)
    p32 = pkg.synth.make_params(w, affine="random", dtype=torch.float32)
    finite = torch.tensor([b for b in range(256) if b not in (0x7F, 0xFF)], dtype=torch.uint8)
    g = torch.Generator().manual_seed(5)

    def codes_like(shape):
        n = int(np.prod(shape))
        return finite[torch.randint(0, len(finite), (n,), generator=g)].reshape(shape)

    codes = {
        "U_in_q": codes_like((w.d_in, w.r3)),
        "U_in_scale": torch.rand(w.r3, generator=g) * 0.02,
        "core_q": codes_like((w.r1, w.r3, w.r2)),
        "core_scale": torch.rand(w.r1, w.r2, generator=g) * 0.02,
        "U_out_q": codes_like((w.r2, w.d_out)),
        "U_out_scale": torch.rand(w.d_out, generator=g) * 0.02,
    }
    codes["U_in_scale"][::7] = 0
    codes["core_scale"][1, ::5] = 0        # rank 1 of every 5th column: 0 between non-zero
    codes["core_scale"][-1, 3::11] = 0     # the last rank
    codes["U_out_scale"][::13] = 0
    # NaN codes (0x7F, 0xFF) in zero-scaled channels: a zero scale zeroes its channel
    codes["U_in_q"][::3, ::7] = 0x7F
    codes["U_in_q"][1::3, ::7] = 0xFF
    codes["core_q"][1, ::4, ::5] = 0xFF
    codes["core_q"][-1, 1::3, 3::11] = 0x7F
    codes["U_out_q"][::2, ::13] = 0xFF
    params = {k: v.to(torch.bfloat16) for k, v in p32.items()}
    ref = _fp8_reference(params, codes)
    x = pkg.synth.make_x(w)
    got = _run(_fp8_module(pkg, dev, w, params, codes, fold), x, dev)
    _check(w, got, onp.forward_f64(x, ref, w.k), "fp8 codes/zero scales")


@pytest.mark.parametrize("T", [40, 600])
@pytest.mark.parametrize("E,k", [(16, 2), (256, 8)])
def test_exact_ties_pick_lower_index(pkg, dev, T, E, k):
    """Duplicated router rows give exactly equal logits; zero router rows give
    +0 and -0 logits for positive / negative x. The lower expert index must
    win (the oracle's stable argsort); T = 40 / 600 take the small-T / large-tile
    kernels."""
    w = pkg.Workload("ties", T, 512, 256, E, k, 4, 128, 256, torch.bfloat16, 123)
    params = pkg.synth.make_params(w, affine="random")
    rw = params["router.weight"].clone()
    for dst, src in ((3, 1), (5, 1), (9, 7), (E - 1, 0)):
        rw[dst] = rw[src]
    rw[E - 2] = 0
    rw[E - 3] = 0
    params["router.weight"] = rw
    x = pkg.synth.make_x(w)
    got = _run(_module(pkg, dev, w, params), x, dev)
    ref64 = onp.forward_f64(x, params, w.k)
    idx = got[1].numpy()
    assert np.array_equal(idx, ref64["idx"][:T]), np.nonzero((idx != ref64["idx"][:T]).any(1))[0][:8]
    assert onp.rel_l2(got[0].numpy(), ref64["out"][:T]) <= TOL[w.dtype]


@pytest.mark.parametrize("name,T", [("C1", 64), ("C2", 32), ("C3", 1024), ("C4", 600)])
def test_capped_router_parity(pkg, dev, name, T):
    """The trained checkpoints' router (scale 10, temperature 0.5) on both kernel
    paths, with router weights large enough that the cap saturates."""
    w = pkg.WORKLOADS[name].with_T(T)
    params = pkg.synth.make_params(w, affine="random")
    # E = 256's router weights (std 0.02) give larger logits than N(0, 1/d_in)
    mult = 8 if w.E > 64 else 30
    params["router.weight"] = (params["router.weight"].float() * mult).to(w.dtype)
    x = pkg.synth.make_x(w)
    m = _module(pkg, dev, w, params)
    m.set_router_mode("capped", 10.0, 0.5)
    out, idx, wts, lg = _run(m, x, dev)
    r = ("capped", 10.0, 0.5)
    ref64 = onp.forward_f64(x, params, w.k, router=r)
    gaps = onp.topk_gap(ref64["scores"], w.k)
    # The cap saturates in fp32 (tanh rounds to exactly 1 for |logit| >~ 90), so
    # scores that float64 still separates can tie exactly on the GPU; a tie inside
    # the selected set is broken by the lower index, so the slot order may differ
    # from float64 there. Compare the selected set per row, and the weights per
    # expert: both are what the output depends on.
    gi, ri = np.sort(idx.numpy(), 1), np.sort(ref64["idx"], 1)
    mism = np.nonzero((gi != ri).any(1))[0]
    order = np.nonzero((idx.numpy() != ref64["idx"]).any(1))[0]
    keep = np.setdiff1d(np.arange(T), mism)
    err = onp.rel_l2(out.numpy()[keep], ref64["out"][keep])
    msg = (f"capped {name} T={T}: rel_l2={err:.3e} set_mismatch_rows={len(mism)} "
           f"order_only_rows={len(order) - len(mism)} min_gap={gaps.min():.3e} "
           f"saturated={np.mean(np.abs(ref64['logits']) > 10):.3f}")
    for r_ in mism[:4]:
        srt = np.sort(ref64["scores"][r_])[::-1][: w.k + 2]
        msg += (f"\n  row {r_}: gpu {idx[r_].tolist()} ref {ref64['idx'][r_].tolist()} "
                f"gap {gaps[r_]:.3e} top scores {np.array2string(srt, precision=7)}")
    print(msg, flush=True)
    # a set may only differ where the k-th and (k+1)-th scores are within the fp32
    # logit error of each other (logits ~30 carry ~3e-5, times up to 1/temperature)
    assert all(gaps[r_] < 2e-4 for r_ in mism), msg
    assert len(mism) <= max(1, T // 1000), msg
    for r_ in order:   # an order difference only between equal fp32 scores
        sc32 = ref64["scores"][r_].astype(np.float32)
        assert np.allclose(sc32[idx[r_].numpy()], np.sort(sc32[ref64["idx"][r_]])[::-1], rtol=0,
                           atol=1e-5) or r_ in mism, msg
    wg = np.take_along_axis(wts.numpy(), np.argsort(idx.numpy(), 1), 1)
    wr = np.take_along_axis(ref64["w"], np.argsort(ref64["idx"], 1), 1)
    assert np.abs(wg - wr)[keep].max() < 2e-5, msg
    assert err <= TOL[w.dtype], msg
    assert onp.rel_l2(lg.numpy(), ref64["logits"]) < (1e-6 if w.dtype == torch.float32 else 1e-5)
