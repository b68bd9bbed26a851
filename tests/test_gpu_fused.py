"""The one-launch large-T forward (k_fused_large), the one-launch mid-T forward
(k_fused_mid), the one-launch K-sliced front (k_front_sliced) and the reporting of
lost in-launch signals.

The large-T forward of a folded bf16 plan (r3 = 256, E <= 32, d_out % 288 == 0,
T >= 8192 at the C3 shapes) runs front and out-projection in one persistent grid
that hands c (x) z over inside each XCD's L2 (model.py:68-102 in one kernel).
Checked here: parity with the float64 oracle at ragged T; routing bit-identical to
the two-launch path (TMOE_FLAG_NO_FUSE), whose router logits it sums in the same
order; independence from the workspace's previous contents; graph capture (which
takes the two-launch path); and a clean status block (every work-group ran on the
XCD the schedule assumes). Lost signals: a budget of 0 polls makes every wait give
up at once (every kernel still exits normally), which the status block must report
and the module must raise as RuntimeError."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import tucker_moe_np as onp

pytestmark = pytest.mark.gpu


def _module(pkg, dev, w, params, fuse=True):
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg()).to(dev, w.dtype)
    m.load_state_dict({k: v.to(dev) for k, v in params.items()})
    return m.set_fuse(fuse)


def _forward(m, x):
    with torch.no_grad():
        out, idx, wts, _ = m.forward_with_routing(x)
    torch.cuda.synchronize()
    return out, idx, wts


@pytest.mark.parametrize("T", [16384, 8192 + 100, 12345, 20000])
def test_fused_parity(pkg, dev, T):
    """Against the float64 oracle on every token (rel-L2 <= 1e-2, routing exact),
    and against the two-launch path: identical routing, outputs within bf16
    rounding of c (x) z (z's K sum is associated differently)."""
    w = pkg.WORKLOADS["C3"]
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w, T, stream=11)
    xd = x.to(dev)
    m = _module(pkg, dev, w, params)
    out, idx, wts = _forward(m, xd)
    m.check_signals()   # no lost signal, every work-group on its XCD
    ref = onp.forward_f64(x, params, w.k)
    err = onp.rel_l2(out.float().cpu().numpy(), ref["out"])
    mism = int((idx.cpu().numpy() != ref["idx"]).any(1).sum())
    print(f"fused T={T}: rel_l2(out, f64)={err:.3e} routing_mismatch_rows={mism}", flush=True)
    assert mism == 0 and err <= 1e-2
    assert np.abs(wts.cpu().numpy() - ref["w"]).max() < 1e-5
    m2 = _module(pkg, dev, w, params, fuse=False)
    out2, idx2, wts2 = _forward(m2, xd)
    assert torch.equal(idx, idx2) and torch.equal(wts, wts2)
    d = onp.rel_l2(out.float().cpu().numpy(), out2.float().cpu().numpy().astype(np.float64))
    print(f"fused vs two launches: rel_l2={d:.3e}", flush=True)
    assert d < 1e-3


def test_fused_workspace_reuse_and_graph(pkg, dev):
    """The result does not depend on what the workspace held (0xFF bytes, random
    bytes, the flags of the previous forward); a captured forward (the two-launch
    path) replays to the eager two-launch result, with eager fused forwards between
    the replays."""
    w = pkg.WORKLOADS["C3"]
    T = 8192
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w, T, stream=13).to(dev)
    m = _module(pkg, dev, w, params)
    plan, packed = m.plan(), m.packed()
    L = pkg._lib.lib()
    with torch.no_grad():
        ref = m(x)
    torch.cuda.synchronize()
    ws_bytes = plan.workspace_bytes(T)
    g = torch.Generator(device=dev).manual_seed(5)
    fills = [torch.full((ws_bytes,), 255, dtype=torch.uint8, device=dev),
             torch.randint(0, 256, (ws_bytes,), dtype=torch.uint8, device=dev, generator=g)]
    for ws in fills:
        for _ in range(2):
            out = torch.empty_like(ref)
            pkg._lib.check(L.tmoe_forward(plan.ptr, x.data_ptr(), T, packed.data_ptr(),
                                          out.data_ptr(), None, None, None, ws.data_ptr(),
                                          ws_bytes, torch.cuda.current_stream().cuda_stream))
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
    m.check_signals()
    m2 = _module(pkg, dev, w, params, fuse=False)
    with torch.no_grad():
        ref2 = m2(x)
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
        assert torch.equal(out_g, ref2)
        with torch.no_grad():
            assert torch.equal(m(x), ref)
        torch.cuda.synchronize()
    m.check_signals()


@pytest.mark.parametrize("T", [300, 777, 2048, 3001, 4096])
def test_sliced_front_matches_two_launches(pkg, dev, T):
    """The K-sliced mid-T front in one launch (k_front_sliced: slices, then the
    per-token epilogue once a tile's slices are in; up to T = 2048 inside the
    one-launch mid-T forward k_fused_mid, with the out-projection tiles) against the
    same slices in separate launches (TMOE_FLAG_NO_FUSE: k_front_part + k_front_epi,
    then the out-projection): bit-identical outputs and routing, a clean status
    block, and the float64 oracle."""
    w = pkg.WORKLOADS["C3"]
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w, T, stream=19)
    xd = x.to(dev)
    m = _module(pkg, dev, w, params)
    want = pkg._lib.TMOE_PATH_FUSED_MID if T <= 2048 else pkg._lib.TMOE_PATH_LARGE
    assert m.plan().forward_path(T) == want
    out, idx, wts = _forward(m, xd)
    m.check_signals()
    m2 = _module(pkg, dev, w, params, fuse=False)
    out2, idx2, wts2 = _forward(m2, xd)
    assert torch.equal(out, out2) and torch.equal(idx, idx2) and torch.equal(wts, wts2)
    ref = onp.forward_f64(x, params, w.k)
    err = onp.rel_l2(out.float().cpu().numpy(), ref["out"])
    mism = int((idx.cpu().numpy() != ref["idx"]).any(1).sum())
    print(f"sliced front T={T}: rel_l2(out, f64)={err:.3e} routing_mismatch_rows={mism}",
          flush=True)
    assert mism == 0 and err <= 1e-2


def test_sliced_front_workspace_reuse_and_graph(pkg, dev):
    """The one-launch mid-T forward (k_fused_mid at T = 2048) does not depend on
    what the workspace held (0xFF bytes, random bytes, the flags of the previous
    forward); a captured forward (the sliced front in two launches, then the
    out-projection) replays to the same bits, with eager forwards between the
    replays."""
    w = pkg.WORKLOADS["C3"]
    T = 2048
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w, T, stream=23).to(dev)
    m = _module(pkg, dev, w, params)
    plan, packed = m.plan(), m.packed()
    L = pkg._lib.lib()
    with torch.no_grad():
        ref = m(x)
    torch.cuda.synchronize()
    ws_bytes = plan.workspace_bytes(T)
    g = torch.Generator(device=dev).manual_seed(7)
    fills = [torch.full((ws_bytes,), 255, dtype=torch.uint8, device=dev),
             torch.randint(0, 256, (ws_bytes,), dtype=torch.uint8, device=dev, generator=g)]
    for ws in fills:
        for _ in range(2):
            out = torch.empty_like(ref)
            pkg._lib.check(L.tmoe_forward(plan.ptr, x.data_ptr(), T, packed.data_ptr(),
                                          out.data_ptr(), None, None, None, ws.data_ptr(),
                                          ws_bytes, torch.cuda.current_stream().cuda_stream))
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
    m.check_signals()
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
            assert torch.equal(m(x), ref)
        torch.cuda.synchronize()
    m.check_signals()


# workloads whose forward signals between work-groups of one launch: the
# one-launch large-T forward (C3), the one-launch mid-T forward (C3 at T = 2048),
# the E = 256 front (C4) and the decode launch (C2)
@pytest.mark.parametrize("name,T", [("C3", 16384), ("C3", 2048), ("C4", 600), ("C2", 32)])
def test_lost_signal_is_reported(pkg, dev, name, T):
    """With a wait budget of 0 polls every in-launch wait gives up at once; the
    kernels still complete, the status block records it, and the module raises
    RuntimeError (at the next forward without a synchronisation, or from
    check_signals). With the budget restored the same forward is clean again."""
    w = pkg.WORKLOADS[name]
    params = pkg.synth.make_params(w)
    x = pkg.synth.make_x(w, T, stream=17).to(dev)
    m = _module(pkg, dev, w, params)
    with torch.no_grad():
        ref = m(x)
    m.check_signals()
    prev = pkg._lib.set_wait_polls(0)
    try:
        with torch.no_grad():
            m(x)
        torch.cuda.synchronize()
        mask = ctypes.c_uint32()
        L = pkg._lib.lib()
        assert L.tmoe_signal_status(m.plan().ptr, 0, ctypes.byref(mask)) == pkg._lib.TMOE_ESIGNAL
        assert mask.value & pkg._lib.TMOE_STATUS_SIGNAL
        with pytest.raises(RuntimeError, match="poll budget") as ei:
            with torch.no_grad():
                m(x)   # reports the earlier forward's lost signal before launching
        assert ei.value.code == pkg._lib.TMOE_ESIGNAL
        with torch.no_grad():
            m(x)
        with pytest.raises(RuntimeError, match="poll budget"):
            m.check_signals()
    finally:
        pkg._lib.set_wait_polls(prev)
    with torch.no_grad():
        out = m(x)
    m.check_signals()
    assert torch.equal(out, ref)
