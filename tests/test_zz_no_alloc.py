"""tmoe_forward_static (the forward with its workspace in a static device array,
no allocation) against tmoe_forward with a caller workspace, through the C ABI:
bit-identical outputs, indices and weights on consecutive calls, each smaller than
the one before (the static scratch keeps the previous call's contents)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _module(pkg, dev, w):
    params = pkg.synth.make_params(w, affine="random")
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg()).to(dev, w.dtype)
    m.load_state_dict({k: v.to(dev) for k, v in params.items()})
    return m


def _run(pkg, m, x, static):
    L = pkg._lib.lib()
    plan, packed = m.plan(), m.packed()
    T = x.shape[0]
    dev = x.device
    out = torch.full((T, m.U_out.shape[1]), float("nan"), dtype=x.dtype, device=dev)
    idx = torch.full((T, m.top_k), -1, dtype=torch.int32, device=dev)
    wts = torch.full((T, m.top_k), float("nan"), dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    if static:
        rc = L.tmoe_forward_static(plan.ptr, x.data_ptr(), T, packed.data_ptr(), out.data_ptr(),
                                   idx.data_ptr(), wts.data_ptr(), None, st)
    else:
        nb = plan.workspace_bytes(T)
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
        rc = L.tmoe_forward(plan.ptr, x.data_ptr(), T, packed.data_ptr(), out.data_ptr(),
                            idx.data_ptr(), wts.data_ptr(), None, ws.data_ptr(), nb, st)
    assert rc == 0, L.tmoe_last_error()
    torch.cuda.synchronize()
    return out, idx, wts


@pytest.mark.parametrize("name,sizes", [("C3", (16384, 2048, 300, 40)), ("C2", (200, 32, 5)),
                                        ("C1", (64, 17))])
def test_static_forward_matches_workspace_forward(pkg, dev, name, sizes):
    w = pkg.WORKLOADS[name]
    m = _module(pkg, dev, w)
    x_all = pkg.synth.make_x(w, max(sizes)).to(dev)
    for T in sizes:                      # each call smaller than the previous one
        x = x_all[:T].contiguous()
        print(f"static forward {name} T={T}", flush=True)
        ref = _run(pkg, m, x, static=False)
        got = _run(pkg, m, x, static=True)
        for a, b, what in zip(got, ref, ("out", "idx", "w")):
            assert torch.equal(a, b), (name, T, what)
