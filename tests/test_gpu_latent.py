"""FusedLatentMoE on the GPU (tmoe_latent_forward / _backward) against the float64
formulation of the reference's forward and backward (oracle/latent_np.py):
rel-L2 <= 1e-5 (fp32) and <= 1e-2 (bf16) for out, dx, dG and dp."""
import numpy as np
import pytest
import torch

from oracle import latent_np as ln
from oracle import tucker_moe_np as onp

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def _inputs(B, E, k, r3, r2, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, r3, generator=g).to(dtype)
    G = (torch.randn(E, r3, r2, generator=g) * r3 ** -0.5).to(dtype)
    logits = torch.randn(B, E, generator=g)
    v, idx = torch.topk(logits, k, dim=-1)
    p = torch.softmax(v, -1).to(dtype)
    dout = torch.randn(B, r2, generator=g).to(dtype)
    return x, G, idx, p, dout


@pytest.mark.parametrize("B", [1, 37, 300, 2048])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", [(8, 2, 256, 1024), (4, 1, 64, 128), (16, 4, 128, 512)],
                         ids=lambda s: "E%d_k%d_%dx%d" % s)
def test_latent_forward_backward(pkg, dev, B, dtype, shape):
    E, k, r3, r2 = shape
    x, G, idx, p, dout = _inputs(B, E, k, r3, r2, dtype, B + E)
    xs = x.to(dev).requires_grad_(True)
    Gs = G.to(dev).requires_grad_(True)
    ps = p.to(dev).requires_grad_(True)
    out = pkg.FusedLatentMoE.apply(xs, Gs, idx.to(dev), ps)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    ref = ln.forward(x, G, idx, p)
    dx, dG, dp = ln.backward(x, G, idx, p, dout)
    errs = {"out": onp.rel_l2(out.detach().float().cpu().numpy(), ref),
            "dx": onp.rel_l2(xs.grad.float().cpu().numpy(), dx),
            "dG": onp.rel_l2(Gs.grad.float().cpu().numpy(), dG),
            "dp": onp.rel_l2(ps.grad.float().cpu().numpy(), dp)}
    print(f"B={B} {dtype} {shape}: " + " ".join(f"{n}={v:.2e}" for n, v in errs.items()), flush=True)
    for n, v in errs.items():
        assert v <= TOL[dtype], (n, v)


def test_latent_matches_layer_core(pkg, dev):
    """With G[e] = sum_r U_expert[e, r] core[r] (the reference's G_experts einsum,
    model.py:335), the latent contraction equals the layer's mid computed by the
    forward path from the same routing (the two implementations agree)."""
    w = pkg.WORKLOADS["C2"].with_T(300)
    params = pkg.synth.make_params(w, affine="random", dtype=torch.float32)
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg()).to(dev, torch.float32)
    m.load_state_dict({k_: v.to(dev) for k_, v in params.items()})
    x = pkg.synth.make_x(w, dtype=torch.float32).to(dev)
    from oracle import tucker_moe_torch as ot
    r = ot.forward(x.cpu(), params, w.k, intermediates=True)
    G = torch.einsum("er,rst->est", params["U_expert"], params["core"]).contiguous()
    out = pkg.fused_latent_moe(r["z"].to(dev), G.to(dev), r["idx"].to(dev), r["w"].to(dev))
    assert onp.rel_l2(out.cpu().numpy(), r["mid"].double().numpy()) <= 1e-5


def test_latent_rejects_bad_arguments(pkg, dev):
    x, G, idx, p, _ = _inputs(8, 4, 2, 64, 128, torch.float32, 0)
    with pytest.raises(RuntimeError):
        pkg.fused_latent_moe(x, G, idx, p)                            # CPU tensors
    with pytest.raises(RuntimeError):
        pkg.fused_latent_moe(x.to(dev), G.to(dev).bfloat16(), idx.to(dev), p.to(dev))
    with pytest.raises(pkg._lib.TmoeError):
        pkg.fused_latent_moe(x[:, :48].to(dev), G[:, :48].contiguous().to(dev), idx.to(dev),
                             p.to(dev))                               # r3 = 48 unsupported


def test_training_layer_gradients(pkg, dev):
    """TuckerMoETrain (the reference's TritonTuckerMoE) forward and every parameter
    gradient on the GPU against the same module on the CPU in float64 with the
    latent contraction as a torch expression (oracle/latent_np semantics)."""
    torch.manual_seed(0)
    m = pkg.TuckerMoETrain(128, 96, num_experts=8, top_k=2, r1=4, r2=128, r3=64)
    m.train()
    x = torch.randn(3, 50, 128)
    ref = pkg.TuckerMoETrain(128, 96, num_experts=8, top_k=2, r1=4, r2=128, r3=64).double()
    ref.load_state_dict({k: v.double() for k, v in m.state_dict().items()})
    ref.train()

    def latent_torch(xs, G, idx, p):
        out = 0
        for j in range(idx.shape[1]):
            out = out + p[:, j:j + 1] * torch.einsum("bs,bsq->bq", xs, G[idx[:, j]])
        return out

    import mamba_tuckermoe_amd.latent as lat
    orig = lat.FusedLatentMoE.apply
    lat.FusedLatentMoE.apply = staticmethod(latent_torch)
    try:
        o_ref, lb_ref, z_ref = ref(x.double(), step=700)
        (o_ref.square().mean() + lb_ref + z_ref).backward()
    finally:
        lat.FusedLatentMoE.apply = orig
    m = m.to(dev)
    o, lb, zl = m(x.to(dev), step=700)
    (o.square().mean() + lb + zl).backward()
    torch.cuda.synchronize()
    assert onp.rel_l2(o.detach().cpu().numpy(), o_ref.detach().numpy()) <= 1e-5
    assert abs(lb.item() - lb_ref.item()) <= 1e-5 and abs(zl.item() - z_ref.item()) <= 1e-4
    for (n, p), (_, q) in zip(m.named_parameters(), ref.named_parameters()):
        err = onp.rel_l2(p.grad.cpu().numpy(), q.grad.numpy())
        assert err <= 1e-4, (n, err)


def test_latent_fp32_probs_with_bf16_activations(pkg, dev):
    """bf16 x / G with fp32 top_k_probs: the reference's forward and dG kernels read
    the probabilities in fp32 (model.py:160-174, :196-219) and its dprobs has their
    dtype. The GPU result must match the float64 layer with the fp32 probabilities
    (to the bf16 bar), sit closer to it than to the layer with bf16-rounded ones
    (the probabilities are not rounded on the way), and dp come back as fp32."""
    B, E, k, r3, r2 = 2048, 8, 2, 256, 1024
    x, G, idx, _, dout = _inputs(B, E, k, r3, r2, torch.bfloat16, 77)
    g = torch.Generator().manual_seed(78)
    v = torch.randn(B, k, generator=g).sort(-1, descending=True).values
    p = torch.softmax(v, -1)                        # fp32, not bf16-representable
    assert not torch.equal(p, p.to(torch.bfloat16).float())
    xs = x.to(dev).requires_grad_(True)
    Gs = G.to(dev).requires_grad_(True)
    ps = p.to(dev).requires_grad_(True)
    out = pkg.FusedLatentMoE.apply(xs, Gs, idx.to(dev), ps)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    assert ps.grad.dtype == torch.float32
    pb = p.to(torch.bfloat16).double()
    ref32, refb = ln.forward(x, G, idx, p.double()), ln.forward(x, G, idx, pb)
    dx32, dG32, dp32 = ln.backward(x, G, idx, p.double(), dout)
    _, dGb, _ = ln.backward(x, G, idx, pb, dout)
    o = out.detach().float().cpu().numpy()
    dGg = Gs.grad.float().cpu().numpy()
    errs = {"out": onp.rel_l2(o, ref32), "dx": onp.rel_l2(xs.grad.float().cpu().numpy(), dx32),
            "dG": onp.rel_l2(dGg, dG32), "dp": onp.rel_l2(ps.grad.cpu().numpy(), dp32)}
    print("fp32 probs: " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    for n, e in errs.items():
        assert e <= 1e-2, (n, e)
    assert onp.rel_l2(o, ref32) < 0.85 * onp.rel_l2(o, refb)
    assert onp.rel_l2(dGg, dG32) < 0.85 * onp.rel_l2(dGg, dGb)
