"""Pins the float64 formulation of the latent expert contraction and its backward
(oracle/latent_np.py; sft_cot_bundle/scripts/model.py:160-174, :196-289) against
torch autograd of the forward in float64 and against finite differences, and
checks that planted mistakes are caught."""
import numpy as np
import pytest
import torch

from oracle import latent_np as ln


def _case(seed=0, B=9, E=5, k=2, r3=6, r2=7):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, r3, generator=g, dtype=torch.float64)
    G = torch.randn(E, r3, r2, generator=g, dtype=torch.float64)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(B)])
    p = torch.rand(B, k, generator=g, dtype=torch.float64)
    dout = torch.randn(B, r2, generator=g, dtype=torch.float64)
    return x, G, idx, p, dout


def _torch_forward(x, G, idx, p):
    """The reference forward as a torch expression (autograd-able)."""
    out = 0
    for j in range(idx.shape[1]):
        out = out + p[:, j:j + 1] * torch.einsum("bs,bsq->bq", x, G[idx[:, j]])
    return out


def test_forward_matches_torch_expression():
    x, G, idx, p, _ = _case()
    assert np.allclose(ln.forward(x, G, idx, p), _torch_forward(x, G, idx, p).numpy(), atol=1e-12)


def test_backward_matches_autograd():
    x, G, idx, p, dout = _case(1)
    xs, Gs, ps = (t.clone().requires_grad_(True) for t in (x, G, p))
    _torch_forward(xs, Gs, idx, ps).backward(dout)
    dx, dG, dp = ln.backward(x, G, idx, p, dout)
    assert np.allclose(dx, xs.grad.numpy(), atol=1e-12)
    assert np.allclose(dG, Gs.grad.numpy(), atol=1e-12)
    assert np.allclose(dp, ps.grad.numpy(), atol=1e-12)


def test_backward_finite_differences():
    """Directional derivative of L = <dout, out> along a random direction."""
    x, G, idx, p, dout = _case(2, B=4, E=3, r3=4, r2=5)
    dx, dG, dp = ln.backward(x, G, idx, p, dout)
    g = torch.Generator().manual_seed(3)
    vx, vG, vp = (torch.randn(t.shape, generator=g, dtype=torch.float64) for t in (x, G, p))
    h = 1e-6
    L = lambda a, b, c: float((ln.forward(a, b, idx, c) * dout.numpy()).sum())
    fd = (L(x + h * vx, G + h * vG, p + h * vp) - L(x - h * vx, G - h * vG, p - h * vp)) / (2 * h)
    an = float((dx * vx.numpy()).sum() + (dG * vG.numpy()).sum() + (dp * vp.numpy()).sum())
    assert abs(fd - an) < 1e-6 * max(1.0, abs(an))


def test_repeated_expert_slots_accumulate():
    """Two slots naming the same expert add into dG[e] (np.add.at, not assignment)."""
    x, G, _, p, dout = _case(4, B=3, E=2, k=2)
    idx = torch.zeros(3, 2, dtype=torch.int64)
    xs, Gs = x.clone().requires_grad_(True), G.clone().requires_grad_(True)
    _torch_forward(xs, Gs, idx, p).backward(dout)
    assert np.allclose(ln.backward(x, G, idx, p, dout)[1], Gs.grad.numpy(), atol=1e-12)


@pytest.mark.parametrize("mistake", ["dx without p", "dG transposed", "dp without x"])
def test_planted_mistake_is_caught(mistake):
    x, G, idx, p, dout = _case(5)
    xs, Gs, ps = (t.clone().requires_grad_(True) for t in (x, G, p))
    _torch_forward(xs, Gs, idx, ps).backward(dout)
    dx, dG, dp = ln.backward(x, G, idx, p, dout)
    X, Gm, D = x.numpy(), G.numpy(), dout.numpy()
    if mistake == "dx without p":
        dx = sum(np.einsum("bq,bsq->bs", D, Gm[idx[:, j]]) for j in range(idx.shape[1]))
    elif mistake == "dG transposed":
        dG = np.zeros_like(Gm)
        for j in range(idx.shape[1]):
            np.add.at(dG, idx[:, j].numpy(), p[:, j, None, None].numpy() *
                      np.einsum("bs,bq->bsq", X, D)[:, ::-1, ::-1])
    else:
        dp = np.stack([np.einsum("bq,bsq->b", D, Gm[idx[:, j]]) for j in range(idx.shape[1])], 1)
    ok = (np.allclose(dx, xs.grad.numpy()) and np.allclose(dG, Gs.grad.numpy())
          and np.allclose(dp, ps.grad.numpy()))
    assert not ok, mistake
