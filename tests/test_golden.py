"""Golden fixtures (tests/golden/, written by make_golden.py): the seeded
generator still rebuilds the same inputs, the oracle still produces the stored
outputs, and (GPU) the gfx950 path matches them to the parity bar."""
import os

import numpy as np
import pytest
import torch

from oracle import e4m3
from oracle import tucker_moe_np as onp

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = [("C1", 64, "random"), ("C2", 32, "unit"), ("C3", 32, "unit"), ("C4", 32, "unit")]
FP8_CASES = [("C5", 64, "unit")]
FP8_KEYS = ("U_in", "core", "U_out")


def _load(name):
    return dict(np.load(os.path.join(HERE, f"golden_{name}.npz"), allow_pickle=False))


def _inputs(pkg, name, T, affine):
    w = pkg.WORKLOADS[name]
    return w, pkg.synth.make_params(w, affine=affine), pkg.synth.make_x(w, T)


@pytest.mark.parametrize("name,T,affine", CASES)
def test_inputs_regenerate(pkg, name, T, affine):
    g = _load(name)
    w, params, x = _inputs(pkg, name, T, affine)
    assert int(g["T"]) == T and str(g["affine"]) == affine
    assert pkg.synth.sha256(x) == str(g["sha_x"])
    for k, v in params.items():
        assert pkg.synth.sha256(v) == str(g[f"sha_{k.replace('.', '_')}"]), k


@pytest.mark.parametrize("name,T,affine", CASES)
def test_oracle_reproduces_fixture(pkg, name, T, affine):
    g = _load(name)
    w, params, x = _inputs(pkg, name, T, affine)
    ref = onp.forward_f64(x, params, w.k)
    assert np.array_equal(ref["idx"], g["idx"])
    assert onp.rel_l2(ref["out"], g["out"]) < 1e-6
    assert onp.rel_l2(ref["w"], g["w"]) < 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("name,T,affine", CASES)
def test_gpu_matches_fixture(pkg, dev, name, T, affine):
    g = _load(name)
    w, params, x = _inputs(pkg, name, T, affine)
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg()).to(dev, w.dtype)
    m.load_state_dict({k: v.to(dev) for k, v in params.items()})
    with torch.no_grad():
        out, idx, wts, lg = m.forward_with_routing(x.to(dev), logits=True)
    torch.cuda.synchronize()
    tol = 1e-5 if w.dtype == torch.float32 else 1e-2
    err = onp.rel_l2(out.float().cpu().numpy(), g["out"])
    print(f"golden {name}: rel_l2={err:.3e} (tol {tol}) min_gap={g['topk_gap'].min():.3e}")
    assert np.array_equal(idx.cpu().numpy(), g["idx"])
    assert err <= tol
    assert np.abs(wts.cpu().numpy() - g["w"]).max() < 1e-5


# ---- C5: e4m3 U_in / core / U_out with per-output-channel scales -----------------

def _fp8_inputs(pkg, name, T, affine):
    w = pkg.WORKLOADS[name]
    params, codes, _ = pkg.synth.make_fp8_params(w, affine=affine)
    ref = {k: v.double().numpy() for k, v in params.items()}
    for k in FP8_KEYS:
        ref[k] = e4m3.dequantize(codes[f"{k}_q"].view(torch.uint8).numpy(),
                                 codes[f"{k}_scale"].double().numpy(), k)
    return w, params, codes, ref, pkg.synth.make_x(w, T)


@pytest.mark.parametrize("name,T,affine", FP8_CASES)
def test_fp8_inputs_regenerate(pkg, name, T, affine):
    """The digests cover the e4m3 codes and scales, the bf16 router / U_expert /
    gain / bias and the tokens."""
    g = _load(name)
    w, params, codes, _, x = _fp8_inputs(pkg, name, T, affine)
    assert int(g["T"]) == T and str(g["affine"]) == affine
    assert pkg.synth.sha256(x) == str(g["sha_x"])
    for k, v in codes.items():
        assert pkg.synth.sha256(v) == str(g[f"sha_{k}"]), k
    for k, v in params.items():
        if k not in FP8_KEYS:
            assert pkg.synth.sha256(v) == str(g[f"sha_{k.replace('.', '_')}"]), k


@pytest.mark.parametrize("name,T,affine", FP8_CASES)
def test_fp8_oracle_reproduces_fixture(pkg, name, T, affine):
    g = _load(name)
    w, _, _, ref, x = _fp8_inputs(pkg, name, T, affine)
    out = onp.forward_f64(x, ref, w.k)
    assert np.array_equal(out["idx"], g["idx"])
    assert onp.rel_l2(out["out"], g["out"]) < 1e-6
    assert onp.rel_l2(out["w"], g["w"]) < 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("fold", [True, False], ids=["fold", "nofold"])
@pytest.mark.parametrize("name,T,affine", FP8_CASES)
def test_fp8_gpu_matches_fixture(pkg, dev, name, T, affine, fold):
    """The module fed the e4m3 codes through load_fp8 (small-T kernels at T = 64)."""
    g = _load(name)
    w, params, codes, _, x = _fp8_inputs(pkg, name, T, affine)
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg()).to(dev, w.dtype)
    m.load_state_dict({k: v.to(dev) for k, v in params.items()})
    m.set_fold(fold)
    m.load_fp8(*[codes[k].to(dev) for k in ("U_in_q", "U_in_scale", "core_q", "core_scale",
                                              "U_out_q", "U_out_scale")])
    with torch.no_grad():
        out, idx, wts, lg = m.forward_with_routing(x.to(dev), logits=True)
    torch.cuda.synchronize()
    err = onp.rel_l2(out.float().cpu().numpy(), g["out"])
    print(f"golden {name} fold={fold}: rel_l2={err:.3e} (tol 1e-2) min_gap={g['topk_gap'].min():.3e}")
    assert np.array_equal(idx.cpu().numpy(), g["idx"])
    assert err <= 1e-2
    assert np.abs(wts.cpu().numpy() - g["w"]).max() < 1e-5
