"""Module surface of the drop-in (CPU): constructor, parameters, state_dict keys,
the reference's checkpoint-key loader contract, and loud failure off-GPU."""
import numpy as np
import pytest
import torch

# pure_torch_mlx/model.py:60-66: name -> shape as a function of (d_in, d_out, E, r1, r2, r3)
REF_PARAMS = {
    "router.weight": lambda d_in, d_out, E, r1, r2, r3: (E, d_in),
    "U_in": lambda d_in, d_out, E, r1, r2, r3: (d_in, r3),
    "inner_norm.weight": lambda d_in, d_out, E, r1, r2, r3: (r3,),
    "U_expert": lambda d_in, d_out, E, r1, r2, r3: (E, r1),
    "core": lambda d_in, d_out, E, r1, r2, r3: (r1, r3, r2),
    "U_out": lambda d_in, d_out, E, r1, r2, r3: (r2, d_out),
    "bias": lambda d_in, d_out, E, r1, r2, r3: (d_out,),
}


def test_constructor_and_state_dict(pkg):
    cfg = pkg.TuckerMoEConfig()   # reference defaults: E=8, k=2, r=(32, 512, 256)
    m = pkg.TuckerMoE(768, 4608, cfg)
    sd = m.state_dict()
    assert set(sd) == set(REF_PARAMS)
    for k, f in REF_PARAMS.items():
        assert tuple(sd[k].shape) == f(768, 4608, 8, 32, 512, 256), k
    assert m.top_k == 2 and m.inner_norm.eps == 1e-5
    assert torch.equal(m.bias, torch.zeros(4608)) and torch.equal(m.inner_norm.weight, torch.ones(256))


def test_duck_typed_cfg(pkg):
    class Cfg:   # any object with the fields the reference's Mamba3Config has
        kmoe_num_experts, kmoe_top_k, kmoe_r1, kmoe_r2, kmoe_r3, rms_norm_eps = 4, 1, 2, 64, 64, 1e-6
    m = pkg.TuckerMoE(64, 32, Cfg())
    assert m.core.shape == (2, 64, 64) and m.top_k == 1 and m.inner_norm.eps == 1e-6


def test_load_tucker_keys(pkg):
    w = pkg.WORKLOADS["C1"]
    p = pkg.synth.make_params(w, affine="random")
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg())
    ckpt = {f"blk.ffn.{k}": v.numpy() for k, v in p.items()}
    pkg.load_tucker(m, ckpt, "blk.ffn")
    for k, v in m.state_dict().items():
        assert torch.equal(v, p[k]), k


def test_cpu_forward_raises(pkg):
    w = pkg.WORKLOADS["C1"]
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg())
    m.load_state_dict(pkg.synth.make_params(w))
    with pytest.raises(RuntimeError, match="HIP devices only"):
        m(torch.zeros(4, w.d_in))


def test_synth_is_deterministic_and_prefix_stable(pkg):
    w = pkg.WORKLOADS["C3"]
    a = pkg.synth.make_x(w, 8)
    b = pkg.synth.make_x(w, 64)
    assert torch.equal(a, b[:8])
    assert a.dtype == torch.bfloat16
    p1 = pkg.synth.make_params(w)
    p2 = pkg.synth.make_params(w)
    assert all(torch.equal(p1[k], p2[k]) for k in p1)
    assert not torch.equal(pkg.synth.make_x(w, 8, stream=1), a)


def test_workload_flops_match_baseline(pkg):
    # BASELINE: C3 F = 125.36 GFLOP; C1 59.24 MFLOP; C4 34.36 GFLOP
    assert abs(pkg.WORKLOADS["C3"].flops()["total"] / 1e9 - 125.36) < 0.01
    assert abs(pkg.WORKLOADS["C1"].flops()["total"] / 1e6 - 59.24) < 0.01
    assert abs(pkg.WORKLOADS["C4"].flops()["total"] / 1e9 - 34.36) < 0.01
    assert abs(pkg.WORKLOADS["C3"].hbm_bytes() / 1e6 - 133.49) < 0.05
