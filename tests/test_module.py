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


def test_fp8_quantize_per_channel(pkg):
    """Per-output-channel absmax scales; codes decode (oracle) to within e4m3's
    half-ulp of w / s; all-zero channels get scale 0 and zero codes."""
    from oracle import e4m3
    g = torch.Generator().manual_seed(0)
    for name, shape, dims in (("U_in", (96, 32), (0,)), ("core", (3, 16, 40), (1,)),
                              ("U_out", (64, 48), (0,))):
        w = torch.randn(shape, generator=g) * 0.1
        if name == "core":
            w[1, :, 7] = 0
        else:
            w[:, 5] = 0
        q, s = pkg.fp8.quantize(w, name)
        assert q.dtype == torch.float8_e4m3fn and s.dtype == torch.float32
        amax = w.abs().amax(dim=dims)
        assert torch.equal(s, amax / 448.0)
        v = e4m3.decode(q.view(torch.uint8).numpy())
        assert not np.isnan(v).any() and np.abs(v).max() <= 448.0
        s_b = s.unsqueeze(1).numpy() if name == "core" else s.unsqueeze(0).numpy()
        target = np.where(s_b > 0, w.double().numpy() / np.where(s_b > 0, s_b, 1), 0.0)
        # e4m3 spacing: 2^(floor(log2|t|) - 3) for normals, 2^-9 below 2^-6
        ex = np.floor(np.log2(np.maximum(np.abs(target), 2.0 ** -6)))
        assert (np.abs(v - target) <= 2.0 ** (ex - 4) * (1 + 1e-6)).all()
        if name == "core":
            assert s[1, 7] == 0 and (v[1, :, 7] == 0).all()
        else:
            assert s[5] == 0 and (v[:, 5] == 0).all()
        deq = pkg.fp8.dequantize(q, s, name).double().numpy()
        assert np.allclose(deq, e4m3.dequantize(q.view(torch.uint8).numpy(), s.numpy(), name),
                           rtol=1e-7, atol=0)


def test_fp8_load_validation(pkg):
    w = pkg.WORKLOADS["C5"].with_T(8)
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg()).to(torch.bfloat16)
    params, codes, _ = pkg.synth.make_fp8_params(w)
    m.load_state_dict(params)
    names = ("U_in_q", "U_in_scale", "core_q", "core_scale", "U_out_q", "U_out_scale")
    args = [codes[k] for k in names]
    m.load_fp8(*args)
    assert m.fp8_weights
    # the parameters now hold the dequantised weights (rounded to bf16)
    assert torch.equal(m.U_out, params["U_out"])
    bad = list(args)
    bad[0] = codes["U_in_q"].float()
    with pytest.raises(RuntimeError, match="float8_e4m3fn or uint8"):
        m.load_fp8(*bad)
    bad = list(args)
    bad[3] = codes["core_scale"][:, :-1]
    with pytest.raises(RuntimeError, match="core codes"):
        m.load_fp8(*bad)
    m.clear_fp8()
    assert not m.fp8_weights
    m32 = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg())
    with pytest.raises(RuntimeError, match="bfloat16 module"):
        m32.load_fp8(*args)


def test_data_writes_invalidate_packed_key(pkg):
    """The reference loader writes through `param.data.copy_` (weights.py:74-81),
    which does not move a parameter's version counter: the packed-weight cache key
    must change anyway, for every parameter."""
    w = pkg.WORKLOADS["C1"]
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg())
    m.load_state_dict(pkg.synth.make_params(w))
    for p in m._params():
        k0 = m._key()
        v0 = p._version
        p.data.copy_(p.detach() * 2)
        assert p._version == v0            # what made the old key blind to it
        assert m._key() != k0
    k0 = m._key()
    _ = m.state_dict()
    assert m._key() == k0                  # reading the state does not force a re-pack
    m._packed, m._packed_key = torch.zeros(1), k0
    m.load_state_dict(pkg.synth.make_params(w))
    assert m._packed is None               # load_state_dict forgets the packed copy


def test_data_reads_keep_packed_key(pkg):
    """Reading a weight through `.data` (inspection, norms, copies out) writes
    nothing, so it must not force a re-pack (at C3 a re-fold of W costs ~0.2 ms);
    a write through the same alias still does, as does assigning `.data`."""
    w = pkg.WORKLOADS["C1"]
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg())
    m.load_state_dict(pkg.synth.make_params(w))
    for p in m._params():
        _ = p.data                         # the first access hands out the alias
        k0 = m._key()
        for _ in range(3):
            float(p.data.float().abs().sum())
            _ = p.data.clone()
        assert m._key() == k0
        p.data.mul_(1.0)                   # an in-place write through .data
        k1 = m._key()
        assert k1 != k0
        p.data = p.detach().clone()        # assignment
        assert m._key() != k1


def test_tracked_parameters_survive_conversion(pkg):
    import copy
    w = pkg.WORKLOADS["C1"]
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg())
    m2 = copy.deepcopy(m).to(torch.float64)
    for mm in (m, m2):
        assert all(isinstance(p, pkg.module.TrackedParameter) for p in mm._params())
    assert m2.U_in.dtype == torch.float64 and set(m2.state_dict()) == set(REF_PARAMS)
