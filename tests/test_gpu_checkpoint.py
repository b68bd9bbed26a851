"""The packed file on the GPU: a layer saved with save_packed and loaded into a new
module computes bit for bit what the original computes, using the stored packed
buffer, or packing again from the stored parameters when the file's layout version
differs from the library's."""
import json

import pytest
import torch

pytestmark = pytest.mark.gpu


def _layer(pkg, dev, w, params):
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg()).to(dev, w.dtype)
    m.load_state_dict({k: v.to(dev) for k, v in params.items()})
    return m


def _rewrite_layout(path, layout):
    from safetensors import safe_open
    from safetensors.torch import save_file
    with safe_open(str(path), framework="pt") as f:
        meta = json.loads(f.metadata()["tmoe"])
        t = {k: f.get_tensor(k) for k in f.keys()}
    meta["packed_layout"] = layout
    save_file(t, str(path), metadata={"tmoe": json.dumps(meta)})


@pytest.mark.parametrize("T", [64, 600])
@pytest.mark.parametrize("name", ["C1", "C2"])
def test_save_load_packed_bit_exact(pkg, dev, tmp_path, name, T):
    w = pkg.WORKLOADS[name]
    params = pkg.synth.make_params(w, affine="random")
    x = pkg.synth.make_x(w, T).to(dev)
    m = _layer(pkg, dev, w, params)
    m.set_router_mode("capped", 10.0, 0.5)
    with torch.no_grad():
        ref = m.forward_with_routing(x)
    path = tmp_path / "layer.safetensors"
    pkg.checkpoint.save_packed(m, str(path))
    m2 = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg())
    assert pkg.checkpoint.load_packed(m2, str(path), device=dev) is True
    assert m2.router_mode == ("capped", 10.0, 0.5)
    with torch.no_grad():
        got = m2.forward_with_routing(x)
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
    # a file of another layout version is packed again from its parameters
    _rewrite_layout(path, pkg._lib.lib().tmoe_packed_layout_version() - 1)
    m3 = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg())
    assert pkg.checkpoint.load_packed(m3, str(path), device=dev) is False
    with torch.no_grad():
        assert torch.equal(m3(x), ref[0])


def test_save_load_packed_fp8(pkg, dev, tmp_path):
    w = pkg.WORKLOADS["C5"].with_T(300)
    params, codes, _ = pkg.synth.make_fp8_params(w)
    m = _layer(pkg, dev, w, params)
    m.load_fp8(*[codes[k].to(dev) for k in pkg.checkpoint.FP8_KEYS])
    x = pkg.synth.make_x(w).to(dev)
    with torch.no_grad():
        ref = m(x)
    path = tmp_path / "fp8.safetensors"
    pkg.checkpoint.save_packed(m, str(path))
    m2 = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg())
    assert pkg.checkpoint.load_packed(m2, str(path), device=dev) is True
    assert m2.fp8_weights
    with torch.no_grad():
        assert torch.equal(m2(x), ref)


def test_load_packed_rejects_other_shape(pkg, dev, tmp_path):
    w = pkg.WORKLOADS["C1"]
    m = _layer(pkg, dev, w, pkg.synth.make_params(w))
    path = tmp_path / "l.safetensors"
    pkg.checkpoint.save_packed(m, str(path))
    other = pkg.TuckerMoE(w.d_in, w.d_out + 16, w.cfg())
    with pytest.raises(ValueError, match="d_out"):
        pkg.checkpoint.load_packed(other, str(path), device=dev)
