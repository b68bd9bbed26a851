"""Checkpoint formats on the CPU: the reference's .npz keys (pure_torch_mlx/weights.py)
fill the layer and sub-block modules exactly, and the packed file's metadata checks
(format, version, layout reuse) behave. The packed buffer itself needs the GPU
(tests/test_gpu_checkpoint.py)."""
import json

import numpy as np
import pytest
import torch


def _ref_ffn_arrays(pkg, f, pfx):
    """A TransformerBlock's FFN under the reference checkpoint's keys (weights.py:69-72),
    as float32 arrays like the exported .npz."""
    p = pkg.synth.make_ffn_params(f, dtype=torch.float32)
    names = {"ffn_gate": "ffn.gate_proj", "ffn_up": "ffn.up_proj", "ffn_down": "ffn.down_proj"}
    out = {}
    for k, v in p.items():
        head, _, rest = k.partition(".")
        key = f"{pfx}.{names[head]}.{rest}" if head in names else f"{pfx}.{k}"
        out[key] = v.numpy()
    return p, out


def test_load_ffn_from_reference_keys(pkg, tmp_path):
    f = pkg.FFN_WORKLOADS["F0"]
    pfx = "backbone.layers.3.block"
    p, arrays = _ref_ffn_arrays(pkg, f, pfx)
    path = tmp_path / "ckpt.npz"
    np.savez(path, **arrays)
    loaded = pkg.checkpoint.load_npz(str(path))
    m = pkg.TuckerFFN(f.d, f.cfg())
    pkg.checkpoint.load_ffn(m, loaded, pfx)
    sd = m.state_dict()
    for k, v in p.items():
        assert torch.equal(sd[k], v), k


def test_load_out_proj_from_reference_keys(pkg):
    w = pkg.Workload("op", 8, 128, 128, 8, 2, 4, 64, 128, torch.float32, 5)
    lp = pkg.synth.make_params(w, affine="random")
    pfx = "backbone.layers.0.block"
    arrays = {f"{pfx}.out_proj.{k}": v.numpy() for k, v in lp.items()}
    arrays[f"{pfx}.norm_out_proj.weight"] = np.full(128, 1.5, np.float32)
    arrays[f"{pfx}.ls_out_proj.gamma"] = np.full(128, 0.25, np.float32)
    m = pkg.TuckerOutProj(128, w.cfg())
    pkg.checkpoint.load_out_proj(m, arrays, pfx)
    for k, v in lp.items():
        assert torch.equal(m.out_proj.state_dict()[k], v), k
    assert torch.equal(m.norm_out_proj.weight.data, torch.full((128,), 1.5))
    assert torch.equal(m.ls_out_proj.gamma.data, torch.full((128,), 0.25))


def test_load_layer_bf16_rounds_like_reference(pkg):
    """The reference loader converts the float32 arrays to the module dtype
    (weights.py:11-13); load_layer does the same."""
    w = pkg.Workload("l", 8, 64, 64, 4, 2, 2, 64, 64, torch.float32, 9)
    lp = pkg.synth.make_params(w, affine="random")
    arrays = {f"x.{k}": v.numpy() for k, v in lp.items()}
    m = pkg.TuckerMoE(64, 64, w.cfg()).to(torch.bfloat16)
    pkg.checkpoint.load_layer(m, arrays, "x")
    for k, v in lp.items():
        assert torch.equal(m.state_dict()[k], v.to(torch.bfloat16)), k


def _write(path, meta, tensors=None):
    from safetensors.torch import save_file
    save_file(tensors or {"packed": torch.zeros(16, dtype=torch.uint8)}, str(path),
              metadata={"tmoe": json.dumps(meta)})


def test_packed_file_metadata_checks(pkg, tmp_path):
    ck = pkg.checkpoint
    good = {"format": ck.FORMAT, "format_version": ck.FORMAT_VERSION}
    _write(tmp_path / "a.safetensors", good)
    meta, t = ck.read_packed(str(tmp_path / "a.safetensors"))
    assert meta == good and set(t) == {"packed"}
    _write(tmp_path / "b.safetensors", {"format": "other"})
    with pytest.raises(ValueError, match="not a"):
        ck.read_packed(str(tmp_path / "b.safetensors"))
    _write(tmp_path / "c.safetensors", dict(good, format_version=99))
    with pytest.raises(ValueError, match="version"):
        ck.read_packed(str(tmp_path / "c.safetensors"))
    lv = pkg._lib.lib().tmoe_packed_layout_version()
    assert ck.packed_reusable({"packed_layout": lv, "packed_bytes": 100}, 100)
    assert not ck.packed_reusable({"packed_layout": lv - 1, "packed_bytes": 100}, 100)
    assert not ck.packed_reusable({"packed_layout": lv, "packed_bytes": 99}, 100)


def test_packed_layout_version_exported(pkg):
    assert pkg._lib.lib().tmoe_packed_layout_version() >= 3


def test_export_npz_round_trip(pkg, tmp_path):
    """export_npz (the .pt -> .npz step, export_ckpt_to_npz.py:43-66): a bf16 layer's
    state dict, saved as a torch checkpoint under "model" with a non-tensor entry
    beside it, comes back through load_npz / load_layer bit-exactly; bf16 widens to
    float32 exactly."""
    w = pkg.Workload("x", 8, 64, 96, 4, 2, 2, 64, 64, torch.float32, 21)
    lp = pkg.synth.make_params(w, affine="random")
    src = pkg.TuckerMoE(64, 96, w.cfg()).to(torch.bfloat16)
    src.load_state_dict({k: v.to(torch.bfloat16) for k, v in lp.items()})
    pfx = "backbone.layers.2.block.ffn.up_proj"
    ckpt = tmp_path / "ckpt.pt"
    torch.save({"model": src.state_dict(), "step": 40, "note": "sft"}, ckpt)
    n = pkg.checkpoint.export_npz(str(ckpt), str(tmp_path / "w.npz"), prefix=pfx + ".")
    assert n == len(src.state_dict())
    arrays = pkg.checkpoint.load_npz(str(tmp_path / "w.npz"))
    assert set(arrays) == {f"{pfx}.{k}" for k in src.state_dict()}
    assert all(a.dtype == np.float32 for a in arrays.values())
    dst = pkg.TuckerMoE(64, 96, w.cfg()).to(torch.bfloat16)
    pkg.checkpoint.load_layer(dst, arrays, pfx)
    for k, v in src.state_dict().items():
        assert torch.equal(dst.state_dict()[k], v), k
    # a module and a plain dict give the same arrays
    pkg.checkpoint.export_npz(src, str(tmp_path / "m.npz"), prefix=pfx + ".")
    again = pkg.checkpoint.load_npz(str(tmp_path / "m.npz"))
    assert all(np.array_equal(again[k], arrays[k]) for k in arrays)


def test_export_npz_integer_tensors_as_float32(pkg, tmp_path):
    """As the reference's export (export_ckpt_to_npz.py:59-60, `.float()` on every
    tensor), integer and bool tensors are written as float32 with the same values
    (fp8 codes 0..255 are exact); keep_int=True keeps their dtype."""
    codes = torch.arange(256, dtype=torch.uint8)
    sd = {"U_in_q": codes, "mask": torch.tensor([True, False]), "step": torch.tensor(7),
          "w": torch.ones(3, dtype=torch.bfloat16)}
    pkg.checkpoint.export_npz(sd, str(tmp_path / "a.npz"))
    a = pkg.checkpoint.load_npz(str(tmp_path / "a.npz"))
    assert all(v.dtype == np.float32 for v in a.values())
    assert np.array_equal(a["U_in_q"], np.arange(256, dtype=np.float32))
    assert np.array_equal(a["mask"], np.array([1.0, 0.0], dtype=np.float32))
    assert a["step"] == 7.0
    pkg.checkpoint.export_npz(sd, str(tmp_path / "b.npz"), keep_int=True)
    b = pkg.checkpoint.load_npz(str(tmp_path / "b.npz"))
    assert b["U_in_q"].dtype == np.uint8 and b["mask"].dtype == np.bool_
    assert b["w"].dtype == np.float32


class _Opaque:
    pass


def test_export_npz_refuses_pickled_objects(pkg, tmp_path):
    """Checkpoint files are read with weights_only=True: one holding an arbitrary
    Python object is refused, not unpickled."""
    path = tmp_path / "bad.pt"
    torch.save({"model": {"w": torch.ones(2)}, "obj": _Opaque()}, path)
    with pytest.raises(Exception):
        pkg.checkpoint.export_npz(str(path), str(tmp_path / "o.npz"))
    assert not (tmp_path / "o.npz").exists()
