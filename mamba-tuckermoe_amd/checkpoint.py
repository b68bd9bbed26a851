"""Checkpoint formats: the reference's `.npz` keys, and a versioned packed file.

1. The reference's checkpoint (pure_torch_mlx/weights.py:16-81) is one `.npz` of
   float arrays under block prefixes `backbone.layers.{i}.block`:
     TuckerMoE layer  {pfx}.router.weight, .U_in, .inner_norm.weight, .U_expert,
                      .core, .U_out, .bias                          (weights.py:74-81)
     TransformerBlock FFN  {pfx}.norm_ffn.weight, {pfx}.ffn.gate_proj.*,
                      {pfx}.ffn.up_proj.*, {pfx}.ffn.down_proj.*, {pfx}.ls_ffn.gamma
                                                                    (weights.py:62-72)
     Mamba3Block output  {pfx}.norm_out_proj.weight, {pfx}.out_proj.*,
                      {pfx}.ls_out_proj.gamma                       (weights.py:43-56)
   load_npz reads it with numpy's default loader (no pickles); load_layer,
   load_ffn and load_out_proj fill this package's modules from those keys and
   refresh their packed copies. export_npz writes such a file: every floating
   tensor of a state dict (or of a module, or of a torch checkpoint holding one
   under "model" or "state_dict") as a float32 array under its key, the export
   step of sft_cot_bundle/scripts/export/export_ckpt_to_npz.py:24-66. Checkpoint
   files are read with torch.load(weights_only=True) only: a file that needs
   unpickling of arbitrary objects is refused.

2. The packed file (no counterpart in the reference) holds one TuckerMoE: its
   parameters under the reference's keys (so that it re-derives everything), fp8
   codes and scales when the layer has them, and the kernels' packed buffer, with
   the plan's shape, dtype, router mode and the library's packed-layout version
   (tmoe_packed_layout_version) as metadata. It is a safetensors file (tensors
   plus a string table; nothing in it is executed on load). load_packed uses the
   stored buffer as is when the layout version and size match the running
   library, and packs again from the stored parameters otherwise.
"""
from __future__ import annotations

import json
from typing import Dict, Optional

import numpy as np
import torch

from . import _lib
from .module import PARAM_KEYS, TuckerMoE, load_tucker

FORMAT = "tmoe-packed"
FORMAT_VERSION = 1
FP8_KEYS = ("U_in_q", "U_in_scale", "core_q", "core_scale", "U_out_q", "U_out_scale")


def load_npz(path: str) -> Dict[str, np.ndarray]:
    """The arrays of a reference checkpoint (np.load without pickles)."""
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def checkpoint_state_dict(obj) -> Dict[str, torch.Tensor]:
    """The tensors of a checkpoint object: obj["model"], else obj["state_dict"], else
    obj itself when it is a dict; non-tensor entries are dropped
    (export_ckpt_to_npz.py:24-40). A torch.nn.Module gives its state_dict()."""
    if isinstance(obj, torch.nn.Module):
        obj = obj.state_dict()
    if not isinstance(obj, dict):
        raise TypeError(f"no state dict in a {type(obj).__name__}")
    raw = obj.get("model", obj.get("state_dict", obj))
    if isinstance(raw, torch.nn.Module):
        raw = raw.state_dict()
    if not isinstance(raw, dict):
        raise TypeError("the checkpoint's state dict is not a dict")
    return {str(k): v for k, v in raw.items() if torch.is_tensor(v)}


def export_npz(src, path: str, prefix: str = "", compressed: bool = True,
               keep_int: bool = False) -> int:
    """Writes every tensor of src (a state dict, a module, a checkpoint dict, or the
    path of a torch checkpoint file, read with weights_only=True) to the .npz at path
    as a float32 array (bf16 / fp16 widened exactly), each key prefixed with `prefix`
    (e.g. "backbone.layers.0.block.ffn.gate_proj." for one layer's own state dict).
    As the reference's export step, integer and bool tensors are converted to float32
    too (export_ckpt_to_npz.py:59-60: `.float()` on every tensor; fp8 codes 0..255 are
    exact in float32); keep_int=True writes them in their own dtype instead. Returns
    the number of arrays written (export_ckpt_to_npz.py:43-66)."""
    if isinstance(src, (str, bytes)) or hasattr(src, "__fspath__"):
        src = torch.load(src, map_location="cpu", weights_only=True)
    sd = checkpoint_state_dict(src)
    arrays = {}
    for k, t in sd.items():
        t = t.detach().cpu()
        arrays[prefix + k] = (t if keep_int and not t.is_floating_point() else t.float()).numpy()
    (np.savez_compressed if compressed else np.savez)(path, **arrays)
    return len(arrays)


def load_layer(moe: TuckerMoE, arrays: Dict, pfx: str) -> None:
    """One TuckerMoE from the keys {pfx}.router.weight ... {pfx}.bias (weights.py:74-81)."""
    load_tucker(moe, {k: _as_tensor(v, moe.U_in.dtype) for k, v in arrays.items()
                      if k.startswith(pfx + ".")}, pfx)


def load_ffn(ffn, arrays: Dict, pfx: str) -> None:
    """TuckerFFN from a TransformerBlock's keys (weights.py:69-72): norm_ffn.weight,
    ffn.gate_proj / ffn.up_proj / ffn.down_proj (TuckerMoE keys), ls_ffn.gamma."""
    for name, key in (("ffn_gate", "gate_proj"), ("ffn_up", "up_proj"),
                      ("ffn_down", "down_proj")):
        load_layer(getattr(ffn, name), arrays, f"{pfx}.ffn.{key}")
    _copy(ffn.norm_ffn.weight, arrays[f"{pfx}.norm_ffn.weight"])
    _copy(ffn.ls_ffn.gamma, arrays[f"{pfx}.ls_ffn.gamma"])


def load_out_proj(outp, arrays: Dict, pfx: str) -> None:
    """TuckerOutProj from a Mamba3Block's keys (weights.py:43-56): norm_out_proj.weight,
    out_proj (TuckerMoE keys), ls_out_proj.gamma."""
    load_layer(outp.out_proj, arrays, f"{pfx}.out_proj")
    _copy(outp.norm_out_proj.weight, arrays[f"{pfx}.norm_out_proj.weight"])
    _copy(outp.ls_out_proj.gamma, arrays[f"{pfx}.ls_out_proj.gamma"])


def _as_tensor(v, dtype):
    t = torch.as_tensor(v)
    return t.to(dtype) if t.is_floating_point() else t


def _copy(param, value) -> None:
    with torch.no_grad():
        param.copy_(_as_tensor(value, param.dtype))


# -- the packed file ------------------------------------------------------------------
def _meta(moe: TuckerMoE, plan: _lib.Plan) -> dict:
    s = plan.shape
    return {"format": FORMAT, "format_version": FORMAT_VERSION,
            "packed_layout": int(_lib.lib().tmoe_packed_layout_version()),
            "packed_bytes": plan.packed_bytes(),
            "shape": {"d_in": s.d_in, "d_out": s.d_out, "E": s.E, "k": s.k, "r1": s.r1,
                      "r2": s.r2, "r3": s.r3, "eps": float(s.eps)},
            "dtype": str(moe.U_in.dtype).replace("torch.", ""),
            "fp8_weights": moe.fp8_weights,
            "router": list(moe.router_mode)}


def save_packed(moe: TuckerMoE, path: str) -> None:
    """Writes the layer (parameters, fp8 codes and scales, packed buffer) to `path`."""
    from safetensors.torch import save_file
    plan, packed = moe.plan(), moe.packed()
    tensors = {k: p.detach().contiguous().cpu() for k, p in zip(PARAM_KEYS, moe._params())}
    if moe.fp8_weights:
        tensors.update({k: v.contiguous().cpu() for k, v in zip(FP8_KEYS, moe._fp8_tensors())})
    tensors["packed"] = packed.cpu()
    save_file(tensors, path, metadata={"tmoe": json.dumps(_meta(moe, plan))})


def read_packed(path: str):
    """(metadata dict, tensors dict) of a packed file; raises if it is not one."""
    from safetensors import safe_open
    with safe_open(path, framework="pt") as f:
        meta = json.loads((f.metadata() or {}).get("tmoe", "{}"))
        if meta.get("format") != FORMAT:
            raise ValueError(f"{path}: not a {FORMAT} file")
        if meta.get("format_version") != FORMAT_VERSION:
            raise ValueError(f"{path}: {FORMAT} version {meta.get('format_version')}, this "
                             f"package reads version {FORMAT_VERSION}")
        tensors = {k: f.get_tensor(k) for k in f.keys()}
    return meta, tensors


def packed_reusable(meta: dict, packed_bytes: int) -> bool:
    """Whether a stored packed buffer can feed this library's kernels as is."""
    return (meta.get("packed_layout") == int(_lib.lib().tmoe_packed_layout_version())
            and meta.get("packed_bytes") == packed_bytes)


def load_packed(moe: TuckerMoE, path: str, device: Optional[torch.device] = None) -> bool:
    """Fills `moe` (constructed with the file's shape) from a packed file. Returns
    True when the stored packed buffer was used, False when the layer was packed
    again from the stored parameters (another layout version)."""
    meta, t = read_packed(path)
    sh = meta["shape"]
    d_in, r3 = moe.U_in.shape
    r2, d_out = moe.U_out.shape
    E, r1 = moe.U_expert.shape
    mine = {"d_in": d_in, "d_out": d_out, "E": E, "k": moe.top_k, "r1": r1, "r2": r2, "r3": r3}
    for k, v in mine.items():
        if sh[k] != v:
            raise ValueError(f"{path}: {k} = {sh[k]}, the module has {v}")
    dev = device if device is not None else moe.U_in.device
    dtype = getattr(torch, meta["dtype"])
    moe.to(dev, dtype)
    with torch.no_grad():
        for k, p in zip(PARAM_KEYS, moe._params()):
            p.copy_(t[k].to(dev))
    r = meta["router"]
    moe.set_router_mode(r[0], *r[1:])
    if meta["fp8_weights"]:
        moe.load_fp8(*[t[k] for k in FP8_KEYS])
    else:
        moe.clear_fp8()
    plan = moe.plan()
    if not packed_reusable(meta, plan.packed_bytes()):
        moe.refresh_packed()
        return False
    moe._packed = t["packed"].to(dev)
    moe._packed_key = moe._key()
    return True
