"""Drop-in TuckerMoE module backed by the gfx950 C-ABI library.

Mirrors the reference module pure_torch_mlx/model.py:41-102:
  - constructor TuckerMoE(d_in, d_out, cfg) reading cfg.kmoe_num_experts,
    kmoe_top_k, kmoe_r1/_r2/_r3 and rms_norm_eps (model.py:54-66);
  - the same parameters, shapes and state_dict keys: router.weight (E, d_in),
    U_in (d_in, r3), inner_norm.weight (r3), U_expert (E, r1),
    core (r1, r3, r2), U_out (r2, d_out), bias (d_out), so the reference loader
    _load_tucker (pure_torch_mlx/weights.py:74-81) fills it unchanged;
  - forward(x: (..., d_in)) -> (..., d_out) in the parameter dtype (model.py:68-102).

forward runs only on HIP devices, through libtmoe.so; a CPU tensor, a missing
library or an unsupported shape raises. The module is inference-only: its
output carries no autograd history.

The kernels read a packed copy of the parameters. It is rebuilt when a
parameter's storage, version counter, dtype or device changes. Writes through
`param.data` (which the reference loader uses) do not move the version counter,
so call refresh_packed() after such a write, or load with load_tucker() below.
"""
from __future__ import annotations

import warnings
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib


class RMSNorm(nn.Module):
    """Holds inner_norm.weight and eps (model.py:19-27); applied inside the kernels."""

    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps


class TuckerMoE(nn.Module):
    """Tucker-decomposed top-k MoE layer, forward on MI355X (gfx950)."""

    def __init__(self, d_in: int, d_out: int, cfg):
        super().__init__()
        E = cfg.kmoe_num_experts
        r1, r2, r3 = cfg.kmoe_r1, cfg.kmoe_r2, cfg.kmoe_r3
        self.top_k = cfg.kmoe_top_k
        self.router = nn.Linear(d_in, E, bias=False)
        self.U_in = nn.Parameter(torch.empty(d_in, r3))
        self.inner_norm = RMSNorm(r3, eps=cfg.rms_norm_eps)
        self.U_expert = nn.Parameter(torch.empty(E, r1))
        self.core = nn.Parameter(torch.empty(r1, r3, r2))
        self.U_out = nn.Parameter(torch.empty(r2, d_out))
        self.bias = nn.Parameter(torch.zeros(d_out))
        self._plan: Optional[_lib.Plan] = None
        self._packed: Optional[torch.Tensor] = None
        self._packed_key = None
        self._warned_grad = False

    # -- packed-weight cache -------------------------------------------------
    def _params(self):
        return (self.router.weight, self.U_in, self.inner_norm.weight, self.U_expert,
                self.core, self.U_out, self.bias)

    def _key(self):
        return tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in self._params())

    def plan(self) -> _lib.Plan:
        dtype = self.U_in.dtype
        if self._plan is None or self._plan.dtype != dtype:
            d_in, r3 = self.U_in.shape
            r2, d_out = self.U_out.shape
            E, r1 = self.U_expert.shape
            self._plan = _lib.Plan(d_in, d_out, E, self.top_k, r1, r2, r3, dtype,
                                   float(self.inner_norm.eps))
        return self._plan

    def refresh_packed(self) -> None:
        """Forgets the packed copy; the next forward re-packs the parameters."""
        self._packed = None
        self._packed_key = None

    def packed(self) -> torch.Tensor:
        key = self._key()
        if self._packed is None or self._packed_key != key:
            plan = self.plan()
            params = self._params()
            dev, dtype = params[0].device, params[0].dtype
            for p in params:
                if p.device != dev or p.dtype != dtype:
                    raise RuntimeError("TuckerMoE: all parameters must share one device and dtype")
                if not p.is_contiguous():
                    raise RuntimeError("TuckerMoE: parameters must be contiguous")
            if dev.type != "cuda":
                raise RuntimeError(f"TuckerMoE runs on HIP devices only; parameters are on {dev}")
            buf = torch.empty(plan.packed_bytes(), dtype=torch.uint8, device=dev)
            with torch.cuda.device(dev):
                stream = torch.cuda.current_stream(dev).cuda_stream
                _lib.check(_lib.lib().tmoe_pack_weights(
                    plan.ptr, *[p.data_ptr() for p in params], buf.data_ptr(), stream))
            self._packed, self._packed_key = buf, key
        return self._packed

    def _apply(self, fn, *args, **kwargs):
        self.refresh_packed()
        self._plan = None
        return super()._apply(fn, *args, **kwargs)

    # -- forward ---------------------------------------------------------------
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x: (..., d_in) -> (..., d_out)"""
        return self.forward_with_routing(x, routing=False)[0]

    def forward_with_routing(self, x: torch.Tensor, routing: bool = True, logits: bool = False
                             ) -> Tuple[torch.Tensor, Optional[torch.Tensor],
                                        Optional[torch.Tensor], Optional[torch.Tensor]]:
        """Returns (out, topk_idx int64 (T, k), topk_w (T, k) f32, logits (T, E) f32).

        topk_idx / topk_w are the values model.py:76-77 computes (indices in
        descending logit order); they and `logits` are None unless requested.
        """
        *batch, d_in = x.shape
        dtype = self.U_in.dtype
        if x.device.type != "cuda":
            raise RuntimeError(f"TuckerMoE runs on HIP devices only; input is on {x.device}")
        if x.dtype != dtype:
            raise RuntimeError(f"TuckerMoE: input dtype {x.dtype} != parameter dtype {dtype}")
        if d_in != self.U_in.shape[0]:
            raise RuntimeError(f"TuckerMoE: input feature size {d_in} != d_in {self.U_in.shape[0]}")
        if torch.is_grad_enabled() and (x.requires_grad or self.U_in.requires_grad) \
                and not self._warned_grad:
            warnings.warn("TuckerMoE (gfx950) is forward-only; its output carries no gradient")
            self._warned_grad = True
        X = x.reshape(-1, d_in).contiguous()
        T = X.shape[0]
        d_out = self.U_out.shape[1]
        E = self.U_expert.shape[0]
        plan = self.plan()
        packed = self.packed()
        dev = X.device
        out = torch.empty(T, d_out, dtype=dtype, device=dev)
        idx = torch.empty(T, self.top_k, dtype=torch.int32, device=dev) if routing else None
        w = torch.empty(T, self.top_k, dtype=torch.float32, device=dev) if routing else None
        lg = torch.empty(T, E, dtype=torch.float32, device=dev) if logits else None
        ws_bytes = plan.workspace_bytes(T)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            stream = torch.cuda.current_stream(dev).cuda_stream
            _lib.check(_lib.lib().tmoe_forward(
                plan.ptr, X.data_ptr(), T, packed.data_ptr(), out.data_ptr(),
                idx.data_ptr() if idx is not None else None,
                w.data_ptr() if w is not None else None,
                lg.data_ptr() if lg is not None else None,
                ws.data_ptr(), ws_bytes, stream))
        out = out.reshape(*batch, d_out)
        return out, (idx.long() if idx is not None else None), w, lg


def load_tucker(moe: TuckerMoE, w: dict, pfx: str) -> None:
    """Fills `moe` from checkpoint arrays keyed like pure_torch_mlx/weights.py:74-81
    ({pfx}.router.weight, {pfx}.U_in, ...) and refreshes the packed copy."""
    with torch.no_grad():
        moe.router.weight.copy_(torch.as_tensor(w[f"{pfx}.router.weight"]))
        moe.U_in.copy_(torch.as_tensor(w[f"{pfx}.U_in"]))
        moe.inner_norm.weight.copy_(torch.as_tensor(w[f"{pfx}.inner_norm.weight"]))
        moe.U_expert.copy_(torch.as_tensor(w[f"{pfx}.U_expert"]))
        moe.core.copy_(torch.as_tensor(w[f"{pfx}.core"]))
        moe.U_out.copy_(torch.as_tensor(w[f"{pfx}.U_out"]))
        moe.bias.copy_(torch.as_tensor(w[f"{pfx}.bias"]))
    moe.refresh_packed()
