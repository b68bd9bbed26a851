"""The reference blocks' Tucker-MoE sub-blocks on MI355X (gfx950).

TuckerFFN is the FFN of pure_torch_mlx/model.py's TransformerBlock
(:292-296 parameters, :337-341 forward):
    x_f   = norm_ffn(x_res)
    gate  = ffn_gate(x_f);  up = ffn_up(x_f)
    dn    = ffn_down(F.silu(gate) * up)
    x_res = x_res + ls_ffn(dn)
TuckerOutProj is Mamba3Block's output sub-block (:144, :140, :148 parameters,
:258-260 forward):
    out = mid + ls_out_proj(out_proj(norm_out_proj(mid)))

Both hold the reference's attribute names, so a TransformerBlock / Mamba3Block
state_dict restricted to them loads unchanged. On the device each is a few
launches and no elementwise pass of its own:
    norm       tmoe_rmsnorm_rows
    gate, up   tmoe_forward_glu (the two fronts in one launch)   h = silu(gate) * up
    down       tmoe_forward_epi(TMOE_EPI_RESIDUAL_SCALE, x_res, gamma)
Every product and elementwise op computes in fp32 and rounds to the parameter
dtype where the reference module's op would return a tensor of that dtype.
Inference only; HIP devices only.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from . import _lib
from .module import RMSNorm, TuckerMoE


class LayerScale(nn.Module):
    """gamma (dim), init_value 1.0 (model.py:30-36). Applied inside the
    out-projection's epilogue by the sub-blocks below; called on its own it is
    gamma * x on the device."""

    def __init__(self, dim: int, init_value: float = 1.0):
        super().__init__()
        self.gamma = nn.Parameter(torch.ones(dim) * init_value)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.gamma * x


def _check_input(x: torch.Tensor, d: int, dtype: torch.dtype, who: str) -> None:
    if x.device.type != "cuda":
        raise RuntimeError(f"{who} runs on HIP devices only; input is on {x.device}")
    if x.shape[-1] != d or x.dtype != dtype:
        raise RuntimeError(f"{who}: input (..., {x.shape[-1]}) {x.dtype}; expected (..., {d}) "
                           f"{dtype}")


def _same_plan(a: _lib.Plan, b: _lib.Plan) -> bool:
    return all(getattr(a.shape, f) == getattr(b.shape, f) for f, _ in _lib.TmoeShape._fields_)


def glu_pair(gate: TuckerMoE, up: TuckerMoE, x: torch.Tensor) -> torch.Tensor:
    """R(R(silu(gate(x))) * up(x)) for two layers of one shape (tmoe_forward_glu: the
    two fronts in one launch); (T, d_out). Layers whose plans differ (shape, dtype,
    fp8 weights, router mode) take tmoe_forward then tmoe_forward_epi instead."""
    pg, pu = gate.plan(), up.plan()
    if not _same_plan(pg, pu):
        g = gate(x)
        return up.forward_raw(x, epi=_lib.TMOE_EPI_GLU, epi_a=g, out=g)[0]
    T = x.shape[0]
    d_out = gate.U_out.shape[1]
    packed_g, packed_u = gate.packed(), up.packed()
    out = torch.empty(T, d_out, dtype=x.dtype, device=x.device)
    nws = pg.workspace_bytes(T)
    wsg = torch.empty(max(nws, 1), dtype=torch.uint8, device=x.device)
    wsu = torch.empty(max(nws, 1), dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        _lib.check(_lib.lib().tmoe_forward_glu(
            pg.ptr, x.data_ptr(), T, packed_g.data_ptr(), packed_u.data_ptr(), out.data_ptr(),
            wsg.data_ptr(), wsu.data_ptr(), nws, torch.cuda.current_stream(x.device).cuda_stream))
    return out


class TuckerFFN(nn.Module):
    """TransformerBlock's FFN sub-block (model.py:292-296, :337-341)."""

    def __init__(self, d: int, cfg):
        super().__init__()
        d_ff = getattr(cfg, "ffn_expand", 6) * d       # config.py: ffn_expand = 6
        self.norm_ffn = RMSNorm(d, eps=cfg.rms_norm_eps)
        self.ffn_gate = TuckerMoE(d, d_ff, cfg)
        self.ffn_up = TuckerMoE(d, d_ff, cfg)
        self.ffn_down = TuckerMoE(d_ff, d, cfg)
        self.ls_ffn = LayerScale(d)

    def forward(self, x_res: torch.Tensor, inplace: bool = False) -> torch.Tensor:
        """x_res (..., d) -> x_res + ls_ffn(ffn_down(silu(ffn_gate(x_f)) * ffn_up(x_f))),
        x_f = norm_ffn(x_res). With inplace=True the result is written into x_res
        (which must then be contiguous) and x_res is returned."""
        d = self.norm_ffn.weight.shape[0]
        _check_input(x_res, d, self.ffn_gate.U_in.dtype, "TuckerFFN")
        if inplace and not x_res.is_contiguous():
            raise RuntimeError("TuckerFFN: inplace needs a contiguous x_res")
        X = x_res.reshape(-1, d)
        if not X.is_contiguous():
            X = X.contiguous()
        x_f = self.norm_ffn(X)
        h = glu_pair(self.ffn_gate, self.ffn_up, x_f)
        out = X if inplace else None
        out = self.ffn_down.forward_raw(h, epi=_lib.TMOE_EPI_RESIDUAL_SCALE, epi_a=X,
                                        epi_b=self.ls_ffn.gamma, out=out)[0]
        return x_res if inplace else out.reshape(x_res.shape)

    def stages(self, x_res: torch.Tensor) -> dict:
        """The sub-block's intermediates (x_f, gate, h, out), each (T, .), computed
        by the same launches as forward()."""
        d = self.norm_ffn.weight.shape[0]
        X = x_res.reshape(-1, d).contiguous()
        x_f = self.norm_ffn(X)
        gate = self.ffn_gate(x_f)
        h = self.ffn_up.forward_raw(x_f, epi=_lib.TMOE_EPI_GLU, epi_a=gate)[0]
        out = self.ffn_down.forward_raw(h, epi=_lib.TMOE_EPI_RESIDUAL_SCALE, epi_a=X,
                                        epi_b=self.ls_ffn.gamma)[0]
        return {"x_f": x_f, "gate": gate, "h": h, "out": out}


class TuckerOutProj(nn.Module):
    """Mamba3Block's output sub-block (model.py:140, :144, :148, :258-260)."""

    def __init__(self, d: int, cfg):
        super().__init__()
        self.norm_out_proj = RMSNorm(d, eps=cfg.rms_norm_eps)
        self.out_proj = TuckerMoE(d, d, cfg)
        self.ls_out_proj = LayerScale(d)

    def forward(self, mid: torch.Tensor, inplace: bool = False) -> torch.Tensor:
        """mid (..., d) -> mid + ls_out_proj(out_proj(norm_out_proj(mid)))."""
        d = self.norm_out_proj.weight.shape[0]
        _check_input(mid, d, self.out_proj.U_in.dtype, "TuckerOutProj")
        if inplace and not mid.is_contiguous():
            raise RuntimeError("TuckerOutProj: inplace needs a contiguous input")
        X = mid.reshape(-1, d)
        if not X.is_contiguous():
            X = X.contiguous()
        out = self.out_proj.forward_raw(self.norm_out_proj(X), epi=_lib.TMOE_EPI_RESIDUAL_SCALE,
                                        epi_a=X, epi_b=self.ls_out_proj.gamma,
                                        out=X if inplace else None)[0]
        return mid if inplace else out.reshape(mid.shape)
