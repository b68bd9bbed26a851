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
parameter's storage, version counter, dtype or device changes, or when its
`.data` has been accessed: the reference loader writes every weight through
`param.data.copy_(...)` (pure_torch_mlx/weights.py:74-81), which leaves the
version counter unchanged, so the parameters are TrackedParameter instances
that count those accesses (any access, read or write, forces one re-pack).

fp8 weights (no counterpart in the reference): load_fp8() or quantize_fp8_()
switch a bf16 module to U_in, core and U_out held as e4m3 codes with
per-output-channel fp32 scales (see fp8.py); the layer computed is the
reference layer with the dequantised weights, which those calls also write
into the parameters (rounded to bf16) so that state_dict() describes it. While
fp8 weights are loaded they, not U_in / core / U_out, feed the kernels;
clear_fp8() returns to the parameters.
"""
from __future__ import annotations

import warnings
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib
from . import fp8 as _fp8


class TrackedParameter(nn.Parameter):
    """nn.Parameter whose in-place writes through `.data` are seen.

    In-place writes through `param.data` (the reference loader,
    pure_torch_mlx/weights.py:74-81: `moe.U_in.data.copy_(w[...])`) bypass the
    parameter's version counter, which is what a cache of derived state usually
    keys on: `.data` returns an alias with a version counter of its own. Here the
    getter hands out one alias per parameter storage (kept until the parameter's
    data changes), so writes through it move that alias's counter, which
    `tracked_gen(param)` reports along with the count of `.data` assignments;
    TuckerMoE's packed-weight cache key includes it. Reading `.data` changes
    nothing, so it costs no re-pack. Behaves as nn.Parameter otherwise
    (state_dict, load_state_dict, .to(), deepcopy keep the class)."""

    def __new__(cls, data=None, requires_grad=True):
        return super().__new__(cls, data, requires_grad)

    @property
    def data(self):
        d = self.__dict__
        cur = torch.Tensor.data.__get__(self)
        al = d.get("_tmoe_alias")
        if (al is None or al.data_ptr() != cur.data_ptr() or al.shape != cur.shape
                or al.stride() != cur.stride() or al.dtype != cur.dtype
                or al.device != cur.device):
            # a new alias (first access, or the parameter's data changed): its
            # counter starts anew, so the generation moves
            d["_tmoe_alias"] = cur
            d["_tmoe_gen"] = d.get("_tmoe_gen", 0) + 1
            return cur
        return al

    @data.setter
    def data(self, value):
        self.__dict__["_tmoe_gen"] = self.__dict__.get("_tmoe_gen", 0) + 1
        self.__dict__.pop("_tmoe_alias", None)
        torch.Tensor.data.__set__(self, value)


def tracked_gen(p: torch.Tensor):
    """(assignments of `.data`, writes through the alias `.data` returns) of a
    TrackedParameter; (0, 0) for other tensors."""
    al = p.__dict__.get("_tmoe_alias")
    return (p.__dict__.get("_tmoe_gen", 0), al._version if al is not None else 0)


def _tracked(p: nn.Parameter) -> TrackedParameter:
    return p if isinstance(p, TrackedParameter) else TrackedParameter(p.detach(), p.requires_grad)


# state_dict keys of TuckerMoE's parameters, in the order of TuckerMoE._params()
PARAM_KEYS = ("router.weight", "U_in", "inner_norm.weight", "U_expert", "core", "U_out", "bias")


class RMSNorm(nn.Module):
    """RMSNorm (model.py:19-27): weight (dim) and eps.

    As TuckerMoE.inner_norm it only holds its parameters (the kernels apply it).
    Called, it computes (x / sqrt(mean(x^2) + eps)) * weight over the last axis
    with tmoe_rmsnorm_rows (fp32 arithmetic, one rounding to x's dtype); HIP
    devices only, x and weight of one dtype (bf16 or fp32)."""

    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.weight = TrackedParameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        d = self.weight.shape[0]
        if x.device.type != "cuda":
            raise RuntimeError(f"RMSNorm runs on HIP devices only; input is on {x.device}")
        if x.shape[-1] != d or x.dtype != self.weight.dtype:
            raise RuntimeError(f"RMSNorm: input (..., {x.shape[-1]}) {x.dtype}, weight ({d}) "
                               f"{self.weight.dtype}")
        dt = _lib.dtype_code(x.dtype)
        X = x.reshape(-1, d).contiguous()
        y = torch.empty_like(X) if out is None else out
        with torch.cuda.device(X.device):
            _lib.check(_lib.lib().tmoe_rmsnorm_rows(
                X.data_ptr(), X.shape[0], d, self.weight.data_ptr(), float(self.eps), dt,
                y.data_ptr(), torch.cuda.current_stream(X.device).cuda_stream))
        return y.reshape(x.shape)


class TuckerMoE(nn.Module):
    """Tucker-decomposed top-k MoE layer, forward on MI355X (gfx950)."""

    def __init__(self, d_in: int, d_out: int, cfg):
        super().__init__()
        E = cfg.kmoe_num_experts
        r1, r2, r3 = cfg.kmoe_r1, cfg.kmoe_r2, cfg.kmoe_r3
        self.top_k = cfg.kmoe_top_k
        self.router = nn.Linear(d_in, E, bias=False)
        self.router.weight = _tracked(self.router.weight)
        self.U_in = TrackedParameter(torch.empty(d_in, r3))
        self.inner_norm = RMSNorm(r3, eps=cfg.rms_norm_eps)
        self.U_expert = TrackedParameter(torch.empty(E, r1))
        self.core = TrackedParameter(torch.empty(r1, r3, r2))
        self.U_out = TrackedParameter(torch.empty(r2, d_out))
        self.bias = TrackedParameter(torch.zeros(d_out))
        self._plan: Optional[_lib.Plan] = None
        self._packed: Optional[torch.Tensor] = None
        self._packed_key = None
        self._warned_grad = False
        self._fp8: Optional[dict] = None   # e4m3 codes (uint8) and fp32 scales
        self._router = (_lib.TMOE_ROUTER_SOFTMAX_TOPK, 10.0, 0.5)
        self._plan_flags = 0   # _lib.TMOE_FLAG_*: 0 lets the library choose the form

    # -- packed-weight cache -------------------------------------------------
    def _params(self):
        return (self.router.weight, self.U_in, self.inner_norm.weight, self.U_expert,
                self.core, self.U_out, self.bias)

    def _fp8_tensors(self):
        f = self._fp8
        return (f["U_in_q"], f["U_in_scale"], f["core_q"], f["core_scale"], f["U_out_q"],
                f["U_out_scale"])

    def _key(self):
        ts = self._params() + (self._fp8_tensors() if self._fp8 is not None else ())
        return tuple((p.data_ptr(), p._version, tracked_gen(p), p.dtype, p.device) for p in ts)

    def _load_from_state_dict(self, *args, **kwargs):
        # load_state_dict copies in place (moving the version counters); forget the
        # packed copy regardless
        self.refresh_packed()
        return super()._load_from_state_dict(*args, **kwargs)

    def plan(self) -> _lib.Plan:
        dtype = self.U_in.dtype
        fp8 = self._fp8 is not None
        if (self._plan is None or self._plan.dtype != dtype or self._plan.fp8_weights != fp8
                or self._plan.router != self._router or self._plan.flags != self._plan_flags):
            d_in, r3 = self.U_in.shape
            r2, d_out = self.U_out.shape
            E, r1 = self.U_expert.shape
            self._plan = _lib.Plan(d_in, d_out, E, self.top_k, r1, r2, r3, dtype,
                                   float(self.inner_norm.eps), fp8_weights=fp8,
                                   router=self._router, flags=self._plan_flags)
        return self._plan

    def set_fold(self, enabled: bool = True) -> "TuckerMoE":
        """Whether the library may fold the core into the out-projection (default).

        The folded form computes the same layer as one GEMM of the Khatri-Rao rows
        c (x) z against W = core U_out (packed once), chosen by the library when it
        takes fewer multiply-adds per token; ``set_fold(False)`` keeps the core
        contraction (model.py:87-98) and the out-projection (model.py:101) as two
        GEMMs. Takes effect at the next forward (the weights are re-packed)."""
        flags = (self._plan_flags & ~_lib.TMOE_FLAG_NO_FOLD) | (
            0 if enabled else _lib.TMOE_FLAG_NO_FOLD)
        if flags != self._plan_flags:
            self._plan_flags = flags
            self._plan = None
            self._packed = None
            self._packed_key = None
        return self

    def set_fuse(self, enabled: bool = True) -> "TuckerMoE":
        """Whether the library may run a large-T forward as one launch (default): the
        front and the out-projection in one persistent grid that hands c (x) z over
        inside each XCD (folded bf16 plans with r3 = 256, E <= 32, d_out a multiple
        of 288, T >= 8192 at d_out = 2304). ``set_fuse(False)`` keeps two launches.
        The packed weights are the same either way."""
        flags = (self._plan_flags & ~_lib.TMOE_FLAG_NO_FUSE) | (
            0 if enabled else _lib.TMOE_FLAG_NO_FUSE)
        if flags != self._plan_flags:
            self._plan_flags = flags
            self._plan = None
        return self

    def check_signals(self) -> None:
        """Synchronises the parameters' device and raises RuntimeError (a
        _lib.TmoeError with code TMOE_ESIGNAL) if a forward of this module since the
        last check lost an in-launch signal: a kernel whose work-groups hand data to
        each other gave up waiting (the affected output rows are NaN or stale).
        forward() runs the same check without synchronising, for the forwards that
        have completed."""
        if self._plan is None:
            return
        if self.U_in.device.type == "cuda":
            torch.cuda.synchronize(self.U_in.device)
        self._plan.signal_status(clear=True)

    # -- router mode -------------------------------------------------------------
    def set_router_mode(self, mode: str = "softmax_topk", scale: float = 10.0,
                        temperature: float = 0.5) -> None:
        """"softmax_topk" (default): the reference module's router, model.py:75-77.
        "capped": the router the trained checkpoints use
        (mamba3_mlx/mlx_model/tucker_moe.py:107-114): scores = scale *
        tanh(logits / scale) / temperature, top-k of the scores, weights = the
        softmax over all experts at the selected ones / (their sum + 1e-6)."""
        if mode == "softmax_topk":
            self._router = (_lib.TMOE_ROUTER_SOFTMAX_TOPK, 10.0, 0.5)
        elif mode == "capped":
            if not (scale > 0 and temperature > 0):
                raise ValueError("scale and temperature must be > 0")
            self._router = (_lib.TMOE_ROUTER_CAPPED, float(scale), float(temperature))
        else:
            raise ValueError(f"router mode {mode!r}: 'softmax_topk' or 'capped'")
        self._plan = None

    @property
    def router_mode(self):
        """("softmax_topk",) or ("capped", scale, temperature)."""
        if self._router[0] == _lib.TMOE_ROUTER_CAPPED:
            return ("capped", self._router[1], self._router[2])
        return ("softmax_topk",)

    # -- fp8 weights -----------------------------------------------------------
    def load_fp8(self, U_in_q, U_in_scale, core_q, core_scale, U_out_q, U_out_scale) -> None:
        """Loads e4m3 codes (torch.float8_e4m3fn or their uint8 bits) and fp32
        per-output-channel scales of U_in (d_in, r3) / (r3,), core (r1, r3, r2) /
        (r1, r2) and U_out (r2, d_out) / (d_out,). The module must be bfloat16."""
        if self.U_in.dtype != torch.bfloat16:
            raise RuntimeError(f"TuckerMoE: fp8 weights need a bfloat16 module, not "
                               f"{self.U_in.dtype}")
        dev = self.U_in.device
        shapes = {"U_in": (tuple(self.U_in.shape), (self.U_in.shape[1],)),
                  "core": (tuple(self.core.shape), (self.core.shape[0], self.core.shape[2])),
                  "U_out": (tuple(self.U_out.shape), (self.U_out.shape[1],))}
        given = {"U_in": (U_in_q, U_in_scale), "core": (core_q, core_scale),
                 "U_out": (U_out_q, U_out_scale)}
        f = {}
        for k, (q, sc) in given.items():
            qs, ss = shapes[k]
            if q.dtype not in (torch.float8_e4m3fn, torch.uint8):
                raise RuntimeError(f"TuckerMoE.load_fp8: {k} codes must be float8_e4m3fn or "
                                   f"uint8, not {q.dtype}")
            if tuple(q.shape) != qs or tuple(sc.shape) != ss:
                raise RuntimeError(f"TuckerMoE.load_fp8: {k} codes {tuple(q.shape)} / scales "
                                   f"{tuple(sc.shape)}, expected {qs} / {ss}")
            q8 = q.view(torch.uint8) if q.dtype == torch.float8_e4m3fn else q
            f[f"{k}_q"] = q8.to(dev).contiguous()
            f[f"{k}_scale"] = sc.to(device=dev, dtype=torch.float32).contiguous()
        with torch.no_grad():
            for k, p in (("U_in", self.U_in), ("core", self.core), ("U_out", self.U_out)):
                p.copy_(_fp8.dequantize(f[f"{k}_q"], f[f"{k}_scale"], k).to(p.dtype))
        self._fp8 = f
        self.refresh_packed()
        self._plan = None

    def quantize_fp8_(self) -> None:
        """Quantises the current U_in, core and U_out (per-output-channel absmax
        scaling, fp8.quantize) and loads them with load_fp8()."""
        q = _fp8.quantize_params({"U_in": self.U_in, "core": self.core, "U_out": self.U_out})
        self.load_fp8(q["U_in_q"], q["U_in_scale"], q["core_q"], q["core_scale"],
                      q["U_out_q"], q["U_out_scale"])

    def clear_fp8(self) -> None:
        """Drops the fp8 weights; the parameters feed the kernels again."""
        self._fp8 = None
        self.refresh_packed()
        self._plan = None

    @property
    def fp8_weights(self) -> bool:
        return self._fp8 is not None

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
                if self._fp8 is None:
                    _lib.check(_lib.lib().tmoe_pack_weights(
                        plan.ptr, *[p.data_ptr() for p in params], buf.data_ptr(), stream))
                else:
                    f = self._fp8
                    for t in f.values():
                        if t.device != dev:
                            raise RuntimeError("TuckerMoE: fp8 weights are on "
                                               f"{t.device}, parameters on {dev}")
                    router_w, _, inner_w, U_expert, _, _, bias = params
                    _lib.check(_lib.lib().tmoe_pack_weights_fp8(
                        plan.ptr, router_w.data_ptr(), f["U_in_q"].data_ptr(),
                        f["U_in_scale"].data_ptr(), inner_w.data_ptr(), U_expert.data_ptr(),
                        f["core_q"].data_ptr(), f["core_scale"].data_ptr(),
                        f["U_out_q"].data_ptr(), f["U_out_scale"].data_ptr(), bias.data_ptr(),
                        buf.data_ptr(), stream))
            self._packed, self._packed_key = buf, key
        return self._packed

    def _apply(self, fn, *args, **kwargs):
        self.refresh_packed()
        self._plan = None
        out = super()._apply(fn, *args, **kwargs)
        # a conversion that replaced a parameter object keeps it tracked
        self.router.weight = _tracked(self.router.weight)
        self.inner_norm.weight = _tracked(self.inner_norm.weight)
        for name in ("U_in", "U_expert", "core", "U_out", "bias"):
            p = getattr(self, name)
            if not isinstance(p, TrackedParameter):
                setattr(self, name, _tracked(p))
        if self._fp8 is not None:
            # follow the parameters' device; codes and scales keep their dtypes
            dev = self.U_in.device
            self._fp8 = {k: v.to(dev) for k, v in self._fp8.items()}
        return out

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
        return self.forward_raw(x, routing=routing, logits=logits)

    def forward_raw(self, x: torch.Tensor, routing: bool = False, logits: bool = False,
                    epi: int = 0, epi_a: Optional[torch.Tensor] = None,
                    epi_b: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
        """forward_with_routing with a fused epilogue (tmoe_forward_epi): epi is
        _lib.TMOE_EPI_NONE / _GLU (out = silu(epi_a) * y) / _RESIDUAL_SCALE
        (out = epi_a + epi_b * y), y = this layer's output; epi_a (..., d_out) and
        epi_b (d_out) in the parameter dtype. `out` (T, d_out), which may be
        epi_a itself, receives the result."""
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
        # an earlier forward's kernel that lost an in-launch signal (host memory the
        # kernels write: no synchronisation) is reported before any new work
        plan.signal_status(clear=True)
        packed = self.packed()
        dev = X.device
        if out is None:
            out = torch.empty(T, d_out, dtype=dtype, device=dev)
        elif (out.shape != (T, d_out) or out.dtype != dtype or out.device != dev
              or not out.is_contiguous()):
            raise RuntimeError(f"TuckerMoE: out must be a contiguous ({T}, {d_out}) {dtype} tensor")
        ea = eb = None
        if epi != _lib.TMOE_EPI_NONE:
            ea = epi_a.reshape(T, d_out) if epi_a is not None else None
            if ea is None or ea.dtype != dtype or ea.device != dev or not ea.is_contiguous():
                raise RuntimeError(f"TuckerMoE: epi_a must be a contiguous ({T}, {d_out}) "
                                   f"{dtype} tensor on {dev}")
        if epi == _lib.TMOE_EPI_RESIDUAL_SCALE:
            eb = epi_b
            if (eb is None or eb.shape != (d_out,) or eb.dtype != dtype or eb.device != dev
                    or not eb.is_contiguous()):
                raise RuntimeError(f"TuckerMoE: epi_b must be a contiguous ({d_out},) {dtype} "
                                   f"tensor on {dev}")
        idx = torch.empty(T, self.top_k, dtype=torch.int32, device=dev) if routing else None
        w = torch.empty(T, self.top_k, dtype=torch.float32, device=dev) if routing else None
        lg = torch.empty(T, E, dtype=torch.float32, device=dev) if logits else None
        ws_bytes = plan.workspace_bytes(T)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            stream = torch.cuda.current_stream(dev).cuda_stream
            _lib.check(_lib.lib().tmoe_forward_epi(
                plan.ptr, X.data_ptr(), T, packed.data_ptr(), out.data_ptr(),
                idx.data_ptr() if idx is not None else None,
                w.data_ptr() if w is not None else None,
                lg.data_ptr() if lg is not None else None,
                ws.data_ptr(), ws_bytes, epi, ea.data_ptr() if ea is not None else None,
                eb.data_ptr() if eb is not None else None, stream))
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
