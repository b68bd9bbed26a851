"""ctypes binding of libtmoe.so, the C ABI declared in include/tmoe.h.

This is the binding a user of the reference's PyTorch module path adds: the
reference has no FFI (pure_torch_mlx/model.py is plain PyTorch), so the library
is reached from Python through ctypes. torch is imported first so that the
library resolves libamdhip64.so.7 to the HIP runtime torch already loaded (one
HIP runtime per process).

There is no fallback: if the library is missing, lib() raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (loads torch's HIP runtime before libtmoe.so)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtmoe.so")

ABI_VERSION = 12
TMOE_OK, TMOE_EINVAL, TMOE_EUNSUPPORTED, TMOE_EHIP, TMOE_ESIGNAL = 0, -1, -2, -3, -4
TMOE_F32, TMOE_BF16, TMOE_BF16_FP8W = 0, 1, 2
TMOE_ROUTER_SOFTMAX_TOPK, TMOE_ROUTER_CAPPED = 0, 1
TMOE_EPI_NONE, TMOE_EPI_GLU, TMOE_EPI_RESIDUAL_SCALE = 0, 1, 2
TMOE_FLAG_NO_FOLD = 1
TMOE_FLAG_NO_FUSE = 2
TMOE_STATUS_SIGNAL = 1
TMOE_PATH_SMALL, TMOE_PATH_DECODE, TMOE_PATH_LARGE, TMOE_PATH_FUSED = 1, 2, 3, 4
TMOE_PATH_LARGE_KR = 5
TMOE_PATH_FUSED_MID = 6
PATH_NAMES = {1: "small-T kernels", 2: "one launch (k_sk_decode)",
              3: "front + out-projection launches", 4: "one launch (k_fused_large)",
              5: "front (z, c) + out-projection forming c (x) z (k_outproj_wide_kr)",
              6: "one launch (k_fused_mid)"}
TMOE_LATENT_P_F32 = 0x100   # or'ed into a latent call's dtype: p and dp are fp32
N_STAGES = 3
STAGE_NAMES = ("front", "core", "out_proj")

# Every function include/tmoe.h declares.
EXPORTED = (
    "tmoe_abi_version", "tmoe_last_error", "tmoe_plan_create", "tmoe_plan_destroy",
    "tmoe_packed_bytes", "tmoe_packed_layout_version", "tmoe_workspace_bytes",
    "tmoe_plan_core_rank", "tmoe_plan_folded",
    "tmoe_pack_weights", "tmoe_pack_weights_fp8",
    "tmoe_forward", "tmoe_forward_epi", "tmoe_forward_glu", "tmoe_rmsnorm_rows",
    "tmoe_static_scratch_bytes", "tmoe_forward_static",
    "tmoe_latent_workspace_bytes", "tmoe_latent_forward", "tmoe_latent_backward",
    "tmoe_signal_status", "tmoe_set_wait_polls", "tmoe_forward_path",
    "tmoe_prof_enable", "tmoe_prof_read",
)


class TmoeShape(ctypes.Structure):
    """struct tmoe_shape."""
    _fields_ = [
        ("d_in", ctypes.c_int64), ("d_out", ctypes.c_int64),
        ("E", ctypes.c_int64), ("k", ctypes.c_int64),
        ("r1", ctypes.c_int64), ("r2", ctypes.c_int64), ("r3", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("eps", ctypes.c_float),
        ("router_mode", ctypes.c_int32), ("router_scale", ctypes.c_float),
        ("router_temperature", ctypes.c_float), ("flags", ctypes.c_int32),
    ]


class TmoeError(RuntimeError):
    """A negative return code of the C ABI, with tmoe_last_error()'s message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"tmoe error {code}: {message}")
        self.code = code
        self.message = message


_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """Loads libtmoe.so once; raises if it is not built or is the wrong ABI."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; build it with __graft_entry__.build() "
                "(hipcc --offload-arch=gfx950). There is no fallback path.")
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
        L.tmoe_abi_version.restype = ctypes.c_int
        L.tmoe_abi_version.argtypes = []
        L.tmoe_last_error.restype = ctypes.c_char_p
        L.tmoe_last_error.argtypes = []
        L.tmoe_plan_create.restype = ctypes.c_int
        L.tmoe_plan_create.argtypes = [ctypes.POINTER(TmoeShape), ctypes.POINTER(vp)]
        L.tmoe_plan_destroy.restype = None
        L.tmoe_plan_destroy.argtypes = [vp]
        L.tmoe_packed_bytes.restype = sz
        L.tmoe_packed_bytes.argtypes = [vp]
        L.tmoe_plan_core_rank.restype = ctypes.c_int64
        L.tmoe_plan_core_rank.argtypes = [vp]
        L.tmoe_plan_folded.restype = ctypes.c_int
        L.tmoe_plan_folded.argtypes = [vp]
        L.tmoe_packed_layout_version.restype = ctypes.c_int
        L.tmoe_packed_layout_version.argtypes = []
        L.tmoe_workspace_bytes.restype = sz
        L.tmoe_workspace_bytes.argtypes = [vp, i64]
        L.tmoe_pack_weights.restype = ctypes.c_int
        L.tmoe_pack_weights.argtypes = [vp] * 10
        L.tmoe_pack_weights_fp8.restype = ctypes.c_int
        L.tmoe_pack_weights_fp8.argtypes = [vp] * 13
        L.tmoe_forward.restype = ctypes.c_int
        L.tmoe_forward.argtypes = [vp, vp, i64, vp, vp, vp, vp, vp, vp, sz, vp]
        L.tmoe_forward_epi.restype = ctypes.c_int
        L.tmoe_forward_epi.argtypes = [vp, vp, i64, vp, vp, vp, vp, vp, vp, sz, ctypes.c_int,
                                       vp, vp, vp]
        L.tmoe_static_scratch_bytes.restype = sz
        L.tmoe_static_scratch_bytes.argtypes = []
        L.tmoe_forward_static.restype = ctypes.c_int
        L.tmoe_forward_static.argtypes = [vp, vp, i64, vp, vp, vp, vp, vp, vp]
        L.tmoe_forward_glu.restype = ctypes.c_int
        L.tmoe_forward_glu.argtypes = [vp, vp, i64, vp, vp, vp, vp, vp, sz, vp]
        L.tmoe_rmsnorm_rows.restype = ctypes.c_int
        L.tmoe_rmsnorm_rows.argtypes = [vp, i64, i64, vp, ctypes.c_float, ctypes.c_int, vp, vp]
        L.tmoe_latent_workspace_bytes.restype = sz
        L.tmoe_latent_workspace_bytes.argtypes = [i64, i64, i64, i64, ctypes.c_int, ctypes.c_int]
        L.tmoe_latent_forward.restype = ctypes.c_int
        L.tmoe_latent_forward.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_int,
                                          vp, vp, sz, vp]
        L.tmoe_latent_backward.restype = ctypes.c_int
        L.tmoe_latent_backward.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64,
                                           ctypes.c_int, vp, vp, vp, vp, sz, vp]
        L.tmoe_signal_status.restype = ctypes.c_int
        L.tmoe_signal_status.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_uint32)]
        L.tmoe_forward_path.restype = ctypes.c_int
        L.tmoe_forward_path.argtypes = [vp, i64]
        L.tmoe_set_wait_polls.restype = ctypes.c_int64
        L.tmoe_set_wait_polls.argtypes = [i64]
        L.tmoe_prof_enable.restype = ctypes.c_int
        L.tmoe_prof_enable.argtypes = [ctypes.c_int]
        L.tmoe_prof_read.restype = ctypes.c_int
        L.tmoe_prof_read.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.c_int,
                                     ctypes.POINTER(ctypes.c_int64)]
        v = L.tmoe_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI version {v}, expected {ABI_VERSION}")
        _lib = L
    return _lib


def check(rc: int) -> int:
    """Raises TmoeError for a negative return code."""
    if rc < 0:
        raise TmoeError(rc, lib().tmoe_last_error().decode(errors="replace"))
    return rc


def dtype_code(dtype: torch.dtype) -> int:
    """TMOE_BF16 / TMOE_F32 for an activation dtype; raises for any other."""
    if dtype == torch.bfloat16:
        return TMOE_BF16
    if dtype == torch.float32:
        return TMOE_F32
    raise TmoeError(TMOE_EUNSUPPORTED, f"dtype {dtype}: supported are bfloat16 and float32")


class Plan:
    """Owns a tmoe_plan*. Immutable; safe to share across streams."""

    def __init__(self, d_in, d_out, E, k, r1, r2, r3, dtype: torch.dtype, eps: float,
                 fp8_weights: bool = False, router=(TMOE_ROUTER_SOFTMAX_TOPK, 10.0, 0.5),
                 flags: int = 0):
        if fp8_weights:
            if dtype != torch.bfloat16:
                raise TmoeError(TMOE_EUNSUPPORTED,
                                f"fp8 weights need bfloat16 activations, not {dtype}")
            code = TMOE_BF16_FP8W
        elif dtype == torch.bfloat16:
            code = TMOE_BF16
        elif dtype == torch.float32:
            code = TMOE_F32
        else:
            raise TmoeError(TMOE_EUNSUPPORTED,
                            f"parameter dtype {dtype}: supported are bfloat16 and float32")
        self.shape = TmoeShape(d_in, d_out, E, k, r1, r2, r3, code, eps, int(router[0]),
                               float(router[1]), float(router[2]), int(flags))
        self.flags = int(flags)
        self.router = tuple(router)
        self.dtype = dtype
        self.fp8_weights = fp8_weights
        self._ptr = ctypes.c_void_p()
        L = lib()
        check(L.tmoe_plan_create(ctypes.byref(self.shape), ctypes.byref(self._ptr)))
        self._destroy = L.tmoe_plan_destroy

    @property
    def ptr(self):
        return self._ptr

    def packed_bytes(self) -> int:
        return int(lib().tmoe_packed_bytes(self._ptr))

    def workspace_bytes(self, T: int) -> int:
        return int(lib().tmoe_workspace_bytes(self._ptr, T))

    def core_rank(self) -> int:
        """Rank of the core contraction the kernels run (r1, or E in the expert form)."""
        return int(lib().tmoe_plan_core_rank(self._ptr))

    def folded(self) -> bool:
        """True if the forward runs one GEMM of c (x) z against W = core U_out."""
        return bool(lib().tmoe_plan_folded(self._ptr))

    def forward_path(self, T: int) -> int:
        """TMOE_PATH_* of an eager forward of T tokens on the current device."""
        return check(lib().tmoe_forward_path(self._ptr, int(T)))

    def signal_status(self, clear: bool = True) -> int:
        """The TMOE_STATUS_* bits that completed kernels of this plan's forwards set
        (tmoe_signal_status; reads host memory, no synchronisation). Raises TmoeError
        (code TMOE_ESIGNAL) when any is set; clears them first when `clear`."""
        mask = ctypes.c_uint32()
        check(lib().tmoe_signal_status(self._ptr, 1 if clear else 0, ctypes.byref(mask)))
        return int(mask.value)

    def __del__(self):
        ptr, self._ptr = getattr(self, "_ptr", None), None
        if ptr and getattr(self, "_destroy", None):
            self._destroy(ptr)


def set_wait_polls(polls: int) -> int:
    """Budget of the kernels' in-launch waits, in polls (process-wide); returns the
    previous one. 0 makes every wait give up at once (the lost-signal test hook)."""
    return int(lib().tmoe_set_wait_polls(int(polls)))


def prof_enable(on: bool) -> None:
    check(lib().tmoe_prof_enable(1 if on else 0))


def prof_read():
    """Returns (ms summed per stage, number of forwards) since the last read."""
    ms = (ctypes.c_double * N_STAGES)()
    calls = ctypes.c_int64()
    check(lib().tmoe_prof_read(ms, N_STAGES, ctypes.byref(calls)))
    return list(ms), int(calls.value)
