"""Layer hyper-parameters and the named workloads C1..C5.

`TuckerMoEConfig` carries the fields TuckerMoE.__init__ reads from the
reference's Mamba3Config (pure_torch_mlx/config.py:18,20-24; defaults copied from
there). Any object with those attributes (the reference's own Mamba3Config
included) is accepted by mamba_tuckermoe_amd.TuckerMoE.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch


@dataclass
class TuckerMoEConfig:
    rms_norm_eps: float = 1e-5        # config.py:18
    kmoe_num_experts: int = 8         # config.py:20
    kmoe_top_k: int = 2               # config.py:21
    kmoe_r1: int = 32                 # config.py:22
    kmoe_r2: int = 512                # config.py:23
    kmoe_r3: int = 256                # config.py:24
    ffn_expand: int = 6               # config.py:17 (TuckerFFN: d_ff = ffn_expand * d)


@dataclass(frozen=True)
class Workload:
    """One seeded synthetic configuration of the layer."""
    name: str
    T: int
    d_in: int
    d_out: int
    E: int
    k: int
    r1: int
    r3: int
    r2: int
    dtype: torch.dtype
    seed: int
    router_std: Optional[float] = None   # None: N(0, 1/d_in)
    fp8: bool = False                    # U_in, core, U_out as e4m3 + per-channel scales
    note: str = ""

    def cfg(self, eps: float = 1e-5) -> TuckerMoEConfig:
        return TuckerMoEConfig(rms_norm_eps=eps, kmoe_num_experts=self.E, kmoe_top_k=self.k,
                               kmoe_r1=self.r1, kmoe_r2=self.r2, kmoe_r3=self.r3)

    def with_T(self, T: int) -> "Workload":
        d = dict(self.__dict__)
        d["T"] = T
        return Workload(**d)

    def flops(self, T: Optional[int] = None) -> dict:
        """Algorithmic MFMA work per forward: 2*T*(E*d_in + d_in*r3 + r1*r3*r2 + r2*d_out)."""
        T = self.T if T is None else T
        st = {
            "router": 2 * T * self.E * self.d_in,
            "in_proj": 2 * T * self.d_in * self.r3,
            "core": 2 * T * self.r1 * self.r3 * self.r2,
            "out_proj": 2 * T * self.r2 * self.d_out,
        }
        st["total"] = sum(st.values())
        return st

    def flops_executed(self, T: Optional[int] = None, rk: Optional[int] = None,
                       folded: bool = False) -> dict:
        """MFMA work the kernels run per forward, per stage: with the plan's core rank
        rk (r1, or E in the expert form); a folded plan's core stage only forms the
        Khatri-Rao rows c (x) z (no MFMA) and its out-projection contracts rk*r3."""
        T = self.T if T is None else T
        rk = self.r1 if rk is None else rk
        st = {
            "router": 2 * T * self.E * self.d_in,
            "in_proj": 2 * T * self.d_in * self.r3,
            "core": 0 if folded else 2 * T * rk * self.r3 * self.r2,
            "out_proj": 2 * T * (rk * self.r3 if folded else self.r2) * self.d_out,
        }
        st["total"] = sum(st.values())
        return st

    def stage_bytes(self, T: Optional[int] = None) -> dict:
        """Compulsory bytes per kernel stage: its inputs read once, its outputs
        written once (weights in the packed form the kernels read: the compute
        dtype, plus fp32 gain / U_expert / bias / scales)."""
        T = self.T if T is None else T
        es = 4 if self.dtype == torch.float32 else 2
        E_pad = max(32, 1 << (self.E - 1).bit_length())
        small = 4 * (self.r3 + self.E * self.r1)
        st = {
            "front": T * self.d_in * es + (self.r3 + E_pad) * self.d_in * es + small
                     + T * self.r3 * es + T * self.r1 * 4 + T * self.k * 8,
            "core": T * self.r3 * es + T * self.r1 * 4 + self.r1 * self.r3 * self.r2 * es
                    + T * self.r2 * es,
            "out_proj": T * self.r2 * es + self.d_out * self.r2 * es + 4 * self.d_out
                        + T * self.d_out * es,
        }
        if self.fp8:
            st["front"] += 4 * self.r3
            st["core"] += 8 * self.r1 * self.r2
            st["out_proj"] += 4 * self.d_out
        return st

    def stage_bytes_folded(self, T: Optional[int] = None, rk: Optional[int] = None) -> dict:
        """stage_bytes of a folded plan: the core stage reads z and c and writes
        c (x) z (T, rk*r3); the out-projection reads it and W^T (d_out, rk*r3) bf16.
        Where the front writes c (x) z itself (no z, no core kernel) these bytes stay
        attributed to the core stage; the front's and out-projection's figures are
        those of the split kernels."""
        T = self.T if T is None else T
        rk = self.r1 if rk is None else rk
        st = self.stage_bytes(T)
        K = rk * self.r3
        st["core"] = T * self.r3 * 2 + T * rk * 4 + T * K * 2
        st["out_proj"] = T * K * 2 + self.d_out * K * 2 + 4 * self.d_out + T * self.d_out * 2
        return st

    def stage_bytes_kr(self, T: Optional[int] = None, rk: Optional[int] = None) -> dict:
        """stage_bytes of a folded forward whose out-projection forms c (x) z itself
        (TMOE_PATH_LARGE_KR): the front writes z and c (stage_bytes' front), there is
        no core stage, and the out-projection reads z, c and W^T (d_out, rk*r3)."""
        T = self.T if T is None else T
        rk = self.r1 if rk is None else rk
        st = self.stage_bytes(T)
        es = 4 if self.dtype == torch.float32 else 2
        K = rk * self.r3
        st["core"] = 0
        st["out_proj"] = (T * self.r3 * es + T * rk * 4 + self.d_out * K * 2 + 4 * self.d_out
                          + T * self.d_out * es)
        return st

    def one_launch(self, T: int, rk: int, folded: bool) -> bool:
        """Whether a forward of T tokens is the library's single decode launch
        (k_sk_decode; the selection rule of small_decode_ok in tmoe_kernels.hip,
        outside graph capture)."""
        return (folded and self.dtype == torch.bfloat16 and 0 < T <= 64 and self.E <= 16
                and self.r3 in (64, 128, 256) and rk <= 32)

    def layer_bytes_folded(self, T: Optional[int] = None, rk: Optional[int] = None) -> int:
        """Compulsory bytes of a folded forward in one launch: x, the front weights,
        W^T, the small fp32 vectors, the routing outputs and out (no intermediate
        crosses HBM)."""
        T = self.T if T is None else T
        rk = self.r1 if rk is None else rk
        st = self.stage_bytes_folded(T, rk)
        es = 4 if self.dtype == torch.float32 else 2
        K = rk * self.r3
        return (st["front"] - T * self.r3 * es - T * self.r1 * 4
                + st["out_proj"] - T * K * 2 + T * rk * 4)

    def hbm_bytes(self, T: Optional[int] = None) -> int:
        """Compulsory HBM bytes per forward: x in, out, every weight once (fp8
        workloads: the three projections at one byte plus their fp32 scales)."""
        T = self.T if T is None else T
        es = 4 if self.dtype == torch.float32 else 2
        small = self.E * self.d_in + self.r3 + self.E * self.r1 + self.d_out
        proj = self.d_in * self.r3 + self.r1 * self.r3 * self.r2 + self.r2 * self.d_out
        if self.fp8:
            wbytes = small * es + proj + 4 * (self.r3 + self.r1 * self.r2 + self.d_out)
        else:
            wbytes = (small + proj) * es
        return T * self.d_in * es + T * self.d_out * es + wbytes


WORKLOADS = {
    "C1": Workload("C1", 64, 512, 1024, 8, 2, 4, 128, 256, torch.float32, 1001,
                   note="fp32 everywhere; the reference's CPU-path configuration"),
    "C2": Workload("C2", 32, 1536, 2304, 16, 2, 4, 256, 1024, torch.bfloat16, 1002,
                   note="decode-shaped: batch 32 x 1 step"),
    "C3": Workload("C3", 16384, 1536, 2304, 16, 2, 4, 256, 1024, torch.bfloat16, 1003,
                   note="prefill-shaped: batch 8 x seq 2048"),
    "C4": Workload("C4", 4096, 1536, 2304, 256, 8, 4, 256, 1024, torch.bfloat16, 1004,
                   router_std=0.02, note="expert-count scaling"),
    "C5": Workload("C5", 16384, 1536, 2304, 16, 2, 4, 256, 1024, torch.bfloat16, 1005,
                   fp8=True, note="fp8 e4m3 U_in/core/U_out with per-output-channel scales"),
}


@dataclass(frozen=True)
class FfnWorkload:
    """One seeded synthetic configuration of TransformerBlock's FFN sub-block
    (model.py:292-296): ffn_gate / ffn_up TuckerMoE(d, d_ff), ffn_down
    TuckerMoE(d_ff, d), d_ff = ffn_expand * d."""
    name: str
    T: int
    d: int
    ffn_expand: int
    E: int
    k: int
    r1: int
    r3: int
    r2: int
    dtype: torch.dtype
    seed: int
    note: str = ""

    @property
    def d_ff(self) -> int:
        return self.ffn_expand * self.d

    def cfg(self, eps: float = 1e-5) -> TuckerMoEConfig:
        return TuckerMoEConfig(rms_norm_eps=eps, kmoe_num_experts=self.E, kmoe_top_k=self.k,
                               kmoe_r1=self.r1, kmoe_r2=self.r2, kmoe_r3=self.r3,
                               ffn_expand=self.ffn_expand)

    def layer(self, name: str) -> Workload:
        """The Workload of sub-layer ffn_gate / ffn_up / ffn_down (its own seed)."""
        i = ("ffn_gate", "ffn_up", "ffn_down").index(name)
        d_in, d_out = (self.d, self.d_ff) if i < 2 else (self.d_ff, self.d)
        return Workload(f"{self.name}.{name}", self.T, d_in, d_out, self.E, self.k, self.r1,
                        self.r3, self.r2, self.dtype, self.seed * 8 + 1 + i)


FFN_WORKLOADS = {
    # the reference checkpoint's block (config.py: d_model 768, ffn_expand 6, E 8,
    # k 2, r = (32, 512, 256)); r1 = 32 takes the row-blocked core
    "F1": FfnWorkload("F1", 4096, 768, 6, 8, 2, 32, 256, 512, torch.bfloat16, 2001,
                      note="TransformerBlock FFN at the reference model's dimensions"),
    # the same shape with r1 = 4, on the persistent core
    "F2": FfnWorkload("F2", 4096, 768, 6, 8, 2, 4, 256, 512, torch.bfloat16, 2002,
                      note="FFN with rank r1 = 4"),
    "F0": FfnWorkload("F0", 64, 256, 2, 8, 2, 4, 128, 256, torch.float32, 2000,
                      note="small fp32 FFN for CPU oracle checks"),
}
