"""mamba_tuckermoe_amd — the Tucker-MoE layer forward of s990093/Mamba-TuckerMoE
(pure_torch_mlx/model.py:41-102) on AMD Instinct MI355X (gfx950).

Public surface:
  TuckerMoE(d_in, d_out, cfg)  drop-in nn.Module (module.py)
  TuckerMoEConfig              the cfg fields the module reads (config.py)
  WORKLOADS                    the named seeded workloads C1..C5 (config.py)
  FFN_WORKLOADS                seeded FFN sub-block configurations F0..F2 (config.py)
  load_tucker                  checkpoint-key loader that refreshes packed weights
  TuckerFFN, TuckerOutProj     the reference blocks' Tucker-MoE sub-blocks (block.py):
                               TransformerBlock's FFN, Mamba3Block's out_proj
  RMSNorm, LayerScale          their norm and scale modules
  FusedLatentMoE               the training module's latent expert contraction with its
                               backward (latent.py; autograd.Function, reference signature)
  TuckerMoETrain               the reference's training layer (TritonTuckerMoE) on it
  synth                        seeded synthetic parameters and tokens
  fp8                          e4m3 weights with per-output-channel scales
  checkpoint                   the reference's .npz keys (layers, FFN, out_proj) and the
                               versioned packed file (save_packed / load_packed)
  _lib                         ctypes binding of the C ABI (include/tmoe.h)
"""
from . import _lib, checkpoint, config, fp8, synth
from .config import FFN_WORKLOADS, WORKLOADS, FfnWorkload, TuckerMoEConfig, Workload
from .module import RMSNorm, TuckerMoE, load_tucker
from .block import LayerScale, TuckerFFN, TuckerOutProj
from .latent import FusedLatentMoE, TuckerMoETrain, fused_latent_moe

__all__ = ["TuckerMoE", "RMSNorm", "LayerScale", "TuckerFFN", "TuckerOutProj",
           "FusedLatentMoE", "TuckerMoETrain", "fused_latent_moe",
           "TuckerMoEConfig", "Workload", "WORKLOADS", "FfnWorkload", "FFN_WORKLOADS", "load_tucker", "synth", "config", "fp8",
           "checkpoint", "_lib"]
