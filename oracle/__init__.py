"""CPU oracle of the Tucker-MoE layer forward — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or, for the CPU baseline, as the timed
host-CPU restatement). The product path (mamba-tuckermoe_amd/) never imports it
and has no CPU fallback.

Modules:
  tucker_moe_torch  op-for-op PyTorch CPU restatement of
                    pure_torch_mlx/model.py:19-27 and :68-102 (the reference's
                    forward, run the way the reference runs it)
  tucker_moe_np     independent float64 numpy formulation (regrouped algebra,
                    argsort top-k) and pure-Python brute force for tiny shapes
  e4m3              OCP FP8 E4M3 decoding and per-output-channel dequantisation
                    of the fp8 weight format (the fp8 configuration is the
                    reference layer on the dequantised weights)

Pinning (tests/test_oracle.py): the two formulations agree with each other and
with the brute force; the special cases fixed by the mathematics hold (E = k = 1
dense chain; one-hot U_expert gives per-expert cores; k = 1 scale invariance;
U_out = 0 gives bias; linearity in core / U_out / bias; softmax weights sum to
one; token-permutation equivariance; RMSNorm of a constant row; top-k against a
stable argsort); and planted mistakes in these oracle functions fail at least
one check. e4m3 decoding is pinned against torch.float8_e4m3fn on all 256 codes
and the format's fixed points (zero, smallest subnormal, smallest normal, 448,
NaN codes). The reference ships no golden vectors for this path
(pure_torch_mlx has no tests), so no function here is pinned by reference data.
"""
