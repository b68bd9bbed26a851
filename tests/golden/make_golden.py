"""Writes the golden fixtures of tests/golden/: seeded workload inputs (their
SHA-256, not the data: the generator in mamba-tuckermoe_amd/synth.py rebuilds
them bit for bit) and the float64 oracle's outputs on them.

    python tests/golden/make_golden.py [CASE ...]     (default: every case)

Cases: C1 (all 64 tokens, fp32, random gain/bias), C2 (all 32 tokens, bf16),
the first 32 tokens of C3 and C4 (bf16), and the first 64 tokens of C5 (e4m3
U_in / core / U_out with per-output-channel scales: the digests cover the codes
and scales; the oracle runs on their float64 dequantisation by oracle/e4m3.py).
The oracle is oracle/tucker_moe_np.forward_f64, itself pinned by
tests/test_oracle.py.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402
from oracle import e4m3  # noqa: E402
from oracle import tucker_moe_np as onp  # noqa: E402

CASES = [("C1", 64, "random"), ("C2", 32, "unit"), ("C3", 32, "unit"), ("C4", 32, "unit")]
FP8_CASES = [("C5", 64, "unit")]
FP8_KEYS = ("U_in", "core", "U_out")


def case_inputs(pkg, name, T, affine):
    w = pkg.WORKLOADS[name]
    return w, pkg.synth.make_params(w, affine=affine), pkg.synth.make_x(w, T)


def fp8_case_inputs(pkg, name, T, affine):
    """(workload, bf16 params, e4m3 codes, float64 reference params, x): the
    reference holds the bf16 values and the oracle's dequantised weights."""
    w = pkg.WORKLOADS[name]
    params, codes, _ = pkg.synth.make_fp8_params(w, affine=affine)
    ref = {k: v.double().numpy() for k, v in params.items()}
    for k in FP8_KEYS:
        q = codes[f"{k}_q"].view(torch.uint8).numpy()
        ref[k] = e4m3.dequantize(q, codes[f"{k}_scale"].double().numpy(), k)
    return w, params, codes, ref, pkg.synth.make_x(w, T)


def write(name, w, T, affine, x, ref, digests, pkg):
    out = onp.forward_f64(x, ref, w.k)
    np.savez_compressed(
        os.path.join(HERE, f"golden_{name}.npz"),
        T=T, affine=affine, sha_x=pkg.synth.sha256(x),
        out=out["out"].astype(np.float32), idx=out["idx"].astype(np.int32),
        w=out["w"].astype(np.float32), logits=out["logits"].astype(np.float32),
        topk_gap=onp.topk_gap(out["logits"], w.k).astype(np.float64),
        **digests)
    print(f"golden_{name}.npz: T={T} affine={affine} min_gap={onp.topk_gap(out['logits'], w.k).min():.3e}")


def main(names):
    pkg = __graft_entry__.load_package()
    for name, T, affine in FP8_CASES:
        if names and name not in names:
            continue
        w, params, codes, ref, x = fp8_case_inputs(pkg, name, T, affine)
        digests = {f"sha_{k.replace('.', '_')}": pkg.synth.sha256(v) for k, v in params.items()
                   if k not in FP8_KEYS}
        digests.update({f"sha_{k}": pkg.synth.sha256(v) for k, v in codes.items()})
        write(name, w, T, affine, x, ref, digests, pkg)
    for name, T, affine in CASES:
        if names and name not in names:
            continue
        w, params, x = case_inputs(pkg, name, T, affine)
        digests = {f"sha_{k.replace('.', '_')}": pkg.synth.sha256(v) for k, v in params.items()}
        write(name, w, T, affine, x, params, digests, pkg)


if __name__ == "__main__":
    main(sys.argv[1:])
