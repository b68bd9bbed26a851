"""Writes the golden fixtures of tests/golden/: seeded workload inputs (their
SHA-256, not the data: the generator in mamba-tuckermoe_amd/synth.py rebuilds
them bit for bit) and the float64 oracle's outputs on them.

    python tests/golden/make_golden.py

Cases: C1 (all 64 tokens, fp32, random gain/bias), C2 (all 32 tokens, bf16),
and the first 32 tokens of C3 and C4 (bf16). The oracle is
oracle/tucker_moe_np.forward_f64, itself pinned by tests/test_oracle.py.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402
from oracle import tucker_moe_np as onp  # noqa: E402

CASES = [("C1", 64, "random"), ("C2", 32, "unit"), ("C3", 32, "unit"), ("C4", 32, "unit")]


def case_inputs(pkg, name, T, affine):
    w = pkg.WORKLOADS[name]
    return w, pkg.synth.make_params(w, affine=affine), pkg.synth.make_x(w, T)


def main():
    pkg = __graft_entry__.load_package()
    for name, T, affine in CASES:
        w, params, x = case_inputs(pkg, name, T, affine)
        ref = onp.forward_f64(x, params, w.k)
        digests = {f"sha_{k.replace('.', '_')}": pkg.synth.sha256(v) for k, v in params.items()}
        np.savez_compressed(
            os.path.join(HERE, f"golden_{name}.npz"),
            T=T, affine=affine, sha_x=pkg.synth.sha256(x),
            out=ref["out"].astype(np.float32), idx=ref["idx"].astype(np.int32),
            w=ref["w"].astype(np.float32), logits=ref["logits"].astype(np.float32),
            topk_gap=onp.topk_gap(ref["logits"], w.k).astype(np.float64),
            **digests)
        print(f"golden_{name}.npz: T={T} affine={affine} min_gap={onp.topk_gap(ref['logits'], w.k).min():.3e}")


if __name__ == "__main__":
    main()
