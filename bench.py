#!/usr/bin/env python3
"""Tucker-MoE layer forward throughput on one MI355X.

One step = one tmoe_forward (the whole layer: router/top-k, in-projection +
RMSNorm, core contraction, out-projection) over one batch of T synthetic tokens
already resident in HBM. The default workload is C3 (T=16384, d_in=1536,
d_out=2304, E=16, top-2, r=(4,256,1024), bf16), the configuration BASELINE's
metric is quoted on.

Buffer sets (tokens, outputs, workspace and a copy of the packed weights) are
rotated so that the working set exceeds the 256 MB Infinity Cache and each step
reads its operands from HBM.

Prints ONE JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "TuckerMoE layer tokens/sec + % bf16 MFMA peak at T=16384; vs host-CPU ref"
PEAK_TFLOPS = {"bf16": 2516.6, "f32": 157.3}   # MI355X dense MFMA
HBM_PEAK_GBS = 8000.0                            # MI355X HBM3E
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), with its family / model / stepping and
    the number of online CPUs, which tell EPYC generations apart where the name is
    generic."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = line.split(":", 1)
                info.setdefault(k.strip(), v.strip())
    except OSError:
        pass
    name = info.get("model name") or platform.processor() or "unknown"
    extra = [f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info]
    return f"{name} ({', '.join(extra + [f'{os.cpu_count()} online CPUs'])})"


def profile_figure(workload: str, key: str, stage: str):
    """A per-launch figure of `stage` from the committed rocprofv3 counter summaries
    (profiles/tmoe_forward_<workload>_counters.md, then ..._traffic.md; a line
    '<key> <stage> <value>'), or None when it has not been measured.
    key 'traffic_bytes': FETCH_SIZE + WRITE_SIZE bytes, calibrated against a copy;
    key 'mfma_util': SQ_VALU_MFMA_BUSY_CYCLES over the GPU-active cycles x SIMDs."""
    for name in (f"tmoe_forward_{workload}_counters.md", f"tmoe_forward_{workload}_traffic.md"):
        path = os.path.join(ROOT, "profiles", name)
        if not os.path.exists(path):
            continue
        for line in open(path):
            f = line.strip().strip("`").split()
            if len(f) == 3 and f[0] == key and f[1] == stage:
                return float(f[2])
    return None


def traffic_per_launch(workload: str, kernel: str):
    """HBM bytes per launch of stage `kernel` (see profile_figure)."""
    return profile_figure(workload, "traffic_bytes", kernel)


def cpu_threads():
    """Host threads for the CPU baseline: the process's CPU affinity
    (os.sched_getaffinity), capped by OMP_NUM_THREADS when the host sets it (the
    GPU box sets its CPU share there). Returns (threads, affinity count)."""
    n_aff = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS")
    n = min(n_aff, int(cap)) if cap and cap.isdigit() and int(cap) > 0 else n_aff
    return n, n_aff


def cpu_baseline(fwd, x0, T, chunk, seconds, wl_name, dt_name, what, oracle_mode):
    """Times fwd(x, chunk=...) on the host: one warm-up pass, then the median of 3
    passes over a sample of whole chunks sized so the 4 passes take about
    `seconds` (at most all T tokens). With oracle_mode, the same op sequence in
    float32 on the bf16-valued inputs (the parity reference) is timed too."""
    import torch
    threads, n_aff = cpu_threads()
    torch.set_num_threads(threads)
    chunk = min(chunk, T)
    t_a = time.perf_counter()
    fwd(x0[:chunk], chunk=chunk)                       # sizes the sample
    rate = chunk / (time.perf_counter() - t_a)
    n_cpu = int(min(T, max(chunk, seconds * rate / 4)) // chunk * chunk)

    def median3(**kw):
        fwd(x0[:n_cpu], chunk=chunk, **kw)             # warm-up pass
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            fwd(x0[:n_cpu], chunk=chunk, **kw)
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    cpu_s = median3()
    out = {
        "value": n_cpu / cpu_s, "unit": "tokens/s", "cores": threads, "kind": "port",
        "sample": (f"first {n_cpu} of the {T} {wl_name} tokens, {dt_name} tensors, {what}, "
                   f"chunks of {chunk}, 1 warm-up + median of 3 passes, torch "
                   f"{torch.__version__} with {threads} threads (affinity {n_aff} CPUs) on "
                   f"{cpu_model()}"),
        "seconds": cpu_s, "tokens": n_cpu, "cpu_model": cpu_model(), "affinity_cpus": n_aff,
    }
    if oracle_mode:
        s32 = median3(compute_dtype=torch.float32)
        out["oracle_mode_f32"] = {"value": n_cpu / s32, "unit": "tokens/s", "seconds": s32,
                                  "sample": "the same passes in float32 on the bf16-valued inputs"}
    return out


FFN_METRIC = "TransformerBlock FFN sub-block tokens/sec (norm, gate, up, silu*up, down, residual)"


def bench_ffn(args) -> None:
    """--ffn NAME: one step = TuckerFFN.forward over T tokens of the FFN workload
    NAME (model.py:337-341: RMSNorm, three TuckerMoE layers, silu(gate) * up and
    the LayerScale residual fused into the layers' out-projection stores). The
    same launches with the two elementwise ops done by separate torch kernels
    (the reference's op sequence on the GPU) are timed beside it."""
    import torch
    import torch.nn.functional as F

    import __graft_entry__
    pkg = __graft_entry__.load_package()
    f = pkg.FFN_WORKLOADS[args.ffn]
    T = args.tokens or f.T
    dev = torch.device("cuda:0")
    dt_name = "bf16" if f.dtype == torch.bfloat16 else "f32"
    es = 2 if f.dtype == torch.bfloat16 else 4
    params = pkg.synth.make_ffn_params(f)
    x0 = pkg.synth.make_ffn_x(f, T)
    m0 = pkg.TuckerFFN(f.d, f.cfg()).to(dev, f.dtype)
    m0.load_state_dict({k: v.to(dev) for k, v in params.items()})
    packed = sum(getattr(m0, n).packed().numel() for n in ("ffn_gate", "ffn_up", "ffn_down"))
    set_bytes = packed + T * f.d * es * 2 + T * f.d_ff * es * 2
    n_sets = max(3, math.ceil(args.rotate_mb * 1e6 / set_bytes))
    log(f"[bench-ffn] {f.name}: T={T} d={f.d} d_ff={f.d_ff} E={f.E} k={f.k} "
        f"r=({f.r1},{f.r3},{f.r2}) {dt_name}; {n_sets} rotated sets x {set_bytes / 1e6:.1f} MB")
    gen = torch.Generator(device=dev).manual_seed(f.seed)
    sets = []
    for i in range(n_sets):
        if i == 0:
            m = m0
        else:
            m = pkg.TuckerFFN(f.d, f.cfg()).to(dev, f.dtype)
            m.load_state_dict(m0.state_dict())
        for n in ("ffn_gate", "ffn_up", "ffn_down"):
            getattr(m, n).packed()
        x = x0.to(dev) if i == 0 else torch.randn(T, f.d, device=dev, generator=gen).to(f.dtype)
        sets.append((m, x))

    def fused(i):
        m, x = sets[i % n_sets]
        return m(x)

    def unfused(i):
        m, x = sets[i % n_sets]
        x_f = m.norm_ffn(x)
        h = F.silu(m.ffn_gate(x_f)) * m.ffn_up(x_f)
        return x + m.ls_ffn.gamma * m.ffn_down(h)

    def timed(fn):
        with torch.no_grad():
            for i in range(args.warmup):
                fn(i)
            torch.cuda.synchronize()
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record()
            for i in range(args.steps):
                fn(i)
            ev1.record()
            torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) / args.steps

    ms = timed(fused)
    ms_unfused = timed(unfused)
    tok_s = T / (ms * 1e-3)
    flops = sum(f.layer(n).flops(T)["total"] for n in ("ffn_gate", "ffn_up", "ffn_down"))
    # what the kernels execute: the core at the plan's kernel rank (E < r1: the
    # expert form, E of the r1 ranks' multiply-adds)
    m0 = sets[0][0]
    executed = 0
    for n in ("ffn_gate", "ffn_up", "ffn_down"):
        pl = getattr(m0, n).plan()
        executed += f.layer(n).flops_executed(T, pl.core_rank(), pl.folded())["total"]
    peak = PEAK_TFLOPS[dt_name]
    tflops = flops / (ms * 1e-3) / 1e12
    tflops_exec = executed / (ms * 1e-3) / 1e12
    log(f"[bench-ffn] fused {ms * 1e3:.1f} us/step ({tok_s / 1e6:.2f} M tok/s, {tflops:.0f} "
        f"TFLOP/s of the reference form, {tflops_exec:.0f} executed); separate elementwise "
        f"kernels {ms_unfused * 1e3:.1f} us/step")

    from oracle import tucker_ffn_torch as ft
    from oracle import tucker_moe_np as onp
    n_par = min(T, 256)
    m, x = sets[0]
    with torch.no_grad():
        st = m.stages(x[:n_par])
        got_idx = {"ffn_gate": m.ffn_gate.forward_with_routing(st["x_f"])[1],
                   "ffn_up": m.ffn_up.forward_with_routing(st["x_f"])[1],
                   "ffn_down": m.ffn_down.forward_with_routing(st["h"])[1]}
    torch.cuda.synchronize()
    ref = ft.ffn_forward(x0[:n_par], params, f.k, compute_dtype=torch.float32, intermediates=True)
    # rows that route alike in all three layers; the others sit on a near-tie that
    # the bf16 rounding of a layer input moves (the GPU tests bound them)
    same = torch.ones(n_par, dtype=torch.bool)
    for name, gi in got_idx.items():
        same &= (gi.cpu().sort(1).values == ref["idx"][name].sort(1).values).all(1)
    y = st["out"].float().cpu()
    parity = {"tokens": n_par, "rows_routed_alike": int(same.sum()),
              "rel_l2_out": onp.rel_l2(y[same].numpy(), ref["out"][same].double().numpy()),
              "reference": "oracle/tucker_ffn_torch fp32 on the bf16-valued inputs, over the "
                           "rows routed alike in all three layers"}
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(lambda xs, **kw: ft.ffn_forward(xs, params, f.k, **kw), x0, T, 256,
                           args.cpu_seconds, f.name, dt_name,
                           "reference op sequence (oracle/tucker_ffn_torch)", oracle_mode=False)
    print(json.dumps({
        "metric": FFN_METRIC, "value": tok_s, "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": dt_name,
        "data": "synthetic (seeded N(0,1) tokens, N(0,1/fan_in) weights; no checkpoint)",
        "config": {"workload": f"{f.name}: TransformerBlock FFN sub-block, one GPU", "T": T,
                   "d": f.d, "d_ff": f.d_ff, "E": f.E, "top_k": f.k, "r1": f.r1, "r3": f.r3,
                   "r2": f.r2, "rotated_sets": n_sets},
        "mfma": {"tflops": tflops, "peak": peak, "frac": tflops / peak, "flops_per_step": flops,
                 "executed_tflops": tflops_exec, "executed_frac": tflops_exec / peak,
                 "executed_flops_per_step": executed},
        "separate_elementwise_ms_per_step": ms_unfused,
        "parity": parity, "cpu_baseline": cpu,
    }), flush=True)


LATENT_METRIC = "FusedLatentMoE forward + backward tokens/sec (training path)"


def bench_latent(args) -> None:
    """--latent: one step = FusedLatentMoE forward and backward (the training
    module's latent contraction, sft_cot_bundle/scripts/model.py:225-289) over T
    tokens at the training config's ranks (E 8, k 2, r3 256, r2 1024), bf16."""
    import torch

    import __graft_entry__
    pkg = __graft_entry__.load_package()
    T = args.tokens or 16384
    E, k, r3, r2 = 8, 2, 256, 1024
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(T, r3, device=dev, generator=g).bfloat16().requires_grad_(True)
    G = (torch.randn(E, r3, r2, device=dev, generator=g) * r3 ** -0.5).bfloat16().requires_grad_(True)
    v, idx = torch.topk(torch.randn(T, E, device=dev, generator=g), k, dim=-1)
    p = torch.softmax(v, -1).bfloat16().requires_grad_(True)
    dout = torch.randn(T, r2, device=dev, generator=g).bfloat16()

    def step():
        out = pkg.FusedLatentMoE.apply(x, G, idx, p)
        out.backward(dout)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / args.steps
    algo = 8.0 * T * k * r3 * r2          # out, dx, dp, dG: 2 T k r3 r2 each
    executed = 2.0 * T * r3 * r2 * E * 3  # dense over E: forward, H, dG
    peak = PEAK_TFLOPS["bf16"]
    log(f"[bench-latent] T={T}: {ms * 1e3:.1f} us per forward+backward; "
        f"{executed / (ms * 1e-3) / 1e12:.0f} TFLOP/s executed (dense over E)")
    print(json.dumps({
        "metric": LATENT_METRIC, "value": T / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "FusedLatentMoE forward+backward, one GPU", "T": T, "E": E,
                   "top_k": k, "r3": r3, "r2": r2},
        "mfma": {"executed_tflops": executed / (ms * 1e-3) / 1e12,
                 "algorithmic_tflops": algo / (ms * 1e-3) / 1e12, "peak": peak,
                 "executed_frac": executed / (ms * 1e-3) / 1e12 / peak},
    }), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="C3")
    ap.add_argument("--tokens", type=int, default=None, help="override T")
    ap.add_argument("--rotate-mb", type=float, default=640.0,
                    help="minimum total size of the rotated buffer sets")
    ap.add_argument("--cpu-seconds", type=float, default=24.0,
                    help="approximate CPU work of the host baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the host-CPU baseline")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="after the timed work, copy a buffer of this many MiB 3 times (a plain "
                         "copy kernel of known size, to scale profiler byte counters)")
    ap.add_argument("--ffn", default=None,
                    help="time the FFN sub-block of this FFN workload (F0, F1, F2) instead")
    ap.add_argument("--no-fold", action="store_true",
                    help="keep the core and the out-projection as two GEMMs (TMOE_FLAG_NO_FOLD)")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the extra workloads (C2, C4, C3 at T=2048 and T=1) of the C3 run")
    ap.add_argument("--no-probes", action="store_true",
                    help="skip the hardware probes and the vendor-library GEMM (C3 runs only)")
    ap.add_argument("--no-fuse", action="store_true",
                    help="never run the large-T forward as one launch (TMOE_FLAG_NO_FUSE)")
    ap.add_argument("--latent", action="store_true",
                    help="time FusedLatentMoE forward + backward (training path) instead")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported in this "
              "build (the layer shards by tokens with no exchange; see the design notes).",
              file=sys.stderr)
        sys.exit(2)
    if args.ffn:
        bench_ffn(args)
        return
    if args.latent:
        bench_latent(args)
        return

    import torch

    import __graft_entry__
    pkg = __graft_entry__.load_package()
    w = pkg.WORKLOADS[args.workload]
    if args.tokens:
        w = w.with_T(args.tokens)
    r = measure(pkg, w, args, steps=args.steps, warmup=args.warmup, rotate_mb=args.rotate_mb,
                no_fold=args.no_fold, no_fuse=args.no_fuse, cpu=not args.no_cpu, label="bench")
    res = r["result"]
    # the other workloads' figures, measured in the same run (their own parity slices;
    # the headline above is unchanged by them)
    if not args.no_extra and args.workload == "C3" and not args.tokens:
        extra = {}
        for key, name, T in EXTRA_WORKLOADS:
            we = pkg.WORKLOADS[name].with_T(T) if T else pkg.WORKLOADS[name]
            e = measure(pkg, we, args, steps=args.steps, warmup=args.warmup,
                        rotate_mb=args.rotate_mb, no_fold=args.no_fold, no_fuse=args.no_fuse,
                        cpu=False, label=f"extra {key}")
            rr = e["result"]
            extra[key] = {
                "workload": rr["config"]["workload"], "T": rr["config"]["T"],
                "ms_per_step": rr["ms_per_step"], "avg_us": rr["ms_per_step"] * 1e3,
                "tokens_per_s": rr["value"], "path": rr["config"]["path"],
                "roofline": {k: rr["roofline"][k] for k in
                             ("bound", "kernel", "achieved", "peak", "unit", "frac", "avg_us")},
                "layer": {k: rr["layer"][k] for k in
                          ("executed_tflops", "executed_mfma_frac", "tflops", "mfma_frac",
                           "hbm_gbs_compulsory")},
                "parity": rr["parity"],
            }
        res["extra"] = extra
    if not args.no_probes and args.workload == "C3" and not args.tokens:
        res["probes"] = hw_probes(pkg, w, res)
    print(json.dumps(res), flush=True)


def hw_probes(pkg, w, res) -> dict:
    """What this MI355X sustains on the resources the layer's kernels are bound by
    (include/tmoe_probe.h, libtmoe_probe.so), and the vendor library (hipBLASLt via
    torch.matmul) on the layer's out-projection GEMM, measured in the same run. Not
    part of the timed region; the headline and its roofline are unchanged by it."""
    import ctypes

    import torch
    out = {}
    lib_path = os.path.join(os.path.dirname(pkg._lib.LIB_PATH), "libtmoe_probe.so")
    if os.path.exists(lib_path):
        L = ctypes.CDLL(lib_path)
        dp = ctypes.POINTER(ctypes.c_double)
        L.tmoe_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, dp, dp]
        L.tmoe_probe_l2_stream.argtypes = [ctypes.c_int, ctypes.c_int, dp]
        for name, rnd in (("constant", 0), ("random", 1)):
            tf, mhz = ctypes.c_double(), ctypes.c_double()
            if L.tmoe_probe_mfma(rnd, 20000, ctypes.byref(tf), ctypes.byref(mhz)) == 0:
                out[f"mfma_bf16_{name}_operands"] = {"tflops": tf.value, "frac_of_peak": tf.value / PEAK_TFLOPS["bf16"],
                                                     "shader_mhz": mhz.value}
        l2 = {}
        for dma in (0, 1):
            for waves in (4, 8):
                g = ctypes.c_double()
                if L.tmoe_probe_l2_stream(dma, waves, ctypes.byref(g)) == 0:
                    l2[f"{'lds_dma' if dma else 'registers'}_{waves}_waves"] = g.value
        out["l2_stream_gbs_per_cu"] = l2
    else:
        out["missing"] = lib_path
    # hipBLASLt on the out-projection's GEMM: (T x K) x (K x d_out), bf16 in, fp32 accumulate
    dev = torch.device("cuda:0")
    K = w.r1 * w.r3 if res["config"]["form"] == "folded" else w.r2

    def lib_gemm(M, N, Kd):
        a = torch.randn(M, Kd, device=dev).to(torch.bfloat16)
        b = torch.randn(Kd, N, device=dev).to(torch.bfloat16)
        for _ in range(3):
            a @ b
        torch.cuda.synchronize()
        best = None
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(10):
                a @ b
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / 10 * 1e3
            best = us if best is None else min(best, us)
        return {"shape_mnk": [M, N, Kd], "us": best, "tflops": 2.0 * M * N * Kd / best * 1e-6}

    out["hipblaslt_outproj_gemm"] = lib_gemm(res["config"]["T"], w.d_out, K)
    out["hipblaslt_square_8192"] = lib_gemm(8192, 8192, 8192)
    log(f"[probes] {json.dumps(out)}")
    return out


# the workloads measured beside the C3 headline: (key, workload, T or None)
EXTRA_WORKLOADS = (("C2", "C2", None), ("C4", "C4", None),
                   ("C3_T2048", "C3", 2048), ("C3_T1", "C3", 1))


def measure(pkg, w, args, *, steps, warmup, rotate_mb, no_fold, no_fuse, cpu, label):
    """One workload: warm-up, `steps` timed forwards over rotated buffer sets, the
    per-stage event pass, parity on a slice and (cpu) the host baseline. Returns
    {"result": the JSON fields of the bench line}."""
    import torch
    L = pkg._lib.lib()
    T = w.T
    dev = torch.device("cuda:0")
    dt_name = "bf16" if w.dtype == torch.bfloat16 else "f32"
    es = 2 if w.dtype == torch.bfloat16 else 4

    # -- model and rotated buffer sets -----------------------------------------
    from oracle import e4m3
    if w.fp8:
        # e4m3 U_in / core / U_out + per-output-channel scales; the reference layer
        # is run on the dequantised weights (the oracle's e4m3 decoding)
        params, codes, _ = pkg.synth.make_fp8_params(w)
        ref_params = {k: v.float() for k, v in params.items()}
        for k in ("U_in", "core", "U_out"):
            ref_params[k] = torch.from_numpy(e4m3.dequantize(
                codes[f"{k}_q"].view(torch.uint8).numpy(), codes[f"{k}_scale"].double().numpy(),
                k)).float()
    else:
        params = pkg.synth.make_params(w)
        codes, ref_params = None, params
    x0 = pkg.synth.make_x(w)
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg()).to(dev, w.dtype)
    m.load_state_dict({k: v.to(dev) for k, v in params.items()})
    m.set_fold(not no_fold)
    m.set_fuse(not no_fuse)
    if codes is not None:
        m.load_fp8(*[codes[k].to(dev) for k in ("U_in_q", "U_in_scale", "core_q", "core_scale",
                                                  "U_out_q", "U_out_scale")])
    plan = m.plan()
    packed0 = m.packed()
    folded = plan.folded()
    rk = plan.core_rank()
    path = plan.forward_path(T)
    form = ("folded: c (x) z against W = core U_out, one GEMM of width %d" % (rk * w.r3)
            if folded else "two GEMMs: core (rank %d) then U_out" % rk)
    log(f"[{label}] plan form: {form}; kernels: {pkg._lib.PATH_NAMES.get(path, path)}")
    ws_bytes = plan.workspace_bytes(T)
    set_bytes = T * w.d_in * es + T * w.d_out * es + ws_bytes + packed0.numel()
    n_sets = max(3, math.ceil(rotate_mb * 1e6 / set_bytes))
    log(f"[{label}] workload {w.name}: T={T} d_in={w.d_in} d_out={w.d_out} E={w.E} k={w.k} "
        f"r=({w.r1},{w.r3},{w.r2}) {dt_name}; {n_sets} rotated sets x {set_bytes / 1e6:.1f} MB")
    gen = torch.Generator(device=dev).manual_seed(w.seed)
    sets = []
    for i in range(n_sets):
        x = x0.to(dev) if i == 0 else torch.randn(T, w.d_in, device=dev, generator=gen).to(w.dtype)
        pk = packed0 if i == 0 else packed0.clone()
        sets.append(dict(
            x=x, pk=pk,
            out=torch.empty(T, w.d_out, dtype=w.dtype, device=dev),
            ws=torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)))
    stream = torch.cuda.current_stream(dev)
    sptr = stream.cuda_stream

    def step(i):
        s = sets[i % n_sets]
        rc = L.tmoe_forward(plan.ptr, s["x"].data_ptr(), T, s["pk"].data_ptr(), s["out"].data_ptr(),
                            None, None, None, s["ws"].data_ptr(), ws_bytes, sptr)
        if rc != 0:
            pkg._lib.check(rc)

    # -- warmup + timed region ------------------------------------------------
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = gpu_ms / steps
    tok_s = T * steps / (gpu_ms / 1e3)
    log(f"[{label}] {steps} steps: {gpu_ms:.3f} ms on the stream ({wall * 1e3:.3f} ms wall), "
        f"{ms_per_step * 1e3:.2f} us/step, {tok_s / 1e6:.2f} M tok/s")
    plan.signal_status()   # raises if a kernel lost an in-launch signal

    # -- per-stage kernel durations (HIP events recorded by the library) ---------
    pkg._lib.prof_enable(True)
    try:
        for i in range(steps):
            step(i)
        torch.cuda.synchronize()
        stage_ms, calls = pkg._lib.prof_read()
    finally:
        pkg._lib.prof_enable(False)
    stage_avg_us = {n: stage_ms[j] / calls * 1e3 for j, n in enumerate(pkg._lib.STAGE_NAMES)}
    fl_algo = w.flops()
    fl = w.flops_executed(T, rk, folded)        # the dominant kernel's own work
    fl["front"] = fl["router"] + fl["in_proj"]   # one kernel computes both
    kr = path == pkg._lib.TMOE_PATH_LARGE_KR
    sb = (w.stage_bytes_kr(T, rk) if kr else
          w.stage_bytes_folded(T, rk) if folded else w.stage_bytes())
    one_launch = path in (pkg._lib.TMOE_PATH_DECODE, pkg._lib.TMOE_PATH_FUSED,
                          pkg._lib.TMOE_PATH_FUSED_MID)
    kname = {pkg._lib.TMOE_PATH_DECODE: "k_sk_decode", pkg._lib.TMOE_PATH_FUSED: "k_fused_large",
             pkg._lib.TMOE_PATH_FUSED_MID: "k_fused_mid"}
    if one_launch:
        # the one kernel (recorded as the front stage) runs the whole layer; the other
        # two stages record no kernel
        fl["front"] = fl["total"]
        sb["front"] = w.layer_bytes_folded(T, rk)
        log(f"[{label}] one launch ({kname[path]}): the front stage is the whole layer")
    dom = max(stage_avg_us, key=stage_avg_us.get)
    dom_label = (f"front = whole layer ({kname[path]}, one launch)"
                 if one_launch and dom == "front" else dom)
    dom_tflops = fl[dom] / (stage_avg_us[dom] * 1e-6) / 1e12
    dom_gbs = sb[dom] / (stage_avg_us[dom] * 1e-6) / 1e9
    peak = PEAK_TFLOPS[dt_name]
    # the bound of the dominant kernel: MFMA when its arithmetic intensity is above
    # the ridge (peak flop/s over HBM bytes/s), HBM otherwise
    mfma_bound = fl[dom] / sb[dom] >= peak * 1e12 / (HBM_PEAK_GBS * 1e9)
    layer_tflops = fl_algo["total"] / (ms_per_step * 1e-3) / 1e12
    layer_exec_tflops = fl["total"] / (ms_per_step * 1e-3) / 1e12
    log(f"[{label}] per-stage avg us: " + ", ".join(f"{k}={v:.2f}" for k, v in stage_avg_us.items()))
    log(f"[{label}] dominant kernel {dom}: {dom_tflops:.1f} TFLOP/s = {dom_tflops / peak:.3f} of peak, "
        f"{dom_gbs:.1f} GB/s = {dom_gbs / HBM_PEAK_GBS:.3f} of HBM; "
        f"layer {layer_exec_tflops:.1f} TFLOP/s executed = {layer_exec_tflops / peak:.3f} of peak; "
        f"{layer_tflops:.1f} TFLOP/s = {layer_tflops / peak:.3f} counting the reference form's flops")

    if getattr(args, "copy_calibration_mib", 0) and label == "bench":
        n = args.copy_calibration_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[{label}] copy calibration: 3 x {args.copy_calibration_mib} MiB device copies")

    full_size = T == pkg.WORKLOADS[w.name].T
    stage_key = dom + ("_fused" if path in (pkg._lib.TMOE_PATH_FUSED,
                                            pkg._lib.TMOE_PATH_FUSED_MID) else
                       "_kr" if kr else "_folded" if folded else "")
    traffic = traffic_per_launch(w.name, stage_key) if full_size else None
    # MFMA-busy share of the dominant stage from the committed counter pass (the
    # timing-derived share is `frac`: executed flops / avg duration / peak at 2.4 GHz)
    mfma_util = (profile_figure(w.name, "mfma_util", stage_key)
                 if full_size and folded else None)

    # -- parity on a slice (GPU result of set 0 vs the fp32 reference path) --------
    from oracle import tucker_moe_np as onp
    from oracle import tucker_moe_torch as ot
    n_par = min(T, 512)
    s0 = sets[0]
    idx = torch.empty(T, w.k, dtype=torch.int32, device=dev)
    pkg._lib.check(L.tmoe_forward(plan.ptr, s0["x"].data_ptr(), T, s0["pk"].data_ptr(),
                                  s0["out"].data_ptr(), idx.data_ptr(), None, None,
                                  s0["ws"].data_ptr(), ws_bytes, sptr))
    torch.cuda.synchronize()
    ref = ot.forward(x0[:n_par], ref_params, w.k, compute_dtype=torch.float32, intermediates=True)
    parity = {
        "tokens": n_par,
        "rel_l2_out": onp.rel_l2(s0["out"][:n_par].float().cpu().numpy(), ref["out"].double().numpy()),
        "topk_idx_equal": bool(torch.equal(idx[:n_par].long().cpu(), ref["idx"])),
        "min_topk_gap": float(onp.topk_gap(ref["logits"].double().numpy(), w.k).min()),
        "reference": "oracle/tucker_moe_torch fp32 on the bf16-valued inputs"
                     + (" and the dequantised e4m3 weights" if w.fp8 else ""),
    }
    log(f"[{label}] parity on {n_par} tokens: {parity}")

    # -- host-CPU baseline (rank 0, N=1): the reference op sequence on the CPU --------
    cpu_res = None
    if cpu:
        cpu_res = cpu_baseline(lambda xs, **kw: ot.forward(xs, params, w.k, **kw), x0, T, 512,
                               args.cpu_seconds, f"{w.name}", dt_name,
                               "reference op sequence (oracle/tucker_moe_torch)",
                               oracle_mode=dt_name != "f32")
        log(f"[{label}] CPU baseline: {cpu_res['value']:.1f} tok/s on {cpu_res['cores']} threads "
            f"({cpu_res['tokens']} tokens, median of 3 passes {cpu_res['seconds']:.2f} s)")

    res = {
        "metric": METRIC,
        "value": tok_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dt_name,
        "data": "synthetic (seeded N(0,1) tokens, N(0,1/fan_in) weights; no checkpoint)",
        "config": {"workload": f"{w.name}: Tucker-MoE layer forward, one GPU", "T": T,
                   "d_in": w.d_in, "d_out": w.d_out, "E": w.E, "top_k": w.k,
                   "r1": w.r1, "r3": w.r3, "r2": w.r2, "rotated_sets": n_sets,
                   "weights": (("U_in/core/U_out fp8 e4m3 + per-output-channel fp32 scales; U_in "
                                "unpacked exactly to bf16, W = core U_out formed from the "
                                "dequantised weights and rounded once to bf16; bf16 MFMA")
                               if w.fp8 and folded else
                               "U_in/core/U_out fp8 e4m3 + per-output-channel fp32 scales, "
                               "unpacked exactly to bf16; bf16 MFMA" if w.fp8 else dt_name),
                   "form": form, "path": pkg._lib.PATH_NAMES.get(path, str(path))},
        "roofline": ({"bound": "mfma", "kernel": dom_label, "achieved": dom_tflops, "peak": peak,
                      "unit": "TFLOP/s", "frac": dom_tflops / peak, "traffic": traffic,
                      "mfma_util_counter": mfma_util,
                      "mfma_util_source": (f"profiles/tmoe_forward_{w.name}_counters.md"
                                           if mfma_util is not None else None),
                      "avg_us": stage_avg_us[dom], "flops_per_launch": fl[dom]}
                     if mfma_bound else
                     {"bound": "hbm", "kernel": dom_label, "achieved": dom_gbs, "peak": HBM_PEAK_GBS,
                      "unit": "GB/s", "frac": dom_gbs / HBM_PEAK_GBS, "traffic": traffic,
                      "mfma_util_counter": mfma_util,
                      "avg_us": stage_avg_us[dom], "bytes_per_launch": sb[dom]}),
        # executed: the MFMA work the kernels run (the folded form skips the core's);
        # the algorithmic figures count the reference form's flops
        "layer": {"executed_tflops": layer_exec_tflops,
                  "executed_mfma_frac": layer_exec_tflops / peak,
                  "tflops": layer_tflops, "mfma_frac": layer_tflops / peak,
                  "flops_per_step": fl_algo["total"],
                  "executed_flops_per_step": fl["total"],
                  "hbm_gbs_compulsory": w.hbm_bytes() / (ms_per_step * 1e-3) / 1e9,
                  "stage_avg_us": stage_avg_us},
        "parity": parity,
        "cpu_baseline": cpu_res,
        "speedup_vs_cpu": (tok_s / cpu_res["value"]) if cpu_res else None,
    }
    del sets
    torch.cuda.empty_cache()
    return {"result": res}


if __name__ == "__main__":
    main()
