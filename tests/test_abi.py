"""The C-ABI library: loads, exports every symbol include/tmoe.h declares, and
rejects bad arguments on the host before any GPU call (so these run anywhere)."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions(header="tmoe.h"):
    src = open(os.path.join(ROOT, "include", header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(tmoe_[a-z0-9_]+)\s*\(", src)))


def test_exports_every_header_symbol(pkg):
    L = pkg._lib.lib()
    declared = _header_functions()
    assert set(declared) == set(pkg._lib.EXPORTED)
    for name in declared:
        assert hasattr(L, name), name


def test_probe_library_exports_its_header(pkg):
    """The measurement harness's probe library (bench.py's "probes") loads and
    exports what include/tmoe_probe.h declares; a bad argument is refused on the
    host."""
    path = os.path.join(os.path.dirname(pkg._lib.LIB_PATH), "libtmoe_probe.so")
    L = ctypes.CDLL(path)
    declared = _header_functions("tmoe_probe.h")
    assert declared == ["tmoe_probe_l2_stream", "tmoe_probe_mfma"]
    for name in declared:
        assert hasattr(L, name), name
    L.tmoe_probe_l2_stream.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    g = ctypes.c_double()
    assert L.tmoe_probe_l2_stream(0, 5, ctypes.byref(g)) == -1   # waves must be 4 or 8


def test_abi_version(pkg):
    assert pkg._lib.lib().tmoe_abi_version() == pkg._lib.ABI_VERSION


def _shape(pkg, **kw):
    d = dict(d_in=512, d_out=1024, E=8, k=2, r1=4, r2=256, r3=128, dtype=pkg._lib.TMOE_F32,
             eps=1e-5)
    d.update(kw)
    return pkg._lib.TmoeShape(**d)


def _create(pkg, **kw):
    L = pkg._lib.lib()
    p = ctypes.c_void_p()
    rc = L.tmoe_plan_create(ctypes.byref(_shape(pkg, **kw)), ctypes.byref(p))
    return rc, p, L.tmoe_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(k=9), -1, "exceeds the number of experts"),
    (dict(k=0), -1, "positive"),
    (dict(d_in=-1), -1, "positive"),
    (dict(dtype=7), -1, "dtype"),
    (dict(eps=-1.0), -1, "eps"),
    (dict(d_in=100), -2, "d_in"),
    (dict(r3=96), -2, "r3"),
    (dict(r2=100), -2, "r2"),
    (dict(d_out=1000), -2, "d_out"),
    (dict(E=300, k=2), -2, "E=300"),
    (dict(E=32, k=17), -2, "top_k=17"),
    (dict(r1=65), -2, "r1"),
    (dict(router_mode=2), -1, "router_mode"),
    (dict(flags=4), -1, "flags"),
    (dict(router_mode=1, router_scale=0.0, router_temperature=0.5), -1, "router_scale"),
    (dict(router_mode=1, router_scale=10.0, router_temperature=-1.0), -1, "router_temperature"),
])
def test_plan_create_rejects(pkg, kw, code, msg):
    rc, p, err = _create(pkg, **kw)
    assert rc == code and msg in err and not p.value


def test_plan_sizes(pkg):
    rc, p, _ = _create(pkg)
    L = pkg._lib.lib()
    assert rc == 0
    try:
        assert L.tmoe_workspace_bytes(p, 0) == 0
        ws64 = L.tmoe_workspace_bytes(p, 64)
        assert ws64 >= 64 * (128 * 4 + 4 * 4 + 2 * 4 + 2 * 4 + 256 * 4)
        assert L.tmoe_workspace_bytes(p, 128) > ws64
        assert L.tmoe_workspace_bytes(p, -1) == 0
        pb = L.tmoe_packed_bytes(p)
        # every weight once (router rows padded to 16), f32
        assert pb >= 4 * (16 * 512 + 512 * 128 + 128 + 8 * 4 + 4 * 128 * 256 + 256 * 1024 + 1024)
    finally:
        L.tmoe_plan_destroy(p)


def test_forward_validation_never_launches(pkg):
    """Every argument error is returned before the first HIP call."""
    rc, p, _ = _create(pkg)
    L = pkg._lib.lib()
    fwd = L.tmoe_forward
    ok = 0x10000   # 16-byte aligned dummy addresses, never dereferenced
    ws = L.tmoe_workspace_bytes(p, 64)
    try:
        assert fwd(None, ok, 64, ok, ok, None, None, None, ok, ws, None) == -1
        assert fwd(p, ok, -1, ok, ok, None, None, None, ok, ws, None) == -1
        assert fwd(p, ok, 0, None, None, None, None, None, None, 0, None) == 0   # T == 0: no-op
        assert fwd(p, None, 64, ok, ok, None, None, None, ok, ws, None) == -1
        assert fwd(p, ok, 64, ok, None, None, None, None, ok, ws, None) == -1
        assert fwd(p, ok + 4, 64, ok, ok, None, None, None, ok, ws, None) == -1
        assert "aligned" in L.tmoe_last_error().decode()
        assert fwd(p, ok, 64, ok, ok, None, None, None, ok, ws - 1, None) == -1
        assert "workspace" in L.tmoe_last_error().decode()
        assert fwd(p, ok, 1 << 31, ok, ok, None, None, None, ok, ws, None) == -2
        pk = L.tmoe_pack_weights
        assert pk(p, ok, ok, ok, None, ok, ok, ok, ok, None) == -1
        assert "U_expert" in L.tmoe_last_error().decode()
        assert pk(p, ok, ok, ok, ok, ok, ok, ok, ok + 8, None) == -1
        assert pk(None, ok, ok, ok, ok, ok, ok, ok, ok, None) == -1
    finally:
        L.tmoe_plan_destroy(p)


def test_plan_wrapper_raises(pkg):
    with pytest.raises(pkg._lib.TmoeError) as e:
        pkg._lib.Plan(512, 1024, 8, 9, 4, 256, 128, torch.float32, 1e-5)
    assert e.value.code == -1
    with pytest.raises(pkg._lib.TmoeError):
        pkg._lib.Plan(512, 1024, 8, 2, 4, 256, 128, torch.float16, 1e-5)


def test_prof_read_empty(pkg):
    ms, calls = pkg._lib.prof_read()
    assert calls == 0 and ms == [0.0] * pkg._lib.N_STAGES


def test_fp8_plan_and_pack_validation(pkg):
    """TMOE_BF16_FP8W plans: larger packed buffer (the scale arrays), packed only
    by tmoe_pack_weights_fp8, and every argument error before any HIP call."""
    L = pkg._lib.lib()
    rc, p8, _ = _create(pkg, dtype=pkg._lib.TMOE_BF16_FP8W)
    rc2, pb, _ = _create(pkg, dtype=pkg._lib.TMOE_BF16)
    assert rc == 0 and rc2 == 0
    ok = 0x10000
    try:
        # + U_in scales (r3), core scale table (r1 * r2), U_out scales (d_out), f32
        assert L.tmoe_packed_bytes(p8) >= L.tmoe_packed_bytes(pb) + 4 * (128 + 4 * 256 + 1024)
        assert L.tmoe_workspace_bytes(p8, 64) == L.tmoe_workspace_bytes(pb, 64)
        pk, pk8 = L.tmoe_pack_weights, L.tmoe_pack_weights_fp8
        assert pk(p8, ok, ok, ok, ok, ok, ok, ok, ok, None) == -1
        assert "tmoe_pack_weights_fp8" in L.tmoe_last_error().decode()
        args = [ok] * 11
        assert pk8(pb, *args, None) == -1
        assert "TMOE_BF16_FP8W" in L.tmoe_last_error().decode()
        for i, name in enumerate(["router_w", "U_in_q", "U_in_scale", "inner_w", "U_expert",
                                  "core_q", "core_scale", "U_out_q", "U_out_scale", "bias",
                                  "packed"]):
            a = list(args)
            a[i] = None
            assert pk8(p8, *a, None) == -1, name
            assert name in L.tmoe_last_error().decode()
        a = list(args)
        a[10] = ok + 4
        assert pk8(p8, *a, None) == -1 and "aligned" in L.tmoe_last_error().decode()
    finally:
        L.tmoe_plan_destroy(p8)
        L.tmoe_plan_destroy(pb)
    with pytest.raises(pkg._lib.TmoeError):
        pkg._lib.Plan(512, 1024, 8, 2, 4, 256, 128, torch.float32, 1e-5, fp8_weights=True)


def test_forward_epi_and_rmsnorm_validation_never_launch(pkg):
    """tmoe_forward_epi and tmoe_rmsnorm_rows reject bad epilogue / norm
    arguments before any HIP call."""
    rc, p, _ = _create(pkg)
    L = pkg._lib.lib()
    lb = pkg._lib
    fe = L.tmoe_forward_epi
    ok = 0x10000
    ws = L.tmoe_workspace_bytes(p, 64)
    try:
        assert fe(p, ok, 64, ok, ok, None, None, None, ok, ws, 7, ok, ok, None) == -1
        assert "epi_mode" in L.tmoe_last_error().decode()
        assert fe(p, ok, 64, ok, ok, None, None, None, ok, ws, lb.TMOE_EPI_GLU, None, None,
                  None) == -1
        assert "epi_a" in L.tmoe_last_error().decode()
        assert fe(p, ok, 64, ok, ok, None, None, None, ok, ws, lb.TMOE_EPI_GLU, ok + 2, None,
                  None) == -1
        assert fe(p, ok, 64, ok, ok, None, None, None, ok, ws, lb.TMOE_EPI_RESIDUAL_SCALE, ok,
                  None, None) == -1
        assert "gamma" in L.tmoe_last_error().decode()
        # argument errors of tmoe_forward are still reported with an epilogue
        assert fe(p, ok, 64, ok, ok, None, None, None, ok, ws - 1, lb.TMOE_EPI_GLU, ok, None,
                  None) == -1
        assert "workspace" in L.tmoe_last_error().decode()
        assert fe(p, ok, 0, None, None, None, None, None, None, 0, lb.TMOE_EPI_GLU, ok, None,
                  None) == 0
    finally:
        L.tmoe_plan_destroy(p)
    rn = L.tmoe_rmsnorm_rows
    assert rn(ok, 4, 64, ok, 1e-5, 5, ok, None) == -1
    assert "dtype" in L.tmoe_last_error().decode()
    assert rn(ok, -1, 64, ok, 1e-5, lb.TMOE_BF16, ok, None) == -1
    assert rn(ok, 4, 0, ok, 1e-5, lb.TMOE_BF16, ok, None) == -1
    assert rn(ok, 4, 64, ok, -1.0, lb.TMOE_BF16, ok, None) == -1
    assert rn(ok, 4, 64, None, 1e-5, lb.TMOE_BF16, ok, None) == -1
    assert rn(None, 0, 64, None, 1e-5, lb.TMOE_BF16, None, None) == 0   # T == 0: no-op


def test_forward_glu_validation_never_launches(pkg):
    rc, p, _ = _create(pkg)
    L = pkg._lib.lib()
    fg = L.tmoe_forward_glu
    ok, ok2 = 0x10000, 0x20000
    ws = L.tmoe_workspace_bytes(p, 64)
    try:
        assert fg(None, ok, 64, ok, ok, ok, ok, ok2, ws, None) == -1
        assert fg(p, ok, -1, ok, ok, ok, ok, ok2, ws, None) == -1
        assert fg(p, ok, 0, None, None, None, None, None, 0, None) == 0   # T == 0: no-op
        assert fg(p, ok, 64, ok, None, ok, ok, ok2, ws, None) == -1
        assert fg(p, ok, 64, ok, ok, ok, ok, ok, ws, None) == -1
        assert "coincide" in L.tmoe_last_error().decode()
        assert fg(p, ok, 64, ok, ok, ok, ok, ok2 + 8, ws, None) == -1
        assert "aligned" in L.tmoe_last_error().decode()
        assert fg(p, ok, 64, ok, ok, ok, ok, ok2, ws - 1, None) == -1
        assert "workspace" in L.tmoe_last_error().decode()
    finally:
        L.tmoe_plan_destroy(p)


@pytest.mark.parametrize("kw,rank", [
    (dict(E=16, r1=4, dtype=1), 4),                # the north-star shape: r1 form
    (dict(E=8, r1=32, r2=512, r3=256, dtype=1), 8),   # reference ranks: expert form
    (dict(E=8, r1=32, r2=512, r3=256, dtype=0), 8),   # fp32: expert form (k_core)
    (dict(E=3, k=2, r1=8, dtype=1), 8),            # bf16: E = 3 would leave the persistent core
    (dict(E=3, k=2, r1=8, dtype=0), 3),
    (dict(E=1, k=1, r1=4, dtype=1), 1),
    (dict(E=8, r1=32, r2=512, r3=256, dtype=2), 32),  # fp8 weights: never re-formed
])
def test_plan_core_rank(pkg, kw, rank):
    """tmoe_plan_core_rank: E for plans with fewer experts than ranks (not fp8, and
    not trading the persistent core for the Khatri-Rao one), else r1."""
    rc, p, err = _create(pkg, **kw)
    assert rc == 0, err
    L = pkg._lib.lib()
    try:
        assert L.tmoe_plan_core_rank(p) == rank
    finally:
        L.tmoe_plan_destroy(p)
    assert L.tmoe_plan_core_rank(None) == 0


BF16 = 1
FP8W = 2


@pytest.mark.parametrize("kw,folded", [
    # the BASELINE ranks (4, 1024, 256): 1024 * 2304 < 4 * 256 * 1024 + 1024 * 2304
    (dict(d_in=1536, d_out=2304, E=16, k=2, r1=4, r2=1024, r3=256, dtype=BF16), 1),
    (dict(d_in=1536, d_out=2304, E=256, k=8, r1=4, r2=1024, r3=256, dtype=BF16), 1),
    (dict(d_in=1536, d_out=2304, E=16, k=2, r1=4, r2=1024, r3=256, dtype=FP8W), 1),
    (dict(d_in=1536, d_out=2304, E=16, k=2, r1=4, r2=1024, r3=256, dtype=BF16, flags=1), 0),
    # fp32 plans keep two GEMMs
    (dict(d_in=512, d_out=1024, E=8, k=2, r1=4, r2=256, r3=128), 0),
    # the deployed checkpoint ranks (32, 512, 256): 8192 * 4608 > 32 * 256 * 512 + 512 * 4608
    (dict(d_in=768, d_out=4608, E=8, k=2, r1=32, r2=512, r3=256, dtype=BF16), 0),
    # expert form (rank E = 8 < r1 = 64): folds over the E ranks, 8 * 64 * 128 < ...
    (dict(d_in=128, d_out=128, E=8, k=2, r1=64, r2=128, r3=64, dtype=BF16), 1),
])
def test_plan_folded(pkg, kw, folded):
    rc, p, msg = _create(pkg, **kw)
    assert rc == 0, msg
    L = pkg._lib.lib()
    try:
        assert L.tmoe_plan_folded(p) == folded
        if folded:
            # the two-GEMM form's buffers + W^T (d_out, rk * r3) bf16 - P^T (rk * r2, r3)
            # bf16 (the unfolded core's operand, which a folded forward never reads;
            # bf16 plans with rk in {1, 2, 4} or 4G have it, not fp8 ones with rk = 4G)
            un = dict(kw, flags=1)
            rc2, p2, msg2 = _create(pkg, **un)
            assert rc2 == 0, msg2
            rk = L.tmoe_plan_core_rank(p)
            wt = kw["d_out"] * rk * kw["r3"] * 2
            pt = rk * kw["r2"] * kw["r3"] * 2
            extra = L.tmoe_packed_bytes(p) - L.tmoe_packed_bytes(p2)
            assert any(abs(extra - (wt - d)) < 256 for d in (0, pt)), (extra, wt, pt)
            if kw.get("dtype") == BF16 and rk in (1, 2, 4):
                assert abs(extra - (wt - pt)) < 256    # P^T dropped
            L.tmoe_plan_destroy(p2)
    finally:
        L.tmoe_plan_destroy(p)
    assert L.tmoe_plan_folded(None) == 0


def test_forward_static_rejects_before_gpu_work(pkg):
    """tmoe_forward_static: every size and pointer check happens on the host before
    the static scratch is looked up (no GPU needed for these paths)."""
    L = pkg._lib.lib()
    assert L.tmoe_static_scratch_bytes() == 48 << 20
    rc, p, msg = _create(pkg, d_in=1536, d_out=2304, E=16, k=2, r1=4, r2=1024, r3=256, dtype=BF16)
    assert rc == 0, msg
    try:
        assert L.tmoe_forward_static(None, 16, 4, 16, 16, None, None, None, None) == -1
        assert L.tmoe_forward_static(p, 16, 0, 16, 16, None, None, None, None) == 0   # T = 0
        assert L.tmoe_forward_static(p, 16, -1, 16, 16, None, None, None, None) == -1
        # the C3 shape: 16384 tokens fit, twice that does not
        assert L.tmoe_workspace_bytes(p, 16384) <= L.tmoe_static_scratch_bytes()
        rc = L.tmoe_forward_static(p, 16, 32768, 16, 16, None, None, None, None)
        assert rc == -2 and b"static maximum" in L.tmoe_last_error()
        assert L.tmoe_forward_static(p, None, 64, 16, 16, None, None, None, None) == -1
        assert L.tmoe_forward_static(p, 8, 64, 16, 16, None, None, None, None) == -1  # misaligned
    finally:
        L.tmoe_plan_destroy(p)


def test_signal_status_host_side(pkg):
    """tmoe_signal_status reads the plan's status block on the host: a null plan is
    EINVAL; a fresh plan reports nothing (on a machine without a GPU the block is
    never allocated and nothing can have run). tmoe_set_wait_polls returns the
    previous budget and ignores a negative one."""
    L = pkg._lib.lib()
    mask = ctypes.c_uint32(7)
    assert L.tmoe_signal_status(None, 0, ctypes.byref(mask)) == pkg._lib.TMOE_EINVAL
    assert mask.value == 0 and "null plan" in L.tmoe_last_error().decode()
    rc, p, _ = _create(pkg)
    assert rc == 0
    try:
        assert L.tmoe_signal_status(p, 1, ctypes.byref(mask)) == pkg._lib.TMOE_OK
        assert mask.value == 0
        assert L.tmoe_signal_status(p, 0, None) == pkg._lib.TMOE_OK
    finally:
        L.tmoe_plan_destroy(p)
    plan = pkg._lib.Plan(512, 1024, 8, 2, 4, 256, 128, torch.float32, 1e-5)
    assert plan.signal_status() == 0
    prev = pkg._lib.set_wait_polls(-1)
    assert prev >= 0
    try:
        assert pkg._lib.set_wait_polls(5) == prev
        assert pkg._lib.set_wait_polls(-3) == 5
    finally:
        pkg._lib.set_wait_polls(prev)
    assert pkg._lib.set_wait_polls(-1) == prev


@pytest.mark.parametrize("flags,ok", [(0, True), (1, True), (2, True), (3, True), (4, False),
                                      (8, False)])
def test_plan_flags(pkg, flags, ok):
    """TMOE_FLAG_NO_FOLD (1) and TMOE_FLAG_NO_FUSE (2) are the only plan flags."""
    rc, p, err = _create(pkg, flags=flags)
    try:
        assert (rc == 0) == ok, err
        if not ok:
            assert rc == pkg._lib.TMOE_EINVAL and "flags" in err
    finally:
        if p.value:
            pkg._lib.lib().tmoe_plan_destroy(p)


def test_forward_path_rules(pkg):
    """tmoe_forward_path's host-side selection (no GPU: as on a 256-compute-unit
    MI355X): decode in one launch, the one-launch large-T and mid-T forwards, the
    wide-router forward whose out-projection forms c (x) z itself, and the plain
    launches."""
    cases = [("C2", 32, pkg._lib.TMOE_PATH_DECODE), ("C3", 16384, pkg._lib.TMOE_PATH_FUSED),
             ("C5", 16384, pkg._lib.TMOE_PATH_FUSED), ("C3", 4096, pkg._lib.TMOE_PATH_LARGE),
             ("C4", 4096, pkg._lib.TMOE_PATH_LARGE_KR), ("C4", 600, pkg._lib.TMOE_PATH_LARGE),
             ("C3", 2048, pkg._lib.TMOE_PATH_FUSED_MID), ("C3", 257, pkg._lib.TMOE_PATH_FUSED_MID),
             ("C3", 3001, pkg._lib.TMOE_PATH_LARGE), ("C3", 200, pkg._lib.TMOE_PATH_SMALL)]
    for name, T, want in cases:
        w = pkg.WORKLOADS[name]
        m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg()).to(w.dtype)
        assert m.plan().forward_path(T) == want, (name, T)
    w = pkg.WORKLOADS["C4"]
    m = pkg.TuckerMoE(w.d_in, w.d_out, w.cfg()).to(w.dtype).set_fold(False)
    assert m.plan().forward_path(4096) == pkg._lib.TMOE_PATH_LARGE   # unfolded: no c (x) z
