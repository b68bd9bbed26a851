// Host side of the C ABI declared in include/tmoe.h: argument validation, the
// plan (packed-weight and workspace layout), and the launch sequence.
//
// Every entry point validates on the host before its first HIP call, so each
// error path is reachable without a GPU.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <new>
#include <vector>

#include "tmoe.h"
#include "tmoe_internal.h"

struct tmoe_plan {
  tmoe_shape s;
  int64_t E_pad;
  size_t es;     // element size of the activations (and of the packed weights)
  bool fp8w;     // TMOE_BF16_FP8W: weights arrive as e4m3 + scales, kernels run bf16
  int kdtype;    // dtype the kernels compute in (TMOE_BF16 / TMOE_F32)
  // packed-weight layout (byte offsets); the front operand is U_in^T (r3 rows)
  // immediately followed by the router rows (E_pad rows, zero past E). fp8 plans
  // add the U_in column scales, the core scale table and the U_out column scales.
  size_t off_front, off_router, off_gain, off_uexp, off_core, off_uout, off_bias;
  size_t off_sin, off_cscale, off_sout, off_craw, packed_bytes;
  bool core_p;      // the core runs k_core_pp (T > kSmallT) from P^T at off_core_p
  size_t off_core_p;
  bool wfrag;       // the front operand also in k_front_ks's fragment order, at off_wfrag
  size_t off_wfrag;
  // rank of the contraction the kernels run: r1, or E for plans packed in the
  // expert form (fewer experts than ranks, weights not fp8): U_expert packed as
  // the identity (E x E) and core as G_e = sum_r U_expert[e, r] core_r
  int64_t rk;
  // folded form (large T): W^T (d_out, rk*r3) at off_fold, one GEMM of c (x) z against W
  bool fold;
  size_t off_fold;
  // status block (tmoe::kStatusWords words of pinned host memory mapped for the
  // device, set by kernels; null on a machine without a GPU): host and device address
  uint32_t* status_host;
  uint32_t* status_dev;
};

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(TMOE_EHIP, "%s: %s", what, hipGetErrorString(e));
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// budget of the kernels' waits for in-launch signals, in polls (tmoe_set_wait_polls)
std::atomic<int> g_wait_polls{tmoe::kDefaultWaitPolls};

// The plan's status block: pinned host memory the kernels write through a mapped
// device address. Left null when no GPU is present (plans stay usable for every
// host-side call) or when the allocation fails (the kernels then report only
// through the workspace's error word).
void alloc_status(tmoe_plan* p) {
  p->status_host = p->status_dev = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    (void)hipGetLastError();   // leave no sticky error behind
    return;
  }
  void* h = nullptr;
  if (hipHostMalloc(&h, tmoe::kStatusWords * sizeof(uint32_t),
                    hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent) !=
          hipSuccess ||
      !h) {
    (void)hipGetLastError();
    return;
  }
  memset(h, 0, tmoe::kStatusWords * sizeof(uint32_t));
  void* d = nullptr;
  if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess || !d) {
    (void)hipGetLastError();
    (void)hipHostFree(h);
    return;
  }
  p->status_host = static_cast<uint32_t*>(h);
  p->status_dev = static_cast<uint32_t*>(d);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int kStages = 3;

// Per-stage event record of tmoe_prof_enable.
struct Prof {
  std::mutex mu;
  bool on = false;
  std::vector<hipEvent_t> free_ev;
  std::vector<std::vector<hipEvent_t>> pending;   // kStages + 1 events per forward
};
Prof g_prof;

hipEvent_t prof_event() {
  if (!g_prof.free_ev.empty()) {
    hipEvent_t e = g_prof.free_ev.back();
    g_prof.free_ev.pop_back();
    return e;
  }
  // timing only: no system-scope fence (its cache writeback and invalidation at
  // every stage boundary slowed the following kernel by up to ~15%)
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
  return e;
}

struct Layout {
  size_t z, c, idx, w, mid, raw, mpart, sync, total;
  int split, fsplit;
};

Layout workspace_layout(const tmoe_plan* p, int64_t T) {
  Layout L{};
  size_t o = 0;
  // k_core_pp reads c and stores mid in whole 256-token tiles; a folded plan's
  // out-projection reads its A operand (c (x) z in mid) in whole 256-row tiles
  const int64_t tile_rows = p->core_p || p->fold
                                ? (T + tmoe::kCorePRows - 1) / tmoe::kCorePRows * tmoe::kCorePRows
                                : T;
  // z in whole tiles too: a folded plan's out-projection may read it as its A operand
  L.z = o;   o = align256(o + (size_t)(p->fold ? tile_rows : T) * p->s.r3 * p->es);
  L.c = o;   o = align256(o + (size_t)tile_rows * p->rk * sizeof(float));
  L.idx = o; o = align256(o + (size_t)T * p->s.k * sizeof(int32_t));
  L.w = o;   o = align256(o + (size_t)T * p->s.k * sizeof(float));
  // mid: (T, r2), or c (x) z (T, rk*r3) in a folded plan's large-T forward
  const int64_t mid_cols =
      p->fold && T > tmoe::kSmallT && p->rk * p->s.r3 > p->s.r2 ? p->rk * p->s.r3 : p->s.r2;
  L.mid = o; o = align256(o + (size_t)tile_rows * mid_cols * p->es);
  L.raw = o;
  L.fsplit = tmoe::front_split(T, p->s.d_in, p->E_pad, p->kdtype == TMOE_BF16);
  if (T <= tmoe::kSmallT || L.fsplit > 1) {
    int64_t raw_floats = L.fsplit * T * tmoe::raw_stride(p->s.r3, p->s.E);
    // the one-launch decode's scratch (z columns, sums of squares, c)
    if (T <= tmoe::kDecodeMaxT)
      raw_floats = std::max(raw_floats, tmoe::sk_decode_scratch_floats(T, p->s.r3, p->rk));
    o = align256(o + (size_t)raw_floats * sizeof(float));
  }
  // k_core_pp in rank groups: fp32 partial sums of mid
  L.mpart = 0;
  L.split = 1;
  if (p->core_p && tmoe::core_p_grouped(p->rk) && T > tmoe::kSmallT) {
    L.split = tmoe::core_p_split(T, p->rk, p->s.r2);
    L.mpart = o;
    o = align256(o + (size_t)L.split * tile_rows * p->s.r2 * sizeof(float));
  }
  // error word and flags of the kernels that signal between work-groups
  L.sync = o;
  if (T > 0)
    o = align256(o + (size_t)tmoe::sync_words(
                             T, std::max<int64_t>(T <= tmoe::kDecodeMaxT
                                                      ? tmoe::sk_decode_flags(p->s.r3) : 0,
                                                  tmoe::front_sliced_flags(T, L.fsplit))) *
                         sizeof(uint32_t));
  L.total = o;
  return L;
}

// The kernels' arguments for one forward of plan p (epilogue fields unset).
tmoe::FwdArgs make_args(const tmoe_plan* p, const void* x, int64_t T, const void* packed,
                        void* out, int32_t* topk_idx, float* topk_w, float* logits,
                        void* workspace, const Layout& L) {
  const tmoe_shape& s = p->s;
  const char* pk = static_cast<const char*>(packed);
  char* ws = static_cast<char*>(workspace);
  tmoe::FwdArgs a{};
  a.dtype = p->kdtype;
  a.router_mode = s.router_mode;
  a.router_scale = s.router_scale;
  a.router_temperature = s.router_temperature;
  a.T = T; a.d_in = s.d_in; a.d_out = s.d_out; a.E = s.E; a.E_pad = p->E_pad; a.k = s.k;
  a.r1 = p->rk; a.r2 = s.r2; a.r3 = s.r3; a.eps = s.eps;
  a.x = x;
  a.wfront = pk + p->off_front;
  a.wfrag = p->wfrag ? pk + p->off_wfrag : nullptr;
  a.gain = reinterpret_cast<const float*>(pk + p->off_gain);
  a.uexp = reinterpret_cast<const float*>(pk + p->off_uexp);
  a.coreT = pk + p->off_core;
  a.coreP = p->core_p ? pk + p->off_core_p : nullptr;
  a.uoutT = pk + p->off_uout;
  a.bias = reinterpret_cast<const float*>(pk + p->off_bias);
  if (p->fp8w) {
    a.zscale = reinterpret_cast<const float*>(pk + p->off_sin);
    a.core_scale = reinterpret_cast<const float*>(pk + p->off_cscale);
    a.out_scale = reinterpret_cast<const float*>(pk + p->off_sout);
    a.core_scale_raw = reinterpret_cast<const float*>(pk + p->off_craw);
  }
  a.out = out;
  a.idx = topk_idx ? topk_idx : reinterpret_cast<int32_t*>(ws + L.idx);
  a.w = topk_w ? topk_w : reinterpret_cast<float*>(ws + L.w);
  a.logits = logits;
  a.c = reinterpret_cast<float*>(ws + L.c);
  a.z = ws + L.z;
  a.mid = ws + L.mid;
  a.mid_rows_256 = p->core_p || p->fold;   // workspace_layout's tile_rows
  a.raw = reinterpret_cast<float*>(ws + L.raw);
  a.mpart = L.mpart ? reinterpret_cast<float*>(ws + L.mpart) : nullptr;
  a.core_split = L.split;
  a.front_split = L.fsplit;
  a.sync = reinterpret_cast<uint32_t*>(ws + L.sync);
  a.wait_polls = g_wait_polls.load(std::memory_order_relaxed);
  a.status = p->status_dev;
  return a;
}

// W^T of a folded plan from the packed core^T and U_out^T (fp8 plans: with the raw
// core channel scales and the U_out column scales).
hipError_t pack_fold(const tmoe_plan* p, char* base, hipStream_t st) {
  const tmoe_shape& s = p->s;
  auto f32at = [&](size_t off) { return reinterpret_cast<const float*>(base + off); };
  return tmoe::launch_fold_out_t(reinterpret_cast<const uint16_t*>(base + p->off_core),
                                 reinterpret_cast<const uint16_t*>(base + p->off_uout),
                                 p->fp8w ? f32at(p->off_craw) : nullptr,
                                 p->fp8w ? f32at(p->off_sout) : nullptr,
                                 reinterpret_cast<uint16_t*>(base + p->off_fold), p->rk * s.r3,
                                 s.r3, s.r2, s.d_out, st);
}

// A folded plan's large-T stages 2 and 3: c (x) z into mid, then the out-projection
// kernel as one GEMM of width rk*r3 against W.
tmoe::FwdArgs folded_args(const tmoe_plan* p, const tmoe::FwdArgs& a, const void* packed,
                          hipStream_t st) {
  tmoe::FwdArgs f = a;
  f.r2 = p->rk * p->s.r3;
  f.uoutT = static_cast<const char*>(packed) + p->off_fold;
  f.out_scale = nullptr;
  // the out-projection forms c (x) z itself where it can (z and c from the
  // front); else the front writes c (x) z into mid where it can, else
  // k_expand_cz does
  f.kr = tmoe::outproj_kr_ok(f);
  f.cz = !f.kr && tmoe::front_fuses_cz(f, st) ? f.mid : nullptr;
  return f;
}

hipError_t launch_nothing(const tmoe::FwdArgs&, hipStream_t) { return hipSuccess; }

using Launch = hipError_t (*)(const tmoe::FwdArgs&, hipStream_t);

// The small-T stages (front, core, out-projection) of a forward with args a: the
// front epilogue runs inside the core (or, folded, the out-projection) when that
// kernel's LDS holds it, else as its own kernel after the front's GEMM.
void small_stages(const tmoe::FwdArgs& a, bool fold, hipStream_t stream, Launch (&st)[kStages]) {
  if (fold && tmoe::small_decode_ok(a, stream)) {   // one launch
    st[0] = tmoe::launch_small_decode;
    st[1] = launch_nothing;
    st[2] = launch_nothing;
  } else if (tmoe::small_epi_fused_ok(a)) {
    st[0] = tmoe::launch_small_front_raw;
    st[1] = fold ? launch_nothing : tmoe::launch_small_core_epi;
    st[2] = fold ? tmoe::launch_small_out_epi : tmoe::launch_small_out;
  } else {
    st[0] = tmoe::launch_small_front;
    st[1] = fold ? launch_nothing : tmoe::launch_small_core;
    st[2] = fold ? tmoe::launch_small_out_kr : tmoe::launch_small_out;
  }
}

// stage 2 of a folded plan: c (x) z, unless the front already wrote it or the
// out-projection forms it
hipError_t launch_cz(const tmoe::FwdArgs& f, hipStream_t st) {
  return f.cz || f.kr ? hipSuccess : tmoe::launch_expand_cz(f, st);
}

}  // namespace

extern "C" {

int tmoe_abi_version(void) { return TMOE_ABI_VERSION; }

const char* tmoe_last_error(void) { return g_err; }

int tmoe_plan_create(const tmoe_shape* shape, tmoe_plan** plan_out) {
  g_err[0] = 0;
  if (!shape || !plan_out) return fail(TMOE_EINVAL, "tmoe_plan_create: null argument");
  *plan_out = nullptr;
  const tmoe_shape& s = *shape;
  if (s.dtype != TMOE_BF16 && s.dtype != TMOE_F32 && s.dtype != TMOE_BF16_FP8W)
    return fail(TMOE_EINVAL, "dtype %d is not TMOE_BF16, TMOE_F32 or TMOE_BF16_FP8W", s.dtype);
  if (s.d_in <= 0 || s.d_out <= 0 || s.E <= 0 || s.k <= 0 || s.r1 <= 0 || s.r2 <= 0 || s.r3 <= 0)
    return fail(TMOE_EINVAL,
                "dimensions must be positive (d_in=%lld d_out=%lld E=%lld k=%lld r=(%lld,%lld,%lld))",
                (long long)s.d_in, (long long)s.d_out, (long long)s.E, (long long)s.k,
                (long long)s.r1, (long long)s.r2, (long long)s.r3);
  if (s.k > s.E)   // torch.topk raises for k > size (model.py:76)
    return fail(TMOE_EINVAL, "top_k=%lld exceeds the number of experts E=%lld", (long long)s.k,
                (long long)s.E);
  if (!(s.eps >= 0.f)) return fail(TMOE_EINVAL, "eps must be >= 0");
  if (s.router_mode != TMOE_ROUTER_SOFTMAX_TOPK && s.router_mode != TMOE_ROUTER_CAPPED)
    return fail(TMOE_EINVAL, "router_mode %d is neither TMOE_ROUTER_SOFTMAX_TOPK nor "
                             "TMOE_ROUTER_CAPPED", s.router_mode);
  if (s.router_mode == TMOE_ROUTER_CAPPED &&
      !(s.router_scale > 0.f && s.router_temperature > 0.f && s.router_scale < INFINITY &&
        s.router_temperature < INFINITY))
    return fail(TMOE_EINVAL, "router_scale and router_temperature must be finite and > 0");
  if (s.d_in % 64)
    return fail(TMOE_EUNSUPPORTED, "d_in=%lld: must be a multiple of 64", (long long)s.d_in);
  if (s.r3 != 64 && s.r3 != 128 && s.r3 != 256)
    return fail(TMOE_EUNSUPPORTED, "r3=%lld: supported values are 64, 128, 256",
                (long long)s.r3);
  if (s.r2 % 64)
    return fail(TMOE_EUNSUPPORTED, "r2=%lld: must be a multiple of 64", (long long)s.r2);
  if (s.d_out % 16)
    return fail(TMOE_EUNSUPPORTED, "d_out=%lld: must be a multiple of 16", (long long)s.d_out);
  if (s.E > tmoe::kMaxExperts)
    return fail(TMOE_EUNSUPPORTED, "E=%lld: at most %d experts", (long long)s.E,
                tmoe::kMaxExperts);
  if (s.k > tmoe::kMaxTopK)
    return fail(TMOE_EUNSUPPORTED, "top_k=%lld: at most %d", (long long)s.k, tmoe::kMaxTopK);
  if (s.r1 > 64)
    return fail(TMOE_EUNSUPPORTED, "r1=%lld: at most 64", (long long)s.r1);
  if (s.flags & ~(TMOE_FLAG_NO_FOLD | TMOE_FLAG_NO_FUSE))
    return fail(TMOE_EINVAL, "flags 0x%x: unknown bits", (unsigned)s.flags);
  // a GEMM tile (at most 512 operand rows of at most 4 MB) spans < 4 GB: the
  // kernels address it with 32-bit offsets
  if (s.d_in > (1 << 20) || s.r2 > (1 << 20))
    return fail(TMOE_EUNSUPPORTED, "d_in=%lld, r2=%lld: at most %d each", (long long)s.d_in,
                (long long)s.r2, 1 << 20);

  tmoe_plan* p = new (std::nothrow) tmoe_plan();
  if (!p) return fail(TMOE_EINVAL, "out of host memory");
  p->s = s;
  p->fp8w = s.dtype == TMOE_BF16_FP8W;
  p->kdtype = s.dtype == TMOE_F32 ? TMOE_F32 : TMOE_BF16;
  p->es = p->kdtype == TMOE_BF16 ? 2 : 4;
  int64_t ep = 32;
  while (ep < s.E) ep *= 2;   // router column blocks of 32: widths 32, 64, 128, 256
  p->E_pad = ep;
  size_t o = 0;
  p->off_front = o;
  p->off_router = o + (size_t)s.r3 * s.d_in * p->es;
  o = align256(p->off_router + (size_t)p->E_pad * s.d_in * p->es);
  p->off_gain = o; o = align256(o + (size_t)s.r3 * sizeof(float));
  // the expert form when it contracts fewer ranks and keeps the persistent core
  const bool bf = p->kdtype == TMOE_BF16;
  p->rk = s.r1;
  if (!p->fp8w && s.E < s.r1 &&
      (tmoe::core_p_supported(s.E, s.r2, bf, false) || !tmoe::core_p_supported(s.r1, s.r2, bf, false)))
    p->rk = s.E;
  p->off_uexp = o; o = align256(o + (size_t)s.E * p->rk * sizeof(float));
  p->off_core = o; o = align256(o + (size_t)s.r2 * p->rk * s.r3 * p->es);
  p->off_uout = o; o = align256(o + (size_t)s.d_out * s.r2 * p->es);
  p->off_bias = o; o = align256(o + (size_t)s.d_out * sizeof(float));
  p->off_sin = p->off_cscale = p->off_sout = p->off_craw = 0;
  if (p->fp8w) {
    p->off_sin = o;    o = align256(o + (size_t)s.r3 * sizeof(float));
    p->off_cscale = o; o = align256(o + (size_t)s.r1 * s.r2 * sizeof(float));
    p->off_sout = o;   o = align256(o + (size_t)s.d_out * sizeof(float));
    p->off_craw = o;   o = align256(o + (size_t)s.r1 * s.r2 * sizeof(float));
  }
  // folded form: bf16 kernels, fewer multiply-adds per token
  const int64_t K = p->rk * s.r3;
  p->fold = bf && !(s.flags & TMOE_FLAG_NO_FOLD) && K * s.d_out < K * s.r2 + s.r2 * s.d_out;
  // P^T feeds only the unfolded core (k_core_pp); a folded forward never reads it
  p->core_p = !p->fold && tmoe::core_p_supported(p->rk, s.r2, bf, p->fp8w);
  p->off_core_p = 0;
  if (p->core_p) { p->off_core_p = o; o = align256(o + (size_t)p->rk * s.r2 * s.r3 * p->es); }
  p->off_fold = 0;
  if (p->fold) { p->off_fold = o; o = align256(o + (size_t)s.d_out * K * p->es); }
  // the register-weight front (k_front_ks): bf16 kernels, r3 = 256, one router block
  p->wfrag = bf && s.r3 == 256 && p->E_pad == 32;
  p->off_wfrag = 0;
  if (p->wfrag) {
    p->off_wfrag = o;
    o = align256(o + (size_t)(s.r3 + p->E_pad) * s.d_in * p->es);
  }
  p->packed_bytes = o;
  alloc_status(p);
  *plan_out = p;
  return TMOE_OK;
}

void tmoe_plan_destroy(tmoe_plan* plan) {
  if (!plan) return;
  if (plan->status_host) (void)hipHostFree(plan->status_host);
  delete plan;
}

size_t tmoe_packed_bytes(const tmoe_plan* plan) { return plan ? plan->packed_bytes : 0; }

int64_t tmoe_plan_core_rank(const tmoe_plan* plan) { return plan ? plan->rk : 0; }

int tmoe_plan_folded(const tmoe_plan* plan) { return plan && plan->fold ? 1 : 0; }

// 1: front operand, gain, U_expert, core^T, U_out^T, bias, fp8 tables; 2: + P^T for
// r1 in {1, 2, 4}; 3: P^T also for r1 = 4G in rank-group order; 4: plans with fewer
// experts than ranks packed in the expert form (identity U_expert, core G); 5: folded
// plans add W^T = (core U_out)^T; 7: bf16 plans with r3 = 256 and E_pad = 32 add the
// front operand in fragment order (k_front_ks).
int tmoe_packed_layout_version(void) { return 7; }

size_t tmoe_workspace_bytes(const tmoe_plan* plan, int64_t T) {
  if (!plan || T < 0) return 0;
  return workspace_layout(plan, T).total;
}

int tmoe_pack_weights(const tmoe_plan* p, const void* router_w, const void* U_in,
                      const void* inner_w, const void* U_expert, const void* core,
                      const void* U_out, const void* bias, void* packed, void* stream) {
  g_err[0] = 0;
  if (!p) return fail(TMOE_EINVAL, "tmoe_pack_weights: null plan");
  if (p->fp8w)
    return fail(TMOE_EINVAL, "tmoe_pack_weights: a TMOE_BF16_FP8W plan is packed by "
                             "tmoe_pack_weights_fp8");
  const void* ptrs[] = {router_w, U_in, inner_w, U_expert, core, U_out, bias, packed};
  const char* names[] = {"router_w", "U_in", "inner_w", "U_expert", "core", "U_out", "bias",
                         "packed"};
  for (int i = 0; i < 8; ++i) {
    if (!ptrs[i]) return fail(TMOE_EINVAL, "tmoe_pack_weights: %s is null", names[i]);
    if (i == 7 && !aligned16(ptrs[i]))
      return fail(TMOE_EINVAL, "tmoe_pack_weights: packed is not 16-byte aligned");
  }
  const tmoe_shape& s = p->s;
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* base = static_cast<char*>(packed);
  const int es = (int)p->es;
  hipError_t e;
  if ((e = tmoe::launch_transpose(U_in, base + p->off_front, s.d_in, s.r3, es, st)) != hipSuccess)
    return hip_fail(e, "pack U_in");
  if ((e = tmoe::launch_copy_pad(router_w, base + p->off_router, s.E * s.d_in,
                                 p->E_pad * s.d_in, es, st)) != hipSuccess)
    return hip_fail(e, "pack router");
  if (p->wfrag && (e = tmoe::launch_pack_frag(base + p->off_front, base + p->off_wfrag,
                                              s.r3 + p->E_pad, s.d_in, st)) != hipSuccess)
    return hip_fail(e, "pack front fragments");
  if ((e = tmoe::launch_to_f32(inner_w, reinterpret_cast<float*>(base + p->off_gain), s.r3,
                               s.dtype, st)) != hipSuccess)
    return hip_fail(e, "pack inner_norm.weight");
  if (p->rk != s.r1) {
    // expert form: core^T of G, P^T from it, U_expert the identity
    if ((e = tmoe::launch_eye(reinterpret_cast<float*>(base + p->off_uexp), s.E, st)) !=
        hipSuccess)
      return hip_fail(e, "pack U_expert (identity)");
    if ((e = tmoe::launch_mix_core_t(U_expert, core, base + p->off_core, s.E, s.r1, s.r3, s.r2,
                                     es, st)) != hipSuccess)
      return hip_fail(e, "pack core (expert form)");
    if (p->core_p &&
        (e = tmoe::launch_pack_core_p(base + p->off_core, false, nullptr,
                                      reinterpret_cast<uint16_t*>(base + p->off_core_p), p->rk,
                                      s.r3, s.r2, st, true)) != hipSuccess)
      return hip_fail(e, "pack core (P layout)");
  } else {
    if ((e = tmoe::launch_to_f32(U_expert, reinterpret_cast<float*>(base + p->off_uexp),
                                 s.E * s.r1, s.dtype, st)) != hipSuccess)
      return hip_fail(e, "pack U_expert");
    if ((e = tmoe::launch_transpose(core, base + p->off_core, s.r1 * s.r3, s.r2, es, st)) !=
        hipSuccess)
      return hip_fail(e, "pack core");
    if (p->core_p &&
        (e = tmoe::launch_pack_core_p(core, false, nullptr,
                                      reinterpret_cast<uint16_t*>(base + p->off_core_p), s.r1,
                                      s.r3, s.r2, st)) != hipSuccess)
      return hip_fail(e, "pack core (P layout)");
  }
  if ((e = tmoe::launch_transpose(U_out, base + p->off_uout, s.r2, s.d_out, es, st)) !=
      hipSuccess)
    return hip_fail(e, "pack U_out");
  if ((e = tmoe::launch_to_f32(bias, reinterpret_cast<float*>(base + p->off_bias), s.d_out,
                               s.dtype, st)) != hipSuccess)
    return hip_fail(e, "pack bias");
  if (p->fold && (e = pack_fold(p, base, st)) != hipSuccess) return hip_fail(e, "pack W (fold)");
  return TMOE_OK;
}

int tmoe_pack_weights_fp8(const tmoe_plan* p, const void* router_w, const uint8_t* U_in_q,
                          const float* U_in_scale, const void* inner_w, const void* U_expert,
                          const uint8_t* core_q, const float* core_scale,
                          const uint8_t* U_out_q, const float* U_out_scale, const void* bias,
                          void* packed, void* stream) {
  g_err[0] = 0;
  if (!p) return fail(TMOE_EINVAL, "tmoe_pack_weights_fp8: null plan");
  if (!p->fp8w)
    return fail(TMOE_EINVAL, "tmoe_pack_weights_fp8: the plan's dtype is not TMOE_BF16_FP8W");
  const void* ptrs[] = {router_w, U_in_q, U_in_scale, inner_w, U_expert, core_q,
                        core_scale, U_out_q, U_out_scale, bias, packed};
  const char* names[] = {"router_w", "U_in_q", "U_in_scale", "inner_w", "U_expert", "core_q",
                         "core_scale", "U_out_q", "U_out_scale", "bias", "packed"};
  for (int i = 0; i < 11; ++i)
    if (!ptrs[i]) return fail(TMOE_EINVAL, "tmoe_pack_weights_fp8: %s is null", names[i]);
  if (!aligned16(packed))
    return fail(TMOE_EINVAL, "tmoe_pack_weights_fp8: packed is not 16-byte aligned");
  const tmoe_shape& s = p->s;
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* base = static_cast<char*>(packed);
  auto f32at = [&](size_t off) { return reinterpret_cast<float*>(base + off); };
  auto bf16at = [&](size_t off) { return reinterpret_cast<uint16_t*>(base + off); };
  hipError_t e;
  // a zero scale packs its channel as zeros (whatever its codes, NaN included);
  // U_in's and U_out's scales are per column: group = all rows
  if ((e = tmoe::launch_transpose_e4m3(U_in_q, bf16at(p->off_front), s.d_in, s.r3, U_in_scale,
                                       s.d_in, st)) != hipSuccess)
    return hip_fail(e, "pack U_in");
  if ((e = tmoe::launch_copy_pad(router_w, base + p->off_router, s.E * s.d_in,
                                 p->E_pad * s.d_in, 2, st)) != hipSuccess)
    return hip_fail(e, "pack router");
  if (p->wfrag && (e = tmoe::launch_pack_frag(base + p->off_front, base + p->off_wfrag,
                                              s.r3 + p->E_pad, s.d_in, st)) != hipSuccess)
    return hip_fail(e, "pack front fragments");
  if ((e = tmoe::launch_to_f32(inner_w, f32at(p->off_gain), s.r3, TMOE_BF16, st)) != hipSuccess)
    return hip_fail(e, "pack inner_norm.weight");
  if ((e = tmoe::launch_to_f32(U_expert, f32at(p->off_uexp), s.E * s.r1, TMOE_BF16, st)) !=
      hipSuccess)
    return hip_fail(e, "pack U_expert");
  // core (r1, r3, r2) -> (r2, r1*r3); channel (r, q) of row r*r3 + s, column q
  if ((e = tmoe::launch_transpose_e4m3(core_q, bf16at(p->off_core), s.r1 * s.r3, s.r2,
                                       core_scale, s.r3, st)) != hipSuccess)
    return hip_fail(e, "pack core");
  if ((e = tmoe::launch_core_scales(core_scale, f32at(p->off_cscale), s.r1, s.r2, st)) !=
      hipSuccess)
    return hip_fail(e, "pack core scales");
  if (p->core_p &&
      (e = tmoe::launch_pack_core_p(core_q, true, core_scale, bf16at(p->off_core_p), s.r1, s.r3,
                                    s.r2, st)) != hipSuccess)
    return hip_fail(e, "pack core (P layout)");
  if ((e = tmoe::launch_transpose_e4m3(U_out_q, bf16at(p->off_uout), s.r2, s.d_out, U_out_scale,
                                       s.r2, st)) != hipSuccess)
    return hip_fail(e, "pack U_out");
  if ((e = tmoe::launch_to_f32(bias, f32at(p->off_bias), s.d_out, TMOE_BF16, st)) != hipSuccess)
    return hip_fail(e, "pack bias");
  if ((e = tmoe::launch_to_f32(U_in_scale, f32at(p->off_sin), s.r3, TMOE_F32, st)) !=
      hipSuccess)
    return hip_fail(e, "pack U_in scales");
  if ((e = tmoe::launch_to_f32(U_out_scale, f32at(p->off_sout), s.d_out, TMOE_F32, st)) !=
      hipSuccess)
    return hip_fail(e, "pack U_out scales");
  if ((e = tmoe::launch_to_f32(core_scale, f32at(p->off_craw), s.r1 * s.r2, TMOE_F32, st)) !=
      hipSuccess)
    return hip_fail(e, "pack core scales");
  if (p->fold && (e = pack_fold(p, base, st)) != hipSuccess) return hip_fail(e, "pack W (fold)");
  return TMOE_OK;
}

int tmoe_forward(const tmoe_plan* p, const void* x, int64_t T, const void* packed, void* out,
                 int32_t* topk_idx, float* topk_w, float* logits, void* workspace,
                 size_t workspace_bytes, void* stream) {
  return tmoe_forward_epi(p, x, T, packed, out, topk_idx, topk_w, logits, workspace,
                          workspace_bytes, TMOE_EPI_NONE, nullptr, nullptr, stream);
}

namespace {
// The forward of tmoe_forward_epi (argument checks included). With prof_ok false
// no profiling event is recorded (tmoe_forward_static).
int forward_impl(const tmoe_plan* p, const void* x, int64_t T, const void* packed, void* out,
                 int32_t* topk_idx, float* topk_w, float* logits, void* workspace,
                 size_t workspace_bytes, int epi_mode, const void* epi_a, const void* epi_b,
                 void* stream, bool prof_ok) {
  if (!p) return fail(TMOE_EINVAL, "tmoe_forward: null plan");
  if (epi_mode != TMOE_EPI_NONE && epi_mode != TMOE_EPI_GLU && epi_mode != TMOE_EPI_RESIDUAL_SCALE)
    return fail(TMOE_EINVAL, "tmoe_forward_epi: epi_mode %d is not a TMOE_EPI_* value", epi_mode);
  if (epi_mode != TMOE_EPI_NONE && (!epi_a || !aligned16(epi_a)))
    return fail(TMOE_EINVAL, "tmoe_forward_epi: epi_a must be a 16-byte aligned (T, d_out) tensor");
  if (epi_mode == TMOE_EPI_RESIDUAL_SCALE && (!epi_b || !aligned16(epi_b)))
    return fail(TMOE_EINVAL, "tmoe_forward_epi: epi_b (gamma) must be 16-byte aligned");
  if (T < 0) return fail(TMOE_EINVAL, "tmoe_forward: T=%lld < 0", (long long)T);
  if (T > (int64_t)1 << 30) return fail(TMOE_EUNSUPPORTED, "tmoe_forward: T=%lld too large",
                                        (long long)T);
  if (T == 0) return TMOE_OK;
  if (!x || !packed || !out || !workspace)
    return fail(TMOE_EINVAL, "tmoe_forward: null x/packed/out/workspace");
  if (!aligned16(x) || !aligned16(packed) || !aligned16(workspace) || !aligned16(out))
    return fail(TMOE_EINVAL, "tmoe_forward: x/packed/out/workspace must be 16-byte aligned");
  const Layout L = workspace_layout(p, T);
  if (workspace_bytes < L.total)
    return fail(TMOE_EINVAL, "tmoe_forward: workspace of %zu bytes, %zu needed for T=%lld",
                workspace_bytes, L.total, (long long)T);
  tmoe::FwdArgs a = make_args(p, x, T, packed, out, topk_idx, topk_w, logits, workspace, L);
  a.epi_mode = epi_mode;
  a.epi_a = epi_mode != TMOE_EPI_NONE ? epi_a : nullptr;
  a.epi_b = epi_mode == TMOE_EPI_RESIDUAL_SCALE ? epi_b : nullptr;

  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool small = T <= tmoe::kSmallT;
  const bool fold = p->fold;
  // the K-sliced front in one launch where the device and the stream allow
  a.front_one = !(p->s.flags & TMOE_FLAG_NO_FUSE) && tmoe::front_sliced_ok(a, st);
  if (fold) a = folded_args(p, a, packed, st);
  // the large-T folded forward in one launch where the plan, T and the device allow
  const bool fuse_ok = fold && !small && !(p->s.flags & TMOE_FLAG_NO_FUSE);
  const bool fused = fuse_ok && tmoe::fused_large_ok(a, st);
  // the mid-T folded forward in one launch (K-sliced front + 128 x 144 tiles)
  const bool fused_mid = fuse_ok && !fused && tmoe::fused_mid_ok(a, st);
  const Launch big_path[kStages] = {
      fused ? tmoe::launch_fused_large : fused_mid ? tmoe::launch_fused_mid : tmoe::launch_front,
      fused || fused_mid ? launch_nothing : fold ? launch_cz : tmoe::launch_core,
      fused || fused_mid ? launch_nothing : tmoe::launch_outproj};
  // folded: the out-projection builds c (x) z from z and c itself (no core stage)
  Launch small_path[kStages];
  small_stages(a, fold, st, small_path);
  const Launch* stages = small ? small_path : big_path;
  const char* stage_names[kStages] = {"front (router + in-projection)", "core",
                                      "out-projection"};

  std::vector<hipEvent_t> ev;
  std::unique_lock<std::mutex> lk(g_prof.mu);
  const bool prof = g_prof.on && prof_ok;
  if (!prof) lk.unlock();
  // on an error the events taken so far go back to the pool (the lock is held)
  auto release = [&](hipEvent_t extra) {
    for (hipEvent_t e : ev) g_prof.free_ev.push_back(e);
    if (extra) g_prof.free_ev.push_back(extra);
    ev.clear();
  };
  for (int i = 0; i < kStages; ++i) {
    if (prof) {
      hipEvent_t e = prof_event();
      if (!e || hipEventRecord(e, st) != hipSuccess) {
        release(e);
        return fail(TMOE_EHIP, "profiling event");
      }
      ev.push_back(e);
    }
    const hipError_t e = stages[i](a, st);
    if (e != hipSuccess) {
      if (prof) release(nullptr);
      return hip_fail(e, stage_names[i]);
    }
  }
  if (prof) {
    hipEvent_t e = prof_event();
    if (!e || hipEventRecord(e, st) != hipSuccess) {
      release(e);
      return fail(TMOE_EHIP, "profiling event");
    }
    ev.push_back(e);
    g_prof.pending.push_back(std::move(ev));
  }
  return TMOE_OK;
}
}  // namespace

int tmoe_forward_epi(const tmoe_plan* p, const void* x, int64_t T, const void* packed, void* out,
                     int32_t* topk_idx, float* topk_w, float* logits, void* workspace,
                     size_t workspace_bytes, int epi_mode, const void* epi_a, const void* epi_b,
                     void* stream) {
  g_err[0] = 0;
  return forward_impl(p, x, T, packed, out, topk_idx, topk_w, logits, workspace, workspace_bytes,
                      epi_mode, epi_a, epi_b, stream, true);
}

size_t tmoe_static_scratch_bytes(void) { return tmoe::kStaticScratchBytes; }

int tmoe_forward_static(const tmoe_plan* p, const void* x, int64_t T, const void* packed,
                        void* out, int32_t* topk_idx, float* topk_w, float* logits,
                        void* stream) {
  g_err[0] = 0;
  if (!p) return fail(TMOE_EINVAL, "tmoe_forward_static: null plan");
  if (T < 0) return fail(TMOE_EINVAL, "tmoe_forward_static: T=%lld < 0", (long long)T);
  if (T > (int64_t)1 << 30)
    return fail(TMOE_EUNSUPPORTED, "tmoe_forward_static: T=%lld too large", (long long)T);
  if (T == 0) return TMOE_OK;
  // every check that needs no GPU comes before the scratch lookup
  const size_t need = workspace_layout(p, T).total;
  if (need > tmoe::kStaticScratchBytes)
    return fail(TMOE_EUNSUPPORTED,
                "tmoe_forward_static: T=%lld needs %zu bytes of scratch, more than the static "
                "maximum of %zu (use tmoe_forward with a workspace, or fewer tokens per call)",
                (long long)T, need, tmoe::kStaticScratchBytes);
  if (!x || !packed || !out) return fail(TMOE_EINVAL, "tmoe_forward_static: null x/packed/out");
  if (!aligned16(x) || !aligned16(packed) || !aligned16(out))
    return fail(TMOE_EINVAL, "tmoe_forward_static: x/packed/out must be 16-byte aligned");
  void* ws = nullptr;
  if (hipError_t e = tmoe::static_scratch(static_cast<hipStream_t>(stream), &ws); e != hipSuccess)
    return hip_fail(e, "tmoe_forward_static: static scratch address");
  return forward_impl(p, x, T, packed, out, topk_idx, topk_w, logits, ws,
                      tmoe::kStaticScratchBytes, TMOE_EPI_NONE, nullptr, nullptr, stream, false);
}

int tmoe_forward_glu(const tmoe_plan* p, const void* x, int64_t T, const void* packed_gate,
                     const void* packed_up, void* out, void* ws_gate, void* ws_up,
                     size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  if (!p) return fail(TMOE_EINVAL, "tmoe_forward_glu: null plan");
  if (T < 0) return fail(TMOE_EINVAL, "tmoe_forward_glu: T=%lld < 0", (long long)T);
  if (T > (int64_t)1 << 30)
    return fail(TMOE_EUNSUPPORTED, "tmoe_forward_glu: T=%lld too large", (long long)T);
  if (T == 0) return TMOE_OK;
  if (!x || !packed_gate || !packed_up || !out || !ws_gate || !ws_up)
    return fail(TMOE_EINVAL, "tmoe_forward_glu: null pointer");
  if (!aligned16(x) || !aligned16(packed_gate) || !aligned16(packed_up) || !aligned16(out) ||
      !aligned16(ws_gate) || !aligned16(ws_up))
    return fail(TMOE_EINVAL, "tmoe_forward_glu: pointers must be 16-byte aligned");
  if (ws_gate == ws_up) return fail(TMOE_EINVAL, "tmoe_forward_glu: the two workspaces coincide");
  const Layout L = workspace_layout(p, T);
  if (workspace_bytes < L.total)
    return fail(TMOE_EINVAL, "tmoe_forward_glu: workspaces of %zu bytes, %zu needed for T=%lld",
                workspace_bytes, L.total, (long long)T);
  tmoe::FwdArgs g = make_args(p, x, T, packed_gate, out, nullptr, nullptr, nullptr, ws_gate, L);
  tmoe::FwdArgs u = make_args(p, x, T, packed_up, out, nullptr, nullptr, nullptr, ws_up, L);
  u.epi_mode = tmoe::kEpiGlu;   // out = silu(gate) * up, the gate output read from `out`
  u.epi_a = out;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (p->fold) {
    g = folded_args(p, g, packed_gate, st);
    u = folded_args(p, u, packed_up, st);
  }
  if (T <= tmoe::kSmallT) {
    for (const tmoe::FwdArgs* a : {&g, &u}) {
      Launch small[kStages];
      small_stages(*a, p->fold, st, small);
      for (int i = 0; i < kStages; ++i)
        if ((e = small[i](*a, st)) != hipSuccess) return hip_fail(e, "tmoe_forward_glu");
    }
    return TMOE_OK;
  }
  const Launch mid = p->fold ? launch_cz : tmoe::launch_core;
  if ((e = tmoe::launch_front_pair(g, u, st)) != hipSuccess ||
      (e = mid(g, st)) != hipSuccess || (e = mid(u, st)) != hipSuccess ||
      (e = tmoe::launch_outproj(g, st)) != hipSuccess ||
      (e = tmoe::launch_outproj(u, st)) != hipSuccess)
    return hip_fail(e, "tmoe_forward_glu");
  return TMOE_OK;
}

int tmoe_rmsnorm_rows(const void* x, int64_t T, int64_t d, const void* weight, float eps,
                      int dtype, void* out, void* stream) {
  g_err[0] = 0;
  if (dtype != TMOE_BF16 && dtype != TMOE_F32)
    return fail(TMOE_EINVAL, "tmoe_rmsnorm_rows: dtype %d is not TMOE_BF16 or TMOE_F32", dtype);
  if (T < 0 || d <= 0)
    return fail(TMOE_EINVAL, "tmoe_rmsnorm_rows: T=%lld, d=%lld", (long long)T, (long long)d);
  if (!(eps >= 0.f)) return fail(TMOE_EINVAL, "tmoe_rmsnorm_rows: eps must be >= 0");
  if (T == 0) return TMOE_OK;
  if (!x || !weight || !out) return fail(TMOE_EINVAL, "tmoe_rmsnorm_rows: null x/weight/out");
  const hipError_t e = tmoe::launch_rmsnorm_rows(x, T, d, weight, eps, dtype, out,
                                                 static_cast<hipStream_t>(stream));
  return e == hipSuccess ? TMOE_OK : hip_fail(e, "tmoe_rmsnorm_rows");
}

namespace {
int latent_check(const char* who, int64_t B, int64_t E, int64_t k, int64_t r3, int64_t r2,
                 int dtype) {
  if (dtype != TMOE_BF16 && dtype != TMOE_F32)
    return fail(TMOE_EINVAL, "%s: dtype %d is not TMOE_BF16 or TMOE_F32", who, dtype);
  if (B < 0 || E < 1 || k < 1 || k > E)
    return fail(TMOE_EINVAL, "%s: B=%lld E=%lld k=%lld", who, (long long)B, (long long)E,
                (long long)k);
  if (k > tmoe::kMaxTopK || E > 64)
    return fail(TMOE_EUNSUPPORTED, "%s: at most 64 experts and top_k 16", who);
  if ((r3 != 64 && r3 != 128 && r3 != 256) || r2 <= 0 || r2 % 64)
    return fail(TMOE_EUNSUPPORTED, "%s: r3=%lld (64, 128 or 256), r2=%lld (a multiple of 64)",
                who, (long long)r3, (long long)r2);
  if (B > (int64_t)1 << 24)
    return fail(TMOE_EUNSUPPORTED, "%s: B=%lld too large", who, (long long)B);
  return TMOE_OK;
}
}  // namespace

size_t tmoe_latent_workspace_bytes(int64_t B, int64_t E, int64_t r3, int64_t r2, int dtype,
                                   int backward) {
  dtype &= ~TMOE_LATENT_P_F32;
  if (B < 0 || E < 1 || r3 < 1 || r2 < 1 || (dtype != TMOE_BF16 && dtype != TMOE_F32)) return 0;
  return tmoe::latent_workspace_bytes(B, E, r3, r2, dtype == TMOE_BF16 ? 2 : 4, backward != 0);
}

int tmoe_latent_forward(const void* x, const void* G, const int64_t* idx, const void* p,
                        int64_t B, int64_t E, int64_t k, int64_t r3, int64_t r2, int dtype,
                        void* out, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  const bool p_f32 = (dtype & TMOE_LATENT_P_F32) != 0;
  dtype &= ~TMOE_LATENT_P_F32;
  if (int rc = latent_check("tmoe_latent_forward", B, E, k, r3, r2, dtype)) return rc;
  if (B == 0) return TMOE_OK;
  if (!x || !G || !idx || !p || !out || !workspace)
    return fail(TMOE_EINVAL, "tmoe_latent_forward: null pointer");
  if (!aligned16(x) || !aligned16(G) || !aligned16(out) || !aligned16(workspace))
    return fail(TMOE_EINVAL, "tmoe_latent_forward: x/G/out/workspace must be 16-byte aligned");
  const size_t need = tmoe::latent_workspace_bytes(B, E, r3, r2, dtype == TMOE_BF16 ? 2 : 4, false);
  if (workspace_bytes < need)
    return fail(TMOE_EINVAL, "tmoe_latent_forward: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  tmoe::LatentArgs l{};
  l.dtype = dtype; l.p_f32 = p_f32; l.B = B; l.E = E; l.k = k; l.r3 = r3; l.r2 = r2;
  l.x = x; l.G = G; l.idx = idx; l.p = p; l.out = out; l.ws = workspace;
  const hipError_t e = tmoe::latent_forward(l, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? TMOE_OK : hip_fail(e, "tmoe_latent_forward");
}

int tmoe_latent_backward(const void* x, const void* G, const int64_t* idx, const void* p,
                         const void* dout, int64_t B, int64_t E, int64_t k, int64_t r3,
                         int64_t r2, int dtype, void* dx, void* dG, void* dp, void* workspace,
                         size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  const bool p_f32 = (dtype & TMOE_LATENT_P_F32) != 0;
  dtype &= ~TMOE_LATENT_P_F32;
  if (int rc = latent_check("tmoe_latent_backward", B, E, k, r3, r2, dtype)) return rc;
  if (B == 0) return TMOE_OK;
  if (!x || !G || !idx || !p || !dout || !dx || !dG || !dp || !workspace)
    return fail(TMOE_EINVAL, "tmoe_latent_backward: null pointer");
  if (!aligned16(x) || !aligned16(G) || !aligned16(dout) || !aligned16(dx) || !aligned16(dG) ||
      !aligned16(workspace))
    return fail(TMOE_EINVAL, "tmoe_latent_backward: x/G/dout/dx/dG/workspace must be 16-byte "
                             "aligned");
  const size_t need = tmoe::latent_workspace_bytes(B, E, r3, r2, dtype == TMOE_BF16 ? 2 : 4, true);
  if (workspace_bytes < need)
    return fail(TMOE_EINVAL, "tmoe_latent_backward: workspace of %zu bytes, %zu needed",
                workspace_bytes, need);
  tmoe::LatentArgs l{};
  l.dtype = dtype; l.p_f32 = p_f32; l.B = B; l.E = E; l.k = k; l.r3 = r3; l.r2 = r2;
  l.x = x; l.G = G; l.idx = idx; l.p = p; l.dout = dout; l.dx = dx; l.dG = dG; l.dp = dp;
  l.ws = workspace;
  const hipError_t e = tmoe::latent_backward(l, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? TMOE_OK : hip_fail(e, "tmoe_latent_backward");
}

int tmoe_forward_path(const tmoe_plan* p, int64_t T) {
  g_err[0] = 0;
  if (!p) return fail(TMOE_EINVAL, "tmoe_forward_path: null plan");
  if (T < 0) return fail(TMOE_EINVAL, "tmoe_forward_path: T=%lld < 0", (long long)T);
  if (T == 0) return 0;
  // the arguments of an eager forward with stand-in addresses (nothing is launched
  // or dereferenced: the selection rules look at shapes and at which buffers exist)
  char* const fake = reinterpret_cast<char*>(uintptr_t(1) << 20);
  const Layout L = workspace_layout(p, T);
  tmoe::FwdArgs a = make_args(p, fake, T, fake, fake, nullptr, nullptr, nullptr, fake, L);
  if (T <= tmoe::kSmallT) {
    if (p->fold) {
      tmoe::FwdArgs f = folded_args(p, a, fake, nullptr);
      if (tmoe::small_decode_shape_ok(f)) return TMOE_PATH_DECODE;
    }
    return TMOE_PATH_SMALL;
  }
  if (p->fold) {
    const tmoe::FwdArgs f = folded_args(p, a, fake, nullptr);
    if (!(p->s.flags & TMOE_FLAG_NO_FUSE) && tmoe::fused_large_shape_ok(f)) return TMOE_PATH_FUSED;
    if (!(p->s.flags & TMOE_FLAG_NO_FUSE) && tmoe::fused_mid_shape_ok(f))
      return TMOE_PATH_FUSED_MID;
    if (f.kr) return TMOE_PATH_LARGE_KR;
  }
  return TMOE_PATH_LARGE;
}

int tmoe_signal_status(const tmoe_plan* plan, int clear, uint32_t* mask) {
  g_err[0] = 0;
  if (mask) *mask = 0;
  if (!plan) return fail(TMOE_EINVAL, "tmoe_signal_status: null plan");
  if (!plan->status_host) return TMOE_OK;   // no GPU: no kernel ever ran
  volatile uint32_t* w = plan->status_host;
  uint32_t m = 0;
  if (w[tmoe::kStatusSignalWord]) m |= TMOE_STATUS_SIGNAL;
  if (clear) w[tmoe::kStatusSignalWord] = 0;
  if (mask) *mask = m;
  if (!m) return TMOE_OK;
  return fail(TMOE_ESIGNAL, "a kernel's wait for another work-group of its launch ran out of "
                            "its poll budget (the affected output rows are NaN or stale)");
}

int64_t tmoe_set_wait_polls(int64_t polls) {
  const int64_t prev = g_wait_polls.load(std::memory_order_relaxed);
  if (polls >= 0) g_wait_polls.store(polls > INT32_MAX ? INT32_MAX : (int)polls,
                                     std::memory_order_relaxed);
  return prev;
}

int tmoe_prof_enable(int on) {
  std::lock_guard<std::mutex> lk(g_prof.mu);
  g_prof.on = on != 0;
  return TMOE_OK;
}

int tmoe_prof_read(double* ms, int n, int64_t* calls) {
  g_err[0] = 0;
  std::lock_guard<std::mutex> lk(g_prof.mu);
  for (int i = 0; i < n && ms; ++i) ms[i] = 0.0;
  int64_t count = 0;
  int rc = kStages;
  for (auto& ev : g_prof.pending) {
    if (rc == kStages) {
      const hipError_t e = hipEventSynchronize(ev.back());
      if (e != hipSuccess) rc = hip_fail(e, "tmoe_prof_read");
    }
    if (rc == kStages) {
      for (int i = 0; i < kStages && i < n && ms; ++i) {
        float t = 0.f;
        if (hipEventElapsedTime(&t, ev[i], ev[i + 1]) == hipSuccess) ms[i] += t;
      }
      ++count;
    }
    for (hipEvent_t e : ev) g_prof.free_ev.push_back(e);
  }
  g_prof.pending.clear();
  if (calls) *calls = count;
  return rc;
}

}  // extern "C"
