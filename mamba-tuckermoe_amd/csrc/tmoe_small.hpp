// Small-T path: the layer for a few tokens (decode-shaped batches), where the
// cost is streaming the weights once and the large-tile kernels would leave most
// CUs idle with one long K loop each.
//
// Every projection is a "skinny" GEMM out (T x N) = A (T x K) * B^T (N x K)^T
// with the weight as B. A work-group owns 16 output columns for up to 16 * MF
// tokens; its W waves split K, each streaming its share of the 16 weight rows
// (and of A) straight from memory into registers in the 16x16 MFMA operand
// layout, so all of a wave's loads are in flight at once. The W partial tiles are
// added through LDS and the work-group's epilogue writes them out. No weight
// byte is read by more than one work-group per 16*MF tokens.
//
// Kernels (model.py line numbers as in tmoe_kernels.hpp):
//   k_sk_front   raw (T, r3 + E) fp32 = x [U_in | W_r^T]           (:75, :80)
//   k_front_epi  per token: RMSNorm of the raw z, top-k, softmax, c  (:76-81, :93)
//   k_sk_core    mid = (c (x) z) core^T, Khatri-Rao A built in registers (:87-98)
//   k_sk_out     out = mid U_out + bias                              (:101)
#pragma once

#include "tmoe_kernels.hpp"

namespace tmoe {
namespace dev {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// One 16x16 output block += A(16 x Ks) * B(Ks x 16) for one 16-byte chunk per
// lane: lane l supplies row / column (l & 15) and chunk elements at K offsets
// (l >> 4) * CE ... (CE = 8 bf16 or 4 f32 per chunk), so a step covers Ks = 4 CE.
// bf16: one v_mfma_f32_16x16x32_bf16. f32: four v_mfma_f32_16x16x4f32, chunk
// element j feeding MFMA j (A and B use the same order, so the sum is exact).
// Result element i of lane l: row 4 (l >> 4) + i, column l & 15.
__device__ __forceinline__ void mma16(f32x4& acc, u32x4 a, u32x4 b, EltBF16) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
}
__device__ __forceinline__ void mma16(f32x4& acc, u32x4 a, u32x4 b, EltF32) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[j]), __uint_as_float(b[j]), acc,
                                               0, 0, 0);
}

// A operand sources: chunk(row, k) = the 16 bytes of A row `row` (of the
// work-group's block) starting at element k. Rows past the end are clamped to the
// last row (their results are never stored).
template <class Elt>
struct SkRows {
  const char* base;   // first row of the block
  int64_t row_bytes;
  int rows_valid;
  __device__ __forceinline__ u32x4 chunk(int row, int64_t k) const {
    const int r = row < rows_valid ? row : rows_valid - 1;
    return *reinterpret_cast<const u32x4*>(base + r * row_bytes +
                                           k * (int64_t)sizeof(typename Elt::T));
  }
};

// A[t, r * r3 + s] = c[t, r] * z[t, s], rounded to the element type exactly as
// KhatriRaoLoader does; a chunk never straddles two ranks (r3 % 8 == 0).
template <class Elt>
struct SkKhatriRao {
  const char* z;      // first row of the block, (., r3)
  const float* c;     // first row of the block, (., r1)
  int r1, r3, rows_valid;
  __device__ __forceinline__ u32x4 chunk(int row, int64_t k) const {
    typedef typename Elt::T T;
    const int t = row < rows_valid ? row : rows_valid - 1;
    const int r = (int)(k / r3), s = (int)(k - (int64_t)r * r3);
    const u32x4 v = *reinterpret_cast<const u32x4*>(z + ((int64_t)t * r3 + s) * (int64_t)sizeof(T));
    const float cc = c[(int64_t)t * r1 + r];
    u32x4 o;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_bf16x2(bf16_bits_to_f32(v[j] & 0xffffu) * cc, bf16_bits_to_f32(v[j] >> 16) * cc);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = __float_as_uint(__uint_as_float(v[j]) * cc);
    }
    return o;
  }
};

// The skinny GEMM body. Each wave accumulates its K share for MF row blocks and
// the work-group's 16 columns; K is walked in groups of two steps (2 Ks
// elements), split evenly over the waves. rank_len > 0 (fp8 core only): K is
// made of ranks of rank_len elements whose partial sums are scaled by
// rank_scale[rank * rank_stride + column] before they are added. Returns, for
// every thread, nothing: the summed tile is left in `red` (LDS, [MF * 16][16]
// floats, row-major) after the final barrier.
// The B chunks of a wave's first batch (skinny_tile's first loads), loaded ahead
// by a caller with other latency to cover (skinny_b_first, then skinny_tile with
// kPre and the same arguments).
template <class Elt, int W, int GB>
__device__ __forceinline__ void skinny_b_first(const char* b, int64_t b_row_bytes, int cols_valid,
                                               int64_t K, u32x4 (&bv)[GB][2]) {
  typedef typename Elt::T T;
  constexpr int CE = 16 / (int)sizeof(T);
  constexpr int KS = 4 * CE, KG = 2 * KS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const char* brow = b + (col < cols_valid ? col : cols_valid - 1) * b_row_bytes;
  const int64_t ng = K / KG;
  const int64_t g0 = wave * ng / W, g1 = (wave + 1) * ng / W;
  const int kq = (lane >> 4) * CE;
#pragma unroll
  for (int q = 0; q < GB; ++q) {
    const int64_t g = g0 + q < g1 ? g0 + q : g0;
#pragma unroll
    for (int s = 0; s < 2; ++s)
      bv[q][s] = g0 < g1 ? *reinterpret_cast<const u32x4*>(brow + (g * KG + s * KS + kq) *
                                                               (int64_t)sizeof(T))
                         : u32x4{0u, 0u, 0u, 0u};   // a wave with no share loads nothing
  }
}

template <class Elt, int MF, int W, int GB, class ASrc, bool kPre = false>
__device__ __forceinline__ void skinny_tile(const ASrc& asrc, const char* b, int64_t b_row_bytes,
                                            int cols_valid, int64_t K, float* red,
                                            int64_t rank_len = 0, const float* rank_scale = nullptr,
                                            int64_t rank_stride = 0,
                                            const u32x4 (*bpre)[2] = nullptr) {
  typedef typename Elt::T T;
  constexpr int CE = 16 / (int)sizeof(T);
  constexpr int KS = 4 * CE;            // elements per MFMA step
  constexpr int KG = 2 * KS;            // elements per group
  // GB: groups whose loads are all issued before their MFMAs (a wave's whole
  // share when it has at most GB groups)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15;
  const int colc = col < cols_valid ? col : cols_valid - 1;
  const char* brow = b + colc * b_row_bytes;
  const int64_t ng = K / KG;
  const int64_t g0 = wave * ng / W, g1 = (wave + 1) * ng / W;
  const int kq = (lane >> 4) * CE;

  f32x4 acc[MF], tot[MF];
#pragma unroll
  for (int f = 0; f < MF; ++f) {
    acc[f] = f32x4{0.f, 0.f, 0.f, 0.f};
    tot[f] = acc[f];
  }
  for (int64_t gb = g0; gb < g1; gb += GB) {
    u32x4 bv[GB][2], av[GB][2][MF];
#pragma unroll
    for (int q = 0; q < GB; ++q) {
      // past the share: reload the batch's first group (in bounds, not used)
      const int64_t g = gb + q < g1 ? gb + q : gb;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int64_t k = g * KG + s * KS + kq;
        if (kPre && gb == g0) bv[q][s] = bpre[q][s];   // loaded ahead (skinny_b_first)
        else bv[q][s] = *reinterpret_cast<const u32x4*>(brow + k * (int64_t)sizeof(T));
#pragma unroll
        for (int f = 0; f < MF; ++f) av[q][s][f] = asrc.chunk(f * 16 + (lane & 15), k);
      }
    }
#pragma unroll
    for (int q = 0; q < GB; ++q) {
      const int64_t g = gb + q;
      if (g < g1) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int f = 0; f < MF; ++f) mma16(acc[f], av[q][s][f], bv[q][s], Elt{});
        if (rank_len > 0 && ((g + 1) * KG % rank_len == 0 || g + 1 == g1)) {
          // end of a rank (or of this wave's share): scale and set aside
          const int64_t r = g * KG / rank_len;
          const float sc = col < cols_valid ? rank_scale[r * rank_stride + col] : 0.f;
#pragma unroll
          for (int f = 0; f < MF; ++f) {
            tot[f] += acc[f] * sc;
            acc[f] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
        }
      }
    }
  }
  mfma_drain();   // the last MFMAs sit in a conditional block
  if (rank_len == 0) {
#pragma unroll
    for (int f = 0; f < MF; ++f) tot[f] = acc[f];
  }

  // partial tiles of the W waves -> red[row][col], summed in wave order
  float* part = red + MF * 256;   // [W][MF][64 lanes][4]
#pragma unroll
  for (int f = 0; f < MF; ++f)
    *reinterpret_cast<f32x4*>(part + ((wave * MF + f) * 64 + lane) * 4) = tot[f];
  __syncthreads();
  for (int e = threadIdx.x; e < MF * 256; e += 64 * W) {
    const int row = e >> 4, c = e & 15;
    const int f = row >> 4, rr = row & 15;
    const int src_lane = (rr >> 2) * 16 + c, i = rr & 3;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) v += part[((w * MF + f) * 64 + src_lane) * 4 + i];
    red[e] = v;
  }
  __syncthreads();
}

template <int MF, int W>
struct SkLds {
  static constexpr int kFloats = MF * 256 + W * MF * 256;
};

// raw (T, r3 + E) fp32 = x [U_in | W_r^T] (the router rows past E are not computed)
template <class Elt, int MF, int W>
__global__ __launch_bounds__(64 * W) void k_sk_front(FwdArgs a, float* raw) {
  typedef typename Elt::T T;
  __shared__ float red[SkLds<MF, W>::kFloats];
  const int64_t n0 = (int64_t)blockIdx.x * 16, m0 = (int64_t)blockIdx.y * MF * 16;
  const int64_t N = a.r3 + a.E;
  const int rows_valid = (int)(a.T - m0 < MF * 16 ? a.T - m0 : MF * 16);
  const int cols_valid = (int)(N - n0 < 16 ? N - n0 : 16);
  const int64_t rb = a.d_in * (int64_t)sizeof(T);
  SkRows<Elt> as{reinterpret_cast<const char*>(a.x) + m0 * rb, rb, rows_valid};
  skinny_tile<Elt, MF, W, 2>(as, reinterpret_cast<const char*>(a.wfront) + n0 * rb, rb,
                             cols_valid, a.d_in, red);
  for (int e = threadIdx.x; e < MF * 256; e += 64 * W) {
    const int row = e >> 4, c = e & 15;
    if (row < rows_valid && c < cols_valid) raw[(m0 + row) * N + n0 + c] = red[e];
  }
}

// The per-token front epilogue, one wave per token: z = RMSNorm(raw z (* U_in
// scales)) * gain; logits; top-k (rank_key order: larger first, NaN above
// numbers, lower index on ties); softmax over the selected; c = sum_j w_j
// U_expert[e_j]. epi_load issues a token's loads (the lane's z columns lane + 64 q
// and logits lane + 64 q of every raw plane, added in plane order; gain and
// U_in scales); epi_finish computes and writes the results.
struct EpiLoad {
  float zr[4], lr[4], gv[4], zs[4];
};

__device__ __forceinline__ void epi_load(const FwdArgs& a, const float* raw, int nplanes,
                                         int64_t plane_stride, int64_t t, int lane, EpiLoad& L) {
  const int R3 = (int)a.r3, E = (int)a.E;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    L.zr[q] = 0.f; L.lr[q] = 0.f; L.gv[q] = 0.f; L.zs[q] = 1.f;
    const int j = lane + 64 * q;
    if (j < R3) {
      L.gv[q] = a.gain[j];
      if (a.zscale) L.zs[q] = a.zscale[j];
    }
  }
  const float* row = raw + t * (R3 + E);
  float zp[kMaxFrontPlanes][4], lp[kMaxFrontPlanes][4];
#pragma unroll
  for (int p = 0; p < kMaxFrontPlanes; ++p)
    if (p < nplanes)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j = lane + 64 * q;
        zp[p][q] = j < R3 ? row[p * plane_stride + j] : 0.f;
        lp[p][q] = j < E ? row[p * plane_stride + R3 + j] : 0.f;
      }
#pragma unroll
  for (int p = 0; p < kMaxFrontPlanes; ++p)
    if (p < nplanes)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        L.zr[q] += zp[p][q];
        L.lr[q] += lp[p][q];
      }
}

// Token t's results from its loads L (every lane of the wave calls it). ue:
// U_expert (E x r1 floats, LDS). routing: write idx, w, logits and c to a's
// outputs; z_global: write z (or, when a.cz is set, the Khatri-Rao row c (x) z)
// to a's buffers; z_row / c_row (LDS, or null): the token's z as stored (r3
// elements) and c (r1 floats).
template <class Elt>
__device__ __forceinline__ void epi_finish(const FwdArgs& a, int64_t t, int lane, const EpiLoad& L,
                                           const float* ue, bool routing, bool z_global,
                                           typename Elt::T* z_row, float* c_row) {
  typedef typename Elt::T T;
  const int R3 = (int)a.r3, E = (int)a.E, K = (int)a.k, R1 = (int)a.r1;
  float zv[4];
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int j = lane + 64 * q;
    float v = 0.f;
    if (j < R3) {
      v = L.zr[q];
      if (a.zscale) v *= L.zs[q];
    }
    zv[q] = v;
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float inv_rms = 1.f / sqrtf(ss / (float)R3 + a.eps);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int j = lane + 64 * q;
    zv[q] = round_as((zv[q] * inv_rms) * L.gv[q], Elt{});   // z as stored
    if (j < R3) {
      if (z_global && !a.cz) store_from_f32(reinterpret_cast<T*>(a.z) + t * R3 + j, zv[q]);
      if (z_row) store_from_f32(z_row + j, zv[q]);
    }
  }
  uint64_t key[4];   // rank_key order; 0 past E and once taken
  float sv[4];       // the ranked scores (router_mode 1: capped ones)
  const int mode = a.router_mode;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = lane + 64 * q;
    const float lv = e < E ? L.lr[q] : 0.f;
    if (routing && a.logits && e < E) a.logits[t * E + e] = lv;
    sv[q] = mode ? capped_score(lv, a.router_scale, a.router_temperature) : lv;
    key[q] = e < E ? rank_key(sv[q], e) : 0;
  }
  // K rounds of a wave max-key; lane kk keeps round kk's winner (K <= 16 < 64)
  float selv = 0.f;
  int si = 0;
#pragma unroll 1
  for (int kk = 0; kk < K; ++kk) {
    uint64_t best = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) best = key[q] > best ? key[q] : best;
    best = wave_max_key(best);
#pragma unroll
    for (int q = 0; q < 4; ++q) key[q] = key[q] == best ? 0 : key[q];
    if (kk == lane) {   // k <= E: best names a candidate, index < E
      selv = key_value(best);
      si = key_index(best);
    }
  }
  const float vmax = lane_value(selv, 0);
  const float ex = lane < K ? expf(selv - vmax) : 0.f;
  const float ssum = wave_sum(ex);
  float wk;
  if (mode) {
    // softmax over all E, then the selected renormalised (+1e-6)
    float sa = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) sa += lane + 64 * q < E ? expf(sv[q] - vmax) : 0.f;
    sa = wave_sum(sa);
    float ps = 0.f;
    for (int j = 0; j < K; ++j) ps += lane_value(ex, j) / sa;
    wk = (ex / sa) / (ps + 1e-6f);
  } else {
    wk = ex / ssum;
  }
  if (routing && lane < K) {
    a.idx[t * K + lane] = si;
    a.w[t * K + lane] = wk;
  }
  float cr = 0.f;
#pragma unroll 1
  for (int kk = 0; kk < K; ++kk) {
    const float w = lane_value(wk, kk);
    const int i = lane_value(si, kk);
    if (lane < R1) cr += w * ue[i * R1 + lane];
  }
  if (lane < R1) {
    if (routing) a.c[t * R1 + lane] = cr;
    if (c_row) c_row[lane] = cr;
  }
  if (z_global && a.cz) {   // folded plans: the Khatri-Rao row c (x) z in place of z
    T* dst = static_cast<T*>(a.cz) + t * R1 * R3;
#pragma unroll 1
    for (int r = 0; r < R1; ++r) {
      const float c_r = lane_value(cr, r);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j = lane + 64 * q;
        if (j < R3) store_from_f32(dst + r * R3 + j, c_r * zv[q]);
      }
    }
  }
}

// The front epilogue as a kernel, one wave per token. raw: nplanes (<=
// kMaxFrontPlanes) planes of T rows (plane_stride floats apart), added in plane
// order (the large-T front in K slices; the small-T front writes one).
template <class Elt>
__global__ __launch_bounds__(256) void k_front_epi(FwdArgs a, const float* raw, int nplanes,
                                                   int64_t plane_stride) {
  // U_expert (E x r1 floats: the launch's dynamic LDS) is staged while the rows load
  extern __shared__ float ue[];
  const int lane = threadIdx.x & 63;
  const int E = (int)a.E, R1 = (int)a.r1;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const bool live = t < a.T;   // whole waves
  EpiLoad L;
  if (live) epi_load(a, raw, nplanes, plane_stride, t, lane, L);
  for (int i = threadIdx.x; i < E * R1; i += 256) ue[i] = a.uexp[i];
  __syncthreads();
  if (!live) return;   // no barriers below
  epi_finish<Elt>(a, t, lane, L, ue, true, true, nullptr, nullptr);
}

// The Khatri-Rao A operand from z and c rows staged in LDS (SkKhatriRao's
// arithmetic: A[t, r r3 + s] = R(c[t, r] z[t, s])).
template <class Elt>
struct SkKhatriRaoLds {
  const typename Elt::T* z;   // (MF 16, r3)
  const float* c;             // (MF 16, r1)
  int r1, r3, rows_valid;
  __device__ __forceinline__ u32x4 chunk(int row, int64_t k) const {
    typedef typename Elt::T T;
    const int t = row < rows_valid ? row : rows_valid - 1;
    const int r = (int)(k / r3), s = (int)(k - (int64_t)r * r3);
    const u32x4 v = *reinterpret_cast<const u32x4*>(z + t * r3 + s);
    const float cc = c[t * r1 + r];
    u32x4 o;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_bf16x2(bf16_bits_to_f32(v[j] & 0xffffu) * cc, bf16_bits_to_f32(v[j] >> 16) * cc);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = __float_as_uint(__uint_as_float(v[j]) * cc);
    }
    return o;
  }
};

// Dynamic LDS bytes of k_sk_epi_gemm: z rows, c rows, U_expert.
inline size_t sk_epi_dyn_bytes(int mf, const FwdArgs& a) {
  const size_t es = a.dtype == 1 ? 2 : 4;   // TMOE_BF16: 2-byte elements
  return (size_t)mf * 16 * a.r3 * es + (size_t)mf * 16 * a.r1 * 4 + (size_t)a.E * a.r1 * 4;
}

// The front epilogue fused into the Khatri-Rao GEMM that follows it (small T, raw
// from k_sk_front in one plane): every work-group runs the epilogue of its MF 16
// tokens into LDS (the token loads are issued first, for every token of a wave),
// then its 16 columns of the GEMM with A = c (x) z from LDS. Work-groups of
// column block 0 write the routing outputs (idx, w, logits, c). kCore: mid = A
// core^T (as k_sk_core; fp8 rank scales), else out = A W^T + bias (as k_sk_out
// with KR: folded plans, the fused FFN epilogues).
template <class Elt, int MF, int W, bool kCore>
__global__ __launch_bounds__(64 * W) void k_sk_epi_gemm(FwdArgs a) {
  typedef typename Elt::T T;
  __shared__ float red[SkLds<MF, W>::kFloats];
  extern __shared__ u32x4 dynv[];   // 16-byte aligned: z rows are read as 16-byte chunks
  float* dyn = reinterpret_cast<float*>(dynv);
  const int R3 = (int)a.r3, R1 = (int)a.r1, E = (int)a.E;
  T* zl = reinterpret_cast<T*>(dyn);                       // (MF 16, r3)
  float* cl = reinterpret_cast<float*>(zl + MF * 16 * R3);   // (MF 16, r1)
  float* ue = cl + MF * 16 * R1;                             // (E, r1)
  const int64_t n0 = (int64_t)blockIdx.x * 16, m0 = (int64_t)blockIdx.y * MF * 16;
  const int rows_valid = (int)(a.T - m0 < MF * 16 ? a.T - m0 : MF * 16);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int TPW = (MF * 16 + W - 1) / W;   // tokens per wave
  // the GEMM's first weight chunks go out first: their latency overlaps the
  // epilogue's
  const int64_t K = (int64_t)R1 * R3;
  const int64_t rb = K * (int64_t)sizeof(T);
  const int64_t NB = kCore ? a.r2 : a.d_out;
  const int cols_valid = (int)(NB - n0 < 16 ? NB - n0 : 16);
  const char* bsrc = reinterpret_cast<const char*>(kCore ? a.coreT : a.uoutT) + n0 * rb;
  u32x4 bpre[1][2];
  skinny_b_first<Elt, W, 1>(bsrc, rb, cols_valid, K, bpre);
  EpiLoad L[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int row = wave + W * i;
    if (row < rows_valid) epi_load(a, a.raw, 1, 0, m0 + row, lane, L[i]);
  }
  for (int i = threadIdx.x; i < E * R1; i += 64 * W) ue[i] = a.uexp[i];
  __syncthreads();
  const bool routing = blockIdx.x == 0;
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int row = wave + W * i;
    if (row < rows_valid)
      epi_finish<Elt>(a, m0 + row, lane, L[i], ue, routing, false, zl + row * R3, cl + row * R1);
  }
  __syncthreads();
  SkKhatriRaoLds<Elt> as{zl, cl, R1, R3, rows_valid};
  if constexpr (kCore) {
    skinny_tile<Elt, MF, W, 1, SkKhatriRaoLds<Elt>, true>(
        as, bsrc, rb, cols_valid, K, red, a.core_scale_raw ? a.r3 : 0,
        a.core_scale_raw ? a.core_scale_raw + n0 : nullptr, a.r2, bpre);
    for (int e = threadIdx.x; e < MF * 256; e += 64 * W) {
      const int row = e >> 4, c = e & 15;
      if (row < rows_valid && c < cols_valid)
        store_from_f32(reinterpret_cast<T*>(a.mid) + (m0 + row) * a.r2 + n0 + c, red[e]);
    }
  } else {
    const int c = threadIdx.x & 15;
    const float bias = c < cols_valid ? a.bias[n0 + c] : 0.f;
    const float sc = a.out_scale && c < cols_valid ? a.out_scale[n0 + c] : 1.f;
    skinny_tile<Elt, MF, W, 1, SkKhatriRaoLds<Elt>, true>(as, bsrc, rb, cols_valid, K, red, 0,
                                                          nullptr, 0, bpre);
    for (int e = threadIdx.x; e < MF * 256; e += 64 * W) {
      const int row = e >> 4;
      if (row < rows_valid && c < cols_valid) {
        const int64_t oi = (m0 + row) * a.d_out + n0 + c;
        float y = red[e] * sc + bias;
        if (a.epi_mode != kEpiNone)
          y = epi_value<Elt>(a.epi_mode, round_as(y, Elt{}),
                             load_as_f32(static_cast<const T*>(a.epi_a) + oi),
                             a.epi_mode == kEpiResScale
                                 ? load_as_f32(static_cast<const T*>(a.epi_b) + n0 + c) : 0.f);
        store_from_f32(reinterpret_cast<T*>(a.out) + oi, y);
      }
    }
  }
}

// mid (T, r2) = (c (x) z) core^T; fp8 weights: rank r's partial sums scaled by
// core_scale_raw[r, q]
template <class Elt, int MF, int W>
__global__ __launch_bounds__(64 * W) void k_sk_core(FwdArgs a) {
  typedef typename Elt::T T;
  __shared__ float red[SkLds<MF, W>::kFloats];
  const int64_t n0 = (int64_t)blockIdx.x * 16, m0 = (int64_t)blockIdx.y * MF * 16;
  const int rows_valid = (int)(a.T - m0 < MF * 16 ? a.T - m0 : MF * 16);
  const int cols_valid = (int)(a.r2 - n0 < 16 ? a.r2 - n0 : 16);
  const int64_t K = a.r1 * a.r3;
  SkKhatriRao<Elt> as{reinterpret_cast<const char*>(a.z) + m0 * a.r3 * (int64_t)sizeof(T),
                      a.c + m0 * a.r1, (int)a.r1, (int)a.r3, rows_valid};
  const int64_t rb = K * (int64_t)sizeof(T);
  skinny_tile<Elt, MF, W, 1>(as, reinterpret_cast<const char*>(a.coreT) + n0 * rb, rb,
                             cols_valid, K, red, a.core_scale_raw ? a.r3 : 0,
                             a.core_scale_raw ? a.core_scale_raw + n0 : nullptr, a.r2);
  for (int e = threadIdx.x; e < MF * 256; e += 64 * W) {
    const int row = e >> 4, c = e & 15;
    if (row < rows_valid && c < cols_valid)
      store_from_f32(reinterpret_cast<T*>(a.mid) + (m0 + row) * a.r2 + n0 + c, red[e]);
  }
}

// out (T, d_out) = mid U_out (* U_out scales) + bias; with KR (folded plans) the A
// operand is c (x) z built in registers from z and c (as k_sk_core's), a.r2 = r1 * r3
// and a.uoutT = W^T
template <class Elt, int MF, int W, bool KR = false>
__global__ __launch_bounds__(64 * W) void k_sk_out(FwdArgs a) {
  typedef typename Elt::T T;
  __shared__ float red[SkLds<MF, W>::kFloats];
  const int64_t n0 = (int64_t)blockIdx.x * 16, m0 = (int64_t)blockIdx.y * MF * 16;
  const int rows_valid = (int)(a.T - m0 < MF * 16 ? a.T - m0 : MF * 16);
  const int cols_valid = (int)(a.d_out - n0 < 16 ? a.d_out - n0 : 16);
  const int64_t rb = a.r2 * (int64_t)sizeof(T);
  // this thread's epilogue column is threadIdx.x & 15: its constants load first
  const int c = threadIdx.x & 15;
  const float bias = c < cols_valid ? a.bias[n0 + c] : 0.f;
  const float sc = a.out_scale && c < cols_valid ? a.out_scale[n0 + c] : 1.f;
  if constexpr (KR) {
    SkKhatriRao<Elt> as{reinterpret_cast<const char*>(a.z) + m0 * a.r3 * (int64_t)sizeof(T),
                        a.c + m0 * a.r1, (int)a.r1, (int)a.r3, rows_valid};
    skinny_tile<Elt, MF, W, 1>(as, reinterpret_cast<const char*>(a.uoutT) + n0 * rb, rb,
                               cols_valid, a.r2, red);
  } else {
    SkRows<Elt> as{reinterpret_cast<const char*>(a.mid) + m0 * rb, rb, rows_valid};
    skinny_tile<Elt, MF, W, 1>(as, reinterpret_cast<const char*>(a.uoutT) + n0 * rb, rb,
                               cols_valid, a.r2, red);
  }
  for (int e = threadIdx.x; e < MF * 256; e += 64 * W) {
    const int row = e >> 4;
    if (row < rows_valid && c < cols_valid) {
      const int64_t oi = (m0 + row) * a.d_out + n0 + c;
      float y = red[e] * sc + bias;
      if (a.epi_mode != kEpiNone)   // the fused FFN epilogue on the rounded layer output
        y = epi_value<Elt>(a.epi_mode, round_as(y, Elt{}), load_as_f32(static_cast<const T*>(a.epi_a) + oi),
                           a.epi_mode == kEpiResScale
                               ? load_as_f32(static_cast<const T*>(a.epi_b) + n0 + c) : 0.f);
      store_from_f32(reinterpret_cast<T*>(a.out) + oi, y);
    }
  }
}

}  // namespace dev
}  // namespace tmoe
