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
template <class Elt, int MF, int W, int GB, class ASrc>
__device__ __forceinline__ void skinny_tile(const ASrc& asrc, const char* b, int64_t b_row_bytes,
                                            int cols_valid, int64_t K, float* red,
                                            int64_t rank_len = 0, const float* rank_scale = nullptr,
                                            int64_t rank_stride = 0) {
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
        bv[q][s] = *reinterpret_cast<const u32x4*>(brow + k * (int64_t)sizeof(T));
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

// One wave per token: z = RMSNorm(raw z (* U_in scales)) * gain; logits; top-k
// (rank_key order: larger first, NaN above numbers, lower index on ties);
// softmax over the selected; c = sum_j w_j U_expert[e_j].
// raw: nplanes (<= kMaxFrontPlanes) planes of T rows (plane_stride floats apart),
// added in plane order (the large-T front in K slices; the small-T front writes one).
template <class Elt>
__global__ __launch_bounds__(256) void k_front_epi(FwdArgs a, const float* raw, int nplanes,
                                                   int64_t plane_stride) {
  typedef typename Elt::T T;
  // U_expert (E x r1 floats: the launch's dynamic LDS) is staged while the rows load
  extern __shared__ float ue[];
  const int lane = threadIdx.x & 63;
  const int R3 = (int)a.r3, E = (int)a.E, K = (int)a.k, R1 = (int)a.r1;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const bool live = t < a.T;   // whole waves
  // this lane's raw values (z columns lane + 64 q, logits lane + 64 q) of every
  // plane, all loads issued before any is used and before the U_expert staging
  // barrier; then added in plane order
  float zr[4] = {0.f, 0.f, 0.f, 0.f}, lr[4] = {0.f, 0.f, 0.f, 0.f};
  float gv[4] = {0.f, 0.f, 0.f, 0.f}, zs[4] = {1.f, 1.f, 1.f, 1.f};
  if (live) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int j = lane + 64 * q;
      if (j < R3) {
        gv[q] = a.gain[j];
        if (a.zscale) zs[q] = a.zscale[j];
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
          zr[q] += zp[p][q];
          lr[q] += lp[p][q];
        }
  }
  for (int i = threadIdx.x; i < E * R1; i += 256) ue[i] = a.uexp[i];
  __syncthreads();
  if (!live) return;   // no barriers below
  float zv[4];
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int j = lane + 64 * q;
    float v = 0.f;
    if (j < R3) {
      v = zr[q];
      if (a.zscale) v *= zs[q];
    }
    zv[q] = v;
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float inv_rms = 1.f / sqrtf(ss / (float)R3 + a.eps);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int j = lane + 64 * q;
    zv[q] = round_as((zv[q] * inv_rms) * gv[q], Elt{});   // z as stored
    if (j < R3 && !a.cz) store_from_f32(reinterpret_cast<T*>(a.z) + t * R3 + j, zv[q]);
  }
  uint64_t key[4];   // rank_key order; 0 past E and once taken
  float sv[4];       // the ranked scores (router_mode 1: capped ones)
  const int mode = a.router_mode;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = lane + 64 * q;
    const float lv = e < E ? lr[q] : 0.f;
    if (a.logits && e < E) a.logits[t * E + e] = lv;
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
  if (lane < K) {
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
  if (lane < R1) a.c[t * R1 + lane] = cr;
  if (a.cz) {   // folded plans: the Khatri-Rao row c (x) z in place of z
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
