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
    // 32-bit division (k < r1 r3 < 2^31): the 64-bit one is a long inlined routine
    const int r = (int)((uint32_t)k / (uint32_t)r3), s = (int)k - r * r3;
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

// raw (T, r3 + E) fp32 = x [U_in | W_r^T] (the router rows past E are not computed),
// rows raw_stride(r3, E) floats apart
template <class Elt, int MF, int W>
__global__ __launch_bounds__(64 * W) void k_sk_front(FwdArgs a, float* raw) {
  typedef typename Elt::T T;
  __shared__ float red[SkLds<MF, W>::kFloats];
  const int64_t n0 = (int64_t)blockIdx.x * 16, m0 = (int64_t)blockIdx.y * MF * 16;
  const int64_t N = a.r3 + a.E, RS = raw_stride(a.r3, a.E);
  const int rows_valid = (int)(a.T - m0 < MF * 16 ? a.T - m0 : MF * 16);
  const int cols_valid = (int)(N - n0 < 16 ? N - n0 : 16);
  const int64_t rb = a.d_in * (int64_t)sizeof(T);
  SkRows<Elt> as{reinterpret_cast<const char*>(a.x) + m0 * rb, rb, rows_valid};
  skinny_tile<Elt, MF, W, 2>(as, reinterpret_cast<const char*>(a.wfront) + n0 * rb, rb,
                             cols_valid, a.d_in, red);
  for (int e = threadIdx.x; e < MF * 256; e += 64 * W) {
    const int row = e >> 4, c = e & 15;
    if (row < rows_valid && c < cols_valid) raw[(m0 + row) * RS + n0 + c] = red[e];
  }
}

// The per-token front epilogue, one wave per token: z = RMSNorm(raw z (* U_in
// scales)) * gain; logits; top-k (rank_key order: larger first, NaN above
// numbers, lower index on ties); softmax over the selected; c = sum_j w_j
// U_expert[e_j]. Lane l holds the z columns G l .. G l + G - 1 (G = r3 / 64: one
// 4-, 8- or 16-byte load per raw plane) and the logits l + 64 q (q < LQ, E <= 64
// LQ). epi_load issues a token's loads (every raw plane, added in plane order;
// gain and U_in scales) with no branch between them, so that they are all in
// flight at once; epi_finish computes and writes the results.
struct EpiLoad {
  float zr[4], lr[4], gv[4], zs[4];   // z, gain, U_in scale: [q] = column G l + q
};

// G consecutive floats at p into v[0 .. G-1] (p aligned to 4 G bytes)
template <int G>
__device__ __forceinline__ void load_cols(const float* p, float (&v)[4]) {
  if constexpr (G == 4) {
    const float4 u = *reinterpret_cast<const float4*>(p);
    v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
  } else if constexpr (G == 2) {
    const float2 u = *reinterpret_cast<const float2*>(p);
    v[0] = u.x; v[1] = u.y;
  } else {
    v[0] = p[0];
  }
}

typedef uint32_t u32x2e __attribute__((ext_vector_type(2)));

// v[0 .. G-1] as G consecutive elements at p (aligned to G elements)
template <int G>
__device__ __forceinline__ void store_cols(uint16_t* p, const float (&v)[4]) {
  if constexpr (G == 4) {
    u32x2e u;
    u.x = pack_bf16x2(v[0], v[1]);
    u.y = pack_bf16x2(v[2], v[3]);
    *reinterpret_cast<u32x2e*>(p) = u;
  } else if constexpr (G == 2) {
    *reinterpret_cast<uint32_t*>(p) = pack_bf16x2(v[0], v[1]);
  } else {
    *p = f32_to_bf16_bits(v[0]);
  }
}
template <int G>
__device__ __forceinline__ void store_cols(float* p, const float (&v)[4]) {
  if constexpr (G == 4) *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  else if constexpr (G == 2) *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
  else p[0] = v[0];
}

// nplanes (1 .. KP) raw planes, plane_stride floats apart. KP planes are loaded:
// those past nplanes load the last plane again (in bounds) and are not added.
// Logit loads past E read logit E - 1 (in bounds) and are not added.
template <int G, int KP, int LQ>
__device__ __forceinline__ void epi_load(const FwdArgs& a, const float* raw, int nplanes,
                                         int64_t plane_stride, int64_t t, int lane, EpiLoad& L) {
  constexpr int R3 = 64 * G;
  const int E = (int)a.E;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    L.zr[q] = 0.f; L.lr[q] = 0.f; L.gv[q] = 0.f; L.zs[q] = 1.f;
  }
  load_cols<G>(a.gain + G * lane, L.gv);
  if (a.zscale) load_cols<G>(a.zscale + G * lane, L.zs);
  const float* row = raw + t * raw_stride(R3, E);
  float zp[KP][4], lp[KP][LQ];
#pragma unroll
  for (int p = 0; p < KP; ++p) {
    const float* pr = row + (p < nplanes ? p : nplanes - 1) * plane_stride;
    load_cols<G>(pr + G * lane, zp[p]);
#pragma unroll
    for (int q = 0; q < LQ; ++q) {
      const int e = lane + 64 * q;
      lp[p][q] = pr[R3 + (e < E ? e : E - 1)];
    }
  }
#pragma unroll
  for (int p = 0; p < KP; ++p) {
    const bool on = p < nplanes;
#pragma unroll
    for (int q = 0; q < G; ++q) L.zr[q] = on ? L.zr[q] + zp[p][q] : L.zr[q];
#pragma unroll
    for (int q = 0; q < LQ; ++q)
      L.lr[q] = on && lane + 64 * q < E ? L.lr[q] + lp[p][q] : L.lr[q];
  }
}

// Token t's results from its loads L (every lane of the wave calls it). ue:
// U_expert (E x r1 floats, LDS). routing: write idx, w, logits and c to a's
// outputs; z_global: write z (or, when a.cz is set, the Khatri-Rao row c (x) z)
// to a's buffers; z_row / c_row (LDS, or null): the token's z as stored (r3
// elements) and c (r1 floats).
template <class Elt, int G>
__device__ __forceinline__ void epi_finish(const FwdArgs& a, int64_t t, int lane, const EpiLoad& L,
                                           const float* ue, bool routing, bool z_global,
                                           typename Elt::T* z_row, float* c_row) {
  typedef typename Elt::T T;
  constexpr int R3 = 64 * G;
  const int E = (int)a.E, K = (int)a.k, R1 = (int)a.r1;
  float zv[4];
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float v = 0.f;
    if (q < G) {
      v = L.zr[q];
      if (a.zscale) v *= L.zs[q];
    }
    zv[q] = v;
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float inv_rms = 1.f / sqrtf(ss / (float)R3 + a.eps);
#pragma unroll
  for (int q = 0; q < 4; ++q) zv[q] = round_as((zv[q] * inv_rms) * L.gv[q], Elt{});   // z as stored
  if (z_global && !a.cz) store_cols<G>(reinterpret_cast<T*>(a.z) + t * R3 + G * lane, zv);
  if (z_row) store_cols<G>(z_row + G * lane, zv);
  uint64_t key[4];   // rank_key order; 0 past E and once taken
  float sv[4];       // the ranked scores (router_mode 1: capped ones)
  const int mode = a.router_mode;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = lane + 64 * q;
    const float lv = e < E ? L.lr[q] : 0.f;
    if (routing && a.logits && e < E) a.logits[t * E + e] = lv;
    sv[q] = lv;
  }
  if (mode) {   // a uniform branch (selected, the exp and divisions ran in mode 0 too)
#pragma unroll
    for (int q = 0; q < 4; ++q) sv[q] = capped_score(sv[q], a.router_scale, a.router_temperature);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) key[q] = lane + 64 * q < E ? rank_key(sv[q], lane + 64 * q) : 0;
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
    T* dst = static_cast<T*>(a.cz) + t * R1 * R3 + G * lane;
#pragma unroll 1
    for (int r = 0; r < R1; ++r) {
      const float c_r = lane_value(cr, r);
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = c_r * zv[q];
      store_cols<G>(dst + r * R3, v);
    }
  }
}

// The front epilogue as a kernel, one wave per token. raw: nplanes (<= KP)
// planes of T rows (plane_stride floats apart), added in plane order (the large-T
// front in K slices; the small-T front writes one). G = r3 / 64, E <= 64 LQ.
template <class Elt, int G, int KP, int LQ>
__global__ __launch_bounds__(256) void k_front_epi(FwdArgs a, const float* raw, int nplanes,
                                                   int64_t plane_stride) {
  // U_expert (E x r1 floats: the launch's dynamic LDS) is staged while the rows load
  extern __shared__ float ue[];
  const int lane = threadIdx.x & 63;
  const int E = (int)a.E, R1 = (int)a.r1;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const bool live = t < a.T;   // whole waves
  EpiLoad L;
  if (live) epi_load<G, KP, LQ>(a, raw, nplanes, plane_stride, t, lane, L);
  for (int i = threadIdx.x; i < E * R1; i += 256) ue[i] = a.uexp[i];
  __syncthreads();
  if (!live) return;   // no barriers below
  epi_finish<Elt, G>(a, t, lane, L, ue, true, true, nullptr, nullptr);
}

// The Khatri-Rao A operand from z and c rows staged in LDS (SkKhatriRao's
// arithmetic: A[t, r r3 + s] = R(c[t, r] z[t, s])).
// LDS row stride (elements) of the z rows a Khatri-Rao GEMM reads: r3 plus 16
// bytes. The GEMM's 16 lanes of a fragment read 16 rows at one K offset; with
// rows a multiple of 256 bytes apart (r3 = 128, 256 bf16) they all hit the same
// bank group (16-way conflicts), 16 bytes more puts them on 16 different ones.
template <class T>
__device__ __host__ constexpr int sk_z_stride(int r3) {
  return r3 + 16 / (int)sizeof(T);
}

template <class Elt>
struct SkKhatriRaoLds {
  const typename Elt::T* z;   // (MF 16, r3), rows sk_z_stride(r3) elements apart
  const float* c;             // (MF 16, r1)
  int r1, r3, rows_valid;
  __device__ __forceinline__ u32x4 chunk(int row, int64_t k) const {
    typedef typename Elt::T T;
    const int t = row < rows_valid ? row : rows_valid - 1;
    // 32-bit division (k < r1 r3 < 2^31): the 64-bit one is a long inlined routine
    const int r = (int)((uint32_t)k / (uint32_t)r3), s = (int)k - r * r3;
    const u32x4 v = *reinterpret_cast<const u32x4*>(z + t * sk_z_stride<T>(r3) + s);
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
  const size_t zs = es == 2 ? sk_z_stride<uint16_t>((int)a.r3) : sk_z_stride<float>((int)a.r3);
  return (size_t)mf * 16 * zs * es + (size_t)mf * 16 * a.r1 * 4 + (size_t)a.E * a.r1 * 4;
}

// k_sk_epi_gemm's epilogue of its MF 16 tokens (TPW per wave, W waves) into LDS
// (z rows zl, ZS elements apart; c rows cl), with U_expert staged into ue: every
// token's loads first, then the results. Ends with a barrier.
template <class Elt, int G, int TPW, int W>
__device__ __forceinline__ void sk_epi_tokens(const FwdArgs& a, int64_t m0, int rows_valid,
                                              bool routing, float* ue, typename Elt::T* zl,
                                              int ZS, float* cl) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int E = (int)a.E, R1 = (int)a.r1;
  EpiLoad L[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int row = wave + W * i;
    if (row < rows_valid) epi_load<G, 1, 4>(a, a.raw, 1, 0, m0 + row, lane, L[i]);
  }
  for (int i = threadIdx.x; i < E * R1; i += 64 * W) ue[i] = a.uexp[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int row = wave + W * i;
    if (row < rows_valid)
      epi_finish<Elt, G>(a, m0 + row, lane, L[i], ue, routing, false, zl + row * ZS,
                         cl + row * R1);
  }
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
  const int ZS = sk_z_stride<T>(R3);
  T* zl = reinterpret_cast<T*>(dyn);                       // (MF 16, r3), row stride ZS
  float* cl = reinterpret_cast<float*>(zl + MF * 16 * ZS);   // (MF 16, r1)
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
  const bool routing = blockIdx.x == 0;
  if (R3 == 256) sk_epi_tokens<Elt, 4, TPW, W>(a, m0, rows_valid, routing, ue, zl, ZS, cl);
  else if (R3 == 128) sk_epi_tokens<Elt, 2, TPW, W>(a, m0, rows_valid, routing, ue, zl, ZS, cl);
  else sk_epi_tokens<Elt, 1, TPW, W>(a, m0, rows_valid, routing, ue, zl, ZS, cl);
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

// ---- the small-T folded layer in one launch (decode) -----------------------
// Producers: kDecodeRowGroups work-groups per 16-column block of [z | logits]
// (NZ = r3 / 16 z blocks, then the router block of E <= 16 logit columns), each
// over up to 16 of the T tokens and all of d_in (skinny_tile): the z blocks publish
// their z columns (fp8 plans: the column scales), the router block's work-groups
// run the routing epilogue of their tokens (route_row16: one 16-lane row per
// token) and publish c. Consumers: the other work-groups own 16 columns of out
// each; they load their GEMM's first weight chunks, wait for the producers' flags
// (sync flags 0 .. (NZ + 1) kDecodeRowGroups - 1, several consumers per flag, so
// no flag is reset: the launcher does not use this kernel under graph capture),
// load z and c, form z = RMSNorm(z) * gain and its bf16 rounding into LDS, and run
// the GEMM of k_sk_epi_gemm against W^T with A = c (x) z from LDS. Producer data
// crosses the work-groups through the scratch at a.raw, 16 bytes per device-scope
// access: zr (T, r3) fp32, cs (T, r1) fp32. T <= MF * 16: one token block; the z a
// thread loads is held in registers (kDecodeGroups 4-column groups per thread).
constexpr int kDecodeRowGroups = 4;   // T <= 64: at most 16 tokens a producer
struct SkDecodeScratch {
  float *zr, *cs;
  __device__ __forceinline__ SkDecodeScratch(const FwdArgs& a) {
    zr = a.raw;
    cs = zr + a.T * a.r3;
  }
};
constexpr int kDecodeGroups = 4;
// Dynamic LDS bytes of k_sk_decode: a router work-group's U_expert and c rows; a
// consumer's z rows (bf16) and c rows.
inline size_t sk_decode_dyn_bytes(int mf, const FwdArgs& a) {
  const size_t rows = (size_t)mf * 16;
  const size_t router = ((size_t)a.E * a.r1 + 16 * a.r1) * 4;
  const size_t consumer = rows * sk_z_stride<uint16_t>((int)a.r3) * 2 + rows * a.r1 * 4;
  return router > consumer ? router : consumer;
}

// 16-byte device-scope accesses: buffer instructions with the sc1 cache policy
// (the path of store_coherent / load_coherent, four words at a time). n_floats
// bounds the descriptor: an offset past it reads 0 and writes nothing.
constexpr int kCPolSC1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const float* base,
                                                                int64_t n_floats) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0,
                                           (int)(n_floats * 4), 0x00020000);
}
__device__ __forceinline__ f32x4 load_coherent4(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCPolSC1));
}
__device__ __forceinline__ void store_coherent4(__amdgpu_buffer_rsrc_t r, int byte_off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, byte_off, 0, kCPolSC1);
}

// Sum over aligned groups of G in {16, 32, 64} lanes (every lane active), the
// result in every lane of the group: the 16-lane rows' DPP butterflies, then the
// rows' sums read into scalars (lanes 0, 16, 32, 48) and paired. VALU and scalar
// reads only, like wave_sum.
__device__ __forceinline__ float lane_group_sum(float v, int G) {
  group_sum<8>(v);
  dpp_add_step<0x140>(v);   // row_mirror: the two 8-lane halves of a row
  if (G == 16) return v;
  const int b = __float_as_int(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
  if (G == 32) return (threadIdx.x & 63) < 32 ? r0 + r1 : r2 + r3;
  return (r0 + r1) + (r2 + r3);
}

// The routing epilogue of token t on one 16-lane row of a wave (sl: the lane's
// index in the row; E <= 16, K <= E, r1 <= 32; every lane of the row calls it):
// epi_finish's routing with the row's DPP steps in place of the wave's (the same
// selection rounds, slot order and sums), c into c_row (LDS) and a's outputs.
__device__ __forceinline__ void route_row16(const FwdArgs& a, int64_t t, int sl, float lv,
                                            const float* ue, float* c_row) {
  const int E = (int)a.E, K = (int)a.k, R1 = (int)a.r1;
  const int mode = a.router_mode;
  if (a.logits && sl < E) a.logits[t * E + sl] = lv;
  float sv = lv;
  if (mode) sv = capped_score(lv, a.router_scale, a.router_temperature);   // uniform branch
  uint64_t key = sl < E ? rank_key(sv, sl) : 0;
  float selv = 0.f, vmax = 0.f;
  int si = 0;
#pragma unroll 1
  for (int kk = 0; kk < K; ++kk) {
    uint64_t best = key;
    group_max_key<8>(best);
    dpp_max_step<0x140>(best);   // row_mirror: the two 8-lane halves
    key = key == best ? 0 : key;
    if (kk == 0) vmax = key_value(best);
    if (kk == sl) {
      selv = key_value(best);
      si = key_index(best);
    }
  }
  const float ex = sl < K ? expf(selv - vmax) : 0.f;
  float ssum = ex;
  group_sum<8>(ssum);
  dpp_add_step<0x140>(ssum);
  float wk;
  if (mode) {
    float sa = sl < E ? expf(sv - vmax) : 0.f;
    group_sum<8>(sa);
    dpp_add_step<0x140>(sa);
    float ps = 0.f;
    for (int j = 0; j < K; ++j) ps += __shfl(ex, j, 16) / sa;
    wk = (ex / sa) / (ps + 1e-6f);
  } else {
    wk = ex / ssum;
  }
  if (sl < K) {
    a.idx[t * K + sl] = si;
    a.w[t * K + sl] = wk;
  }
  float c0 = 0.f, c1 = 0.f;
#pragma unroll 1
  for (int kk = 0; kk < K; ++kk) {
    const float w = __shfl(wk, kk, 16);
    const int i = __shfl(si, kk, 16);
    if (sl < R1) c0 += w * ue[i * R1 + sl];
    if (sl + 16 < R1) c1 += w * ue[i * R1 + sl + 16];
  }
  if (sl < R1) {
    a.c[t * R1 + sl] = c0;
    c_row[sl] = c0;
  }
  if (sl + 16 < R1) {
    a.c[t * R1 + sl + 16] = c1;
    c_row[sl + 16] = c1;
  }
}

template <int MF, int W>
__global__ __launch_bounds__(64 * W) void k_sk_decode(FwdArgs a) {
  static_assert(W == 16, "one 16-lane row per token of a 64-token block");
  typedef EltBF16 Elt;
  typedef typename Elt::T T;
  __shared__ float red[SkLds<MF, W>::kFloats];
  extern __shared__ u32x4 dynv[];
  float* dyn = reinterpret_cast<float*>(dynv);
  const int R3 = (int)a.r3, R1 = (int)a.r1, E = (int)a.E, NZ = R3 / 16;
  const int Tn = (int)a.T;
  const int bid = blockIdx.x;
  const SkDecodeScratch sc(a);
  const int NP = (NZ + 1) * kDecodeRowGroups;
  if (bid < NP) {
    // ---- producers: 16 columns of [z | logits] for up to 16 tokens ----
    const int blk = bid / kDecodeRowGroups, rg = bid - blk * kDecodeRowGroups;
    const int rpg = (Tn + kDecodeRowGroups - 1) / kDecodeRowGroups;
    const int r0 = rg * rpg, rows = Tn - r0 < rpg ? Tn - r0 : rpg;   // may be <= 0
    const int64_t rbx = a.d_in * (int64_t)sizeof(T);
    const int64_t n0 = (int64_t)blk * 16;
    const int cols_valid = blk < NZ ? 16 : E;
    // the router's U_expert, loaded under the GEMM (E r1 <= 512 floats)
    const float uev = blk == NZ && threadIdx.x < E * R1 ? a.uexp[threadIdx.x] : 0.f;
    if (rows > 0) {   // work-group-uniform
      SkRows<Elt> as{reinterpret_cast<const char*>(a.x) + r0 * rbx, rbx, rows};
      skinny_tile<Elt, 1, W, 2>(as, reinterpret_cast<const char*>(a.wfront) + n0 * rbx, rbx,
                                cols_valid, a.d_in, red);
      if (blk < NZ) {
        // z columns (scaled: fp8 plans), four to a store
        const __amdgpu_buffer_rsrc_t rz = coherent_rsrc(sc.zr, (int64_t)Tn * R3);
        for (int e = threadIdx.x; e < rows * 4; e += 64 * W) {
          const int row = e >> 2, g = e & 3;
          f32x4 v;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            v[j] = a.zscale ? red[row * 16 + g * 4 + j] * a.zscale[n0 + g * 4 + j]
                            : red[row * 16 + g * 4 + j];
          store_coherent4(rz, (int)(((int64_t)(r0 + row) * R3 + n0 + g * 4) * 4), v);
        }
      } else {
        // the routing epilogue of these tokens; c into LDS, then published
        float* ue = dyn;             // (E, r1)
        float* cl = ue + E * R1;     // (16, r1)
        if (threadIdx.x < E * R1) ue[threadIdx.x] = uev;
        __syncthreads();
        const int ln = threadIdx.x & 15, row = threadIdx.x >> 4;
        if (row < rows)   // row-uniform
          route_row16(a, r0 + row, ln, ln < E ? red[row * 16 + ln] : 0.f, ue, cl + row * R1);
        __syncthreads();
        for (int q = threadIdx.x; q < rows * R1; q += 64 * W)
          store_coherent(sc.cs + r0 * R1 + q, cl[q]);
      }
    }
    sync_publish(a.sync + sync_flag(bid), a.epoch);
    return;
  }
  // ---- consumers: 16 columns of out = (c (x) z) W^T + bias ----
  const int ZS = sk_z_stride<T>(R3);
  T* zl = reinterpret_cast<T*>(dyn);                          // (MF 16, r3), row stride ZS
  float* cl = reinterpret_cast<float*>(zl + MF * 16 * ZS);    // (MF 16, r1)
  const int64_t n0 = (int64_t)(bid - NP) * 16;
  const int64_t K = (int64_t)R1 * R3;
  const int64_t rb = K * (int64_t)sizeof(T);
  const int cols_valid = (int)(a.d_out - n0 < 16 ? a.d_out - n0 : 16);
  const char* bsrc = reinterpret_cast<const char*>(a.uoutT) + n0 * rb;
  // under the wait: the GEMM's first weight chunks, the column's bias and scale,
  // and the gain of the z groups g = thread + 64 W j (4 columns each) this thread
  // normalises
  u32x4 bpre[1][2];
  skinny_b_first<Elt, W, 1>(bsrc, rb, cols_valid, K, bpre);
  const int c = threadIdx.x & 15;
  const float bias = c < cols_valid ? a.bias[n0 + c] : 0.f;
  const float osc = a.out_scale && c < cols_valid ? a.out_scale[n0 + c] : 1.f;
  const int G = R3 / 4, NG = Tn * G;
  float gv[kDecodeGroups][4];
#pragma unroll
  for (int j = 0; j < kDecodeGroups; ++j) {
    const int g = threadIdx.x + 64 * W * j;
    const int col = (g - (g / G) * G) * 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) gv[j][q] = g < NG ? a.gain[col + q] : 0.f;
  }
  const bool ok = sync_await(a.sync + sync_flag(0), NP, a.epoch, a.sync,
                             reinterpret_cast<int*>(red), false, a.wait_polls, a.status);
  // every load first: the z groups and c
  const __amdgpu_buffer_rsrc_t rz = coherent_rsrc(sc.zr, (int64_t)Tn * R3);
  f32x4 zv[kDecodeGroups];
#pragma unroll
  for (int j = 0; j < kDecodeGroups; ++j) {
    const int g = threadIdx.x + 64 * W * j;
    zv[j] = load_coherent4(rz, g < NG ? g * 16 : Tn * R3 * 4);   // past the end: 0
  }
  for (int q = threadIdx.x; q < Tn * R1; q += 64 * W)
    cl[q] = ok ? load_coherent(sc.cs + q) : __builtin_nanf("");
  // each row's sum of squares: its G groups sit in G consecutive lanes of one wave
  // (G = r3 / 4 in {16, 32, 64}), added by the lanes' cross-lane sum
#pragma unroll
  for (int j = 0; j < kDecodeGroups; ++j) {
    const int g = threadIdx.x + 64 * W * j;
    if ((g & ~63) >= NG) break;   // wave-uniform: no group of this wave left
    const float ss = lane_group_sum(((zv[j][0] * zv[j][0] + zv[j][1] * zv[j][1]) +
                                     zv[j][2] * zv[j][2]) + zv[j][3] * zv[j][3], G);
    const float ir = 1.f / sqrtf(ss / (float)R3 + a.eps);
    if (g < NG) {
      // z as stored by epi_finish: R((z / rms) * gain)
      T* zrow = zl + (g / G) * ZS + (g - (g / G) * G) * 4;   // token g / G, columns 4 (g % G)
#pragma unroll
      for (int q = 0; q < 4; ++q) store_from_f32(zrow + q, (zv[j][q] * ir) * gv[j][q]);
    }
  }
  __syncthreads();
  SkKhatriRaoLds<Elt> as{zl, cl, R1, R3, Tn};
  skinny_tile<Elt, MF, W, 1, SkKhatriRaoLds<Elt>, true>(as, bsrc, rb, cols_valid, K, red, 0,
                                                        nullptr, 0, bpre);
  for (int e = threadIdx.x; e < MF * 256; e += 64 * W) {
    const int row = e >> 4;
    if (row < Tn && c < cols_valid) {
      const int64_t oi = (int64_t)row * a.d_out + n0 + c;
      float y = red[e] * osc + bias;
      if (a.epi_mode != kEpiNone)
        y = epi_value<Elt>(a.epi_mode, round_as(y, Elt{}),
                           load_as_f32(static_cast<const T*>(a.epi_a) + oi),
                           a.epi_mode == kEpiResScale
                               ? load_as_f32(static_cast<const T*>(a.epi_b) + n0 + c) : 0.f);
      store_from_f32(reinterpret_cast<T*>(a.out) + oi, y);
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
