// The latent expert contraction of the reference's training module and its
// backward (sft_cot_bundle/scripts/model.py:160-174 forward, :240-289 backward,
// :196-219 dG): with x = x_shared (B, r3), G = G_experts (E, r3, r2), the
// selected experts idx (B, k) and their probabilities p (B, k),
//   out[b]    = sum_j p[b,j] x[b] G[idx[b,j]]                         (B, r2)
//   dx[b]     = sum_j p[b,j] dout[b] G[idx[b,j]]^T                    (B, r3)
//   dp[b,j]   = dout[b] . (x[b] G[idx[b,j]])                          (B, k)
//   dG[e]     = sum_{b,j: idx[b,j] = e} p[b,j] x[b]^T dout[b]          (E, r3, r2)
// With the dense routing weights w[b,e] = sum_j p[b,j] [idx[b,j] = e] these are
//   out = (w (x) x) G_flat            G_flat = G as (E r3, r2): k_core's Khatri-Rao GEMM
//   H   = dout G_flat^T  (B, E r3)    H[b, (e, s)] = (dout[b] G[e]^T)[s]: an out-projection GEMM
//   dx[b, s] = sum_e w[b,e] H[b,(e,s)],  dp[b,j] = sum_s x[b,s] H[b,(idx[b,j], s)]
//   dG_flat[(e,s), q] = sum_b w[b,e] x[b,s] dout[b,q]: a GEMM over the tokens whose
//                   A rows are products of two token-major rows (WeightedRowLoader)
// so every product runs on the MFMA GEMMs of the layer forward.
#pragma once

#include "tmoe_kernels.hpp"

namespace tmoe {
namespace dev {

// w (B, E) f32 = sum_j p[b, j] [idx[b, j] = e]; one thread per (b, e).
template <class P>
__global__ void k_latent_w(const int64_t* __restrict__ idx, const P* __restrict__ p, int64_t B,
                           int k, int E, float* __restrict__ w) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * E) return;
  const int64_t b = i / E;
  const int e = (int)(i - b * E);
  float v = 0.f;
  for (int j = 0; j < k; ++j)
    if (idx[b * k + j] == e) v += load_as_f32(p + b * k + j);
  w[i] = v;
}

// dst (cols, rows_pad) = src (rows, cols)^T with zeros in columns rows .. rows_pad - 1.
template <class T>
__global__ void k_transpose_pad(const T* __restrict__ src, T* __restrict__ dst, int64_t rows,
                                int64_t cols, int64_t rows_pad) {
  __shared__ T tile[32][33];
  const int64_t c0 = (int64_t)blockIdx.x * 32, r0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8 threads
  for (int y = ty; y < 32; y += 8) {
    const int64_t r = r0 + y, c = c0 + tx;
    tile[y][tx] = (r < rows && c < cols) ? src[r * cols + c] : T(0);
  }
  __syncthreads();
  for (int y = ty; y < 32; y += 8) {
    const int64_t c = c0 + y, r = r0 + tx;   // dst row c, column r
    if (c < cols && r < rows_pad) dst[c * rows_pad + r] = tile[tx][y];
  }
}

// A operand of the dG GEMM: row m = (e, s) of (E r3) rows, K = tokens:
// A[(e, s), b] = w[b, e] * x[b, s], from the token-major transposes xT (r3, Bp) and
// wT (E, Bp) f32, rounded to the element type once (as KhatriRaoLoader does).
template <class Elt>
struct WeightedRowLoader {
  typedef typename Elt::T T;
  static constexpr int CE = 16 / (int)sizeof(T);   // elements per 16-byte chunk
  struct Raw {
    u32x4 v;
    u32x4 w[CE / 4];
  };
  static constexpr int kVmem = 1 + CE / 4;   // x chunk + CE f32 weights
  const char* xT;         // (r3, Bp)
  const float* wT;        // (E, Bp)
  int64_t bp;             // Bp: row length of both, in elements
  int m0, r3, rows;       // first row of the tile; rows of A (E r3)
  __device__ __forceinline__ Raw fetch(int row, int ch, int kt) const {
    constexpr int kTileK = kTileKBytes / (int)sizeof(T);
    int m = m0 + row;
    m = m < rows ? m : rows - 1;
    const int e = m / r3, s = m - e * r3;
    const int64_t k = (int64_t)kt * kTileK + ch * CE;
    Raw o;
    o.v = *reinterpret_cast<const u32x4*>(xT + ((int64_t)s * bp + k) * (int64_t)sizeof(T));
#pragma unroll
    for (int i = 0; i < CE / 4; ++i)
      o.w[i] = *reinterpret_cast<const u32x4*>(wT + (int64_t)e * bp + k + 4 * i);
    return o;
  }
  __device__ __forceinline__ u32x4 finish(const Raw& raw) const {
    u32x4 o;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_bf16x2(bf16_bits_to_f32(raw.v[j] & 0xffffu) * __uint_as_float(raw.w[j / 2][(2 * j) % 4]),
                           bf16_bits_to_f32(raw.v[j] >> 16) * __uint_as_float(raw.w[j / 2][(2 * j) % 4 + 1]));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = __float_as_uint(__uint_as_float(raw.v[j]) * __uint_as_float(raw.w[0][j]));
    }
    return o;
  }
};

// dG partial plane `slice` (E r3, r2) f32 over the slice's K tiles (tokens):
// tile (tm, tn) of sum_b A[(e,s), b] doutT[q, b].
template <class Elt, int BM, int BN, int WM, int WN, int PFA>
__global__ __launch_bounds__(64 * WM * WN) void k_latent_dg(const void* __restrict__ xT,
                                                            const float* __restrict__ wT,
                                                            const void* __restrict__ doutT,
                                                            int64_t bp, int E, int r3, int r2,
                                                            int nslices, float* __restrict__ parts) {
  typedef typename Elt::T T;
  typedef Tile<BM, BN, 0, WM, WN, PFA, 1, 2, false, true, WM * WN / 2> TL;
  __shared__ u32x4 smem[cmax(TL::kLdsBytes, TileStage<TL, float>::kBytes) / 16];
  const int M = E * r3;
  const int ntn = (r2 + BN - 1) / BN;
  const int tm = (int)blockIdx.x / ntn, tn = (int)blockIdx.x - tm * ntn;
  const int sl = (int)blockIdx.y;
  const int nkt = (int)(bp * (int64_t)sizeof(T) / kTileKBytes);
  const int kt0 = sl * nkt / nslices, kt1 = (sl + 1) * nkt / nslices;
  constexpr int kTileK = kTileKBytes / (int)sizeof(T);
  WeightedRowLoader<Elt> al{reinterpret_cast<const char*>(xT) + (int64_t)kt0 * kTileKBytes,
                            wT + (int64_t)kt0 * kTileK, bp, tm * BM, r3, M};
  const int64_t row_bytes = bp * (int64_t)sizeof(T);
  RowLoader bl{reinterpret_cast<const char*>(doutT) + (int64_t)tn * BN * row_bytes +
                   (int64_t)kt0 * kTileKBytes,
               row_bytes, r2 - tn * BN};
  f32x16 acc[TL::FM][TL::FN];
  NoExtra nx;
  gemm_mainloop<TL, Elt>(acc, al, bl, kt1 - kt0, smem, nx);
  char* stage = reinterpret_cast<char*>(smem);
  float zero[TL::FN], one[TL::FN];
#pragma unroll
  for (int j = 0; j < TL::FN; ++j) {
    zero[j] = 0.f;
    one[j] = 1.f;
  }
  stage_tile<TL, float>(acc, stage, zero, one);
  __syncthreads();
  const int m0 = tm * BM, n0 = tn * BN;
  flush_tile<TL, float>(stage, parts + ((int64_t)sl * M + m0) * r2 + n0, r2,
                        M - m0 < BM ? M - m0 : BM, r2 - n0 < BN ? r2 - n0 : BN);
}

// dst (n) = sum over nslices planes of parts (plane stride n), in plane order.
template <class T>
__global__ void k_sum_planes(const float* __restrict__ parts, int nslices, int64_t n,
                             T* __restrict__ dst) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float v = parts[i];
    for (int p = 1; p < nslices; ++p) v += parts[p * n + i];
    store_from_f32(dst + i, v);
  }
}

// One wave per token b: dx[b, s] = sum_e w[b, e] H[b, (e, s)] and
// dp[b, j] = sum_s x[b, s] H[b, (idx[b, j], s)]. The token's H row (E r3 values) is
// read in 16-byte chunks, kRound of a lane's chunks issued at once: with CPR = r3 / CE
// chunks per expert (CE elements a chunk) and 64 a multiple of CPR (r3 in 64 .. 256),
// lane l always holds column chunk l % CPR, of experts (l + 64 i) / CPR. dx adds the
// lanes of one column chunk (a butterfly over strides CPR .. 32); dp takes each
// selected expert's chunks and adds over the wave.
template <class T, class P>
__global__ __launch_bounds__(256) void k_latent_dx_dp(const T* __restrict__ H,
                                                      const float* __restrict__ w,
                                                      const T* __restrict__ x,
                                                      const int64_t* __restrict__ idx, int64_t B,
                                                      int E, int k, int r3, T* __restrict__ dx,
                                                      P* __restrict__ dp) {
  constexpr int CE = 16 / (int)sizeof(T);
  constexpr int kRound = 8;
  const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= B) return;   // whole waves
  const int cpr = r3 / CE;
  const int nch = E * cpr;                    // chunks of the row
  const int sc = lane % cpr;                  // this lane's column chunk
  const u32x4* hb = reinterpret_cast<const u32x4*>(H + b * (int64_t)E * r3);
  const u32x4 xv = reinterpret_cast<const u32x4*>(x + b * r3)[sc];
  const T* xe = reinterpret_cast<const T*>(&xv);
  int64_t sel[kMaxTopK];
  float dpv[kMaxTopK];
  for (int j = 0; j < k; ++j) {
    sel[j] = idx[b * k + j];   // outside [0, E): selects nothing, dp = 0
    dpv[j] = 0.f;
  }
  float acc[CE];
#pragma unroll
  for (int c = 0; c < CE; ++c) acc[c] = 0.f;
  for (int base = 0; base < nch; base += 64 * kRound) {
    u32x4 hv[kRound];
#pragma unroll
    for (int i = 0; i < kRound; ++i)
      if (base + lane + 64 * i < nch) hv[i] = hb[base + lane + 64 * i];
#pragma unroll
    for (int i = 0; i < kRound; ++i) {
      const int ch = base + lane + 64 * i;
      if (ch < nch) {
        const int e = ch / cpr;
        const float we = w[b * E + e];
        const T* he = reinterpret_cast<const T*>(&hv[i]);
        float d = 0.f;
#pragma unroll
        for (int c = 0; c < CE; ++c) {
          const float hc = load_as_f32(he + c);
          acc[c] += we * hc;
          d += load_as_f32(xe + c) * hc;
        }
        for (int j = 0; j < k; ++j)
          if (sel[j] == e) dpv[j] += d;
      }
    }
  }
  for (int off = cpr; off < 64; off <<= 1)
#pragma unroll
    for (int c = 0; c < CE; ++c) acc[c] += __shfl_xor(acc[c], off);
  if (lane < cpr) {
    u32x4 o;
    T* oe = reinterpret_cast<T*>(&o);
#pragma unroll
    for (int c = 0; c < CE; ++c) store_from_f32(oe + c, acc[c]);
    reinterpret_cast<u32x4*>(dx + b * r3)[lane] = o;
  }
  for (int j = 0; j < k; ++j) {
    float v = dpv[j];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    if (lane == 0) store_from_f32(dp + b * k + j, v);
  }
}

}  // namespace dev
}  // namespace tmoe
