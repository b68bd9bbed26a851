// gfx950 kernels of the Tucker-MoE layer forward.
//
// The reference computes (pure_torch_mlx/model.py:68-102), per token row x:
//   s = x W_r^T ; (v, e) = topk(s, k) ; w = softmax(v)            model.py:75-77
//   z = RMSNorm(x U_in) * g                                        model.py:80-81, :25-27
//   mid = sum_j w_j * z (sum_r U_expert[e_j, r] core[r])           model.py:87-98
//   out = mid U_out + bias                                         model.py:101
// Here the middle line is regrouped as mid = sum_{r,s} c_r z_s core[r, s, :],
// with c = sum_j w_j U_expert[e_j] (a (T, r1) matrix): one GEMM with
// K = r1*r3 whose A operand c (x) z is formed while it is staged into LDS.
//
// Four kernels, each one MFMA GEMM over a 128-byte K tile held in LDS:
//   k_router  : logits = x W_r^T (fp32 accumulate), top-k, softmax, c
//   k_inproj  : z = RMSNorm(x U_in) * g, one work-group owns whole r3 rows
//   k_core    : mid = (c (x) z) core_flat
//   k_outproj : out = mid U_out + bias
//
// Operand layout: every GEMM here is "NT": A is (M, K) and B^T is (N, K), both
// K-contiguous, so one lane of an MFMA fragment reads 16 contiguous bytes. The
// weights are re-laid to B^T once, at pack time.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "tmoe_internal.h"

namespace tmoe {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kDtypeBF16 = 1;   // TMOE_BF16

// ---- element types -------------------------------------------------------
struct EltBF16 {
  typedef uint16_t T;   // bf16 bits
};
struct EltF32 {
  typedef float T;
};

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);   // round to nearest even
}

__device__ __forceinline__ float load_as_f32(const uint16_t* p) { return bf16_bits_to_f32(*p); }
__device__ __forceinline__ float load_as_f32(const float* p) { return *p; }
__device__ __forceinline__ void store_from_f32(uint16_t* p, float v) { *p = f32_to_bf16_bits(v); }
__device__ __forceinline__ void store_from_f32(float* p, float v) { *p = v; }

// One 16x16 output block += A(16 x Kc) * B(Kc x 16) for one 16-byte chunk per lane.
// bf16: one v_mfma_f32_16x16x32_bf16 (Kc = 32).
// f32 : four v_mfma_f32_16x16x4_f32, chunk element j feeding MFMA j (Kc = 16).
// Lane l supplies row/column (l & 15) and the K-slice (l >> 4) of the chunk; A
// and B use the same slice mapping, so any consistent K order is exact. The
// result block holds rows 4*(l >> 4) + i, column (l & 15), i = 0..3.
__device__ __forceinline__ void mma(f32x4& acc, u32x4 a, u32x4 b, EltBF16) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x4& acc, u32x4 a, u32x4 b, EltF32) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[j]), __uint_as_float(b[j]), acc,
                                               0, 0, 0);
}

// ---- operand tile loaders ------------------------------------------------
// Both return the 16-byte chunk `ch` (0..7) of tile row `row` for K tile `kt`.
// Rows past the operand's end are clamped to its last row: their products only
// reach output rows/columns that are never stored.

struct RowLoader {          // plain row-major, K-contiguous operand
  const char* base;         // first row of this work-group's tile
  int64_t row_bytes;
  int rows_valid;           // >= 1
  __device__ __forceinline__ u32x4 operator()(int row, int ch, int kt) const {
    const int r = row < rows_valid ? row : rows_valid - 1;
    return *reinterpret_cast<const u32x4*>(base + (int64_t)r * row_bytes + kt * kTileKBytes +
                                           ch * 16);
  }
};

// A operand of the core GEMM: A[t, r*r3 + s] = c[t, r] * z[t, s], rounded to the
// operand type. A K tile never straddles two r blocks (r3 is a multiple of the
// tile's element count).
template <class Elt>
struct KhatriRaoLoader {
  const char* z;            // first row of the tile, (., r3)
  const float* c;           // first row of the tile, (., r1)
  int r1, r3;
  int rows_valid;
  __device__ __forceinline__ u32x4 operator()(int row, int ch, int kt) const {
    constexpr int kTileK = kTileKBytes / (int)sizeof(typename Elt::T);
    const int r = row < rows_valid ? row : rows_valid - 1;
    const int k0 = kt * kTileK;
    const int rr = k0 / r3;
    const int s0 = k0 - rr * r3;
    const u32x4 v = *reinterpret_cast<const u32x4*>(
        z + ((int64_t)r * r3 + s0) * (int64_t)sizeof(typename Elt::T) + ch * 16);
    const float cc = c[(int64_t)r * r1 + rr];
    u32x4 o;
    if constexpr (sizeof(typename Elt::T) == 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = bf16_bits_to_f32(v[j] & 0xffffu) * cc;
        const float hi = bf16_bits_to_f32(v[j] >> 16) * cc;
        o[j] = (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = __float_as_uint(__uint_as_float(v[j]) * cc);
    }
    return o;
  }
};

// ---- the shared GEMM main loop -------------------------------------------
// C tile (BM x BN) of A (M x K) * B^T (N x K)^T, fp32 accumulate, 64*WM*WN threads.
// Waves form a WM x WN grid; wave (wm, wn) owns rows wm*BM/WM.. and columns
// wn*BN/WN.. of the tile as FM x FN MFMA blocks.
//
// LDS holds two stages of [BM + BN rows][8 chunks of 16 B]; chunk ch of row r
// sits at slot ch ^ (r & 7), so the 16 rows one fragment read touches spread over
// all banks. Global loads for tile kt+1 are in flight while tile kt is consumed.
template <int BM, int BN, int WM, int WN>
struct Tile {
  static constexpr int kThreads = 64 * WM * WN;
  static constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
  static constexpr int FM = kWaveM / 16, FN = kWaveN / 16;
  static constexpr int kChunks = kTileKBytes / 16;   // 8 per row
  // chunks each thread moves per K tile (the last round may be partial)
  static constexpr int kAPerThread = (BM * kChunks + kThreads - 1) / kThreads;
  static constexpr int kBPerThread = (BN * kChunks + kThreads - 1) / kThreads;
  static constexpr int kStage = (BM + BN) * kChunks;  // u32x4 slots per stage
  static constexpr int kLdsBytes = 2 * kStage * 16;
  static_assert(BM % (16 * WM) == 0 && BN % (16 * WN) == 0, "tile/wave mismatch");
};

template <int BM, int BN, int WM, int WN, class Elt, class ALoad, class BLoad>
__device__ __forceinline__ void gemm_mainloop(f32x4 (&acc)[BM / WM / 16][BN / WN / 16],
                                              const ALoad& aload, const BLoad& bload, int nkt,
                                              u32x4* smem) {
  typedef Tile<BM, BN, WM, WN> TL;
  constexpr int FM = TL::FM, FN = TL::FN, CH = TL::kChunks;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 ra[TL::kAPerThread], rb[TL::kBPerThread];
  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < TL::kAPerThread; ++i) {
      const int q = tid + i * TL::kThreads;
      if (q < BM * CH) ra[i] = aload(q / CH, q % CH, kt);
    }
#pragma unroll
    for (int i = 0; i < TL::kBPerThread; ++i) {
      const int q = tid + i * TL::kThreads;
      if (q < BN * CH) rb[i] = bload(q / CH, q % CH, kt);
    }
  };
  auto sstore = [&](int buf) {
    u32x4* s = smem + buf * TL::kStage;
#pragma unroll
    for (int i = 0; i < TL::kAPerThread; ++i) {
      const int q = tid + i * TL::kThreads;
      const int row = q / CH, ch = q % CH;
      if (q < BM * CH) s[row * CH + (ch ^ (row & 7))] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < TL::kBPerThread; ++i) {
      const int q = tid + i * TL::kThreads;
      const int row = BM + q / CH, ch = q % CH;
      if (q < BN * CH) s[row * CH + (ch ^ (row & 7))] = rb[i];
    }
  };

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nkt; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nkt) gload(kt + 1);
    const u32x4* s = smem + buf * TL::kStage;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int ch = kk * 4 + (lane >> 4);
      u32x4 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm * TL::kWaveM + i * 16 + (lane & 15);
        af[i] = s[row * CH + (ch ^ (row & 7))];
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int row = BM + wn * TL::kWaveN + j * 16 + (lane & 15);
        bfr[j] = s[row * CH + (ch ^ (row & 7))];
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) mma(acc[i][j], af[i], bfr[j], Elt{});
    }
    if (kt + 1 < nkt) sstore(buf ^ 1);
    __syncthreads();
  }
}

// Top-k order: larger logit first, NaN above every number (as torch.topk
// orders NaN), equal values by lower expert index. Index 0x7fffffff marks "no
// candidate" and ranks after every real (value, index) pair.
__device__ __forceinline__ bool ranks_before(float v1, int i1, float v2, int i2) {
  if (i2 == 0x7fffffff) return i1 != 0x7fffffff;
  if (i1 == 0x7fffffff) return false;
  const bool n1 = v1 != v1, n2 = v2 != v2;
  if (n1 || n2) return n1 && (!n2 || i1 < i2);
  return v1 > v2 || (v1 == v2 && i1 < i2);
}

// ---- K1: router logits, top-k, softmax, expert coefficients ---------------
// model.py:75-77 (+ the U_expert gather of :93 folded into c). One work-group:
// 64 tokens x E_pad = 16*FN experts; wave w owns tokens 16w..16w+15.
// Top-k: k rounds of a wave-wide arg-max over the row; larger logit first, equal
// logits resolve to the lower expert index.
template <class Elt, int FN>
__global__ __launch_bounds__(256) void k_router(FwdArgs a) {
  typedef typename Elt::T T;
  constexpr int BM = kRouterBM, BN = 16 * FN, WM = 4, WN = 1;
  typedef Tile<BM, BN, WM, WN> TL;
  __shared__ u32x4 smem[TL::kLdsBytes / 16];

  const int64_t m0 = (int64_t)blockIdx.x * BM;
  const int rows_valid = (int)(a.T - m0 < BM ? a.T - m0 : BM);
  const int64_t row_bytes = a.d_in * (int64_t)sizeof(T);
  RowLoader al{reinterpret_cast<const char*>(a.x) + m0 * row_bytes, row_bytes, rows_valid};
  RowLoader bl{reinterpret_cast<const char*>(a.wr), row_bytes, (int)a.E_pad};
  f32x4 acc[TL::FM][TL::FN];
  gemm_mainloop<BM, BN, WM, WN, Elt>(acc, al, bl, (int)(row_bytes / kTileKBytes), smem);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int LD = BN + 1;
  float* lg = reinterpret_cast<float*>(smem);   // [BM][LD]; the main loop ended on a barrier
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      lg[(wave * 16 + 4 * (lane >> 4) + i) * LD + j * 16 + (lane & 15)] = acc[0][j][i];
  __syncthreads();

  constexpr int PL = (BN + 63) / 64;   // logits per lane
  const int E = (int)a.E, K = (int)a.k, R1 = (int)a.r1;
  for (int rr = 0; rr < 16; ++rr) {
    const int row = wave * 16 + rr;
    if (row >= rows_valid) break;      // uniform across the wave
    const int64_t g = m0 + row;
    float v[PL];
    unsigned taken = 0;
#pragma unroll
    for (int p = 0; p < PL; ++p) {
      const int col = lane + 64 * p;
      v[p] = col < BN ? lg[row * LD + col] : 0.f;
      if (a.logits && col < E) a.logits[g * E + col] = v[p];
    }
    float sel_v[kMaxTopK];
    int sel_i[kMaxTopK];
#pragma unroll
    for (int kk = 0; kk < kMaxTopK; ++kk) {
      sel_v[kk] = 0.f;
      sel_i[kk] = 0;
      if (kk < K) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;   // "no candidate": loses to every real one
#pragma unroll
        for (int p = 0; p < PL; ++p) {
          const int col = lane + 64 * p;
          const bool ok = col < E && !((taken >> p) & 1u);
          if (ok && ranks_before(v[p], col, bv, bi)) {
            bv = v[p];
            bi = col;
          }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
          const float ov = __shfl_xor(bv, off);
          const int oi = __shfl_xor(bi, off);
          if (ranks_before(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
          }
        }
        // k <= E, so a candidate always remains and bi < E here.
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        sel_v[kk] = bv;
        sel_i[kk] = bi;
      }
    }
    // softmax over the selected logits (sel_v[0] is the largest)
    float e[kMaxTopK];
    float ssum = 0.f;
#pragma unroll
    for (int kk = 0; kk < kMaxTopK; ++kk) {
      e[kk] = 0.f;
      if (kk < K) {
        e[kk] = expf(sel_v[kk] - sel_v[0]);
        ssum += e[kk];
      }
    }
#pragma unroll
    for (int kk = 0; kk < kMaxTopK; ++kk) {
      if (kk < K && lane == kk) {
        a.idx[g * K + kk] = sel_i[kk];
        a.w[g * K + kk] = e[kk] / ssum;
      }
    }
    // c[r] = sum_j w_j * U_expert[e_j, r]
    for (int r = lane; r < R1; r += 64) {
      float cr = 0.f;
#pragma unroll
      for (int kk = 0; kk < kMaxTopK; ++kk)
        if (kk < K) cr += (e[kk] / ssum) * a.uexp[(int64_t)sel_i[kk] * R1 + r];
      a.c[g * R1 + r] = cr;
    }
  }
}

// ---- K2: z = RMSNorm(x U_in) * g  (model.py:80-81, RMSNorm :25-27) ---------
// One work-group: 64 tokens x all R3 columns; the four waves split the columns.
// rms = sqrt(mean(z^2) + eps); z / rms * g, as the reference orders it.
template <class Elt, int R3>
__global__ __launch_bounds__(256) void k_inproj(FwdArgs a) {
  typedef typename Elt::T T;
  constexpr int BM = kInBM, BN = R3, WM = 1, WN = 4;
  typedef Tile<BM, BN, WM, WN> TL;
  __shared__ u32x4 smem[TL::kLdsBytes / 16];

  const int64_t m0 = (int64_t)blockIdx.x * BM;
  const int rows_valid = (int)(a.T - m0 < BM ? a.T - m0 : BM);
  const int64_t row_bytes = a.d_in * (int64_t)sizeof(T);
  RowLoader al{reinterpret_cast<const char*>(a.x) + m0 * row_bytes, row_bytes, rows_valid};
  RowLoader bl{reinterpret_cast<const char*>(a.uinT), row_bytes, R3};
  f32x4 acc[TL::FM][TL::FN];
  gemm_mainloop<BM, BN, WM, WN, Elt>(acc, al, bl, (int)(row_bytes / kTileKBytes), smem);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float* red = reinterpret_cast<float*>(smem);   // [WN][BM]
  float ss[TL::FM][4];
#pragma unroll
  for (int i = 0; i < TL::FM; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < TL::FN; ++j) s += acc[i][j][q] * acc[i][j][q];
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) s += __shfl_xor(s, off);
      ss[i][q] = s;
    }
  if ((lane & 15) == 0) {
#pragma unroll
    for (int i = 0; i < TL::FM; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) red[wave * BM + i * 16 + 4 * (lane >> 4) + q] = ss[i][q];
  }
  __syncthreads();
  T* z = reinterpret_cast<T*>(a.z);
#pragma unroll
  for (int i = 0; i < TL::FM; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = i * 16 + 4 * (lane >> 4) + q;
      const float tot = red[row] + red[BM + row] + red[2 * BM + row] + red[3 * BM + row];
      const float rms = sqrtf(tot / (float)R3 + a.eps);
      if (row < rows_valid) {
#pragma unroll
        for (int j = 0; j < TL::FN; ++j) {
          const int col = wave * TL::kWaveN + j * 16 + (lane & 15);
          store_from_f32(&z[(m0 + row) * R3 + col], (acc[i][j][q] / rms) * a.gain[col]);
        }
      }
    }
}

// ---- K3: mid = (c (x) z) core_flat  (model.py:87-98) ----------------------
template <class Elt, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void k_core(FwdArgs a) {
  typedef typename Elt::T T;
  typedef Tile<BM, BN, WM, WN> TL;
  __shared__ u32x4 smem[TL::kLdsBytes / 16];

  const int64_t m0 = (int64_t)blockIdx.x * BM;
  const int64_t n0 = (int64_t)blockIdx.y * BN;
  const int rows_valid = (int)(a.T - m0 < BM ? a.T - m0 : BM);
  const int64_t K = a.r1 * a.r3;
  const int64_t b_row_bytes = K * (int64_t)sizeof(T);
  KhatriRaoLoader<Elt> al{reinterpret_cast<const char*>(a.z) + m0 * a.r3 * (int64_t)sizeof(T),
                          a.c + m0 * a.r1, (int)a.r1, (int)a.r3, rows_valid};
  RowLoader bl{reinterpret_cast<const char*>(a.coreT) + n0 * b_row_bytes, b_row_bytes,
               (int)(a.r2 - n0)};
  f32x4 acc[TL::FM][TL::FN];
  gemm_mainloop<BM, BN, WM, WN, Elt>(acc, al, bl, (int)(b_row_bytes / kTileKBytes), smem);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  T* mid = reinterpret_cast<T*>(a.mid);
#pragma unroll
  for (int i = 0; i < TL::FM; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = wm * TL::kWaveM + i * 16 + 4 * (lane >> 4) + q;
      if (row < rows_valid) {
#pragma unroll
        for (int j = 0; j < TL::FN; ++j) {
          const int64_t col = n0 + wn * TL::kWaveN + j * 16 + (lane & 15);
          if (col < a.r2) store_from_f32(&mid[(m0 + row) * a.r2 + col], acc[i][j][q]);
        }
      }
    }
}

// ---- K4: out = mid U_out + bias  (model.py:101) --------------------------
template <class Elt, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void k_outproj(FwdArgs a) {
  typedef typename Elt::T T;
  typedef Tile<BM, BN, WM, WN> TL;
  __shared__ u32x4 smem[TL::kLdsBytes / 16];

  const int64_t m0 = (int64_t)blockIdx.x * BM;
  const int64_t n0 = (int64_t)blockIdx.y * BN;
  const int rows_valid = (int)(a.T - m0 < BM ? a.T - m0 : BM);
  const int64_t row_bytes = a.r2 * (int64_t)sizeof(T);
  RowLoader al{reinterpret_cast<const char*>(a.mid) + m0 * row_bytes, row_bytes, rows_valid};
  RowLoader bl{reinterpret_cast<const char*>(a.uoutT) + n0 * row_bytes, row_bytes,
               (int)(a.d_out - n0)};
  f32x4 acc[TL::FM][TL::FN];
  gemm_mainloop<BM, BN, WM, WN, Elt>(acc, al, bl, (int)(row_bytes / kTileKBytes), smem);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  T* out = reinterpret_cast<T*>(a.out);
#pragma unroll
  for (int j = 0; j < TL::FN; ++j) {
    const int64_t col = n0 + wn * TL::kWaveN + j * 16 + (lane & 15);
    const float b = col < a.d_out ? a.bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < TL::FM; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = wm * TL::kWaveM + i * 16 + 4 * (lane >> 4) + q;
        if (row < rows_valid && col < a.d_out)
          store_from_f32(&out[(m0 + row) * a.d_out + col], acc[i][j][q] + b);
      }
  }
}

// ---- packing kernels -----------------------------------------------------
template <class T>
__global__ void k_transpose(const T* __restrict__ src, T* __restrict__ dst, int64_t rows,
                            int64_t cols) {
  __shared__ T tile[32][33];
  const int64_t c0 = (int64_t)blockIdx.x * 32, r0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8 threads
  for (int y = ty; y < 32; y += 8) {
    const int64_t r = r0 + y, c = c0 + tx;
    if (r < rows && c < cols) tile[y][tx] = src[r * cols + c];
  }
  __syncthreads();
  for (int y = ty; y < 32; y += 8) {
    const int64_t c = c0 + y, r = r0 + tx;   // dst row c, column r
    if (r < rows && c < cols) dst[c * rows + r] = tile[tx][y];
  }
}

template <class T>
__global__ void k_copy_pad(const T* __restrict__ src, T* __restrict__ dst, int64_t n,
                           int64_t n_pad) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_pad;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = i < n ? src[i] : T(0);
}

template <class T>
__global__ void k_to_f32(const T* __restrict__ src, float* __restrict__ dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = load_as_f32(src + i);
}

inline unsigned cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

template <class Elt>
hipError_t launch_router_t(const FwdArgs& a, hipStream_t st) {
  const dim3 grid(cdiv(a.T, kRouterBM)), block(256);
  switch (a.E_pad / 16) {
    case 1: hipLaunchKernelGGL((k_router<Elt, 1>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((k_router<Elt, 2>), grid, block, 0, st, a); break;
    case 4: hipLaunchKernelGGL((k_router<Elt, 4>), grid, block, 0, st, a); break;
    case 8: hipLaunchKernelGGL((k_router<Elt, 8>), grid, block, 0, st, a); break;
    case 16: hipLaunchKernelGGL((k_router<Elt, 16>), grid, block, 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <class Elt>
hipError_t launch_inproj_t(const FwdArgs& a, hipStream_t st) {
  const dim3 grid(cdiv(a.T, kInBM)), block(256);
  switch (a.r3) {
    case 64: hipLaunchKernelGGL((k_inproj<Elt, 64>), grid, block, 0, st, a); break;
    case 128: hipLaunchKernelGGL((k_inproj<Elt, 128>), grid, block, 0, st, a); break;
    case 256: hipLaunchKernelGGL((k_inproj<Elt, 256>), grid, block, 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_router(const FwdArgs& a, hipStream_t st) {
  return a.dtype == kDtypeBF16 ? launch_router_t<EltBF16>(a, st) : launch_router_t<EltF32>(a, st);
}

hipError_t launch_inproj(const FwdArgs& a, hipStream_t st) {
  return a.dtype == kDtypeBF16 ? launch_inproj_t<EltBF16>(a, st) : launch_inproj_t<EltF32>(a, st);
}

hipError_t launch_core(const FwdArgs& a, hipStream_t st) {
  const dim3 grid(cdiv(a.T, kCoreBM), cdiv(a.r2, kCoreBN)), block(256);
  if (a.dtype == kDtypeBF16)
    hipLaunchKernelGGL((k_core<EltBF16, kCoreBM, kCoreBN, 2, 2>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((k_core<EltF32, kCoreBM, kCoreBN, 2, 2>), grid, block, 0, st, a);
  return hipGetLastError();
}

hipError_t launch_outproj(const FwdArgs& a, hipStream_t st) {
  const dim3 grid(cdiv(a.T, kOutBM), cdiv(a.d_out, kOutBN)), block(256);
  if (a.dtype == kDtypeBF16)
    hipLaunchKernelGGL((k_outproj<EltBF16, kOutBM, kOutBN, 2, 2>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((k_outproj<EltF32, kOutBM, kOutBN, 2, 2>), grid, block, 0, st, a);
  return hipGetLastError();
}

hipError_t launch_transpose(const void* src, void* dst, int64_t rows, int64_t cols, int es,
                            hipStream_t st) {
  if (rows == 0 || cols == 0) return hipSuccess;
  const dim3 grid(cdiv(cols, 32), cdiv(rows, 32)), block(256);
  if (es == 2)
    hipLaunchKernelGGL(k_transpose<uint16_t>, grid, block, 0, st,
                       static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), rows, cols);
  else
    hipLaunchKernelGGL(k_transpose<float>, grid, block, 0, st, static_cast<const float*>(src),
                       static_cast<float*>(dst), rows, cols);
  return hipGetLastError();
}

hipError_t launch_copy_pad(const void* src, void* dst, int64_t n, int64_t n_pad, int es,
                           hipStream_t st) {
  if (n_pad == 0) return hipSuccess;
  const dim3 grid(cdiv(n_pad, 256) < 4096 ? cdiv(n_pad, 256) : 4096), block(256);
  if (es == 2)
    hipLaunchKernelGGL(k_copy_pad<uint16_t>, grid, block, 0, st,
                       static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), n, n_pad);
  else
    hipLaunchKernelGGL(k_copy_pad<float>, grid, block, 0, st, static_cast<const float*>(src),
                       static_cast<float*>(dst), n, n_pad);
  return hipGetLastError();
}

hipError_t launch_to_f32(const void* src, float* dst, int64_t n, int dtype, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const dim3 grid(cdiv(n, 256) < 4096 ? cdiv(n, 256) : 4096), block(256);
  if (dtype == kDtypeBF16)
    hipLaunchKernelGGL(k_to_f32<uint16_t>, grid, block, 0, st, static_cast<const uint16_t*>(src),
                       dst, n);
  else
    hipLaunchKernelGGL(k_to_f32<float>, grid, block, 0, st, static_cast<const float*>(src), dst,
                       n);
  return hipGetLastError();
}

}  // namespace tmoe
