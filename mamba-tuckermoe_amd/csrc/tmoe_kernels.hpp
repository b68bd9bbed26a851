// gfx950 device code of the Tucker-MoE layer forward (templates; the launch
// configurations used by the library are chosen in tmoe_kernels.hip).
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
// Three kernels, each an MFMA GEMM over 128-byte K tiles staged through LDS:
//   k_front   : [z | logits] = x [U_in | W_r^T]; RMSNorm epilogue on z;
//               top-k, softmax and c epilogue on the logits (x is read once)
//   k_core    : mid = (c (x) z) core_flat
//   k_outproj : out = mid U_out + bias
//
// Operand layout: every GEMM here is "NT": A is (M, K) and B^T is (N, K), both
// K-contiguous, so one lane of an MFMA fragment reads 16 contiguous bytes. The
// weights are re-laid to B^T once, at pack time.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "tmoe_internal.h"

namespace tmoe {
namespace dev {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

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
// Two floats to two bf16 (round to nearest even) in one register; as a vector
// conversion this is a single v_cvt_pk_bf16_f32.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ float load_as_f32(const uint16_t* p) { return bf16_bits_to_f32(*p); }
__device__ __forceinline__ float load_as_f32(const float* p) { return *p; }
__device__ __forceinline__ void store_from_f32(uint16_t* p, float v) { *p = f32_to_bf16_bits(v); }
__device__ __forceinline__ void store_from_f32(float* p, float v) { *p = v; }

// One 32x32 output block += A(32 x Ks) * B(Ks x 32), where one K step is 32
// bytes of each operand row: lane l supplies row/column (l & 31) and the 16-byte
// half (l >> 5) of the step.
// bf16: one v_mfma_f32_32x32x16_bf16 (Ks = 16). On gfx950 this shape issues at
//       the full 1024 flop/clk/SIMD; the 16x16x32 shape sustains about 60% of it.
// f32 : four v_mfma_f32_32x32x2_f32, chunk element j feeding MFMA j (Ks = 8).
// A and B use the same slice mapping, so any consistent K order is exact.
// Accumulator element e of lane l holds row acc_row(l, e), column (l & 31).
__device__ __forceinline__ int acc_row(int lane, int e) {
  return 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
}
__device__ __forceinline__ void mma(f32x16& acc, u32x4 a, u32x4 b, EltBF16) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x16& acc, u32x4 a, u32x4 b, EltF32) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[j]), __uint_as_float(b[j]), acc,
                                               0, 0, 0);
}
__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int e = 0; e < 16; ++e) z[e] = 0.f;
  return z;
}

// ---- operand tile loaders ------------------------------------------------
// fetch(row, ch, kt) issues the global load of 16-byte chunk `ch` (0..7) of tile
// row `row` for K tile `kt`; finish(raw) turns what arrived into the chunk that
// is written to LDS. Splitting the two lets loads for later K tiles stay in
// flight while earlier ones are consumed. Rows past the operand's end are
// clamped to its last row: their products only reach output rows/columns that
// are never stored. A tile's rows span less than 4 GB (the plan bounds d_in and
// r2), so offsets from the tile's first row are 32-bit: the base stays uniform
// and a lane carries one 32-bit offset per load.

struct RowLoader {          // plain row-major, K-contiguous operand
  typedef u32x4 Raw;
  static constexpr int kVmem = 1;   // vector memory instructions per fetch
  const char* base;         // first row of this work-group's tile
  int64_t row_bytes;
  int rows_valid;           // >= 1
  __device__ __forceinline__ const char* gaddr(int row, int ch, int kt) const {
    const int r = row < rows_valid ? row : rows_valid - 1;
    return base + ((uint32_t)r * (uint32_t)row_bytes + (uint32_t)(kt * kTileKBytes + ch * 16));
  }
  __device__ __forceinline__ Raw fetch(int row, int ch, int kt) const {
    return *reinterpret_cast<const u32x4*>(gaddr(row, ch, kt));
  }
  __device__ __forceinline__ u32x4 finish(const Raw& v) const { return v; }
};

// A operand of the core GEMM: A[t, r*r3 + s] = c[t, r] * z[t, s], rounded to the
// operand type. A K tile never straddles two r blocks (r3 is a multiple of the
// tile's element count).
template <class Elt>
struct KhatriRaoLoader {
  struct Raw {
    u32x4 v;
    float c;
  };
  static constexpr int kVmem = 2;   // z chunk + c scalar
  const char* z;            // first row of the tile, (., r3)
  const float* c;           // first row of the tile, (., r1)
  int r1, r3;
  int rows_valid;
  __device__ __forceinline__ Raw fetch(int row, int ch, int kt) const {
    constexpr int kTileK = kTileKBytes / (int)sizeof(typename Elt::T);
    const int r = row < rows_valid ? row : rows_valid - 1;
    const int k0 = kt * kTileK;
    const int rr = k0 / r3;
    const int s0 = k0 - rr * r3;
    Raw o;
    o.v = *reinterpret_cast<const u32x4*>(
        z + ((int64_t)r * r3 + s0) * (int64_t)sizeof(typename Elt::T) + ch * 16);
    o.c = c[(int64_t)r * r1 + rr];
    return o;
  }
  __device__ __forceinline__ u32x4 finish(const Raw& raw) const {
    u32x4 o;
    if constexpr (sizeof(typename Elt::T) == 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_bf16x2(bf16_bits_to_f32(raw.v[j] & 0xffffu) * raw.c,
                           bf16_bits_to_f32(raw.v[j] >> 16) * raw.c);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = __float_as_uint(__uint_as_float(raw.v[j]) * raw.c);
    }
    return o;
  }
};

// ---- the shared GEMM main loop -------------------------------------------
// C tile (BM x BN) of A (M x K) * B^T (N x K)^T, fp32 accumulate, 64*WM*WN threads.
// Waves form a WM x WN grid; wave (wm, wn) owns rows wm*BM/WM.. and columns
// wn*BN/WN.. of the tile as FM x FN blocks of 32 x 32. BX further B rows are
// staged with the tile for an `extra` consumer (the router columns of k_front).
//
// LDS holds NS stages of [BM + BN + BX rows][8 chunks of 16 B], XOR-swizzled
// (lds_slot). Each operand reaches LDS one of two ways:
//  * DMA (ADMA / BDMA): global_load_lds_dwordx4 writes LDS directly; one wave
//    instruction fills one 1 KB block of 8 rows, each lane fetching the logical
//    chunk its slot holds (dma_chunk). Tile kt + NS - 1 is issued while tile kt
//    is computed.
//  * a register ring of PFA / PFB tiles (for an operand that is transformed on
//    the way, or streamed from HBM and wanting more tiles in flight); tile kt+1
//    is written to LDS in between the MFMAs of tile kt.
// WA > 0 splits the loads by wave: waves 0 .. WA-1 run the register rings and
// issue no DMA, the others issue the DMA and no register loads (see
// gemm_mainloop).
// One barrier per K tile, preceded by an explicit wait for exactly the loads
// tile kt + 1 needs (the compiler's own barrier would wait for every load).
template <int BM_, int BN_, int BX_, int WM_, int WN_, int PFA_, int PFB_, int NS_ = 2,
          bool ADMA_ = false, bool BDMA_ = false, int WA_ = 0>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, BX = BX_, WM = WM_, WN = WN_;
  static constexpr int PFA = PFA_, PFB = PFB_, NS = NS_, WA = WA_;
  static constexpr bool ADMA = ADMA_, BDMA = BDMA_;
  static constexpr int kThreads = 64 * WM * WN;
  static constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
  static constexpr int FM = kWaveM / 32, FN = kWaveN / 32;
  static constexpr int kChunks = kTileKBytes / 16;   // 8 per row
  static constexpr int kBRows = BN + BX;
  static constexpr int kStage = (BM + kBRows) * kChunks;  // u32x4 slots per stage
  static constexpr int kLdsBytes = NS * kStage * 16;
  static_assert(BM % (32 * WM) == 0 && BN % (32 * WN) == 0, "tile/wave mismatch");
  static_assert(PFA >= 1 && PFA <= 8 && PFB >= 1 && PFA % PFB == 0, "prefetch rings");
  static_assert(NS >= 2 && NS <= 4, "LDS stages");
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
  static_assert(WA >= 0 && WA < WM * WN, "load roles");
  static_assert(WA == 0 || (!ADMA && BDMA), "load roles: A by register ring, B by DMA");
};

typedef __attribute__((address_space(3))) void* lds_vptr;
typedef const __attribute__((address_space(1))) void* gbl_cvptr;

// s_waitcnt with vmcnt <= VM and lgkmcnt == 0 (gfx9 encoding: vmcnt in bits 3:0 and
// 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int VM>
__device__ __forceinline__ void wait_vm_lds() {
  static_assert(VM >= 0 && VM < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4));
}

// 24 wait states: more than the longest MFMA result latency a following VALU,
// LDS or memory instruction must respect (16-pass fp32 MFMAs need 18 or 19).
// Issued at the end of every main-loop K tile: the last MFMAs may sit in a
// conditional block, and the compiler's own padding before the copies it makes
// of the accumulators at the loop exit was found one wait state short there.
__device__ __forceinline__ void mfma_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }

// Work-group barrier that orders LDS traffic only; loads still in flight stay in
// flight. The empty asm statements keep the compiler from moving memory
// accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);   // no instruction is scheduled across it
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}

// Chunk ch of tile row r lives at slot ch ^ ((r >> 1) & 7) of the row. A 32x32
// fragment read touches rows r0 .. r0 + 31 at one chunk; with this swizzle any 16
// consecutive of them fall on 16 distinct 16-byte bank groups (measured: no LDS
// bank conflicts, against half the LDS cycles lost with a (r & 7) swizzle).
__device__ __forceinline__ int lds_slot(int row, int ch) { return row * 8 + (ch ^ ((row >> 1) & 7)); }
// For a DMA of 8-row block blk, lane l writes slot 64 blk + l: row 8 blk + (l >> 3),
// physical chunk l & 7, which holds this logical chunk.
__device__ __forceinline__ int dma_chunk(int lane, int blk) {
  return (lane & 7) ^ ((lane >> 4) | ((blk & 1) << 2));
}

// A main-loop consumer: load(frag, s, kstep, ch) reads what K step kstep needs
// from the stage (issued with the main operands' fragments, one step ahead),
// compute(frag, kstep, af) runs after that step's MFMAs with its A fragments;
// tile_begin(kt, acc) runs before the MFMAs of K tile kt.
__device__ __forceinline__ int cmin_dev(int a, int b) { return a < b ? a : b; }

struct NoExtra {
  struct Frag {};
  __device__ __forceinline__ void load(Frag&, const u32x4*, int, int) const {}
  template <class AF>
  __device__ __forceinline__ void compute(const Frag&, int, const AF&) const {}
  template <class ACC>
  __device__ __forceinline__ void tile_begin(int, ACC&) const {}
};

// One wave's part of the main loop. ROLE 0: every load kind; ROLE 1: the
// register rings only (waves 0 .. WA-1); ROLE 2: the DMA only (waves WA ..).
//
// Every iteration issues the same loads: near the end of K the DMA and the ring
// refills fetch the last tile again (in bounds; into a stage or ring slot no
// later tile reads), so the vmcnt bounds below are exact and the compiler's own
// waits for the ring registers see the same count of younger loads in every
// iteration (conditional loads made it wait for all of them). Only the tail of
// nkt % PFA tiles runs under a condition.
template <int ROLE, class TL, class Elt, class ALoad, class BLoad, class Extra>
__device__ __forceinline__ void gemm_mainloop_role(f32x16 (&acc)[TL::FM][TL::FN],
                                                   const ALoad& aload, const BLoad& bload,
                                                   int nkt, u32x4* smem, Extra& extra) {
  constexpr int FM = TL::FM, FN = TL::FN, CH = TL::kChunks, NS = TL::NS;
  constexpr bool ADMA = TL::ADMA, BDMA = TL::BDMA;
  constexpr int PFA = ADMA ? 1 : TL::PFA, PFB = BDMA ? 1 : TL::PFB;
  constexpr int kKSteps = kTileKBytes / 32;   // MFMA K steps per K tile
  constexpr int W = TL::kThreads / 64;
  constexpr int kARows = TL::BM, kBRows = TL::kBRows;
  constexpr bool kRing = ROLE != 2, kDma = ROLE != 1;
  // threads sharing the ring loads, waves sharing the DMA
  constexpr int NL = ROLE == 1 ? 64 * TL::WA : TL::kThreads;
  constexpr int NWD = ROLE == 2 ? W - TL::WA : W;
  constexpr int AP = (kRing && !ADMA) ? (kARows * CH + NL - 1) / NL : 0;
  constexpr int BP = (kRing && !BDMA) ? (kBRows * CH + NL - 1) / NL : 0;
  // every ring thread issues the same loads, so one vmcnt count holds for all
  static_assert(AP * NL == (kRing && !ADMA ? kARows * CH : 0), "register-staged A: full rounds");
  static_assert(BP * NL == (kRing && !BDMA ? kBRows * CH : 0), "register-staged B: full rounds");
  // DMA instructions each DMA wave issues per tile. When the 8-row blocks do not
  // split evenly over the waves, the extra slots repeat the last block: the same
  // bytes to the same LDS slots, waited for like any other, so every wave issues
  // the same count and one vmcnt bound holds for all.
  constexpr int kANBlk = kARows / 8, kBNBlk = kBRows / 8;
  constexpr int ADN = (kDma && ADMA) ? (kANBlk + NWD - 1) / NWD : 0;
  constexpr int BDN = (kDma && BDMA) ? (kBNBlk + NWD - 1) / NWD : 0;
  static_assert(kARows % 16 == 0 && kBRows % 8 == 0, "DMA blocks of 8 rows");
  // vector memory instructions per tile: register rings (per fetch) and DMA
  constexpr int FA = AP * ALoad::kVmem, FB = BP * BLoad::kVmem, D = ADN + BDN;
  // loads issued after tile kt+1's DMA until the end of iteration kt
  constexpr int kVmAfter = (NS - 2) * D + (NS - 1) * (FA + FB);
  static_assert(kVmAfter < 63 && (NS - 2) * D + PFA * FA + PFB * FB < 63, "vmcnt range");
  // Memory instructions are spread over the K steps of a tile, each after that
  // step's MFMAs, so a wave never stalls on a full memory queue with MFMAs left
  // to issue: DMA of tile kt + NS - 1 over the first kDmaSteps steps; the
  // register-staged LDS stores of tile kt + 1 and the ring refills that reuse
  // their registers over the last kStashSteps steps (all steps for a wave that
  // issues no DMA).
  constexpr int kStashSteps = D > 0 ? 2 : kKSteps;
  constexpr int kDmaSteps = AP + BP > 0 ? kKSteps - kStashSteps : kKSteps;
  constexpr int kPerStep = (AP + BP + kStashSteps - 1) / kStashSteps;
  constexpr int kDmaPerStep = (D + (kDmaSteps > 0 ? kDmaSteps : 1) - 1) / (kDmaSteps > 0 ? kDmaSteps : 1);
  // fragment buffers: two (reads one K step ahead) when the registers allow
  constexpr int PIPE = FM + FN <= 4 ? 2 : 1;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / TL::WN, wn = wave % TL::WN;
  const int rtid = ROLE == 2 ? tid - 64 * TL::WA : tid;   // index within the role
  const int rwave = rtid >> 6;

#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = zero16();

  // Register rings: tile t in A slot t % PFA and B slot t % PFB.
  typename ALoad::Raw ra[PFA][AP > 0 ? AP : 1];
  typename BLoad::Raw rb[PFB][BP > 0 ? BP : 1];

  auto fetch_a = [&](int kt, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < AP; ++i) {
      const int q = rtid + i * NL;
      ra[slot][i] = aload.fetch(q / CH, q % CH, kt);
    }
  };
  auto fetch_b = [&](int kt, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      const int q = rtid + i * NL;
      rb[slot][i] = bload.fetch(q / CH, q % CH, kt);
    }
  };
  // DMA instruction j < ADN + BDN of tile kt into LDS stage `stage` (A blocks
  // first, then B blocks)
  auto dma_one = [&](int j, int kt, int stage) __attribute__((always_inline)) {
    u32x4* s = smem + stage * TL::kStage;
    if (j < ADN) {
      if constexpr (ADN > 0) {
        const int blk = cmin_dev(rwave + j * NWD, kANBlk - 1);
        __builtin_amdgcn_global_load_lds(
            (gbl_cvptr)aload.gaddr(blk * 8 + (lane >> 3), dma_chunk(lane, blk), kt),
            (lds_vptr)(s + blk * 64), 16, 0, 0);
      }
    } else if (j < ADN + BDN) {
      if constexpr (BDN > 0) {
        // kARows is a multiple of 16, so the block parity within B equals the
        // parity of its LDS block
        const int blk = cmin_dev(rwave + (j - ADN) * NWD, kBNBlk - 1);
        __builtin_amdgcn_global_load_lds(
            (gbl_cvptr)bload.gaddr(blk * 8 + (lane >> 3), dma_chunk(lane, blk), kt),
            (lds_vptr)(s + (kARows + blk * 8) * 8), 16, 0, 0);
      }
    }
  };
  auto dma = [&](int kt, int stage) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < D; ++j) dma_one(j, kt, stage);
  };
  // ring refill of register-staged chunk c for tile kt (A slot sa / B slot sb)
  auto refill_chunk = [&](int c, int kta, int ktb, int sa, int sb) __attribute__((always_inline)) {
    if (c < AP) {
      const int q = rtid + c * NL;
      ra[sa][c] = aload.fetch(q / CH, q % CH, kta);
    } else if (c < AP + BP) {
      const int q = rtid + (c - AP) * NL;
      rb[sb][c - AP] = bload.fetch(q / CH, q % CH, ktb);
    }
  };
  // register-staged chunk c < AP + BP: A chunks first, then B chunks
  auto stash_chunk = [&](int c, int sa, int sb, u32x4* s) __attribute__((always_inline)) {
    if (c < AP) {
      const int q = rtid + c * NL;
      s[lds_slot(q / CH, q % CH)] = aload.finish(ra[sa][c]);
    } else if (c < AP + BP) {
      const int q = rtid + (c - AP) * NL;
      s[lds_slot(kARows + q / CH, q % CH)] = bload.finish(rb[sb][c - AP]);
    }
  };
  // MFMAs of tile kt, with the memory work of this iteration in between: DMA of
  // tile kt + NS - 1; stores of ring slots (sa, sb) (tile kt + 1) to that tile's
  // stage and their refill with tiles kt + 1 + PFA / kt + 1 + PFB. Past the last
  // tile these fetch tile nkt - 1 again.
  auto iteration = [&](int kt, int sa, int sb) __attribute__((always_inline)) {
    const int ktd = cmin_dev(kt + NS - 1, nkt - 1);
    const int kta = cmin_dev(kt + 1 + PFA, nkt - 1), ktb = cmin_dev(kt + 1 + PFB, nkt - 1);
    const u32x4* s = smem + (kt % NS) * TL::kStage;
    u32x4* so = smem + ((kt + 1) % NS) * TL::kStage;
    const int sd = (kt + NS - 1) % NS;
    extra.tile_begin(kt, acc);
    // fragments of K step ks in buffer ks % PIPE; with two buffers step ks + 1 is
    // read before step ks's MFMAs issue
    u32x4 af[PIPE][FM], bfr[PIPE][FN];
    typename Extra::Frag xf[PIPE];
    auto load_frags = [&](int ks, int b) __attribute__((always_inline)) {
      const int ch = ks * 2 + (lane >> 5);
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[b][i] = s[lds_slot(wm * TL::kWaveM + i * 32 + (lane & 31), ch)];
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[b][j] = s[lds_slot(kARows + wn * TL::kWaveN + j * 32 + (lane & 31), ch)];
      extra.load(xf[b], s, kt * kKSteps + ks, ch);
    };
    if constexpr (PIPE == 2) load_frags(0, 0);
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) {
      const int b = ks % PIPE;
      if constexpr (PIPE == 1) load_frags(ks, 0);
      else if (ks + 1 < kKSteps) load_frags(ks + 1, (ks + 1) % PIPE);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) mma(acc[i][j], af[b][i], bfr[b][j], Elt{});
      extra.compute(xf[b], kt * kKSteps + ks, af[b]);
      if constexpr (D > 0) {
        if (ks < kDmaSteps) {
#pragma unroll
          for (int j = 0; j < kDmaPerStep; ++j)
            dma_one(ks * kDmaPerStep + j, ktd, sd);
        }
        // no later load may be scheduled above the DMA: the vmcnt bounds count
        // the loads issued after it
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (AP + BP > 0) {
        if (ks >= kKSteps - kStashSteps) {
          const int c0 = (ks - (kKSteps - kStashSteps)) * kPerStep;
#pragma unroll
          for (int c = 0; c < kPerStep; ++c) stash_chunk(c0 + c, sa, sb, so);
#pragma unroll
          for (int c = 0; c < kPerStep; ++c) refill_chunk(c0 + c, kta, ktb, sa, sb);
        }
      }
    }
    // the accumulators may be copied at the loop exit right after a skipped
    // conditional MFMA block
    mfma_drain();
    // tile kt + 1 must be in LDS: its DMA and this wave's LDS stores. A ring-only
    // wave waits for its LDS stores alone (the compiler waited for the ring
    // registers it stored).
    if constexpr (ROLE == 1) wait_vm_lds<63>();
    else wait_vm_lds<kVmAfter>();
    lds_barrier();
  };

  // prologue: tile 0 complete in stage 0; DMA tiles 1 .. NS-2; ring tiles
  // 1 .. PFA / PFB in flight
  fetch_a(0, 0);
  fetch_b(0, 0);
  dma(0, 0);
  __builtin_amdgcn_sched_barrier(0);   // the ring fetches below stay after the DMA
#pragma unroll
  for (int c = 0; c < AP + BP; ++c) stash_chunk(c, 0, 0, smem);
#pragma unroll
  for (int t = 1; t <= NS - 2; ++t) dma(cmin_dev(t, nkt - 1), t);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int p = 1; p <= PFA; ++p)
    if constexpr (AP > 0) fetch_a(cmin_dev(p, nkt - 1), p % PFA);
#pragma unroll
  for (int p = 1; p <= PFB; ++p)
    if constexpr (BP > 0) fetch_b(cmin_dev(p, nkt - 1), p % PFB);
  if constexpr (ROLE == 1) wait_vm_lds<63>();
  else wait_vm_lds<(NS - 2) * D + PFA * FA + PFB * FB>();
  lds_barrier();

  // ring slots of tile kt + 1 (k0 is a multiple of PFA, hence of PFB)
  int k0 = 0;
  for (; k0 + PFA <= nkt; k0 += PFA) {
#pragma unroll
    for (int p = 0; p < PFA; ++p) iteration(k0 + p, (p + 1) % PFA, (p + 1) % PFB);
  }
#pragma unroll
  for (int p = 0; p + 1 < PFA; ++p)
    if (k0 + p < nkt) iteration(k0 + p, (p + 1) % PFA, (p + 1) % PFB);
  // the refetches of the last tile land before the caller reuses the LDS
  wait_vm_lds<0>();
  lds_barrier();
}

template <class TL, class Elt, class ALoad, class BLoad, class Extra>
__device__ __forceinline__ void gemm_mainloop(f32x16 (&acc)[TL::FM][TL::FN], const ALoad& aload,
                                              const BLoad& bload, int nkt, u32x4* smem,
                                              Extra& extra) {
  if constexpr (TL::WA > 0) {
    // vmcnt counts one wave's loads, which complete in issue order: a wave that
    // waited for a one-tile-deep DMA would also wait for every ring load issued
    // before it. Split by wave, the ring keeps PFA tiles in flight.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (wave < TL::WA) gemm_mainloop_role<1, TL, Elt>(acc, aload, bload, nkt, smem, extra);
    else gemm_mainloop_role<2, TL, Elt>(acc, aload, bload, nkt, smem, extra);
  } else {
    gemm_mainloop_role<0, TL, Elt>(acc, aload, bload, nkt, smem, extra);
  }
}

// ---- ping-pong main loop (both operands by DMA, 8 waves) ----------------
// Waves 0-3 (group 0) and 4-7 (group 1) sit one of each on every SIMD. Group 1
// starts one barrier late, so the two alternate between a memory phase (read
// all of tile kt's fragments into registers; group 0 also issues the DMA of
// tile kt + 1) and a compute phase (the tile's MFMAs, from registers): while
// one wave of a SIMD issues MFMAs, the other issues its memory instructions.
// With phase p lying between barriers p - 1 and p:
//   group 0: memory(kt) = phase 2kt, compute(kt) = phase 2kt + 1
//   group 1: memory(kt) = phase 2kt + 1, compute(kt) = phase 2kt + 2
// DMA(kt + 1) is issued in phase 2kt into the stage of tile kt - 1, whose last
// reader (group 1, phase 2kt - 1) waited for its LDS reads before barrier
// 2kt - 1; group 0 waits for the DMA at the end of phase 2kt + 1, before either
// group reads tile kt + 1.
// Group 0 issues every DMA, tile 0's included, and group 1 never waits on vmcnt:
// stores group 1 issued before the call keep draining while it runs.
// The MFMAs take B as their first operand, so acc[i][j] holds the transposed
// block: lane l has row l & 31 of row block i and, in elements 4q .. 4q + 3,
// columns 8q + 4 (l >> 5) .. + 3 of column block j (stage_tile_t).
template <class TL, class Elt, class ALoad, class BLoad>
__device__ __forceinline__ void gemm_mainloop_pingpong(f32x16 (&acc)[TL::FM][TL::FN],
                                                       const ALoad& aload, const BLoad& bload,
                                                       int nkt, u32x4* smem) {
  constexpr int FM = TL::FM, FN = TL::FN;
  constexpr int kKSteps = kTileKBytes / 32;
  constexpr int kARows = TL::BM, kBRows = TL::kBRows;
  constexpr int kABlk = kARows / 8, kBBlk = kBRows / 8;   // 1 KB DMA blocks per tile
  static_assert(TL::kThreads == 512 && TL::NS == 2 && TL::BX == 0, "ping-pong: 8 waves, 2 stages");
  static_assert((kABlk + kBBlk) % 4 == 0, "DMA blocks split over group 0's four waves");
  constexpr int kDmaPerWave = (kABlk + kBBlk) / 4;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = wave >> 2;
  const int wm = wave / TL::WN, wn = wave % TL::WN;

#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = zero16();

  auto dma_block = [&](int blk, int kt, int stage) __attribute__((always_inline)) {
    u32x4* s = smem + stage * TL::kStage;
    const int lc = dma_chunk(lane, blk);   // kABlk is even: block parity is kept
    if (blk < kABlk)
      __builtin_amdgcn_global_load_lds((gbl_cvptr)aload.gaddr(blk * 8 + (lane >> 3), lc, kt),
                                       (lds_vptr)(s + blk * 64), 16, 0, 0);
    else
      __builtin_amdgcn_global_load_lds(
          (gbl_cvptr)bload.gaddr((blk - kABlk) * 8 + (lane >> 3), lc, kt),
          (lds_vptr)(s + (kARows + (blk - kABlk) * 8) * 8), 16, 0, 0);
  };

  // prologue: tile 0 by group 0
  if (grp == 0) {
    for (int blk = wave; blk < kABlk + kBBlk; blk += 4) dma_block(blk, 0, 0);
    wait_vm_lds<0>();
  }
  lds_barrier();
  if (grp == 1) lds_barrier();

  for (int kt = 0; kt < nkt; ++kt) {
    const u32x4* s = smem + (kt & 1) * TL::kStage;
    // -- memory phase ---------------------------------------------------------
    u32x4 af[kKSteps][FM], bfr[kKSteps][FN];
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) {
      const int ch = ks * 2 + (lane >> 5);
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[ks][i] = s[lds_slot(wm * TL::kWaveM + i * 32 + (lane & 31), ch)];
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[ks][j] = s[lds_slot(kARows + wn * TL::kWaveN + j * 32 + (lane & 31), ch)];
    }
    if (grp == 0 && kt + 1 < nkt) {
#pragma unroll
      for (int j = 0; j < kDmaPerWave; ++j) dma_block(wave + 4 * j, kt + 1, (kt + 1) & 1);
    }
    wait_vm_lds<63>();   // this wave's fragment reads (lgkmcnt 0); DMA stays in flight
    lds_barrier();
    // -- compute phase --------------------------------------------------------
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) mma(acc[i][j], bfr[ks][j], af[ks][i], Elt{});
    if (grp == 0) wait_vm_lds<0>();   // DMA of tile kt + 1 has landed
    lds_barrier();
  }
  if (grp == 0) lds_barrier();
  mfma_drain();
}

// Work-group -> tile order for 2-D grids launched as 1-D. Consecutive
// work-groups land on different XCDs (round robin over 8); this hands each XCD a
// contiguous run of tiles, row-major over (m, n), so the A rows of an m tile are
// fetched into one XCD's L2 and reused for all its n tiles.
__device__ __forceinline__ void tile_coords_of(int b, int n_tiles_n, int n_tiles, int& tm,
                                               int& tn) {
  const int per = n_tiles / 8;
  const int t = b < per * 8 ? (b % 8) * per + b / 8 : b;
  tm = t / n_tiles_n;
  tn = t - tm * n_tiles_n;
}
__device__ __forceinline__ void tile_coords(int n_tiles_n, int n_tiles, int& tm, int& tn) {
  tile_coords_of(blockIdx.x, n_tiles_n, n_tiles, tm, tn);
}

// ---- C tile store through LDS ----------------------------------------------
// The MFMA result layout gives each lane one column of sixteen rows, so direct
// stores would be 2- or 4-byte scatters. The tile is instead converted into LDS
// (rows padded by 16 bytes, which puts the two row groups one store instruction
// touches on distinct banks) and written out as 16-byte, row-contiguous chunks.
template <class TL, class T>
struct TileStage {
  static constexpr int kRowBytes = TL::BN * (int)sizeof(T) + 16;
  static constexpr int kBytes = TL::BM * kRowBytes;
};

// Stores acc * colm[j] + colv[j] as T (colm, colv: a per-column multiplier and
// addend this lane holds for each of its FN column blocks, loaded once before the
// loop). A multiplier of 1 leaves acc + colv exactly.
template <class TL, class T>
__device__ __forceinline__ void stage_tile(const f32x16 (&acc)[TL::FM][TL::FN], char* stage,
                                           const float (&colv)[TL::FN],
                                           const float (&colm)[TL::FN]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / TL::WN, wn = wave % TL::WN;
  constexpr int RB = TileStage<TL, T>::kRowBytes;
#pragma unroll
  for (int j = 0; j < TL::FN; ++j) {
    const int col = wn * TL::kWaveN + j * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < TL::FM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = wm * TL::kWaveM + i * 32 + acc_row(lane, e);
        const float v = acc[i][j][e] * colm[j] + colv[j];
        store_from_f32(reinterpret_cast<T*>(stage + row * RB + col * (int)sizeof(T)), v);
      }
  }
}

// Copies a staged tile to dst (the tile's origin, leading dimension ld
// elements). Columns are only ever cut at multiples of 16, so a 16-byte chunk is
// wholly inside or wholly outside the valid columns. The stores are streaming
// (nontemporal): the tile is not read again by this kernel, and allocating it in
// L2 would evict the operand tiles the next work-groups read.
template <class TL, class T>
__device__ __forceinline__ void flush_tile(const char* stage, T* dst, int64_t ld, int rows_valid,
                                           int cols_valid) {
  constexpr int RB = TileStage<TL, T>::kRowBytes;
  constexpr int CPR = TL::BN * (int)sizeof(T) / 16;   // chunks per row
  constexpr int EPC = 16 / (int)sizeof(T);           // elements per chunk
  for (int c = threadIdx.x; c < TL::BM * CPR; c += TL::kThreads) {
    const int row = c / CPR, ch = c - row * CPR;
    if (row < rows_valid && ch * EPC < cols_valid)
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(stage + row * RB + ch * 16),
                                  reinterpret_cast<u32x4*>(dst + row * ld + ch * EPC));
  }
}

// Stages a bf16 tile from transposed accumulators (gemm_mainloop_pingpong): a
// lane's elements 4q .. 4q + 3 of block (i, j) are four consecutive columns of
// one row, stored as one 8-byte LDS write of (acc * scale + bias). Columns are
// cut at multiples of 16 only, so a group of four is wholly valid or not. bias
// and scale point at the tile's first column and are 16-byte aligned.
// With gamma (bf16, the tile's first column; kEpiResScale), each staged value is
// R(gamma[col] * R(y)) instead of R(y): the scaled half of the residual epilogue.
template <class TL>
__device__ __forceinline__ void stage_tile_t(const f32x16 (&acc)[TL::FM][TL::FN], char* stage,
                                             const float* bias, const float* scale, int cols_valid,
                                             const uint16_t* gamma = nullptr) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / TL::WN, wn = wave % TL::WN;
  constexpr int RB = TileStage<TL, uint16_t>::kRowBytes;
#pragma unroll
  for (int j = 0; j < TL::FN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = wn * TL::kWaveN + j * 32 + 8 * q + 4 * (lane >> 5);
      // columns past the end read column 0 (16-byte aligned); they are not stored
      const int cc = col < cols_valid ? col : 0;
      const float4 bv = *reinterpret_cast<const float4*>(bias + cc);
      const float4 sv = scale ? *reinterpret_cast<const float4*>(scale + cc)
                              : float4{1.f, 1.f, 1.f, 1.f};
      const uint2 gv = gamma ? *reinterpret_cast<const uint2*>(gamma + cc) : uint2{0u, 0u};
#pragma unroll
      for (int i = 0; i < TL::FM; ++i) {
        const int row = wm * TL::kWaveM + i * 32 + (lane & 31);
        uint2 v;
        v.x = pack_bf16x2(acc[i][j][4 * q] * sv.x + bv.x, acc[i][j][4 * q + 1] * sv.y + bv.y);
        v.y = pack_bf16x2(acc[i][j][4 * q + 2] * sv.z + bv.z,
                          acc[i][j][4 * q + 3] * sv.w + bv.w);
        if (gamma) {
          v.x = pack_bf16x2(bf16_bits_to_f32(gv.x & 0xffffu) * bf16_bits_to_f32(v.x & 0xffffu),
                            bf16_bits_to_f32(gv.x >> 16) * bf16_bits_to_f32(v.x >> 16));
          v.y = pack_bf16x2(bf16_bits_to_f32(gv.y & 0xffffu) * bf16_bits_to_f32(v.y & 0xffffu),
                            bf16_bits_to_f32(gv.y >> 16) * bf16_bits_to_f32(v.y >> 16));
        }
        *reinterpret_cast<uint2*>(stage + row * RB + col * 2) = v;
      }
    }
}

// ---- fused FFN epilogues of the out-projection -----------------------------
// The FFN sub-block of the reference's TransformerBlock (model.py:337-341) passes
// an out-projection's output y (the layer output, already rounded to the module
// dtype) through one elementwise op, which is fused into its store:
//   kEpiGlu       out = R(R(silu(g)) * y), g = epi_a[row, col]     F.silu(gate) * up
//   kEpiResScale  out = R(x + R(gamma[col] * y)), x = epi_a[row, col], gamma = epi_b
//                                                    x_res + ls_ffn(dn)   (:35-36, :341)
// R rounds to the module dtype, as each of the reference module's ops does;
// silu(g) = g / (1 + exp(-g)) in fp32 (see silu_as).
__device__ __forceinline__ float round_as(float v, EltBF16) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }
__device__ __forceinline__ float round_as(float v, EltF32) { return v; }
// silu(g) before rounding to the dtype. fp32: g / (1 + expf(-g)). bf16: g times
// the hardware reciprocal of 1 + 2^(-g log2 e) (v_exp_f32, v_rcp_f32; a few fp32
// units in the last place, which the rounding to bf16 absorbs but for about one
// element in 10^4, then one bf16 unit apart). Limits: g -> -inf gives -0, g ->
// +inf gives g, NaN stays NaN.
__device__ __forceinline__ float silu_as(float g, EltF32) { return g / (1.f + expf(-g)); }
__device__ __forceinline__ float silu_as(float g, EltBF16) {
  return g * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(g * -1.44269504f));
}
template <class Elt>
__device__ __forceinline__ float epi_value(int mode, float y, float ea, float eb) {
#pragma clang fp contract(off)   // x + gamma * y is two rounded ops, as in the reference
  if (mode == kEpiGlu) return round_as(round_as(silu_as(ea, Elt{}), Elt{}) * y, Elt{});
  return round_as(ea + round_as(eb * y, Elt{}), Elt{});
}
// epi_value over one 16-byte chunk y of output row `row`, columns col .. col + 16 /
// sizeof(T) - 1 (chunks never straddle the valid columns)
template <class T>
__device__ __forceinline__ u32x4 epi_chunk(const FwdArgs& a, u32x4 y, int64_t row, int64_t col) {
  const u32x4 ea =
      *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.epi_a) + row * a.d_out + col);
  const u32x4 eb = a.epi_mode == kEpiResScale
                       ? *reinterpret_cast<const u32x4*>(static_cast<const T*>(a.epi_b) + col)
                       : u32x4{0u, 0u, 0u, 0u};
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (sizeof(T) == 2) {
      const float lo = epi_value<EltBF16>(a.epi_mode, bf16_bits_to_f32(y[j] & 0xffffu),
                                          bf16_bits_to_f32(ea[j] & 0xffffu),
                                          bf16_bits_to_f32(eb[j] & 0xffffu));
      const float hi = epi_value<EltBF16>(a.epi_mode, bf16_bits_to_f32(y[j] >> 16),
                                          bf16_bits_to_f32(ea[j] >> 16),
                                          bf16_bits_to_f32(eb[j] >> 16));
      o[j] = pack_bf16x2(lo, hi);   // exact: both are bf16 values
    } else {
      o[j] = __float_as_uint(epi_value<EltF32>(a.epi_mode, __uint_as_float(y[j]),
                                               __uint_as_float(ea[j]), __uint_as_float(eb[j])));
    }
  }
  return o;
}

// The fused epilogue of a bf16 out-projection tile staged in LDS, by NT threads
// in two steps. epi_tile_load issues the loads of this thread's epi_a chunks
// (chunks tid, tid + NT, ...; zero past the valid rows and columns) into e, before
// the tile is staged, so that their latency overlaps the staging; only loads are
// issued, so a wave that never stores keeps its vector-memory counter free of
// stores. epi_tile_apply, after the staging barrier, combines them with the
// staged values in place: for kEpiGlu out = R(R(silu(g)) * y); for kEpiResScale
// the stage holds R(gamma * y) already (stage_tile_t) and out = R(x + that).
template <class TL, int NT>
struct EpiTile {
  static constexpr int kCPR = TL::BN * 2 / 16;
  static constexpr int kIters = TL::BM * kCPR / NT;
  static_assert(TL::BM * kCPR % NT == 0, "whole iterations");
};
template <class TL, int NT>
__device__ __forceinline__ void epi_tile_load(u32x4* e, const FwdArgs& a, int64_t m0, int64_t n0,
                                              int rows_valid, int cols_valid, int tid) {
  constexpr int CPR = EpiTile<TL, NT>::kCPR;
  const uint16_t* ea = static_cast<const uint16_t*>(a.epi_a) + m0 * a.d_out + n0;
  // opaque copy: the chunk offsets below are recomputed per tile rather than
  // hoisted out of a persistent tile loop (where they would be spilled)
  asm volatile("" : "+v"(tid));
#pragma unroll
  for (int i = 0; i < EpiTile<TL, NT>::kIters; ++i) {
    const int c = tid + i * NT, row = c / CPR, ch = c - row * CPR;
    e[i] = u32x4{0u, 0u, 0u, 0u};
    if (row < rows_valid && ch * 8 < cols_valid)
      e[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ea + row * a.d_out + ch * 8));
  }
}
template <class TL, int NT>
__device__ __forceinline__ void epi_tile_apply(char* stage, const u32x4* e, const FwdArgs& a,
                                               int tid) {
  constexpr int RB = TileStage<TL, uint16_t>::kRowBytes;
  constexpr int CPR = EpiTile<TL, NT>::kCPR;
  const bool glu = a.epi_mode == kEpiGlu;
  asm volatile("" : "+v"(tid));
#pragma unroll
  for (int i = 0; i < EpiTile<TL, NT>::kIters; ++i) {
    const int c = tid + i * NT, row = c / CPR, ch = c - row * CPR;
    u32x4* slot = reinterpret_cast<u32x4*>(stage + row * RB + ch * 16);
    const u32x4 y = *slot;
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float y0 = bf16_bits_to_f32(y[j] & 0xffffu), y1 = bf16_bits_to_f32(y[j] >> 16);
      const float e0 = bf16_bits_to_f32(e[i][j] & 0xffffu), e1 = bf16_bits_to_f32(e[i][j] >> 16);
      o[j] = glu ? pack_bf16x2(round_as(silu_as(e0, EltBF16{}), EltBF16{}) * y0,
                               round_as(silu_as(e1, EltBF16{}), EltBF16{}) * y1)
                 : pack_bf16x2(e0 + y0, e1 + y1);
    }
    *slot = o;   // rows and columns past the valid ones are never stored
  }
}

// Writes an out-projection tile staged in LDS to out (origin (m0, n0)) by the NT
// threads t0 .. t0 + NT - 1 of the work-group (tid: this thread's index among
// them), through the fused epilogue a.epi_mode unless kStagedFinal (the stage
// holds the final values already, epi_tile_apply).
template <class TL, class T, int NT, bool kStagedFinal = false>
__device__ __forceinline__ void flush_tile_by(const char* stage, const FwdArgs& a, int64_t m0,
                                              int64_t n0, int rows_valid, int cols_valid, int tid) {
  constexpr int RB = TileStage<TL, T>::kRowBytes;
  constexpr int CPR = TL::BN * (int)sizeof(T) / 16;
  constexpr int EPC = 16 / (int)sizeof(T);
  T* dst = reinterpret_cast<T*>(a.out) + m0 * a.d_out + n0;
  for (int c = tid; c < TL::BM * CPR; c += NT) {
    const int row = c / CPR, ch = c - row * CPR;
    if (row < rows_valid && ch * EPC < cols_valid) {
      u32x4 v = *reinterpret_cast<const u32x4*>(stage + row * RB + ch * 16);
      if (!kStagedFinal && a.epi_mode != kEpiNone) v = epi_chunk<T>(a, v, m0 + row, n0 + ch * EPC);
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst + row * a.d_out + ch * EPC));
    }
  }
}

constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int cmin(int a, int b) { return a < b ? a : b; }

// ---- signals between the work-groups of one launch -------------------------
// A producer work-group writes the data it hands over with device-scope stores
// (store_coherent), then sets a flag word to the launch's epoch; its consumer
// waits for that value and reads the data with device-scope loads
// (load_coherent). Both sides go through the point of coherence of the XCDs'
// caches for those words only: release and acquire fences would write back or
// invalidate the whole L2 of an XCD, under the work-groups still computing there
// (measured: the E_pad = 256 front at T = 4096 went from 35 to 72 us with an
// acquire in the wait loop). sync_publish waits for the work-group's stores to
// complete before the flag is written. (The one-launch large-T forward hands its
// c (x) z rows over inside one XCD's L2 with plain stores and loads instead:
// producer and consumers run on the same XCD, see tmoe_fused.hpp.)
// Consumers have higher work-group indices than their producers, or all
// work-groups of the launch are resident at once (one per compute unit), so a
// waiting consumer never keeps its producer from running. A wait is bounded by a
// number of polls of its flags (FwdArgs::wait_polls, set by the host; a poll
// costs a device-scope load round trip and ~128 clocks of sleep). Past it the
// epoch goes into sync[0], word kStatusSignal of the launch's host-visible status
// block (FwdArgs::status) is set, and the consumer goes on with NaN in place of
// the data, so that a lost signal surfaces as an error the host can read and as
// NaN output, never as a hang. A budget of 0 gives up without polling (the host's
// way to exercise this path with every kernel still exiting normally). When a
// flag has one consumer, that consumer sets it back to 0 once seen (a second
// launch with the same epoch, as a graph replay, then waits again); launches
// whose flags have several consumers, or whose consumer may give up, are kept
// out of graph capture by the launcher.
constexpr int kStatusSignal = kStatusSignalWord;

__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sets word `which` of the host-visible status block (no-op without one).
__device__ __forceinline__ void report_status(uint32_t* status, int which) {
  if (status) __hip_atomic_store(status + which, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ void sync_publish(uint32_t* flag, uint32_t epoch) {
  wait_vm_lds<0>();   // this thread's stores have completed (the barrier alone
  __syncthreads();    // does not wait for them), then every thread's have
  if (threadIdx.x == 0)
    __hip_atomic_store(flag, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Called by every thread: waits for the n flags flags[0], flags[kSyncStride], ...;
// true once all were seen, false when the wait ran out of its budget of `polls`
// polls (see above; the error is then recorded in *err and the status block).
// The first wave polls: lane l watches flags l, l + 64, ..., so that flags set at
// about the same time cost one round trip, not one each. reset: the caller is the
// flags' only consumer and sets them back to 0 once seen. seen_all: one word of
// the kernel's LDS array for the answer (a __shared__ variable of its own changed
// how the compiler tracks the kernel's LDS DMA: it then waited for every DMA
// before each fragment read of the main loop). The work-group has at least 64
// threads.
__device__ __forceinline__ bool sync_await(uint32_t* flags, int n, uint32_t epoch, uint32_t* err,
                                           int* seen_all, bool reset, int polls,
                                           uint32_t* status) {
  if (threadIdx.x < 64) {   // the whole first wave
    const int l = threadIdx.x;
    int next = l;   // the lane's first flag not yet seen
    bool seen = n <= 0;
    for (int p = 0; p < polls && !seen; ++p) {
      while (next < n && __hip_atomic_load(flags + (int64_t)next * kSyncStride, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT) == epoch)
        next += 64;
      if (__all(next >= n)) {
        seen = true;
        break;
      }
      __builtin_amdgcn_s_sleep(2);   // ~128 clocks between polls
    }
    if (!seen) {
      if (l == 0) {
        __hip_atomic_store(err, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        report_status(status, kStatusSignal);
      }
    } else if (reset) {
      for (int i = l; i < n; i += 64)
        __hip_atomic_store(flags + (int64_t)i * kSyncStride, 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (l == 0) *seen_all = seen ? 1 : 0;
  }
  __syncthreads();
  return *seen_all != 0;
}

// ---- k_front: in-projection + RMSNorm, router + top-k + softmax + c --------
// model.py:75-81 (+ the U_expert gather of :93 folded into c). One work-group:
// BM tokens x (R3 z columns + EP router columns), NW = R3 / 32 (at most 4) waves
// side by side over the z columns in each of WMF row groups (a wave owns BM / WMF
// rows). The row groups share the weight stages in LDS. With BM = 32 and one
// row group the LDS stays under 80 KB, so two work-groups share a CU and one's
// epilogue overlaps the other's main loop.
//  z part: epilogue z = (z / rms) * g with rms = sqrt(mean(z^2) + eps)
//  (model.py:25-27), the division taken as a multiply by 1 / rms.
//  router part (NR = EP/32 column blocks): with NR < NW every wave computes all
//  router columns of its rows over every NW-th K step and the partial sums are
//  added in wave order; otherwise the waves split the router columns. Top-k:
//  k rounds of a max over rank_key (torch.topk's order) within a group of lanes
//  per row.
// Top-k order (torch.topk, model.py:76): larger logit first, NaN above every
// number, equal values by lower expert index. As one unsigned 64-bit key,
// larger = ranks first: high word the logit mapped to an order-preserving
// unsigned integer (-0 canonicalised to +0 so that it ties with +0; every NaN
// mapped to the top), low word ~index (a lower index wins a tie). Key 0 is below
// every candidate and stands for "none".
__device__ __forceinline__ uint64_t rank_key(float v, int idx) {
  const float c = v + 0.f;   // -0 + 0 = +0 (round to nearest)
  const uint32_t u = __float_as_uint(c);
  uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  k = (c != c) ? 0xffffffffu : k;
  return ((uint64_t)k << 32) | (uint32_t)~(uint32_t)idx;
}
__device__ __forceinline__ int key_index(uint64_t key) { return (int)~(uint32_t)key; }
__device__ __forceinline__ float key_value(uint64_t key) {   // the canonical logit
  const uint32_t k = (uint32_t)(key >> 32);
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Max-key over aligned groups of G in {1, 2, 4, 8} lanes with DPP moves (VALU
// cross-lane reads, no LDS traffic): quad_perm [1,0,3,2] and [2,3,0,1] combine
// lanes at xor 1 and xor 2, row_half_mirror lane i with 7 - i of its 8-lane
// half row. After the steps every lane of a group holds the group's best.
template <int CTRL>
__device__ __forceinline__ void dpp_max_step(uint64_t& key) {
  const uint32_t lo = __builtin_amdgcn_mov_dpp((int)(uint32_t)key, CTRL, 0xf, 0xf, false);
  const uint32_t hi = __builtin_amdgcn_mov_dpp((int)(uint32_t)(key >> 32), CTRL, 0xf, 0xf, false);
  const uint64_t o = ((uint64_t)hi << 32) | lo;
  key = o > key ? o : key;
}
template <int G>
__device__ __forceinline__ void group_max_key(uint64_t& key) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8, "group size");
  if constexpr (G >= 2) dpp_max_step<0xb1>(key);    // quad_perm [1,0,3,2]
  if constexpr (G >= 4) dpp_max_step<0x4e>(key);    // quad_perm [2,3,0,1]
  if constexpr (G >= 8) dpp_max_step<0x141>(key);   // row_half_mirror
}
// Sum over the same lane groups (every lane ends with the group's sum).
template <int CTRL>
__device__ __forceinline__ void dpp_add_step(float& v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
// Sum over each half-wave (lanes 0-31, 32-63), left in lanes 31 and 63: DPP
// butterflies within 16-lane rows (xor 1, xor 2, half-row and row mirrors), then
// row_bcast:15 adds row 0's (row 2's) lane 15 into row 1 (row 3).
__device__ __forceinline__ float half_wave_sum(float v) {
  dpp_add_step<0xb1>(v);    // quad_perm [1,0,3,2]
  dpp_add_step<0x4e>(v);    // quad_perm [2,3,0,1]
  dpp_add_step<0x141>(v);   // row_half_mirror
  dpp_add_step<0x140>(v);   // row_mirror
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, false));
}
// Over all 64 lanes (every lane active), the result in every lane: the 16-lane
// DPP butterflies above, then the four rows' results (lanes 0, 16, 32, 48) read
// into scalars and combined in row order. VALU and scalar reads only: no LDS
// round trips, which a chain of __shfl_xor steps costs at each step.
__device__ __forceinline__ float wave_sum(float v) {
  dpp_add_step<0xb1>(v);    // quad_perm [1,0,3,2]
  dpp_add_step<0x4e>(v);    // quad_perm [2,3,0,1]
  dpp_add_step<0x141>(v);   // row_half_mirror
  dpp_add_step<0x140>(v);   // row_mirror
  const int b = __float_as_int(v);
  return (__int_as_float(__builtin_amdgcn_readlane(b, 0)) +
          __int_as_float(__builtin_amdgcn_readlane(b, 16))) +
         (__int_as_float(__builtin_amdgcn_readlane(b, 32)) +
          __int_as_float(__builtin_amdgcn_readlane(b, 48)));
}
__device__ __forceinline__ uint64_t wave_max_key(uint64_t key) {
  dpp_max_step<0xb1>(key);
  dpp_max_step<0x4e>(key);
  dpp_max_step<0x141>(key);
  dpp_max_step<0x140>(key);   // row_mirror: lane i with 15 - i
  uint64_t best = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key, 16 * r);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(key >> 32), 16 * r);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    best = o > best ? o : best;
  }
  return best;
}
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ int lane_value(int v, int lane) {
  return __builtin_amdgcn_readlane(v, lane);
}
template <int G>
__device__ __forceinline__ void group_sum(float& v) {
  if constexpr (G >= 2) dpp_add_step<0xb1>(v);
  if constexpr (G >= 4) dpp_add_step<0x4e>(v);
  if constexpr (G >= 8) dpp_add_step<0x141>(v);
}

// Router score of the trained-checkpoint mode (router_mode 1): the logit capped
// as scale * tanh(x / scale), tanh(u) taken as 2 sigmoid(2u) - 1, then divided
// by the temperature (mamba3_mlx/mlx_model/ops.py:9-14,
// mamba3_mlx/mlx_model/tucker_moe.py:107-109).
__device__ __forceinline__ float capped_score(float raw, float scale, float temperature) {
  const float u = raw * (1.f / scale);
  const float sg = 1.f / (1.f + expf(-2.f * u));
  return ((2.f * sg - 1.f) * scale) / temperature;
}
// Weight of selected slot kk. router_mode 0 (model.py:77): softmax over the k
// selected logits, ex_kk / sum_j ex_j. router_mode 1 (tucker_moe.py:110-114):
// softmax over all E, p_kk = ex_kk / sum_all, renormalised over the selected as
// p_kk / (sum_j p_j + 1e-6). ex = exp(score - max score) throughout.
__device__ __forceinline__ float slot_weight(int mode, const float* ex, int K, int kk,
                                             float sum_top, float sum_all) {
  if (mode == 0) return ex[kk] / sum_top;
  float ps = 0.f;
  for (int j = 0; j < K; ++j) ps += ex[j] / sum_all;
  return (ex[kk] / sum_all) / (ps + 1e-6f);
}

template <class Elt, int FM, int NR, int NW>
struct RouterExtra {
  static constexpr bool kSplitK = NR < NW;
  static constexpr int RT = kSplitK ? NR : NR / NW;   // router column blocks per wave
  static_assert(kSplitK || NR % NW == 0, "router split");
  f32x16 racc[FM][RT];
  int wave, lane, brow0;   // brow0: LDS row of router column 0
  __device__ __forceinline__ void init(int w, int l, int r0) {
    // wave-uniform in a scalar register: the K-step test below is then a scalar
    // branch around the MFMAs (they would run with an empty EXEC mask too)
    wave = __builtin_amdgcn_readfirstlane(w);
    lane = l;
    brow0 = r0;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < RT; ++j) racc[i][j] = zero16();
  }
  struct Frag {
    u32x4 b[RT];
  };
  __device__ __forceinline__ void load(Frag& f, const u32x4* s, int kstep, int ch) const {
    if (kSplitK && (kstep % NW) != wave) return;
#pragma unroll
    for (int j = 0; j < RT; ++j) {
      const int col0 = (kSplitK ? j : wave * RT + j) * 32;
      f.b[j] = s[lds_slot(brow0 + col0 + (lane & 31), ch)];
    }
  }
  template <class AF>
  __device__ __forceinline__ void compute(const Frag& f, int kstep, const AF& af) {
    if (kSplitK && (kstep % NW) != wave) return;
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
      for (int i = 0; i < FM; ++i) mma(racc[i][j], af[i], f.b[j], Elt{});
  }
  template <class ACC>
  __device__ __forceinline__ void tile_begin(int, ACC&) const {}
};

// z = RMSNorm(x U_in) * g for the BM rows of a front tile (model.py:80-81, :25-27):
// fp8 column scales, the row sums of squares (lane shuffles, then the waves'
// partial sums in wave order by one thread per row), z / rms as z * (1 / rms)
// (within one fp32 rounding of the division), staged in LDS at zst and written as
// 16-byte chunks. red: LDS for [NW][BM] partial sums followed by [BM] 1 / rms.
// Called by every thread of the work-group.
template <class TL, class Elt, int R3>
__device__ __forceinline__ void front_z_epilogue(f32x16 (&acc)[TL::FM][TL::FN], const FwdArgs& a,
                                                 int64_t m0, int rows_valid, char* zst,
                                                 float* red) {
  typedef typename Elt::T T;
  constexpr int FM = TL::FM, NW = TL::WN, BM = TL::BM;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wn = wave % NW, wrow = (wave / NW) * TL::kWaveM;
  // -- fp8 weights: z column j = (x . q_in[:, j]) * s_in[j] ----------------
  if (a.zscale) {
#pragma unroll
    for (int j = 0; j < TL::FN; ++j) {
      const float sc = a.zscale[wn * TL::kWaveN + j * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] *= sc;
    }
  }

  // -- RMSNorm row sums of squares ------------------------------------------
  // the 32 lanes of each half-wave hold the same rows; their sum lands in lanes
  // 31 and 63
  float ss[FM][16];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float v = 0.f;
#pragma unroll
      for (int j = 0; j < TL::FN; ++j) v += acc[i][j][e] * acc[i][j][e];
      ss[i][e] = half_wave_sum(v);
    }
  if ((lane & 31) == 31) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) red[wn * BM + wrow + i * 32 + acc_row(lane, e)] = ss[i][e];
  }
  __syncthreads();
  // one thread per row: the waves' partial sums in wave order, then 1 / rms
  float* inv = red + NW * BM;   // [BM]
  if (threadIdx.x < BM) {
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += red[w * BM + threadIdx.x];
    inv[threadIdx.x] = 1.f / sqrtf(tot / (float)R3 + a.eps);
  }
  __syncthreads();

  // -- z = (z / rms) * g, staged in LDS then written as 16-byte chunks ----------
  {
    constexpr int RB = TileStage<TL, T>::kRowBytes;
    float gcol[TL::FN];
#pragma unroll
    for (int j = 0; j < TL::FN; ++j) gcol[j] = a.gain[wn * TL::kWaveN + j * 32 + (lane & 31)];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = wrow + i * 32 + acc_row(lane, e);
        const float inv_rms = inv[row];
#pragma unroll
        for (int j = 0; j < TL::FN; ++j) {
          const int col = wn * TL::kWaveN + j * 32 + (lane & 31);
          store_from_f32(reinterpret_cast<T*>(zst + row * RB + col * (int)sizeof(T)),
                         (acc[i][j][e] * inv_rms) * gcol[j]);
        }
      }
  }
  __syncthreads();
  // a front that writes c (x) z keeps the staged tile for that and stores no z
  if (!a.cz) flush_tile<TL, T>(zst, reinterpret_cast<T*>(a.z) + m0 * R3, R3, rows_valid, R3);
}

// Folded plans: the Khatri-Rao rows of a front tile, cz[t][r R3 + s] = R(c[t][r] z[t][s]),
// from the staged bf16 z tile (TileStage layout) and c (rows x rk floats in LDS), in
// 16-byte chunks that run contiguously through the tile's rows of cz. Regular
// (cached) stores: the out-projection reads them next.
template <class TL, int R3>
__device__ __forceinline__ void flush_cz(const char* zst, const float* cl, const FwdArgs& a,
                                         int64_t m0, int rows_valid) {
  constexpr int RB = TileStage<TL, uint16_t>::kRowBytes;
  constexpr int CPR = R3 * 2 / 16;   // z chunks per row
  const int rk = (int)a.r1;
  uint16_t* dst = static_cast<uint16_t*>(a.cz) + m0 * rk * R3;
  const int n = rows_valid * rk * CPR;
  for (int q = threadIdx.x; q < n; q += TL::kThreads) {
    const int ch = q % CPR, rr = q / CPR, row = rr / rk;
    const u32x4 zv = *reinterpret_cast<const u32x4*>(zst + row * RB + ch * 16);
    const float cr = cl[rr];   // rr = row * rk + r
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack_bf16x2(bf16_bits_to_f32(zv[j] & 0xffffu) * cr, bf16_bits_to_f32(zv[j] >> 16) * cr);
    *reinterpret_cast<u32x4*>(dst + (int64_t)rr * R3 + ch * 8) = o;
  }
}

// LDS floats of front_topk's per-row record: exp weights, indices and final
// weights of the k rounds, the sum over the selected and the sum over all E.
template <int BM>
constexpr int kTopkRecFloats = BM * (3 * kMaxTopK + 2);

// Top-k, softmax and c for the BM rows of a front tile whose logits are in LDS
// (model.py:76-77, :93): NP planes of [BM][LD] floats, a logit being the sum of
// its planes in plane order. rec: kTopkRecFloats<BM> floats of LDS followed by
// ue_bytes for U_expert. Called by every one of the NT threads of the work-group.
// A row is resolved by a group of G lanes (1 to 8; as many as fill the
// work-group, and at least EP / 32) holding EP / G <= 32 logits each (columns
// gl, gl + G, ...): K rounds of a serial arg-max over the lane's logits and a
// DPP arg-max over the group, with no LDS traffic in the rounds. Round kk's
// exp(v - v_max) and index go to LDS; then the softmax weights and c are
// formed in parallel over (row, round) and (row, r). U_expert is read from
// LDS when it fits in ue_bytes.
template <int EP, int BM, int NT, int NP>
__device__ __forceinline__ void front_topk(const FwdArgs& a, int64_t m0, int rows_valid,
                                           const float* lg, int LD, float* rec, int ue_bytes,
                                           float* c_lds = nullptr) {
  constexpr int NWT = NT / 64;
  constexpr int kFill = NT / BM;
  constexpr int G = cmin(8, cmax(EP / 32, kFill < 1 ? 1 : kFill));
  constexpr int PL = EP / G;          // logits per lane
  static_assert(PL <= 32 && EP % G == 0, "taken-mask width");
  constexpr int RPW = 64 / G;         // rows per wave per pass
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int E = (int)a.E, K = (int)a.k, R1 = (int)a.r1;
  float* rec_ex = rec;                                              // [BM][kMaxTopK]
  int* rec_i = reinterpret_cast<int*>(rec_ex + BM * kMaxTopK);      // [BM][kMaxTopK]
  float* rec_w = reinterpret_cast<float*>(rec_i + BM * kMaxTopK);   // [BM][kMaxTopK]
  float* rec_sum = rec_w + BM * kMaxTopK;         // [BM] over the selected
  float* rec_all = rec_sum + BM;                  // [BM] over all E (router_mode 1)
  float* ue = rec_all + BM;
  const int mode = a.router_mode;
  const bool ue_lds = E * R1 * 4 <= ue_bytes;
  if (ue_lds) {
    // four loads in flight per thread before their stores (a load-store loop waited
    // for each load in turn)
    constexpr int U = 4;
    for (int i0 = threadIdx.x; i0 < E * R1; i0 += U * NT) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = i0 + u * NT < E * R1 ? a.uexp[i0 + u * NT] : 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (i0 + u * NT < E * R1) ue[i0 + u * NT] = v[u];
    }
  }
  const float* uex = ue_lds ? ue : a.uexp;
  const int gl = lane % G;
  for (int row0 = wave * RPW; row0 < BM; row0 += NWT * RPW) {
    const int row_raw = row0 + lane / G;
    const bool inb = row_raw < BM;
    const int row = inb ? row_raw : BM - 1;   // lanes past the tile repeat its last row
    const bool live = inb && row < rows_valid;
    const int64_t g = m0 + row;
    uint64_t key[PL];   // 0 for columns past E
    float sv[PL];       // the scores the keys rank (router_mode 1: capped ones)
    // every logit read before any is stored (a store behind a branch between the
    // reads made each read wait for the one before)
#pragma unroll
    for (int p = 0; p < PL; ++p) {
      const int col = gl + G * p;
      float sc = 0.f;
#pragma unroll
      for (int w = 0; w < NP; ++w) sc += lg[(w * BM + row) * LD + col];
      sv[p] = sc;
    }
    if (a.logits && live) {
#pragma unroll
      for (int p = 0; p < PL; ++p)
        if (gl + G * p < E) a.logits[g * E + gl + G * p] = sv[p];
    }
    // a branch on the uniform mode: selected per key, the capped score's exp and
    // divisions ran for every key in mode 0 as well
    if (mode) {
#pragma unroll
      for (int p = 0; p < PL; ++p) sv[p] = capped_score(sv[p], a.router_scale, a.router_temperature);
    }
#pragma unroll
    for (int p = 0; p < PL; ++p) key[p] = gl + G * p < E ? rank_key(sv[p], gl + G * p) : 0;
    float vmax = 0.f, ssum = 0.f;
    // round kk takes the largest key below the one round kk - 1 took (keys are
    // distinct: they hold the column), so no key is cleared between the rounds
    uint64_t prev = 0;
#pragma unroll 1
    for (int kk = 0; kk < K; ++kk) {
      uint64_t best = 0;
      if (kk == 0) {
#pragma unroll
        for (int p = 0; p < PL; ++p) best = key[p] > best ? key[p] : best;
      } else {
#pragma unroll
        for (int p = 0; p < PL; ++p) best = key[p] < prev && key[p] > best ? key[p] : best;
      }
      group_max_key<G>(best);
      prev = best;
      // k <= E, so a candidate always remains: best > 0 and its index is < E
      const int bi = key_index(best);
      const float bv = key_value(best);
      if (kk == 0) vmax = bv;   // the largest
      const float ex = expf(bv - vmax);
      ssum += ex;
      if (gl == 0 && inb) {
        rec_ex[row * kMaxTopK + kk] = ex;
        rec_i[row * kMaxTopK + kk] = bi;
      }
    }
    if (mode) {   // softmax denominator over all E
      float sa = 0.f;
#pragma unroll
      for (int p = 0; p < PL; ++p) sa += gl + G * p < E ? expf(sv[p] - vmax) : 0.f;
      group_sum<G>(sa);
      if (gl == 0 && inb) rec_all[row] = sa;
    }
    if (gl == 0 && inb) rec_sum[row] = ssum;
  }
  __syncthreads();
  // routing weights (model.py:77) and c = sum_j w_j U_expert[e_j] (model.py:93)
  for (int q = threadIdx.x; q < rows_valid * K; q += NT) {
    const int row = q / K, kk = q - row * K;
    const float wk = slot_weight(mode, rec_ex + row * kMaxTopK, K, kk, rec_sum[row],
                                 mode ? rec_all[row] : 0.f);
    a.idx[(m0 + row) * K + kk] = rec_i[row * kMaxTopK + kk];
    a.w[(m0 + row) * K + kk] = wk;
    rec_w[row * kMaxTopK + kk] = wk;
  }
  __syncthreads();
  for (int q = threadIdx.x; q < rows_valid * R1; q += NT) {
    const int row = q / R1, r = q - row * R1;
    float cr = 0.f;
    for (int kk = 0; kk < K; ++kk)
      cr += rec_w[row * kMaxTopK + kk] * uex[rec_i[row * kMaxTopK + kk] * R1 + r];
    a.c[(m0 + row) * R1 + r] = cr;
    if (c_lds) c_lds[q] = cr;   // q = row * R1 + r
  }
}

// The front of token tile `tile` (rows tile * BM ..) of the layer `a`: k_front's body.
template <class Elt, int R3, int NR, int PFA, int BM, int NS, int WMF>
__device__ __forceinline__ void front_tile(const FwdArgs& a, int tile) {
  typedef typename Elt::T T;
  constexpr int EP = 32 * NR;
  constexpr int NW = R3 / 32 < 4 ? R3 / 32 : 4;   // waves across the z columns
  constexpr int NWT = NW * WMF;                      // all waves (WMF row groups)
  // x (streamed from HBM once) and the weight rows (from L2, shared by the WMF row
  // groups) both go to LDS by DMA from every wave. With x through half of the
  // waves' register ring (PFA K tiles ahead) and the weights by the other half's
  // DMA the launch took longer, bit-identical: 26.6-26.7 against 24.4-25.0 us at
  // the C3 shapes, T = 6144 (32-token tiles).
  typedef Tile<BM, R3, EP, WMF, NW, PFA, 1, NS, true, true, 0> TL;
  constexpr int FM = TL::FM;   // a wave covers the BM / WMF rows of its group
  typedef RouterExtra<Elt, FM, NR, NW> RX;
  // epilogue LDS: staged z tile, then the logits plane(s), then RMSNorm partials
  // and 1 / rms, then the top-k record
  constexpr int LD = EP + 1;
  constexpr int kPlanes = RX::kSplitK ? NW : 1;
  constexpr int kZBytes = TileStage<TL, T>::kBytes;
  constexpr int kEpiBytes = kZBytes + (kPlanes * BM * LD + NW * BM + BM + kTopkRecFloats<BM>) * 4;
  // U_expert is staged after that: at least 4 KB (E = 256, r1 = 4) of room
  constexpr int kSmemBytes = cmax(TL::kLdsBytes, kEpiBytes + 4096);
  __shared__ u32x4 smem[kSmemBytes / 16];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wn = wave % NW, wrow = (wave / NW) * TL::kWaveM;   // column wave, first row
  const int64_t m0 = (int64_t)tile * BM;
  const int rows_valid = (int)(a.T - m0 < BM ? a.T - m0 : BM);
  const int64_t row_bytes = a.d_in * (int64_t)sizeof(T);
  RowLoader al{reinterpret_cast<const char*>(a.x) + m0 * row_bytes, row_bytes, rows_valid};
  RowLoader bl{reinterpret_cast<const char*>(a.wfront), row_bytes, R3 + EP};
  f32x16 acc[FM][TL::FN];
  RX rx;
  rx.init(wn, lane, BM + R3);
  gemm_mainloop<TL, Elt>(acc, al, bl, (int)(row_bytes / kTileKBytes), smem, rx);

  // -- router logits -> LDS, [BM][EP + 1] (split-K: one partial plane per wave) --
  char* zst = reinterpret_cast<char*>(smem);
  float* lg = reinterpret_cast<float*>(zst + kZBytes);
  float* red = lg + kPlanes * BM * LD;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < RX::RT; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = wrow + i * 32 + acc_row(lane, e);
        if constexpr (RX::kSplitK)
          lg[(wn * BM + row) * LD + j * 32 + (lane & 31)] = rx.racc[i][j][e];
        else
          lg[row * LD + (wn * RX::RT + j) * 32 + (lane & 31)] = rx.racc[i][j][e];
      }
  front_z_epilogue<TL, Elt, R3>(acc, a, m0, rows_valid, zst, red);
  // c goes to LDS over the logits (read before the top-k record is complete) when
  // the tile also writes c (x) z: BM x r1 <= BM x (EP + 1) floats
  front_topk<EP, BM, TL::kThreads, kPlanes>(a, m0, rows_valid, lg, LD, red + NW * BM + BM,
                                            kSmemBytes - kEpiBytes, a.cz ? lg : nullptr);
  if constexpr (std::is_same<Elt, EltBF16>::value) {
    if (a.cz) {
      __syncthreads();
      flush_cz<TL, R3>(zst, lg, a, m0, rows_valid);
    }
  }
}

template <class Elt, int R3, int NR, int PFA = kFrontPFA, int BM = kFrontBM, int NS = 2,
          int WMF = kFrontWM>
__global__ __launch_bounds__(64 * WMF * (R3 / 32 < 4 ? R3 / 32 : 4)) void k_front(FwdArgs a) {
  front_tile<Elt, R3, NR, PFA, BM, NS, WMF>(a, (int)blockIdx.x);
}

// The fronts of two layers with one input (TransformerBlock's ffn_gate and ffn_up,
// model.py:338-339) in one launch: work-groups 0 .. ntiles - 1 run a0's token
// tiles, the next ntiles a1's, so the two run side by side on the compute units.
template <class Elt, int R3, int NR, int PFA, int BM, int NS, int WMF>
__global__ __launch_bounds__(64 * WMF * (R3 / 32 < 4 ? R3 / 32 : 4)) void k_front_pair(
    FwdArgs a0, FwdArgs a1, int ntiles) {
  const bool second = (int)blockIdx.x >= ntiles;   // uniform over the work-group
  front_tile<Elt, R3, NR, PFA, BM, NS, WMF>(second ? a1 : a0,
                                            (int)blockIdx.x - (second ? ntiles : 0));
}

// The front in K slices, for token counts whose 64-token tiles leave most compute
// units idle while K = d_in is long: work-group (tile, slice) computes the slice's
// share of x [U_in | W_r^T] with k_front's main loop and writes it as fp32 to raw
// plane `slice` (T rows of r3 + E floats); k_front_epi then adds the planes in
// plane order and runs the per-token epilogue (RMSNorm, top-k, softmax, c).
// Both operands go to LDS by DMA, issued by every wave (a slice is 3-8 K tiles: the
// whole slice is in flight after the first tiles' issue). With x through four
// waves' register ring and the weights by the other four waves' DMA (k_front's
// scheme) the slices took longer, bit-identical: at the C3 shapes k_front_sliced
// 23.4 -> 20.8 us at T = 4096 and 21.3 -> 19.5 us at T = 3001, k_front_part 12.0 ->
// 11.1 us and the one-launch k_fused_mid 30.6 -> 29.3 us at T = 2048.
template <class Elt, int R3, int NR, int PFA = kFrontPFA, int BM = kFrontBM, int NS = 2,
          int WMF = kFrontWM>
struct FrontPartGeom {
  static constexpr int EP = 32 * NR;
  static constexpr int NW = R3 / 32 < 4 ? R3 / 32 : 4;
  static constexpr int NWT = NW * WMF;
  typedef Tile<BM, R3, EP, WMF, NW, PFA, 1, NS, true, true, 0> TL;
  typedef RouterExtra<Elt, TL::FM, NR, NW> RX;
  static constexpr int LD = EP + 1;
  static constexpr int kPlanes = RX::kSplitK ? NW : 1;
  static constexpr int kSmemBytes = cmax(TL::kLdsBytes, kPlanes * BM * LD * 4);
};

// K slice `sl` of nslices of front tile `tile` (the work of one k_front_part
// work-group): smem holds FrontPartGeom::kSmemBytes of LDS.
template <class Elt, int R3, int NR, int PFA, int BM, int NS, int WMF>
__device__ __forceinline__ void front_part_tile(const FwdArgs& a, float* __restrict__ raw,
                                                int nslices, int tile, int sl, u32x4* smem) {
  typedef typename Elt::T T;
  typedef FrontPartGeom<Elt, R3, NR, PFA, BM, NS, WMF> G;
  constexpr int EP = G::EP, NW = G::NW, LD = G::LD, kPlanes = G::kPlanes;
  typedef typename G::TL TL;
  typedef typename G::RX RX;
  constexpr int FM = TL::FM;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wn = wave % NW, wrow = (wave / NW) * TL::kWaveM;
  const int64_t m0 = (int64_t)tile * BM;
  const int rows_valid = (int)(a.T - m0 < BM ? a.T - m0 : BM);
  const int64_t row_bytes = a.d_in * (int64_t)sizeof(T);
  const int nkt = (int)(row_bytes / kTileKBytes);
  const int kt0 = sl * nkt / nslices, kt1 = (sl + 1) * nkt / nslices;
  RowLoader al{reinterpret_cast<const char*>(a.x) + m0 * row_bytes + (int64_t)kt0 * kTileKBytes,
               row_bytes, rows_valid};
  RowLoader bl{reinterpret_cast<const char*>(a.wfront) + (int64_t)kt0 * kTileKBytes, row_bytes,
               R3 + EP};
  f32x16 acc[FM][TL::FN];
  RX rx;
  rx.init(wn, lane, BM + R3);
  gemm_mainloop<TL, Elt>(acc, al, bl, kt1 - kt0, smem, rx);

  const int W = (int)raw_stride(R3, a.E);
  float* plane = raw + (int64_t)sl * a.T * W + m0 * W;
  // z columns through LDS (rows of R3 + 4 floats), then out as 16-byte row chunks
  // (the accumulators give a lane one column of 16 rows: 4-byte stores)
  constexpr int ZL = R3 + 4;
  static_assert(BM * ZL * 4 <= G::kSmemBytes, "the z tile fits the LDS");
  float* zt = reinterpret_cast<float*>(smem);
  __syncthreads();   // the main loop's last LDS reads are done
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < TL::FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = wrow + i * 32 + acc_row(lane, e);
        zt[row * ZL + wn * TL::kWaveN + j * 32 + (lane & 31)] = acc[i][j][e];
      }
  __syncthreads();
  for (int idx = threadIdx.x; idx < rows_valid * (R3 / 4); idx += TL::kThreads) {
    const int row = idx / (R3 / 4), c4 = idx - row * (R3 / 4);
    *reinterpret_cast<float4*>(plane + (int64_t)row * W + 4 * c4) =
        *reinterpret_cast<const float4*>(zt + row * ZL + 4 * c4);
  }
  // router columns: through LDS (split-K router: one partial plane per wave, added
  // in wave order), the first E of them
  __syncthreads();
  float* lg = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < RX::RT; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = wrow + i * 32 + acc_row(lane, e);
        if constexpr (RX::kSplitK)
          lg[(wn * BM + row) * LD + j * 32 + (lane & 31)] = rx.racc[i][j][e];
        else
          lg[row * LD + (wn * RX::RT + j) * 32 + (lane & 31)] = rx.racc[i][j][e];
      }
  __syncthreads();
  const int E = (int)a.E;
  for (int idx = threadIdx.x; idx < BM * E; idx += TL::kThreads) {
    const int row = idx / E, c = idx - row * E;
    if (row < rows_valid) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kPlanes; ++w) v += lg[(w * BM + row) * LD + c];
      plane[(int64_t)row * W + R3 + c] = v;
    }
  }
}

template <class Elt, int R3, int NR, int PFA = kFrontPFA, int BM = kFrontBM, int NS = 2,
          int WMF = kFrontWM>
__global__ __launch_bounds__(64 * WMF * (R3 / 32 < 4 ? R3 / 32 : 4)) void k_front_part(
    FwdArgs a, float* __restrict__ raw, int nslices) {
  typedef FrontPartGeom<Elt, R3, NR, PFA, BM, NS, WMF> G;
  __shared__ u32x4 smem[G::kSmemBytes / 16];
  front_part_tile<Elt, R3, NR, PFA, BM, NS, WMF>(a, raw, nslices, (int)blockIdx.x,
                                                 (int)blockIdx.y, smem);
}

// The front for wide routers (E_pad = 32 NR > 128 with r3 = R3 = 256), in two kinds
// of work-group over 32-token tiles: the first ceil(T / 32) compute the logits (x
// against the router rows, top-k, softmax, c), the others z (x against U_in^T,
// RMSNorm). Splitting them doubles the work-groups (128 of the single kind at T =
// 4096 left half of 256 CUs idle) and halves the weight rows each streams. 4 waves
// each, wave tile 32 x (columns / 4). Folded plans (a.cz set): router work-group tm
// hands its tile's c to z work-group tm through sync flag tm (device-scope stores
// and loads, sync_publish / sync_await), which then writes the tile's c (x) z rows
// from its staged z in place of z (the separate k_expand_cz pass it replaces took
// 6-8 us at T = 4096).
template <class Elt, int R3, int NR, int PFA, int NS>
__global__ __launch_bounds__(256) void k_front_split(FwdArgs a) {
  typedef typename Elt::T T;
  constexpr int BM = 32, EP = 32 * NR, NW = 4;
  static_assert(R3 == 256 && EP >= 128, "split front: r3 = 256, E_pad >= 128");
  // x and the weight rows both by LDS DMA from every wave (with x through two waves'
  // register ring and the weights by the other two's DMA the launch took 26.9-27.1
  // against 22.8-22.9 us at C4, bit-identical)
  typedef Tile<BM, R3, 0, 1, NW, PFA, 1, NS, true, true, 0> TLZ;
  typedef Tile<BM, EP, 0, 1, NW, PFA, 1, NS, true, true, 0> TLR;
  constexpr int LD = EP + 1;
  constexpr int kZEpi = TileStage<TLZ, T>::kBytes + (NW * BM + BM) * 4;
  constexpr int kREpi = (BM * LD + kTopkRecFloats<BM>) * 4;
  constexpr int kUe = 4096;   // U_expert (E = 256, r1 = 4) when it fits
  constexpr int kCRows = BM * 32 * 4 + 16;   // c rows of the tile (r1 <= 32), a flag word
  constexpr int kSmemBytes =
      cmax(cmax(TLZ::kLdsBytes, TLR::kLdsBytes), cmax(kZEpi + kCRows, kREpi + kUe));
  __shared__ u32x4 smem[kSmemBytes / 16];

  const int ntm = (int)((a.T + BM - 1) / BM);
  // router work-groups first: with a.cz set, z work-group tm waits for router
  // work-group tm's c (sync flag tm) and writes the tile's c (x) z rows itself
  const bool zpart = (int)blockIdx.x >= ntm;   // uniform over the work-group
  const int tm = zpart ? (int)blockIdx.x - ntm : (int)blockIdx.x;
  const int64_t m0 = (int64_t)tm * BM;
  const int rows_valid = (int)(a.T - m0 < BM ? a.T - m0 : BM);
  const int64_t row_bytes = a.d_in * (int64_t)sizeof(T);
  const int nkt = (int)(row_bytes / kTileKBytes);
  RowLoader al{reinterpret_cast<const char*>(a.x) + m0 * row_bytes, row_bytes, rows_valid};
  NoExtra nx;
  if (zpart) {
    RowLoader bl{reinterpret_cast<const char*>(a.wfront), row_bytes, R3};
    f32x16 acc[TLZ::FM][TLZ::FN];
    gemm_mainloop<TLZ, Elt>(acc, al, bl, nkt, smem, nx);
    char* zst = reinterpret_cast<char*>(smem);
    front_z_epilogue<TLZ, Elt, R3>(acc, a, m0, rows_valid, zst,
                                   reinterpret_cast<float*>(zst + TileStage<TLZ, T>::kBytes));
    if constexpr (std::is_same<Elt, EltBF16>::value) {
      if (a.cz) {
        // c of the tile's rows from the router work-group, into LDS after the
        // RMSNorm partials; NaN when the wait ran out of time
        float* cl = reinterpret_cast<float*>(zst + kZEpi);
        const bool ok = sync_await(a.sync + sync_flag(tm), 1, a.epoch, a.sync,
                                   reinterpret_cast<int*>(cl + BM * 32), true, a.wait_polls,
                                   a.status);
        const int n = rows_valid * (int)a.r1;
        for (int q = threadIdx.x; q < n; q += TLZ::kThreads)
          cl[q] = ok ? load_coherent(a.c + m0 * a.r1 + q) : __builtin_nanf("");
        __syncthreads();
        flush_cz<TLZ, R3>(zst, cl, a, m0, rows_valid);
      }
    }
  } else {
    RowLoader bl{reinterpret_cast<const char*>(a.wfront) + R3 * row_bytes, row_bytes, EP};
    f32x16 acc[TLR::FM][TLR::FN];
    gemm_mainloop<TLR, Elt>(acc, al, bl, nkt, smem, nx);
    const int lane = threadIdx.x & 63, wn = (threadIdx.x >> 6) % NW;
    float* lg = reinterpret_cast<float*>(smem);   // [BM][LD]
#pragma unroll
    for (int i = 0; i < TLR::FM; ++i)
#pragma unroll
      for (int j = 0; j < TLR::FN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          lg[(i * 32 + acc_row(lane, e)) * LD + wn * TLR::kWaveN + j * 32 + (lane & 31)] =
              acc[i][j][e];
    __syncthreads();
    // c also into LDS over the logits (read before the top-k record is complete)
    front_topk<EP, BM, TLR::kThreads, 1>(a, m0, rows_valid, lg, LD, lg + BM * LD,
                                         kSmemBytes - kREpi, a.cz ? lg : nullptr);
    if (a.cz) {   // c of the tile's rows for z work-group tm, device-scope
      __syncthreads();
      const int n = rows_valid * (int)a.r1;
      for (int q = threadIdx.x; q < n; q += TLR::kThreads) store_coherent(a.c + m0 * a.r1 + q, lg[q]);
      sync_publish(a.sync + sync_flag(tm), a.epoch);
    }
  }
}

// ---- k_core: mid = (c (x) z) core_flat  (model.py:87-98) ------------------
// A (c (x) z) is formed in registers on its way to LDS (a ring of PFA tiles);
// B (core^T) arrives by DMA.
// fp8 core weights G[r, s, q] = g[r, s, q] * sc[r, q] (per output channel (r, q)).
// The K tiles of rank r (tiles_per_r consecutive ones) accumulate
// sum_s A[t, (r, s)] g[r, s, q] unscaled; entering rank r + 1 the accumulator is
// multiplied by cs[r, q] = sc[r, q] / sc[r + 1, q], and the epilogue multiplies by
// cs[r1 - 1, q] = sc[r1 - 1, q], which leaves sum_r sc[r, q] * (rank r's sum).
// The ratios of the next rank change are loaded one change ahead; columns at or
// past r2 (a partial last tile) read nothing and keep factor 1.
template <int FM, int FN>
struct CoreRescale {
  const float* cs;   // (r1, r2) as above
  int tiles_per_r, r1, r2;
  int colbase;       // this lane's column of block j is colbase + 32 j
  float nxt[FN];
  __device__ __forceinline__ void init(const float* cs_, int tpr, int r1_, int r2_, int col0) {
    cs = cs_;
    tiles_per_r = tpr;
    r1 = r1_;
    r2 = r2_;
    colbase = col0;
#pragma unroll
    for (int j = 0; j < FN; ++j)
      nxt[j] = (cs && r1 > 1 && colbase + 32 * j < r2) ? cs[colbase + 32 * j] : 1.f;
  }
  struct Frag {};
  __device__ __forceinline__ void load(Frag&, const u32x4*, int, int) const {}
  template <class AF>
  __device__ __forceinline__ void compute(const Frag&, int, const AF&) const {}
  template <class ACC>
  __device__ __forceinline__ void tile_begin(int kt, ACC& acc) {
    if (!cs || kt == 0 || kt % tiles_per_r != 0) return;
    const int r = kt / tiles_per_r;   // entering rank r >= 1: multiply by cs[r - 1, :]
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const float f = nxt[j];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] *= f;
    }
    if (r + 1 < r1) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
        if (colbase + 32 * j < r2) nxt[j] = cs[(int64_t)r * r2 + colbase + 32 * j];
    }
  }
};

template <class Elt, int BM, int BN, int WM, int WN, int PFA>
__global__ __launch_bounds__(64 * WM * WN) void k_core(FwdArgs a) {
  typedef typename Elt::T T;
  // half of the waves form c (x) z through the register ring, the other half
  // issue the core^T DMA
  typedef Tile<BM, BN, 0, WM, WN, PFA, 1, 2, false, true, WM * WN / 2> TL;
  __shared__ u32x4 smem[cmax(TL::kLdsBytes, TileStage<TL, T>::kBytes) / 16];

  const int ntn = (int)((a.r2 + BN - 1) / BN);
  const int ntm = (int)((a.T + BM - 1) / BM);
  int tm, tn;
  tile_coords(ntn, ntm * ntn, tm, tn);
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t n0 = (int64_t)tn * BN;
  const int rows_valid = (int)(a.T - m0 < BM ? a.T - m0 : BM);
  const int64_t K = a.r1 * a.r3;
  const int64_t b_row_bytes = K * (int64_t)sizeof(T);
  KhatriRaoLoader<Elt> al{reinterpret_cast<const char*>(a.z) + m0 * a.r3 * (int64_t)sizeof(T),
                          a.c + m0 * a.r1, (int)a.r1, (int)a.r3, rows_valid};
  RowLoader bl{reinterpret_cast<const char*>(a.coreT) + n0 * b_row_bytes, b_row_bytes,
               (int)(a.r2 - n0)};
  f32x16 acc[TL::FM][TL::FN];
  const int wn = (threadIdx.x >> 6) % WN, lane = threadIdx.x & 63;
  const int col0 = wn * TL::kWaveN + (lane & 31);   // column of block j: col0 + 32 j
  CoreRescale<TL::FM, TL::FN> rs;
  rs.init(a.core_scale, (int)(a.r3 * (int64_t)sizeof(T) / kTileKBytes), (int)a.r1, (int)a.r2,
          (int)n0 + col0);
  gemm_mainloop<TL, Elt>(acc, al, bl, (int)(b_row_bytes / kTileKBytes), smem, rs);

  char* stage = reinterpret_cast<char*>(smem);
  float zero[TL::FN], last[TL::FN];
#pragma unroll
  for (int j = 0; j < TL::FN; ++j) {
    zero[j] = 0.f;
    const int col = col0 + 32 * j;
    last[j] = a.core_scale && col < a.r2 - n0
                  ? a.core_scale[(a.r1 - 1) * a.r2 + n0 + col] : 1.f;
  }
  stage_tile<TL, T>(acc, stage, zero, last);
  __syncthreads();
  flush_tile<TL, T>(stage, reinterpret_cast<T*>(a.mid) + m0 * a.r2 + n0, a.r2, rows_valid,
                    (int)(a.r2 - n0));
}

// ---- k_core_pp: mid = sum_r c_r (z P_r), persistent ping-pong  (model.py:87-98)
// The north star's form of the core: one GEMM Y = z P with K = r3, where P is
// core viewed as (r3, r1 * r2), fused with the weighted reduction over r1:
//   mid[t, q] = sum_r c[t, r] * sc[r, q] * Y[t, (r, q)]      (sc = 1 without fp8)
// P^T is packed with its rows in blocks of 32 output channels q, each block
// holding the R1 ranks in turn (row (qb * R1 + r) * 32 + qq = channel
// (r, 32 qb + qq)), so the R1 column blocks a wave owns for one group of 32
// channels hold the same (row, q) in the same lane and the reduction over r is
// elementwise over accumulators. Both operands arrive by DMA.
//
// 256 x 256 tiles (256 tokens x 256 / R1 channels), 8 waves as 4 x 2, each wave
// 64 rows x 4 column blocks (QG = 4 / R1 channel groups). The work-group runs
// its tiles b, b + grid, ... as one stream of K tiles (r3 / 64 per tile) through
// the two-group ping-pong of gemm_mainloop_pingpong, so the DMA never stops at a
// tile boundary: after the compute phase of a tile's last K tile each wave
// reduces its accumulators over r and stores its part of mid straight from
// registers (8 bytes a lane; group 0, the DMA issuer, after its wait for the
// next K tile), then starts the next tile with zeroed
// accumulators. With r1 = 4 G, G > 1 (R1 = 4), P^T holds the ranks in groups
// of 4 (row ((g * nqb + qb) * 4 + rr) * 32 + qq) and an output tile (256 tokens x
// 64 channels) takes G consecutive tiles of the work-group, one per rank group:
// the reduction over each group's 4 ranks is added to the fp32 partial sum of
// the groups before it, carried in a.mpart (each lane reads back what it wrote),
// and the last group stores mid. SPP K steps of a K tile are read per memory phase (2: two
// memory/compute phase pairs per K tile, which halves the fragment registers).
// A tile's rows of c reach LDS by DMA with its first K tile (three buffers: the
// second group still reads tile i - 1's while tile i + 1's lands), so the
// epilogue issues no global load and waits on nothing. The stores are
// unconditional: the workspace holds mid for whole 256-row tiles.
template <int R1, int SPP, bool kGrouped = false>
__global__ __launch_bounds__(512) void k_core_pp(FwdArgs a) {
  static_assert(!kGrouped || R1 == 4, "rank groups of 4");
  typedef Tile<256, 256, 0, 4, 2, 1, 1, 2, true, true> TL;
  constexpr int FM = TL::FM, FN = TL::FN;   // 2 x 4 blocks of 32 x 32
  static_assert(FN % R1 == 0, "rank blocks per wave");
  constexpr int QG = FN / R1;               // channel groups of 32 per wave
  constexpr int kKSteps = kTileKBytes / 32;
  static_assert(kKSteps % SPP == 0, "steps per phase");
  constexpr int kHalves = kKSteps / SPP;    // memory/compute phase pairs per K tile
  constexpr int kABlk = TL::BM / 8, kBBlk = TL::BN / 8;
  constexpr int kDmaPerWave = (kABlk + kBBlk) / 4;
  constexpr int kScaleFloats = (int)kCorePScales;   // fp8 channel scales staged in LDS
  constexpr int kCBuf = TL::BM * R1;                // floats of c per tile
  constexpr int kCDma = kCBuf / 256;                // 1 KB DMA instructions per tile's c
  static_assert(kCDma <= 4, "c DMA by group 0's waves");
  __shared__ u32x4 smem[TL::kLdsBytes / 16 + kScaleFloats / 4 + 3 * kCBuf / 4];
  float* sc_lds = reinterpret_cast<float*>(smem + TL::kLdsBytes / 16);
  float* c_lds = sc_lds + kScaleFloats;   // [3][BM][R1]
  // without fp8 scales their region holds each wave's 2 KB transposition slot
  static_assert(kScaleFloats * 4 >= 8 * 2048, "transposition slots");
  char* slot = reinterpret_cast<char*>(sc_lds) + (threadIdx.x >> 6) * 2048;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, grp = wave >> 2;
  const int wm = wave / TL::WN, wn = wave % TL::WN;
  const int64_t r2 = a.r2, r3 = a.r3;
  const int G = kGrouped ? (int)(a.r1 / R1) : 1;   // rank groups per output tile
  const int S = kGrouped ? a.core_split : 1;     // parts of an output tile's rank groups
  const int Gp = G / S;                          // rank groups per part
  const int ntn = (int)(R1 * r2 / TL::BN);       // tiles per token tile and rank group
  const int ntm = (int)((a.T + TL::BM - 1) / TL::BM);
  const int nout = ntm * ntn;                    // output tiles
  const int nunits = nout * S;                   // work units: (output tile, part)
  const int nkt = (int)(r3 * 2 / kTileKBytes);   // K tiles per tile
  const int my_units = ((int)blockIdx.x < nunits) ? (nunits - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
  const int total = my_units * Gp * nkt;
  const int64_t row_bytes = r3 * 2;
  const int kt_rot = ((int)blockIdx.x >> 3) % nkt;
  const bool fp8 = a.core_scale_raw != nullptr;
  if (fp8) {   // the plan bounds r1 * r2 by kScaleFloats for fp8 weights
    for (int i = tid; i < R1 * (int)r2; i += 512) sc_lds[i] = a.core_scale_raw[i];
  }

  // tile i of this work-group: work unit u = blockIdx.x + (i / Gp) gridDim.x, i.e.
  // output tile o = u % nout (token tile tm, channel tile tn; the parts of one
  // output tile are nout apart, on one XCD when nout is a multiple of 8) and part
  // u / nout, whose rank groups are rg = part Gp .. part Gp + Gp - 1
  auto coords = [&](int i, int& tm, int& tn, int& rg, int& o) __attribute__((always_inline)) {
    const int u = (int)blockIdx.x + (i / Gp) * (int)gridDim.x;
    o = u % nout;
    rg = (u / nout) * Gp + i % Gp;
    tile_coords_of(o, ntn, nout, tm, tn);
  };
  // DMA of K tile g of this work-group's stream into `stage` (group 0's waves)
  auto dma_g = [&](int g, int stage) __attribute__((always_inline)) {
    int tm, tn, rg, ot;
    coords(g / nkt, tm, tn, rg, ot);
    // work-groups on one XCD start their tiles' K loops at different K tiles:
    // they read the same P^T rows, and reading the same lines at the same moment
    // measured 20% slower (the sum's order per output element is fixed per tile)
    const int kt = (g % nkt + kt_rot) % nkt;
    const int64_t m0 = (int64_t)tm * TL::BM;
    const int rows_valid = (int)(a.T - m0 < TL::BM ? a.T - m0 : TL::BM);
    RowLoader al{reinterpret_cast<const char*>(a.z) + m0 * row_bytes, row_bytes, rows_valid};
    RowLoader bl{reinterpret_cast<const char*>(a.coreP) +
                     (int64_t)(rg * ntn + tn) * TL::BN * row_bytes,
                 row_bytes, TL::BN};
    if (g % nkt == 0 && wave < kCDma) {
      // 16 bytes of the tile's c rows a lane (with G > 1: row wave * 64 + lane,
      // ranks 4 rg .. 4 rg + 3); the workspace holds c for whole tiles (rows past T
      // are never used for an output row below T)
      const int i = g / nkt;
      const float* src = G == 1 ? a.c + m0 * R1 + (int64_t)wave * 256 + lane * 4
                                : a.c + (m0 + wave * 64 + lane) * a.r1 + rg * R1;
      __builtin_amdgcn_global_load_lds((gbl_cvptr)src,
                                       (lds_vptr)(c_lds + (i % 3) * kCBuf + wave * 256), 16, 0, 0);
    }
    u32x4* s = smem + stage * TL::kStage;
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) {
      const int blk = wave + 4 * j;
      const int lc = dma_chunk(lane, blk);   // kABlk is even: block parity is kept
      if (blk < kABlk)
        __builtin_amdgcn_global_load_lds((gbl_cvptr)al.gaddr(blk * 8 + (lane >> 3), lc, kt),
                                         (lds_vptr)(s + blk * 64), 16, 0, 0);
      else
        __builtin_amdgcn_global_load_lds(
            (gbl_cvptr)bl.gaddr((blk - kABlk) * 8 + (lane >> 3), lc, kt),
            (lds_vptr)(s + (TL::BM + (blk - kABlk) * 8) * 8), 16, 0, 0);
    }
  };
  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = zero16();
  if (total == 0) return;   // uniform over the work-group

  // epilogue of tile i: mid[row, q] = sum_r c[row, r] sc[r, q] acc (transposed
  // accumulators: lane l holds row l & 31 of block f and, in elements 4 u .. 4 u + 3,
  // channels 8 u + 4 (l >> 5) .. + 3 of each column block)
  auto epilogue = [&](int i, auto fp8_tag) __attribute__((always_inline)) {
    constexpr bool kFp8 = decltype(fp8_tag)::value;
    int tm, tn, rg, ot;
    coords(i, tm, tn, rg, ot);
    const int64_t m0 = (int64_t)tm * TL::BM;
    // rank groups: this lane's partial sums, float4 (f, u) of wave `wave` of output
    // tile ot, one region of nout * 64 KB per part
    const int prt = rg / Gp, gi = rg % Gp;
    const int64_t part_floats = (int64_t)nout * 8 * FM * 4 * 64 * 4;
    float4* part = G > 1 ? reinterpret_cast<float4*>(a.mpart + prt * part_floats) +
                               (((int64_t)ot * 8 + wave) * FM * 4) * 64 + lane
                         : nullptr;
    // the part's running sum comes in from its previous group and goes out to its
    // next group or, at its last group when S > 1, to k_core_combine
    const bool carry_in = G > 1 && gi > 0, carry_out = G > 1 && (gi < Gp - 1 || S > 1);
#pragma unroll
    for (int g = 0; g < QG; ++g) {
      // channel block of column blocks g * R1 .. g * R1 + R1 - 1 of this wave
      const int qb = tn * (TL::BN / 32 / R1) + (wn * FN) / R1 + g;
#pragma unroll
      for (int f = 0; f < FM; ++f) {
        // one row block at a time (the scheduler would otherwise interleave the
        // blocks and spill)
        __builtin_amdgcn_sched_barrier(0);
        float4 pin[4];
        if (carry_in) {
#pragma unroll
          for (int u = 0; u < 4; ++u) pin[u] = part[(f * 4 + u) * 64];
        }
        float cf[R1];
#pragma unroll
        for (int r = 0; r < R1; ++r)
          cf[r] = c_lds[(i % 3) * kCBuf + (wm * TL::kWaveM + 32 * f + (lane & 31)) * R1 + r];
        const int64_t row = m0 + wm * TL::kWaveM + 32 * f + (lane & 31);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int q = qb * 32 + 8 * u + 4 * (lane >> 5);
          float o[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            float sum = 0.f;
#pragma unroll
            for (int r = 0; r < R1; ++r) {
              const float y = kFp8 ? acc[f][g * R1 + r][4 * u + v] * sc_lds[r * r2 + q + v]
                                   : acc[f][g * R1 + r][4 * u + v];
              sum += cf[r] * y;
            }
            o[v] = sum;
          }
          if (carry_in) {
            o[0] += pin[u].x;
            o[1] += pin[u].y;
            o[2] += pin[u].z;
            o[3] += pin[u].w;
          }
          if (carry_out) {
            part[(f * 4 + u) * 64] = float4{o[0], o[1], o[2], o[3]};
            continue;
          }
          uint2 pk;
          pk.x = pack_bf16x2(o[0], o[1]);
          pk.y = pack_bf16x2(o[2], o[3]);
          if constexpr (kFp8) {
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.mid) + row * r2 + q) = pk;
          } else {
            // into this wave's slot: row lane & 31, 16-byte chunk u (swizzled by
            // row >> 2), half lane >> 5
            const int r = lane & 31;
            *reinterpret_cast<uint2*>(slot + r * 64 + 16 * (u ^ ((r >> 2) & 3)) +
                                      8 * (lane >> 5)) = pk;
          }
        }
        if (carry_out) continue;
        if constexpr (!kFp8) {
          // the block's 32 rows x 32 channels leave as row-contiguous 64-byte pieces,
          // 16 rows a store instead of 32 rows of 16 bytes (LDS operations of one
          // wave complete in order: the reads see the writes above, and the next
          // block's writes follow these reads)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const int rr = 16 * hh + (lane >> 2), ch = lane & 3;
            const u32x4 v =
                *reinterpret_cast<const u32x4*>(slot + rr * 64 + 16 * (ch ^ ((rr >> 2) & 3)));
            const int64_t orow = m0 + wm * TL::kWaveM + 32 * f + rr;
            *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(a.mid) + orow * r2 + qb * 32 +
                                      8 * ch) = v;
          }
        }
      }
    }
#pragma unroll
    for (int f = 0; f < FM; ++f)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[f][j] = zero16();
  };

  // prologue: K tile 0 by group 0; group 1 starts one barrier late
  if (grp == 0) {
    dma_g(0, 0);
    wait_vm_lds<0>();
  }
  __syncthreads();   // also publishes the staged scales
  if (grp == 1) lds_barrier();

  for (int g = 0; g < total; ++g) {
    const u32x4* s = smem + (g & 1) * TL::kStage;
    const bool last_kt = g % nkt == nkt - 1;
#pragma unroll
    for (int h = 0; h < kHalves; ++h) {
      // -- memory phase: fragments of K steps h * SPP .. + SPP - 1 ------------
      u32x4 af[SPP][FM], bfr[SPP][FN];
#pragma unroll
      for (int ks = 0; ks < SPP; ++ks) {
        const int ch = (h * SPP + ks) * 2 + (lane >> 5);
#pragma unroll
        for (int f = 0; f < FM; ++f)
          af[ks][f] = s[lds_slot(wm * TL::kWaveM + f * 32 + (lane & 31), ch)];
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bfr[ks][j] = s[lds_slot(TL::BM + wn * TL::kWaveN + j * 32 + (lane & 31), ch)];
      }
      if (h == 0 && grp == 0 && g + 1 < total) dma_g(g + 1, (g + 1) & 1);
      wait_vm_lds<63>();   // this wave's fragment reads; the DMA stays in flight
      lds_barrier();
      // -- compute phase --------------------------------------------------------
#pragma unroll
      for (int ks = 0; ks < SPP; ++ks)
#pragma unroll
        for (int f = 0; f < FM; ++f)
#pragma unroll
          for (int j = 0; j < FN; ++j) mma(acc[f][j], bfr[ks][j], af[ks][f], EltBF16{});
      if (h == kHalves - 1) {
        if (last_kt) {
          mfma_drain();
          // DMA of K tile g + 1 has landed. Waited for before the stores below
          // are issued: loads and stores on one counter may complete out of
          // order. The stores drain during the next K tile, whose wait covers them.
          if (grp == 0) wait_vm_lds<0>();
          if (fp8) epilogue(g / nkt, std::true_type{});
          else epilogue(g / nkt, std::false_type{});
        } else if (grp == 0) {
          wait_vm_lds<0>();   // DMA of K tile g + 1 has landed
        }
      }
      lds_barrier();
    }
  }
  if (grp == 0) lds_barrier();
}

// mid = sum over the S parts of k_core_pp's grouped partial sums, in part order
// (rank groups split over S work units, so that T / 256 x r2 / 64 output tiles fill
// the compute units). One thread per float4 of a part, in the lane-private layout
// the core stored: output tile o, wave w (4 x 2 waves), row block f, chunk u, lane l
// holds rows 64 (w / 2) + 32 f + (l & 31) and channels 32 qb + 8 u + 4 (l >> 5) .. + 3,
// qb = 2 tn + w % 2, of token tile tm and channel tile tn (tile_coords_of).
__global__ __launch_bounds__(256) void k_core_combine(FwdArgs a) {
  const int ntn = (int)(a.r2 / 64);
  const int ntm = (int)((a.T + kCorePRows - 1) / kCorePRows);
  const int nout = ntm * ntn;
  const int64_t per_part = (int64_t)nout * 8 * 2 * 4 * 64;   // float4s
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= per_part) return;
  const int lane = (int)(i & 63), u = (int)((i >> 6) & 3), f = (int)((i >> 8) & 1),
            w = (int)((i >> 9) & 7);
  const int o = (int)(i >> 12);
  int tm, tn;
  tile_coords_of(o, ntn, nout, tm, tn);
  const float4* src = reinterpret_cast<const float4*>(a.mpart) + i;
  float4 t = src[0];
  for (int p = 1; p < a.core_split; ++p) {
    const float4 v = src[p * per_part];
    t.x += v.x;
    t.y += v.y;
    t.z += v.z;
    t.w += v.w;
  }
  const int64_t row = (int64_t)tm * kCorePRows + 64 * (w / 2) + 32 * f + (lane & 31);
  const int64_t q = (int64_t)(2 * tn + w % 2) * 32 + 8 * u + 4 * (lane >> 5);
  uint2 pk;
  pk.x = pack_bf16x2(t.x, t.y);
  pk.y = pack_bf16x2(t.z, t.w);
  *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.mid) + row * a.r2 + q) = pk;
}

// ---- k_outproj: out = mid U_out + bias  (model.py:101) --------------------
// Both operands arrive by DMA through NS LDS stages.
template <class Elt, int BM, int BN, int WM, int WN, int NS>
__global__ __launch_bounds__(64 * WM * WN) void k_outproj(FwdArgs a) {
  typedef typename Elt::T T;
  typedef Tile<BM, BN, 0, WM, WN, 1, 1, NS, true, true> TL;
  __shared__ u32x4 smem[cmax(TL::kLdsBytes, TileStage<TL, T>::kBytes) / 16];

  const int ntn = (int)((a.d_out + BN - 1) / BN);
  const int ntm = (int)((a.T + BM - 1) / BM);
  int tm, tn;
  tile_coords(ntn, ntm * ntn, tm, tn);
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t n0 = (int64_t)tn * BN;
  const int rows_valid = (int)(a.T - m0 < BM ? a.T - m0 : BM);
  const int64_t row_bytes = a.r2 * (int64_t)sizeof(T);
  RowLoader al{reinterpret_cast<const char*>(a.mid) + m0 * row_bytes, row_bytes, rows_valid};
  RowLoader bl{reinterpret_cast<const char*>(a.uoutT) + n0 * row_bytes, row_bytes,
               (int)(a.d_out - n0)};
  f32x16 acc[TL::FM][TL::FN];
  NoExtra nx;
  gemm_mainloop<TL, Elt>(acc, al, bl, (int)(row_bytes / kTileKBytes), smem, nx);

  char* stage = reinterpret_cast<char*>(smem);
  const int cols_valid = (int)(a.d_out - n0);
  float bcol[TL::FN], scol[TL::FN];
  {
    const int wn = (threadIdx.x >> 6) % WN, lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < TL::FN; ++j) {
      const int col = wn * TL::kWaveN + j * 32 + (lane & 31);
      bcol[j] = col < cols_valid ? a.bias[n0 + col] : 0.f;
      scol[j] = a.out_scale && col < cols_valid ? a.out_scale[n0 + col] : 1.f;
    }
  }
  stage_tile<TL, T>(acc, stage, bcol, scol);
  __syncthreads();
  flush_tile_by<TL, T, TL::kThreads>(stage, a, m0, n0, rows_valid, cols_valid, (int)threadIdx.x);
}

// Persistent bf16 out-projection (8 waves, ping-pong main loop): work-group b
// takes tiles b, b + gridDim.x, ... Each tile is staged in LDS by all waves and
// written out by group 1 alone, whose stores then drain during the next tile's
// main loop (group 1 never waits on vmcnt; group 0 issues every DMA).
template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void k_outproj_pp(FwdArgs a) {
  typedef uint16_t T;
  typedef Tile<BM, BN, 0, WM, WN, 1, 1, 2, true, true> TL;
  static_assert(TL::kThreads == 512, "ping-pong: 8 waves");
  __shared__ u32x4 smem[cmax(TL::kLdsBytes, TileStage<TL, T>::kBytes) / 16];
  const int ntn = (int)((a.d_out + BN - 1) / BN);
  const int ntm = (int)((a.T + BM - 1) / BM);
  const int ntiles = ntm * ntn;
  const int grp = (threadIdx.x >> 6) >> 2;
  const int64_t row_bytes = a.r2 * (int64_t)sizeof(T);
  char* stage = reinterpret_cast<char*>(smem);
  for (int t = blockIdx.x; t < ntiles; t += gridDim.x) {
    int tm, tn;
    tile_coords_of(t, ntn, ntiles, tm, tn);
    const int64_t m0 = (int64_t)tm * BM;
    const int64_t n0 = (int64_t)tn * BN;
    const int rows_valid = (int)(a.T - m0 < BM ? a.T - m0 : BM);
    const int cols_valid = (int)(a.d_out - n0);
    RowLoader al{reinterpret_cast<const char*>(a.mid) + m0 * row_bytes, row_bytes, rows_valid};
    RowLoader bl{reinterpret_cast<const char*>(a.uoutT) + n0 * row_bytes, row_bytes, cols_valid};
    f32x16 acc[TL::FM][TL::FN];
    gemm_mainloop_pingpong<TL, EltBF16>(acc, al, bl, (int)(row_bytes / kTileKBytes), smem);
    // fused epilogue: all 8 waves load their share of epi_a (before the staging
    // where the registers allow: 128-token tiles) and apply it to the staged tile
    // after the barrier (group 0 only loads); group 1 then stores the tile as a
    // plain one
    constexpr bool kEarly = BM <= 128;
    const bool epi = a.epi_mode != kEpiNone;
    u32x4 e[EpiTile<TL, 512>::kIters];
    if (kEarly && epi)
      epi_tile_load<TL, 512>(e, a, m0, n0, rows_valid, cols_valid, (int)threadIdx.x);
    stage_tile_t<TL>(acc, stage, a.bias + n0, a.out_scale ? a.out_scale + n0 : nullptr,
                     cols_valid,
                     a.epi_mode == kEpiResScale ? static_cast<const uint16_t*>(a.epi_b) + n0
                                                : nullptr);
    wait_vm_lds<63>();   // LDS writes done; stores of the previous tile may still drain
    lds_barrier();
    if (epi) {
      if (!kEarly)
        epi_tile_load<TL, 512>(e, a, m0, n0, rows_valid, cols_valid, (int)threadIdx.x);
      epi_tile_apply<TL, 512>(stage, e, a, (int)threadIdx.x);
      wait_vm_lds<63>();
      lds_barrier();
    }
    if (grp == 1)
      flush_tile_by<TL, T, 256, true>(stage, a, m0, n0, rows_valid, cols_valid,
                                      (int)threadIdx.x - 256);
    wait_vm_lds<63>();   // the staged tile is read before the next tile's DMA reuses it
    lds_barrier();
  }
}

// ---- packing kernels -----------------------------------------------------
// W^T of a folded plan: dst[n][kk] = os[n] * sum_q uoutT[n][q] * coreT[q][kk] * cs[kk / r3][q]
// (bf16 bits in and out, fp32 sums in q order, one rounding), i.e. W = core (K x r2)
// times U_out (r2 x d_out) stored transposed (d_out rows of K). 32 x 32 output tiles,
// 256 threads each holding 4 rows n; K and r2 are multiples of 32, d_out of 16.
__global__ void k_fold_out_t(const uint16_t* __restrict__ coreT, const uint16_t* __restrict__ uoutT,
                             const float* __restrict__ cs, const float* __restrict__ os,
                             uint16_t* __restrict__ dst, int64_t K, int64_t r3, int64_t r2,
                             int64_t d_out) {
  __shared__ float ct[32][33];   // [q][kk]
  __shared__ float ut[32][33];   // [n][q]
  const int64_t k0 = (int64_t)blockIdx.x * 32, n0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8 threads
  const int64_t rank = (k0 + tx) / r3;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t q0 = 0; q0 < r2; q0 += 32) {
    for (int y = ty; y < 32; y += 8) {
      float v = bf16_bits_to_f32(coreT[(q0 + y) * K + k0 + tx]);
      if (cs) v *= cs[rank * r2 + q0 + y];
      ct[y][tx] = v;
      ut[y][tx] = n0 + y < d_out ? bf16_bits_to_f32(uoutT[(n0 + y) * r2 + q0 + tx]) : 0.f;
    }
    __syncthreads();
#pragma unroll 8
    for (int qq = 0; qq < 32; ++qq) {
      const float c = ct[qq][tx];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = fmaf(ut[ty + 8 * i][qq], c, acc[i]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t n = n0 + ty + 8 * i;
    if (n < d_out) dst[n * K + k0 + tx] = f32_to_bf16_bits(os ? acc[i] * os[n] : acc[i]);
  }
}

// The A operand of a folded plan's single GEMM: mid[t][r R3 + s] = R(c[t][r] * z[t][s])
// (z bf16 (T, R3), c fp32 (T, rk), mid bf16 (T, rk R3)). A thread reads one 16-byte
// chunk of z (8 elements) and writes its rk scaled copies; the R3 / 8 threads of a
// row are consecutive, so each copy is stored as whole row segments. Grid-stride
// over the T * R3 / 8 chunks.
template <int R3>
__global__ void k_expand_cz(const FwdArgs a) {
  constexpr int CPR = R3 / 8;   // chunks per z row
  const int rk = (int)a.r1;
  const uint64_t n = (uint64_t)a.T * CPR;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t t = i / CPR;
    const uint32_t s8 = (uint32_t)(i % CPR) * 8;
    const u32x4 zv = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.z) +
                                                     t * R3 + s8);
    float zf[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      zf[2 * j] = bf16_bits_to_f32(zv[j] & 0xffffu);
      zf[2 * j + 1] = bf16_bits_to_f32(zv[j] >> 16);
    }
    const float* crow = a.c + t * rk;
    uint16_t* dst = static_cast<uint16_t*>(a.mid) + t * rk * R3 + s8;
    for (int r = 0; r < rk; ++r) {
      const float cr = crow[r];
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = pack_bf16x2(zf[2 * j] * cr, zf[2 * j + 1] * cr);
      *reinterpret_cast<u32x4*>(dst + r * R3) = o;
    }
  }
}

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

// The expert form of the core for plans with fewer experts than ranks:
// mid = sum_r c_r z core_r with c = sum_j w_j U_expert[e_j] equals
// sum_j w_j z G_{e_j} with G_e = sum_r U_expert[e, r] core_r (E x r3 x r2), a
// contraction over E instead of r1 ranks. Each element is summed over r in rank
// order in fp32 and rounded once to T, and written transposed as the core^T
// operand: dst[q][e r3 + s] = G[e][s][q] (r2 rows of E r3). 32 x 32 tiles of
// (e r3 + s, q): r3 and r2 are multiples of 32, so a tile lies in one e; r1 <= 64.
template <class T>
__global__ void k_mix_core_t(const T* __restrict__ uexp, const T* __restrict__ core,
                             T* __restrict__ dst, int64_t E, int64_t r1, int64_t r3, int64_t r2) {
  __shared__ float ue[64];
  __shared__ float tile[32][33];
  const int64_t q0 = (int64_t)blockIdx.x * 32, row0 = (int64_t)blockIdx.y * 32;
  const int64_t e = row0 / r3, s0 = row0 - e * r3;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8 threads
  if (threadIdx.x < r1) ue[threadIdx.x] = load_as_f32(uexp + e * r1 + threadIdx.x);
  __syncthreads();
  for (int y = ty; y < 32; y += 8) {
    float v = 0.f;
    for (int64_t r = 0; r < r1; ++r)
      v = fmaf(ue[r], load_as_f32(core + (r * r3 + s0 + y) * r2 + q0 + tx), v);
    tile[y][tx] = v;
  }
  __syncthreads();
  for (int y = ty; y < 32; y += 8) store_from_f32(dst + (q0 + y) * (E * r3) + row0 + tx, tile[tx][y]);
}

// dst (n x n floats) = the identity: U_expert of a plan packed in the expert form.
__global__ void k_eye(float* __restrict__ dst, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n * n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = i / n == i % n ? 1.f : 0.f;
}

// OCP e4m3 (1-4-3, bias 7, no infinities, S.1111.111 = NaN) to bf16 bits. Every
// e4m3 value is exactly representable in bf16.
__device__ __forceinline__ uint16_t e4m3_to_bf16_bits(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 8;
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  if (e == 15u && m == 7u) return (uint16_t)(sign | 0x7fc0u);
  // normal: (8 + m) 2^(e - 10); subnormal (e = 0): m 2^-9
  const float v = e ? ldexpf((float)(8u + m), (int)e - 10) : ldexpf((float)m, -9);
  return (uint16_t)(sign | (__float_as_uint(v) >> 16));
}

// dst (cols, rows) bf16 = e4m3 src (rows, cols) transposed. With colscale
// (scale of (row / group, col) at colscale[(row / group) * cols + col]) an entry
// whose scale is zero is stored as zero.
__global__ void k_transpose_e4m3(const uint8_t* __restrict__ src, uint16_t* __restrict__ dst,
                                 int64_t rows, int64_t cols, const float* __restrict__ colscale,
                                 int64_t group) {
  __shared__ uint16_t t[32][33];
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
  for (int i = threadIdx.x; i < 32 * 32; i += blockDim.x) {
    const int rr = i / 32, cc = i % 32;
    const int64_t r = r0 + rr, c = c0 + cc;
    uint16_t v = 0;
    if (r < rows && c < cols) {
      v = e4m3_to_bf16_bits(src[r * cols + c]);
      if (colscale && colscale[(r / group) * cols + c] == 0.f) v = 0;
    }
    t[rr][cc] = v;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 32 * 32; i += blockDim.x) {
    const int cc = i / 32, rr = i % 32;
    const int64_t r = r0 + rr, c = c0 + cc;
    if (r < rows && c < cols) dst[c * rows + r] = t[rr][cc];
  }
}

// P^T of k_core_pp from core (r1, r3, r2): with R = min(r1, 4) ranks per group and
// rank r = R g + rr, row ((g * nqb + qb) * R + rr) * 32 + qq (nqb = r2 / 32), column
// s holds core[r, s, 32 qb + qq] (for r1 <= 4: row (qb * r1 + r) * 32 + qq). Source
// bf16 bits (codes == false) or e4m3 codes with per-channel scales sc (r1, r2), a
// channel whose scale is zero packed as zeros. One work-group per (channel block
// qb, 32 columns s, rank r).
// src_t: the source is core^T (r2, r1 r3) instead of core (r1, r3, r2).
template <bool kE4M3>
__global__ void k_pack_core_p(const void* __restrict__ src, uint16_t* __restrict__ dst,
                              int64_t r1, int64_t r3, int64_t r2, const float* __restrict__ sc,
                              bool src_t) {
  __shared__ uint16_t t[32][33];
  const int64_t qb = blockIdx.x, s0 = (int64_t)blockIdx.y * 32, r = blockIdx.z;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8 threads
  for (int y = ty; y < 32; y += 8) {
    const int64_t i = src_t ? (qb * 32 + tx) * (r1 * r3) + r * r3 + s0 + y
                            : (r * r3 + s0 + y) * r2 + qb * 32 + tx;
    uint16_t v;
    if constexpr (kE4M3) {
      v = e4m3_to_bf16_bits(static_cast<const uint8_t*>(src)[i]);
      if (sc && sc[r * r2 + qb * 32 + tx] == 0.f) v = 0;
    } else {
      v = static_cast<const uint16_t*>(src)[i];
    }
    t[y][tx] = v;
  }
  __syncthreads();
  const int64_t R = r1 < 4 ? r1 : 4, nqb = r2 / 32;
  const int64_t prow = (((r / R) * nqb + qb) * R + r % R) * 32;
  for (int y = ty; y < 32; y += 8) dst[(prow + y) * r3 + s0 + tx] = t[tx][y];
}

// Core scale table of CoreRescale from sc (r1, r2): cs[r, q] = sc'[r, q] /
// sc'[r + 1, q] for r < r1 - 1 and cs[r1 - 1, q] = sc'[r1 - 1, q], where sc' is sc
// with zeros replaced by 1 (those channels' weights are packed as zero).
__global__ void k_core_scales(const float* __restrict__ sc, float* __restrict__ cs, int64_t r1,
                              int64_t r2) {
  for (int64_t q = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; q < r2;
       q += (int64_t)gridDim.x * blockDim.x) {
    for (int64_t r = 0; r < r1; ++r) {
      const float a = sc[r * r2 + q] == 0.f ? 1.f : sc[r * r2 + q];
      if (r + 1 < r1) {
        const float b = sc[(r + 1) * r2 + q] == 0.f ? 1.f : sc[(r + 1) * r2 + q];
        cs[r * r2 + q] = a / b;
      } else {
        cs[r * r2 + q] = a;
      }
    }
  }
}

template <class T>
__global__ void k_copy_pad(const T* __restrict__ src, T* __restrict__ dst, int64_t n,
                           int64_t n_pad) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_pad;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = i < n ? src[i] : T(0);
}

// out[t, :] = (x[t, :] / sqrt(mean(x[t, :]^2) + eps)) * w, computed in fp32 and rounded
// to T once (model.py:25-27: the sqrt, then the division, then the gain); one wave
// per row, the sum of squares in lane order then a wave reduction.
template <class T>
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const T* __restrict__ x, int64_t n_rows,
                                                      int64_t d, const T* __restrict__ w, float eps,
                                                      T* __restrict__ out) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n_rows) return;   // whole waves: no barrier follows
  const T* xr = x + row * d;
  float ss = 0.f;
  for (int64_t i = lane; i < d; i += 64) {
    const float v = load_as_f32(xr + i);
    ss += v * v;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  const float rms = sqrtf(ss / (float)d + eps);
  T* orow = out + row * d;
  for (int64_t i = lane; i < d; i += 64)
    store_from_f32(orow + i, (load_as_f32(xr + i) / rms) * load_as_f32(w + i));
}

// k_rmsnorm_rows for rows of nch = d * sizeof(T) / 16 <= 64 * kMaxChunks 16-byte
// chunks (16-byte aligned x, w and out): each lane holds chunks lane, lane + 64,
// ... in registers, so a row is read from memory once, with 16-byte accesses.
template <class T, int kMaxChunks>
__global__ __launch_bounds__(256) void k_rmsnorm_rows_v(const T* __restrict__ x, int64_t n_rows,
                                                        int64_t d, const T* __restrict__ w,
                                                        float eps, T* __restrict__ out) {
  constexpr int EPC = 16 / (int)sizeof(T);
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n_rows) return;   // whole waves: no barrier follows
  const int nch = (int)(d / EPC);
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * d);
  u32x4 v[kMaxChunks];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxChunks; ++k) {
    const int c = lane + 64 * k;
    v[k] = c < nch ? __builtin_nontemporal_load(xr + c) : u32x4{0u, 0u, 0u, 0u};
    const T* e = reinterpret_cast<const T*>(&v[k]);
#pragma unroll
    for (int j = 0; j < EPC; ++j) {
      const float f = load_as_f32(e + j);
      ss += f * f;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  const float rms = sqrtf(ss / (float)d + eps);
  const u32x4* wr = reinterpret_cast<const u32x4*>(w);
  u32x4* orow = reinterpret_cast<u32x4*>(out + row * d);
#pragma unroll
  for (int k = 0; k < kMaxChunks; ++k) {
    const int c = lane + 64 * k;
    if (c < nch) {
      const u32x4 wv = wr[c];
      u32x4 o;
      const T* e = reinterpret_cast<const T*>(&v[k]);
      const T* g = reinterpret_cast<const T*>(&wv);
      T* oe = reinterpret_cast<T*>(&o);
#pragma unroll
      for (int j = 0; j < EPC; ++j) store_from_f32(oe + j, (load_as_f32(e + j) / rms) * load_as_f32(g + j));
      orow[c] = o;
    }
  }
}

template <class T>
__global__ void k_to_f32(const T* __restrict__ src, float* __restrict__ dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = load_as_f32(src + i);
}

}  // namespace dev
}  // namespace tmoe
