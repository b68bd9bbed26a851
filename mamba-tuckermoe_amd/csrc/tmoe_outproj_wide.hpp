// The large-T bf16 out-projection out = A W^T + bias as a persistent GEMM with
// 256 x 288 output tiles (reference: model.py:101's `core @ self.U_out + bias`,
// here with A = mid or, for folded plans, c (x) z, and W^T = U_out^T or
// (core U_out)^T).
//
// One work-group of 4 waves per compute unit, one wave per SIMD. A wave owns 32 FM
// rows x 288 columns (tiles of 128 FM tokens, FM = 2 for large T, 1 for mid-size
// T): 9 FM accumulator blocks of 32 x 32, up to 16 of them pinned to the AGPRs and
// the rest to VGPRs through inline-asm MFMAs (builtin MFMAs on this many
// accumulators made the compiler copy them between the register files around
// every MFMA). K tiles of 64 (128 bytes of a row) stream by DMA into two LDS
// stages of BM + 288 rows (A, then W^T) with the swizzle of lds_slot.
//
// The epilogue stores come from the accumulators directly (lanes l and l + 32
// swap halves with v_permlane32_swap so that each lane writes 16 contiguous
// bytes). On gfx9 one counter (vmcnt) covers loads and stores in issue order,
// so a wait for a DMA issued after a burst of stores also waits for the
// stores. The next tile's first two K tiles are therefore issued before the
// stores, and the waits that follow leave the stores outstanding: they drain
// under the next tile's first K tiles. The bias columns come through the
// scalar unit (no LDS read after the DMA, which would wait for it).
//
// The A operand is either stored rows of K elements (mid, or c (x) z written by
// the front), or, for folded plans with r1 = 4 and r3 = 256 (KR), formed in the
// loop: the DMA brings z's rows (r3 = 256 elements) into the A part of a stage,
// K tile kt reading z's columns 64 (kt % 4) .. and belonging to rank r = kt / 4,
// and each A fragment is scaled by its row's c_r on its way from LDS to the
// MFMA, R(c_r R(z)) exactly as the front would have stored it. A stage then
// holds a quarter of the A bytes it would otherwise (z instead of c (x) z), and
// the 4x larger c (x) z is never written.
//
// Shape contract (checked by the host): K % 64 == 0, N % 288 == 0 (W^T rows
// read in whole tiles), A (or z and c) allocated for T rounded up to 256 rows
// (rows past T are read, their results never stored), no column scale and no
// fused epilogue; KR: K = 4 * 256.
#pragma once

namespace tmoe {
namespace dev {

namespace wide {

constexpr int FN = 9;            // 32-column blocks per tile
constexpr int BN = 32 * FN;      // 288 columns
constexpr int kAgprBlk = 16;     // accumulator blocks in AGPRs; the rest in VGPRs

// Tiles of BM = 128 FM tokens: FM 32-row blocks per wave (FM = 2: 256 x 288, the
// large-T tile; FM = 1: 128 x 288, twice as many tiles for mid-size T).
template <int FM_>
struct Cfg {
  static constexpr int FM = FM_;
  static constexpr int BM = 128 * FM;
  static constexpr int kRows = BM + BN;            // operand rows per K tile
  static constexpr int kStage = kRows * 8;         // 16-byte slots per stage
  static constexpr int kBlocks = kRows / 8;        // 8-row DMA blocks per stage
  static constexpr int kDmaPerWave = kBlocks / 4;
  static constexpr int kABlocksPerWave = BM / 32;
  static constexpr int kStores = 2 * FN * FM;      // epilogue stores per wave of a full tile
  static_assert(kBlocks % 4 == 0, "DMA blocks split evenly over 4 waves");
  static_assert(kDmaPerWave + kStores <= 63, "counted waits within the vmcnt range");
  static_assert(2 * kStage * 16 <= 160 * 1024, "LDS");
};
constexpr int BM = Cfg<2>::BM;   // the large-T tile

constexpr int kKrR1 = 4, kKrR3 = 256;   // the KR operand's ranks
constexpr int kKrTilesPerRank = kKrR3 / 64;
// Fragment steps of a K step: A fragment reads at steps 0 .. FM - 1, W^T fragment
// reads at FM .. FM + FN - 1; with the KR operand, dword d of A fragment i is
// scaled at step kKrScale0 + 4 i + d (four MFMAs after the A reads, one 16-byte
// group's 5 VALU instructions per MFMA gap)
constexpr int kKrScale0 = 4;
constexpr int frag_steps(int fm) {
  return fm + FN > kKrScale0 + 4 * fm ? fm + FN : kKrScale0 + 4 * fm;
}

}  // namespace wide

#define TMOE_MFMA_A(acc, b, a) \
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(b), "v"(a))
#define TMOE_MFMA_V(acc, b, a) \
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(b), "v"(a))
#define TMOE_MFMA_A0(acc, b, a) \
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=a"(acc) : "v"(b), "v"(a))
#define TMOE_MFMA_V0(acc, b, a) \
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=v"(acc) : "v"(b), "v"(a))

// One K step (16 of K) of a wave's 18 blocks, W^T fragment first (transposed
// result: lane l holds row l & 31 of the block and columns 8 q + 4 (l >> 5) +
// 0..3 in elements 4 q .. 4 q + 3). ld(b) runs after the b-th MFMA: the next
// step's fragment reads and (KR operand) the scaling of its A fragments, spread
// between the MFMAs (wide::frag_steps(FM) steps b in all).
template <bool kZero, int FM, class LD>
__device__ __forceinline__ void wide_step(f32x16 (&acc)[FM][wide::FN], const u32x4 (&af)[FM],
                                          const u32x4 (&bf)[wide::FN], LD&& ld) {
#pragma unroll
  for (int j = 0; j < wide::FN; ++j)
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int blk = j * FM + i;
      if (kZero) {
        if (blk < wide::kAgprBlk) TMOE_MFMA_A0(acc[i][j], bf[j], af[i]);
        else TMOE_MFMA_V0(acc[i][j], bf[j], af[i]);
      } else {
        if (blk < wide::kAgprBlk) TMOE_MFMA_A(acc[i][j], bf[j], af[i]);
        else TMOE_MFMA_V(acc[i][j], bf[j], af[i]);
      }
      ld(blk);
      __builtin_amdgcn_sched_barrier(0);
    }
  // fewer MFMAs than fragment steps (FM = 1: 9 against 10): the rest after the last
#pragma unroll
  for (int m = FM * wide::FN; m < wide::frag_steps(FM); ++m) ld(m);
}

// The tile loop of a work-group: out = A Bt^T + bias over the tiles a schedule
// hands it. Sched: start(tm, tn) gives the first tile (false: none) and
// advance(tm, tn) the next (false: no more), both called uniformly by the whole
// work-group. A (M rows, K), Bt (N rows, K), C (M, N) bf16 bits; bias (N) fp32.
// KR: A is z (M rows, 256) and cr is c (M rows, 4 floats), K = 1024.
// smem: 2 Cfg<FM>::kStage 16-byte slots of LDS.
template <int FM_, class Sched, bool KR = false>
__device__ __forceinline__ void wide_loop(const uint16_t* __restrict__ A,
                                          const uint16_t* __restrict__ Bt,
                                          uint16_t* __restrict__ C,
                                          const float* __restrict__ bias, int M, int N, int K,
                                          u32x4* smem, Sched& sched,
                                          const float* __restrict__ cr = nullptr) {
  using wide::FN;
  using wide::BN;
  using wide::kAgprBlk;
  typedef wide::Cfg<FM_> Cf;
  constexpr int FM = Cf::FM, BM = Cf::BM, kStage = Cf::kStage;
  constexpr int kDmaPerWave = Cf::kDmaPerWave, kABlocksPerWave = Cf::kABlocksPerWave;
  constexpr int kStores = Cf::kStores;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nkt = K / 64;
  const uint32_t row_bytes = (uint32_t)K * 2;
  const uint32_t a_row_bytes = KR ? (uint32_t)wide::kKrR3 * 2 : row_bytes;

  f32x16 acc[FM][FN];
  u32x4 fa[2][FM], fb[2][FN];
  // KR: c (all 4 ranks) of this lane's row in the wave's row blocks 0 and 1 (named
  // registers: an array of them was kept in scratch memory)
  float4 ca0 = {0.f, 0.f, 0.f, 0.f}, ca1 = {0.f, 0.f, 0.f, 0.f};
  static_assert(FM <= 2, "KR: at most two row blocks per wave");
  auto load_c = [&](int tm_) __attribute__((always_inline)) {
    if constexpr (KR) {
      const float* c0 = cr + (int64_t)(tm_ * BM + wave * (32 * FM) + (lane & 31)) * wide::kKrR1;
      ca0 = *reinterpret_cast<const float4*>(c0);
      if constexpr (FM > 1) ca1 = *reinterpret_cast<const float4*>(c0 + 32 * wide::kKrR1);
    }
  };
  // c_r of row block m for K tile kt (rank kt / 4), by selects
  auto c_of = [&](int m, int kt) __attribute__((always_inline)) -> float {
    const int r = kt / wide::kKrTilesPerRank;
    const float4 v = m == 0 ? ca0 : ca1;
    return r == 0 ? v.x : r == 1 ? v.y : r == 2 ? v.z : v.w;
  };

  int tm, tn;
  if (!sched.start(tm, tn)) return;
  load_c(tm);

  // DMA block wave + 4 d of a stage: A rows 32 d + 8 wave + (lane >> 3) for
  // d < kABlocksPerWave, else W^T rows 32 (d - kABlocksPerWave) + 8 wave +
  // (lane >> 3). Whole tiles are in bounds, so one per-lane offset serves all.
  const uint32_t voff = (uint32_t)(8 * wave + (lane >> 3)) * row_bytes +
                        (uint32_t)dma_chunk(lane, wave) * 16u;
  const uint32_t voff_a = KR ? (uint32_t)(8 * wave + (lane >> 3)) * a_row_bytes +
                                   (uint32_t)dma_chunk(lane, wave) * 16u
                             : voff;
  auto dma = [&](int d, int kt, int stage, int tm_, int tn_) __attribute__((always_inline)) {
    const char* base;
    uint32_t off;
    if (d < kABlocksPerWave) {
      base = reinterpret_cast<const char*>(A) + (int64_t)tm_ * BM * a_row_bytes +
             (int64_t)d * 32 * a_row_bytes +
             (KR ? kt % wide::kKrTilesPerRank : kt) * kTileKBytes;
      off = voff_a;
    } else {
      base = reinterpret_cast<const char*>(Bt) + (int64_t)tn_ * BN * row_bytes +
             (int64_t)(d - kABlocksPerWave) * 32 * row_bytes + kt * kTileKBytes;
      off = voff;
    }
    // the LDS address goes through an integer, as in the measured build of this
    // loop (a pointer with provenance changes the compiler's DMA alias tracking)
    const uint32_t lds = (uint32_t)(size_t)(__attribute__((address_space(3))) u32x4*)(
        smem + stage * kStage + (wave + 4 * d) * 64);
    __builtin_amdgcn_global_load_lds((gbl_cvptr)(base + off), (lds_vptr)(size_t)lds, 16, 0, 0);
  };
  // fragment step m of K step ks of K tile kt into buffer buf (see frag_steps):
  // m < FM reads A fragment m (KR: its raw z into ra[m]), FM <= m < FM + FN reads
  // W^T fragment m - FM, and (KR) step kKrScale0 + 4 i + d scales dword d of A
  // fragment i, R(c_r R(z)) as the front's flush_cz forms it
  u32x4 ra[FM];
  auto read_frag = [&](int kt, int ks, int buf, int m) __attribute__((always_inline)) {
    const u32x4* s = smem + (kt & 1) * kStage;
    const int ch = ks * 2 + (lane >> 5);
    if (m < FM) {
      const u32x4 v = s[lds_slot(wave * (32 * FM) + m * 32 + (lane & 31), ch)];
      if constexpr (KR) ra[m] = v;
      else fa[buf][m] = v;
    } else if (m < FM + FN) {
      fb[buf][m - FM] = s[lds_slot(BM + (m - FM) * 32 + (lane & 31), ch)];
    }
    if constexpr (KR) {
      const int q = m - wide::kKrScale0;
      if (q >= 0 && q < 4 * FM) {
        const int i = q / 4, d = q % 4;
        const float c = c_of(i, kt);
        fa[buf][i][d] = pack_bf16x2(bf16_bits_to_f32(ra[i][d] & 0xffffu) * c,
                                    bf16_bits_to_f32(ra[i][d] >> 16) * c);
      }
    }
  };
  auto read_frags = [&](int kt, int ks, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < wide::frag_steps(FM); ++m) read_frag(kt, ks, buf, m);
  };

  // One K tile: the MFMAs of its 4 K steps from fragments read one step ahead;
  // the DMA of tile kt + 1 (unless issued earlier) over steps 0-1; wait +
  // barrier after step 2, then the first fragments of tile kt + 1 are read
  // under step 3's MFMAs. keep_stores: the wait leaves the previous tile's
  // kStores stores outstanding (issued after this tile's K tile 1 DMA).
  auto ktile = [&](int kt, bool first, bool more, bool issue, bool keep_stores)
                   __attribute__((always_inline)) {
    if (more && issue) {
#pragma unroll
      for (int d = 0; d < kDmaPerWave / 2; ++d) dma(d, kt + 1, (kt + 1) & 1, tm, tn);
    }
    __builtin_amdgcn_sched_barrier(0);
    {
      auto ld = [&](int m) __attribute__((always_inline)) { read_frag(kt, 1, 1, m); };
      if (first) wide_step<true, FM>(acc, fa[0], fb[0], ld);
      else wide_step<false, FM>(acc, fa[0], fb[0], ld);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (more && issue) {
#pragma unroll
      for (int d = kDmaPerWave / 2; d < kDmaPerWave; ++d) dma(d, kt + 1, (kt + 1) & 1, tm, tn);
    }
    __builtin_amdgcn_sched_barrier(0);
    wide_step<false, FM>(acc, fa[1], fb[1],
                     [&](int m) __attribute__((always_inline)) { read_frag(kt, 2, 0, m); });
    __builtin_amdgcn_sched_barrier(0);
    wide_step<false, FM>(acc, fa[0], fb[0],
                     [&](int m) __attribute__((always_inline)) { read_frag(kt, 3, 1, m); });
    __builtin_amdgcn_sched_barrier(0);
    if (keep_stores) wait_vm_lds<kStores>();
    else wait_vm_lds<0>();
    lds_barrier();
    wide_step<false, FM>(acc, fa[1], fb[1], [&](int m) __attribute__((always_inline)) {
      if (more) read_frag(kt + 1, 0, 0, m);
    });
    __builtin_amdgcn_sched_barrier(0);
    // after a tile's last MFMA its accumulator writes land before the registers
    // are read
    if (!more) mfma_drain();
  };

  // prologue of the first tile
#pragma unroll
  for (int d = 0; d < kDmaPerWave; ++d) dma(d, 0, 0, tm, tn);
  wait_vm_lds<0>();
  lds_barrier();
  read_frags(0, 0, 0);

  bool pre = false;        // K tile 1 of this tile went out before the previous stores
  bool pre_full = false;   // ... and all kStores of those stores were issued
  for (;;) {
    ktile(0, true, nkt > 1, !pre, pre && pre_full);
    for (int kt = 1; kt + 1 < nkt; ++kt) ktile(kt, false, true, true, false);
    if (nkt > 1) ktile(nkt - 1, false, false, true, false);
    // the next tile's first two K tiles into stages 0 and 1 (both free: every
    // read of them completed before the last barrier), ahead of the stores
    int tm2 = tm, tn2 = tn;
    const bool has_next = sched.advance(tm2, tn2);
    const bool early = has_next && nkt > 1;
    // the next tile's c (every A fragment of this tile has been read): older than
    // its DMAs, so the counted waits below also cover it
    if (has_next) load_c(tm2);
    if (has_next) {
#pragma unroll
      for (int d = 0; d < kDmaPerWave; ++d) dma(d, 0, 0, tm2, tn2);
      if (early) {
#pragma unroll
        for (int d = 0; d < kDmaPerWave; ++d) dma(d, 1, 1, tm2, tn2);
      }
    }
    const bool full = (tm + 1) * BM <= M;
    {
      // lane-derived values are recomputed here rather than kept live through
      // the main loop
      int ln = threadIdx.x & 63;
      asm volatile("" : "+v"(ln));
      const int n0 = tn * BN;
      const int m0 = tm * BM + wave * (32 * FM);
      const bool hi = ln >= 32;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        // the block's 32 bias values: uniform loads
        float bj[32];
        {
          const float4* bp = reinterpret_cast<const float4*>(bias + n0 + j * 32);
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            const float4 v = bp[c];
            bj[4 * c] = v.x; bj[4 * c + 1] = v.y; bj[4 * c + 2] = v.z; bj[4 * c + 3] = v.w;
          }
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int row = m0 + i * 32 + (ln & 31);
          uint32_t pk[4][2];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (j * FM + i < kAgprBlk)   // read the AGPR here, not all at the loop exit
                asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v[e]) : "a"(acc[i][j][4 * q + e]));
              else
                v[e] = acc[i][j][4 * q + e];
              v[e] += hi ? bj[8 * q + 4 + e] : bj[8 * q + e];
            }
            pk[q][0] = pack_bf16x2(v[0], v[1]);
            pk[q][1] = pack_bf16x2(v[2], v[3]);
          }
          if (row < M) {
            // lanes l and l + 32 swap halves: lane l then holds columns 16 p + 0..7
            // and lane l + 32 columns 16 p + 8..15 of the block
#pragma unroll
            for (int p = 0; p < 2; ++p) {
              const auto sx = __builtin_amdgcn_permlane32_swap(pk[2 * p][0], pk[2 * p + 1][0],
                                                                false, false);
              const auto sy = __builtin_amdgcn_permlane32_swap(pk[2 * p][1], pk[2 * p + 1][1],
                                                                false, false);
              const u32x4 val = {sx[0], sy[0], sx[1], sy[1]};
              const int col = n0 + j * 32 + 16 * p + 8 * (ln >> 5);
              *reinterpret_cast<u32x4*>(C + (int64_t)row * N + col) = val;
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (!has_next) break;
    tm = tm2;
    tn = tn2;
    // K tile 0 has landed once at most the DMAs of K tile 1 and the stores remain
    // (all kStores of them only for a full tile; else the stores are waited for too)
    if (early && full) wait_vm_lds<kDmaPerWave + kStores>();
    else if (early) wait_vm_lds<kDmaPerWave>();
    else wait_vm_lds<0>();
    lds_barrier();
    read_frags(0, 0, 0);
    pre = early;
    pre_full = full;
  }
}


// Work-group b's tiles: b, b + grid, ... of the (M / BM) x (N / BN) tile grid, in
// tile_coords_of's XCD-aware order.
struct WideGridSched {
  int t, ntn, ntiles;
  __device__ __forceinline__ bool start(int& tm, int& tn) {
    t = blockIdx.x;
    if (t >= ntiles) return false;
    tile_coords_of(t, ntn, ntiles, tm, tn);
    return true;
  }
  __device__ __forceinline__ bool advance(int& tm, int& tn) {
    t += (int)gridDim.x;
    if (t >= ntiles) return false;
    tile_coords_of(t, ntn, ntiles, tm, tn);
    return true;
  }
};

// The pointers are separate restrict parameters: that lets the compiler read bias
// through the scalar unit (it may assume no store of C clobbers it).
template <int FM_>
__global__ __launch_bounds__(256) void k_outproj_wide(const uint16_t* __restrict__ A,
                                                      const uint16_t* __restrict__ Bt,
                                                      uint16_t* __restrict__ C,
                                                      const float* __restrict__ bias, int M,
                                                      int N, int K) {
  typedef wide::Cfg<FM_> Cf;
  __shared__ u32x4 smem[2 * Cf::kStage];
  WideGridSched sched{0, N / wide::BN, ((M + Cf::BM - 1) / Cf::BM) * (N / wide::BN)};
  wide_loop<FM_>(A, Bt, C, bias, M, N, K, smem, sched);
}

// The same GEMM with the KR operand: A = c (x) z formed from z (M, 256) and c
// (M, 4) in the loop, K = 1024.
template <int FM_>
__global__ __launch_bounds__(256) void k_outproj_wide_kr(const uint16_t* __restrict__ Z,
                                                         const float* __restrict__ c,
                                                         const uint16_t* __restrict__ Bt,
                                                         uint16_t* __restrict__ C,
                                                         const float* __restrict__ bias, int M,
                                                         int N, int K) {
  typedef wide::Cfg<FM_> Cf;
  __shared__ u32x4 smem[2 * Cf::kStage];
  WideGridSched sched{0, N / wide::BN, ((M + Cf::BM - 1) / Cf::BM) * (N / wide::BN)};
  wide_loop<FM_, WideGridSched, true>(Z, Bt, C, bias, M, N, K, smem, sched, c);
}

#undef TMOE_MFMA_A
#undef TMOE_MFMA_V
#undef TMOE_MFMA_A0
#undef TMOE_MFMA_V0

}  // namespace dev
}  // namespace tmoe
