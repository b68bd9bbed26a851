// The mid-T bf16 out-projection out = A W^T + bias (reference: model.py:101's
// `core @ self.U_out + bias`; A = mid or, folded, c (x) z): 128 x 144 output
// tiles, so that T = 2048 at d_out = 2304 gives 16 x 16 = 256 work-groups, one per
// compute unit (the 256 x 192 and 128 x 192 tiles of k_outproj_pp gave 96-192,
// each walking its K loop with one tile in flight).
//
// 4 waves, one per SIMD; a wave owns 32 tokens x 144 columns as 2 x 9 blocks of
// 16 x 16 (v_mfma_f32_16x16x32_bf16, W^T fragment first: lane l holds token
// l & 15 of its row block and columns 4 (l >> 4) .. + 3 of its column block).
// K tiles of 64 stream by DMA into four LDS stages of 272 rows (128 of A, 144 of
// W^T), three tiles ahead of the MFMAs: in this regime every work-group has one
// tile and the time is the DMA latency each K tile would otherwise expose.
// The bias is loaded at the start (each lane's 4 columns of each block). The
// output tile goes out through LDS as 16-byte chunks of whole rows (the MFMA
// layout's own stores were 32-byte pieces of 16 rows each: 15.5 -> 14.4 us per
// launch at T = 2048).
//
// Shape contract (checked by the host): K % 64 == 0, N % 144 == 0, A allocated
// for T rounded up to 128 rows (rows past T are read, their results never
// stored), no column scale, no fused epilogue.
#pragma once

namespace tmoe {
namespace dev {

namespace mid {

constexpr int BM = 128;          // tokens per tile
constexpr int BN = 144;          // columns per tile
constexpr int FM = 2;            // 16-row blocks per wave (32 tokens)
constexpr int FN = 9;            // 16-column blocks per wave (all 144)
constexpr int NS = 4;            // LDS stages
constexpr int kRows = BM + BN;   // 272 operand rows per K tile
constexpr int kStage = kRows * 8;          // 16-byte slots per stage
constexpr int kBlocks = kRows / 8;         // 34 DMA blocks of 8 rows
constexpr int kABlocks = BM / 8;           // 16
constexpr int kDmaPerWave = (kBlocks + 3) / 4;   // 9 (the last block repeats)
constexpr int kFrags = FM + FN;            // fragment reads per K step
constexpr int kSteps = FM * FN;            // MFMAs per K step
constexpr int kDmaSlot0 = kSteps - kDmaPerWave;   // the MFMA a tile's first DMA follows
static_assert(NS * kStage * 16 <= 160 * 1024, "LDS");
static_assert((NS - 1) * kDmaPerWave <= 63, "vmcnt range");
static_assert(kFrags <= kSteps && kDmaSlot0 >= 0, "reads and DMAs fit between the MFMAs");

}  // namespace mid

typedef float f32x4m __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2m __attribute__((ext_vector_type(2)));

// One K step (32 of K) of a wave's 2 x 9 blocks, W^T fragment first. ld(b) runs
// after the b-th MFMA (the next step's fragment reads, DMAs), each MFMA and its
// ld fenced so that the compiler keeps them interleaved (left to itself it read
// two fragments, waited for them, ran their MFMAs and so on: ~3x the MFMA time).
// kZero: the accumulators' first step (C = 0), so that no instruction writes
// them before an MFMA reads them (the compiler does not see these MFMAs and
// would not keep the wait states such a write needs).
template <bool kZero, class LD>
__device__ __forceinline__ void mid_step(f32x4m (&acc)[mid::FM][mid::FN],
                                         const u32x4 (&af)[mid::FM],
                                         const u32x4 (&bf)[mid::FN], LD&& ld) {
#pragma unroll
  for (int j = 0; j < mid::FN; ++j)
#pragma unroll
    for (int i = 0; i < mid::FM; ++i) {
      if (kZero)
        asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0"
                     : "=a"(acc[i][j])
                     : "v"(bf[j]), "v"(af[i]));
      else
        asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                     : "+a"(acc[i][j])
                     : "v"(bf[j]), "v"(af[i]));
      ld(j * mid::FM + i);
      __builtin_amdgcn_sched_barrier(0);
    }
}

// Output tile (tm, tn) of out = A Bt^T + bias, by the work-group's threads 0 ..
// 255 (waves 0-3; no other wave may be alive at its barriers). A (M rows, K), Bt
// (N rows, K), C (M, N) bf16 bits; bias (N) fp32; smem: NS kStage 16-byte slots.
// before(): runs after the first tile's W^T DMAs are issued and before any read of
// A (the one-launch forward's wait for its A rows).
template <class Before>
__device__ __forceinline__ void outproj_mid_tile(const uint16_t* __restrict__ A,
                                                 const uint16_t* __restrict__ Bt,
                                                 uint16_t* __restrict__ C,
                                                 const float* __restrict__ bias, int M, int N,
                                                 int K, int tm, int tn, u32x4* smem,
                                                 Before&& before) {
  using namespace mid;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nkt = K / 64;
  const int64_t row_bytes = (int64_t)K * 2;
  const int n0 = tn * BN;

  // this lane's bias columns: block j, columns 16 j + 4 (lane >> 4) + 0..3
  float4 bv[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j)
    bv[j] = *reinterpret_cast<const float4*>(bias + n0 + j * 16 + 4 * (lane >> 4));

  // DMA instruction d of this wave: block min(wave + 4 d, kBlocks - 1); blocks
  // below kABlocks are A rows, the rest W^T rows
  const char* abase = reinterpret_cast<const char*>(A) + (int64_t)tm * BM * row_bytes;
  const char* bbase = reinterpret_cast<const char*>(Bt) + (int64_t)n0 * row_bytes;
  auto dma_one = [&](int kt, int stage, int d) __attribute__((always_inline)) {
    u32x4* s = smem + stage * kStage;
    const int blk = cmin_dev(wave + 4 * d, kBlocks - 1);
    const int r = 8 * blk + (lane >> 3);   // stage row
    const char* src = blk < kABlocks ? abase + (int64_t)r * row_bytes
                                     : bbase + (int64_t)(r - BM) * row_bytes;
    src += (int64_t)kt * kTileKBytes + dma_chunk(lane, blk) * 16;
    // the LDS address goes through an integer (as in k_outproj_wide): with a
    // pointer the compiler makes the fragment reads of the other stages wait for
    // this DMA
    const uint32_t lds = (uint32_t)(size_t)(__attribute__((address_space(3))) u32x4*)(s + blk * 64);
    __builtin_amdgcn_global_load_lds((gbl_cvptr)src, (lds_vptr)(size_t)lds, 16, 0, 0);
  };

  f32x4m acc[FM][FN];   // written first by tile 0's first K step (C = 0)

  // fragment b of K step ks (32 of K) of a stage: b < FM the wave's A rows, else
  // the W^T rows of column block b - FM
  u32x4 fa[2][FM], fb[2][FN];   // [0]: the tile's first K step, [1]: its second
  auto frag = [&](const u32x4* s, int ks, int b, u32x4 (&af)[FM], u32x4 (&bf)[FN])
      __attribute__((always_inline)) {
    const int ch = ks * 4 + (lane >> 4);
    if (b < FM) af[b] = s[lds_slot(wave * 32 + b * 16 + (lane & 15), ch)];
    else bf[b - FM] = s[lds_slot(BM + (b - FM) * 16 + (lane & 15), ch)];
  };

  // prologue: tiles 0 .. NS - 2 in flight (those that exist): tile 0's W^T blocks
  // (DMA instructions d >= kADma of each wave), before(), tile 0's A blocks, then
  // tiles 1 and 2 whole; tile 0 landed, its first K step's fragments read. Only one
  // tile's W^T goes out before before(): a wait's first poll returns after every
  // DMA issued ahead of it (the in-order vmcnt), and three tiles' W^T (55 KB) put
  // ~1 us in front of the one-launch forward's poll (0.5 us per launch slower at
  // T = 2048 than this order, same output).
  constexpr int kADma = kABlocks / 4;   // a wave's A DMAs per tile: d < kADma
  static_assert(kABlocks % 4 == 0, "a wave's A blocks are its first DMAs of a tile");
#pragma unroll
  for (int d = kADma; d < kDmaPerWave; ++d) dma_one(0, 0, d);
  before();
#pragma unroll
  for (int d = 0; d < kADma; ++d) dma_one(0, 0, d);
#pragma unroll
  for (int t = 1; t < NS - 1; ++t)
    if (t < nkt)
#pragma unroll
      for (int d = 0; d < kDmaPerWave; ++d) dma_one(t, t, d);
  static_assert(NS == 4, "the waits below count the tiles issued after the one awaited");
  if (nkt > 2) wait_vm_lds<2 * kDmaPerWave>();
  else if (nkt > 1) wait_vm_lds<kDmaPerWave>();
  else wait_vm_lds<0>();
  lds_barrier();
#pragma unroll
  for (int b = 0; b < kFrags; ++b) frag(smem, 0, b, fa[0], fb[0]);

  // Each K tile: its first K step's MFMAs with the second step's fragment reads
  // between them; the wait for tile kt + 1 and the barrier; the second step's
  // MFMAs with tile kt + 1's first-step reads and the DMA of tile kt + NS - 1
  // (into the stage tile kt - 1 used: every wave read it before this barrier)
  // between them. Every iteration is the same code: past the last tile the
  // reads fetch a stage no MFMA uses and the DMAs fetch the last tile again (in
  // bounds, into a stage no later tile reads), so the wait has one count. With a
  // branch or a peeled last tile the compiler copied accumulators between AGPRs
  // right after the MFMAs that write them, which it cannot see through the
  // MFMAs' asm statements (a read of an MFMA result needs wait states first).
  for (int kt = 0; kt < nkt; ++kt) {
    const u32x4* s = smem + (kt % NS) * kStage;
    auto ld1 = [&](int b) __attribute__((always_inline)) {
      if (b < kFrags) frag(s, 1, b, fa[1], fb[1]);
    };
    if (kt == 0) mid_step<true>(acc, fa[0], fb[0], ld1);
    else mid_step<false>(acc, fa[0], fb[0], ld1);
    // tile kt + 1 has landed once at most the DMAs issued after it remain:
    // those of iteration kt - 1 (tile kt + 2 or a repeat; in iteration 0 the
    // prologue's tile 2, if there is one)
    if (kt == 0) {
      if (nkt > 2) wait_vm_lds<kDmaPerWave>();
      else wait_vm_lds<0>();
    } else {
      wait_vm_lds<kDmaPerWave>();
    }
    lds_barrier();
    const u32x4* sn = smem + ((kt + 1) % NS) * kStage;
    const int kd = cmin_dev(kt + NS - 1, nkt - 1), sd = (kt + NS - 1) % NS;
    mid_step<false>(acc, fa[1], fb[1], [&](int b) __attribute__((always_inline)) {
      if (b < kFrags) frag(sn, 0, b, fa[0], fb[0]);
      if (b >= kDmaSlot0) dma_one(kd, sd, b - kDmaSlot0);
    });
  }
  mfma_drain();
  wait_vm_lds<0>();   // the repeated DMAs land before the work-group's LDS is released

  // epilogue: lane l holds token 32 wave + 16 i + (l & 15), columns 16 j + 4 (l >> 4)
  // + 0..3; the tile goes through LDS (rows of 288 + 16 bytes) and out as 16-byte
  // chunks of whole rows
  constexpr int kOutRowBytes = BN * 2 + 16;
  lds_barrier();   // every wave's last fragment reads are done
  char* ot = reinterpret_cast<char*>(smem);
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int r = wave * 32 + i * 16 + (lane & 15);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      u32x2m v;
      v.x = pack_bf16x2(acc[i][j][0] + bv[j].x, acc[i][j][1] + bv[j].y);
      v.y = pack_bf16x2(acc[i][j][2] + bv[j].z, acc[i][j][3] + bv[j].w);
      *reinterpret_cast<u32x2m*>(ot + r * kOutRowBytes + (j * 16 + 4 * (lane >> 4)) * 2) = v;
    }
  }
  __syncthreads();
  constexpr int kChunks = BN * 2 / 16;   // 18 per row
  for (int c = threadIdx.x; c < BM * kChunks; c += 256) {
    const int r = c / kChunks, q = c - r * kChunks;
    const int row = tm * BM + r;
    if (row < M)
      *reinterpret_cast<u32x4*>(C + (int64_t)row * N + n0 + q * 8) =
          *reinterpret_cast<const u32x4*>(ot + r * kOutRowBytes + q * 16);
  }
}

// A (M rows, K), Bt (N rows, K), C (M, N) bf16 bits; bias (N) fp32.
__global__ __launch_bounds__(256) void k_outproj_mid(const uint16_t* __restrict__ A,
                                                     const uint16_t* __restrict__ Bt,
                                                     uint16_t* __restrict__ C,
                                                     const float* __restrict__ bias, int M,
                                                     int N, int K) {
  __shared__ u32x4 smem[mid::NS * mid::kStage];
  const int ntn = N / mid::BN;
  const int ntiles = ((M + mid::BM - 1) / mid::BM) * ntn;
  int tm, tn;
  tile_coords_of(blockIdx.x, ntn, ntiles, tm, tn);
  outproj_mid_tile(A, Bt, C, bias, M, N, K, tm, tn, smem, [] {});
}

}  // namespace dev
}  // namespace tmoe
