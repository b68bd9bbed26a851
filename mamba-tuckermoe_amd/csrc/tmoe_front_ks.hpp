// k_front_ks: the large-T bf16 front (model.py:75-81) with the weight operand in
// registers, for r3 = 256 and one router block (E_pad = 32; with two the kernel
// needs more registers than a wave has and spills).
//
// A work-group of 8 waves owns 64 tokens. Wave w = (kh = w / 4, wn = w % 4) owns
// all 64 rows x the FN column blocks wn*FN .. of z for the K steps 2 kh, 2 kh + 1
// of every K tile (a K split in two halves), so no two waves use the same weight
// fragment: the weights come straight from memory into VGPRs, in a fragment
// layout packed once with the plan (the wfrag region, k_pack_frag), one coalesced
// 1 KB load per fragment, DW K tiles ahead (a ring of RD tiles). x, which all
// column waves share, goes through LDS: each wave loads one 1 KB block of 8 rows
// per K tile into the same ring and stores it to one of three LDS stages two tiles
// ahead. (With x by LDS DMA the compiler waited for every outstanding load before
// the fragment reads, the weight loads included.) The router's 32-column blocks
// take one MFMA per wave and K tile: wave (wn, kh) runs K step 2 kh + (wn & 1) of
// row block wn >> 1, so its partial logits are plane 2 kh + (wn & 1) of four
// split-K planes (front_topk adds planes in plane order). After the K loop the two
// K halves of z are added through LDS (wave (wn, kh) keeps row block kh) and the
// epilogue is k_front's (front_z_epilogue, front_topk, flush_cz). Against k_front
// the z sums are associated differently (two K halves), so z and c (x) z may
// differ from it in the last bf16 place; the routing outputs are the same sums.
#pragma once

namespace tmoe {
namespace dev {

// 16-byte load at uniform base + 32-bit per-lane offset, in the scalar-base form
// (the base pinned to SGPRs: left alone, the compiler hoisted base + lane offset
// into a 64-bit VGPR pointer per load)
typedef const __attribute__((address_space(1))) char* gchar_ptr;
__device__ __forceinline__ u32x4 gload_sbase(const char* base, uint32_t voff) {
  gchar_ptr b = (gchar_ptr)base;
  asm volatile("" : "+s"(b));
  return *(const __attribute__((address_space(1))) u32x4*)(b + voff);
}

namespace fks {
constexpr int BM = 64;     // tokens per work-group
constexpr int RD = 4;      // weight ring slots (K tiles)
constexpr int DW = 3;      // weight K tiles loaded ahead
constexpr int DX = 5;      // x K tiles loaded ahead (stored to LDS 2 ahead)
constexpr int kXStage = BM * 8;   // 16-byte slots per x stage
}  // namespace fks

// wfrag: fragment (g, cb) of the front operand [U_in^T ; W_r ; 0] (NCB column
// blocks of 32, K steps g of 16) at byte ((g * NCB) + cb) * 1024; lane l's 16
// bytes are row 32 cb + (l & 31), elements 16 g + 8 (l >> 5) .. + 7.
//
// k_pack_frag writes that layout from the packed front operand (N = 32 NCB rows of
// d_in elements, row-major): one thread per 16-byte chunk.
__global__ void k_pack_frag(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                            int64_t ncb, int64_t d_in) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // chunk index
  const int64_t nchunks = (d_in / 16) * ncb * 64;
  if (q >= nchunks) return;
  const int l = (int)(q & 63);
  const int64_t f = q >> 6;                  // fragment g * ncb + cb
  const int64_t g = f / ncb, cb = f - g * ncb;
  const int64_t row = 32 * cb + (l & 31), col = 16 * g + 8 * (l >> 5);
  *reinterpret_cast<u32x4*>(dst + q * 8) = *reinterpret_cast<const u32x4*>(src + row * d_in + col);
}

template <int R3, int NR>
__global__ __launch_bounds__(512) void k_front_ks(FwdArgs a, const uint16_t* __restrict__ wfrag) {
  typedef uint16_t T;
  using namespace fks;
  constexpr int EP = 32 * NR;
  constexpr int FN = R3 / 128;           // z column blocks per wave
  constexpr int NCB = R3 / 32 + NR;      // fragment column blocks
  constexpr int kWPerTile = 2 * FN + NR; // weight fragment loads per wave and K tile
  constexpr int kOps = 1 + kWPerTile;    // vector memory instructions per wave and K tile
  static_assert(R3 == 128 || R3 == 256, "4 column waves of 32 or 64 z columns");
  static_assert(NR >= 1 && NR <= 3, "router split over K");
  static_assert(kOps * DW < 63, "vmcnt range");
  // epilogue geometry: k_front's 64-token tile (2 row groups x 4 column waves)
  typedef Tile<BM, R3, EP, 2, 4, 1, 1, 2, true, true, 0> TL;
  typedef RouterExtra<EltBF16, 1, NR, 4> RX;
  constexpr int LD = EP + 1;
  constexpr int kPlanes = 4;
  constexpr int kZBytes = TileStage<TL, T>::kBytes;
  constexpr int kEpiBytes = kZBytes + (kPlanes * BM * LD + 4 * BM + BM + kTopkRecFloats<BM>) * 4;
  constexpr int kRedBytes = 8 * FN * 16 * 64 * 4;   // the K halves' exchanged row blocks
  constexpr int kSmemBytes = cmax(cmax(3 * kXStage * 16, kRedBytes), kEpiBytes + 4096);
  static_assert(kSmemBytes <= 160 * 1024, "LDS");
  __shared__ u32x4 smem[kSmemBytes / 16];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kh = wave >> 2, wn = wave & 3;
  const int64_t m0 = (int64_t)blockIdx.x * BM;
  const int rows_valid = (int)(a.T - m0 < BM ? a.T - m0 : BM);
  const int64_t row_bytes = a.d_in * (int64_t)sizeof(T);
  const int nkt = (int)(row_bytes / kTileKBytes);
  RowLoader al{reinterpret_cast<const char*>(a.x) + m0 * row_bytes, row_bytes, rows_valid};

  f32x16 acc[2][FN], racc[NR];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = zero16();
#pragma unroll
  for (int r = 0; r < NR; ++r) racc[r] = zero16();

  // uniform fragment addresses plus one 32-bit lane offset (scalar-base loads)
  const char* wbase = reinterpret_cast<const char*>(wfrag);
  const uint32_t wlane = (uint32_t)lane * 16u;
  const int rks = 2 * kh + (wn & 1);   // the router's K step in a tile
  // this wave's block of x: row 8 wave + (lane >> 3), chunk lane & 7
  const int xrow = wave * 8 + (lane >> 3), xch = lane & 7;
  // rings (slot = K tile % RD): x tiles DX ahead, weight tiles DW ahead
  u32x4 xr[RD], wz[RD][2][FN], wr[RD][NR];
  auto load_x = [&](int kt, int slot) __attribute__((always_inline)) {
    xr[slot] = al.fetch(xrow, xch, kt);
  };
  auto load_w = [&](int kt, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int g = 4 * kt + 2 * kh + s2, cb = wn * FN + j;
        wz[slot][s2][j] = gload_sbase(wbase + ((int64_t)g * NCB + cb) * 1024, wlane);
      }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int g = 4 * kt + rks, cb = R3 / 32 + r;
      wr[slot][r] = gload_sbase(wbase + ((int64_t)g * NCB + cb) * 1024, wlane);
    }
  };
  // x of ring slot `slot` into LDS stage `stage`
  auto stash = [&](int slot, int stage) __attribute__((always_inline)) {
    smem[stage * kXStage + lds_slot(xrow, xch)] = xr[slot];
  };
  // x fragments of the tile in LDS stage `stage`: [s2][row block]
  auto read_x = [&](u32x4 (&xf)[2][2], int stage) __attribute__((always_inline)) {
    const u32x4* s = smem + stage * kXStage;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int i = 0; i < 2; ++i)
        xf[s2][i] = s[lds_slot(i * 32 + (lane & 31), 2 * (2 * kh + s2) + (lane >> 5))];
  };

  // prologue (past the last tile the last one is fetched again: in bounds, into
  // a slot or stage no later tile reads): x tiles 0 .. RD - 1, weight tiles
  // 0 .. DW - 1; x tiles 0 and 1 into stages 0 and 1, then x tile RD into the
  // slot tile 0 left
#pragma unroll
  for (int t = 0; t < RD; ++t) load_x(cmin_dev(t, nkt - 1), t);
#pragma unroll
  for (int t = 0; t < DW; ++t) load_w(cmin_dev(t, nkt - 1), t);
  stash(0, 0);
  stash(1, 1);
  load_x(cmin_dev(RD, nkt - 1), 0);
  wait_vm_lds<63>();   // the LDS stores (lgkmcnt 0); the loads stay in flight
  lds_barrier();
  u32x4 xf[2][2][2];   // x fragments of tiles kt (buffer kt & 1) and kt + 1
  read_x(xf[0], 0);

  // Iteration kt (ring slot p = kt % RD, fragment buffer b = kt & 1): fragments
  // of tile kt + 1 (stage (kt + 1) % 3, stored an iteration ago) read under the
  // MFMAs of tile kt; x tile kt + 2 stored into the stage tile kt - 1 used (its
  // fragments were read before the last barrier but one); loads of x tile
  // kt + DX and weight tile kt + DW into the slots tiles kt + 1 and kt left.
  auto iteration = [&](int kt, int p, int b) __attribute__((always_inline)) {
    read_x(xf[b ^ 1], (kt + 1) % 3);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) mma(acc[i][j], xf[b][s2][i], wz[p][s2][j], EltBF16{});
    // router: K step s2 = wn & 1 of row block wn >> 1, the operand picked by
    // selects (branches around the MFMA made the compiler copy its accumulators)
    {
      const u32x4 x0 = (wn >> 1) ? xf[b][0][1] : xf[b][0][0];
      const u32x4 x1 = (wn >> 1) ? xf[b][1][1] : xf[b][1][0];
      const u32x4 xs = (wn & 1) ? x1 : x0;
#pragma unroll
      for (int r = 0; r < NR; ++r) mma(racc[r], xs, wr[p][r], EltBF16{});
    }
    mfma_drain();
    stash((p + 2) % RD, (kt + 2) % 3);
    load_x(cmin_dev(kt + DX, nkt - 1), (p + DX) % RD);
    load_w(cmin_dev(kt + DW, nkt - 1), (p + DW) % RD);
    wait_vm_lds<63>();
    lds_barrier();
  };
  static_assert(RD == DW + 1 && DX == RD + 1 && RD % 2 == 0, "load rings");
  int k0 = 0;
  for (; k0 + RD <= nkt; k0 += RD) {
#pragma unroll
    for (int p = 0; p < RD; ++p) iteration(k0 + p, p, p & 1);
  }
#pragma unroll
  for (int p = 0; p + 1 < RD; ++p)
    if (k0 + p < nkt) iteration(k0 + p, p, p & 1);
  wait_vm_lds<0>();   // the refetches past the last tile
  lds_barrier();

  // -- the K halves of z: wave (wn, kh) keeps row block kh, gives row block 1 - kh
  float* red = reinterpret_cast<float*>(smem);
  f32x16 accz[1][FN];
  {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const f32x16 give = kh ? acc[0][j] : acc[1][j];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float4 v = {give[4 * q], give[4 * q + 1], give[4 * q + 2], give[4 * q + 3]};
        *reinterpret_cast<float4*>(red + (((wave * FN + j) * 4 + q) * 64 + lane) * 4) = v;
      }
    }
    __syncthreads();
    const int pw = wave ^ 4;   // the other K half's wave of this column range
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      f32x16 keep = kh ? acc[1][j] : acc[0][j];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 v = *reinterpret_cast<const float4*>(red + (((pw * FN + j) * 4 + q) * 64 + lane) * 4);
        keep[4 * q] += v.x; keep[4 * q + 1] += v.y; keep[4 * q + 2] += v.z; keep[4 * q + 3] += v.w;
      }
      accz[0][j] = keep;
    }
    __syncthreads();
  }

  // -- router logits -> LDS: plane 2 kh + (wn & 1), rows of row block wn >> 1 --
  char* zst = reinterpret_cast<char*>(smem);
  float* lg = reinterpret_cast<float*>(zst + kZBytes);
  float* rred = lg + kPlanes * BM * LD;
  {
    const int plane = 2 * kh + (wn & 1), rb = wn >> 1;
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        lg[(plane * BM + rb * 32 + acc_row(lane, e)) * LD + r * 32 + (lane & 31)] = racc[r][e];
  }
  front_z_epilogue<TL, EltBF16, R3>(accz, a, m0, rows_valid, zst, rred);
  front_topk<EP, BM, 512, kPlanes>(a, m0, rows_valid, lg, LD, rred + 4 * BM + BM,
                                   kSmemBytes - kEpiBytes, a.cz ? lg : nullptr);
  if (a.cz) {
    __syncthreads();
    flush_cz<TL, R3>(zst, lg, a, m0, rows_valid);
  }
}

}  // namespace dev
}  // namespace tmoe
