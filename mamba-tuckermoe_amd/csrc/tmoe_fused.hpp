// k_fused_large: the whole large-T forward of a folded bf16 plan in one launch
// (model.py:68-102: router, top-k, softmax, in-projection, RMSNorm, the core and the
// out-projection as (c (x) z) W + bias), for r3 = 256 and one router block
// (E_pad = 32), with d_out a multiple of 288.
//
// One work-group of 4 waves per compute unit, 256 in all (8 XCDs x 32). Work-groups
// are dispatched round robin over the XCDs, starting at an XCD that carries over
// from earlier dispatches (measured: b % 8 held for a run of launches, then, after
// other kernels, no longer), so a work-group takes its XCD x from the hardware's
// XCC_ID register and its index among that XCD's work-groups as b / 8, which under
// any rotation numbers each XCD's 32 work-groups 0..31. The 256-token row tiles of
// the output are dealt to the XCDs, row tile rt to XCD rt % 8; the 32 work-groups
// of an XCD first run the fronts of that XCD's row tiles (64-token tiles, four per
// row tile), each of which stores its c (x) z rows with plain stores and sets a
// flag, and then the
// out-projection tiles (256 x 288) of the same row tiles, whose A operand they read
// by DMA once the four flags of the row tile are set. Producer and consumers of a
// row of c (x) z share one XCD, so the rows pass through that XCD's L2: no L2
// write-back or invalidation is needed, and no launch boundary lies between the
// two phases (two launches cost ~10-12 us each at T = 16384 outside their work-
// groups' own time, much of it the write-back of the front's 33.5 MB).
//
// Every work-group finishes all its front tiles before it waits for any flag, and
// all 256 work-groups are resident at once (one per compute unit), so every wait
// ends; a wait is still bounded (FwdArgs::wait_polls) and reports a lost signal in
// the status block. A dispatch that is not a rotation would leave some (x, i) slot
// without a work-group (its front tiles unpublished: the waits for them run out and
// report) and give another two (which compute the same tiles, the same values).
// The flags have several consumers and are never reset, so the launcher keeps this
// kernel out of graph capture (a replay would reuse the epoch).
//
// The front tile (front4_tile) is k_front_ks's with the work of its 8 waves on 4:
// wave w owns all 64 rows x z columns 64 w .. 64 w + 63 over every K step (no K
// halves to add), its weight fragments straight from memory into VGPRs (the plan's
// fragment-order copy, three K tiles ahead), x through three LDS stages; the
// router's 32 columns take K step w of every K tile for both row blocks (four
// split-K planes, added in plane order by the top-k). The epilogue is k_front's
// (front_z_epilogue, front_topk, flush_cz). The out-projection tiles run
// k_outproj_wide's loop (wide_loop) over this work-group's tiles.
#pragma once

namespace tmoe {
namespace dev {

// Hardware id of the XCD the calling wave runs on (HW_REG_XCC_ID, bits 3:0).
__device__ __forceinline__ int xcc_id() {
  int v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(v));
  return v;
}

namespace fused {
constexpr int kXcds = 8;           // XCDs of an MI355X
constexpr int kGroupsPerXcd = 32;  // compute units per XCD: one work-group each
constexpr int kGrid = kXcds * kGroupsPerXcd;
constexpr int BM = 64;             // tokens per front tile
constexpr int kFrontPerRow = wide::BM / BM;   // front tiles per out-projection row tile
constexpr int RD = 4;              // weight ring slots (K tiles)
constexpr int DW = 3;              // weight K tiles loaded ahead
constexpr int DX = 5;              // x K tiles loaded ahead (stored to LDS 2 ahead)
constexpr int kXStage = BM * 8;    // 16-byte slots per x stage
constexpr int kPlanes = 4;         // split-K planes of the router logits

// The front tile's LDS: three x stages in the main loop; the epilogue's staged z
// tile, logits planes, RMSNorm partials, top-k record and U_expert after it.
template <int R3, int NR>
struct FrontGeom {
  static constexpr int EP = 32 * NR;
  // epilogue geometry: one row group of 4 waves side by side over the z columns
  typedef Tile<BM, R3, EP, 1, 4, 1, 1, 2, true, true, 0> TL;
  static constexpr int LD = EP + 1;
  static constexpr int kZBytes = TileStage<TL, uint16_t>::kBytes;
  static constexpr int kEpiBytes =
      kZBytes + (kPlanes * BM * LD + 4 * BM + BM + kTopkRecFloats<BM>) * 4;
  static constexpr int kBytes = cmax(3 * kXStage * 16, kEpiBytes + 4096);
};

// LDS of the kernel: the out-projection's two stages (the larger phase), then one
// 16-byte slot for the wait's answer
constexpr int kWideBytes = 2 * wide::Cfg<2>::kStage * 16;
constexpr int kCtrlSlot = kWideBytes / 16;
constexpr int kSmemSlots = kCtrlSlot + 1;
static_assert(FrontGeom<256, 1>::kBytes <= kWideBytes, "front tile LDS within the kernel's");
static_assert(kSmemSlots * 16 <= 160 * 1024, "LDS");

// Row tiles of XCD x (rt = x, x + 8, ...) among n_rt
__device__ __forceinline__ int xcd_rows(int n_rt, int x) {
  return n_rt > x ? (n_rt - x + kXcds - 1) / kXcds : 0;
}
}  // namespace fused

// The front of 64-token tile `tile` with 4 waves (see the file comment); stores
// c (x) z, c, idx and w of the tile's rows. smem: FrontGeom::kBytes of LDS.
template <int R3, int NR>
__device__ __forceinline__ void front4_tile(const FwdArgs& a, int tile,
                                            const uint16_t* __restrict__ wfrag, u32x4* smem) {
  typedef uint16_t T;
  using namespace fused;
  typedef FrontGeom<R3, NR> G;
  typedef typename G::TL TL;
  constexpr int FN = R3 / 128;           // z column blocks per wave
  constexpr int NCB = R3 / 32 + NR;      // fragment column blocks
  static_assert(R3 == 256, "4 waves of 64 z columns");
  static_assert(NR == 1, "one router block: four K steps, four waves");
  const int lane = threadIdx.x & 63;
  const int wn = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t m0 = (int64_t)tile * BM;
  const int rows_valid = (int)(a.T - m0 < BM ? a.T - m0 : BM);
  const int64_t row_bytes = a.d_in * (int64_t)sizeof(T);
  const int nkt = (int)(row_bytes / kTileKBytes);
  RowLoader al{reinterpret_cast<const char*>(a.x) + m0 * row_bytes, row_bytes, rows_valid};

  f32x16 acc[2][FN], racc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = zero16();
    racc[i] = zero16();
  }

  const char* wbase = reinterpret_cast<const char*>(wfrag);
  const uint32_t wlane = (uint32_t)lane * 16u;
  // this thread's two x chunks: rows xr0 and xr0 + 32, chunk xch
  const int xr0 = wn * 8 + (lane >> 3), xch = lane & 7;
  // rings (slot = K tile % RD): x tiles DX ahead, weight tiles DW ahead
  u32x4 xr[RD][2], wz[RD][4][FN], wr[RD];
  auto load_x = [&](int kt, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h) xr[slot][h] = al.fetch(xr0 + 32 * h, xch, kt);
  };
  auto load_w = [&](int kt, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int g = 4 * kt + s, cb = wn * FN + j;
        wz[slot][s][j] = gload_sbase(wbase + ((int64_t)g * NCB + cb) * 1024, wlane);
      }
    const int g = 4 * kt + wn, cb = R3 / 32;
    wr[slot] = gload_sbase(wbase + ((int64_t)g * NCB + cb) * 1024, wlane);
  };
  auto stash = [&](int slot, int stage) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h) smem[stage * kXStage + lds_slot(xr0 + 32 * h, xch)] = xr[slot][h];
  };
  // x fragments of K step s of the tile in LDS stage `stage`: [row block]
  auto read_x = [&](u32x4 (&xf)[2], int stage, int s) __attribute__((always_inline)) {
    const u32x4* st = smem + stage * kXStage;
#pragma unroll
    for (int i = 0; i < 2; ++i) xf[i] = st[lds_slot(i * 32 + (lane & 31), 2 * s + (lane >> 5))];
  };

  // prologue (past the last tile the last one is fetched again: in bounds, into a
  // slot or stage no later tile reads): x tiles 0 .. RD - 1, weight tiles
  // 0 .. DW - 1; x tiles 0 and 1 into stages 0 and 1, then x tile RD into the slot
  // tile 0 left
#pragma unroll
  for (int t = 0; t < RD; ++t) load_x(cmin_dev(t, nkt - 1), t);
#pragma unroll
  for (int t = 0; t < DW; ++t) load_w(cmin_dev(t, nkt - 1), t);
  stash(0, 0);
  stash(1, 1);
  load_x(cmin_dev(RD, nkt - 1), 0);
  wait_vm_lds<63>();   // the LDS stores (lgkmcnt 0); the loads stay in flight
  lds_barrier();
  u32x4 xf[2][2];      // x fragments of the current and the next K step
  read_x(xf[0], 0, 0);

  // Iteration kt (ring slot p = kt % RD): the 4 K steps of tile kt, each step's
  // MFMAs from fragments read one step ahead (the last step reads step 0 of tile
  // kt + 1, stage (kt + 1) % 3, stored an iteration ago); the router's K step wn
  // from fragments read at the start; x tile kt + 2 stored into the stage tile
  // kt - 1 used; loads of x tile kt + DX and weight tile kt + DW into the slots
  // tiles kt + 1 and kt - 1 left.
  auto iteration = [&](int kt, int p) __attribute__((always_inline)) {
    const int stage = kt % 3;
    u32x4 xs[2];
    read_x(xs, stage, wn);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s < 3) read_x(xf[(s + 1) & 1], stage, s + 1);
      else read_x(xf[0], (kt + 1) % 3, 0);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) mma(acc[i][j], xf[s & 1][i], wz[p][s][j], EltBF16{});
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) mma(racc[i], xs[i], wr[p], EltBF16{});
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
    for (int p = 0; p < RD; ++p) iteration(k0 + p, p);
  }
#pragma unroll
  for (int p = 0; p + 1 < RD; ++p)
    if (k0 + p < nkt) iteration(k0 + p, p);
  wait_vm_lds<0>();   // the refetches past the last tile
  lds_barrier();

  // -- router logits -> LDS: plane wn, both row blocks -------------------------
  char* zst = reinterpret_cast<char*>(smem);
  float* lg = reinterpret_cast<float*>(zst + G::kZBytes);
  float* rred = lg + kPlanes * BM * G::LD;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e)
      lg[(wn * BM + i * 32 + acc_row(lane, e)) * G::LD + (lane & 31)] = racc[i][e];
  front_z_epilogue<TL, EltBF16, R3>(acc, a, m0, rows_valid, zst, rred);
  front_topk<G::EP, BM, 256, kPlanes>(a, m0, rows_valid, lg, G::LD, rred + 4 * BM + BM,
                                      kWideBytes - G::kEpiBytes, lg);
  __syncthreads();
  flush_cz<TL, R3>(zst, lg, a, m0, rows_valid);
}

// Out-projection tiles of work-group (x, i): o = i, i + 32, ... of its XCD's
// n_rt_x * ntn tiles, tile o = (row tile x + 8 (o / ntn), column tile o % ntn).
struct FusedSched {
  int x, o, n_tasks, ntn;
  __device__ __forceinline__ void coords(int& tm, int& tn) const {
    const int j = o / ntn;
    tm = x + fused::kXcds * j;
    tn = o - j * ntn;
  }
  __device__ __forceinline__ bool start(int& tm, int& tn) {
    if (o >= n_tasks) return false;
    coords(tm, tn);
    return true;
  }
  __device__ __forceinline__ bool advance(int& tm, int& tn) {
    o += fused::kGroupsPerXcd;
    if (o >= n_tasks) return false;
    coords(tm, tn);
    return true;
  }
};

// a: the folded forward's arguments (a.mid = a.cz = c (x) z, a.uoutT = W^T,
// a.r2 = K = r1 r3); A, Wt, C, bias: a.cz, a.uoutT, a.out, a.bias as restrict
// parameters (the bias is then read through the scalar unit).
template <int R3, int NR>
__global__ __launch_bounds__(256) void k_fused_large(FwdArgs a, const uint16_t* __restrict__ wfrag,
                                                     const uint16_t* __restrict__ A,
                                                     const uint16_t* __restrict__ Wt,
                                                     uint16_t* __restrict__ C,
                                                     const float* __restrict__ bias) {
  using namespace fused;
  __shared__ u32x4 smem[kSmemSlots];
  const int x = xcc_id(), i = (int)blockIdx.x / kXcds;
  const int n_rt = (int)((a.T + wide::BM - 1) / wide::BM);
  const int n_ft = (int)((a.T + BM - 1) / BM);
  const int nrx = xcd_rows(n_rt, x);

  // -- the front tiles of this XCD's row tiles: f = i, i + 32, ... -------------
  for (int f = i; f < kFrontPerRow * nrx; f += kGroupsPerXcd) {
    const int ft = kFrontPerRow * (x + kXcds * (f / kFrontPerRow)) + f % kFrontPerRow;
    if (ft >= n_ft) continue;   // past T in the last row tile
    front4_tile<R3, NR>(a, ft, wfrag, smem);
    sync_publish(a.sync + sync_flag(ft), a.epoch);
    __syncthreads();   // the tile's LDS is free before the next one
  }

  // -- out-projection tiles ---------------------------------------------------
  const int N = (int)a.d_out, K = (int)a.r2;
  FusedSched sched{x, i, nrx * (N / wide::BN), N / wide::BN};
  if (sched.o >= sched.n_tasks) return;
  {
    // wait once for the flags of every front tile this work-group's tiles read:
    // tile k of the work-group (o = i + 32 k) reads row tile x + 8 (o / ntn), whose
    // front tiles are 4 rt .. 4 rt + 3 (those below n_ft)
    const int n_my = (sched.n_tasks - i + kGroupsPerXcd - 1) / kGroupsPerXcd;
    const int nfl = kFrontPerRow * n_my;
    int* seen_all = reinterpret_cast<int*>(smem + kCtrlSlot);
    if (threadIdx.x < 64) {
      const int l = threadIdx.x;
      int next = l;   // lane's next flag index (l, l + 64, ...)
      auto flag_of = [&](int q) -> int {
        const int o = i + kGroupsPerXcd * (q / kFrontPerRow);
        const int rt = x + kXcds * (o / sched.ntn);
        const int ft = kFrontPerRow * rt + q % kFrontPerRow;
        return ft < n_ft ? ft : -1;   // -1: no such front tile, nothing to wait for
      };
      auto settled = [&](int q) -> bool {
        const int ft = flag_of(q);
        return ft < 0 || __hip_atomic_load(a.sync + sync_flag(ft), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT) == a.epoch;
      };
      bool seen = false;
      for (int p = 0; p < a.wait_polls; ++p) {
        while (next < nfl && settled(next)) next += 64;
        if (__all(next >= nfl)) {
          seen = true;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      if (!seen && l == 0) {
        __hip_atomic_store(a.sync, a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        report_status(a.status, kStatusSignal);
      }
      if (l == 0) *seen_all = seen ? 1 : 0;
    }
    __syncthreads();
    // on a lost signal the tiles are computed from whatever the rows hold (in
    // bounds); the status block reports the error
  }
  wide_loop<2>(A, Wt, C, bias, (int)a.T, N, K, smem, sched);
}

}  // namespace dev
}  // namespace tmoe
