// k_fused_mid: the whole mid-T forward of a folded bf16 plan in one launch
// (model.py:68-102: router, top-k, softmax, in-projection, RMSNorm, the core and the
// out-projection as (c (x) z) W + bias) for the sizes whose front runs in K slices
// and whose out-projection tiles of 128 x 144 number at most 32 per XCD (T <= 2048
// at d_out = 2304): k_front_sliced's slices and per-token epilogues, then
// k_outproj_mid's tiles, in one persistent grid.
//
// One work-group of 8 waves per compute unit, 256 in all (8 XCDs x 32), each taking
// its XCD x from XCC_ID and its index i among that XCD's work-groups as b / 8 (as
// k_fused_large and k_front_sliced do). The out-projection's 128-token row tiles are
// dealt to the XCDs, row tile rt to XCD rt % 8, and with them their two 64-token
// front tiles 2 rt and 2 rt + 1, so that c (x) z passes from the front's epilogue to
// the out-projection's DMA inside one XCD's L2:
//  * phase 1: work-group i of XCD x computes K slice i % S of the XCD's front tile
//    i / S (front_slice_work: its plane, the slice flag, the wait for the tile's S
//    slices, the epilogue of 64 / S of the tile's tokens, whose c (x) z rows it
//    stores with plain stores), then sets its epilogue flag;
//  * phase 2: waves 4-7 end; waves 0-3 take the XCD's out-projection tile i (row tile
//    x + 8 (i / ntn), column tile i % ntn), issue the DMAs of its first W^T tile,
//    wait for the 2 S epilogue flags of its row tile's front tiles and run
//    k_outproj_mid's tile (outproj_mid_tile).
// Same slices, same arithmetic as k_front_sliced + k_outproj_mid: bit-identical.
//
// Every work-group finishes phase 1 before it waits in phase 2, and all work-groups
// are resident at once (the host launches this only on a device of 256 compute
// units, one work-group each), so every wait ends; waits are still bounded
// (FwdArgs::wait_polls) and a lost signal is reported in the status block (the
// consumer then reads whatever the rows hold, in bounds). A barrier waits for the
// waves of the work-group that have not ended, so phase 2's barriers count waves
// 0-3. The flags have several consumers and are never reset: the launcher keeps
// this kernel out of graph capture.
#pragma once

namespace tmoe {
namespace dev {

namespace fmid {
constexpr int kXcds = 8;            // XCDs of an MI355X
constexpr int kGroupsPerXcd = 32;   // compute units per XCD: one work-group each
constexpr int kGrid = kXcds * kGroupsPerXcd;
constexpr int kFrontPerRow = mid::BM / 64;   // 64-token front tiles per row tile
}  // namespace fmid

// raw: S planes (front_slice_work); the slice flags of front tile ft are
// sync_flag(ft S + sl), its epilogue flags sync_flag((n_ft + ft) S + sl). A = c (x) z
// (a.cz; T rows rounded up to 256), Wt = W^T (d_out, r1 r3), C = out, bias (d_out).
template <class Elt, int R3, int NR, int PFA, int BM, int NS, int WMF>
__global__ __launch_bounds__(64 * WMF * (R3 / 32 < 4 ? R3 / 32 : 4)) void k_fused_mid(
    FwdArgs a, float* __restrict__ raw, int S, const uint16_t* __restrict__ A,
    const uint16_t* __restrict__ Wt, uint16_t* __restrict__ C, const float* __restrict__ bias) {
  typedef FrontPartGeom<Elt, R3, NR, PFA, BM, NS, WMF> G;
  static_assert(BM * fmid::kFrontPerRow == mid::BM, "two front tiles per row tile");
  static_assert(64 * G::NWT >= 256, "the out-projection's four waves");
  // the out-projection's stages and one more slot for phase 2's wait
  constexpr int kSlots = cmax(G::kSmemBytes / 16, mid::NS * mid::kStage + 1);
  __shared__ u32x4 smem[kSlots];
  const int x = xcc_id(), i = (int)blockIdx.x / fmid::kXcds;
  const int n_ft = (int)((a.T + BM - 1) / BM);
  const int n_rt = (int)((a.T + mid::BM - 1) / mid::BM);
  const int nrx = (n_rt - x + fmid::kXcds - 1) / fmid::kXcds;   // row tiles x, x + 8, ...

  // -- phase 1: slice i % S of the XCD's front tile i / S ----------------------
  if (i < fmid::kFrontPerRow * nrx * S) {
    const int q = i / S, sl = i % S;
    const int ft = fmid::kFrontPerRow * (x + fmid::kXcds * (q / fmid::kFrontPerRow)) +
                   q % fmid::kFrontPerRow;
    if (ft < n_ft) {
      front_slice_work<Elt, R3, NR, PFA, BM, NS, WMF>(a, raw, S, ft, sl, smem);
      sync_publish(a.sync + sync_flag((int64_t)(n_ft + ft) * S + sl), a.epoch);
    }
  }

  // -- phase 2: the XCD's out-projection tile i, on waves 0-3 ------------------
  if (threadIdx.x >= 256) return;
  const int N = (int)a.d_out, K = (int)a.r2;
  const int ntn = N / mid::BN;
  if (i >= nrx * ntn) return;
  const int rt = x + fmid::kXcds * (i / ntn), tn = i % ntn;
  const int f0 = fmid::kFrontPerRow * rt;
  const int nf = n_ft - f0 < fmid::kFrontPerRow ? n_ft - f0 : fmid::kFrontPerRow;
  // the wait's word of LDS: the slot past the NS stages (the DMAs issued before the
  // wait write into the stages)
  int* seen_all = reinterpret_cast<int*>(smem + mid::NS * mid::kStage);
  // the first K tile's W^T DMAs go out before the wait; on a lost signal (reported) the tile
  // is computed from whatever the rows hold
  outproj_mid_tile(A, Wt, C, bias, (int)a.T, N, K, rt, tn, smem, [&] {
    (void)sync_await(a.sync + sync_flag((int64_t)(n_ft + f0) * S), nf * S, a.epoch, a.sync,
                     seen_all, false, a.wait_polls, a.status);
  });
}

}  // namespace dev
}  // namespace tmoe
