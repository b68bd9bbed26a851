// k_front_sliced: the K-sliced mid-T front in one launch (model.py:75-81 and the
// U_expert gather of :93): k_front_part's tiles and K slices, then k_front_epi's
// per-token epilogue over the slices' fp32 planes, without a launch between them.
//
// One work-group per compute unit, 256 in all (8 XCDs x 32), each taking its XCD x
// from the hardware's XCC_ID register and its index i among that XCD's work-groups
// as b / 8 (work-groups are dispatched round robin over the XCDs, from an XCD that
// carries over between launches: i numbers each XCD's 32 work-groups 0..31 under
// any rotation). The 64-token tiles are dealt to the XCDs, tile ft to XCD ft % 8,
// and work-group i of XCD x computes K slice i % S of the XCD's tile i / S: its
// plane of fp32 partial sums (z columns and router logits) goes to the workspace
// with plain stores, then it sets the slice's flag. It then waits for the S flags
// of its tile and runs the epilogue of its share of the tile's tokens (the sl-th
// of S equal parts of the 64), reading the S planes in plane order. Producers and
// consumers of a tile's planes share one XCD, so the planes pass through that
// XCD's L2: no write-back or invalidation of L2 is needed (the consumer's vector
// L1 holds none of those lines: the launch began with it invalidated and the
// work-group reads no plane before the flags are set).
//
// The arithmetic is k_front_part + k_front_epi's with the same S slices (same K
// ranges, planes added in the same order): the two-launch path is bit-identical.
//
// Every work-group publishes its slice before it waits, and all work-groups are
// resident at once (the host launches this only on a device of 256 compute units,
// one work-group each), so every wait ends; a wait is still bounded
// (FwdArgs::wait_polls) and a lost signal is reported in the status block (the
// epilogue then reads whatever the planes hold, in bounds). A dispatch that is not
// a rotation would leave some (x, i) slot without a work-group: the waits for its
// slice run out and report. The flags have several consumers and are never reset,
// so the launcher keeps this kernel out of graph capture (a replay would reuse the
// epoch).
#pragma once

namespace tmoe {
namespace dev {

namespace sliced {
constexpr int kXcds = 8;            // XCDs of an MI355X
constexpr int kGroupsPerXcd = 32;   // compute units per XCD: one work-group each
constexpr int kGrid = kXcds * kGroupsPerXcd;
}  // namespace sliced

// Slice sl of front tile ft, then the epilogue of its share of the tile's tokens:
// k_front_sliced's work for one (tile, slice), by all the work-group's threads.
// raw: S planes of T rows of raw_stride(r3, E) floats; the flags of tile ft are
// sync_flag(ft S) .. sync_flag(ft S + S - 1). smem: FrontPartGeom::kSmemBytes.
template <class Elt, int R3, int NR, int PFA, int BM, int NS, int WMF>
__device__ __forceinline__ void front_slice_work(const FwdArgs& a, float* __restrict__ raw,
                                                 int S, int ft, int sl, u32x4* smem) {
  typedef FrontPartGeom<Elt, R3, NR, PFA, BM, NS, WMF> G;
  constexpr int kThreads = 64 * G::NWT;
  // U_expert: E <= E_pad <= 128 experts (the K-sliced front's routers), r1 <= 64
  static_assert(G::kSmemBytes >= 16 + 4 * 64 * 128, "U_expert fits the LDS");
  front_part_tile<Elt, R3, NR, PFA, BM, NS, WMF>(a, raw, S, ft, sl, smem);
  sync_publish(a.sync + sync_flag((int64_t)ft * S + sl), a.epoch);

  // U_expert (E x r1 floats) into LDS while the other slices finish (the main
  // loop's LDS is free: sync_publish ended with a barrier); word 0 is the wait's
  const int E = (int)a.E, R1 = (int)a.r1;
  int* seen_all = reinterpret_cast<int*>(smem);
  float* ue = reinterpret_cast<float*>(smem + 1);
  for (int j = threadIdx.x; j < E * R1; j += kThreads) ue[j] = a.uexp[j];
  // on a lost signal (reported) the epilogue reads whatever the planes hold
  (void)sync_await(a.sync + sync_flag((int64_t)ft * S), S, a.epoch, a.sync, seen_all, false,
                   a.wait_polls, a.status);   // ends with a barrier: ue is in place

  // the epilogue of this slice's share of the tile's tokens, one token per wave
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t m0 = (int64_t)ft * BM;
  const int64_t t0 = m0 + (int64_t)sl * BM / S;
  int64_t t1 = m0 + (int64_t)(sl + 1) * BM / S;
  if (t1 > a.T) t1 = a.T;
  const int64_t plane_stride = a.T * raw_stride(R3, E);
  for (int64_t t = t0 + wave; t < t1; t += G::NWT) {
    EpiLoad L;
    epi_load<R3 / 64, kMaxFrontPlanes, 2>(a, raw, S, plane_stride, t, lane, L);
    epi_finish<Elt, R3 / 64>(a, t, lane, L, ue, true, true, nullptr, nullptr);
  }
}

template <class Elt, int R3, int NR, int PFA, int BM, int NS, int WMF>
__global__ __launch_bounds__(64 * WMF * (R3 / 32 < 4 ? R3 / 32 : 4)) void k_front_sliced(
    FwdArgs a, float* __restrict__ raw, int S) {
  typedef FrontPartGeom<Elt, R3, NR, PFA, BM, NS, WMF> G;
  __shared__ u32x4 smem[G::kSmemBytes / 16];
  const int x = xcc_id(), i = (int)blockIdx.x / sliced::kXcds;
  const int n_ft = (int)((a.T + BM - 1) / BM);
  const int nfx = (n_ft - x + sliced::kXcds - 1) / sliced::kXcds;   // tiles x, x + 8, ...
  if (i >= nfx * S) return;   // no slice for this work-group
  front_slice_work<Elt, R3, NR, PFA, BM, NS, WMF>(a, raw, S, x + sliced::kXcds * (i / S), i % S,
                                                  smem);
}

}  // namespace dev
}  // namespace tmoe
