// Internal interface between the C-ABI host code (tmoe_api.cpp) and the gfx950
// kernels (tmoe_kernels.hip). Not installed; the public ABI is include/tmoe.h.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tmoe {

// Tile geometry shared by the host (workspace / grid sizing, validation) and
// the kernels. K-direction tiles are 128 bytes of one operand row: 64 bf16 or
// 32 f32 elements.
constexpr int kTileKBytes = 128;
// Bytes of the static scratch of tmoe_forward_static (tmoe_static.hip): the
// forward's workspace for up to T = 16384 tokens at the reference's C3 shape.
constexpr size_t kStaticScratchBytes = (size_t)48 << 20;
// Device address of the static scratch on the GPU that `stream` belongs to (the
// current GPU for the null stream), looked up once per GPU.
hipError_t static_scratch(hipStream_t stream, void** ptr);

constexpr int kFrontBM = 64;    // tokens per k_front work-group (whole r3 and E rows)
// depth of an x register ring (Tile's PFA); the fronts' loops now bring x to LDS
// by DMA, where the ring depth has no effect
constexpr int kFrontPFA = 8;
constexpr int kFrontWM = 2;     // row groups of waves per k_front work-group
constexpr int kMaxTopK = 16;
constexpr int kMaxExperts = 256;

// Device pointers of one forward, resolved by the host.
struct FwdArgs {
  int dtype;                    // TMOE_BF16 / TMOE_F32
  int router_mode;              // TMOE_ROUTER_SOFTMAX_TOPK / TMOE_ROUTER_CAPPED
  float router_scale, router_temperature;   // router_mode 1
  int64_t T, d_in, d_out, E, E_pad, k, r1, r2, r3;
  float eps;
  const void* x;
  // packed weights
  const void* wfront;           // (r3 + E_pad, d_in)   U_in^T rows, then router rows
                                //                      (zero rows past E)
  const void* wfrag;            // wfront in k_front_ks's fragment order (bf16 plans
                                //                      with r3 = 256, E_pad = 32), else null
  const float* gain;            // (r3)                 inner_norm.weight
  const float* uexp;            // (E, r1)              U_expert
  const void* coreT;            // (r2, r1*r3)          core as (r1*r3, r2), transposed
  const void* coreP;            // (r1*r2, r3)          k_core_pp's P^T: row (qb*r1 + r)*32 + qq
                                //                      = channel (r, 32 qb + qq); null when
                                //                      the plan does not use k_core_pp
  const void* uoutT;            // (d_out, r2)          U_out transposed
  const float* bias;            // (d_out)
  // fp8-weight plans only (null otherwise): per-output-channel scales
  const float* zscale;          // (r3)                 U_in column scales
  const float* core_scale;      // (r1, r2)             rank-change ratios, last rank's scales
  const float* out_scale;       // (d_out)              U_out column scales
  const float* core_scale_raw;  // (r1, r2)             core channel scales (small-T path)
  // outputs / workspace
  void* out;
  int32_t* idx;                 // (T, k)
  float* w;                     // (T, k)
  float* logits;                // (T, E) or null
  float* c;                     // (T, r1)
  void* z;                      // (T, r3)
  void* mid;                    // (T, r2); folded plans: c (x) z (T, r1*r3)
  bool mid_rows_256;            // mid is allocated for T rounded up to 256 rows
  void* cz;                     // folded plans whose front writes c (x) z itself (= mid;
                                //                      then z is not stored), else null
  bool kr;                      // folded plans whose out-projection forms c (x) z from z
                                //                      and c in its loop (outproj_kr_ok):
                                //                      no c (x) z is stored; z and c are
                                //                      allocated for T rounded up to 256 rows
  float* raw;                   // (T, raw_stride) fp32 small-T path: x [U_in | W_r^T];
                                //                      K-sliced front: front_split planes
  float* mpart;                 // (S, T_pad, r2) fp32  k_core_pp with r1 > 4: partial sums
                                //                      over rank groups (null otherwise)
  int core_split;               // S: parts an output tile's rank groups are split into
  int front_split;              // K slices of the large-T front (raw holds that many
                                //                      (T, r3 + E) fp32 planes), 1: none
  bool front_one;               // front_split > 1: slices and epilogue in one launch
                                //                      (k_front_sliced, front_sliced_ok)
  // elementwise op fused into the out-projection's store (kEpi*): the FFN
  // sub-block's silu(gate) * up, or its residual + LayerScale
  int epi_mode;
  const void* epi_a;            // (T, d_out) dtype     gate output / residual input
  const void* epi_b;            // (d_out) dtype        LayerScale gamma
  // signals between the work-groups of one launch (kernels that publish data for
  // other work-groups of the same grid): sync[0] records a wait that ran out of
  // time, sync[sync_flag(i)] is flag i; epoch is the value a flag takes when
  // published, drawn fresh by the launcher (next_epoch)
  uint32_t* sync;
  uint32_t epoch;
  // a wait for a flag gives up after this many polls (kDefaultWaitPolls unless the
  // host set another budget; 0: at once), then sets word kStatusSignal of `status`
  int wait_polls;
  // the plan's status block in host-visible memory (words kStatus*, set to 1 by a
  // kernel that met the condition; read by tmoe_signal_status), or null
  uint32_t* status;
};

// Default budget of a wait for an in-launch signal, in polls of its flags (a poll is
// a device-scope load round trip plus ~128 clocks of sleep: about a second in all)
constexpr int kDefaultWaitPolls = 1000000;
// words of a plan's status block (host memory mapped for the device): word
// kStatusSignalWord is set when a wait ran out of polls (the others are spare)
constexpr int kStatusWords = 4;
constexpr int kStatusSignalWord = 0;

// FwdArgs::sync: the error word, then one flag per 32-token tile of the largest T a
// launch that signals may have, each flag alone in its 256-byte block (polls and
// publications of different flags do not meet on one cache line)
constexpr int64_t kSyncTileRows = 32;
constexpr int64_t kSyncStride = 64;   // words
// flags: one per 32-token tile, at least min_flags (the small-T decode kernel's
// producers)
constexpr int64_t sync_words(int64_t T, int64_t min_flags = 0) {
  return kSyncStride * (1 + ((T + kSyncTileRows - 1) / kSyncTileRows > min_flags
                                 ? (T + kSyncTileRows - 1) / kSyncTileRows : min_flags));
}
constexpr int64_t sync_flag(int64_t i) { return kSyncStride * (1 + i); }
// a nonzero value no earlier launch of this process used (the counter starts at a
// random point, so words a previous process left in reused memory match with
// probability 2^-32)
uint32_t next_epoch();

// fused out-projection epilogues (TMOE_EPI_* of include/tmoe.h)
constexpr int kEpiNone = 0, kEpiGlu = 1, kEpiResScale = 2;

// Token counts up to kSmallT take the small-T path (tmoe_small.hpp). Measured at the
// C3 shapes (folded): T = 256 takes 42.8 us there against 49.4 us on the large-tile
// kernels (49 us for any T from 96 up), T = 512 59.0 us against 41-43 us.
constexpr int64_t kSmallT = 256;

// k_core_pp (the persistent core for bf16 plans): ranks r1 in {1, 2, 4}, r1 * r2 a
// multiple of its 256-row tiles, and for fp8 weights at most kCorePScales channel
// scales (staged in LDS); or, bf16 weights only, r1 = 4 G (G > 1) with r2 a
// multiple of 64, in rank groups of 4 (partial sums in the workspace's mpart).
// Its 256-token tiles store whole tiles of mid, so the workspace holds mid for T
// rounded up to kCorePRows rows.
constexpr int kCorePRows = 256;
constexpr int64_t kCorePScales = 4096;
inline bool core_p_grouped(int64_t r1) { return r1 > 4; }
// K slices of the large-T bf16 front (router widths E_pad <= 128): when its
// 64-token tiles number at most a quarter of kCoreUnits and d_in spans at least 16
// K tiles. The slices fill one XCD's 32 compute units with that XCD's tiles (tile
// ft on XCD ft % 8, as k_front_sliced deals them): 32 / ceil(tiles / 8) slices, of
// at least kFrontSliceKTiles K tiles each, at most kMaxFrontPlanes.
// Row stride (floats) of the fp32 front planes (FwdArgs::raw): r3 z columns, then
// E logits, padded to a multiple of 4 so that every row starts 16-byte aligned
// (the plane writers store and the epilogue loads z columns 16 bytes at a time).
constexpr int64_t raw_stride(int64_t r3, int64_t E) { return r3 + (E + 3) / 4 * 4; }
constexpr int64_t kFrontMinKTiles = 16;
constexpr int64_t kFrontSliceKTiles = 3;
constexpr int kMaxFrontPlanes = 8;
constexpr int64_t kFrontXcds = 8, kFrontGroupsPerXcd = 32;
inline int front_split(int64_t T, int64_t d_in, int64_t E_pad, bool bf16) {
  // E_pad = 256 measured slower sliced (C4: front 44.6 us against 34.8 us for the
  // split z / router front plus 7.7 us of k_expand_cz)
  if (!bf16 || T <= 256 || E_pad > 128) return 1;
  const int64_t tiles = (T + 63) / 64, nkt = d_in * 2 / 128;
  // measured at d_in = 1536: slices win up to 64 tiles (T = 4096); at 128 tiles
  // the 32-token front is faster
  if (4 * tiles > 256 || nkt < kFrontMinKTiles) return 1;
  int64_t s = kFrontGroupsPerXcd / ((tiles + kFrontXcds - 1) / kFrontXcds);
  if (s > nkt / kFrontSliceKTiles) s = nkt / kFrontSliceKTiles;
  if (s > kMaxFrontPlanes) s = kMaxFrontPlanes;
  return s > 1 ? (int)s : 1;
}
// signal flags of the K-sliced front in one launch: one per (64-token tile, slice)
// for the slice, and (k_fused_mid) one more per (tile, slice) for its epilogue
inline int64_t front_sliced_flags(int64_t T, int split) {
  return split > 1 ? 2 * ((T + 63) / 64) * split : 0;
}

// Output tiles (256 tokens x 64 channels) of the grouped core and the split S of
// their r1 / 4 rank groups: the smallest divisor of r1 / 4 that gives at least
// kCoreUnits work units (one per compute unit of an MI355X), at most r1 / 4.
constexpr int64_t kCoreUnits = 256;
inline int64_t core_p_out_tiles(int64_t T, int64_t r2) {
  return (T + kCorePRows - 1) / kCorePRows * (r2 / 64);
}
inline int core_p_split(int64_t T, int64_t r1, int64_t r2) {
  const int64_t G = r1 / 4, n = core_p_out_tiles(T, r2);
  for (int64_t s = 1; s < G; ++s)
    if (G % s == 0 && n * s >= kCoreUnits) return (int)s;
  return (int)G;
}
inline bool core_p_supported(int64_t r1, int64_t r2, bool bf16, bool fp8w) {
  if (!bf16) return false;
  if (core_p_grouped(r1)) return r1 % 4 == 0 && r2 % 64 == 0 && !fp8w;
  return (r1 == 1 || r1 == 2 || r1 == 4) && (r1 * r2) % 256 == 0 &&
         (!fp8w || r1 * r2 <= kCorePScales);
}

// The latent expert contraction of the training module (tmoe_latent.hpp) and its
// backward: x (B, r3), G (E, r3, r2), idx (B, k) int64, p (B, k), all but idx in
// dtype; outputs out (B, r2) or dx (B, r3), dG (E, r3, r2), dp (B, k).
struct LatentArgs {
  int dtype;
  bool p_f32;   // p and dp are fp32 (else dtype)
  int64_t B, E, k, r3, r2;
  const void* x;
  const void* G;
  const int64_t* idx;
  const void* p;
  const void* dout;   // backward
  void* out;          // forward
  void* dx;
  void* dG;
  void* dp;
  void* ws;
};
// Workspace bytes of latent_forward (backward = false) or latent_backward.
size_t latent_workspace_bytes(int64_t B, int64_t E, int64_t r3, int64_t r2, int es,
                              bool backward);
hipError_t latent_forward(const LatentArgs& l, hipStream_t stream);
hipError_t latent_backward(const LatentArgs& l, hipStream_t stream);

// Each launcher enqueues one kernel on `stream` and returns hipGetLastError().
hipError_t launch_front(const FwdArgs& a, hipStream_t stream);
// the fronts of two layers of one shape over the same tokens, in one launch where
// the kernels allow (bf16, r3 = 256, the plain front), else one after the other
hipError_t launch_front_pair(const FwdArgs& a0, const FwdArgs& a1, hipStream_t stream);
hipError_t launch_core(const FwdArgs& a, hipStream_t stream);
hipError_t launch_outproj(const FwdArgs& a, hipStream_t stream);
// Small-T path with the front epilogue fused into the next GEMM (3 launches for
// unfolded plans, 2 for folded): k_sk_front only, then the core or the folded
// out-projection, each of whose work-groups runs the epilogue of its tokens.
// small_epi_fused_ok: the fused kernel's LDS fits (else the separate epilogue).
hipError_t launch_small_front_raw(const FwdArgs& a, hipStream_t stream);
hipError_t launch_small_core_epi(const FwdArgs& a, hipStream_t stream);
hipError_t launch_small_out_epi(const FwdArgs& a, hipStream_t stream);
bool small_epi_fused_ok(const FwdArgs& a);
// the whole small-T folded layer in one launch (k_sk_decode): bf16, T <= 64,
// T r3 <= 16384, E <= 16, r1 <= 32, r3 in {64, 128, 256}, sync words present, and
// the stream not being captured
bool small_decode_ok(const FwdArgs& a, hipStream_t stream);
hipError_t launch_small_decode(const FwdArgs& a, hipStream_t stream);
constexpr int64_t kDecodeMaxT = 64;
// floats of its scratch at FwdArgs::raw: z columns (T, r3), c (T, r1)
constexpr int64_t sk_decode_scratch_floats(int64_t T, int64_t r3, int64_t r1) {
  return T * r3 + T * r1;
}
// its sync flags: one per producer work-group, four per column block
constexpr int64_t sk_decode_flags(int64_t r3) { return (r3 / 16 + 1) * 4; }
// folded plans (T > kSmallT): mid (T, r1*r3) = c (x) z, the Khatri-Rao row product
// mid[t, r*r3 + s] = c[t, r] z[t, s] rounded to bf16; launch_outproj then runs with
// r2 := r1 * r3 and uoutT := W^T
hipError_t launch_expand_cz(const FwdArgs& a, hipStream_t stream);
// Whether the large-T front kernel that launch_front picks for `a` can write c (x) z
// itself (a.cz): the single-kind front (not the K-sliced one nor the split one of
// the widest routers) with at most 32 ranks. Then no launch_expand_cz is needed.
bool front_fuses_cz(const FwdArgs& a, hipStream_t stream);
// The K-sliced front's slices and per-token epilogue in one launch (k_front_sliced):
// bf16, front_split > 1, the workspace's signal words, a device of 256 compute units
// (8 XCDs of 32), and the stream not being captured (its flags have several
// consumers and stay set). Same arithmetic as the two-launch path.
bool front_sliced_ok(const FwdArgs& a, hipStream_t stream);
// The whole mid-T forward of a folded plan in one launch (k_fused_mid): the K-sliced
// front (r3 = 256, E_pad = 32) and the 128 x 144 out-projection tiles, at most 32
// of each kind per XCD, c (x) z handed over inside each XCD's L2; on a device of 256
// compute units and not under graph capture (f: the folded forward's arguments).
bool fused_mid_ok(const FwdArgs& f, hipStream_t stream);
bool fused_mid_shape_ok(const FwdArgs& f);
hipError_t launch_fused_mid(const FwdArgs& f, hipStream_t stream);
// Folded bf16 plans (r1 = 4, r3 = 256, K = 1024, E_pad = 256) whose large-T
// out-projection is k_outproj_wide: it forms c (x) z in its loop from the z and c
// the front stores.
bool outproj_kr_ok(const FwdArgs& a);
// The whole large-T forward of a folded plan in one launch (k_fused_large): front
// tiles and out-projection tiles in one persistent grid of one work-group per
// compute unit, c (x) z handed over inside each XCD's L2. fused_large_ok: the plan,
// T, the device and the stream allow it (f: the folded forward's arguments).
bool fused_large_ok(const FwdArgs& f, hipStream_t stream);
// the same rules without the stream's capture state (an eager forward)
bool fused_large_shape_ok(const FwdArgs& f);
bool small_decode_shape_ok(const FwdArgs& a);
hipError_t launch_fused_large(const FwdArgs& f, hipStream_t stream);
// small-T path: front = skinny GEMM + per-token epilogue; core; out-projection
hipError_t launch_small_front(const FwdArgs& a, hipStream_t stream);
hipError_t launch_small_core(const FwdArgs& a, hipStream_t stream);
hipError_t launch_small_out(const FwdArgs& a, hipStream_t stream);
// folded plans: out = (c (x) z) W + bias with c (x) z built from z and c in registers
// (a.r2 = r1 * r3, a.uoutT = W^T); bf16 only
hipError_t launch_small_out_kr(const FwdArgs& a, hipStream_t stream);

// Weight packing helpers (stream-ordered).
// dst(cols, rows) bf16 = e4m3 src(rows, cols)^T; with colscale, entries whose
// scale colscale[(row / group) * cols + col] is zero are stored as zero.
hipError_t launch_transpose_e4m3(const uint8_t* src, uint16_t* dst, int64_t rows, int64_t cols,
                                 const float* colscale, int64_t group, hipStream_t stream);
// k_core_pp's P^T (r1*r2, r3) from core (r1, r3, r2), or with src_t from core^T
// (r2, r1*r3): bf16 bits, or e4m3 codes with channel scales sc (r1, r2) (null for
// bf16; a zero scale packs its channel as zeros).
// k_front_ks's fragment order of the packed front operand (rows % 32 == 0)
hipError_t launch_pack_frag(const void* wfront, void* dst, int64_t rows, int64_t d_in,
                            hipStream_t stream);
hipError_t launch_pack_core_p(const void* core, bool e4m3, const float* sc, uint16_t* dst,
                              int64_t r1, int64_t r3, int64_t r2, hipStream_t stream,
                              bool src_t = false);
// core^T (r2, E*r3) of the expert form G_e = sum_r U_expert[e, r] core_r from
// U_expert (E, r1) and core (r1, r3, r2), element size es (2: bf16, 4: fp32).
hipError_t launch_mix_core_t(const void* uexp, const void* core, void* dst, int64_t E, int64_t r1,
                             int64_t r3, int64_t r2, int es, hipStream_t stream);
// W^T (d_out, K) bf16 of a folded plan, K = rk * r3: W = core (K, r2) U_out (r2, d_out)
// from the packed core^T (r2, K) and U_out^T (d_out, r2) (bf16 bits); with fp8
// weights each core entry takes its channel scale cs[(kk / r3) * r2 + q] and each
// output column the U_out scale os[n] (both null otherwise). fp32 sums, one rounding.
hipError_t launch_fold_out_t(const uint16_t* coreT, const uint16_t* uoutT, const float* cs,
                             const float* os, uint16_t* dst, int64_t K, int64_t r3, int64_t r2,
                             int64_t d_out, hipStream_t stream);
// dst (n, n) fp32 = identity
hipError_t launch_eye(float* dst, int64_t n, hipStream_t stream);
// core scale table (r1, r2) from the per-channel scales sc (r1, r2)
hipError_t launch_core_scales(const float* sc, float* cs, int64_t r1, int64_t r2,
                              hipStream_t stream);
// dst(cols, rows) = src(rows, cols)^T, element size es (2 or 4 bytes).
hipError_t launch_transpose(const void* src, void* dst, int64_t rows, int64_t cols, int es,
                            hipStream_t stream);
// dst[i] = i < n ? src[i] : 0 over n_pad elements, same element size.
hipError_t launch_copy_pad(const void* src, void* dst, int64_t n, int64_t n_pad, int es,
                           hipStream_t stream);
// dst[i] = float(src[i]) for n elements of dtype (TMOE_BF16 / TMOE_F32).
hipError_t launch_to_f32(const void* src, float* dst, int64_t n, int dtype, hipStream_t stream);
// out (T, d) = RMSNorm of each row of x (T, d) with gain w (d), dtype TMOE_BF16 / TMOE_F32.
hipError_t launch_rmsnorm_rows(const void* x, int64_t T, int64_t d, const void* w, float eps,
                               int dtype, void* out, hipStream_t stream);

}  // namespace tmoe
