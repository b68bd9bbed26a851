// Launch configurations of the gfx950 kernels (device code: tmoe_kernels.hpp).
#include <atomic>
#include <chrono>

#include "tmoe_kernels.hpp"
#include "tmoe_small.hpp"
#include "tmoe_latent.hpp"
#include "tmoe_outproj_wide.hpp"
#include "tmoe_outproj_mid.hpp"
#include "tmoe_front_ks.hpp"
#include "tmoe_fused.hpp"
#include "tmoe_front_sliced.hpp"
#include "tmoe_fused_mid.hpp"

namespace tmoe {
namespace {

using dev::EltBF16;
using dev::EltF32;

constexpr int kDtypeBF16 = 1;   // TMOE_BF16
// K steps per ping-pong phase of k_core_pp: 2 keeps its fragments in 236 VGPRs
// (4 spills past the 256 of a two-wave-per-SIMD launch)
constexpr int kCorePSteps = 2;

inline unsigned cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

// GEMM tiles per kernel and dtype: BM x BN, WM x WN waves; core: register ring
// depth PFA of the c (x) z operand; out-projection: LDS stages NS. bf16 choices
// measured at T=16384.
struct CoreCfgBF16 { static constexpr int BM = 256, BN = 256, WM = 2, WN = 4, P = 1; };
struct OutCfgBF16 { static constexpr int BM = 256, BN = 192, WM = 4, WN = 2, P = 2; };
struct CoreCfgF32 { static constexpr int BM = 128, BN = 128, WM = 2, WN = 2, P = 2; };
struct OutCfgF32 { static constexpr int BM = 128, BN = 128, WM = 2, WN = 2, P = 2; };

// Front tiles: kFrontBM tokens in kFrontWM row groups; with the widest router
// (E > 128) one group of 32 tokens, whose smaller LDS footprint measured faster,
// or, with r3 = 256, separate z and router work-groups of 32 tokens.
// The weight rows come from L2 one DMA per K tile; a third LDS stage (when it
// fits) issues them two tiles ahead, which hides the L2 latency.
int cu_count();

template <class Elt, int R3, int NR>
hipError_t launch_front_nr(const FwdArgs& a, hipStream_t st) {
  constexpr int NW = R3 / 32 < 4 ? R3 / 32 : 4;
  if constexpr (std::is_same<Elt, EltBF16>::value) {
    if (a.front_split > 1) {
      // K slices of 64-token tiles (k_front_part), then the per-token epilogue over
      // their planes: in one launch (k_front_sliced, a fresh epoch for its signals)
      // or two
      constexpr int kStageBytes = (kFrontBM + R3 + 32 * NR) * 128;
      constexpr int NS = 3 * kStageBytes <= 160 * 1024 ? 3 : 2;
      if (a.front_one) {
        FwdArgs b = a;
        b.epoch = next_epoch();
        hipLaunchKernelGGL(
            (dev::k_front_sliced<Elt, R3, NR, kFrontPFA, kFrontBM, NS, kFrontWM>),
            dim3(dev::sliced::kGrid), dim3(64 * NW * kFrontWM), 0, st, b, b.raw, b.front_split);
        return hipGetLastError();
      }
      const int64_t stride = a.T * raw_stride(a.r3, a.E);
      hipLaunchKernelGGL((dev::k_front_part<Elt, R3, NR, kFrontPFA, kFrontBM, NS, kFrontWM>),
                         dim3(cdiv(a.T, kFrontBM), a.front_split), dim3(64 * NW * kFrontWM), 0,
                         st, a, a.raw, a.front_split);
      if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
      hipLaunchKernelGGL((dev::k_front_epi<Elt, R3 / 64, kMaxFrontPlanes, 2>),
                         dim3(cdiv(a.T, 4)), dim3(256), (size_t)(a.E * a.r1) * sizeof(float), st,
                         a, (const float*)a.raw, a.front_split, stride);
      return hipGetLastError();
    }
  }
  if constexpr (R3 == 256 && NR == 8 && std::is_same<Elt, EltBF16>::value) {
    // router and z work-groups of 32 tokens (k_front_split), three LDS stages;
    // with c (x) z to write, the z work-groups wait for the router's c (a fresh
    // epoch for the signals)
    FwdArgs b = a;
    b.epoch = next_epoch();
    const dim3 grid(2 * cdiv(a.T, 32)), block(256);
    hipLaunchKernelGGL((dev::k_front_split<Elt, R3, NR, kFrontPFA, 3>), grid, block, 0, st, b);
    return hipGetLastError();
  }
  constexpr int BM = NR >= 8 ? 32 : kFrontBM, WM = NR >= 8 ? 1 : kFrontWM;
  constexpr int kStageBytes = (BM + R3 + 32 * NR) * 128;
  constexpr int NS = 3 * kStageBytes <= 160 * 1024 ? 3 : 2;
  if constexpr (BM > 32 && std::is_same<Elt, EltBF16>::value) {
    // tiles of 32 tokens when they all fit in one round of the compute units: a
    // 32-token work-group takes ~0.9 of a 64-token one's time (both stream every
    // weight row from L2), so half-filled second rounds lose (T = 12288: 50 us
    // against 33 us with 192 work-groups of 64 tokens)
    if ((int64_t)cdiv(a.T, 32) <= cu_count()) {
      constexpr int kStage32 = (32 + R3 + 32 * NR) * 128;
      constexpr int NS32 = 3 * kStage32 <= 160 * 1024 ? 3 : 2;
      hipLaunchKernelGGL((dev::k_front<Elt, R3, NR, kFrontPFA, 32, NS32, 1>), dim3(cdiv(a.T, 32)),
                         dim3(64 * NW), 0, st, a);
      return hipGetLastError();
    }
  }
  if constexpr (R3 == 256 && NR == 1 && std::is_same<Elt, EltBF16>::value) {
    // the weight operand from registers (k_front_ks): 64-token tiles, 8 waves
    // (measured at T = 16384: 31.7 against 33.7 us for k_front; with k_front's x
    // by DMA, 39.6-40.0 against 40.5-40.7 us in the bench's rotated-input loop)
    if (a.wfrag) {
      hipLaunchKernelGGL((dev::k_front_ks<R3, NR>), dim3(cdiv(a.T, 64)), dim3(512), 0, st, a,
                         static_cast<const uint16_t*>(a.wfrag));
      return hipGetLastError();
    }
  }
  const dim3 grid(cdiv(a.T, BM)), block(64 * NW * WM);
  hipLaunchKernelGGL((dev::k_front<Elt, R3, NR, kFrontPFA, BM, NS, WM>), grid, block, 0, st, a);
  return hipGetLastError();
}


// Two layers' fronts in one launch (k_front_pair) when both take the plain bf16
// k_front path; otherwise one after the other.
template <class Elt, int R3, int NR>
hipError_t launch_front_pair_nr(const FwdArgs& a0, const FwdArgs& a1, hipStream_t st) {
  if constexpr (NR < 8 && std::is_same<Elt, EltBF16>::value) {
    if (a0.front_split == 1 && a1.front_split == 1 && a0.T == a1.T) {
      constexpr int NW = R3 / 32 < 4 ? R3 / 32 : 4;
      if (2 * (int64_t)cdiv(a0.T, 32) <= cu_count()) {   // one round, as in launch_front_nr
        constexpr int kStage32 = (32 + R3 + 32 * NR) * 128;
        constexpr int NS32 = 3 * kStage32 <= 160 * 1024 ? 3 : 2;
        const int nt = (int)cdiv(a0.T, 32);
        hipLaunchKernelGGL((dev::k_front_pair<Elt, R3, NR, kFrontPFA, 32, NS32, 1>),
                           dim3(2 * nt), dim3(64 * NW), 0, st, a0, a1, nt);
      } else {
        constexpr int kStageBytes = (kFrontBM + R3 + 32 * NR) * 128;
        constexpr int NS = 3 * kStageBytes <= 160 * 1024 ? 3 : 2;
        const int nt = (int)cdiv(a0.T, kFrontBM);
        hipLaunchKernelGGL((dev::k_front_pair<Elt, R3, NR, kFrontPFA, kFrontBM, NS, kFrontWM>),
                           dim3(2 * nt), dim3(64 * NW * kFrontWM), 0, st, a0, a1, nt);
      }
      return hipGetLastError();
    }
  }
  if (hipError_t e = launch_front_nr<Elt, R3, NR>(a0, st); e != hipSuccess) return e;
  return launch_front_nr<Elt, R3, NR>(a1, st);
}

template <class Elt, int R3>
hipError_t launch_front_pair_r3(const FwdArgs& a0, const FwdArgs& a1, hipStream_t st) {
  switch (a0.E_pad / 32) {
    case 1: return launch_front_pair_nr<Elt, R3, 1>(a0, a1, st);
    case 2: return launch_front_pair_nr<Elt, R3, 2>(a0, a1, st);
    case 4: return launch_front_pair_nr<Elt, R3, 4>(a0, a1, st);
    case 8: return launch_front_pair_nr<Elt, R3, 8>(a0, a1, st);
    default: return hipErrorInvalidValue;
  }
}

template <class Elt, int R3>
hipError_t launch_front_r3(const FwdArgs& a, hipStream_t st) {
  switch (a.E_pad / 32) {
    case 1: return launch_front_nr<Elt, R3, 1>(a, st);
    case 2: return launch_front_nr<Elt, R3, 2>(a, st);
    case 4: return launch_front_nr<Elt, R3, 4>(a, st);
    case 8: return launch_front_nr<Elt, R3, 8>(a, st);
    default: return hipErrorInvalidValue;
  }
}

template <class Elt>
hipError_t launch_front_t(const FwdArgs& a, hipStream_t st) {
  switch (a.r3) {
    case 64: return launch_front_r3<Elt, 64>(a, st);
    case 128: return launch_front_r3<Elt, 128>(a, st);
    case 256: return launch_front_r3<Elt, 256>(a, st);
    default: return hipErrorInvalidValue;
  }
}

// Persistent core: one work-group per compute unit, at most one per output tile.
template <int R1, bool kGrouped = false>
hipError_t launch_core_pp_r(const FwdArgs& a, hipStream_t st);

template <class Elt, class C>
hipError_t launch_core_t(const FwdArgs& a, hipStream_t st) {
  const dim3 grid(cdiv(a.T, C::BM) * cdiv(a.r2, C::BN)), block(64 * C::WM * C::WN);
  hipLaunchKernelGGL((dev::k_core<Elt, C::BM, C::BN, C::WM, C::WN, C::P>), grid, block, 0, st, a);
  return hipGetLastError();
}

template <class Elt, class C>
hipError_t launch_outproj_t(const FwdArgs& a, hipStream_t st) {
  const dim3 grid(cdiv(a.T, C::BM) * cdiv(a.d_out, C::BN)), block(64 * C::WM * C::WN);
  hipLaunchKernelGGL((dev::k_outproj<Elt, C::BM, C::BN, C::WM, C::WN, C::P>), grid, block, 0, st,
                     a);
  return hipGetLastError();
}

// Compute units of the current device (cached per device id).
int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

// k_outproj_wide / k_outproj_mid's contract: bf16, no column scale, no fused
// epilogue, K a multiple of 64, whole 288- (144-) column tiles, A (mid) allocated
// for T rounded up to 256 rows (the workspace rounds its tile rows to 256 for
// these plans).
bool outproj_tiled_ok(const FwdArgs& a) {
  if (a.dtype != kDtypeBF16 || a.out_scale || a.epi_mode != kEpiNone) return false;
  return a.r2 % 64 == 0 && a.d_out % dev::wide::BN == 0 && a.mid_rows_256;
}

// The out-projection's 128 x 144 tiles (k_outproj_mid) number at most the compute
// units: launch_outproj_bf16 takes k_outproj_mid, else k_outproj_wide.
bool outproj_mid_tiles(const FwdArgs& a) {
  return (int64_t)cdiv(a.T, dev::mid::BM) * (a.d_out / dev::mid::BN) <= cu_count();
}


// bf16 out-projection: persistent, one work-group per compute unit (its LDS
// holds one), each looping over the tiles b, b + grid, ...
hipError_t launch_outproj_bf16(const FwdArgs& a, hipStream_t st) {
  typedef OutCfgBF16 C;
  const int64_t ncu = cu_count();
  if (outproj_tiled_ok(a)) {
    // measured at d_out = 2304, K = 1024 (plain GEMM, us): T = 2048: 128 x 144 tiles
    // 19.3, 128 x 288 23.8, 256 x 288 32.8; T = 4096: 36.2, 26.4, 34.0; T = 6144:
    // 52.2, 42.7, 35.8; T = 8192: 69.4, 47.8, 39.5 (k_outproj_pp: 27 at 2048, 31 at
    // 4096). The smallest tile whose count fits one round of compute units wins
    // up to T = 4096; above, the 256 x 288 tiles, also in a partial round.
    const uint16_t* A = static_cast<const uint16_t*>(a.mid);
    const uint16_t* Bt = static_cast<const uint16_t*>(a.uoutT);
    uint16_t* out = static_cast<uint16_t*>(a.out);
    const int T = (int)a.T, N = (int)a.d_out, K = (int)a.r2;
    const int64_t ntn = a.d_out / dev::wide::BN;
    const int64_t t128 = cdiv(a.T, dev::wide::Cfg<1>::BM) * ntn;
    const int64_t t256 = cdiv(a.T, dev::wide::Cfg<2>::BM) * ntn;
    if (a.kr) {   // A = c (x) z formed from z and c in the loop (outproj_kr_ok)
      const uint16_t* Z = static_cast<const uint16_t*>(a.z);
      if (t128 <= ncu) {
        hipLaunchKernelGGL(dev::k_outproj_wide_kr<1>, dim3((unsigned)t128), dim3(256), 0, st, Z,
                           a.c, Bt, out, a.bias, T, N, K);
      } else {
        const dim3 grid((unsigned)(t256 < ncu ? t256 : ncu));
        hipLaunchKernelGGL(dev::k_outproj_wide_kr<2>, grid, dim3(256), 0, st, Z, a.c, Bt, out,
                           a.bias, T, N, K);
      }
      return hipGetLastError();
    }
    if (outproj_mid_tiles(a)) {
      const int64_t t_mid = cdiv(a.T, dev::mid::BM) * (a.d_out / dev::mid::BN);
      hipLaunchKernelGGL(dev::k_outproj_mid, dim3((unsigned)t_mid), dim3(256), 0, st, A, Bt, out,
                         a.bias, T, N, K);
    } else if (t128 <= ncu) {
      hipLaunchKernelGGL(dev::k_outproj_wide<1>, dim3((unsigned)t128), dim3(256), 0, st, A, Bt,
                         out, a.bias, T, N, K);
    } else {
      const dim3 grid((unsigned)(t256 < ncu ? t256 : ncu));
      hipLaunchKernelGGL(dev::k_outproj_wide<2>, grid, dim3(256), 0, st, A, Bt, out, a.bias, T, N,
                         K);
    }
    return hipGetLastError();
  }
  const int64_t tiles = (int64_t)cdiv(a.T, C::BM) * cdiv(a.d_out, C::BN);
  if (2 * tiles <= ncu) {
    // at most half the compute units busy: tiles of 128 tokens, twice as many
    const int64_t t128 = (int64_t)cdiv(a.T, 128) * cdiv(a.d_out, C::BN);
    const dim3 grid((unsigned)(t128 < ncu ? t128 : ncu)), block(64 * C::WM * C::WN);
    hipLaunchKernelGGL((dev::k_outproj_pp<128, C::BN, C::WM, C::WN>), grid, block, 0, st, a);
    return hipGetLastError();
  }
  const dim3 grid((unsigned)(tiles < ncu ? tiles : ncu)), block(64 * C::WM * C::WN);
  hipLaunchKernelGGL((dev::k_outproj_pp<C::BM, C::BN, C::WM, C::WN>), grid, block, 0, st, a);
  return hipGetLastError();
}

template <int R1, bool kGrouped>
hipError_t launch_core_pp_r(const FwdArgs& a, hipStream_t st) {
  // work units: output tiles, times the split of their rank groups when grouped
  const int64_t tiles = (int64_t)cdiv(a.T, kCorePRows) * (R1 * a.r2 / 256) *
                        (kGrouped ? a.core_split : 1);
  const int64_t ncu = cu_count();
  const dim3 grid((unsigned)(tiles < ncu ? tiles : ncu)), block(512);
  hipLaunchKernelGGL((dev::k_core_pp<R1, kCorePSteps, kGrouped>), grid, block, 0, st, a);
  if (kGrouped && a.core_split > 1) {
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    const int64_t n = (int64_t)cdiv(a.T, kCorePRows) * (a.r2 / 64) * 4096;   // float4s a part
    hipLaunchKernelGGL(dev::k_core_combine, dim3(cdiv(n, 256)), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

// small-T path: 16-column work-groups of kSkW waves over blocks of 16 MF tokens
constexpr int kSkW = 16;

template <int MF, class Elt>
hipError_t launch_small_front_t(const FwdArgs& a, hipStream_t st) {
  const dim3 grid(cdiv(a.r3 + a.E, 16), cdiv(a.T, 16 * MF)), block(64 * kSkW);
  hipLaunchKernelGGL((dev::k_sk_front<Elt, MF, kSkW>), grid, block, 0, st, a, a.raw);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  const dim3 eg(cdiv(a.T, 4)), eb(256);
  const size_t ue_bytes = (size_t)(a.E * a.r1) * sizeof(float);
  const float* raw = a.raw;
  if (a.r3 == 256)
    hipLaunchKernelGGL((dev::k_front_epi<Elt, 4, 1, 4>), eg, eb, ue_bytes, st, a, raw, 1, (int64_t)0);
  else if (a.r3 == 128)
    hipLaunchKernelGGL((dev::k_front_epi<Elt, 2, 1, 4>), eg, eb, ue_bytes, st, a, raw, 1, (int64_t)0);
  else
    hipLaunchKernelGGL((dev::k_front_epi<Elt, 1, 1, 4>), eg, eb, ue_bytes, st, a, raw, 1, (int64_t)0);
  return hipGetLastError();
}

template <int MF, class Elt>
hipError_t launch_small_core_t(const FwdArgs& a, hipStream_t st) {
  const dim3 grid(cdiv(a.r2, 16), cdiv(a.T, 16 * MF)), block(64 * kSkW);
  hipLaunchKernelGGL((dev::k_sk_core<Elt, MF, kSkW>), grid, block, 0, st, a);
  return hipGetLastError();
}

template <int MF, class Elt, bool KR = false>
hipError_t launch_small_out_t(const FwdArgs& a, hipStream_t st) {
  const dim3 grid(cdiv(a.d_out, 16), cdiv(a.T, 16 * MF)), block(64 * kSkW);
  hipLaunchKernelGGL((dev::k_sk_out<Elt, MF, kSkW, KR>), grid, block, 0, st, a);
  return hipGetLastError();
}

// the small-T front's GEMM alone (raw), for a consumer that runs the epilogue
template <int MF, class Elt>
hipError_t launch_small_front_raw_t(const FwdArgs& a, hipStream_t st) {
  const dim3 grid(cdiv(a.r3 + a.E, 16), cdiv(a.T, 16 * MF)), block(64 * kSkW);
  hipLaunchKernelGGL((dev::k_sk_front<Elt, MF, kSkW>), grid, block, 0, st, a, a.raw);
  return hipGetLastError();
}

// the front epilogue fused into the following Khatri-Rao GEMM (core, or the
// folded out-projection)
template <int MF, class Elt, bool kCore>
hipError_t launch_small_epi_gemm_t(const FwdArgs& a, hipStream_t st) {
  const int64_t N = kCore ? a.r2 : a.d_out;
  const dim3 grid(cdiv(N, 16), cdiv(a.T, 16 * MF)), block(64 * kSkW);
  hipLaunchKernelGGL((dev::k_sk_epi_gemm<Elt, MF, kSkW, kCore>), grid, block,
                     dev::sk_epi_dyn_bytes(MF, a), st, a);
  return hipGetLastError();
}

// rows per work-group: 16, 32 or 64 tokens
inline int small_mf(int64_t T) { return T <= 16 ? 1 : T <= 32 ? 2 : 4; }

template <template <int, class> class L>
hipError_t by_rows(const FwdArgs& a, hipStream_t st) {
  const bool bf = a.dtype == kDtypeBF16;
  if (a.T <= 16) return bf ? L<1, EltBF16>::run(a, st) : L<1, EltF32>::run(a, st);
  if (a.T <= 32) return bf ? L<2, EltBF16>::run(a, st) : L<2, EltF32>::run(a, st);
  return bf ? L<4, EltBF16>::run(a, st) : L<4, EltF32>::run(a, st);
}
template <int MF, class Elt>
struct SmallFront {
  static hipError_t run(const FwdArgs& a, hipStream_t st) { return launch_small_front_t<MF, Elt>(a, st); }
};
template <int MF, class Elt>
struct SmallCore {
  static hipError_t run(const FwdArgs& a, hipStream_t st) { return launch_small_core_t<MF, Elt>(a, st); }
};
template <int MF, class Elt>
struct SmallOut {
  static hipError_t run(const FwdArgs& a, hipStream_t st) { return launch_small_out_t<MF, Elt>(a, st); }
};
template <int MF, class Elt>
struct SmallFrontRaw {
  static hipError_t run(const FwdArgs& a, hipStream_t st) { return launch_small_front_raw_t<MF, Elt>(a, st); }
};
template <int MF, class Elt>
struct SmallCoreEpi {
  static hipError_t run(const FwdArgs& a, hipStream_t st) { return launch_small_epi_gemm_t<MF, Elt, true>(a, st); }
};
template <int MF, class Elt>
struct SmallOutEpi {
  static hipError_t run(const FwdArgs& a, hipStream_t st) {
    if constexpr (std::is_same<Elt, EltBF16>::value) return launch_small_epi_gemm_t<MF, Elt, false>(a, st);
    return hipErrorInvalidValue;   // folded plans are bf16
  }
};
template <int MF, class Elt>
struct SmallOutKR {
  static hipError_t run(const FwdArgs& a, hipStream_t st) {
    if constexpr (std::is_same<Elt, EltBF16>::value) return launch_small_out_t<MF, Elt, true>(a, st);
    return hipErrorInvalidValue;   // folded plans are bf16
  }
};

}  // namespace

bool outproj_kr_ok(const FwdArgs& a) {
  // Only where the front cannot write c (x) z without a hand-off: the split front
  // of the widest routers (E_pad = 256: z and the router in different work-groups)
  // would make its z work-groups wait for c (or a separate k_expand_cz pass run).
  // Elsewhere the front's own c (x) z stores cost about what the scaling costs the
  // loop (C3, two launches: front 38.8 -> 31.9 us, out-projection 83.9 -> 91.1 us;
  // the one-launch forward 116.2 -> 121.2 us), while C4 gains ~4 us.
  // Every large-T front stores z (bf16) and c (fp32) when a.cz is unset; z and c
  // are allocated in whole 256-row tiles (a.mid_rows_256: the folded layout).
  return a.T > kSmallT && outproj_tiled_ok(a) && a.E_pad > 128 && a.r1 == dev::wide::kKrR1 &&
         a.r3 == dev::wide::kKrR3 && a.r2 == dev::wide::kKrR1 * dev::wide::kKrR3 &&
         !outproj_mid_tiles(a);
}

hipError_t launch_small_front(const FwdArgs& a, hipStream_t st) { return by_rows<SmallFront>(a, st); }
hipError_t launch_small_core(const FwdArgs& a, hipStream_t st) { return by_rows<SmallCore>(a, st); }
hipError_t launch_small_out(const FwdArgs& a, hipStream_t st) { return by_rows<SmallOut>(a, st); }
hipError_t launch_small_out_kr(const FwdArgs& a, hipStream_t st) { return by_rows<SmallOutKR>(a, st); }
hipError_t launch_small_front_raw(const FwdArgs& a, hipStream_t st) { return by_rows<SmallFrontRaw>(a, st); }
hipError_t launch_small_core_epi(const FwdArgs& a, hipStream_t st) { return by_rows<SmallCoreEpi>(a, st); }
hipError_t launch_small_out_epi(const FwdArgs& a, hipStream_t st) { return by_rows<SmallOutEpi>(a, st); }

bool small_epi_fused_ok(const FwdArgs& a) {
  const int mf = small_mf(a.T);
  // a wave runs the epilogue of MF 16 / 16 tokens one after the other: at 4 (T > 32)
  // the separate epilogue kernel measured faster (C1, T = 64: 36.0 us against 32.6)
  if (mf > 2) return false;
  const size_t stat = (size_t)mf * 256 * (1 + kSkW) * sizeof(float);   // SkLds<MF, kSkW>
  return stat + dev::sk_epi_dyn_bytes(mf, a) <= (size_t)160 * 1024 && a.r3 % 8 == 0;
}

bool stream_capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone;
}

bool small_decode_shape_ok(const FwdArgs& a) {
  if (a.dtype != kDtypeBF16 || a.T > kDecodeMaxT || a.T * a.r3 > 16384 || a.E > 16 ||
      (a.r3 != 64 && a.r3 != 128 && a.r3 != 256) || !a.sync || a.r1 > 32)
    return false;
  const int mf = small_mf(a.T);
  const size_t stat = (size_t)mf * 256 * (1 + kSkW) * sizeof(float);   // SkLds<MF, kSkW>
  return stat + dev::sk_decode_dyn_bytes(mf, a) <= (size_t)160 * 1024;
}

bool small_decode_ok(const FwdArgs& a, hipStream_t st) {
  // the consumers wait on flags that stay set (several per flag): a replayed graph
  // would find them set, so a captured forward takes the two-launch path
  return small_decode_shape_ok(a) && !stream_capturing(st);
}

template <int MF>
hipError_t launch_small_decode_t(const FwdArgs& a, hipStream_t st) {
  FwdArgs b = a;
  b.epoch = next_epoch();
  const dim3 grid((unsigned)((a.r3 / 16 + 1) * dev::kDecodeRowGroups + cdiv(a.d_out, 16))),
      block(64 * kSkW);
  hipLaunchKernelGGL((dev::k_sk_decode<MF, kSkW>), grid, block, dev::sk_decode_dyn_bytes(MF, a),
                     st, b);
  return hipGetLastError();
}

hipError_t launch_small_decode(const FwdArgs& a, hipStream_t st) {
  switch (small_mf(a.T)) {
    case 1: return launch_small_decode_t<1>(a, st);
    case 2: return launch_small_decode_t<2>(a, st);
    default: return launch_small_decode_t<4>(a, st);
  }
}

hipError_t launch_front_pair(const FwdArgs& a0, const FwdArgs& a1, hipStream_t st) {
  if (a0.dtype != kDtypeBF16 || a0.r3 != 256 || a0.E_pad != a1.E_pad || a0.r3 != a1.r3) {
    if (hipError_t e = launch_front(a0, st); e != hipSuccess) return e;
    return launch_front(a1, st);
  }
  return launch_front_pair_r3<EltBF16, 256>(a0, a1, st);
}

hipError_t launch_front(const FwdArgs& a, hipStream_t st) {
  return a.dtype == kDtypeBF16 ? launch_front_t<EltBF16>(a, st) : launch_front_t<EltF32>(a, st);
}

hipError_t launch_core(const FwdArgs& a, hipStream_t st) {
  if (a.dtype == kDtypeBF16 && a.coreP) {
    switch (a.r1) {
      case 1: return launch_core_pp_r<1>(a, st);
      case 2: return launch_core_pp_r<2>(a, st);
      case 4: return launch_core_pp_r<4>(a, st);
      default:
        if (core_p_grouped(a.r1) && a.mpart) return launch_core_pp_r<4, true>(a, st);
        return hipErrorInvalidValue;
    }
  }
  return a.dtype == kDtypeBF16 ? launch_core_t<EltBF16, CoreCfgBF16>(a, st)
                               : launch_core_t<EltF32, CoreCfgF32>(a, st);
}

hipError_t launch_pack_frag(const void* wfront, void* dst, int64_t rows, int64_t d_in,
                            hipStream_t st) {
  if (rows % 32 || d_in % 16) return hipErrorInvalidValue;
  const int64_t nchunks = (d_in / 16) * (rows / 32) * 64;
  if (nchunks == 0) return hipSuccess;
  hipLaunchKernelGGL(dev::k_pack_frag, dim3((unsigned)cdiv(nchunks, 256)), dim3(256), 0, st,
                     static_cast<const uint16_t*>(wfront), static_cast<uint16_t*>(dst), rows / 32,
                     d_in);
  return hipGetLastError();
}

hipError_t launch_pack_core_p(const void* core, bool e4m3, const float* sc, uint16_t* dst,
                              int64_t r1, int64_t r3, int64_t r2, hipStream_t st, bool src_t) {
  if (r1 == 0 || r2 == 0 || r3 == 0) return hipSuccess;
  const dim3 grid(cdiv(r2, 32), cdiv(r3, 32), (unsigned)r1), block(256);
  if (e4m3)
    hipLaunchKernelGGL(dev::k_pack_core_p<true>, grid, block, 0, st, core, dst, r1, r3, r2, sc,
                       src_t);
  else
    hipLaunchKernelGGL(dev::k_pack_core_p<false>, grid, block, 0, st, core, dst, r1, r3, r2, sc,
                       src_t);
  return hipGetLastError();
}

hipError_t launch_mix_core_t(const void* uexp, const void* core, void* dst, int64_t E, int64_t r1,
                             int64_t r3, int64_t r2, int es, hipStream_t st) {
  if (E == 0 || r2 == 0 || r3 == 0) return hipSuccess;
  if (r1 > 64 || r3 % 32 || r2 % 32) return hipErrorInvalidValue;
  const dim3 grid(cdiv(r2, 32), cdiv(E * r3, 32)), block(256);
  if (es == 2)
    hipLaunchKernelGGL(dev::k_mix_core_t<uint16_t>, grid, block, 0, st,
                       static_cast<const uint16_t*>(uexp), static_cast<const uint16_t*>(core),
                       static_cast<uint16_t*>(dst), E, r1, r3, r2);
  else
    hipLaunchKernelGGL(dev::k_mix_core_t<float>, grid, block, 0, st,
                       static_cast<const float*>(uexp), static_cast<const float*>(core),
                       static_cast<float*>(dst), E, r1, r3, r2);
  return hipGetLastError();
}

hipError_t launch_fold_out_t(const uint16_t* coreT, const uint16_t* uoutT, const float* cs,
                             const float* os, uint16_t* dst, int64_t K, int64_t r3, int64_t r2,
                             int64_t d_out, hipStream_t st) {
  if (K == 0 || d_out == 0) return hipSuccess;
  if (K % 32 || r2 % 32 || r3 % 32) return hipErrorInvalidValue;
  hipLaunchKernelGGL(dev::k_fold_out_t, dim3(cdiv(K, 32), cdiv(d_out, 32)), dim3(256), 0, st,
                     coreT, uoutT, cs, os, dst, K, r3, r2, d_out);
  return hipGetLastError();
}

// k_fused_large (tmoe_fused.hpp): a folded bf16 plan whose front is k_front_ks's
// (r3 = 256, E_pad = 32, the fragment-order weights packed) and writes c (x) z,
// whose out-projection is k_outproj_wide's (outproj_tiled_ok), with at least one
// 256 x 288 tile per work-group (T >= 8192 at d_out = 2304), on a device of 256
// compute units (8 XCDs of 32), with the workspace's signal words, and not under
// graph capture (its flags have several consumers and stay set).
bool fused_large_shape_ok(const FwdArgs& a) {
  if (a.dtype != kDtypeBF16 || !a.cz || !a.wfrag || a.r3 != 256 || a.E_pad != 32 || !a.sync)
    return false;
  if (!outproj_tiled_ok(a) || a.r2 % 64) return false;
  const int64_t tiles = (int64_t)cdiv(a.T, dev::wide::BM) * (a.d_out / dev::wide::BN);
  // a signal flag per 64-token front tile fits the workspace's flags (one per
  // kSyncTileRows tokens); rows are addressed in int
  return tiles >= dev::fused::kGrid && cu_count() == dev::fused::kGrid &&
         a.T <= ((int64_t)1 << 30);
}

bool fused_large_ok(const FwdArgs& a, hipStream_t st) {
  return fused_large_shape_ok(a) && !stream_capturing(st);
}

hipError_t launch_fused_large(const FwdArgs& a, hipStream_t st) {
  FwdArgs b = a;
  b.epoch = next_epoch();
  hipLaunchKernelGGL((dev::k_fused_large<256, 1>), dim3(dev::fused::kGrid), dim3(256), 0, st, b,
                     static_cast<const uint16_t*>(a.wfrag), static_cast<const uint16_t*>(a.cz),
                     static_cast<const uint16_t*>(a.uoutT), static_cast<uint16_t*>(a.out),
                     a.bias);
  return hipGetLastError();
}

bool front_fuses_cz(const FwdArgs& a, hipStream_t st) {
  // launch_front_nr: k_front_part + k_front_epi when front_split > 1 (the per-token
  // epilogue writes c (x) z for any r1), else k_front_split for r3 = 256 with
  // E_pad = 256 (z and router in separate work-groups: no), else k_front (front_tile:
  // c fits over the logits for r1 <= 32, BM x (E_pad + 1) floats)
  if (a.dtype != kDtypeBF16 || a.T <= kSmallT) return false;
  if (a.front_split > 1) return true;
  // k_front_split (r3 = 256, E_pad = 256): the z work-groups wait for the router
  // work-groups' c through the workspace's sync words
  // (not under graph capture: a consumer that gave up on its flag would leave it
  // to be found set on a replay with the same epoch; the captured forward runs
  // k_expand_cz instead)
  if (a.r3 == 256 && a.E_pad == 256) return a.r1 <= 32 && a.sync != nullptr && !stream_capturing(st);
  return a.r1 <= 32;
}

bool front_sliced_ok(const FwdArgs& a, hipStream_t st) {
  if (a.dtype != kDtypeBF16 || a.front_split <= 1 || !a.sync || a.E_pad > 128) return false;
  // every (XCD, slot) pair of the grid holds at most one slice
  const int64_t per_xcd = ((int64_t)cdiv(a.T, kFrontBM) + dev::sliced::kXcds - 1) /
                          dev::sliced::kXcds;
  return per_xcd * a.front_split <= dev::sliced::kGroupsPerXcd &&
         cu_count() == dev::sliced::kGrid && !stream_capturing(st);
}

bool fused_mid_shape_ok(const FwdArgs& a) {
  if (a.dtype != kDtypeBF16 || !a.cz || a.kr || a.front_split <= 1 || a.r3 != 256 ||
      a.E_pad != 32 || !a.sync || a.r2 % 64 || !outproj_tiled_ok(a) || !outproj_mid_tiles(a))
    return false;
  // per XCD: at most 32 out-projection tiles and 32 front slices
  const int64_t n_rt = cdiv(a.T, dev::mid::BM);
  const int64_t nrx = (n_rt + dev::fmid::kXcds - 1) / dev::fmid::kXcds;
  return nrx * (a.d_out / dev::mid::BN) <= dev::fmid::kGroupsPerXcd &&
         dev::fmid::kFrontPerRow * nrx * a.front_split <= dev::fmid::kGroupsPerXcd &&
         cu_count() == dev::fmid::kGrid;
}

bool fused_mid_ok(const FwdArgs& a, hipStream_t st) {
  return fused_mid_shape_ok(a) && !stream_capturing(st);
}

hipError_t launch_fused_mid(const FwdArgs& a, hipStream_t st) {
  constexpr int R3 = 256, NR = 1;
  constexpr int kStageBytes = (kFrontBM + R3 + 32 * NR) * 128;
  constexpr int NS = 3 * kStageBytes <= 160 * 1024 ? 3 : 2;
  constexpr int NW = R3 / 32 < 4 ? R3 / 32 : 4;
  FwdArgs b = a;
  b.epoch = next_epoch();
  hipLaunchKernelGGL(
      (dev::k_fused_mid<EltBF16, R3, NR, kFrontPFA, kFrontBM, NS, kFrontWM>),
      dim3(dev::fmid::kGrid), dim3(64 * NW * kFrontWM), 0, st, b, b.raw, b.front_split,
      static_cast<const uint16_t*>(a.cz), static_cast<const uint16_t*>(a.uoutT),
      static_cast<uint16_t*>(a.out), a.bias);
  return hipGetLastError();
}

uint32_t next_epoch() {
  // a random start (clock and an address of this image), then one per launch
  static std::atomic<uint32_t> ctr{[] {
    uint64_t v = (uint64_t)std::chrono::high_resolution_clock::now().time_since_epoch().count();
    v ^= (uint64_t)(uintptr_t)&ctr * 0x9e3779b97f4a7c15ull;
    return (uint32_t)(v ^ (v >> 32));
  }()};
  uint32_t e;
  do {
    e = ctr.fetch_add(1, std::memory_order_relaxed) + 1;
  } while (e == 0);
  return e;
}

hipError_t launch_expand_cz(const FwdArgs& a, hipStream_t st) {
  if (a.dtype != kDtypeBF16) return hipErrorInvalidValue;
  const int64_t n = a.T * (a.r3 / 8);   // 16-byte chunks of z, one per thread and pass
  if (n == 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256;
  const dim3 grid((unsigned)(blocks < (1 << 20) ? blocks : (1 << 20))), block(256);
  switch (a.r3) {
    case 64: hipLaunchKernelGGL(dev::k_expand_cz<64>, grid, block, 0, st, a); break;
    case 128: hipLaunchKernelGGL(dev::k_expand_cz<128>, grid, block, 0, st, a); break;
    case 256: hipLaunchKernelGGL(dev::k_expand_cz<256>, grid, block, 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_eye(float* dst, int64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const dim3 grid(cdiv(n * n, 256) < 1024 ? cdiv(n * n, 256) : 1024), block(256);
  hipLaunchKernelGGL(dev::k_eye, grid, block, 0, st, dst, n);
  return hipGetLastError();
}

hipError_t launch_outproj(const FwdArgs& a, hipStream_t st) {
  return a.dtype == kDtypeBF16 ? launch_outproj_bf16(a, st)
                               : launch_outproj_t<EltF32, OutCfgF32>(a, st);
}

hipError_t launch_transpose(const void* src, void* dst, int64_t rows, int64_t cols, int es,
                            hipStream_t st) {
  if (rows == 0 || cols == 0) return hipSuccess;
  const dim3 grid(cdiv(cols, 32), cdiv(rows, 32)), block(256);
  if (es == 2)
    hipLaunchKernelGGL(dev::k_transpose<uint16_t>, grid, block, 0, st,
                       static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), rows, cols);
  else
    hipLaunchKernelGGL(dev::k_transpose<float>, grid, block, 0, st,
                       static_cast<const float*>(src), static_cast<float*>(dst), rows, cols);
  return hipGetLastError();
}

hipError_t launch_transpose_e4m3(const uint8_t* src, uint16_t* dst, int64_t rows, int64_t cols,
                                 const float* colscale, int64_t group, hipStream_t st) {
  if (rows == 0 || cols == 0) return hipSuccess;
  const dim3 grid(cdiv(cols, 32), cdiv(rows, 32)), block(256);
  hipLaunchKernelGGL(dev::k_transpose_e4m3, grid, block, 0, st, src, dst, rows, cols, colscale,
                     group);
  return hipGetLastError();
}

hipError_t launch_core_scales(const float* sc, float* cs, int64_t r1, int64_t r2,
                              hipStream_t st) {
  if (r1 == 0 || r2 == 0) return hipSuccess;
  const dim3 grid(cdiv(r2, 256) < 1024 ? cdiv(r2, 256) : 1024), block(256);
  hipLaunchKernelGGL(dev::k_core_scales, grid, block, 0, st, sc, cs, r1, r2);
  return hipGetLastError();
}

hipError_t launch_copy_pad(const void* src, void* dst, int64_t n, int64_t n_pad, int es,
                           hipStream_t st) {
  if (n_pad == 0) return hipSuccess;
  const dim3 grid(cdiv(n_pad, 256) < 4096 ? cdiv(n_pad, 256) : 4096), block(256);
  if (es == 2)
    hipLaunchKernelGGL(dev::k_copy_pad<uint16_t>, grid, block, 0, st,
                       static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), n, n_pad);
  else
    hipLaunchKernelGGL(dev::k_copy_pad<float>, grid, block, 0, st,
                       static_cast<const float*>(src), static_cast<float*>(dst), n, n_pad);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_rows(const void* x, int64_t T, int64_t d, const void* w, float eps,
                               int dtype, void* out, hipStream_t st) {
  if (T == 0) return hipSuccess;
  const dim3 grid(cdiv(T, 4)), block(256);
  const int es = dtype == kDtypeBF16 ? 2 : 4;
  const bool vec = (d * es) % 16 == 0 && d * es <= 64 * 8 * 16 &&
                   ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                     reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  if (vec) {   // rows of at most 8 KB, held in registers
    if (dtype == kDtypeBF16)
      hipLaunchKernelGGL((dev::k_rmsnorm_rows_v<uint16_t, 8>), grid, block, 0, st,
                         static_cast<const uint16_t*>(x), T, d, static_cast<const uint16_t*>(w),
                         eps, static_cast<uint16_t*>(out));
    else
      hipLaunchKernelGGL((dev::k_rmsnorm_rows_v<float, 8>), grid, block, 0, st,
                         static_cast<const float*>(x), T, d, static_cast<const float*>(w), eps,
                         static_cast<float*>(out));
    return hipGetLastError();
  }
  if (dtype == kDtypeBF16)
    hipLaunchKernelGGL(dev::k_rmsnorm_rows<uint16_t>, grid, block, 0, st,
                       static_cast<const uint16_t*>(x), T, d, static_cast<const uint16_t*>(w), eps,
                       static_cast<uint16_t*>(out));
  else
    hipLaunchKernelGGL(dev::k_rmsnorm_rows<float>, grid, block, 0, st, static_cast<const float*>(x),
                       T, d, static_cast<const float*>(w), eps, static_cast<float*>(out));
  return hipGetLastError();
}

hipError_t launch_to_f32(const void* src, float* dst, int64_t n, int dtype, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const dim3 grid(cdiv(n, 256) < 4096 ? cdiv(n, 256) : 4096), block(256);
  if (dtype == kDtypeBF16)
    hipLaunchKernelGGL(dev::k_to_f32<uint16_t>, grid, block, 0, st,
                       static_cast<const uint16_t*>(src), dst, n);
  else
    hipLaunchKernelGGL(dev::k_to_f32<float>, grid, block, 0, st, static_cast<const float*>(src),
                       dst, n);
  return hipGetLastError();
}

}  // namespace tmoe

// ---- latent expert contraction (training path) ------------------------------
namespace tmoe {
namespace {

size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

struct LatentLayout {
  size_t w, gt, zero, h, xt, dt, wt, parts, total;
  int64_t bp;
  int slices;
};

constexpr int kDgBM = 128, kDgBN = 128;

LatentLayout latent_layout(int64_t B, int64_t E, int64_t r3, int64_t r2, int es, bool bwd) {
  LatentLayout L{};
  size_t o = 0;
  L.w = o; o = al256(o + (size_t)B * E * 4);
  if (!bwd) {
    L.gt = o; o = al256(o + (size_t)r2 * E * r3 * es);
  } else {
    const int64_t M = E * r3;
    L.bp = (B + 63) / 64 * 64;
    L.zero = o; o = al256(o + (size_t)M * 4);
    L.h = o; o = al256(o + (size_t)B * M * es);
    L.xt = o; o = al256(o + (size_t)r3 * L.bp * es);
    L.dt = o; o = al256(o + (size_t)r2 * L.bp * es);
    L.wt = o; o = al256(o + (size_t)E * L.bp * 4);
    // K slices of the dG GEMM: about 256 work-groups, each at least 4 K tiles
    const int64_t tiles = (M + kDgBM - 1) / kDgBM * ((r2 + kDgBN - 1) / kDgBN);
    const int64_t nkt = L.bp * es / kTileKBytes;
    int64_t sl = (256 + tiles - 1) / tiles;
    if (sl > nkt / 4) sl = nkt / 4;
    L.slices = sl > 1 ? (int)sl : 1;
    L.parts = o; o = al256(o + (size_t)L.slices * M * r2 * 4);
  }
  L.total = o;
  return L;
}

template <class T>
hipError_t transpose_pad(const void* src, void* dst, int64_t rows, int64_t cols, int64_t rows_pad,
                         hipStream_t st) {
  const dim3 grid(cdiv(cols, 32), cdiv(rows_pad, 32)), block(256);
  hipLaunchKernelGGL(dev::k_transpose_pad<T>, grid, block, 0, st, static_cast<const T*>(src),
                     static_cast<T*>(dst), rows, cols, rows_pad);
  return hipGetLastError();
}

template <class T>
hipError_t latent_weights(const LatentArgs& l, float* w, hipStream_t st) {
  const int64_t n = l.B * l.E;
  hipLaunchKernelGGL(dev::k_latent_w<T>, dim3(cdiv(n, 256)), dim3(256), 0, st, l.idx,
                     static_cast<const T*>(l.p), l.B, (int)l.k, (int)l.E, w);
  return hipGetLastError();
}

}  // namespace

size_t latent_workspace_bytes(int64_t B, int64_t E, int64_t r3, int64_t r2, int es, bool bwd) {
  return latent_layout(B, E, r3, r2, es, bwd).total;
}

hipError_t latent_forward(const LatentArgs& l, hipStream_t st) {
  const bool bf = l.dtype == kDtypeBF16;
  const int es = bf ? 2 : 4;
  const LatentLayout L = latent_layout(l.B, l.E, l.r3, l.r2, es, false);
  char* ws = static_cast<char*>(l.ws);
  float* w = reinterpret_cast<float*>(ws + L.w);
  hipError_t e = bf && !l.p_f32 ? latent_weights<uint16_t>(l, w, st) : latent_weights<float>(l, w, st);
  if (e != hipSuccess) return e;
  // G as (E r3, r2), transposed: the B^T operand (r2, E r3) of the Khatri-Rao GEMM
  if ((e = launch_transpose(l.G, ws + L.gt, l.E * l.r3, l.r2, es, st)) != hipSuccess) return e;
  FwdArgs a{};
  a.dtype = l.dtype;
  a.T = l.B; a.r1 = l.E; a.r3 = l.r3; a.r2 = l.r2;
  a.z = const_cast<void*>(l.x);
  a.c = w;
  a.coreT = ws + L.gt;
  a.mid = l.out;
  return bf ? launch_core_t<EltBF16, CoreCfgBF16>(a, st) : launch_core_t<EltF32, CoreCfgF32>(a, st);
}

hipError_t latent_backward(const LatentArgs& l, hipStream_t st) {
  const bool bf = l.dtype == kDtypeBF16;
  const int es = bf ? 2 : 4;
  const LatentLayout L = latent_layout(l.B, l.E, l.r3, l.r2, es, true);
  const int64_t M = l.E * l.r3;
  char* ws = static_cast<char*>(l.ws);
  float* w = reinterpret_cast<float*>(ws + L.w);
  hipError_t e = bf && !l.p_f32 ? latent_weights<uint16_t>(l, w, st) : latent_weights<float>(l, w, st);
  if (e != hipSuccess) return e;
  // H = dout G_flat^T (B, E r3): the out-projection GEMM with U_out^T := G as (E r3, r2)
  if ((e = launch_copy_pad(nullptr, ws + L.zero, 0, M, 4, st)) != hipSuccess) return e;
  FwdArgs a{};
  a.dtype = l.dtype;
  a.T = l.B; a.r2 = l.r2; a.d_out = M;
  a.mid = const_cast<void*>(l.dout);
  a.uoutT = l.G;
  a.bias = reinterpret_cast<const float*>(ws + L.zero);
  a.out = ws + L.h;
  if ((e = launch_outproj(a, st)) != hipSuccess) return e;
  // dx and dp from H
  if (bf && l.p_f32)
    hipLaunchKernelGGL((dev::k_latent_dx_dp<uint16_t, float>), dim3(cdiv(l.B, 4)), dim3(256), 0,
                       st, reinterpret_cast<const uint16_t*>(ws + L.h), w,
                       static_cast<const uint16_t*>(l.x), l.idx, l.B, (int)l.E, (int)l.k,
                       (int)l.r3, static_cast<uint16_t*>(l.dx), static_cast<float*>(l.dp));
  else if (bf)
    hipLaunchKernelGGL((dev::k_latent_dx_dp<uint16_t, uint16_t>), dim3(cdiv(l.B, 4)), dim3(256), 0,
                       st, reinterpret_cast<const uint16_t*>(ws + L.h), w,
                       static_cast<const uint16_t*>(l.x), l.idx, l.B, (int)l.E, (int)l.k,
                       (int)l.r3, static_cast<uint16_t*>(l.dx), static_cast<uint16_t*>(l.dp));
  else
    hipLaunchKernelGGL((dev::k_latent_dx_dp<float, float>), dim3(cdiv(l.B, 4)), dim3(256), 0, st,
                       reinterpret_cast<const float*>(ws + L.h), w, static_cast<const float*>(l.x),
                       l.idx, l.B, (int)l.E, (int)l.k, (int)l.r3, static_cast<float*>(l.dx),
                       static_cast<float*>(l.dp));
  if ((e = hipGetLastError()) != hipSuccess) return e;
  // dG: token-major transposes (zero-padded to Bp tokens), then the weighted GEMM
  // in K slices and the sum of the slices
  if (bf) {
    if ((e = transpose_pad<uint16_t>(l.x, ws + L.xt, l.B, l.r3, L.bp, st)) != hipSuccess) return e;
    if ((e = transpose_pad<uint16_t>(l.dout, ws + L.dt, l.B, l.r2, L.bp, st)) != hipSuccess) return e;
  } else {
    if ((e = transpose_pad<float>(l.x, ws + L.xt, l.B, l.r3, L.bp, st)) != hipSuccess) return e;
    if ((e = transpose_pad<float>(l.dout, ws + L.dt, l.B, l.r2, L.bp, st)) != hipSuccess) return e;
  }
  if ((e = transpose_pad<float>(w, ws + L.wt, l.B, l.E, L.bp, st)) != hipSuccess) return e;
  const int64_t tiles = (M + kDgBM - 1) / kDgBM * ((l.r2 + kDgBN - 1) / kDgBN);
  float* parts = reinterpret_cast<float*>(ws + L.parts);
  const dim3 grid((unsigned)tiles, (unsigned)L.slices), block(64 * 2 * 2);
  if (bf)
    hipLaunchKernelGGL((dev::k_latent_dg<EltBF16, kDgBM, kDgBN, 2, 2, 2>), grid, block, 0, st,
                       (const void*)(ws + L.xt), reinterpret_cast<const float*>(ws + L.wt),
                       (const void*)(ws + L.dt), L.bp, (int)l.E, (int)l.r3, (int)l.r2, L.slices,
                       parts);
  else
    hipLaunchKernelGGL((dev::k_latent_dg<EltF32, kDgBM, kDgBN, 2, 2, 2>), grid, block, 0, st,
                       (const void*)(ws + L.xt), reinterpret_cast<const float*>(ws + L.wt),
                       (const void*)(ws + L.dt), L.bp, (int)l.E, (int)l.r3, (int)l.r2, L.slices,
                       parts);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const int64_t n = M * l.r2;
  if (bf)
    hipLaunchKernelGGL(dev::k_sum_planes<uint16_t>, dim3(cdiv(n, 1024) < 4096 ? cdiv(n, 1024) : 4096),
                       dim3(256), 0, st, parts, L.slices, n, static_cast<uint16_t*>(l.dG));
  else
    hipLaunchKernelGGL(dev::k_sum_planes<float>, dim3(cdiv(n, 1024) < 4096 ? cdiv(n, 1024) : 4096),
                       dim3(256), 0, st, parts, L.slices, n, static_cast<float*>(l.dG));
  return hipGetLastError();
}

}  // namespace tmoe
