// Hardware probes for the measurement side of bench.py: what the MI355X itself
// sustains on the two resources the layer's kernels are bound by, measured on the
// box the bench runs on (built as libtmoe_probe.so, not part of libtmoe.so).
//
//  * tmoe_probe_mfma: bf16 v_mfma_f32_32x32x16 throughput of the whole chip, one
//    work-group of 4 waves per compute unit, 8 independent accumulators per wave,
//    with constant or random operands (the latter moves more bits per cycle and
//    the chip lowers its clock to stay within its power limit), and the mean
//    shader clock over the run (s_memtime against the 100 MHz s_memrealtime).
//  * tmoe_probe_l2_stream: bytes per second one compute unit streams from L2 when
//    every compute unit reads the same L2-resident 1 MB (rotated per work-group),
//    by 16-byte-per-lane loads into registers or by LDS DMA (global_load_lds),
//    with a given number of waves and of 1 KB loads in flight per wave.
//
// Only bench.py calls these; every launch here is synchronous and self-contained.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tmoe_probe.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// clk[4 b + 2 at], clk[4 b + 2 at + 1]: the shader clock and the 100 MHz clock of
// work-group b at its start (at = 0) and end (at = 1), read by wave 0, lane 0
__device__ __forceinline__ void clock_stamp(unsigned long long* clk, int at) {
  if (threadIdx.x == 0) {
    clk[4 * blockIdx.x + 2 * at] = __builtin_amdgcn_s_memtime();
    clk[4 * blockIdx.x + 2 * at + 1] = __builtin_amdgcn_s_memrealtime();
  }
}

__global__ __launch_bounds__(256) void k_probe_mfma(float* sink, unsigned long long* clk, int iters,
                                                    int random_operands) {
  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = f32x16{};
  u32x4 ra[4], rb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (random_operands) {
        // bf16 pairs with random sign and mantissa, exponents near 1
        const uint32_t h = mix32(threadIdx.x * 131u + blockIdx.x * 7919u + (uint32_t)(i * 4 + e));
        ra[i][e] = (h & 0x807f807fu) | 0x3f003f00u;
        rb[i][e] = (mix32(h + 99u) & 0x807f807fu) | 0x3f003f00u;
      } else {
        ra[i][e] = 0x3f803f80u;   // 1.0, 1.0
        rb[i][e] = 0x3f803f80u;
      }
    }
  clock_stamp(clk, 0);
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                   : "+a"(acc[i])
                   : "v"(ra[i & 3]), "v"(rb[(i + it) & 3]));
  }
  clock_stamp(clk, 1);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += acc[i][threadIdx.x & 15];
  if (s == 1234.5f) sink[0] = s;   // keeps the accumulators live
}

constexpr int kStreamChunks = 1024;   // 1 KB chunks of the 1 MB buffer

template <int NW, int U>
__global__ __launch_bounds__(64 * NW) void k_probe_stream(const u32x4* __restrict__ buf,
                                                           uint32_t* sink, int passes) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rot = blockIdx.x * 37;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int p = 0; p < passes; ++p)
    for (int c0 = wave * U; c0 < kStreamChunks; c0 += NW * U) {
      u32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = buf[((c0 + u + rot) & (kStreamChunks - 1)) * 64 + lane];
#pragma unroll
      for (int u = 0; u < U; ++u) acc += v[u];
    }
  if (acc.x == 0x12345u && acc.w == 7u) sink[0] = acc.y;
}

template <int NW, int U>
__global__ __launch_bounds__(64 * NW) void k_probe_stream_dma(const u32x4* __restrict__ buf,
                                                               uint32_t* sink, int passes) {
  __shared__ u32x4 stage[NW * U * 64];
  typedef __attribute__((address_space(3))) void* lds_vptr;
  typedef const __attribute__((address_space(1))) void* gbl_cvptr;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rot = blockIdx.x * 37;
  for (int p = 0; p < passes; ++p)
    for (int c0 = wave * U; c0 < kStreamChunks; c0 += NW * U) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        __builtin_amdgcn_global_load_lds(
            (gbl_cvptr)(buf + ((c0 + u + rot) & (kStreamChunks - 1)) * 64 + lane),
            (lds_vptr)(stage + (wave * U + u) * 64), 16, 0, 0);
      __builtin_amdgcn_s_waitcnt(0);   // every counter at zero
    }
  __syncthreads();
  if (stage[lane].x == 0x12345u && stage[lane].w == 7u) sink[0] = stage[lane].y;
}

int cu_count() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return n;
}

struct Timer {
  hipEvent_t e0 = nullptr, e1 = nullptr;
  bool ok() { return hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess; }
  ~Timer() {
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
  }
};

}  // namespace

extern "C" int tmoe_probe_mfma(int random_operands, int iters, double* tflops, double* shader_mhz) {
  if (!tflops || !shader_mhz || iters < 1) return -1;
  const int ncu = cu_count();
  if (ncu <= 0) return -3;
  float* sink = nullptr;
  unsigned long long* clk = nullptr;
  Timer t;
  int rc = 0;
  if (hipMalloc(&sink, 64) != hipSuccess || hipMalloc(&clk, sizeof(unsigned long long) * 4 * ncu) != hipSuccess ||
      !t.ok()) {
    rc = -3;
  } else {
    float ms = 0.f;
    hipLaunchKernelGGL(k_probe_mfma, dim3(ncu), dim3(256), 0, 0, sink, clk, iters, random_operands);
    bool good = hipDeviceSynchronize() == hipSuccess && hipEventRecord(t.e0, 0) == hipSuccess;
    if (good) hipLaunchKernelGGL(k_probe_mfma, dim3(ncu), dim3(256), 0, 0, sink, clk, iters, random_operands);
    good = good && hipEventRecord(t.e1, 0) == hipSuccess && hipEventSynchronize(t.e1) == hipSuccess &&
           hipEventElapsedTime(&ms, t.e0, t.e1) == hipSuccess && ms > 0.f;
    unsigned long long* h = new unsigned long long[4 * ncu];
    good = good && hipMemcpy(h, clk, sizeof(unsigned long long) * 4 * ncu, hipMemcpyDeviceToHost) == hipSuccess;
    if (good) {
      double mhz = 0.0;
      int n = 0;
      for (int b = 0; b < ncu; ++b) {
        const double dc = (double)(h[4 * b + 2] - h[4 * b]), dr = (double)(h[4 * b + 3] - h[4 * b + 1]);
        if (dr > 0.0) {
          mhz += dc / dr * 100.0;
          ++n;
        }
      }
      // per wave and iteration 8 MFMAs of 2 * 32 * 32 * 16 flops; 4 waves per compute unit
      const double flop = 2.0 * 32 * 32 * 16 * 8.0 * (double)iters * 4.0 * ncu;
      *tflops = flop / ((double)ms * 1e-3) * 1e-12;
      *shader_mhz = n ? mhz / n : 0.0;
    } else {
      rc = -3;
    }
    delete[] h;
  }
  if (sink) (void)hipFree(sink);
  if (clk) (void)hipFree(clk);
  return rc;
}

extern "C" int tmoe_probe_l2_stream(int lds_dma, int waves, double* gbps_per_cu) {
  if (!gbps_per_cu || (waves != 4 && waves != 8)) return -1;
  const int ncu = cu_count();
  if (ncu <= 0) return -3;
  u32x4* buf = nullptr;
  uint32_t* sink = nullptr;
  Timer t;
  int rc = 0;
  const int passes = 16;
  if (hipMalloc(&buf, 1 << 20) != hipSuccess || hipMalloc(&sink, 64) != hipSuccess || !t.ok() ||
      hipMemset(buf, 1, 1 << 20) != hipSuccess) {
    rc = -3;
  } else {
    auto launch = [&]() {
      if (!lds_dma && waves == 4)
        hipLaunchKernelGGL((k_probe_stream<4, 8>), dim3(ncu), dim3(256), 0, 0, buf, sink, passes);
      else if (!lds_dma)
        hipLaunchKernelGGL((k_probe_stream<8, 8>), dim3(ncu), dim3(512), 0, 0, buf, sink, passes);
      else if (waves == 4)
        hipLaunchKernelGGL((k_probe_stream_dma<4, 8>), dim3(ncu), dim3(256), 0, 0, buf, sink, passes);
      else
        hipLaunchKernelGGL((k_probe_stream_dma<8, 8>), dim3(ncu), dim3(512), 0, 0, buf, sink, passes);
    };
    float ms = 0.f;
    launch();
    bool good = hipDeviceSynchronize() == hipSuccess && hipEventRecord(t.e0, 0) == hipSuccess;
    if (good) launch();
    good = good && hipEventRecord(t.e1, 0) == hipSuccess && hipEventSynchronize(t.e1) == hipSuccess &&
           hipEventElapsedTime(&ms, t.e0, t.e1) == hipSuccess && ms > 0.f;
    if (good)
      *gbps_per_cu = (double)(1 << 20) * passes / ((double)ms * 1e-3) * 1e-9;
    else
      rc = -3;
  }
  if (buf) (void)hipFree(buf);
  if (sink) (void)hipFree(sink);
  return rc;
}
