/* Hardware probes of the measurement harness (libtmoe_probe.so, built beside
 * libtmoe.so). They have no counterpart in the reference: bench.py reports their
 * figures next to the layer's roofline, as what this MI355X sustains on the two
 * resources the layer's kernels are bound by. Return 0, or -1 (bad argument) /
 * -3 (HIP error). Synchronous; they allocate and free their own small buffers. */
#ifndef TMOE_PROBE_H
#define TMOE_PROBE_H

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 MFMA (v_mfma_f32_32x32x16_bf16) throughput of the whole device in TFLOP/s,
 * one 4-wave work-group per compute unit, `iters` x 8 MFMAs per wave; operands
 * constant (random_operands = 0) or random bf16; *shader_mhz: the mean shader
 * clock over the timed launch. */
int tmoe_probe_mfma(int random_operands, int iters, double* tflops, double* shader_mhz);

/* GB/s one compute unit streams from L2 (every compute unit reads the same
 * L2-resident 1 MB, 8 KB in flight per wave), by loads into registers
 * (lds_dma = 0) or by LDS DMA (lds_dma = 1), with `waves` = 4 or 8 per work-group. */
int tmoe_probe_l2_stream(int lds_dma, int waves, double* gbps_per_cu);

#ifdef __cplusplus
}
#endif

#endif /* TMOE_PROBE_H */
