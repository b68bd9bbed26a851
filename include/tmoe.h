/*
 * tmoe.h — C ABI of the MI355X (gfx950) Tucker-MoE layer forward.
 *
 * The reference exposes this path only as a PyTorch module, not an FFI:
 *   pure_torch_mlx/model.py:41-102  class TuckerMoE(nn.Module)
 *     __init__(d_in, d_out, cfg)    model.py:54-66   (cfg fields: config.py:18,20-24)
 *     forward(x) -> out             model.py:68-102
 *   pure_torch_mlx/weights.py:74-81 _load_tucker  (parameter / checkpoint key contract)
 * Each entry point below names the part of that interface it replaces. A
 * ctypes binding (the reference host language is Python) is the intended caller;
 * every signature uses plain C types and pointers, no torch or HIP types.
 *
 * Conventions
 *   - All data pointers are DEVICE pointers owned by the caller, 16-byte aligned,
 *     row-major and contiguous. Nothing here allocates device memory or
 *     synchronises the host with the device, except tmoe_prof_read().
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream). Work is
 *     enqueued on it in order; results are ready when the stream reaches them.
 *   - Every call validates its arguments on the host before any HIP call and
 *     returns 0 on success or a negative TMOE_E* code; tmoe_last_error() then
 *     holds a message (thread-local). Validation failures never touch the GPU,
 *     so every error path can be exercised on a machine without one.
 *   - A plan is immutable after creation: concurrent tmoe_forward calls with one
 *     plan on different streams are safe when their workspaces differ.
 */
#ifndef TMOE_H
#define TMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TMOE_ABI_VERSION 12

/* error codes */
#define TMOE_OK            0
#define TMOE_EINVAL       -1  /* bad argument: null/misaligned pointer, bad size     */
#define TMOE_EUNSUPPORTED -2  /* valid for the reference, not supported by a kernel */
#define TMOE_EHIP         -3  /* a HIP runtime call failed                           */
#define TMOE_ESIGNAL      -4  /* an earlier forward's kernel recorded a lost in-launch
                                 signal (tmoe_signal_status)                          */

/* element types */
#define TMOE_F32  0
#define TMOE_BF16 1
/* bf16 activations, output, router_w, inner_w, U_expert and bias; U_in, core and
 * U_out as OCP fp8 e4m3 with one fp32 scale per output channel (packed by
 * tmoe_pack_weights_fp8). The kernels convert e4m3 to bf16 exactly and compute as
 * for TMOE_BF16, applying the scales in fp32. */
#define TMOE_BF16_FP8W 2

/* router modes (tmoe_shape.router_mode) */
#define TMOE_ROUTER_SOFTMAX_TOPK 0  /* the reference module: softmax over the k selected logits */
#define TMOE_ROUTER_CAPPED       1  /* the trained checkpoints' router, see tmoe_shape */

/* Layer hyper-parameters.
 * Replaces TuckerMoE.__init__(d_in, d_out, cfg) (model.py:54-66):
 *   E = cfg.kmoe_num_experts, k = cfg.kmoe_top_k, r1/r2/r3 = cfg.kmoe_r1/_r2/_r3,
 *   eps = cfg.rms_norm_eps (config.py:18,20-24). dtype = the module's parameter
 *   dtype, which the reference forward also computes in.
 * router_mode TMOE_ROUTER_SOFTMAX_TOPK (0) is model.py:75-77. TMOE_ROUTER_CAPPED (1)
 * is the router the trained checkpoints use (mamba3_mlx/mlx_model/tucker_moe.py:107-114,
 * ops.py:9-14): score = router_scale * tanh(logit / router_scale) / router_temperature
 * with tanh(u) = 2 sigmoid(2u) - 1; top-k by score; weights = softmax over all E of the
 * scores, taken at the selected experts and divided by (their sum + 1e-6). The
 * reference's inference values are router_scale = 10, router_temperature = 0.5; both
 * must be > 0 (unused in mode 0). */
/* plan flags (tmoe_shape.flags) */
#define TMOE_FLAG_NO_FOLD 1  /* keep the core and the out-projection as two GEMMs */
#define TMOE_FLAG_NO_FUSE 2  /* never run the large-T forward as one launch (see
                                tmoe_forward): front and out-projection as two */

typedef struct tmoe_shape {
  int64_t d_in, d_out;
  int64_t E, k;
  int64_t r1, r2, r3;
  int32_t dtype;   /* TMOE_BF16 or TMOE_F32: activations, weights and output;
                      TMOE_BF16_FP8W: bf16 activations, e4m3 projection weights */
  float   eps;
  int32_t router_mode;
  float   router_scale, router_temperature;
  int32_t flags;   /* TMOE_FLAG_* (0: the library chooses) */
} tmoe_shape;

typedef struct tmoe_plan tmoe_plan;

/* Returns TMOE_ABI_VERSION of the loaded library. */
int tmoe_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* tmoe_last_error(void);

/* Validates `shape` and builds a plan (host memory only).
 * Replaces the shape checks torch performs inside TuckerMoE.forward: a top_k
 * larger than E raises in torch.topk (model.py:76) and gives TMOE_EINVAL here.
 * Shapes the reference accepts but these kernels do not (see the message) give
 * TMOE_EUNSUPPORTED. */
int tmoe_plan_create(const tmoe_shape* shape, tmoe_plan** plan_out);
void tmoe_plan_destroy(tmoe_plan* plan);

/* Bytes of the packed-weight buffer for tmoe_pack_weights. */
size_t tmoe_packed_bytes(const tmoe_plan* plan);

/* Rank of the core contraction the kernels run for this plan (0 for a null plan):
 * r1, or E when the plan has fewer experts than ranks and its weights are not fp8
 * (and the persistent core kernel is kept). Then tmoe_pack_weights packs the
 * expert form of model.py:87-98, G_e = sum_r U_expert[e, r] core[r] (E x r3 x r2,
 * summed in fp32 and rounded once to the weight dtype, as the reference's per-slot
 * einsum rounds its product), with U_expert the identity: the same layer with E/r1
 * of the core's multiply-adds. No counterpart in the reference (its module always
 * forms the per-token expert matrices). */
int64_t tmoe_plan_core_rank(const tmoe_plan* plan);

/* 1 if the plan's forward runs the folded form, else 0 (also for a null plan). The layer is linear after the routing, so with c = sum_j w_j
 * U_expert[e_j] (model.py:91-93) and z the normalised in-projection (:80-81),
 *   out = sum_r c_r (z core_r) U_out + bias = (c (x) z) W + bias,
 *   W = core viewed as (r1*r3, r2) times U_out: (r1*r3, d_out),
 * with (c (x) z)[t, r*r3 + s] = c[t, r] z[t, s] (the Khatri-Rao row product).
 * tmoe_pack_weights then also packs W (summed in fp32 over r2, rounded once to
 * bf16; fp8 plans fold the dequantised core and U_out), and the forward runs one
 * GEMM of c (x) z (T, r1*r3) against W: for T > 256 the rows are written in place of
 * mid, for T <= 256 the out-projection forms them from z and c. Chosen for bf16
 * and fp8-weight plans when it takes fewer multiply-adds per token,
 * r1*r3*d_out < r1*r3*r2 + r2*d_out (the reference's ranks (4, 1024, 256):
 * 2.36 M against 3.41 M), unless shape.flags has TMOE_FLAG_NO_FOLD. No counterpart
 * in the reference, which contracts z with the per-token core (model.py:87-98)
 * and then projects through U_out (:101). */
int tmoe_plan_folded(const tmoe_plan* plan);

/* Version of the packed-weight layout that tmoe_pack_weights / _fp8 write and
 * tmoe_forward reads. No counterpart in the reference (whose checkpoints hold the
 * module parameters, pure_torch_mlx/weights.py:74-81): a packed buffer saved to a
 * file is valid for a library of the same layout version and plan shape; for any
 * other, re-pack from the parameters. */
int tmoe_packed_layout_version(void);

/* Bytes of device workspace tmoe_forward needs for T tokens (T >= 0). */
size_t tmoe_workspace_bytes(const tmoe_plan* plan, int64_t T);

/* Re-lays the module parameters into the kernels' operand layouts.
 * Replaces the parameter set of TuckerMoE (model.py:60-66, loaded by
 * weights.py:74-81). Inputs are the parameters as the module holds them, in the
 * plan's dtype:
 *   router_w (E, d_in)   U_in (d_in, r3)   inner_w (r3)   U_expert (E, r1)
 *   core (r1, r3, r2)    U_out (r2, d_out) bias (d_out)
 * `packed` must hold tmoe_packed_bytes(plan) bytes. Stream-ordered. The packed
 * buffer is derived state: pack again whenever a parameter changes. */
int tmoe_pack_weights(const tmoe_plan* plan,
                      const void* router_w, const void* U_in, const void* inner_w,
                      const void* U_expert, const void* core, const void* U_out,
                      const void* bias, void* packed, void* stream);

/* tmoe_pack_weights for a TMOE_BF16_FP8W plan (TMOE_EINVAL for any other plan,
 * and tmoe_pack_weights gives TMOE_EINVAL for this one). The reference has no
 * fp8 parameters: the layer it computes is TuckerMoE (model.py:60-66) with the
 * dequantised weights
 *   U_in[i, j]     = e4m3(U_in_q[i, j])     * U_in_scale[j]          (d_in, r3), scales (r3)
 *   core[r, s, q]  = e4m3(core_q[r, s, q])  * core_scale[r * r2 + q] (r1, r3, r2), scales (r1, r2)
 *   U_out[i, n]    = e4m3(U_out_q[i, n])    * U_out_scale[n]         (r2, d_out), scales (d_out)
 * i.e. one scale per output channel of each projection (for core, per column of
 * its (r3, r1*r2) matrix view). e4m3 is OCP FP8 E4M3 (bias 7, no infinities,
 * 0x7f / 0xff are NaN). router_w, inner_w, U_expert and bias are bf16. Scales
 * must be finite; a zero scale zeroes its channel. */
int tmoe_pack_weights_fp8(const tmoe_plan* plan, const void* router_w,
                          const uint8_t* U_in_q, const float* U_in_scale,
                          const void* inner_w, const void* U_expert,
                          const uint8_t* core_q, const float* core_scale,
                          const uint8_t* U_out_q, const float* U_out_scale,
                          const void* bias, void* packed, void* stream);

/* The layer forward for T tokens: out = TuckerMoE.forward(x) (model.py:68-102).
 *   x        (T, d_in)   plan dtype
 *   out      (T, d_out)  plan dtype
 *   topk_idx (T, k) int32, nullable: selected experts, descending logit (router
 *            mode 1: descending score), ties to the lower index (torch.topk's
 *            indices, model.py:76)
 *   topk_w   (T, k) f32, nullable: the routing weights (mode 0: softmax over the k
 *            selected logits, model.py:77)
 *   logits   (T, E) f32, nullable: router scores x @ router_w^T (model.py:75)
 *   workspace of at least tmoe_workspace_bytes(plan, T) bytes. Its contents need
 *            no initialisation: kernels whose work-groups hand data to each other
 *            inside one launch (the T <= 64 bf16 decode launch, the E = 256 front,
 *            the one-launch large-T forward) tag their signal words with a value
 *            drawn per launch, and wait for one at most a budget of polls
 *            (tmoe_set_wait_polls; about a second by default). Past it the affected
 *            rows come out NaN (or stale), the launch still completes, and the
 *            plan's status records it: tmoe_signal_status reports TMOE_ESIGNAL.
 * The large-T forward of a folded bf16 plan with r3 = 256, E <= 32 and d_out a
 * multiple of 288 runs as one launch (front and out-projection in one persistent
 * grid, one work-group per compute unit) on a 256-compute-unit device when its
 * 256 x 288 output tiles number at least 256 (T >= 8192 at d_out = 2304), unless
 * the plan has TMOE_FLAG_NO_FUSE.
 * T == 0 is a no-op. Stream-ordered, no allocation, no host synchronisation. Under
 * HIP graph capture the kernels whose signal flags have several consumers are not
 * used (their flags would read as already set on a replay): decode-size batches,
 * the large-T forward and the E = 256 front take their multi-launch paths. */
int tmoe_forward(const tmoe_plan* plan, const void* x, int64_t T, const void* packed,
                 void* out, int32_t* topk_idx, float* topk_w, float* logits,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Fused elementwise epilogues of tmoe_forward_epi (the FFN sub-block of the
 * reference's TransformerBlock, model.py:337-341). y is the layer output
 * TuckerMoE.forward(x) rounded to the plan dtype; R() rounds to the plan dtype.
 *   TMOE_EPI_NONE            out = y
 *   TMOE_EPI_GLU             out = R(R(silu(epi_a)) * y)        F.silu(gate) * up   (:340)
 *                            epi_a = gate (T, d_out), silu(g) = g / (1 + exp(-g))
 *   TMOE_EPI_RESIDUAL_SCALE  out = R(epi_a + R(epi_b * y))       x_res + ls_ffn(dn)  (:341)
 *                            epi_a = x_res (T, d_out), epi_b = LayerScale gamma (d_out)
 *                            (LayerScale.forward, model.py:35-36) */
#define TMOE_EPI_NONE           0
#define TMOE_EPI_GLU            1
#define TMOE_EPI_RESIDUAL_SCALE 2

/* tmoe_forward with one of the TMOE_EPI_* ops fused into the out-projection's
 * store: no counterpart of its own in the reference, it computes the expression
 * of model.py:340 or :341 that consumes this layer's output (ffn_up's output with
 * epi = GLU of the gate output; ffn_down's with epi = RESIDUAL_SCALE). epi_a and
 * epi_b are device tensors in the plan's activation dtype (bf16 for
 * TMOE_BF16_FP8W), 16-byte aligned; epi_a may be `out` itself (each element is
 * read before it is written, by the same thread), which updates a residual
 * stream in place. Other arguments and errors as tmoe_forward; tmoe_forward is
 * tmoe_forward_epi with TMOE_EPI_NONE. */
int tmoe_forward_epi(const tmoe_plan* plan, const void* x, int64_t T, const void* packed,
                     void* out, int32_t* topk_idx, float* topk_w, float* logits,
                     void* workspace, size_t workspace_bytes, int epi_mode,
                     const void* epi_a, const void* epi_b, void* stream);

/* tmoe_forward without a workspace argument: no counterpart in the reference. For
 * callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc): the forward's workspace is a
 * static device array of tmoe_static_scratch_bytes() bytes (48 MiB: T up to 16384
 * at the reference's C3 shape) that each GPU the library runs on holds until the
 * process ends; this call allocates nothing. T whose workspace
 * (tmoe_workspace_bytes) exceeds it gives TMOE_EUNSUPPORTED before any GPU work.
 * All calls on one GPU share that GPU's array: calls that overlap on one GPU (on
 * different streams, or from different threads without ordering) race. The array
 * used is that of the device `stream` belongs to (the current device for the null
 * stream). Arguments, results and errors otherwise as tmoe_forward; not recorded by
 * tmoe_prof_*. */
size_t tmoe_static_scratch_bytes(void);
int tmoe_forward_static(const tmoe_plan* plan, const void* x, int64_t T, const void* packed,
                        void* out, int32_t* topk_idx, float* topk_w, float* logits,
                        void* stream);

/* The kernel sequence an eager tmoe_forward of T tokens runs with this plan on the
 * current device (on a machine without a GPU: as on a 256-compute-unit MI355X).
 * No counterpart in the reference; for measurement tools, which attribute time
 * per kernel. Returns one of TMOE_PATH_* (0 for T == 0) or a negative error. */
#define TMOE_PATH_SMALL  1  /* T <= 256: skinny kernels, two or three launches        */
#define TMOE_PATH_DECODE 2  /* T <= 64, bf16, folded: the whole layer in one launch   */
#define TMOE_PATH_LARGE  3  /* front, (core or c (x) z), out-projection launches      */
#define TMOE_PATH_FUSED  4  /* large T, folded: the whole layer in one launch         */
#define TMOE_PATH_LARGE_KR 5 /* large T, folded, E > 128: front (stores z and c) and an
                               out-projection that forms c (x) z in its loop            */
#define TMOE_PATH_FUSED_MID 6 /* mid T (256 < T <= 2048 at d_out = 2304), folded, r3 = 256,
                                E <= 32: the whole layer in one launch (K-sliced front and
                                128 x 144 out-projection tiles)                          */
int tmoe_forward_path(const tmoe_plan* plan, int64_t T);

/* Lost in-launch signals. No counterpart in the reference (its forward has no
 * kernels that wait for each other; torch raises its errors from the call).
 * A kernel whose wait for another work-group of its launch runs out of its poll
 * budget sets a word of the plan's status block (pinned host memory the kernels
 * write directly; allocated by tmoe_plan_create when a GPU is present).
 * tmoe_signal_status reads it without synchronising: it reflects the kernels of
 * this plan that have completed. For a definitive answer about a forward,
 * synchronise its stream first. Returns TMOE_OK, or TMOE_ESIGNAL with *mask
 * (nullable) holding the TMOE_STATUS_* bits; clear != 0 resets the block. Rows
 * affected by a lost signal are NaN or stale; nothing else of the forward is. */
#define TMOE_STATUS_SIGNAL    1u  /* a wait ran out of its poll budget */
int tmoe_signal_status(const tmoe_plan* plan, int clear, uint32_t* mask);

/* Sets the budget of every in-launch wait of later forwards, in polls of the
 * awaited flags (default 1000000, about a second), process-wide; returns the
 * previous budget. polls < 0 only returns it. A budget of 0 makes every wait give
 * up without looking at its flags, so that the lost-signal path can be exercised
 * with every kernel still exiting normally (its forwards then produce NaN rows and
 * TMOE_ESIGNAL). No counterpart in the reference. */
int64_t tmoe_set_wait_polls(int64_t polls);

/* out = R(R(silu(gate(x))) * up(x)) for two layers of one plan over the same input:
 * F.silu(ffn_gate(x_f)) * ffn_up(x_f) of model.py:338-340, i.e. tmoe_forward of the
 * gate's packed weights into `out` followed by tmoe_forward_epi(TMOE_EPI_GLU, out) of
 * the up's (bit for bit the same result). The two layers' fronts run in one launch
 * where the kernels allow (bf16, r3 = 256: the two run side by side on the compute
 * units, which a T that leaves most of them idle per layer rewards). ws_gate and
 * ws_up: two distinct workspaces of workspace_bytes >= tmoe_workspace_bytes(plan, T)
 * each. No routing outputs; not recorded by tmoe_prof_*. */
int tmoe_forward_glu(const tmoe_plan* plan, const void* x, int64_t T, const void* packed_gate,
                     const void* packed_up, void* out, void* ws_gate, void* ws_up,
                     size_t workspace_bytes, void* stream);

/* out (T, d) = RMSNorm(x) (T, d) with gain weight (d): RMSNorm.forward of
 * model.py:25-27, (x / sqrt(mean(x^2) + eps)) * weight, computed in fp32 and
 * rounded to dtype (TMOE_BF16 or TMOE_F32) once. The FFN sub-block's norm_ffn
 * (model.py:337). out may not overlap x. Stream-ordered, no allocation. */
int tmoe_rmsnorm_rows(const void* x, int64_t T, int64_t d, const void* weight, float eps,
                      int dtype, void* out, void* stream);

/* The latent expert contraction of the reference's training module and its
 * backward: FusedLatentMoE.forward / .backward (sft_cot_bundle/scripts/model.py:225-289,
 * with the dG kernel :196-219), as called by TritonTuckerMoE.forward (:336-338).
 *   x    x_shared     (B, r3)      dtype      out  (B, r2)  dtype
 *   G    G_experts    (E, r3, r2)  dtype      dx   (B, r3)  dtype
 *   idx  top_k_indices (B, k)      int64      dG   (E, r3, r2) dtype
 *   p    top_k_probs   (B, k)      dtype      dp   (B, k)   dtype
 *   out[b] = sum_j p[b,j] x[b] G[idx[b,j]];  with dout = dL/dout:
 *   dx[b] = sum_j p[b,j] dout[b] G[idx[b,j]]^T,  dp[b,j] = dout[b] . (x[b] G[idx[b,j]]),
 *   dG[e] = sum_{b,j: idx[b,j] = e} p[b,j] x[b]^T dout[b].
 * dtype TMOE_BF16 or TMOE_F32 (products in fp32 accumulators, each output rounded
 * once), optionally OR'ed with TMOE_LATENT_P_F32: p and dp are then fp32 whatever
 * dtype is (the reference's kernels read top_k_probs in their own dtype, and its
 * dprobs has that dtype; model.py:160-174, :196-219, :250); r3 in {64, 128, 256}, r2 a multiple of 64, 1 <= k <= min(E, 16), E <= 64.
 * An index outside [0, E) selects nothing. All pointers device, 16-byte aligned;
 * workspace of at least tmoe_latent_workspace_bytes(...) bytes. B == 0 is a no-op.
 * Stream-ordered, no allocation, no host synchronisation. */
#define TMOE_LATENT_P_F32 0x100
size_t tmoe_latent_workspace_bytes(int64_t B, int64_t E, int64_t r3, int64_t r2, int dtype,
                                   int backward);
int tmoe_latent_forward(const void* x, const void* G, const int64_t* idx, const void* p,
                        int64_t B, int64_t E, int64_t k, int64_t r3, int64_t r2, int dtype,
                        void* out, void* workspace, size_t workspace_bytes, void* stream);
int tmoe_latent_backward(const void* x, const void* G, const int64_t* idx, const void* p,
                         const void* dout, int64_t B, int64_t E, int64_t k, int64_t r3,
                         int64_t r2, int dtype, void* dx, void* dG, void* dp, void* workspace,
                         size_t workspace_bytes, void* stream);

/* Per-stage timing, no counterpart in the reference (measurement support).
 * While enabled, every tmoe_forward records a HIP event before each of its
 * kernels and one after the last, on the forward's stream. tmoe_prof_read waits
 * for those events, writes the summed milliseconds per stage into ms[0..n-1]
 * (stage order: front = router + in-projection, core, out-projection), the number of
 * forwards into *calls, and clears the record. Returns the stage count. Not
 * thread-safe; for benchmarks only. */
int tmoe_prof_enable(int on);
int tmoe_prof_read(double* ms, int n, int64_t* calls);

#ifdef __cplusplus
}
#endif

#endif /* TMOE_H */
