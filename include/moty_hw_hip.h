/* moty_hw_hip.h -- libmoty-hw-hip: the MI355X (gfx950) backend for moty's
 * quantized-matmul and MoE hot path, as a plain C ABI.
 *
 * Two surfaces:
 *  1. Host-pointer drop-ins with the reference's own signatures and argument
 *     meaning.  Weights are uploaded once, on first use, into a device cache
 *     keyed by the host pointer (weights are persistent for a model's life in
 *     the reference, nn/nn_mat.h:18-25); x is uploaded and y downloaded per
 *     call; the call is synchronous, like the CPU kernels.
 *  2. Device-pointer entry points (suffix _dev): every pointer is device
 *     memory, work is queued on `stream` (a hipStream_t, NULL = the default
 *     stream) and returns without synchronising.
 *
 * Every function returns MOTY_HIP_OK (0) or an error code, and never aborts;
 * moty_hip_last_error() describes the failure of this thread's last call
 * (empty after a call that succeeded).  A caller that keeps a CPU path (as
 * engines/glm.c:798-810 does for its CUDA matmul) falls back on a nonzero
 * return.  Calls share library-owned scratch per device and are not
 * re-entrant from several host threads at once, like the reference's
 * process-static activation buffers (nn/matmul.c:55-58).  Sequential _dev
 * calls may use different streams: a call whose stream differs from the
 * previous scratch user's is ordered behind that stream's queued work.
 * Under HIP graph capture that ordering is not added: capture the calls of
 * one device on one stream.
 *
 * Numerics match the reference's x86-64 AVX512-VNNI build: int8 activations
 * and int32 accumulators bit-exact, float steps in the reference's order
 * (including the FMAs gcc contracts), expf identical to glibc's.
 */
#ifndef MOTY_HW_HIP_H
#define MOTY_HW_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOTY_HIP_OK 0
#define MOTY_HIP_EINVAL 1  /* bad argument or shape */
#define MOTY_HIP_EHIP 2    /* HIP runtime error (no device, fault, ...) */
#define MOTY_HIP_ENOMEM 3  /* device allocation failed */
#define MOTY_HIP_EUNSUP 4  /* shape/format this backend does not serve */

/* combine order of the MoE layer */
#define MOTY_MOE_ORDER_TOPK 0   /* per token, experts in top-k order: engines/olmoe.c:230-243 */
#define MOTY_MOE_ORDER_EXPERT 1 /* per token, ascending expert id: nn/moe.c:186-203 */

/* ---------------- library ---------------- */
/* Select the device for this thread's calls and create its stream/scratch.
 * Optional: every entry point initialises device 0 on first use. */
int moty_hip_init(int device);
/* Free the weight cache, scratch and stream of every initialised device. */
int moty_hip_shutdown(void);
const char *moty_hip_last_error(void);
/* Kernel tier string, the analogue of HW_IDOT_KERNEL/HW_F32_KERNEL
 * (hw/hw.h:160-208): "gfx950-mfma-i8/gfx950-f32". */
const char *moty_hip_kernel_tier(void);
/* No reference counterpart (the CPU kernels never wait on each other).
 * The one-launch form of the S = 1 Q8 dense FFN (moty_hip_set_ffn1) hands h
 * between workgroups through device memory; every such wait is bounded.  Waits for the current thread's device and returns in *count
 * the number of calls since the last query whose wait ran out (0: every
 * output since then is valid), and clears it. */
int moty_hip_wait_errors(int *count);
/* No reference counterpart: on = 1 routes the S = 1 Q8 dense FFN (when
 * D % 1024 == 0, D <= 2048, I % 1024 == 0, I <= 4096 on a 256-CU device)
 * through the one-launch form instead of the two GEMV launches (gate/up +
 * SiLU, then down), for this thread's device.  Default off (slower on
 * MI355X); env MOTY_FFN1=1 at set-up turns it on.  Both give the same bits. */
int moty_hip_set_ffn1(int on);

/* ---------------- host-pointer drop-ins ---------------- */
/* moty_matmul_q_s (nn/nn_matmul.h:64, nn/matmul.c:51-66): Q8_0 per-row int8
 * weights q [O][I] + scale [O]; x [S][I] f32 token-major; y [S][O].  IDOT=0
 * in the environment is reported as MOTY_HIP_EUNSUP (the f32xint8 variant
 * stays on the CPU). */
int moty_hip_matmul_q_s(float *y, const float *x, const int8_t *q, const float *scale, int S, int I, int O);
/* moty_matmul_i4_grouped_s (nn/nn_matmul.h:67-68, nn/matmul.c:164-197):
 * nibbles q4 [O][(I+1)/2], f32 group scales [O][ceil(I/gs)].  IDOT4 is read
 * from the environment once per process (nn/matmul.c:171): IDOT4=1 with
 * gs == 32, I % 64 == 0, I <= 16384 selects the int8-activation path,
 * anything else the exact f32 path (served for gs == 32, I % 32 == 0). */
int moty_hip_matmul_i4_grouped_s(float *y, const float *x, const uint8_t *q4, const float *scale, int S, int I,
                                 int O, int gs);
/* moty_matmul_q4r4_s (nn/nn_matmul.h:72, nn/matmul.c:395-431): Q4R4 weights
 * (nn/quant.c:157-177) -- 4-row blocks, per (block, group of 32) 64 bytes of
 * packed codes q4 [ceil(O/4)][I/32][4][16] and f16 scales s16
 * [ceil(O/4)][I/32][4]; activations quantized per group of 32
 * (moty_hw_quant_g32).  I % 32 == 0. */
int moty_hip_matmul_q4r4_s(float *y, const float *x, const uint8_t *q4, const uint16_t *s16, int S, int I, int O);
/* moty_matmul_q8r4_s (nn/nn_matmul.h:70, nn/matmul.c:435-466): the int8
 * sibling, q8 [ceil(O/4)][I/32][4][32] signed codes, same scale stream. */
int moty_hip_matmul_q8r4_s(float *y, const float *x, const int8_t *q8, const uint16_t *s16, int S, int I, int O);
/* moty_matmul (nn/nn_matmul.h:63, nn/matmul.c:15-27): f32 W [O][I], dot_f32
 * in the AVX512 order (hw/hw_avx512.h:231-243).  The f32 MoE router. */
int moty_hip_matmul(float *y, const float *x, const float *W, int S, int I, int O);

/* The MoE layer's inputs (the device analogue of MotyMoeView, nn/moe.h:19-33,
 * with the experts resident instead of behind an ExpertCache):
 * router [E][D] f32; experts stacked g,u [E][I][D], d [E][D][I] int8 with
 * per-row scales gs,us [E][I], ds [E][D] (ExpertSlot, runtime/moe.h:35-39,
 * quantized by moty_quantize_rows with EBITS=8). */
typedef struct MotyHipMoe {
    const float *router;
    const float *logit_bias; /* [E] added to the logits before softmax, or NULL */
    const int8_t *g, *u, *d;
    const float *gs, *us, *ds;
    int E, K, I, D;
    int norm_topk;           /* moty_moe_topk's norm_topk (runtime/moecache.c:97) */
    int combine_order;       /* MOTY_MOE_ORDER_* */
    int32_t *idx_out;        /* optional [S][K] expert ids (same memory kind as x) */
    float *w_out;            /* optional [S][K] routing weights */
    int32_t *counts_out;     /* optional [E] tokens per expert */
} MotyHipMoe;

/* moty_nn_moe_topk_batch (nn/moe.h:38, nn/moe.c:159-208; no shared expert)
 * with combine_order = EXPERT and norm_topk = 1, or the olmoe engine's
 * per-token MoE (engines/olmoe.c:219-244) with combine_order = TOPK.
 * Host pointers; out [S][D].  Served for D, I multiples of 32, E <= 256, K <= 64. */
int moty_hip_moe_topk(const MotyHipMoe *m, const float *x, int S, float *out);

/* ---- expert residency (runtime/moe.h:35-102, runtime/moecache.c:4-95) ----
 * The per-layer ExpertCache with its slots in device memory.  Bookkeeping
 * is the reference's decision for decision (LFRU = heat << 8 | recency,
 * io/tier.c:23-26; pins; hit/miss counters), so the same expert lands in
 * the same slot.  A load calls the caller's loader on a host slot (pinned
 * staging buffers owned by the cache), then copies it to the device slot. */
typedef struct MotyHipExpertSlot { /* ExpertSlot (runtime/moe.h:35-39) */
    int eid;
    int8_t *g, *u, *d;     /* gate [inter][hidden], up [inter][hidden], down [hidden][inter] */
    float *gs, *us, *ds;   /* row scales [inter], [inter], [hidden] */
} MotyHipExpertSlot;
/* LoadExpertFn (runtime/moe.h:54-56): fill s->g/u/d/gs/us/ds (host memory) */
typedef void (*MotyHipLoadExpertFn)(void *ctx, int layer, int eid, MotyHipExpertSlot *s, int inter, int hidden);
typedef struct MotyHipExpertCache MotyHipExpertCache;
/* moty_expert_cache_init / _free (runtime/moecache.c:4-22): cap slots
 * (cap < 1 -> 1), heat/pin tracking for n_experts (0 = none).  Device
 * memory is taken on the first load, for that load's inter/hidden. */
int moty_hip_expert_cache_init(MotyHipExpertCache **lc, int cap, int n_experts);
int moty_hip_expert_cache_free(MotyHipExpertCache *lc);
/* moty_expert_get / moty_expert_pin (runtime/moecache.c:24-89): *slot gets
 * the expert's device slot (device pointers), loaded and ready on return.
 * A slot evicted here must no longer be read by work the caller queued. */
int moty_hip_expert_get(MotyHipExpertCache *lc, void *ctx, int layer, int eid, MotyHipLoadExpertFn fn, int inter,
                        int hidden, MotyHipExpertSlot **slot);
int moty_hip_expert_pin(MotyHipExpertCache *lc, void *ctx, int layer, int eid, MotyHipLoadExpertFn fn, int inter,
                        int hidden, MotyHipExpertSlot **slot);
/* the bookkeeping: filled slots, slot_eids [cap], heat/last [n_experts]
 * (any pointer may be NULL) */
int moty_hip_expert_cache_stats(const MotyHipExpertCache *lc, int *n, int *slot_eids, uint32_t *heat,
                                uint32_t *last, uint32_t *clock, long long *hits, long long *misses);
/* moty_moe_route_bias (runtime/moecache.c:91-95) on host logits [E] */
void moty_hip_moe_route_bias(float *logits, const MotyHipExpertCache *lc, float bias);
/* The MoE layer of moty_hip_moe_topk with the experts behind the cache
 * (m->g/u/d/gs/us/ds unused): moe_batch_core's expert_get per active expert
 * in ascending id (combine_order EXPERT, nn/moe.c:186-203) or olmoe's per
 * token in top-k order (TOPK, engines/olmoe.c:230-233).  Output identical
 * to the uncached layer; reads the routing back to the host once per call. */
int moty_hip_moe_topk_cached(const MotyHipMoe *m, MotyHipExpertCache *lc, void *ctx, int layer,
                             MotyHipLoadExpertFn fn, const float *x, int S, float *out);

/* GGUF block types (io/st.h:74): the dtype argument of the GGUF calls */
#define MOTY_GGUF_Q8_0 4
#define MOTY_GGUF_Q4_0 5
#define MOTY_GGUF_Q4_K 6
#define MOTY_GGUF_Q5_K 7
#define MOTY_GGUF_Q6_K 8

/* gguf_dequant (io/gguf.h:316-326), the g_st_dequant_fn hook of
 * st_read_f32: numel elements (a multiple of the type's block: 32 or 256)
 * from raw blocks to f32.  Host pointers; unknown types -> EUNSUP (the
 * reference exits). */
int moty_hip_gguf_dequant(int dtype, const void *raw, int64_t numel, float *out);
/* gguf_repack_q4_0 (io/gguf.h:340-357) as load_mat_q4_0 uses it
 * (runtime/rt_model_load.h:26-34): Q4_0 blocks of an [O][I] matrix ->
 * grouped int4 q4 [O][I/2] + f32 scales qs [O][I/32], bit-preserving.
 * I a multiple of 32.  Host pointers. */
int moty_hip_gguf_repack_q4_0(const uint8_t *blocks, uint8_t *q4, float *qs, int64_t O, int64_t I);

/* Drop the cached device copy of a host weight buffer (after the caller
 * frees or rewrites it). */
int moty_hip_weight_forget(const void *host_ptr);

/* HwBackend.matmul_i8 slot (hw/hw_backend.h:57-58), which returns void:
 * on failure every y[S*O] is set to a quiet NaN and moty_hip_last_error()
 * says why (it is "" after a call that succeeded).  A caller that keeps the
 * CPU path calls moty_hip_matmul_q_s instead and falls back on nonzero. */
void moty_hip_hw_matmul_i8(float *y, const float *x, const int8_t *q, const float *scale, int S, int I, int O);

/* moty_matmul_i4_s (nn/nn_matmul.h:66, nn/matmul.c:75-145), per-row int4
 * weights (WF_I4): q4 [O][(I+1)/2] nibbles (even element low) + f32 scale
 * [O].  IDOT4 read from the environment once, as nn/matmul.c:76-77.
 * Served for I % 16 == 0 (q4 8-byte, x 16-byte aligned). */
int moty_hip_matmul_i4_s(float *y, const float *x, const uint8_t *q4, const float *scale, int S, int I, int O);
/* HwBackend.matmul_i4 slot (hw/hw_backend.h:59-60), void: on failure every
 * y[S*O] is a quiet NaN and moty_hip_last_error() says why. */
void moty_hip_hw_matmul_i4(float *y, const float *x, const uint8_t *q4, const float *scale, int S, int I, int O);

/* ---------------- device-pointer entry points ---------------- */
/* qrow_i8 over S rows (hw/hw_quant.h:9-16): q [S][I], sx [S]; xg [S][I/32]
 * group sums when non-NULL (I % 32 == 0). */
int moty_hip_qrow_i8_dev(const float *x, int8_t *q, float *sx, int32_t *xg, int S, int I, void *stream);
/* qrow_i8 of up to 4 independent row sets in one launch (job j: x[j] [S[j]][I[j]]
 * -> q[j], sx[j]; I[j] <= 4096, I[j] % 16 == 0, dense 16-byte aligned rows).
 * No counterpart in the reference, which quantizes inside each
 * moty_matmul_q_s call (nn/matmul.c:29-36): for callers that run several
 * prefill GEMMs whose inputs are all ready, so that their quantizations
 * pay one launch. */
int moty_hip_qrow_i8_multi_dev(int n, const float *const *x, int8_t *const *q, float *const *sx, const int *S,
                               const int *I, void *stream);
/* moty_quantize_rows (nn/quant.c:12-33) */
int moty_hip_quantize_rows_dev(const float *w, int8_t *q, float *scale, int O, int I, int bits, void *stream);
/* moty_pack_int4_grouped (nn/quant.c:57-83); gs % 16 == 0 as the reference requires */
int moty_hip_pack_int4_grouped_dev(const float *w, uint8_t *q4, float *scale, int O, int I, int gs,
                                   void *stream);
/* moty_pack_int4 (nn/quant.c:34-55): per-row int4 q4 [O][(I+1)/2], scale [O] */
int moty_hip_pack_int4_dev(const float *w, uint8_t *q4, float *scale, int O, int I, void *stream);
/* moty_matmul_i4_s; idot4 selects the int8-activation path explicitly */
int moty_hip_matmul_i4_s_dev(float *y, const float *x, const uint8_t *q4, const float *scale, int S, int I, int O,
                             int idot4, void *stream);
/* moty_matmul_q_s: S <= 4 runs the decode GEMV with fused activation
 * quantization, larger S quantizes then runs the int8 MFMA GEMM. */
int moty_hip_matmul_q_s_dev(float *y, const float *x, const int8_t *q, const float *scale, int S, int I, int O,
                            void *stream);
/* the Q8 GEMM on activations already quantized by moty_hip_qrow_i8_dev
 * (several projections of one input share one quantization) */
int moty_hip_matmul_q8_preq_dev(float *y, const int8_t *xq, const float *sx, const int8_t *q, const float *scale,
                                int S, int I, int O, void *stream);
/* moty_matmul_i4_grouped_s; idot4 selects the path explicitly */
int moty_hip_matmul_i4_grouped_s_dev(float *y, const float *x, const uint8_t *q4, const float *scale, int S,
                                     int I, int O, int gs, int idot4, void *stream);
/* moty_matmul (f32, dot_f32 order) */
int moty_hip_matmul_dev(float *y, const float *x, const float *W, int S, int I, int O, void *stream);
/* moty_hw_silu_mul (hw/hw_ops.h:19-21): g = silu(g) * u */
int moty_hip_silu_mul_dev(float *g, const float *u, int64_t n, void *stream);
/* moty_softmax_row (nn/norm.c:10, hw/hw_ops.h:22-26) over S rows of n, in place */
int moty_hip_softmax_rows_dev(float *x, int S, int n, void *stream);
/* expf over an array, bit-identical to the glibc expf the reference calls
 * (hw/hw_ops.h:20); the device routine every SiLU/softmax here uses. */
int moty_hip_expf_dev(const float *x, float *y, int64_t n, void *stream);
/* Dense SwiGLU FFN over Q8 weights, moty_nn_dense_ffn (nn/ffn.c:26-55):
 * gate,up [I][D] + scales [I], down [D][I] + scale [D]; x [S][D]; out [S][D]. */
int moty_hip_dense_ffn_q8_dev(float *out, const float *x, int S, const int8_t *gate, const float *gs,
                              const int8_t *up, const float *us, const int8_t *down, const float *ds, int D, int I,
                              void *stream);
/* The decode half of that FFN before the down projection, fused: one pass
 * over the gate and up rows, h [S][I] = silu(x.gate^T) * (x.up^T) -- the
 * gate_up + silu_rows step of nn/ffn.c:28-37.  S <= 4. */
int moty_hip_gate_up_silu_q8_dev(float *h, const float *x, int S, const int8_t *gate, const float *gs,
                                 const int8_t *up, const float *us, int D, int I, void *stream);
/* The same fused decode step over grouped-int4 weights (gs = 32, IDOT4 int8
 * activations): h [I] = silu(x.gate^T) * (x.up^T), one token, D % 64 == 0. */
int moty_hip_gate_up_silu_i4g_dev(float *h, const float *x, const uint8_t *gate, const float *gs,
                                  const uint8_t *up, const float *us, int D, int I, void *stream);
/* moty_nn_dense_ffn (nn/ffn.c:26-55) over grouped-int4 Mats (WF_I4G, gs =
 * 32): gate, up [I][D/2] nibbles + f32 scales [I][D/32], down [D][I/2] +
 * [D][I/32]; x [S][D] -> out [S][D].  idot4 = 1: int8 activations
 * (nn/matmul.c:164-197; gate and up in one pass with the SiLU epilogue);
 * 0: the exact f32 path.  D, I multiples of 32. */
int moty_hip_dense_ffn_i4g_dev(float *out, const float *x, int S, const uint8_t *gate, const float *gs,
                               const uint8_t *up, const float *us, const uint8_t *down, const float *ds, int D,
                               int I, int idot4, void *stream);
/* moty_matmul_q4r4_s / moty_matmul_q8r4_s on device pointers: S <= 3 runs
 * the decode GEMV with fused activation quantization (the reference's
 * per-token form), larger S quantizes then runs the MFMA GEMM (tokens below
 * 4*floor(S/4) in the reference's 4-token tile form, the rest per token). */
int moty_hip_matmul_q4r4_s_dev(float *y, const float *x, const uint8_t *q4, const uint16_t *s16, int S, int I, int O,
                               void *stream);
int moty_hip_matmul_q8r4_s_dev(float *y, const float *x, const int8_t *q8, const uint16_t *s16, int S, int I, int O,
                               void *stream);
/* Decode gate/up + SiLU over a row-fused R4 gate_up matrix (moty_mat_fuse_rows,
 * nn/mat.c:32-68: the I gate rows then the I up rows, I % 4 == 0), the
 * gate_up + silu_rows step of nn/ffn.c:28-37 for one token:
 * h [I] = silu(x.gate^T) * (x.up^T). */
int moty_hip_gate_up_silu_q4r4_dev(float *h, const float *x, const uint8_t *gate_up, const uint16_t *s16, int D,
                                   int I, void *stream);
int moty_hip_gate_up_silu_q8r4_dev(float *h, const float *x, const int8_t *gate_up, const uint16_t *s16, int D,
                                   int I, void *stream);
/* moty_nn_dense_ffn (nn/ffn.c:26-41) with a row-fused R4 gate_up [2I][D]
 * and down [D][I]: x [S][D] -> out [S][D].  D, I multiples of 32. */
int moty_hip_dense_ffn_q4r4_dev(float *out, const float *x, int S, const uint8_t *gate_up, const uint16_t *gus16,
                                const uint8_t *down, const uint16_t *ds16, int D, int I, void *stream);
int moty_hip_dense_ffn_q8r4_dev(float *out, const float *x, int S, const int8_t *gate_up, const uint16_t *gus16,
                                const int8_t *down, const uint16_t *ds16, int D, int I, void *stream);
/* moty_hw_quant_g32 (hw/hw_q4r4.h:36-46) over S rows: xq [S][I], xs and
 * xsum [S][I/32] */
int moty_hip_quant_g32_dev(const float *x, int8_t *xq, float *xs, int32_t *xsum, int S, int I, void *stream);
/* Weight packers: moty_pack_q4r4_block / moty_pack_q8r4_block
 * (nn/quant.c:135-177) over every 4-row block of w [O][I] f32. */
int moty_hip_pack_q4r4_dev(const float *w, uint8_t *q4, uint16_t *s16, int O, int I, void *stream);
int moty_hip_pack_q8r4_dev(const float *w, int8_t *q8, uint16_t *s16, int O, int I, void *stream);
/* GGUF loading on the device: the same two conversions with raw, out,
 * blocks, q4, qs in device memory (out and q4 16-byte aligned, qs 4-byte).
 * Chained with moty_hip_quantize_rows_dev / moty_hip_pack_int4_grouped_dev
 * they give load_mat_bits' QBITS=8 / QBITS=4 paths for every GGUF block
 * type (runtime/rt_model_load.h:122-157). */
int moty_hip_gguf_dequant_dev(int dtype, const void *raw, int64_t numel, float *out, void *stream);
int moty_hip_gguf_repack_q4_0_dev(const uint8_t *blocks, uint8_t *q4, float *qs, int64_t O, int64_t I,
                                  void *stream);
/* the MoE layer, all pointers in m and x/out on the device; x, out, router
 * and g/u/d 16-byte aligned (MOTY_HIP_EUNSUP otherwise) */
int moty_hip_moe_topk_dev(const MotyHipMoe *m, const float *x, int S, float *out, void *stream);
/* No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The MoE layer of moty_hip_moe_topk_dev, bit for bit, with its
 * scratch in a fixed 64 MiB device array the library holds per GPU until
 * the process ends.  Its set-up (the array's device address, one event) is
 * done by moty_hip_init, which the calling thread must have called first
 * (it allocates; this entry point returns MOTY_HIP_EINVAL otherwise); the
 * call itself does no hipMalloc/hipFree.  Shapes whose scratch exceeds
 * 64 MiB return MOTY_HIP_EINVAL (the OLMoE layer fits up to T = 256 tokens:
 * about 27 MiB).  Every call on one GPU shares that array.  Sequential calls
 * are ordered on the device even across streams: a call on another stream
 * than the previous call's waits for that call's work (an event recorded
 * after each call; not under graph capture, where the caller orders
 * replays).  Calls that overlap in time on one GPU (several host threads at
 * once) race. */
int moty_hip_moe_topk_noalloc_dev(const MotyHipMoe *m, const float *x, int S, float *out, void *stream);
/* the cached layer with m's router/bias/outputs and x/out on the device;
 * synchronises `stream` once (the routing read-back) */
int moty_hip_moe_topk_cached_dev(const MotyHipMoe *m, MotyHipExpertCache *lc, void *ctx, int layer,
                                 MotyHipLoadExpertFn fn, const float *x, int S, float *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* MOTY_HW_HIP_H */
