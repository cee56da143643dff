/* ref_glue.c -- TEST INFRASTRUCTURE ONLY: flat C entry points over the
 * reference's own compiled sources (built by oracle/Makefile from
 * /root/reference/c into oracle/_ref/), so tests can call the real
 * reference kernels through ctypes.  Nothing here re-implements arithmetic
 * except ref_moe_olmoe, which replays the call sequence of
 * engines/olmoe.c:219-244 (a static function of an engine executable that
 * cannot be linked on its own) over the reference's public functions, built
 * with the reference's own compiler flags. */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include "hw/hw.h"
#include "nn/nn_quant.h"
#include "nn/nn_matmul.h"
#include "nn/nn_norm.h"
#include "nn/moe.h"
#include "io/gguf.h"

#define R_EXPORT __attribute__((visibility("default")))

/* IDOT4 is read once per process by nn/matmul.c:171 (and :76-77 for the
 * per-row int4 path); call before anything. */
R_EXPORT void ref_init(int idot4) {
    unsetenv("IDOT");
    if (idot4) setenv("IDOT4", "1", 1); else unsetenv("IDOT4");
    /* latch both knobs now, with one tiny call each */
    static float x[64], y[1], s[2] = {1.f, 1.f};
    static int8_t q[64]; static uint8_t q4[32];
    moty_matmul_q_s(y, x, q, s, 1, 64, 1);
    moty_matmul_i4_grouped_s(y, x, q4, s, 1, 64, 1, 32);
    moty_matmul_i4_s(y, x, q4, s, 1, 64, 1);  /* its own latch (nn/matmul.c:76-77) */
}
R_EXPORT const char *ref_tier(void) { return HW_IDOT_KERNEL "/" HW_F32_KERNEL; }
R_EXPORT float ref_qrow_i8(const float *x, int8_t *q, int n) { return moty_hw_qrow_i8(x, q, n); }
R_EXPORT int32_t ref_dot_i8i8(const int8_t *w, const int8_t *x, int n) { return moty_hw_dot_i8i8(w, x, n); }
R_EXPORT float ref_dot_f32(const float *a, const float *b, int n) { return moty_hw_dot_f32(a, b, n); }
R_EXPORT float ref_dot_i4g8p(const uint8_t *w4, const float *scl, const int8_t *x, const int32_t *xg, int I) {
    return moty_hw_dot_i4g8p(w4, scl, x, xg, I);
}
R_EXPORT void ref_quantize_rows(const float *w, int8_t *q, float *s, int O, int I, int bits) {
    moty_quantize_rows(w, q, s, O, I, bits);
}
R_EXPORT void ref_pack_int4_grouped(const float *w, uint8_t *q4, float *s, int O, int I, int gs) {
    moty_pack_int4_grouped(w, q4, s, O, I, gs);
}
R_EXPORT void ref_matmul_q_s(float *y, const float *x, const int8_t *q, const float *s, int S, int I, int O) {
    moty_matmul_q_s(y, x, q, s, S, I, O);
}
R_EXPORT void ref_matmul_i4_grouped_s(float *y, const float *x, const uint8_t *q4, const float *s,
                                      int S, int I, int O, int gs) {
    moty_matmul_i4_grouped_s(y, x, q4, s, S, I, O, gs);
}
R_EXPORT void ref_matmul(float *y, const float *x, const float *W, int S, int I, int O) {
    moty_matmul(y, x, W, S, I, O);
}
R_EXPORT void ref_silu_mul(float *g, const float *u, int64_t n) { moty_hw_silu_mul(g, u, n); }
R_EXPORT void ref_softmax(float *x, int n) { moty_softmax_row(x, n); }
R_EXPORT float ref_expf(float x) { return expf(x); }
R_EXPORT void ref_topk(const float *p, int E, int K, int *idx, float *w, int norm) {
    moty_moe_topk(p, E, K, idx, w, norm);
}

/* experts stacked: G,U [E][I][D], Dn [E][D][I], scales [E][I], [E][D] */
typedef struct { const int8_t *G, *U, *Dn; const float *GS, *US, *DS; } Stack;
static void stack_load(void *ctx, int layer, int eid, ExpertSlot *s, int inter, int hidden) {
    (void)layer;
    const Stack *st = ctx;
    int64_t n = (int64_t)inter * hidden;
    memcpy(s->g, st->G + eid * n, n); memcpy(s->u, st->U + eid * n, n);
    memcpy(s->d, st->Dn + eid * n, n);
    memcpy(s->gs, st->GS + (int64_t)eid * inter, sizeof(float) * inter);
    memcpy(s->us, st->US + (int64_t)eid * inter, sizeof(float) * inter);
    memcpy(s->ds, st->DS + (int64_t)eid * hidden, sizeof(float) * hidden);
}

/* moty_nn_moe_topk_batch (nn/moe.c:159-208), f32 router, no shared expert,
 * over an ExpertCache of `cap` slots (cap >= E: every expert resident) */
R_EXPORT void ref_moe_batch_cap(float *out, const float *x, int S, const float *Wr,
                                const int8_t *G, const float *GS, const int8_t *U, const float *US,
                                const int8_t *Dn, const float *DS, int E, int K, int I, int D, int cap) {
    Mat router; memset(&router, 0, sizeof router);
    router.fmt = WF_F32; router.f = (float *)Wr; router.O = E; router.I = D;
    ExpertCache ec; moty_expert_cache_init(&ec, cap, E);
    Stack st = { G, U, Dn, GS, US, DS };
    MotyMoeView v; memset(&v, 0, sizeof v);
    v.router = &router; v.ec = &ec; v.load_expert = stack_load; v.ectx = &st;
    v.E = E; v.K = K; v.I = I; v.D = D; v.ebits = 8;
    moty_nn_moe_topk_batch(&v, x, S, out);
    moty_expert_cache_free(&ec);
}
R_EXPORT void ref_moe_batch(float *out, const float *x, int S, const float *Wr,
                            const int8_t *G, const float *GS, const int8_t *U, const float *US,
                            const int8_t *Dn, const float *DS, int E, int K, int I, int D) {
    ref_moe_batch_cap(out, x, S, Wr, G, GS, U, US, Dn, DS, E, K, I, D, E);
}

/* moty_nn_moe_topk_d1 (nn/moe.c:33-153, S = 1): route_topk (always
 * normalised, nn/moe.c:27-30), then the serial top-k-order combine */
R_EXPORT void ref_moe_d1(float *out, const float *x, const float *Wr,
                         const int8_t *G, const float *GS, const int8_t *U, const float *US,
                         const int8_t *Dn, const float *DS, int E, int K, int I, int D) {
    Mat router; memset(&router, 0, sizeof router);
    router.fmt = WF_F32; router.f = (float *)Wr; router.O = E; router.I = D;
    ExpertCache ec; moty_expert_cache_init(&ec, E, E);
    Stack st = { G, U, Dn, GS, US, DS };
    Scratch scr; memset(&scr, 0, sizeof scr);
    MotyMoeView v; memset(&v, 0, sizeof v);
    v.router = &router; v.ec = &ec; v.load_expert = stack_load; v.ectx = &st;
    v.E = E; v.K = K; v.I = I; v.D = D; v.ebits = 8; v.scr = &scr;
    moty_nn_moe_topk_d1(&v, x, out);
    moty_scr_free(&scr);
    moty_expert_cache_free(&ec);
}

/* engines/olmoe.c:219-244 replayed over the reference's public functions */
R_EXPORT void ref_moe_olmoe(float *out, const float *x, int S, const float *Wr,
                            const int8_t *G, const float *GS, const int8_t *U, const float *US,
                            const int8_t *Dn, const float *DS, int E, int K, int I, int D,
                            int norm, int *idx_out) {
    float *logits = malloc(sizeof(float) * (size_t)S * E);
    moty_matmul(logits, x, Wr, S, D, E);
    memset(out, 0, sizeof(float) * (size_t)S * D);
    float *g = malloc(sizeof(float) * I), *u = malloc(sizeof(float) * I), *hh = malloc(sizeof(float) * D);
    int idx[64]; float w[64];
    int64_t n = (int64_t)I * D;
    for (int s = 0; s < S; s++) {
        float *pr = logits + (int64_t)s * E;
        moty_softmax_row(pr, E);
        moty_moe_topk(pr, E, K, idx, w, norm);
        if (idx_out) memcpy(idx_out + (int64_t)s * K, idx, sizeof(int) * K);
        const float *xs = x + (int64_t)s * D;
        for (int kk = 0; kk < K; kk++) {
            int e = idx[kk];
            moty_matmul_q(g, xs, G + e * n, GS + (int64_t)e * I, D, I);
            moty_matmul_q(u, xs, U + e * n, US + (int64_t)e * I, D, I);
            for (int i = 0; i < I; i++) { float gv = g[i]; g[i] = (gv / (1.f + expf(-gv))) * u[i]; }
            moty_matmul_q(hh, g, Dn + e * n, DS + (int64_t)e * D, I, D);
            float weight = w[kk];
            float *os = out + (int64_t)s * D;
            for (int d = 0; d < D; d++) os[d] += weight * hh[d];
        }
    }
    free(logits); free(g); free(u); free(hh);
}

/* GGUF block formats (io/gguf.h, header-only): the lossless Q4_0 -> int4
 * grouped repack and the block dequantisers behind st_read_f32. */
R_EXPORT void ref_gguf_repack_q4_0(const uint8_t *blocks, uint8_t *q4, float *qs, int64_t O, int64_t I) {
    gguf_repack_q4_0(blocks, q4, qs, O, I);
}
R_EXPORT void ref_gguf_dequant(int dtype, const void *raw, int64_t numel, float *out) {
    gguf_dequant(dtype, raw, numel, out);
}
