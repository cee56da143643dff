/* mat_apply_hip.c -- TEST HARNESS: the reference-side binding of
 * libmoty-hw-hip, compiled as a maintainer would add it to moty's C tree,
 * run against the reference's own kernels.
 *
 * Built by oracle/Makefile (target `harness`) against the reference headers
 * and objects under oracle/_ref (compiled from /root/reference/c) and
 * libmoty_hw_hip.so; run by tests/test_gpu_harness.py on the GPU box.
 *
 * What it binds, each with the reference's CPU function as the fallback:
 *   hip_mat_apply        moty_mat_apply (nn/mat.c:70-83): WF_I8, WF_I4G,
 *                        WF_I4, WF_F32, WF_Q4R4, WF_Q8R4 through the HIP
 *                        drop-ins, everything else (and any MOTY_HIP_EUNSUP)
 *                        through the reference's own dispatch
 *   HwBackend slots      matmul_i8 / matmul_i4 (hw/hw_backend.h:57-60)
 *   hip_moe_topk_d1      moty_nn_moe_topk_d1 (nn/moe.c:33-153)
 *   hip_moe_topk_batch   moty_nn_moe_topk_batch (nn/moe.c:159-208)
 * and checks every result bit for bit against the reference function on the
 * same inputs.  Prints one line per case and "ALL PASS" (exit 0) at the end.
 * IDOT4 comes from the environment, read once by both sides. */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "hw/hw_backend.h"
#include "moty_hw_hip.h"
#include "nn/moe.h"
#include "nn/nn_mat.h"
#include "nn/nn_matmul.h"
#include "nn/nn_quant.h"

/* ---- the binding (what goes into nn/mat.c under #ifdef MOTY_HIP) ---- */
static int g_hip_enabled = 1;

static void hip_mat_apply(float *y, const float *x, const Mat *w, int S) {
    if (g_hip_enabled && !omp_in_parallel()) {
        int rc = MOTY_HIP_EUNSUP;
        switch (w->fmt) {
        case WF_I8:   rc = moty_hip_matmul_q_s(y, x, w->q, w->qs, S, w->I, w->O); break;
        case WF_I4G:  rc = moty_hip_matmul_i4_grouped_s(y, x, w->q4, w->qs, S, w->I, w->O, w->gs); break;
        case WF_I4:   rc = moty_hip_matmul_i4_s(y, x, w->q4, w->qs, S, w->I, w->O); break;
        case WF_F32:  rc = moty_hip_matmul(y, x, w->f, S, w->I, w->O); break;
        case WF_Q4R4: rc = moty_hip_matmul_q4r4_s(y, x, w->q4, w->s16, S, w->I, w->O); break;
        case WF_Q8R4: rc = moty_hip_matmul_q8r4_s(y, x, (const int8_t *)w->q4, w->s16, S, w->I, w->O); break;
        default: break;
        }
        if (rc == MOTY_HIP_OK) return;
        if (rc != MOTY_HIP_EUNSUP) fprintf(stderr, "[HIP] %s; falling back to CPU\n", moty_hip_last_error());
    }
    moty_mat_apply(y, x, w, S);
}

/* the device backend's batch slots, as a runtime-dispatch build fills them */
static HwBackend hip_backend(void) {
    HwBackend b;
    memset(&b, 0, sizeof b);
    b.name = "gfx950";
    b.matmul_i8 = moty_hip_hw_matmul_i8;
    b.matmul_i4 = moty_hip_hw_matmul_i4;
    return b;
}

/* stacked experts: g,u [E][I][D], d [E][D][I] + row scales */
typedef struct { const int8_t *G, *U, *Dn; const float *GS, *US, *DS; } Stack;

static int hip_moe(const MotyMoeView *v, const Stack *st, const float *x, int S, float *out, int order) {
    MotyHipMoe m;
    memset(&m, 0, sizeof m);
    m.router = v->router->f;
    m.g = st->G; m.u = st->U; m.d = st->Dn;
    m.gs = st->GS; m.us = st->US; m.ds = st->DS;
    m.E = v->E; m.K = v->K; m.I = v->I; m.D = v->D;
    m.norm_topk = 1;          /* route_topk always normalises (nn/moe.c:27-30) */
    m.combine_order = order;  /* d1: serial top-k order (nn/moe.c:145-148); batch: ascending id */
    return moty_hip_moe_topk(&m, x, S, out);
}

static void hip_moe_topk_d1(const MotyMoeView *v, const Stack *st, const float *x, float *out) {
    if (g_hip_enabled && hip_moe(v, st, x, 1, out, MOTY_MOE_ORDER_TOPK) == MOTY_HIP_OK) return;
    moty_nn_moe_topk_d1(v, x, out);
}

static void hip_moe_topk_batch(const MotyMoeView *v, const Stack *st, const float *x, int S, float *out) {
    if (g_hip_enabled && hip_moe(v, st, x, S, out, MOTY_MOE_ORDER_EXPERT) == MOTY_HIP_OK) return;
    moty_nn_moe_topk_batch(v, x, S, out);
}

/* ---- the harness ---- */
static uint64_t h_rng = 0x4D4F5459u;
static float frand(void) { /* splitmix64 -> uniform (-1, 1) */
    uint64_t z = (h_rng += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)((double)(z >> 11) / 4503599627370496.0 - 1.0);
}
static float *rnd(int64_t n, float scale) {
    float *a = malloc(sizeof(float) * (size_t)n);
    for (int64_t i = 0; i < n; i++) a[i] = frand() * scale;
    return a;
}

static int g_fail = 0, g_cases = 0;
static void check(const char *what, const float *a, const float *b, int64_t n) {
    g_cases++;
    int64_t bad = 0;
    for (int64_t i = 0; i < n; i++) bad += memcmp(a + i, b + i, 4) != 0;
    printf("%-52s %s", what, bad ? "FAIL" : "ok");
    if (bad) printf(" (%lld of %lld differ)", (long long)bad, (long long)n);
    printf("\n");
    if (bad) g_fail++;
}

static Mat mat_of(int fmt, const float *w, int O, int I) {
    Mat m;
    memset(&m, 0, sizeof m);
    m.fmt = fmt; m.O = O; m.I = I;
    switch (fmt) {
    case WF_F32: m.f = (float *)w; break;
    case WF_I8:
        m.q = malloc((size_t)O * I); m.qs = malloc(sizeof(float) * O);
        moty_quantize_rows(w, m.q, m.qs, O, I, 8);
        break;
    case WF_I4:
        m.q4 = malloc((size_t)O * ((I + 1) / 2)); m.qs = malloc(sizeof(float) * O);
        moty_pack_int4(w, m.q4, m.qs, O, I);
        break;
    case WF_I4G:
        m.gs = 32;
        m.q4 = malloc((size_t)O * ((I + 1) / 2)); m.qs = malloc(sizeof(float) * O * ((I + 31) / 32));
        moty_pack_int4_grouped(w, m.q4, m.qs, O, I, 32);
        break;
    case WF_Q4R4: case WF_Q8R4: {
        const int gb = fmt == WF_Q8R4 ? 128 : 64, nb = I / 32, O4 = (O + 3) / 4;
        m.q4 = malloc((size_t)O4 * nb * gb); m.s16 = malloc(sizeof(uint16_t) * (size_t)O4 * nb * 4);
        for (int b = 0; b < O4; b++) {
            const int rows = O - 4 * b < 4 ? O - 4 * b : 4;
            if (fmt == WF_Q8R4)
                moty_pack_q8r4_block(w + (int64_t)b * 4 * I, rows, I, (int8_t *)m.q4 + (int64_t)b * nb * gb,
                                     m.s16 + (int64_t)b * nb * 4);
            else
                moty_pack_q4r4_block(w + (int64_t)b * 4 * I, rows, I, m.q4 + (int64_t)b * nb * gb,
                                     m.s16 + (int64_t)b * nb * 4);
        }
        break;
    }
    }
    return m;
}

static void mat_case(const char *name, int fmt, int S, int I, int O) {
    float *w = rnd((int64_t)O * I, 0.05f), *x = rnd((int64_t)S * I, 2.f);
    Mat m = mat_of(fmt, w, O, I);
    float *y = malloc(sizeof(float) * (size_t)S * O), *y2 = malloc(sizeof(float) * (size_t)S * O);
    hip_mat_apply(y, x, &m, S);
    moty_mat_apply(y2, x, &m, S);
    char what[96];
    snprintf(what, sizeof what, "mat_apply %-5s S=%d I=%d O=%d", name, S, I, O);
    check(what, y, y2, (int64_t)S * O);
    /* the Mat's weights are about to be freed: drop the device copies */
    moty_hip_weight_forget(m.q); moty_hip_weight_forget(m.qs); moty_hip_weight_forget(m.q4);
    moty_hip_weight_forget(m.s16); moty_hip_weight_forget(m.f);
    if (fmt != WF_F32) { free(m.q); free(m.qs); free(m.q4); free(m.s16); }
    free(w); free(x); free(y); free(y2);
}

static void slot_case(int i4, int S, int I, int O) {
    HwBackend b = hip_backend();
    float *w = rnd((int64_t)O * I, 0.05f), *x = rnd((int64_t)S * I, 2.f);
    Mat m = mat_of(i4 ? WF_I4 : WF_I8, w, O, I);
    float *y = malloc(sizeof(float) * (size_t)S * O), *y2 = malloc(sizeof(float) * (size_t)S * O);
    if (i4) { b.matmul_i4(y, x, m.q4, m.qs, S, I, O); moty_matmul_i4_s(y2, x, m.q4, m.qs, S, I, O); }
    else { b.matmul_i8(y, x, m.q, m.qs, S, I, O); moty_matmul_q_s(y2, x, m.q, m.qs, S, I, O); }
    char what[96];
    snprintf(what, sizeof what, "HwBackend.matmul_%s S=%d I=%d O=%d", i4 ? "i4" : "i8", S, I, O);
    check(what, y, y2, (int64_t)S * O);
    moty_hip_weight_forget(m.q); moty_hip_weight_forget(m.qs); moty_hip_weight_forget(m.q4);
    free(m.q); free(m.qs); free(m.q4); free(w); free(x); free(y); free(y2);
}

static void stack_load(void *ctx, int layer, int eid, ExpertSlot *s, int inter, int hidden) {
    (void)layer;
    const Stack *st = ctx;
    const int64_t n = (int64_t)inter * hidden;
    memcpy(s->g, st->G + eid * n, n); memcpy(s->u, st->U + eid * n, n); memcpy(s->d, st->Dn + eid * n, n);
    memcpy(s->gs, st->GS + (int64_t)eid * inter, sizeof(float) * inter);
    memcpy(s->us, st->US + (int64_t)eid * inter, sizeof(float) * inter);
    memcpy(s->ds, st->DS + (int64_t)eid * hidden, sizeof(float) * hidden);
}

static void moe_case(int E, int K, int I, int D, int S) {
    const int64_t n = (int64_t)E * I * D;
    float *wg = rnd(n, 0.05f), *wu = rnd(n, 0.05f), *wd = rnd(n, 0.05f), *wr = rnd((int64_t)E * D, 0.05f);
    int8_t *G = malloc(n), *U = malloc(n), *Dn = malloc(n);
    float *GS = malloc(sizeof(float) * E * I), *US = malloc(sizeof(float) * E * I), *DS = malloc(sizeof(float) * E * D);
    moty_quantize_rows(wg, G, GS, E * I, D, 8);
    moty_quantize_rows(wu, U, US, E * I, D, 8);
    moty_quantize_rows(wd, Dn, DS, E * D, I, 8);
    Stack st = {G, U, Dn, GS, US, DS};
    Mat router;
    memset(&router, 0, sizeof router);
    router.fmt = WF_F32; router.f = wr; router.O = E; router.I = D;
    ExpertCache ec;
    moty_expert_cache_init(&ec, E, E);
    Scratch scr;
    memset(&scr, 0, sizeof scr);
    MotyMoeView v;
    memset(&v, 0, sizeof v);
    v.router = &router; v.ec = &ec; v.load_expert = stack_load; v.ectx = &st;
    v.E = E; v.K = K; v.I = I; v.D = D; v.ebits = 8; v.scr = &scr;
    float *x = rnd((int64_t)S * D, 2.f);
    float *y = malloc(sizeof(float) * (size_t)S * D), *y2 = malloc(sizeof(float) * (size_t)S * D);
    char what[96];
    hip_moe_topk_d1(&v, &st, x, y);
    moty_nn_moe_topk_d1(&v, x, y2);
    snprintf(what, sizeof what, "moe_topk_d1 E=%d K=%d I=%d D=%d", E, K, I, D);
    check(what, y, y2, D);
    hip_moe_topk_batch(&v, &st, x, S, y);
    moty_nn_moe_topk_batch(&v, x, S, y2);
    snprintf(what, sizeof what, "moe_topk_batch E=%d K=%d I=%d D=%d S=%d", E, K, I, D, S);
    check(what, y, y2, (int64_t)S * D);
    const void *held[] = {G, U, Dn, GS, US, DS, wr};
    for (int i = 0; i < 7; i++) moty_hip_weight_forget(held[i]);
    moty_scr_free(&scr);
    moty_expert_cache_free(&ec);
    free(wg); free(wu); free(wd); free(wr); free(G); free(U); free(Dn); free(GS); free(US); free(DS);
    free(x); free(y); free(y2);
}

int main(void) {
    const char *e = getenv("IDOT4");
    printf("mat_apply_hip: IDOT4=%s, HIP tier %s, reference tier %s/%s\n", e ? e : "(unset)",
           moty_hip_kernel_tier(), HW_IDOT_KERNEL, HW_F32_KERNEL);
    static const int fmts[] = {WF_I8, WF_I4G, WF_I4, WF_F32, WF_Q4R4, WF_Q8R4};
    static const char *names[] = {"I8", "I4G", "I4", "F32", "Q4R4", "Q8R4"};
    static const int shapes[][3] = {{1, 1024, 3072}, {4, 2048, 512}, {33, 1024, 300}, {512, 1024, 1024}, {7, 96, 40}};
    for (int f = 0; f < 6; f++)
        for (int s = 0; s < 5; s++) mat_case(names[f], fmts[f], shapes[s][0], shapes[s][1], shapes[s][2]);
    /* shapes the backend does not serve fall back to the reference */
    mat_case("I8", WF_I8, 3, 40, 17);
    mat_case("I4", WF_I4, 3, 40, 17);
    mat_case("I4G", WF_I4G, 5, 33, 9);
    for (int i4 = 0; i4 < 2; i4++) {
        slot_case(i4, 1, 1024, 256);
        slot_case(i4, 9, 512, 100);
    }
    moe_case(16, 4, 128, 256, 24);
    moe_case(64, 8, 1024, 2048, 40);
    printf("%d cases, %d failed\n%s\n", g_cases, g_fail, g_fail ? "FAILED" : "ALL PASS");
    moty_hip_shutdown();
    return g_fail ? 1 : 0;
}
