/* moty_oracle.c -- CPU restatement of moty's quantized-matmul + MoE path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP library in
 * moty_amd/: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product path never calls into it.
 *
 * Every function restates one reference function (cited as file:line relative
 * to the reference's c/ directory).  Floating-point steps are written out in
 * the exact order the reference's x86-64 AVX512-VNNI build evaluates them
 * (gcc -O2, whose default -ffp-contract=fast turns `a += b*c` into an FMA);
 * this file is compiled with -ffp-contract=off, so every FMA below is explicit.
 *
 * Pinning (what checks each function beyond retyping it):
 *   o_qrow_i8, o_quantize_rows, o_pack_int4_grouped, o_pack_int4 -> compiled reference
 *       (oracle/_ref), reconstruction bound |x - s*q| <= s/2, golden fixtures
 *   o_dot_i8i8, o_matmul_q_s   -> brute-force int64 sums, _ref, fixtures,
 *       batch invariance (S rows == S single calls)
 *   o_dot_i4g8p, o_matmul_i4g_idot4, o_matmul_i4g_f32 -> _ref, and a double
 *       dequant reference within the reference's own tolerance
 *   o_matmul_i4_idot4 (per-row int4) -> _ref, brute-force int64 sums
 *   o_matmul_i4_f32 -> _ref bit-exact at I % 16 == 0, double dequant sum
 *   o_dot_f32 (AVX512 lane order), o_matmul_f32  -> _ref bit-exact, double sum
 *   o_expf     -> exhaustive over all 2^32 inputs against libm expf
 *   o_softmax, o_silu_mul, o_topk -> _ref, naive greedy top-k
 *   o_moe_batch / o_moe_olmoe -> _ref (moty_nn_moe_topk_batch and the
 *       olmoe call sequence), plus the permutation property of the grouping
 *   o_f16_to_f32 / o_f32_to_f16 -> every half round-trips, numpy's IEEE
 *       binary16 conversions, _ref
 *   o_quant_g32, o_pack_q4r4, o_pack_q8r4, o_matmul_q4r4, o_matmul_q8r4 ->
 *       _ref bit-exact (moty_hw_quant_g32, moty_pack_q{4,8}r4_block,
 *       moty_matmul_q{4,8}r4_s), the no-clip packing bounds and the double
 *       dequantized reference of c/tests/q4r4_tests.c
 *   o_gguf_repack_q4_0, o_gguf_dequant -> _ref bit-exact (io/gguf.h built
 *       from the reference tree), the hand-built known-answer blocks of
 *       c/tests/headers_tests.c:131-211 and qwen_tests.c:799-847, and
 *       repack/dequant agreement (dequantizing the repacked int4 equals
 *       the Q4_0 dequant)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define O_EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ */
/* a1: per-row symmetric int8 activation quantization.                  */
/* hw/hw_quant.h:9-16                                                   */
O_EXPORT float o_qrow_i8(const float *x, int8_t *q, int n) {
    float amax = 0.f;
    for (int i = 0; i < n; i++) { float a = fabsf(x[i]); if (a > amax) amax = a; }
    float s = amax / 127.f;
    if (s < 1e-12f) s = 1e-12f;
    float inv = 1.f / s;
    for (int i = 0; i < n; i++) q[i] = (int8_t)lrintf(x[i] * inv);
    return s;
}

/* a2: int8 x int8 -> int32 (hw/hw_scalar.h:8-12; the VNNI kernel of
 * hw/hw_avx512.h:24-54 is exact integer arithmetic, so any order agrees). */
O_EXPORT int32_t o_dot_i8i8(const int8_t *w, const int8_t *x, int n) {
    int64_t s = 0;
    for (int i = 0; i < n; i++) s += (int64_t)w[i] * x[i];
    return (int32_t)s;
}

/* a4: weight quantization, per row, division by s (not *inv).
 * nn/quant.c:12-33 */
O_EXPORT void o_quantize_rows(const float *w, int8_t *q, float *scale, int O, int I, int bits) {
    int qmax = (1 << (bits - 1)) - 1;
    for (int o = 0; o < O; o++) {
        const float *wr = w + (int64_t)o * I;
        float amax = 0.f;
        for (int i = 0; i < I; i++) { float a = fabsf(wr[i]); if (a > amax) amax = a; }
        float s = amax / (float)qmax;
        if (s < 1e-8f) s = 1e-8f;
        scale[o] = s;
        for (int i = 0; i < I; i++) {
            int v = (int)lrintf(wr[i] / s);
            if (v > qmax) v = qmax;
            if (v < -qmax - 1) v = -qmax - 1;
            q[(int64_t)o * I + i] = (int8_t)v;
        }
    }
}

/* a6: grouped int4 packing, f32 scale amax/7 per group, nibble = v+8,
 * even element in the low nibble.  nn/quant.c:57-83 (gs % 16 == 0 is
 * checked by the caller, quant.c:80). */
/* Per-row int4 weights (WF_I4): nn/quant.c:34-55 (pack_int4_part, bits 4):
 * s = amax/7.f clamped at 1e-8, v = clip(lrintf(w/s), -8, 7), byte =
 * (v0+8) | (v1+8) << 4 with the even element in the low nibble. */
O_EXPORT void o_pack_int4(const float *w, uint8_t *q4, float *scale, int O, int I) {
    int rb = (I + 1) / 2;
    for (int o = 0; o < O; o++) {
        const float *wr = w + (int64_t)o * I;
        float amax = 0.f;
        for (int i = 0; i < I; i++) { float a = fabsf(wr[i]); if (a > amax) amax = a; }
        float s = amax / 7.f;
        if (s < 1e-8f) s = 1e-8f;
        scale[o] = s;
        uint8_t *qr = q4 + (int64_t)o * rb;
        for (int i = 0; i < I; i += 2) {
            int v0 = (int)lrintf(wr[i] / s);
            if (v0 > 7) v0 = 7;
            if (v0 < -8) v0 = -8;
            int v1 = 0;
            if (i + 1 < I) {
                v1 = (int)lrintf(wr[i + 1] / s);
                if (v1 > 7) v1 = 7;
                if (v1 < -8) v1 = -8;
            }
            qr[i >> 1] = (uint8_t)((v0 + 8) | ((v1 + 8) << 4));
        }
    }
}

/* moty_matmul_i4_s (nn/matmul.c:75-100), IDOT4 = 1 and I <= 16384: x
 * quantized per row (qrow_i8), dot_i4i8 (hw/hw_scalar.h:14-22: sum of
 * (n-8)*x, exact), y = (scale[o]*sx[s]) * (float)dot. */
O_EXPORT void o_matmul_i4_idot4(float *y, const float *x, const uint8_t *q4, const float *scale,
                                int S, int I, int O) {
    int8_t *xi = malloc((size_t)S * I);
    float *sx = malloc(sizeof(float) * (size_t)S);
    for (int s = 0; s < S; s++) sx[s] = o_qrow_i8(x + (int64_t)s * I, xi + (int64_t)s * I, I);
    int rb = (I + 1) / 2;
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const uint8_t *w4 = q4 + (int64_t)o * rb;
        for (int s = 0; s < S; s++) {
            const int8_t *xs = xi + (int64_t)s * I;
            int64_t d = 0;
            for (int i = 0; i < I; i++) {
                int n = (i & 1) ? (w4[i >> 1] >> 4) : (w4[i >> 1] & 15);
                d += (int64_t)(n - 8) * xs[i];
            }
            y[(int64_t)s * O + o] = (scale[o] * sx[s]) * (float)(int32_t)d;
        }
    }
    free(xi); free(sx);
}

/* moty_matmul_i4_s, exact f32 path (i4_f32_rows, nn/matmul.c:102-145) as
 * the x86-64 AVX2 branch evaluates it for I % 16 == 0: eight accumulator
 * lanes, lane j takes elements i+j (first FMA) and i+8+j (second) of each
 * 16-element step, acc = fma(x, (float)(n-8), acc); then simd_hsum256_f32
 * (hw/hw_avx2.h:16-20): (l0+l4, l1+l5, l2+l6, l3+l7), then (a0+a2, a1+a3),
 * then their sum; y = a * scale[o]. */
O_EXPORT void o_matmul_i4_f32(float *y, const float *x, const uint8_t *q4, const float *scale,
                              int S, int I, int O) {
    int rb = (I + 1) / 2;
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const uint8_t *w = q4 + (int64_t)o * rb;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int i = 0; i + 16 <= I; i += 16) {
                for (int j = 0; j < 8; j++) {
                    int e = i + j, n = (e & 1) ? (w[e >> 1] >> 4) : (w[e >> 1] & 15);
                    acc[j] = fmaf(xs[e], (float)(n - 8), acc[j]);
                }
                for (int j = 0; j < 8; j++) {
                    int e = i + 8 + j, n = (e & 1) ? (w[e >> 1] >> 4) : (w[e >> 1] & 15);
                    acc[j] = fmaf(xs[e], (float)(n - 8), acc[j]);
                }
            }
            float a0 = acc[0] + acc[4], a1 = acc[1] + acc[5], a2 = acc[2] + acc[6], a3 = acc[3] + acc[7];
            float b0 = a0 + a2, b1 = a1 + a3;
            y[(int64_t)s * O + o] = (b0 + b1) * scale[o];
        }
    }
}

O_EXPORT void o_pack_int4_grouped(const float *w, uint8_t *q4, float *scale, int O, int I, int gs) {
    int rb = (I + 1) / 2, ng = (I + gs - 1) / gs;
    for (int o = 0; o < O; o++) {
        const float *wr = w + (int64_t)o * I;
        uint8_t *qr = q4 + (int64_t)o * rb;
        float *scl = scale + (int64_t)o * ng;
        for (int g = 0; g * gs < I; g++) {
            int base = g * gs, glen = gs;
            if (base + glen > I) glen = I - base;
            float amax = 0.f;
            for (int i = base; i < base + glen; i++) { float a = fabsf(wr[i]); if (a > amax) amax = a; }
            float s = amax / 7.f;
            if (s < 1e-8f) s = 1e-8f;
            scl[g] = s;
            for (int i = base; i < base + glen; i += 2) {
                int v0 = (int)lrintf(wr[i] / s);
                if (v0 > 7) v0 = 7;
                if (v0 < -8) v0 = -8;
                int v1 = 0;
                if (i + 1 < base + glen) {
                    v1 = (int)lrintf(wr[i + 1] / s);
                    if (v1 > 7) v1 = 7;
                    if (v1 < -8) v1 = -8;
                }
                qr[i >> 1] = (uint8_t)((v0 + 8) | ((v1 + 8) << 4));
            }
        }
    }
}

/* a3: Q8 GEMV/GEMM, IDOT path (default).  nn/matmul.c:51-66 + :29-36.
 * y[s*O+o] = (scale[o] * sx[s]) * (float)dot, two plain multiplies. */
O_EXPORT void o_matmul_q_s(float *y, const float *x, const int8_t *q, const float *scale,
                           int S, int I, int O) {
    int8_t *xi = malloc((size_t)S * I + 1);
    float *sx = malloc(sizeof(float) * (size_t)(S + 1));
    for (int s = 0; s < S; s++) sx[s] = o_qrow_i8(x + (int64_t)s * I, xi + (int64_t)s * I, I);
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++)
        for (int s = 0; s < S; s++) {
            float a = scale[o] * sx[s];
            y[(int64_t)s * O + o] = a * (float)o_dot_i8i8(q + (int64_t)o * I, xi + (int64_t)s * I, I);
        }
    free(xi); free(sx);
}

/* Q8 GEMM on activations already quantized (same arithmetic as above). */
O_EXPORT void o_matmul_q8_preq(float *y, const int8_t *xi, const float *sx, const int8_t *q,
                               const float *scale, int32_t *acc, int S, int I, int O) {
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++)
        for (int s = 0; s < S; s++) {
            int32_t d = o_dot_i8i8(q + (int64_t)o * I, xi + (int64_t)s * I, I);
            if (acc) acc[(int64_t)s * O + o] = d;
            if (y) y[(int64_t)s * O + o] = (scale[o] * sx[s]) * (float)d;
        }
}

/* a7: grouped int4 dot with int8 activations (IDOT4).  hw/hw_avx512.h:155-176.
 * Per group: d = sum(n*x) over unsigned nibbles, then
 * acc = fma(scl[g], (float)(d - 8*xgsum[g]), acc), groups in ascending order
 * (two statements per 64-chunk; gcc contracts each into one FMA). */
O_EXPORT float o_dot_i4g8p(const uint8_t *w4, const float *scl, const int8_t *x,
                           const int32_t *xgsum, int I) {
    float acc = 0.f;
    for (int i = 0; i + 64 <= I; i += 64) {
        for (int h = 0; h < 2; h++) {
            int g = (i >> 5) + h;
            int32_t d = 0;
            for (int j = 0; j < 32; j++) {
                int e = g * 32 + j;
                uint8_t b = w4[e >> 1];
                int n = (e & 1) ? (b >> 4) : (b & 0xF);
                d += n * x[e];
            }
            acc = fmaf(scl[g], (float)(d - 8 * xgsum[g]), acc);
        }
    }
    return acc;
}

/* a8, IDOT4=1 branch: nn/matmul.c:164-197 + i4g_vnni_rows :148-160.
 * Requires gs == 32, I % 64 == 0, I <= 16384 (the caller checks). */
O_EXPORT void o_matmul_i4g_idot4(float *y, const float *x, const uint8_t *q4, const float *scale,
                                 int S, int I, int O) {
    int ng = I / 32, rb = (I + 1) / 2;
    int8_t *xi = malloc((size_t)S * I + 1);
    int32_t *xg = malloc(sizeof(int32_t) * ((size_t)S * ng + 1));
    float *sx = malloc(sizeof(float) * (size_t)(S + 1));
    for (int s = 0; s < S; s++) {
        sx[s] = o_qrow_i8(x + (int64_t)s * I, xi + (int64_t)s * I, I);
        for (int g = 0; g < ng; g++) {
            int32_t a = 0;
            for (int j = 0; j < 32; j++) a += xi[(int64_t)s * I + g * 32 + j];
            xg[(int64_t)s * ng + g] = a;
        }
    }
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++)
        for (int s = 0; s < S; s++)
            y[(int64_t)s * O + o] = sx[s] * o_dot_i4g8p(q4 + (int64_t)o * rb, scale + (int64_t)o * ng,
                                                        xi + (int64_t)s * I, xg + (int64_t)s * ng, I);
    free(xi); free(xg); free(sx);
}

/* The 16-lane horizontal sum of gcc's _mm512_reduce_add_ps: halves 256/128,
 * then lanes {2,3} onto {0,1}, then lane 1 onto lane 0. */
static float hsum16(const float *v) {
    float a[8], b[4];
    for (int j = 0; j < 8; j++) a[j] = v[j + 8] + v[j];
    for (int j = 0; j < 4; j++) b[j] = a[j + 4] + a[j];
    float c0 = b[0] + b[2], c1 = b[1] + b[3];
    return c0 + c1;
}

/* a8, default branch (IDOT4 unset): exact f32 activations times dequantized
 * s*(n-8).  nn/matmul.c:199-253, AVX512 gs == 32 block (:219-235): per group
 * s1 = x[16:32]*w[16:32] (plain product), s0 + s1 contracted by gcc into
 * fma(x[0:16], w[0:16], s1), then a = fma(reduce(.), sc, a).  Restated for gs == 32, I % 32 == 0 only. */
O_EXPORT void o_matmul_i4g_f32(float *y, const float *x, const uint8_t *q4, const float *scale,
                               int S, int I, int O) {
    int ng = I / 32, rb = (I + 1) / 2;
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++) {
        const uint8_t *w = q4 + (int64_t)o * rb;
        const float *scl = scale + (int64_t)o * ng;
        for (int s = 0; s < S; s++) {
            const float *xs = x + (int64_t)s * I;
            float a = 0.f;
            for (int g = 0; g < ng; g++) {
                float t[16];
                for (int j = 0; j < 16; j++) {
                    int e0 = g * 32 + j, e1 = g * 32 + 16 + j;
                    int n0 = (e0 & 1) ? (w[e0 >> 1] >> 4) : (w[e0 >> 1] & 0xF);
                    int n1 = (e1 & 1) ? (w[e1 >> 1] >> 4) : (w[e1 >> 1] & 0xF);
                    float p1 = xs[e1] * (float)(n1 - 8);
                    t[j] = fmaf(xs[e0], (float)(n0 - 8), p1);
                }
                a = fmaf(hsum16(t), scl[g], a);
            }
            y[(int64_t)s * O + o] = a;
        }
    }
}

/* a10: f32 dot, AVX512 order.  hw/hw_avx512.h:231-243: two 16-lane FMA
 * chains over 32-element steps, a 16-element step on chain 0, then
 * reduce(s0 + s1), then a scalar FMA tail. */
O_EXPORT float o_dot_f32(const float *a, const float *b, int n) {
    float s0[16], s1[16];
    for (int l = 0; l < 16; l++) { s0[l] = 0.f; s1[l] = 0.f; }
    int i = 0;
    for (; i + 32 <= n; i += 32)
        for (int l = 0; l < 16; l++) {
            s0[l] = fmaf(a[i + l], b[i + l], s0[l]);
            s1[l] = fmaf(a[i + 16 + l], b[i + 16 + l], s1[l]);
        }
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 16; l++) s0[l] = fmaf(a[i + l], b[i + l], s0[l]);
    float t[16];
    for (int l = 0; l < 16; l++) t[l] = s0[l] + s1[l];
    float s = hsum16(t);
    for (; i < n; i++) s = fmaf(a[i], b[i], s);
    return s;
}

/* moty_matmul (nn/matmul.c:15-27): y[s*O+o] = dot_f32(x[s], W[o], I). */
O_EXPORT void o_matmul_f32(float *y, const float *x, const float *W, int S, int I, int O) {
    #pragma omp parallel for schedule(static)
    for (int o = 0; o < O; o++)
        for (int s = 0; s < S; s++)
            y[(int64_t)s * O + o] = o_dot_f32(x + (int64_t)s * I, W + (int64_t)o * I, I);
}

/* ------------------------------------------------------------------ */
/* expf.  The reference calls glibc 2.35 expf (hw/hw_ops.h:20,24).  glibc's
 * expf is the table-driven method of ARM's optimized-routines (Szabolcs
 * Nagy): k = round(x*N/ln2), N = 32, r = x*N/ln2 - k,
 * exp(x) = 2^(k/N) * (1 + C2 r + C1 r^2 + C0 r^3) evaluated in double, with
 * the x86-64 FMA build contracting every multiply-add.  o_expf restates it;
 * the HIP library uses the same steps.  The 2^(i/32) table is built from
 * exp2l; the whole function is checked against libm expf on every float. */
static uint64_t g_t2[32];
static int g_t2_ready;
static const double EXP_N = 32.0;
static const double EXP_C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
static const double EXP_C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
static const double EXP_C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
static const double EXP_INVLN2N = 0x1.71547652b82fep+0 * 32.0;
static const double EXP_SHIFT = 0x1.8p+52;

static void t2_init(void) {
    if (g_t2_ready) return;
    for (int i = 0; i < 32; i++) {
        double v = (double)exp2l((long double)i / 32.0L);
        uint64_t u; memcpy(&u, &v, 8);
        g_t2[i] = u - ((uint64_t)i << 47);
    }
    g_t2_ready = 1;
}

O_EXPORT void o_expf_table(uint64_t *out32) { t2_init(); memcpy(out32, g_t2, sizeof g_t2); }

O_EXPORT float o_expf(float x) {
    t2_init();
    uint32_t ux; memcpy(&ux, &x, 4);
    uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                       /* |x| >= 88 or nan/inf */
        if (ux == 0xff800000u) return 0.f;       /* -inf */
        if (abstop >= 0x7f8) return x + x;       /* inf or nan */
        if (x > 0x1.62e42ep6f) return INFINITY;  /* overflow */
        if (x < -0x1.9fe368p6f) return 0.f;      /* underflow */
    }
    (void)EXP_N;
    double xd = (double)x;
    double kd = fma(EXP_INVLN2N, xd, EXP_SHIFT);
    uint64_t ki; memcpy(&ki, &kd, 8);
    kd -= EXP_SHIFT;
    double r = fma(EXP_INVLN2N, xd, -kd);
    uint64_t t = g_t2[ki % 32] + (ki << 47);
    double s; memcpy(&s, &t, 8);
    double z = fma(EXP_C0, r, EXP_C1);
    double r2 = r * r;
    double y = fma(EXP_C2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return (float)y;
}

/* Exhaustive comparison of o_expf with libm expf over [lo, hi) of the 32-bit
 * patterns; returns the number of mismatching non-NaN inputs. */
O_EXPORT int64_t o_expf_check_range(uint64_t lo, uint64_t hi) {
    int64_t bad = 0;
    t2_init();
    #pragma omp parallel for reduction(+:bad) schedule(dynamic, 65536)
    for (int64_t u = (int64_t)lo; u < (int64_t)hi; u++) {
        uint32_t b = (uint32_t)u; float x; memcpy(&x, &b, 4);
        if (x != x) continue;
        float p = expf(x), q = o_expf(x);
        uint32_t bp, bq; memcpy(&bp, &p, 4); memcpy(&bq, &q, 4);
        if (bp != bq) bad++;
    }
    return bad;
}

/* a9: g = (g / (1 + expf(-g))) * u.  hw/hw_ops.h:19-21 */
O_EXPORT void o_silu_mul(float *g, const float *u, int64_t n) {
    for (int64_t i = 0; i < n; i++) { float v = g[i]; g[i] = (v / (1.f + expf(-v))) * u[i]; }
}

/* a11: max-subtracted softmax with a sequential sum.  hw/hw_ops.h:22-26 */
O_EXPORT void o_softmax(float *x, int n) {
    float m = -1e30f;
    for (int i = 0; i < n; i++) if (x[i] > m) m = x[i];
    float s = 0.f;
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - m); s += x[i]; }
    for (int i = 0; i < n; i++) x[i] /= s;
}

/* a12: greedy top-K, strict '>', lowest index wins ties, optional
 * normalisation by the sequential sum.  runtime/moecache.c:97-111 */
O_EXPORT void o_topk(const float *p, int E, int K, int *idx, float *w, int norm) {
    for (int kk = 0; kk < K; kk++) {
        int best = -1; float bv = -1e30f;
        for (int e = 0; e < E; e++) {
            int taken = 0;
            for (int j = 0; j < kk; j++) if (idx[j] == e) { taken = 1; break; }
            if (!taken && p[e] > bv) { bv = p[e]; best = e; }
        }
        idx[kk] = best; w[kk] = bv;
    }
    if (norm) {
        float sm = 0.f;
        for (int kk = 0; kk < K; kk++) sm += w[kk];
        if (sm > 0) for (int kk = 0; kk < K; kk++) w[kk] /= sm;
    }
}

/* Router: logits = x . Wr^T (f32, a10), optional per-expert logit bias
 * (moty_moe_route_bias, runtime/moecache.c:91-95 adds to the chosen
 * logits), softmax (a11), top-K (a12). */
O_EXPORT void o_route(const float *x, const float *Wr, const float *bias, int S, int D, int E,
                      int K, int norm, int *idx, float *w, float *probs_out) {
    float *lg = malloc(sizeof(float) * (size_t)S * E);
    o_matmul_f32(lg, x, Wr, S, D, E);
    for (int s = 0; s < S; s++) {
        float *p = lg + (int64_t)s * E;
        if (bias) for (int e = 0; e < E; e++) p[e] += bias[e];
        o_softmax(p, E);
        o_topk(p, E, K, idx + (int64_t)s * K, w + (int64_t)s * K, norm);
    }
    if (probs_out) memcpy(probs_out, lg, sizeof(float) * (size_t)S * E);
    free(lg);
}

/* One expert over one token row: the per-token body of engines/olmoe.c:
 * 230-240 and of nn/moe.c:192-198 (the two agree per row, matmul_q_s is
 * batch-invariant).  Expert weights are stacked [E][I][D] / [E][D][I]. */
static void expert_row(float *hh, const float *xs, const int8_t *G, const float *GS,
                       const int8_t *U, const float *US, const int8_t *Dn, const float *DS,
                       int eid, int I, int D, float *g, float *u) {
    const int8_t *ge = G + (int64_t)eid * I * D, *ue = U + (int64_t)eid * I * D;
    const int8_t *de = Dn + (int64_t)eid * D * I;
    o_matmul_q_s(g, xs, ge, GS + (int64_t)eid * I, 1, D, I);
    o_matmul_q_s(u, xs, ue, US + (int64_t)eid * I, 1, D, I);
    o_silu_mul(g, u, I);
    o_matmul_q_s(hh, g, de, DS + (int64_t)eid * D, 1, I, D);
}

/* a13, olmoe engine order: engines/olmoe.c:219-244.  Per token, experts in
 * top-k order, out[d] = fma(w[kk], hh[d], out[d]). */
O_EXPORT void o_moe_olmoe(float *out, const float *x, int S, const float *Wr, const float *bias,
                          const int8_t *G, const float *GS, const int8_t *U, const float *US,
                          const int8_t *Dn, const float *DS, int E, int K, int I, int D, int norm,
                          int *idx_out, float *w_out) {
    int *idx = malloc(sizeof(int) * (size_t)S * K);
    float *w = malloc(sizeof(float) * (size_t)S * K);
    o_route(x, Wr, bias, S, D, E, K, norm, idx, w, NULL);
    memset(out, 0, sizeof(float) * (size_t)S * D);
    #pragma omp parallel
    {
        float *g = malloc(sizeof(float) * I), *u = malloc(sizeof(float) * I);
        float *hh = malloc(sizeof(float) * D);
        #pragma omp for schedule(dynamic, 1)
        for (int s = 0; s < S; s++) {
            for (int kk = 0; kk < K; kk++) {
                expert_row(hh, x + (int64_t)s * D, G, GS, U, US, Dn, DS, idx[s * K + kk], I, D, g, u);
                float *os = out + (int64_t)s * D;
                for (int d = 0; d < D; d++) os[d] = fmaf(w[s * K + kk], hh[d], os[d]);
            }
        }
        free(g); free(u); free(hh);
    }
    if (idx_out) memcpy(idx_out, idx, sizeof(int) * (size_t)S * K);
    if (w_out) memcpy(w_out, w, sizeof(float) * (size_t)S * K);
    free(idx); free(w);
}

/* a13, shared batch order: nn/moe.c:159-205 (moe_batch_core, no shared
 * expert), routing always normalised (nn/moe.c:27-30).  Experts ascending;
 * each token's contribution from expert eid is added when eid is visited,
 * so per token the combine runs in ascending expert id. */
O_EXPORT void o_moe_batch(float *out, const float *x, int S, const float *Wr, const float *bias,
                          const int8_t *G, const float *GS, const int8_t *U, const float *US,
                          const int8_t *Dn, const float *DS, int E, int K, int I, int D,
                          int *idx_out, float *w_out) {
    int *idx = malloc(sizeof(int) * (size_t)S * K);
    float *w = malloc(sizeof(float) * (size_t)S * K);
    o_route(x, Wr, bias, S, D, E, K, 1, idx, w, NULL);
    memset(out, 0, sizeof(float) * (size_t)S * D);
    #pragma omp parallel
    {
        float *g = malloc(sizeof(float) * I), *u = malloc(sizeof(float) * I);
        float *hh = malloc(sizeof(float) * D);
        int *ord = malloc(sizeof(int) * K);
        #pragma omp for schedule(dynamic, 1)
        for (int s = 0; s < S; s++) {
            /* visit this token's experts in ascending id */
            for (int kk = 0; kk < K; kk++) ord[kk] = kk;
            for (int a = 1; a < K; a++)
                for (int b = a; b > 0 && idx[s * K + ord[b]] < idx[s * K + ord[b - 1]]; b--) {
                    int t = ord[b]; ord[b] = ord[b - 1]; ord[b - 1] = t;
                }
            for (int j = 0; j < K; j++) {
                int kk = ord[j];
                expert_row(hh, x + (int64_t)s * D, G, GS, U, US, Dn, DS, idx[s * K + kk], I, D, g, u);
                float *os = out + (int64_t)s * D;
                for (int d = 0; d < D; d++) os[d] = fmaf(w[s * K + kk], hh[d], os[d]);
            }
        }
        free(g); free(u); free(hh); free(ord);
    }
    if (idx_out) memcpy(idx_out, idx, sizeof(int) * (size_t)S * K);
    if (w_out) memcpy(w_out, w, sizeof(float) * (size_t)S * K);
    free(idx); free(w);
}

/* Dense SwiGLU FFN over Q8 weights: nn/ffn.c:26-55 / engines/qwen.c:659-679
 * (gate, up, silu*up, down through matmul_q_s). */
O_EXPORT void o_dense_ffn_q8(float *out, const float *x, int S, const int8_t *G, const float *GS,
                             const int8_t *U, const float *US, const int8_t *Dn, const float *DS,
                             int D, int I) {
    float *g = malloc(sizeof(float) * (size_t)S * I), *u = malloc(sizeof(float) * (size_t)S * I);
    o_matmul_q_s(g, x, G, GS, S, D, I);
    o_matmul_q_s(u, x, U, US, S, D, I);
    o_silu_mul(g, u, (int64_t)S * I);
    o_matmul_q_s(out, g, Dn, DS, S, I, D);
    free(g); free(u);
}

/* ------------------------------------------------------------------ */
/* Q4R4 / Q8R4: 4-row blocks, groups of 32, f16 group scales.          */
/* hw/hw_q4r4.h, nn/quant.c:110-179, nn/matmul.c:365-466               */

/* IEEE half -> float, exact (hw/hw_q4r4.h:22-33) */
O_EXPORT float o_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff, u;
    if (e == 0) {
        if (m == 0) u = s;
        else {
            int ee = 1;
            while (!(m & 0x400)) { m <<= 1; ee--; }
            m &= 0x3ff;
            u = s | ((uint32_t)(ee + 112) << 23) | (m << 13);
        }
    } else if (e == 31) u = s | 0x7f800000u | (m << 13);
    else u = s | ((e + 112) << 23) | (m << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* float -> IEEE half, round to nearest even (nn/quant.c:111-128) */
O_EXPORT uint16_t o_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000, e = (x >> 23) & 0xff, m = x & 0x7fffff;
    if (e == 0xff) return (uint16_t)(sign | 0x7c00 | (m ? 0x200 : 0));
    int ne = (int)e - 127 + 15;
    if (ne >= 31) return (uint16_t)(sign | 0x7c00);
    if (ne <= 0) {
        if (ne < -10) return (uint16_t)sign;
        m |= 0x800000;
        int sh = 14 - ne;
        uint32_t h = m >> sh, rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (h & 1))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)ne << 10) | (m >> 13), rem = m & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h++;
    return (uint16_t)(sign | h);
}

/* group-32 activation quantization (hw/hw_q4r4.h:36-46): per group
 * s = amax/127 clamped at 1e-30, inv = 1/s, q = rint(x*inv), xsum = sum q */
O_EXPORT void o_quant_g32(const float *x, int I, int8_t *xq, float *xs, int32_t *xsum) {
    for (int g = 0; g < I / 32; g++) {
        const float *xg = x + g * 32;
        float amax = 0.f;
        for (int j = 0; j < 32; j++) { float a = fabsf(xg[j]); if (a > amax) amax = a; }
        float s = amax / 127.f;
        if (s < 1e-30f) s = 1e-30f;
        float inv = 1.f / s;
        int32_t sm = 0;
        for (int j = 0; j < 32; j++) { int q = (int)rintf(xg[j] * inv); xq[g * 32 + j] = (int8_t)q; sm += q; }
        xs[g] = s;
        xsum[g] = sm;
    }
}

/* the "no-clip Q4_0" group scale shared by both packers (nn/quant.c:130-177):
 * mx = the group's largest-magnitude weight (first one wins ties), opp = the
 * largest |w| of the other sign, d = -sign(mx) * max(|mx|/lo, opp/hi) as f16 */
static uint16_t r4_scale(const float *wg, float lo, float hi, float *inv) {
    float mx = 0.f;
    for (int j = 0; j < 32; j++) if (fabsf(wg[j]) > fabsf(mx)) mx = wg[j];
    float opp = 0.f;
    for (int j = 0; j < 32; j++) if ((wg[j] > 0) != (mx > 0) && fabsf(wg[j]) > opp) opp = fabsf(wg[j]);
    float dm = fmaxf(fabsf(mx) / lo, opp / hi);
    uint16_t h = o_f32_to_f16(mx > 0 ? -dm : dm);
    float dd = o_f16_to_f32(h);
    *inv = dd != 0.f ? 1.f / dd : 0.f;
    return h;
}

/* w [O][I] f32 (I % 32 == 0) -> q [ceil(O/4)][I/32][4][16] (row r byte j =
 * c[j] | c[j+16] << 4, c = v + 8), d [ceil(O/4)][I/32][4] f16; missing rows
 * of the last block: codes 0x88, scale 0 (nn/quant.c:157-177) */
O_EXPORT void o_pack_q4r4(const float *w, int O, int I, uint8_t *q, uint16_t *d) {
    int nb = I / 32, O4 = (O + 3) / 4;
    for (int b = 0; b < O4; b++)
        for (int g = 0; g < nb; g++)
            for (int r = 0; r < 4; r++) {
                uint8_t *dst = q + ((size_t)b * nb + g) * 64 + r * 16;
                uint16_t *dp = d + ((size_t)b * nb + g) * 4 + r;
                int row = b * 4 + r;
                if (row >= O) { memset(dst, 0x88, 16); *dp = 0; continue; }
                const float *wg = w + (size_t)row * I + g * 32;
                float inv;
                *dp = r4_scale(wg, 8.f, 7.f, &inv);
                uint8_t c[32];
                for (int j = 0; j < 32; j++) {
                    int v = (int)rintf(wg[j] * inv);
                    if (v < -8) v = -8;
                    if (v > 7) v = 7;
                    c[j] = (uint8_t)(v + 8);
                }
                for (int j = 0; j < 16; j++) dst[j] = (uint8_t)(c[j] | (c[j + 16] << 4));
            }
}

/* the int8 sibling: [ceil(O/4)][I/32][4][32] signed codes (nn/quant.c:135-155) */
O_EXPORT void o_pack_q8r4(const float *w, int O, int I, int8_t *q, uint16_t *d) {
    int nb = I / 32, O4 = (O + 3) / 4;
    for (int b = 0; b < O4; b++)
        for (int g = 0; g < nb; g++)
            for (int r = 0; r < 4; r++) {
                int8_t *dst = q + ((size_t)b * nb + g) * 128 + r * 32;
                uint16_t *dp = d + ((size_t)b * nb + g) * 4 + r;
                int row = b * 4 + r;
                if (row >= O) { memset(dst, 0, 32); *dp = 0; continue; }
                const float *wg = w + (size_t)row * I + g * 32;
                float inv;
                *dp = r4_scale(wg, 128.f, 127.f, &inv);
                for (int j = 0; j < 32; j++) {
                    int v = (int)rintf(wg[j] * inv);
                    if (v < -128) v = -128;
                    if (v > 127) v = 127;
                    dst[j] = (int8_t)v;
                }
            }
}

/* Q4R4 matmul, the x86 build's evaluation (portable kernels = the scalar
 * references, nn/matmul.c:395-431).  Tokens t < 4*floor(S/4) go through the
 * 4-token tile kernel (hw/hw_q4r4.h:70-87): raw sum s = sum c*x over the
 * group, then acc = fma(s, dd*xs, acc) and acc = fma(-dd, xct, acc) with
 * xct = (8*xsum)*xs rounded once (:89-96).  The remaining tokens go through
 * the per-token kernel (:48-64): s -= 8*xsum in integers, acc = fma(s,
 * dd*xs, acc).  Groups in order; y [S][O]. */
O_EXPORT void o_matmul_q4r4(float *y, const float *x, const uint8_t *q, const uint16_t *d, int S, int I, int O) {
    int nb = I / 32, S4 = S / 4 * 4;
    int8_t *xq = malloc((size_t)I);
    float *xs = malloc(sizeof(float) * nb);
    int32_t *xm = malloc(sizeof(int32_t) * nb);
    for (int t = 0; t < S; t++) {
        o_quant_g32(x + (size_t)t * I, I, xq, xs, xm);
        for (int o = 0; o < O; o++) {
            int b = o / 4, r = o % 4;
            float acc = 0.f;
            for (int g = 0; g < nb; g++) {
                const uint8_t *wb = q + ((size_t)b * nb + g) * 64 + r * 16;
                const int8_t *xg = xq + g * 32;
                int32_t s = 0;
                for (int j = 0; j < 16; j++) s += (int32_t)(wb[j] & 0xF) * xg[j] + (int32_t)(wb[j] >> 4) * xg[j + 16];
                float dd = o_f16_to_f32(d[((size_t)b * nb + g) * 4 + r]);
                if (t < S4) {
                    float xct = 8.f * (float)xm[g] * xs[g];
                    acc = fmaf((float)s, dd * xs[g], acc);
                    acc = fmaf(-dd, xct, acc);
                } else {
                    s -= 8 * xm[g];
                    acc = fmaf((float)s, dd * xs[g], acc);
                }
            }
            y[(size_t)t * O + o] = acc;
        }
    }
    free(xq); free(xs); free(xm);
}

/* Q8R4 matmul (nn/matmul.c:435-466): one formula for both kernels,
 * acc = fma(sum c*x, dd*xs, acc) over the groups in order */
O_EXPORT void o_matmul_q8r4(float *y, const float *x, const int8_t *q, const uint16_t *d, int S, int I, int O) {
    int nb = I / 32;
    int8_t *xq = malloc((size_t)I);
    float *xs = malloc(sizeof(float) * nb);
    int32_t *xm = malloc(sizeof(int32_t) * nb);
    for (int t = 0; t < S; t++) {
        o_quant_g32(x + (size_t)t * I, I, xq, xs, xm);
        for (int o = 0; o < O; o++) {
            int b = o / 4, r = o % 4;
            float acc = 0.f;
            for (int g = 0; g < nb; g++) {
                const int8_t *wr = q + ((size_t)b * nb + g) * 128 + r * 32;
                const int8_t *xg = xq + g * 32;
                int32_t s = 0;
                for (int j = 0; j < 32; j++) s += (int32_t)wr[j] * xg[j];
                float dd = o_f16_to_f32(d[((size_t)b * nb + g) * 4 + r]);
                acc = fmaf((float)s, dd * xs[g], acc);
            }
            y[(size_t)t * O + o] = acc;
        }
    }
    free(xq); free(xs); free(xm);
}

/* ------------------------------------------------------------------ */
/* GGUF block formats -> device layouts.                               */
/* io/gguf.h:231-357 (block dequantisers and the Q4_0 repack),         */
/* io/st.h:74-80 (type ids and block sizes)                            */
enum { O_GG_Q8_0 = 4, O_GG_Q4_0 = 5, O_GG_Q4_K = 6, O_GG_Q5_K = 7, O_GG_Q6_K = 8 };

static uint16_t o_rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* elements per block and bytes per block; 0 if the id is not a block type */
O_EXPORT int o_gguf_block(int dtype, int *elems, int *bytes) {
    static const int E[9] = {0, 0, 0, 0, 32, 32, 256, 256, 256};
    static const int B[9] = {0, 0, 0, 0, 34, 18, 144, 176, 210};
    if (dtype < 4 || dtype > 8) return 0;
    *elems = E[dtype]; *bytes = B[dtype];
    return 1;
}

/* Q4_0 holds element i of a 32-block in the low nibble of byte i and element
 * i+16 in the high nibble; the grouped int4 layout holds elements 2k, 2k+1 in
 * byte k (low, high).  Both store v+8, so the repack moves nibbles and
 * widens the f16 scale (io/gguf.h:335-357). */
O_EXPORT void o_gguf_repack_q4_0(const uint8_t *blocks, uint8_t *q4, float *qs, int64_t O, int64_t I) {
    int64_t nblk = O * (I / 32);
    for (int64_t b = 0; b < nblk; b++) {
        const uint8_t *src = blocks + b * 18, *nib = src + 2;
        qs[b] = o_f16_to_f32(o_rd16(src));
        uint8_t el[32];
        for (int i = 0; i < 16; i++) { el[i] = nib[i] & 15; el[i + 16] = nib[i] >> 4; }
        for (int k = 0; k < 16; k++) q4[b * 16 + k] = (uint8_t)(el[2 * k] | (el[2 * k + 1] << 4));
    }
}

/* K-quant 6-bit sub-block scale and min, j = 0..7 (io/gguf.h:253-260):
 * bytes 0-3 carry scales 0-3, bytes 4-7 mins 0-3 (low six bits each);
 * sub-blocks 4-7 take their low four bits from bytes 8-11 and their top two
 * from the spare high bits of bytes 0-7. */
static void o_k4_sm(const uint8_t *s, int j, float d, float dmin, float *sc, float *mn) {
    int a, m;
    if (j < 4) { a = s[j] & 63; m = s[j + 4] & 63; }
    else { a = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4); m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4); }
    *sc = d * (float)a;
    *mn = dmin * (float)m;
}

/* Block dequantisers behind st_read_f32 (io/gguf.h:231-330).  Q4_K / Q5_K
 * compute sc*q - mn, which the reference's x86 build fuses into one FMA; the
 * fusion cannot change a result (sc = f16 * 6-bit integer and q < 32, so
 * sc*q is exact in f32), and the FMA is kept only to mirror that build. */
O_EXPORT int o_gguf_dequant(int dtype, const uint8_t *raw, int64_t numel, float *out) {
    int E, B;
    if (!o_gguf_block(dtype, &E, &B) || numel % E) return -1;
    int64_t nblk = numel / E;
    for (int64_t b = 0; b < nblk; b++) {
        const uint8_t *p = raw + b * B;
        float *y = out + b * E;
        if (dtype == O_GG_Q8_0) {
            float d = o_f16_to_f32(o_rd16(p));
            for (int i = 0; i < 32; i++) y[i] = d * (float)(int8_t)p[2 + i];
        } else if (dtype == O_GG_Q4_0) {
            float d = o_f16_to_f32(o_rd16(p));
            for (int i = 0; i < 16; i++) {
                y[i] = d * (float)((p[2 + i] & 15) - 8);
                y[i + 16] = d * (float)((p[2 + i] >> 4) - 8);
            }
        } else if (dtype == O_GG_Q4_K || dtype == O_GG_Q5_K) {
            /* 4 chunks of 64: low nibbles of 32 bytes (sub-block 2c), then the
             * high nibbles (sub-block 2c+1); Q5_K adds 16 from bit 2c / 2c+1
             * of qh[l] */
            int q5 = dtype == O_GG_Q5_K;
            float d = o_f16_to_f32(o_rd16(p)), dmin = o_f16_to_f32(o_rd16(p + 2));
            const uint8_t *s = p + 4, *qh = p + 16, *ql = p + (q5 ? 48 : 16);
            for (int c = 0; c < 4; c++)
                for (int h = 0; h < 2; h++) {
                    float sc, mn;
                    o_k4_sm(s, 2 * c + h, d, dmin, &sc, &mn);
                    for (int l = 0; l < 32; l++) {
                        int v = h ? ql[32 * c + l] >> 4 : ql[32 * c + l] & 15;
                        if (q5 && ((qh[l] >> (2 * c + h)) & 1)) v += 16;
                        y[64 * c + 32 * h + l] = fmaf(sc, (float)v, -mn);
                    }
                }
        } else {
            /* Q6_K: two halves of 128; element 128n + 32r + l takes its low
             * four bits from ql[64n + l + 32(r&1)] (nibble r>>1), its top two
             * from bits 2r of qh[32n + l], and int8 scale sc[8n + l/16 + 2r];
             * value (d*sc)*(q-32) */
            const uint8_t *ql = p, *qh = p + 128;
            const int8_t *sc = (const int8_t *)(p + 192);
            float d = o_f16_to_f32(o_rd16(p + 208));
            for (int n = 0; n < 2; n++)
                for (int r = 0; r < 4; r++)
                    for (int l = 0; l < 32; l++) {
                        uint8_t lo = ql[64 * n + l + 32 * (r & 1)];
                        int v = ((r >> 1) ? lo >> 4 : lo & 15) | (((qh[32 * n + l] >> (2 * r)) & 3) << 4);
                        y[128 * n + 32 * r + l] = d * (float)sc[8 * n + l / 16 + 2 * r] * (float)(v - 32);
                    }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Expert cache bookkeeping (runtime/moecache.c:4-89, io/tier.c:23-26). */
/* Slots, LFRU heat/recency, pins, hit/miss counters; the weights are   */
/* not modelled (a load is reported to the caller instead).            */
typedef struct {
    int cap, n, n_experts;
    uint32_t clock;
    long long hits, misses;
    int *eid;            /* [cap] */
    uint32_t *heat, *last;
    uint8_t *pinned;
} OCache;

O_EXPORT void *o_ecache_new(int cap, int n_experts) {
    OCache *c = calloc(1, sizeof *c);
    if (cap < 1) cap = 1;
    c->cap = cap;
    c->n_experts = n_experts;
    c->eid = malloc(sizeof(int) * cap);
    for (int i = 0; i < cap; i++) c->eid[i] = -1;
    if (n_experts > 0) {
        c->heat = calloc(n_experts, 4);
        c->last = calloc(n_experts, 4);
        c->pinned = calloc(n_experts, 1);
    }
    return c;
}

O_EXPORT void o_ecache_free(void *p) {
    OCache *c = p;
    free(c->eid); free(c->heat); free(c->last); free(c->pinned); free(c);
}

/* frequency in the high bits, recency (255 - age, floored at 0) in the low 8 */
static uint64_t o_lfru(uint32_t heat, uint32_t last, uint32_t clock) {
    uint32_t age = clock - last;
    return ((uint64_t)heat << 8) | (age < 255 ? 255 - age : 0);
}

static int o_is_pinned(const OCache *c, int e) {
    return c->pinned && e >= 0 && e < c->n_experts && c->pinned[e];
}

/* moty_expert_get: returns the slot; *loaded = 1 on a miss (the slot is
 * refilled with eid).  Victim on a full cache: the unpinned resident of
 * least score (first on ties; slot 0 if every resident is pinned); without
 * heat tracking (n_experts == 0) slot 1, the reference's LRU-by-fill stand-in. */
O_EXPORT int o_ecache_get(void *p, int eid, int *loaded) {
    OCache *c = p;
    if (c->heat && eid >= 0 && eid < c->n_experts) {
        if (c->heat[eid] < 0xFFFFFFFFu) c->heat[eid]++;
        c->last[eid] = c->clock++;
    }
    for (int i = 0; i < c->n; i++)
        if (c->eid[i] == eid) { c->hits++; *loaded = 0; return i; }
    c->misses++;
    int v;
    if (c->n < c->cap) v = c->n++;
    else {
        v = 0;
        if (c->heat) {
            uint64_t worst = UINT64_MAX;
            for (int i = 0; i < c->n; i++) {
                int e = c->eid[i];
                if (o_is_pinned(c, e)) continue;
                uint64_t s = o_lfru(c->heat[e], c->last[e], c->clock);
                if (s < worst) { worst = s; v = i; }
            }
        } else {
            for (int i = 1; i < c->n; i++) if (!o_is_pinned(c, c->eid[i])) { v = i; break; }
        }
    }
    c->eid[v] = eid;
    *loaded = 1;
    return v;
}

/* moty_expert_pin: mark pinned, then always load into a fresh slot, or the
 * first unpinned resident's, or slot 0 */
O_EXPORT int o_ecache_pin(void *p, int eid) {
    OCache *c = p;
    if (c->pinned && eid >= 0 && eid < c->n_experts) c->pinned[eid] = 1;
    int v;
    if (c->n < c->cap) v = c->n++;
    else {
        v = -1;
        for (int i = 0; i < c->n; i++) if (!o_is_pinned(c, c->eid[i])) { v = i; break; }
        if (v < 0) v = 0;
    }
    c->eid[v] = eid;
    return v;
}

O_EXPORT void o_ecache_state(void *p, int *n, int *eids, uint32_t *heat, uint32_t *last, uint32_t *clock,
                             long long *hits, long long *misses) {
    OCache *c = p;
    *n = c->n;
    memcpy(eids, c->eid, sizeof(int) * c->cap);
    if (c->heat) { memcpy(heat, c->heat, 4 * c->n_experts); memcpy(last, c->last, 4 * c->n_experts); }
    *clock = c->clock; *hits = c->hits; *misses = c->misses;
}

/* moty_moe_route_bias (runtime/moecache.c:91-95): logits of every filled
 * slot's expert += bias, once per slot */
O_EXPORT void o_ecache_route_bias(void *p, float *logits, float bias) {
    OCache *c = p;
    if (bias <= 0) return;
    for (int i = 0; i < c->n; i++) if (c->eid[i] >= 0) logits[c->eid[i]] += bias;
}
