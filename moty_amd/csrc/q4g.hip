// q4g.hip -- grouped int4 (group 32, f32 group scales) GEMV/GEMM.
//
// Reference: moty_matmul_i4_grouped_s (nn/matmul.c:164-197).
//  IDOT4=1 (gs == 32, I % 64 == 0):  xq = qrow_i8(x), then per output
//    acc = 0; for g ascending: acc = fma(scl[o][g], (float)(d_g - 8*xg_g), acc)
//    y = sx * acc                      (hw/hw_avx512.h:155-176, matmul.c:148-160)
//  default (exact f32 activations):  per group
//    t[j] = fma(x[j], w[j], x[j+16]*w[j+16]), j < 16; r = hsum16(t);
//    a = fma(r, scl[o][g], a)           (nn/matmul.c:199-253)
//
// The integer group dot d_g - 8*xg_g equals sum (n-8)*x exactly, so the
// kernels expand nibbles straight to signed int8 (n-8) and never need the
// group sums xg.  Group scales multiply a float chain whose order is fixed,
// so each output's chain runs in ascending group order in one lane.
#include "common.h"
#include "kernels.h"

#include <type_traits>

namespace moty {

// ---------------------------------------------------------------------------
// IDOT4 GEMV, S <= 4.  Workgroup: 4 waves, RB rows.  Per 64-group chunk:
// phase 1 -- every lane computes one group's integer dot for each token
// (16 B of nibbles, coalesced) and parks it with the group scale in LDS;
// phase 2 -- one lane per (row, token) extends its FMA chain over the chunk's
// 64 groups in order.  Activations are quantized into LDS at the start.
constexpr int Q4V_NT = 256;
constexpr int Q4V_ROWS = 16;  // rows per workgroup

template <int S_>
__global__ __launch_bounds__(Q4V_NT) void k_gemv_i4g(const float* __restrict__ x, const uint8_t* __restrict__ q4,
                                                     const float* __restrict__ scl, float* __restrict__ y, int I,
                                                     int O) {
  extern __shared__ __align__(16) int8_t xq_s[];  // [S_][I]
  __shared__ int dv[Q4V_ROWS][S_][65];
  __shared__ float sv[Q4V_ROWS][65];
  __shared__ float red[Q4V_NT / MOTY_WAVE][S_];
  __shared__ float sx_s[S_];
  const int lane = threadIdx.x % MOTY_WAVE, wv = threadIdx.x / MOTY_WAVE;
  const int ng = I / 32, rb = I / 2;
  const int ob = blockIdx.x * Q4V_ROWS;
  // activation quantization (qrow_i8) into LDS
#pragma unroll
  for (int s = 0; s < S_; s++) {
    float amax = 0.f;
    for (int i = threadIdx.x * 4; i < I; i += Q4V_NT * 4) {
      const float4 v = *(const float4*)(x + (int64_t)s * I + i);
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    amax = wave_max_f32(amax);
    if (lane == 0) red[wv][s] = amax;
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < S_; s++) {
    float amax = red[0][s];
    for (int i = 1; i < Q4V_NT / MOTY_WAVE; i++) amax = fmaxf(amax, red[i][s]);
    float sc = amax / 127.f;
    if (sc < 1e-12f) sc = 1e-12f;
    const float inv = 1.f / sc;
    if (threadIdx.x == 0) sx_s[s] = sc;
    for (int i = threadIdx.x * 4; i < I; i += Q4V_NT * 4) {
      const float4 v = *(const float4*)(x + (int64_t)s * I + i);
      const uint32_t p = (uint32_t)(rne_int(v.x * inv) & 0xff) | ((uint32_t)(rne_int(v.y * inv) & 0xff) << 8) |
                         ((uint32_t)(rne_int(v.z * inv) & 0xff) << 16) |
                         ((uint32_t)(rne_int(v.w * inv) & 0xff) << 24);
      *(uint32_t*)(xq_s + s * I + i) = p;
    }
  }
  __syncthreads();
  float acc = 0.f;  // chain of lane j = r*S_ + s (j < Q4V_ROWS*S_)
  const int cr = threadIdx.x / S_, cs = threadIdx.x % S_;
  for (int c0 = 0; c0 < ng; c0 += 64) {
    const int g = c0 + lane;
    for (int r = wv; r < Q4V_ROWS; r += Q4V_NT / MOTY_WAVE) {
      const int o = ob + r;
      const bool ok = (o < O) && (g < ng);
      const int4 wb = ok ? *(const int4*)(q4 + (int64_t)o * rb + g * 16) : int4{0, 0, 0, 0};
      const float sc = ok ? scl[(int64_t)o * ng + g] : 0.f;
      const int4 w0 = unpack_nib16(uint2{(uint32_t)wb.x, (uint32_t)wb.y});
      const int4 w1 = unpack_nib16(uint2{(uint32_t)wb.z, (uint32_t)wb.w});
#pragma unroll
      for (int s = 0; s < S_; s++) {
        int d = 0;
        if (g < ng) {
          const int4 x0 = *(const int4*)(xq_s + s * I + g * 32);
          const int4 x1 = *(const int4*)(xq_s + s * I + g * 32 + 16);
          d = dot16(w0, x0, 0);
          d = dot16(w1, x1, d);
        }
        dv[r][s][lane] = d;
      }
      sv[r][lane] = sc;
    }
    __syncthreads();
    if (threadIdx.x < Q4V_ROWS * S_) {
      const int n = (ng - c0) < 64 ? (ng - c0) : 64;
      for (int j = 0; j < n; j++) acc = __fmaf_rn(sv[cr][j], (float)dv[cr][cs][j], acc);
    }
    __syncthreads();
  }
  if (threadIdx.x < Q4V_ROWS * S_) {
    const int o = ob + cr;
    if (o < O) y[(int64_t)cs * O + o] = sx_s[cs] * acc;
  }
}

// v_cvt_off_f32_i4 of byte K of w: the signed nibble in bits [8K, 8K+4)
// divided by 16 (exact), one SDWA-selected conversion
template <int K>
__device__ __forceinline__ float cvt_off_b(uint32_t w) {
  float r;
  if (K == 0)
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(w));
  else if (K == 1)
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(w));
  else if (K == 2)
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(w));
  else
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(w));
  return r;
}

// ---------------------------------------------------------------------------
// IDOT4 GEMV for decode (S = 1), optionally PAIR (gate + up + SiLU).
// Workgroup = 4 waves; a wave owns RW consecutive output rows (of W, and of
// W2 in PAIR mode):
//   1. it issues the nibble loads of its rows' first PD 64-group chunks --
//      lane l takes group l of each chunk (16 B, coalesced along the row) --
//      and each further chunk as the one PD before it is consumed;
//   2. the workgroup quantizes x into LDS (qrow_i8) while those loads fly;
//   3. per chunk, each lane forms its group's exact integer dot sum (n-8)*x
//      and parks it, with the group scale, in the wave's LDS slice;
//   4. one lane per row extends the reference's FMA chain over the chunk's
//      groups in order; y = sx * acc (PAIR: h = silu(g) * u).
template <int RW, int NGC, bool PAIR, int NT, int PD = NGC, bool XF = false>
__global__ __launch_bounds__(NT) void k_gemv1_i4g(const float* __restrict__ x, const uint8_t* __restrict__ q4,
                                                      const float* __restrict__ scl,
                                                      const uint8_t* __restrict__ q4b,
                                                      const float* __restrict__ sclb, float* __restrict__ y, int I,
                                                      int O) {
  constexpr int NM = PAIR ? 2 : 1;
  constexpr int WAVES = NT / MOTY_WAVE;
  constexpr int XV = (NGC * 64 * 32) / (NT * 4);  // float4 of x per thread (I <= 2048 * NGC)
  extern __shared__ __align__(16) int8_t lds[];
  __shared__ float red[WAVES];
  __shared__ float sx_s;
  const int lane = threadIdx.x % MOTY_WAVE, wv = threadIdx.x / MOTY_WAVE;
  const int ng = I / 32, rb = I / 2;
  constexpr int ldv = 66;  // one chunk's 64 groups, padded (even: float4 reads stay aligned)
  int8_t* xq_s = lds;                                                          // [I]
  int* xg8 = (int*)(lds + I);                                                  // [ng] -8 * group sums
  float* xf_s = (float*)lds;  // XF: [ng][36] f32 -- each group's 32 values, rows padded to 144 B so
                              // the lanes' 16-byte reads of their groups spread over the banks
  float2* dv = (float2*)(lds + (XF ? 4 * ng * 36 : I + ng * 4)) + (size_t)wv * (NM * RW * ldv);  // [NM*RW][ldv] (scale, dot) of one chunk
  const int o0 = (blockIdx.x * WAVES + wv) * RW;

  // 1. x (one pass, kept in registers), then every nibble load of this wave
  float4 xr[XV];
#pragma unroll
  for (int j = 0; j < XV; j++) {
    const int i = (threadIdx.x + j * NT) * 4;
    xr[j] = *(const float4*)(x + (i < I ? i : 0));  // clamped: zeroed below
  }
  int4 wb[NM][RW][NGC];
  float wsc[NM][RW][NGC];  // group scales, loaded with the nibbles
  // chunk-major issue order, PD chunks ahead: chunk c of every row is
  // issued before chunk c+1, and chunk c+PD only when chunk c is consumed,
  // so each row's data arrives spread over the stream and its FMA chain
  // (one dependent FMA per group) runs behind it; with every chunk issued
  // at once a row's whole chain would start after its last byte lands
  // (the compiler waits only for the chunk it consumes)
  auto issue = [&](int c) {
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int r = 0; r < RW; r++) {
        const int64_t o = o0 + r < O ? o0 + r : O - 1;
        // clamped (unused past ng): unconditional loads keep the wave's
        // loads in one straight run, with no wait at branch joins
        const int g = c * 64 + lane < ng ? c * 64 + lane : 0;
        {
          const v4i t = __builtin_nontemporal_load((const v4i*)((m ? q4b : q4) + o * rb + g * 16));
          wb[m][r][c] = int4{t.x, t.y, t.z, t.w};
        }
        wsc[m][r][c] = __builtin_nontemporal_load((m ? sclb : scl) + o * ng + g);
      }
  };
#pragma unroll
  for (int c = 0; c < PD; c++) issue(c);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < XV; j++) xr[j] = sel4((threadIdx.x + j * NT) * 4 < I, xr[j]);
  // XF: x into LDS as 16 x (exact) when every |x| < 2^123 -- then the
  // nibbles convert as (n - 8) / 16 and each product, hence each rounding,
  // is the reference's -- else as it is, for the full-width conversion
  bool x16 = false;
  if (XF) {
    bool big = false;
#pragma unroll
    for (int j = 0; j < XV; j++)
      big |= fmaxf(fmaxf(fabsf(xr[j].x), fabsf(xr[j].y)), fmaxf(fabsf(xr[j].z), fabsf(xr[j].w))) >= 0x1p123f;
    x16 = !__syncthreads_or(big);
#pragma unroll
    for (int j = 0; j < XV; j++) {
      const int i = (threadIdx.x + j * NT) * 4;
      float4 v = xr[j];
      if (x16) v = float4{16.f * v.x, 16.f * v.y, 16.f * v.z, 16.f * v.w};
      if (i < I) *(float4*)(xf_s + (i >> 5) * 36 + (i & 31)) = v;
    }
    __syncthreads();
  } else {
  // 2. qrow_i8 of x into LDS
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < XV; j++)
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(xr[j].x), fabsf(xr[j].y)), fmaxf(fabsf(xr[j].z), fabsf(xr[j].w))));
  amax = wave_max_f32(amax);
  if (lane == 0) red[wv] = amax;
  __syncthreads();
  {
    float mx = red[0];
#pragma unroll
    for (int i = 1; i < WAVES; i++) mx = fmaxf(mx, red[i]);
    float sc = mx / 127.f;
    if (sc < 1e-12f) sc = 1e-12f;
    const float inv = 1.f / sc;
    if (threadIdx.x == 0) sx_s = sc;
#pragma unroll
    for (int j = 0; j < XV; j++) {
      const int i = (threadIdx.x + j * NT) * 4;
      const float4 v = xr[j];
      if (i < I)
        *(uint32_t*)(xq_s + i) = (uint32_t)(rne_int(v.x * inv) & 0xff) | ((uint32_t)(rne_int(v.y * inv) & 0xff) << 8) |
                                 ((uint32_t)(rne_int(v.z * inv) & 0xff) << 16) |
                                 ((uint32_t)(rne_int(v.w * inv) & 0xff) << 24);
    }
  }
  __syncthreads();
  // -8 * each group's activation sum: the dots run on the unsigned codes n
  // and start from it, giving sum (n-8)*x exactly
  for (int g = threadIdx.x; g < ng; g += NT) {
    const int4 a = *(const int4*)(xq_s + g * 32), b = *(const int4*)(xq_s + g * 32 + 16);
    xg8[g] = -8 * dot16(b, int4{0x01010101, 0x01010101, 0x01010101, 0x01010101},
                        dot16(a, int4{0x01010101, 0x01010101, 0x01010101, 0x01010101}, 0));
  }
  __syncthreads();
  }
  // 3./4. per 64-group chunk: every lane forms its group's exact integer dot
  // for each row and parks (scale, dot) in the wave's LDS slice; then lane
  // j < NM*RW continues the FMA chain of its row (j % RW of matrix j / RW)
  // over the chunk's groups in order, while later chunks may still arrive.
  // 16-byte LDS reads carry two groups' pairs.
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < NGC; c++) {
    if (c + PD < NGC) {
      issue(c + PD);
      __builtin_amdgcn_sched_barrier(0);
    }
    const int g = c * 64 + lane;
    if (XF && g < ng) {
      // the reference's exact f32 group sum (nn/matmul.c:222-233, the
      // AVX-512 form with FMA contraction): t[j] = fma(x[j], w[j],
      // x[16+j]*w[16+j]), then the 16 -> 8 -> 4 -> 1 reduction tree
      float xv[32];
#pragma unroll
      for (int q = 0; q < 8; q++) *(float4*)(xv + 4 * q) = *(const float4*)(xf_s + g * 36 + 4 * q);
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < RW; r++) {
          const int4 w = wb[m][r][c];
          const uint32_t wd[4] = {(uint32_t)w.x, (uint32_t)w.y, (uint32_t)w.z, (uint32_t)w.w};
          float wf[32];  // element e = byte e/2, low nibble when e is even, minus 8 (exact)
          if (x16) {
            // (n - 8) / 16: n ^ 8 is n - 8 as a signed nibble, and
            // v_cvt_off_f32_i4 gives a signed nibble / 16 from the low
            // 4 bits of its byte-selected operand
#pragma unroll
            for (int q = 0; q < 4; q++) {
              const uint32_t a = wd[q] ^ 0x88888888u, b = a >> 4;
              wf[8 * q + 0] = cvt_off_b<0>(a);
              wf[8 * q + 1] = cvt_off_b<0>(b);
              wf[8 * q + 2] = cvt_off_b<1>(a);
              wf[8 * q + 3] = cvt_off_b<1>(b);
              wf[8 * q + 4] = cvt_off_b<2>(a);
              wf[8 * q + 5] = cvt_off_b<2>(b);
              wf[8 * q + 6] = cvt_off_b<3>(a);
              wf[8 * q + 7] = cvt_off_b<3>(b);
            }
          } else {
#pragma unroll
            for (int q = 0; q < 4; q++) {
              // n - 8 as signed bytes ((n + 0x78) ^ 0x80, carry-free),
              // each then converted from its byte position
              const uint32_t lo = ((wd[q] & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u;
              const uint32_t hi = (((wd[q] >> 4) & 0x0f0f0f0fu) + 0x78787878u) ^ 0x80808080u;
#pragma unroll
              for (int k = 0; k < 4; k++) {
                wf[8 * q + 2 * k] = (float)(int8_t)(lo >> (8 * k));
                wf[8 * q + 2 * k + 1] = (float)(int8_t)(hi >> (8 * k));
              }
            }
          }
          float t[16];
#pragma unroll
          for (int j = 0; j < 16; j++) t[j] = __fmaf_rn(xv[j], wf[j], xv[16 + j] * wf[16 + j]);
          float u[8], v[4];
#pragma unroll
          for (int j = 0; j < 8; j++) u[j] = t[j + 8] + t[j];
#pragma unroll
          for (int j = 0; j < 4; j++) v[j] = u[j + 4] + u[j];
          dv[(m * RW + r) * ldv + lane] = float2{wsc[m][r][c], (v[0] + v[2]) + (v[1] + v[3])};
        }
    }
    if (!XF && g < ng) {
      const int4 x0 = *(const int4*)(xq_s + g * 32);
      const int4 x1 = *(const int4*)(xq_s + g * 32 + 16);
      const int c8 = xg8[g];
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < RW; r++) {
          const int4 w = wb[m][r][c];
          const int4 w0 = unpack_nib16_u(uint2{(uint32_t)w.x, (uint32_t)w.y});
          const int4 w1 = unpack_nib16_u(uint2{(uint32_t)w.z, (uint32_t)w.w});
          const int d = dot16(w1, x1, dot16(w0, x0, c8));
          dv[(m * RW + r) * ldv + lane] = float2{wsc[m][r][c], (float)d};
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < NM * RW) {
      const int gend = ng < (c + 1) * 64 ? ng : (c + 1) * 64;
      const float4* dr = (const float4*)(dv + lane * ldv - c * 64);
      int gg = c * 64;
      for (; gg + 16 <= gend; gg += 16) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = dr[gg / 2 + u];
#pragma unroll
        for (int u = 0; u < 8; u++) {
          acc = __fmaf_rn(v[u].x, v[u].y, acc);
          acc = __fmaf_rn(v[u].z, v[u].w, acc);
        }
      }
      const float2* d2 = dv + lane * ldv - c * 64;
      for (; gg < gend; gg++) acc = __fmaf_rn(d2[gg].x, d2[gg].y, acc);
    }
    // the next chunk's dots overwrite the slice: after these reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // XF: y = a (no activation scale)
  const float sxv = XF ? 0.f : sx_s;
  if (PAIR) {
    const float u = __shfl(acc, (lane + RW) & 63, 64);  // lane r < RW: the up row's chain
    const int o = o0 + lane;
    if (lane < RW && o < O) y[o] = XF ? ref_silu_mul(acc, u) : ref_silu_mul(sxv * acc, sxv * u);
  } else {
    const int o = o0 + lane;
    if (lane < RW && o < O) y[o] = XF ? acc : sxv * acc;
  }
}

// ---------------------------------------------------------------------------
// IDOT4 GEMM on v_mfma_i32_32x32x32_i8: one MFMA per group (K = 32 exactly),
// so each group's integer dot comes out separately and is folded into a
// float accumulator per output, in group order:
//     accf = fma(scl[o][g], (float)d, accf)
// Workgroup: 4 waves as 2 (tokens) x 2 (rows), block tile 64 x 64.  Per
// K block of 4 groups the workgroup stages, by whole-line loads, the int8
// activations (64 x 128 B), the nibbles (64 x 64 B) and the group scales
// (64 x 4) in LDS, the next block's loads in flight in registers.
// Lane l's A fragment is 16 bytes of token row (l % 32) at offset 16*(l/32)
// of the group; its B fragment the matching 8 nibble bytes of weight row
// (l % 32), expanded to signed n-8 -- one scale per lane per group.
constexpr int Q4M_NT = 256;
constexpr int Q4M_KG = 4;             // groups per K block
constexpr int Q4M_AS = 128 + 16;      // LDS row stride: activations
constexpr int Q4M_BS = 64 + 16;       // nibbles
constexpr int Q4M_SS = Q4M_KG + 1;    // scales

template <int NS = 2>
__global__ __launch_bounds__(Q4M_NT, 2) void k_gemm_i4g(const int8_t* __restrict__ xq, const float* __restrict__ sx,
                                                        const uint8_t* __restrict__ q4,
                                                        const float* __restrict__ scl, float* __restrict__ y,
                                                        int M, int I, int O) {
  __shared__ __align__(16) int8_t sA[64 * Q4M_AS];
  __shared__ __align__(16) uint8_t sB[64 * Q4M_BS];
  __shared__ float sS[64 * Q4M_SS];
  const int tid = threadIdx.x, lane = tid % MOTY_WAVE, wv = tid / MOTY_WAVE;
  const int wm = wv >> 1, wn = wv & 1;
  const int r32 = lane & 31, hk = lane >> 5;
  const int mb = blockIdx.y * 64, nb = blockIdx.x * 64;
  const int ng = I / 32, rb = I / 2;
  // copy assignments: A 2 x 16 B chunks (row = q/8, col16 = q%8), B 1 chunk
  // (row = tid/4, col16 = tid%4), S 1 float (row = tid/4, group = tid%4)
  const int8_t* srcA[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int q = tid + i * Q4M_NT;
    int m = mb + (q >> 3);
    m = m < M ? m : M - 1;
    srcA[i] = xq + (int64_t)m * I + (q & 7) * 16;
  }
  int nrow = nb + (tid >> 2);
  nrow = nrow < O ? nrow : O - 1;
  const uint8_t* srcB = q4 + (int64_t)nrow * rb + (tid & 3) * 16;
  const float* srcS = scl + (int64_t)nrow * ng + (tid & 3);
  // epilogue: the activation scale of tile row tid % 64, loaded now so its
  // latency hides behind the K loop (to LDS after it)
  __shared__ float s_sx[64];
  const float sxr = sx[mb + (tid & 63) < M ? mb + (tid & 63) : M - 1];
  // Two register sets: while one K block is consumed from LDS, the next two
  // are in flight.  Loads are unconditional, from clamped addresses (a block
  // past the end re-reads the last one; a chunk past the row end re-reads
  // the row start), and are masked when written to LDS: with no branch
  // around a load the compiler waits only for the set about to be consumed.
  // I % 64 == 0, so a K block of 4 groups (128 elements) is whole or the
  // last 2 groups of the row are missing (I % 128 == 64).
  struct Set {
    int4 a[2];
    int4 b;
    float s;
  };
  Set sets[NS];
  const int glast = (ng - 1) / Q4M_KG * Q4M_KG;
  auto gload = [&](int g0, Set& st) {
    const int gc = g0 < ng ? g0 : glast;
    const int kb = gc * 32;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int q = tid + i * Q4M_NT;
      st.a[i] = *(const int4*)(srcA[i] + (kb + (q & 7) * 16 < I ? kb : -(q & 7) * 16));
    }
    st.b = *(const int4*)(srcB + (gc * 16 + (tid & 3) * 16 < rb ? gc * 16 : -(tid & 3) * 16));
    st.s = srcS[gc + (tid & 3) < ng ? gc : -(tid & 3)];
    __builtin_amdgcn_sched_barrier(0);
  };
  float accf[16];
#pragma unroll
  for (int r = 0; r < 16; r++) accf[r] = 0.f;
  auto stage = [&](int g0, Set& st) {
    const int kb = g0 * 32;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int q = tid + i * Q4M_NT;
      *(int4*)(sA + (q >> 3) * Q4M_AS + (q & 7) * 16) = sel4(kb + (q & 7) * 16 < I, st.a[i]);
    }
    *(int4*)(sB + (tid >> 2) * Q4M_BS + (tid & 3) * 16) = sel4(g0 * 16 + (tid & 3) * 16 < rb, st.b);
    sS[(tid >> 2) * Q4M_SS + (tid & 3)] = g0 + (tid & 3) < ng ? st.s : 0.f;
    __syncthreads();
    gload(g0 + NS * Q4M_KG, st);
    // Straight-line over the block's 4 groups -- fragments, then the 4
    // MFMAs, then the 4 epilogues in group order -- so the MFMAs overlap
    // each other and the fragment reads.  Groups past the row end hold zero
    // codes, activations and scales: their step fma(0, 0, acc) adds
    // exactly nothing (acc is never -0: it starts at +0, and an exact zero
    // result rounds to +0).
    if (g0 < ng) {
      v4i a[Q4M_KG];
      int4 w[Q4M_KG];
      float sc[Q4M_KG];
#pragma unroll
      for (int gg = 0; gg < Q4M_KG; gg++) {
        a[gg] = *(const v4i*)(sA + (wm * 32 + r32) * Q4M_AS + gg * 32 + hk * 16);
        w[gg] = unpack_nib16(*(const uint2*)(sB + (wn * 32 + r32) * Q4M_BS + gg * 16 + hk * 8));
        sc[gg] = sS[(wn * 32 + r32) * Q4M_SS + gg];
      }
      v16i d[Q4M_KG];
#pragma unroll
      for (int gg = 0; gg < Q4M_KG; gg++)
        d[gg] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[gg], *(const v4i*)&w[gg], v16i{}, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);  // all four MFMAs issue before the epilogues
#pragma unroll
      for (int gg = 0; gg < Q4M_KG; gg++)
#pragma unroll
        for (int r = 0; r < 16; r++) accf[r] = __fmaf_rn(sc[gg], (float)d[gg][r], accf[r]);
    }
    __syncthreads();
  };
#pragma unroll
  for (int i = 0; i < NS; i++) gload(i * Q4M_KG, sets[i]);
  for (int g0 = 0; g0 < ng; g0 += NS * Q4M_KG) {
#pragma unroll
    for (int i = 0; i < NS; i++) stage(g0 + i * Q4M_KG, sets[i]);
  }
  // retire the clamped prefetch still in flight once, here: otherwise the
  // compiler waits for every memory operation before each conditional store
  __builtin_amdgcn_s_waitcnt(0);
  if (tid < 64) s_sx[tid] = sxr;
  __syncthreads();
  const int col = nb + wn * 32 + r32;
  if (col >= O) return;
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const int rl = wm * 32 + 8 * (r >> 2) + 4 * hk + (r & 3);
    if (mb + rl < M) y[(int64_t)(mb + rl) * O + col] = s_sx[rl] * accf[r];
  }
}

// ---------------------------------------------------------------------------
// IDOT4 GEMM on f16 MFMA (v_mfma_f32_32x32x16_f16, two per group).  The
// reference's per-group step is acc = fma(scl[o][g], (float)d_g, acc) in group
// order, d_g = sum over the group of (n - 8) * xq: an exact integer.  With f16
// operands -- activation codes in [-127, 127] and weight codes n - 8 in
// [-8, 7] are exact halves, every partial sum is an integer below 2^24 -- the
// MFMA returns d_g already as an exact float, so the epilogue is one FMA per
// output per group instead of a conversion and an FMA.
//
// Weight nibbles become halves with one v_and_or_b32 per pair and no
// float op: in a dword of 4 weight bytes, (w & 0x000f000f) | 0x64006400 is
// the half pair (1024 + n) of the low nibbles of bytes 0 and 2, the mask
// 0x00f000f0 gives (1024 + 16 n) for their high nibbles, and w >> 8 serves
// bytes 1 and 3 alike.  So a lane's 8 bytes of a group (16 codes e0..e15)
// become two 8-half fragments, low nibbles [e0,e4,e2,e6,e8,e12,e10,e14] and
// high nibbles [e1,e5,...] at 16x, matched by k_qrow_f16p's activation
// fragments x and x/16.  With the activations x, the two MFMAs give
//   sum_lo x (1024 + n) + sum_hi x (64 + n) = d_g + 1032 sum_lo x + 72 sum_hi x,
// and two more MFMAs of the same activation fragments against constant
// fragments (-1032 and -1152 = -72 * 16) give the offset, once per token
// tile and group for every weight tile: it enters the first product MFMA as
// its accumulator.  Every value is an integer below 2^23 in magnitude (|x|
// <= 127, 16 terms of each kind), so every sum is exact and d_g comes out
// exactly as the reference's integer group dot.
//
// Block tile BM tokens x BN weight rows, 4 waves as 2 x 2, each wave FM x FN
// 32 x 32 tiles.  K blocks of 4 groups (128 elements) move global -> LDS by
// DMA, S - 1 blocks ahead: per stage BM activation rows of 256 B (16-byte
// chunk c of row r in slot c ^ (r & 15): a ds_read_b128 cycle's 16 rows hit
// 16 distinct bank groups), BN nibble rows of 64 B (chunk c in slot
// c ^ ((r >> 2) & 3)) and BN scale rows of 16 B (the block's 4 group scales).
// Lane l takes, for group j, half h = l / 32 of its rows' group: elements
// [16h, 16h + 16) -- the low-nibble fragment for MFMA 0, the high for MFMA 1.
constexpr int Q4H_NT = 256;

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

// A lane's 8 nibble bytes of a group -> the low- and high-nibble fragments.
// m = 0x000f000f, m4 = 0x00f000f0 and o = 0x64006400 arrive in VGPRs so that
// each pair is one v_and_or_b32 (VOP3 takes no literal here).
__device__ __forceinline__ void nib16_to_h(uint2 w, uint32_t m, uint32_t m4, uint32_t o, v8h& lo, v8h& hi) {
  const uint32_t t0 = w.x >> 8, t1 = w.y >> 8;
  typedef uint32_t u4v __attribute__((ext_vector_type(4)));
  lo = __builtin_bit_cast(v8h, u4v{(w.x & m) | o, (t0 & m) | o, (w.y & m) | o, (t1 & m) | o});
  hi = __builtin_bit_cast(v8h, u4v{(w.x & m4) | o, (t0 & m4) | o, (w.y & m4) | o, (t1 & m4) | o});
}
// T16 (16 x 16 x 32 MFMA, a whole group per instruction): one dword of 4
// weight bytes (codes e0..e7 of a lane's 8-element slice) -> the fragment
// [e0,e4,e2,e6 | e1,e5,e3,e7 at 16x] with the offsets taken off: n - 8 and
// 16 (n - 8), matched by activations [x0,x4,x2,x6 | x1,x5,x3,x7 / 16].
__device__ __forceinline__ v8h nib8_to_h_c(uint32_t w, uint32_t m, uint32_t m4, uint32_t o) {
  typedef uint32_t u4v __attribute__((ext_vector_type(4)));
  const uint32_t t = w >> 8;
  return __builtin_bit_cast(v8h, u4v{(w & m) | o, (t & m) | o, (w & m4) | o, (t & m4) | o}) +
         v8h{-1032, -1032, -1032, -1032, -1152, -1152, -1152, -1152};
}
// The same fragments with the offsets taken off in the halves (packed f16
// adds, exact): n - 8 and 16 (n - 8).
__device__ __forceinline__ void nib16_to_h_c(uint2 w, uint32_t m, uint32_t m4, uint32_t o, v8h& lo, v8h& hi) {
  nib16_to_h(w, m, m4, o, lo, hi);
  lo += v8h{-1032, -1032, -1032, -1032, -1032, -1032, -1032, -1032};
  hi += v8h{-1152, -1152, -1152, -1152, -1152, -1152, -1152, -1152};
}

// PAIR: gate and up rows of the same block tile in one pass (the activation
// fragments serve both), epilogue y = silu(sx*gate) * (sx*up) -- the
// gate_up + silu_rows of nn/ffn.c:28-37.
template <int BM, int BN, int S, int WGM, int NW, bool PAIR, bool T16 = false>
__global__ __launch_bounds__(NW * 64, NW <= 8 ? 8 / NW : 1) void k_gemm_i4g_h(const uint16_t* __restrict__ xh,
                                                                const float* __restrict__ sx,
                                                                const uint8_t* __restrict__ q4,
                                                                const float* __restrict__ scl,
                                                                const uint8_t* __restrict__ q4b,
                                                                const float* __restrict__ sclb,
                                                                float* __restrict__ y, int M, int I, int O) {
  constexpr int NP = PAIR ? 2 : 1;  // weight matrices
  // stage: BM activation rows x 256 B | NP x BN nibble rows x 64 B | NP x BN scale rows x 16 B
  constexpr int SA = BM * 256, SB = BN * 64, SS = BN * 16, STAGE = SA + NP * (SB + SS);
  // 1 KiB DMA instructions per stage: A 4 rows each, B 16 rows, scales 64
  // rows; wave wv takes instruction j * NW + wv of each region (the last
  // repeats when a region's count is not a multiple of NW)
  constexpr int JA = BM / 4, JB = NP * BN / 16, JS = NP * BN / 64;
  constexpr int NA = (JA + NW - 1) / NW, NB = (JB + NW - 1) / NW, NS = (JS + NW - 1) / NW;
  constexpr int NI = NA + NB + NS;
  constexpr int WGN = NW / WGM;  // waves along the tokens x along the rows
  constexpr int MT = T16 ? 16 : 32;  // MFMA tile edge
  constexpr int TM = BM / WGM, TN = BN / WGN, FM = TM / MT, FN = TN / MT;
  constexpr int NR = T16 ? 4 : 16;   // accumulators per lane and tile
  static_assert(BN % 64 == 0 && BM % 64 == 0 && FM >= 1 && FN >= 1, "whole 1 KiB DMA rows");
  __shared__ __align__(1024) uint8_t lds[S * STAGE];
  __shared__ float s_sx[BM];
  const int tid = threadIdx.x, lane = tid % MOTY_WAVE;
  const int wv = __builtin_amdgcn_readfirstlane(tid / MOTY_WAVE);
  const int wm = wv / WGN, wn = wv % WGN;
  const int r32 = lane & 31, h = lane >> 5;
  const int mb = blockIdx.y * BM, nb = blockIdx.x * BN;
  const int ng = I / 32;
  const v4i rA = buf_rsrc(xh, (uint32_t)M * I * 2);
  const v4i rB0 = buf_rsrc(q4, (uint32_t)O * (I / 2)), rS0 = buf_rsrc(scl, (uint32_t)O * ng * 4);
  const v4i rB1 = PAIR ? buf_rsrc(q4b, (uint32_t)O * (I / 2)) : rB0;
  const v4i rS1 = PAIR ? buf_rsrc(sclb, (uint32_t)O * ng * 4) : rS0;
  // per-lane source offsets of this wave's DMAs: A chunk c of row r goes to
  // slot c ^ (r & 15), B chunk c of row r to slot c ^ ((r >> 2) & 3); B and
  // scale instructions past the first matrix's count serve the second
  uint32_t voA[NA], voB[NB], voS[NS];
  int jA[NA], jB[NB], jS[NS];
#pragma unroll
  for (int j = 0; j < NA; j++) {
    jA[j] = j * NW + wv < JA ? j * NW + wv : JA - 1;
    const int row = jA[j] * 4 + (lane >> 4);
    const int c = (lane & 15) ^ (row & 15);
    const int m = mb + row < M ? mb + row : M - 1;
    voA[j] = (uint32_t)m * (uint32_t)I * 2u + (uint32_t)c * 16u;
  }
#pragma unroll
  for (int j = 0; j < NB; j++) {
    jB[j] = j * NW + wv < JB ? j * NW + wv : JB - 1;
    const int row = (jB[j] % (BN / 16)) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((row >> 2) & 3);
    const int n = nb + row < O ? nb + row : O - 1;
    voB[j] = (uint32_t)n * (uint32_t)(I / 2) + (uint32_t)c * 16u;
  }
#pragma unroll
  for (int j = 0; j < NS; j++) {
    jS[j] = j * NW + wv < JS ? j * NW + wv : JS - 1;
    const int row = (jS[j] % (BN / 64)) * 64 + lane;
    const int n = nb + row < O ? nb + row : O - 1;
    voS[j] = (uint32_t)n * (uint32_t)ng * 4u;
  }
  const int nk = I / 128;
  const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
  auto issue = [&](int kb) {
    const uint32_t st0 = lds0 + (uint32_t)(kb % S) * STAGE;
#pragma unroll
    for (int j = 0; j < NA; j++) bdma16_to_lds(rA, voA[j], (uint32_t)kb * 256u, st0 + jA[j] * 1024);
#pragma unroll
    for (int j = 0; j < NB; j++)
      bdma16_to_lds(jB[j] < BN / 16 ? rB0 : rB1, voB[j], (uint32_t)kb * 64u, st0 + SA + jB[j] * 1024);
#pragma unroll
    for (int j = 0; j < NS; j++)
      bdma16_to_lds(jS[j] < BN / 64 ? rS0 : rS1, voS[j], (uint32_t)kb * 16u, st0 + SA + NP * SB + jS[j] * 1024);
  };
  // the tile's activation scales: the oldest load, covered by the waits below
  float sxr;
  {
    const int m = mb + tid % BM;
    sxr = sx[m < M ? m : M - 1];
  }
  uint32_t km, km4, ko;
  asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(km));
  asm volatile("v_mov_b32 %0, 0x00f000f0" : "=v"(km4));
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(ko));
  const v8h c_lo = v8h{-1032, -1032, -1032, -1032, -1032, -1032, -1032, -1032};
  const v8h c_hi = v8h{-1152, -1152, -1152, -1152, -1152, -1152, -1152, -1152};
  float acc[NP][FM][FN][NR];
#pragma unroll
  for (int p = 0; p < NP; p++)
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
#pragma unroll
        for (int r = 0; r < NR; r++) acc[p][i][j][r] = 0.f;
  // A K block's operands in registers: the activation fragments, the raw
  // nibble pairs and the scales of its 4 groups.  The next block's are read
  // from LDS while this one is unpacked and multiplied.
  struct Frags32 {
    v8h a[4][FM][2];
    uint2 b[4][NP][FN];
    float4 s[NP][FN];
  };
  // T16: one 8-half activation fragment and one nibble dword per group
  struct Frags16 {
    v8h a[4][FM];
    uint32_t b[4][NP][FN];
    float4 s[NP][FN];
  };
  using Frags = typename std::conditional<T16, Frags16, Frags32>::type;
  auto read = [&](int kb, Frags& f) {
    const uint8_t* st = lds + (kb % S) * STAGE;
    if constexpr (T16) {
      const int r16 = lane & 15, q = lane >> 4;
#pragma unroll
      for (int p = 0; p < NP; p++)
#pragma unroll
        for (int j = 0; j < FN; j++)
          f.s[p][j] = *(const float4*)(st + SA + NP * SB + p * SS + (wn * TN + j * 16 + r16) * 16);
#pragma unroll
      for (int gl = 0; gl < 4; gl++) {
#pragma unroll
        for (int i = 0; i < FM; i++) {
          const int row = wm * TM + i * 16 + r16;
          f.a[gl][i] = *(const v8h*)(st + row * 256 + (((4 * gl + q) ^ (row & 15)) * 16));
        }
#pragma unroll
        for (int p = 0; p < NP; p++)
#pragma unroll
          for (int j = 0; j < FN; j++) {
            const int row = wn * TN + j * 16 + r16;
            f.b[gl][p][j] = *(const uint32_t*)(st + SA + p * SB + row * 64 + ((gl ^ ((row >> 2) & 3)) * 16) + 4 * q);
          }
      }
      return;
    } else {
#pragma unroll
    for (int p = 0; p < NP; p++)
#pragma unroll
      for (int j = 0; j < FN; j++)
        f.s[p][j] = *(const float4*)(st + SA + NP * SB + p * SS + (wn * TN + j * 32 + r32) * 16);
#pragma unroll
    for (int gl = 0; gl < 4; gl++) {
#pragma unroll
      for (int i = 0; i < FM; i++) {
        const int row = wm * TM + i * 32 + r32;
#pragma unroll
        for (int m = 0; m < 2; m++) {
          const int c = 4 * gl + 2 * h + m;
          f.a[gl][i][m] = *(const v8h*)(st + row * 256 + ((c ^ (row & 15)) * 16));
        }
      }
#pragma unroll
      for (int p = 0; p < NP; p++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
          const int row = wn * TN + j * 32 + r32;
          f.b[gl][p][j] = *(const uint2*)(st + SA + p * SB + row * 64 + ((gl ^ ((row >> 2) & 3)) * 16) + 8 * h);
        }
    }
    }
  };
  // PAIR takes the offsets off in the weight halves (two packed adds per
  // 4 halves, shared by the FM token tiles); the single-matrix form, with
  // one weight tile per wave, computes them on the matrix core instead
  constexpr bool OFS_MFMA = !PAIR;
  auto compute = [&](const Frags& f) {
    if constexpr (T16) {
#pragma unroll
      for (int gl = 0; gl < 4; gl++) {
        v8h fb[NP][FN];
#pragma unroll
        for (int p = 0; p < NP; p++)
#pragma unroll
          for (int j = 0; j < FN; j++) fb[p][j] = nib8_to_h_c(f.b[gl][p][j], km, km4, ko);
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int p = 0; p < NP; p++)
#pragma unroll
            for (int j = 0; j < FN; j++) {
              const v4f d = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.a[gl][i], fb[p][j], v4f{}, 0, 0, 0);
              const float4 sv = f.s[p][j];
              const float s = gl == 0 ? sv.x : gl == 1 ? sv.y : gl == 2 ? sv.z : sv.w;
#pragma unroll
              for (int r = 0; r < 4; r++) acc[p][i][j][r] = __fmaf_rn(s, d[r], acc[p][i][j][r]);
            }
      }
      return;
    } else {
#pragma unroll
    for (int gl = 0; gl < 4; gl++) {
      v8h fb[NP][FN][2];
#pragma unroll
      for (int p = 0; p < NP; p++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
          if (OFS_MFMA) nib16_to_h(f.b[gl][p][j], km, km4, ko, fb[p][j][0], fb[p][j][1]);
          else nib16_to_h_c(f.b[gl][p][j], km, km4, ko, fb[p][j][0], fb[p][j][1]);
        }
#pragma unroll
      for (int i = 0; i < FM; i++) {
        // the offset -1032 sum_lo x - 72 sum_hi x of each token row
        v16f d3 = v16f{};
        if (OFS_MFMA) {
          d3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[gl][i][0], c_lo, d3, 0, 0, 0);
          d3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[gl][i][1], c_hi, d3, 0, 0, 0);
        }
#pragma unroll
        for (int p = 0; p < NP; p++)
#pragma unroll
          for (int j = 0; j < FN; j++) {
            v16f d = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[gl][i][0], fb[p][j][0], d3, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[gl][i][1], fb[p][j][1], d, 0, 0, 0);
            const float4 sv = f.s[p][j];
            const float s = gl == 0 ? sv.x : gl == 1 ? sv.y : gl == 2 ? sv.z : sv.w;
#pragma unroll
            for (int r = 0; r < 16; r++) acc[p][i][j][r] = __fmaf_rn(s, d[r], acc[p][i][j][r]);
          }
      }
    }
    }
  };
  // every stage of the ring in flight, then block 0's operands to registers
#pragma unroll
  for (int s = 0; s < S; s++) issue(s);
  MOTY_WAIT_VMCNT((S - 1) * NI);
  __syncthreads();
  Frags f0, f1;
  read(0, f0);
  for (int kb = 0; kb < nk; kb += 2) {
    // block kb + 1 has landed (the S - 2 later ones may still fly); the
    // barrier also retires every wave's reads of block kb's stage, which the
    // next DMA overwrites.  Blocks past the end read zeros, never consumed.
    MOTY_WAIT_VMCNT((S - 2) * NI);
    __syncthreads();
    issue(kb + S);
    read(kb + 1, f1);
    compute(f0);
    if (kb + 1 >= nk) break;
    MOTY_WAIT_VMCNT((S - 2) * NI);
    __syncthreads();
    issue(kb + 1 + S);
    read(kb + 2, f0);
    compute(f1);
  }
  __builtin_amdgcn_s_waitcnt(0);
  if (tid < BM) s_sx[tid] = sxr;
  __syncthreads();
  if constexpr (T16) {
    const int r16 = lane & 15, q = lane >> 4;
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int n = nb + wn * TN + j * 16 + r16;
      if (n >= O) continue;
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int ml = wm * TM + i * 16 + 4 * q + r;
          if (mb + ml >= M) continue;
          const float sv = s_sx[ml];
          y[(int64_t)(mb + ml) * O + n] =
              PAIR ? ref_silu_mul(sv * acc[0][i][j][r], sv * acc[NP - 1][i][j][r]) : sv * acc[0][i][j][r];
        }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < FN; j++) {
    const int n = nb + wn * TN + j * 32 + r32;
    if (n >= O) continue;
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int ml = wm * TM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (mb + ml >= M) continue;
        const float sv = s_sx[ml];
        y[(int64_t)(mb + ml) * O + n] =
            PAIR ? ref_silu_mul(sv * acc[0][i][j][r], sv * acc[NP - 1][i][j][r]) : sv * acc[0][i][j][r];
      }
  }
}

// The f16-MFMA GEMM (q4b/sclb non-null: PAIR, y = silu(x.q4^T) * (x.q4b^T)).
// Tiles from sweeps on MI355X at M = 256: 128 x 128 block tiles of 8 waves
// when they give at least 160 workgroups (PAIR gate + up, K = 4096, N =
// 12288: three stages 86 us, two 92, 64 x 128 93, 64 x 64 94; the 16 x 16
// form 93) -- except PAIR, where 64 x 192 tiles take over while 128 x 128
// ones would leave CUs idle and they number at least 192 (the same GEMM:
// 256 workgroups on 256 CUs against 192, 81 us against 86-91 alone; three
// stages 84, the 16 x 16 form 87-95).  Their 6 waves each take all 64 tokens
// of 32 gate and 32 up rows, so each unpacked weight fragment serves two
// token tiles: 78-80 us against 80-84 for 12 waves of 32 tokens (the FFN
// 157.0 against 159.6 us), though 6 waves leave two SIMDs a wave short;
// otherwise 64 x 64 tiles, PAIR of 4 waves in three stages, the
// single matrix in the 16 x 16 form: 8 waves of 32 x 16, four stages (down,
// K = 12288, N = 4096: 57 us; five or six stages 57.5 / 58, three 62; the
// 32 x 32 form of 4 waves 66, four stages 69, 128 x 128 113).
static bool gemm_i4g_h_big(int M, int O) { return (int64_t)((M + 127) / 128) * ((O + 127) / 128) >= 160; }
// 128 x 128 tiles give every CU a workgroup
static bool gemm_i4g_h_full(int M, int O) { return (int64_t)((M + 127) / 128) * ((O + 127) / 128) >= 256; }
int gemm_i4g_h_f8(int M, int O, bool pair) { return !pair && !gemm_i4g_h_big(M, O); }

// the f16 GEMM's 32-bit buffer offsets: activations and nibbles under 4 GiB
bool gemm_i4g_h_fits(int M, int I, int O) {
  return (I % 128) == 0 && (int64_t)M * I * 2 < ((int64_t)1 << 32) && (int64_t)O * I / 2 < ((int64_t)1 << 32);
}

int launch_gemm_i4g_h(const uint16_t* xh, const float* sx, const uint8_t* q4, const float* scl, const uint8_t* q4b,
                      const float* sclb, float* y, int M, int I, int O, hipStream_t st) {
  if ((I % 128) || ((((uintptr_t)xh) | ((uintptr_t)q4) | ((uintptr_t)scl) | ((uintptr_t)q4b) | ((uintptr_t)sclb)) & 15))
    return MOTY_EUNSUP;
  if (!gemm_i4g_h_fits(M, I, O)) return MOTY_EUNSUP;
  if (M <= 0 || O <= 0) return MOTY_OK;
  const bool big = gemm_i4g_h_big(M, O);
#define Q4H(BM, BN, S, WGM, NW, P, T16)                                                                         \
  hipLaunchKernelGGL((k_gemm_i4g_h<BM, BN, S, WGM, NW, P, T16>), dim3((O + BN - 1) / BN, (M + BM - 1) / BM),   \
                     dim3(NW * 64), 0, st, xh, sx, q4, scl, q4b, sclb, y, M, I, O)
  const bool pair192 = !gemm_i4g_h_full(M, O) && (int64_t)((M + 63) / 64) * ((O + 191) / 192) >= 192;
  if (q4b) {
    if (pair192) Q4H(64, 192, 2, 1, 6, true, false);
    else if (big) Q4H(128, 128, 3, 2, 8, true, false);
    else Q4H(64, 64, 3, 2, 4, true, false);
  } else {
    if (big) Q4H(128, 128, 2, 2, 8, false, false);
    else Q4H(64, 64, 4, 2, 8, false, true);
  }
#undef Q4H
  LAUNCH_TRY("k_gemm_i4g_h");
  return MOTY_OK;
}

// ---------------------------------------------------------------------------
// Exact f32 path, any S: one lane per (row, token); x rows staged in LDS.
constexpr int Q4F_NT = 256;

__global__ __launch_bounds__(Q4F_NT) void k_i4g_f32(const float* __restrict__ x, const uint8_t* __restrict__ q4,
                                                    const float* __restrict__ scl, float* __restrict__ y, int S,
                                                    int I, int O) {
  const int s = blockIdx.y;
  const int o = blockIdx.x * Q4F_NT + threadIdx.x;
  if (o >= O) return;
  const int ng = I / 32, rb = I / 2;
  const float* xs = x + (int64_t)s * I;
  const uint8_t* w = q4 + (int64_t)o * rb;
  const float* sp = scl + (int64_t)o * ng;
  float a = 0.f;
  for (int g = 0; g < ng; g++) {
    const int4 wb = *(const int4*)(w + g * 16);
    const uint32_t wd[4] = {(uint32_t)wb.x, (uint32_t)wb.y, (uint32_t)wb.z, (uint32_t)wb.w};
    float t[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
      // element j (bytes 0..7) and element 16+j (bytes 8..15)
      const uint32_t b0 = (wd[j >> 3] >> (8 * ((j >> 1) & 3))) & 0xffu;
      const uint32_t b1 = (wd[2 + (j >> 3)] >> (8 * ((j >> 1) & 3))) & 0xffu;
      const int n0 = (j & 1) ? (int)(b0 >> 4) : (int)(b0 & 0xf);
      const int n1 = (j & 1) ? (int)(b1 >> 4) : (int)(b1 & 0xf);
      const float p1 = xs[g * 32 + 16 + j] * (float)(n1 - 8);
      t[j] = __fmaf_rn(xs[g * 32 + j], (float)(n0 - 8), p1);
    }
    float u[8], v[4];
#pragma unroll
    for (int j = 0; j < 8; j++) u[j] = t[j + 8] + t[j];
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = u[j + 4] + u[j];
    const float r = (v[0] + v[2]) + (v[1] + v[3]);
    a = __fmaf_rn(r, sp[g], a);
  }
  y[(int64_t)s * O + o] = a;
}

// ---------------------------------------------------------------------------
// Per-row int4 (WF_I4), exact f32 path of moty_matmul_i4_s
// (nn/matmul.c:102-145) in the x86-64 AVX2 order: eight accumulator lanes,
// lane j takes elements i+j then i+8+j of each 16-element step (an FMA each),
// then simd_hsum256_f32's tree (hw/hw_avx2.h:16-20), y = a * scale.  Lane
// per (row, token), I % 16 == 0.
__global__ __launch_bounds__(256) void k_i4row_f32(const float* __restrict__ x, const uint8_t* __restrict__ q4,
                                                   const float* __restrict__ scale, float* __restrict__ y, int S,
                                                   int I, int O) {
  const int s = blockIdx.y;
  const int o = blockIdx.x * 256 + threadIdx.x;
  if (o >= O) return;
  const float* xs = x + (int64_t)s * I;
  const uint8_t* w = q4 + (int64_t)o * (I / 2);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < I; i += 16) {
    const uint2 wb = *(const uint2*)(w + i / 2);
    const uint32_t wd[2] = {wb.x, wb.y};
    float xv[16];
#pragma unroll
    for (int q = 0; q < 4; q++) *(float4*)(xv + 4 * q) = *(const float4*)(xs + i + 4 * q);
#pragma unroll
    for (int half = 0; half < 2; half++)
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int e = 8 * half + j;  // element i + e: byte e / 2, low nibble when even
        const uint32_t byte = (wd[e >> 3] >> (8 * ((e >> 1) & 3))) & 0xffu;
        const int n = (e & 1) ? (int)(byte >> 4) : (int)(byte & 15u);
        acc[j] = __fmaf_rn(xv[e], (float)(n - 8), acc[j]);
      }
  }
  const float a0 = acc[0] + acc[4], a1 = acc[1] + acc[5], a2 = acc[2] + acc[6], a3 = acc[3] + acc[7];
  const float b0 = a0 + a2, b1 = a1 + a3;
  y[(int64_t)s * O + o] = (b0 + b1) * scale[o];
}

int launch_i4row_f32(const float* x, const uint8_t* q4, const float* scale, float* y, int S, int I, int O,
                     hipStream_t st) {
  if (I % 16 || (((uintptr_t)q4) & 7) || (((uintptr_t)x) & 15)) return MOTY_EUNSUP;
  if (S <= 0 || O <= 0) return MOTY_OK;
  hipLaunchKernelGGL(k_i4row_f32, dim3((O + 255) / 256, S), dim3(256), 0, st, x, q4, scale, y, S, I, O);
  LAUNCH_TRY("k_i4row_f32");
  return MOTY_OK;
}

// NT = 256 or 512 threads: wider workgroups amortize the activation row
// (read once per workgroup) over more weight rows when I is large
template <int RW, int NGC, bool PAIR, int NT, int PD = NGC, bool XF = false>
static int go_gemv1_i4g(const float* x, const uint8_t* q4, const float* scl, const uint8_t* q4b, const float* sclb,
                        float* y, int I, int O, hipStream_t st) {
  constexpr int NM = PAIR ? 2 : 1;
  const int ng = I / 32;
  const size_t lds = (XF ? (size_t)ng * 36 * 4 : (size_t)I + (size_t)ng * 4) + (size_t)(NT / MOTY_WAVE) * NM * RW * 66 * 8;
  if (lds > 150 * 1024) return MOTY_EUNSUP;  // within the CU's 160 KiB, static arrays included
  if (lds > 64 * 1024) {
    // past 64 KiB of dynamic LDS: raise the instance's allowance on this
    // device to what this launch needs (kept when larger)
    static size_t allowed[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
      (void)hipGetLastError();
      return MOTY_EUNSUP;
    }
    if (lds > allowed[dev]) {
      if (hipFuncSetAttribute((const void*)&k_gemv1_i4g<RW, NGC, PAIR, NT, PD, XF>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
        (void)hipGetLastError();  // leave no error for a later call to find
        return MOTY_EUNSUP;
      }
      allowed[dev] = lds;
    }
  }
  const unsigned nb = (unsigned)((O + RW * (NT / MOTY_WAVE) - 1) / (RW * (NT / MOTY_WAVE)));
  hipLaunchKernelGGL((k_gemv1_i4g<RW, NGC, PAIR, NT, PD, XF>), dim3(nb), dim3(NT), lds, st, x, q4, scl, q4b, sclb, y, I, O);
  LAUNCH_TRY("k_gemv1_i4g");
  return MOTY_OK;
}

// The exact-f32 path (IDOT4 unset) for one token: the same workgroup
// structure with x kept as f32 in LDS and each lane's group sum formed in
// the reference's float order.  I % 32 == 0, I <= 16384 (x in LDS: past
// 12288 more than 64 KiB of it), 16-byte aligned x and nibbles.  PAIR (q4b):
// gate + up + SiLU.
int launch_gemv_i4g_xf(const float* x, const uint8_t* q4, const float* scl, const uint8_t* q4b, const float* sclb,
                       float* y, int I, int O, hipStream_t st) {
  if ((I % 32) || I > 16384 || ((((uintptr_t)x) | ((uintptr_t)q4) | ((uintptr_t)q4b)) & 15)) return MOTY_EUNSUP;
  if (O <= 0) return MOTY_OK;
  const int ngc = (I / 32 + 63) / 64;
  if (q4b) {
    // 2 gate + 2 up rows per wave (C3 M = 1 exact-f32 FFN 25.7 -> 25.2 us against 4 + 4)
    if (ngc <= 2) return go_gemv1_i4g<2, 2, true, 256, 1, true>(x, q4, scl, q4b, sclb, y, I, O, st);
    if (ngc <= 4) return go_gemv1_i4g<2, 4, true, 256, 1, true>(x, q4, scl, q4b, sclb, y, I, O, st);
    if (ngc <= 6) return go_gemv1_i4g<2, 6, true, 256, 1, true>(x, q4, scl, q4b, sclb, y, I, O, st);
    return go_gemv1_i4g<2, 8, true, 256, 1, true>(x, q4, scl, q4b, sclb, y, I, O, st);
  }
  if (ngc <= 2) return go_gemv1_i4g<8, 2, false, 256, 1, true>(x, q4, scl, nullptr, nullptr, y, I, O, st);
  if (ngc <= 4) return go_gemv1_i4g<4, 4, false, 256, 1, true>(x, q4, scl, nullptr, nullptr, y, I, O, st);
  // 2 rows per wave (4096 x 12288: 10.6 -> 10.2 us against 4)
  if (ngc <= 6) return go_gemv1_i4g<2, 6, false, 256, 1, true>(x, q4, scl, nullptr, nullptr, y, I, O, st);
  return go_gemv1_i4g<2, 8, false, 256, 1, true>(x, q4, scl, nullptr, nullptr, y, I, O, st);
}

int launch_gemv_i4g(const float* x, const uint8_t* q4, const float* scl, const uint8_t* q4b, const float* sclb,
                    float* y, int S, int I, int O, hipStream_t st) {
  if (S < 1 || S > 4 || (I % 64) || I > 16384) return MOTY_EUNSUP;
  if (O <= 0) return MOTY_OK;
  if (S == 1) {
    // widest instance whose LDS fits, else the next narrower one
    const int ngc = (I / 32 + 63) / 64;
    int rc = MOTY_EUNSUP;
    if (q4b) {
      // up to 2 chunks (I <= 4096): 2 gate + 2 up rows per wave (12288 x
      // 4096 pair: 12.2 us against 12.5 with 4 + 4, 14.2 with 1 + 1, 13.6
      // for 2 + 2 in 2-wave workgroups or with both chunks issued at once)
      if (ngc <= 2) rc = go_gemv1_i4g<2, 2, true, 256, 1>(x, q4, scl, q4b, sclb, y, I, O, st);
      else if (ngc <= 4) {
        rc = go_gemv1_i4g<2, 4, true, 512>(x, q4, scl, q4b, sclb, y, I, O, st);
        if (rc == MOTY_EUNSUP) rc = go_gemv1_i4g<2, 4, true, 256>(x, q4, scl, q4b, sclb, y, I, O, st);
      } else if (ngc <= 8) {
        rc = go_gemv1_i4g<1, 8, true, 512>(x, q4, scl, q4b, sclb, y, I, O, st);
        if (rc == MOTY_EUNSUP) rc = go_gemv1_i4g<1, 8, true, 256>(x, q4, scl, q4b, sclb, y, I, O, st);
      }
      return rc;
    }
    if (ngc <= 2) rc = go_gemv1_i4g<8, 2, false, 256>(x, q4, scl, nullptr, nullptr, y, I, O, st);
    else if (ngc <= 4) {
      rc = go_gemv1_i4g<4, 4, false, 512>(x, q4, scl, nullptr, nullptr, y, I, O, st);
      if (rc == MOTY_EUNSUP) rc = go_gemv1_i4g<4, 4, false, 256>(x, q4, scl, nullptr, nullptr, y, I, O, st);
    } else if (ngc <= 6) {
      // 4096 x 12288 (8B down) in a sweep of rows/wave x workgroup size x
      // chunks in flight on MI355X, graph replays over rotating weights:
      // 4 rows x 256 threads, one chunk ahead 8.0 us; two ahead 9.3, all six
      // 10.9 (the whole row's chains then run after its last byte lands);
      // 2 rows 9.6 / 10.9; 8 rows x 128 threads 10.1
      rc = go_gemv1_i4g<4, 6, false, 256, 1>(x, q4, scl, nullptr, nullptr, y, I, O, st);
    } else if (ngc <= 8) {
      rc = go_gemv1_i4g<2, 8, false, 256>(x, q4, scl, nullptr, nullptr, y, I, O, st);
    }
    if (rc != MOTY_EUNSUP) return rc;
  }
  if (q4b) return MOTY_EUNSUP;
  const unsigned nb = (unsigned)((O + Q4V_ROWS - 1) / Q4V_ROWS);
  const size_t lds = (size_t)S * I;
  switch (S) {
    case 1: hipLaunchKernelGGL(k_gemv_i4g<1>, dim3(nb), dim3(Q4V_NT), lds, st, x, q4, scl, y, I, O); break;
    case 2: hipLaunchKernelGGL(k_gemv_i4g<2>, dim3(nb), dim3(Q4V_NT), lds, st, x, q4, scl, y, I, O); break;
    case 3: hipLaunchKernelGGL(k_gemv_i4g<3>, dim3(nb), dim3(Q4V_NT), lds, st, x, q4, scl, y, I, O); break;
    default: hipLaunchKernelGGL(k_gemv_i4g<4>, dim3(nb), dim3(Q4V_NT), lds, st, x, q4, scl, y, I, O); break;
  }
  LAUNCH_TRY("k_gemv_i4g");
  return MOTY_OK;
}

int launch_gemm_i4g(const int8_t* xq, const float* sx, const uint8_t* q4, const float* scl, float* y, int M,
                    int I, int O, hipStream_t st) {
  if (I % 64) return MOTY_EUNSUP;
  if (M <= 0 || O <= 0) return MOTY_OK;
  dim3 grid((O + 63) / 64, (M + 63) / 64);
  // three K blocks in flight for long rows (I = 4096, O = 12288, M = 256:
  // 76 us vs 82 with two, in a sweep on MI355X)
  if (I >= 4096)
    hipLaunchKernelGGL(k_gemm_i4g<3>, grid, dim3(Q4M_NT), 0, st, xq, sx, q4, scl, y, M, I, O);
  else
    hipLaunchKernelGGL(k_gemm_i4g<2>, grid, dim3(Q4M_NT), 0, st, xq, sx, q4, scl, y, M, I, O);
  LAUNCH_TRY("k_gemm_i4g");
  return MOTY_OK;
}

// ---------------------------------------------------------------------------
// The exact-f32 path (IDOT4 unset) for many tokens, as a tiled GEMM on the
// vector ALUs (the reference's float order admits no matrix-core form: each
// product x*w is rounded on its own).  Workgroup tile: 64 tokens x 64 weight
// rows (PAIR: 32 gate rows and the same 32 up rows), K steps of two groups.
// Per step the workgroup stages x and the nibbles, expanded once to floats
// (n - 8, exact), in LDS; thread (tx, ty) owns tokens ty + 16i and tile rows
// tx + 16j (i, j < 4).  Each group's 32 elements sit in LDS in the order
// 8*(e % 4) + e / 4, so for jj = 0..3 the eight elements
// {jj, jj+4, jj+8, jj+12, jj+16, .., jj+28} that reduce to v[jj] of the
// reference's tree are two 16-byte reads:
//   t[j] = fma(x[j], w[j], x[16+j]*w[16+j])   (j < 16)
//   u[j] = t[j+8] + t[j];  v[j] = u[j+4] + u[j];  r = (v0 + v2) + (v1 + v3)
//   a = fma(r, scale[g], a)                  (groups in ascending order)
// -- nn/matmul.c:222-233 with FMA contraction, as the one-token kernels.
constexpr int XF_BT = 64, XF_BO = 64, XF_KE = 64;  // tokens, weight rows, elements per K step
constexpr int XF_LS = XF_KE + 4;                   // LDS row stride (floats): 16-byte reads conflict-free

__device__ __forceinline__ int xf_pos(int e) { return ((e >> 5) << 5) + 8 * (e & 3) + ((e & 31) >> 2); }

template <bool PAIR>
__global__ __launch_bounds__(256, 2) void k_gemm_i4g_xf(const float* __restrict__ x, const uint8_t* __restrict__ q4,
                                                        const float* __restrict__ scl,
                                                        const uint8_t* __restrict__ q4b,
                                                        const float* __restrict__ sclb, float* __restrict__ y,
                                                        int M, int I, int O) {
  __shared__ __align__(16) float xs[XF_BT * XF_LS];
  __shared__ __align__(16) float ws[XF_BO * XF_LS];
  __shared__ float ss[XF_BO][2];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int tb = blockIdx.y * XF_BT;
  constexpr int OR = PAIR ? XF_BO / 2 : XF_BO;  // output rows per tile
  const int ob = blockIdx.x * OR;
  const int ng = I / 32, rb = I / 2;
  // staging roles: x row tid/4, elements 16*(tid%4) .. +16 of the step;
  // weight row tid/4, nibble bytes 8*(tid%4) .. +8 (elements 16*(tid%4) ..)
  const int sr = tid >> 2, sq = tid & 3;
  const int xt = tb + sr < M ? tb + sr : M - 1;
  const float* xsrc = x + (int64_t)xt * I + 16 * sq;
  const uint8_t* wsrc;
  const float* ssrc;
  {
    int row = PAIR ? (sr & 31) : sr;
    int o = ob + row < O ? ob + row : O - 1;
    const bool up = PAIR && sr >= 32;
    wsrc = (up ? q4b : q4) + (int64_t)o * rb + 8 * sq;
    ssrc = (up ? sclb : scl) + (int64_t)o * ng;
  }
  float4 px[4];
  uint2 pw;
  float psc = 0.f;
  auto gload = [&](int k0) {
#pragma unroll
    for (int q = 0; q < 4; q++) px[q] = *(const float4*)(xsrc + k0 + 4 * q);
    pw = *(const uint2*)(wsrc + k0 / 2);
    if (sq < 2) psc = ssrc[k0 / 32 + sq];
  };
  float a[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) a[i][j] = 0.f;
  gload(0);
  for (int k0 = 0; k0 < I; k0 += XF_KE) {
    __syncthreads();  // the previous step's reads are done
    {
      const float* pv = (const float*)px;
#pragma unroll
      for (int e = 0; e < 16; e++) xs[sr * XF_LS + xf_pos(16 * sq + e)] = pv[e];
      const uint32_t wd[2] = {pw.x, pw.y};
#pragma unroll
      for (int b = 0; b < 8; b++) {
        const uint32_t byte = (wd[b >> 2] >> (8 * (b & 3))) & 0xffu;
        ws[sr * XF_LS + xf_pos(16 * sq + 2 * b)] = (float)(byte & 15u) - 8.f;
        ws[sr * XF_LS + xf_pos(16 * sq + 2 * b + 1)] = (float)(byte >> 4) - 8.f;
      }
      if (sq < 2) ss[sr][sq] = psc;
    }
    __syncthreads();
    if (k0 + XF_KE < I) gload(k0 + XF_KE);
#pragma unroll
    for (int g = 0; g < 2; g++) {
      float w02[4][4], v[4][4];
#pragma unroll
      for (int h = 0; h < 4; h++) {
        const int jj = h == 0 ? 0 : (h == 1 ? 2 : (h == 2 ? 1 : 3));  // v0, v2, then v1, v3
        float X[4][8], W[4][8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          *(float4*)&X[i][0] = *(const float4*)(xs + (ty + 16 * i) * XF_LS + 32 * g + 8 * jj);
          *(float4*)&X[i][4] = *(const float4*)(xs + (ty + 16 * i) * XF_LS + 32 * g + 8 * jj + 4);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
          *(float4*)&W[j][0] = *(const float4*)(ws + (tx + 16 * j) * XF_LS + 32 * g + 8 * jj);
          *(float4*)&W[j][4] = *(const float4*)(ws + (tx + 16 * j) * XF_LS + 32 * g + 8 * jj + 4);
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int j = 0; j < 4; j++) {
            // t at j = jj, jj+4, jj+8, jj+12: slots 0..3, partners in slots 4..7
            float t[4];
#pragma unroll
            for (int k = 0; k < 4; k++) t[k] = __fmaf_rn(X[i][k], W[j][k], X[i][k + 4] * W[j][k + 4]);
            const float vv = (t[3] + t[1]) + (t[2] + t[0]);  // u[jj+4] + u[jj]
            if (h == 0 || h == 2) v[i][j] = vv;
            else if (h == 1) w02[i][j] = v[i][j] + vv;  // v0 + v2
            else a[i][j] = __fmaf_rn(w02[i][j] + (v[i][j] + vv), ss[tx + 16 * j][g], a[i][j]);
          }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int t = tb + ty + 16 * i;
    if (t >= M) continue;
    if (PAIR) {
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int o = ob + tx + 16 * j;
        if (o < O) y[(int64_t)t * O + o] = ref_silu_mul(a[i][j], a[i][j + 2]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int o = ob + tx + 16 * j;
        if (o < O) y[(int64_t)t * O + o] = a[i][j];
      }
    }
  }
}

// many tokens, exact f32: I % 64 == 0, 16-byte aligned x and 8-byte aligned
// nibbles; PAIR (q4b): y = silu(gate) * up
int launch_gemm_i4g_xf(const float* x, const uint8_t* q4, const float* scl, const uint8_t* q4b, const float* sclb,
                       float* y, int M, int I, int O, hipStream_t st) {
  if ((I % XF_KE) || (((uintptr_t)x) & 15) || ((((uintptr_t)q4) | ((uintptr_t)q4b)) & 7)) return MOTY_EUNSUP;
  if (M <= 0 || O <= 0) return MOTY_OK;
  const int orow = q4b ? XF_BO / 2 : XF_BO;
  dim3 grid((O + orow - 1) / orow, (M + XF_BT - 1) / XF_BT);
  if (q4b)
    hipLaunchKernelGGL(k_gemm_i4g_xf<true>, grid, dim3(256), 0, st, x, q4, scl, q4b, sclb, y, M, I, O);
  else
    hipLaunchKernelGGL(k_gemm_i4g_xf<false>, grid, dim3(256), 0, st, x, q4, scl, q4b, sclb, y, M, I, O);
  LAUNCH_TRY("k_gemm_i4g_xf");
  return MOTY_OK;
}

int launch_i4g_f32(const float* x, const uint8_t* q4, const float* scl, float* y, int S, int I, int O,
                   hipStream_t st) {
  if (I % 32) return MOTY_EUNSUP;
  if (S <= 0 || O <= 0) return MOTY_OK;
  dim3 grid((O + Q4F_NT - 1) / Q4F_NT, S);
  hipLaunchKernelGGL(k_i4g_f32, grid, dim3(Q4F_NT), 0, st, x, q4, scl, y, S, I, O);
  LAUNCH_TRY("k_i4g_f32");
  return MOTY_OK;
}

}  // namespace moty
