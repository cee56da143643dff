// quant.hip -- activation and weight quantization kernels.
//
//  k_qrow_i8        per-row symmetric int8 activations  (hw/hw_quant.h:9-16)
//  k_quantize_rows  per-row int8 weights, division by s (nn/quant.c:12-33)
//  k_pack_i4g       group-32 int4 weights + f32 scales  (nn/quant.c:57-83)
//
// All three are HBM-streaming kernels: one workgroup per row, a max
// reduction (order-free, exact), then one rounding pass.  The float steps
// are the reference's: s = amax/127.f (correctly rounded divide),
// clamp, inv = 1.f/s, q = rint(x*inv); weights use w/s per element.
#include "common.h"
#include "kernels.h"

namespace moty {

template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max_f32(v);
  const int w = threadIdx.x / MOTY_WAVE, l = threadIdx.x % MOTY_WAVE;
  if (l == 0) red[w] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int i = 1; i < NT / MOTY_WAVE; i++) m = fmaxf(m, red[i]);
  __syncthreads();
  return m;
}

// One workgroup per row.  x [S][I] f32 -> q [S][I] int8, sx [S];
// xg [S][I/32] int32 group sums when non-null (requires I % 32 == 0).
template <int NT>
__global__ __launch_bounds__(NT) void k_qrow_i8(const float* __restrict__ x, int8_t* __restrict__ q,
                                                float* __restrict__ sx, int32_t* __restrict__ xg,
                                                int I, int64_t ldx, int64_t ldq) {
  __shared__ float red[NT / MOTY_WAVE];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * ldx;
  int8_t* qr = q + row * ldq;
  float amax = 0.f;
  const bool vec = ((I & 3) == 0) && ((((uintptr_t)xr) & 15) == 0) && ((((uintptr_t)qr) & 3) == 0);
  if (vec) {
    for (int i = threadIdx.x * 4; i < I; i += NT * 4) {
      float4 v = *(const float4*)(xr + i);
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
  } else {
    for (int i = threadIdx.x; i < I; i += NT) amax = fmaxf(amax, fabsf(xr[i]));
  }
  amax = block_max<NT>(amax, red);
  float s = amax / 127.f;
  if (s < 1e-12f) s = 1e-12f;
  const float inv = 1.f / s;
  if (threadIdx.x == 0) sx[row] = s;
  if (vec) {
    for (int i = threadIdx.x * 4; i < I; i += NT * 4) {
      float4 v = *(const float4*)(xr + i);
      int a = rne_int(v.x * inv), b = rne_int(v.y * inv), c = rne_int(v.z * inv), d = rne_int(v.w * inv);
      uint32_t p = (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
                   ((uint32_t)(d & 0xff) << 24);
      *(uint32_t*)(qr + i) = p;
      if (xg) {
        // 8 consecutive threads cover one group of 32
        int gsum = a + b + c + d;
        gsum += __shfl_xor(gsum, 1, 64);
        gsum += __shfl_xor(gsum, 2, 64);
        gsum += __shfl_xor(gsum, 4, 64);
        if ((threadIdx.x & 7) == 0) xg[row * (I / 32) + i / 32] = gsum;
      }
    }
  } else {
    for (int i = threadIdx.x; i < I; i += NT) qr[i] = (int8_t)rne_int(xr[i] * inv);
    if (xg) {
      __syncthreads();
      for (int g = threadIdx.x; g < I / 32; g += NT) {
        int a = 0;
        for (int j = 0; j < 32; j++) a += qr[g * 32 + j];
        xg[row * (I / 32) + g] = a;
      }
    }
  }
}

// One wave per row (I <= 1024*NC, I % 16 == 0, no group sums): lane l holds
// elements [c*1024 + 16l, +16) of every chunk c, so a wave-max is the row's
// amax and the row never waits on a workgroup barrier.  Same arithmetic as
// k_qrow_i8.
template <int NC>
__global__ __launch_bounds__(256) void k_qrow_wave(const float* __restrict__ x, int8_t* __restrict__ q,
                                                   float* __restrict__ sx, int S, int I, int64_t ldx, int64_t ldq) {
  const int lane = threadIdx.x % MOTY_WAVE;
  int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / MOTY_WAVE;
  const bool live = row < S;
  row = live ? row : S - 1;
  const float* xr = x + row * ldx;
  float4 v[NC][4];
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const int k = c * 1024 + lane * 16;
#pragma unroll
    for (int j = 0; j < 4; j++) v[c][j] = *(const float4*)(xr + (k < I ? k : 0) + 4 * j);
  }
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const bool ok = c * 1024 + lane * 16 < I;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[c][j] = sel4(ok, v[c][j]);
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[c][j].x), fabsf(v[c][j].y)), fmaxf(fabsf(v[c][j].z), fabsf(v[c][j].w))));
    }
  }
  amax = wave_max_f32(amax);
  float s = amax / 127.f;
  if (s < 1e-12f) s = 1e-12f;
  const float inv = 1.f / s;
  if (!live) return;
  if (lane == 0) sx[row] = s;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const int k = c * 1024 + lane * 16;
    if (k >= I) continue;
    int4 o;
    int* op = (int*)&o;
#pragma unroll
    for (int j = 0; j < 4; j++)
      op[j] = (int)((uint32_t)(rne_int(v[c][j].x * inv) & 0xff) | ((uint32_t)(rne_int(v[c][j].y * inv) & 0xff) << 8) |
                    ((uint32_t)(rne_int(v[c][j].z * inv) & 0xff) << 16) |
                    ((uint32_t)(rne_int(v[c][j].w * inv) & 0xff) << 24));
    *(int4*)(q + row * ldq + k) = o;
  }
}

// Weight rows: s = amax/qmax clamped at 1e-8, v = clip(rint(w/s)).
template <int NT>
__global__ __launch_bounds__(NT) void k_quantize_rows(const float* __restrict__ w, int8_t* __restrict__ q,
                                                      float* __restrict__ scale, int I, int bits) {
  __shared__ float red[NT / MOTY_WAVE];
  const int64_t row = blockIdx.x;
  const float* wr = w + row * (int64_t)I;
  int8_t* qr = q + row * (int64_t)I;
  const int qmax = (1 << (bits - 1)) - 1;
  float amax = 0.f;
  for (int i = threadIdx.x; i < I; i += NT) amax = fmaxf(amax, fabsf(wr[i]));
  amax = block_max<NT>(amax, red);
  float s = amax / (float)qmax;
  if (s < 1e-8f) s = 1e-8f;
  if (threadIdx.x == 0) scale[row] = s;
  for (int i = threadIdx.x; i < I; i += NT) {
    int v = rne_int(wr[i] / s);
    v = v > qmax ? qmax : v;
    v = v < -qmax - 1 ? -qmax - 1 : v;
    qr[i] = (int8_t)v;
  }
}

// The same for rows of I % 4 == 0, I <= 4 * NT * NV (16-byte aligned rows):
// the row is read once, by 16-byte loads kept in registers, and written as
// 4-byte words -- one pass over HBM where the kernel above reads every
// element twice with 4-byte loads and writes single bytes.
template <int NT, int NV>
__global__ __launch_bounds__(NT) void k_quantize_rows_v(const float* __restrict__ w, int8_t* __restrict__ q,
                                                        float* __restrict__ scale, int I, int bits) {
  __shared__ float red[NT / MOTY_WAVE];
  const int64_t row = blockIdx.x;
  const float* wr = w + row * (int64_t)I;
  int8_t* qr = q + row * (int64_t)I;
  const int qmax = (1 << (bits - 1)) - 1;
  float4 v[NV];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = (threadIdx.x + j * NT) * 4;
    v[j] = i < I ? *(const float4*)(wr + i) : float4{0.f, 0.f, 0.f, 0.f};
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
  }
  amax = block_max<NT>(amax, red);
  float s = amax / (float)qmax;
  if (s < 1e-8f) s = 1e-8f;
  if (threadIdx.x == 0) scale[row] = s;
  auto q1 = [&](float x) {
    int c = rne_int(x / s);
    c = c > qmax ? qmax : c;
    c = c < -qmax - 1 ? -qmax - 1 : c;
    return (uint32_t)c & 0xffu;
  };
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int i = (threadIdx.x + j * NT) * 4;
    if (i < I) *(uint32_t*)(qr + i) = q1(v[j].x) | (q1(v[j].y) << 8) | (q1(v[j].z) << 16) | (q1(v[j].w) << 24);
  }
}

// Group-32 packing for I % 32 == 0 (16-byte aligned w, q4): a workgroup of
// NT threads takes NT consecutive groups -- a contiguous NT * 128 bytes of w
// -- into LDS by 16-byte loads, each thread then packs its own group as
// k_pack_i4g does and writes its 16 code bytes and its scale.  Group g
// sits at word 33 * g in LDS, so the lanes reading element j of their
// groups hit different banks.
template <int NT>
__global__ __launch_bounds__(NT) void k_pack_i4g32(const float* __restrict__ w, uint8_t* __restrict__ q4,
                                                   float* __restrict__ scale, int64_t ngt) {
  __shared__ float ws[NT * 33];
  const int64_t g0 = (int64_t)blockIdx.x * NT;
  const int ng = ngt - g0 < NT ? (int)(ngt - g0) : NT;
  const float* src = w + g0 * 32;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int u = threadIdx.x + j * NT;  // float4 unit of the block
    if (u < ng * 8) {
      const float4 t = *(const float4*)(src + 4 * u);
      float* d = ws + (u >> 3) * 33 + (u & 7) * 4;
      d[0] = t.x;
      d[1] = t.y;
      d[2] = t.z;
      d[3] = t.w;
    }
  }
  __syncthreads();
  if ((int)threadIdx.x >= ng) return;
  const float* gw = ws + threadIdx.x * 33;
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(gw[i]));
  float s = amax / 7.f;
  if (s < 1e-8f) s = 1e-8f;
  const int64_t g = g0 + threadIdx.x;
  scale[g] = s;
  uint32_t out[4];
#pragma unroll
  for (int b = 0; b < 4; b++) {
    uint32_t word = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      int v0 = rne_int(gw[8 * b + 2 * k] / s);
      v0 = v0 > 7 ? 7 : (v0 < -8 ? -8 : v0);
      int v1 = rne_int(gw[8 * b + 2 * k + 1] / s);
      v1 = v1 > 7 ? 7 : (v1 < -8 ? -8 : v1);
      word |= (uint32_t)((v0 + 8) | ((v1 + 8) << 4)) << (8 * k);
    }
    out[b] = word;
  }
  *(uint4*)(q4 + g * 16) = uint4{out[0], out[1], out[2], out[3]};
}

// One thread per (row, group).  Odd trailing elements pair with a zero code.
__global__ void k_pack_i4g(const float* __restrict__ w, uint8_t* __restrict__ q4, float* __restrict__ scale,
                           int O, int I, int gs) {
  const int ng = (I + gs - 1) / gs, rb = (I + 1) / 2;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)O * ng) return;
  const int64_t o = t / ng;
  const int g = (int)(t % ng);
  const float* wr = w + o * I;
  const int base = g * gs;
  const int glen = base + gs > I ? I - base : gs;
  float amax = 0.f;
  for (int i = base; i < base + glen; i++) amax = fmaxf(amax, fabsf(wr[i]));
  float s = amax / 7.f;
  if (s < 1e-8f) s = 1e-8f;
  scale[o * ng + g] = s;
  uint8_t* qr = q4 + o * rb;
  for (int i = base; i < base + glen; i += 2) {
    int v0 = rne_int(wr[i] / s);
    v0 = v0 > 7 ? 7 : (v0 < -8 ? -8 : v0);
    int v1 = 0;
    if (i + 1 < base + glen) {
      v1 = rne_int(wr[i + 1] / s);
      v1 = v1 > 7 ? 7 : (v1 < -8 ? -8 : v1);
    }
    qr[i >> 1] = (uint8_t)((v0 + 8) | ((v1 + 8) << 4));
  }
}

// Several qrow_i8 jobs in one launch (each I <= 4096, I % 16 == 0, rows
// dense, 16-byte aligned): workgroups [b0[j], b0[j+1]) take job j, four rows
// each, one wave per row with the arithmetic of k_qrow_wave.  Only the
// chunks a job's rows have are loaded (the branch is wave-uniform).
__global__ __launch_bounds__(256) void k_qrow_multi(QrowJobs jb) {
  int j = 0;
#pragma unroll
  for (int i = 1; i < QROW_MAX_JOBS; i++)
    if (i < jb.n && (int)blockIdx.x >= jb.b0[i]) j = i;
  const int S = jb.S[j], I = jb.I[j];
  const int lane = threadIdx.x % MOTY_WAVE;
  int64_t row = (int64_t)(blockIdx.x - jb.b0[j]) * 4 + threadIdx.x / MOTY_WAVE;
  const bool live = row < S;
  row = live ? row : S - 1;
  const float* xr = jb.x[j] + row * I;
  const int nc = (I + 1023) / 1024;
  float4 v[4][4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const int k = c * 1024 + lane * 16;
    if (c < nc) {
#pragma unroll
      for (int q = 0; q < 4; q++) v[c][q] = *(const float4*)(xr + (k < I ? k : 0) + 4 * q);
    }
  }
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const bool ok = c < nc && c * 1024 + lane * 16 < I;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      v[c][q] = sel4(ok, v[c][q]);
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[c][q].x), fabsf(v[c][q].y)), fmaxf(fabsf(v[c][q].z), fabsf(v[c][q].w))));
    }
  }
  amax = wave_max_f32(amax);
  float s = amax / 127.f;
  if (s < 1e-12f) s = 1e-12f;
  const float inv = 1.f / s;
  if (!live) return;
  if (lane == 0) jb.sx[j][row] = s;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const int k = c * 1024 + lane * 16;
    if (c >= nc || k >= I) continue;
    int4 o;
    int* op = (int*)&o;
#pragma unroll
    for (int q = 0; q < 4; q++)
      op[q] = (int)((uint32_t)(rne_int(v[c][q].x * inv) & 0xff) | ((uint32_t)(rne_int(v[c][q].y * inv) & 0xff) << 8) |
                    ((uint32_t)(rne_int(v[c][q].z * inv) & 0xff) << 16) |
                    ((uint32_t)(rne_int(v[c][q].w * inv) & 0xff) << 24));
    *(int4*)(jb.q[j] + row * I + k) = o;
  }
}

int launch_qrow_multi(QrowJobs jb, hipStream_t st) {
  if (jb.n < 1 || jb.n > QROW_MAX_JOBS) return MOTY_EINVAL;
  int nb = 0;
  for (int j = 0; j < jb.n; j++) {
    if (jb.S[j] < 0 || jb.I[j] <= 0 || jb.I[j] > 4096 || (jb.I[j] % 16)) return MOTY_EUNSUP;
    if (jb.S[j] > 0 && (!jb.x[j] || !jb.q[j] || !jb.sx[j] || ((((uintptr_t)jb.x[j]) | ((uintptr_t)jb.q[j])) & 15)))
      return MOTY_EUNSUP;
    jb.b0[j] = nb;
    nb += (jb.S[j] + 3) / 4;
  }
  for (int j = jb.n; j <= QROW_MAX_JOBS; j++) jb.b0[j] = nb;
  if (nb == 0) return MOTY_OK;
  hipLaunchKernelGGL(k_qrow_multi, dim3((unsigned)nb), dim3(256), 0, st, jb);
  LAUNCH_TRY("k_qrow_multi");
  return MOTY_OK;
}

int launch_qrow_i8(const float* x, int8_t* q, float* sx, int32_t* xg, int S, int I, int64_t ldx,
                   int64_t ldq, hipStream_t st) {
  if (S <= 0) return MOTY_OK;
  if (xg && (I % 32)) return MOTY_EINVAL;
  const bool wave_ok = !xg && I <= 4096 && (I % 16) == 0 && (ldx % 4) == 0 && (ldq % 16) == 0 &&
                       (((uintptr_t)x) & 15) == 0 && (((uintptr_t)q) & 15) == 0;
  if (wave_ok) {
    const unsigned nb = (unsigned)((S + 3) / 4);
    switch ((I + 1023) / 1024) {
      case 1: hipLaunchKernelGGL(k_qrow_wave<1>, dim3(nb), dim3(256), 0, st, x, q, sx, S, I, ldx, ldq); break;
      case 2: hipLaunchKernelGGL(k_qrow_wave<2>, dim3(nb), dim3(256), 0, st, x, q, sx, S, I, ldx, ldq); break;
      case 3: hipLaunchKernelGGL(k_qrow_wave<3>, dim3(nb), dim3(256), 0, st, x, q, sx, S, I, ldx, ldq); break;
      default: hipLaunchKernelGGL(k_qrow_wave<4>, dim3(nb), dim3(256), 0, st, x, q, sx, S, I, ldx, ldq); break;
    }
    LAUNCH_TRY("k_qrow_wave");
    return MOTY_OK;
  }
  hipLaunchKernelGGL(k_qrow_i8<256>, dim3(S), dim3(256), 0, st, x, q, sx, xg, I, ldx, ldq);
  LAUNCH_TRY("k_qrow_i8");
  return MOTY_OK;
}

// qrow_i8 (hw/hw_quant.h:9-16) with the codes written as f16 -- exact, they
// are integers in [-127, 127] -- for the f16-MFMA grouped-int4 GEMM.  Each
// run of 16 codes c0..c15 is stored as the two 8-code fragments that GEMM
// multiplies against the low and the high nibbles of the same 8 weight
// bytes: [c0, c4, c2, c6, c8, c12, c10, c14] and [c1, c5, c3, c7, c9, c13,
// c11, c15] / 16 (a k-permutation shared by both operands; the division by
// 16 is exact and matches the high nibbles' 16x weight halves).  F8: the
// fragments of the 16 x 16 x 32 form, per 8 codes: [c0, c4, c2, c6, c1, c5,
// c3, c7] with the last four / 16.  One workgroup per row, the row held in
// registers: NU runs per thread (run t + NT*j).
template <int NT, int NU, bool F8>
__global__ __launch_bounds__(NT) void k_qrow_f16p(const float* __restrict__ x, uint16_t* __restrict__ xh,
                                                  float* __restrict__ sx, int I) {
  __shared__ float red[NT / MOTY_WAVE];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * I;
  const int nrun = I / 16;
  float4 v[NU][4];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NU; j++) {
    const int r = threadIdx.x + NT * j;
    const int rc = r < nrun ? r : 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      v[j][q] = sel4(r < nrun, *(const float4*)(xr + 16 * rc + 4 * q));
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j][q].x), fabsf(v[j][q].y)), fmaxf(fabsf(v[j][q].z), fabsf(v[j][q].w))));
    }
  }
  amax = block_max<NT>(amax, red);
  float s = amax / 127.f;
  if (s < 1e-12f) s = 1e-12f;
  const float inv = 1.f / s;
  if (threadIdx.x == 0) sx[row] = s;
  auto hb = [](float c) { return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)c); };
#pragma unroll
  for (int j = 0; j < NU; j++) {
    const int r = threadIdx.x + NT * j;
    if (r >= nrun) break;
    float c[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      c[4 * q] = (float)rne_int(v[j][q].x * inv);
      c[4 * q + 1] = (float)rne_int(v[j][q].y * inv);
      c[4 * q + 2] = (float)rne_int(v[j][q].z * inv);
      c[4 * q + 3] = (float)rne_int(v[j][q].w * inv);
    }
    const float k = 0.0625f;
    uint4 lo, hi;
    if (F8) {
      lo = uint4{hb(c[0]) | (hb(c[4]) << 16), hb(c[2]) | (hb(c[6]) << 16), hb(c[1] * k) | (hb(c[5] * k) << 16),
                 hb(c[3] * k) | (hb(c[7] * k) << 16)};
      hi = uint4{hb(c[8]) | (hb(c[12]) << 16), hb(c[10]) | (hb(c[14]) << 16), hb(c[9] * k) | (hb(c[13] * k) << 16),
                 hb(c[11] * k) | (hb(c[15] * k) << 16)};
    } else {
      lo = uint4{hb(c[0]) | (hb(c[4]) << 16), hb(c[2]) | (hb(c[6]) << 16), hb(c[8]) | (hb(c[12]) << 16),
                 hb(c[10]) | (hb(c[14]) << 16)};
      hi = uint4{hb(c[1] * k) | (hb(c[5] * k) << 16), hb(c[3] * k) | (hb(c[7] * k) << 16),
                 hb(c[9] * k) | (hb(c[13] * k) << 16), hb(c[11] * k) | (hb(c[15] * k) << 16)};
    }
    *(uint4*)(xh + row * I + 16 * r) = lo;
    *(uint4*)(xh + row * I + 16 * r + 8) = hi;
  }
}

int launch_qrow_f16p(const float* x, uint16_t* xh, float* sx, int S, int I, int f8, hipStream_t st) {
  if (S <= 0) return MOTY_OK;
  if ((I % 16) || (((uintptr_t)x) & 15) || (((uintptr_t)xh) & 15)) return MOTY_EUNSUP;
  const int runs = (I / 16 + 255) / 256;
#define QF(NU)                                                                                          \
  if (f8) hipLaunchKernelGGL((k_qrow_f16p<256, NU, true>), dim3(S), dim3(256), 0, st, x, xh, sx, I); \
  else hipLaunchKernelGGL((k_qrow_f16p<256, NU, false>), dim3(S), dim3(256), 0, st, x, xh, sx, I)
  if (runs <= 1) QF(1);
  else if (runs <= 2) QF(2);
  else if (runs <= 4) QF(4);
  else return MOTY_EUNSUP;
#undef QF
  LAUNCH_TRY("k_qrow_f16p");
  return MOTY_OK;
}

// Per-row int4 weights (nn/quant.c:34-55): s = amax/7 clamped at 1e-8,
// v = clip(rint(w/s), -8, 7), even element in the low nibble.  One
// workgroup per row.
template <int NT>
__global__ __launch_bounds__(NT) void k_pack_i4row(const float* __restrict__ w, uint8_t* __restrict__ q4,
                                                   float* __restrict__ scale, int I) {
  __shared__ float red[NT / MOTY_WAVE];
  const int64_t row = blockIdx.x;
  const float* wr = w + row * (int64_t)I;
  uint8_t* qr = q4 + row * (int64_t)((I + 1) / 2);
  float amax = 0.f;
  for (int i = threadIdx.x; i < I; i += NT) amax = fmaxf(amax, fabsf(wr[i]));
  amax = block_max<NT>(amax, red);
  float s = amax / 7.f;
  if (s < 1e-8f) s = 1e-8f;
  if (threadIdx.x == 0) scale[row] = s;
  for (int i = 2 * threadIdx.x; i < I; i += 2 * NT) {
    int v0 = rne_int(wr[i] / s);
    v0 = v0 > 7 ? 7 : (v0 < -8 ? -8 : v0);
    int v1 = 0;
    if (i + 1 < I) {
      v1 = rne_int(wr[i + 1] / s);
      v1 = v1 > 7 ? 7 : (v1 < -8 ? -8 : v1);
    }
    qr[i >> 1] = (uint8_t)((v0 + 8) | ((v1 + 8) << 4));
  }
}

int launch_pack_i4row(const float* w, uint8_t* q4, float* scale, int O, int I, hipStream_t st) {
  if (O <= 0) return MOTY_OK;
  hipLaunchKernelGGL(k_pack_i4row<256>, dim3(O), dim3(256), 0, st, w, q4, scale, I);
  LAUNCH_TRY("k_pack_i4row");
  return MOTY_OK;
}

// 16 per-row int4 codes (8 bytes, element 2j in the low nibble of byte j)
// -> the 16 int8 values n - 8 that dot_i4i8 multiplies (hw/hw_scalar.h:14-22).
__device__ __forceinline__ int4 i4row_expand16(uint2 w) {
  const uint32_t wd[2] = {w.x, w.y};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const uint32_t lo = wd[k] & 0x0f0f0f0fu, hi = (wd[k] >> 4) & 0x0f0f0f0fu;
    const uint32_t e01 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // lo0 hi0 lo1 hi1
    const uint32_t e23 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // lo2 hi2 lo3 hi3
    // n - 8 per byte without carries: (n + 0x78) ^ 0x80
    o[2 * k] = (e01 + 0x78787878u) ^ 0x80808080u;
    o[2 * k + 1] = (e23 + 0x78787878u) ^ 0x80808080u;
  }
  return int4{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
}

// moty_matmul_i4_s with IDOT4 (nn/matmul.c:75-86, i4_idot_rows :91-99):
//     y[s*O+o] = scale[o] * sx[s] * (float)dot_i4i8(q4 row o, xq[s], I)
// straight from the nibbles, no int8 copy of the weights.  A wave owns one
// row; lane l covers elements [c*1024 + 16l, +16) of chunk c (8 nibble bytes,
// 512 B per wave-load, coalesced).  Tokens go in blocks of four; a row is
// re-read once per block, from L2 after the first.  I % 16 == 0 (every
// covered 16-element run is whole), q4 8-byte and xq 16-byte aligned.
__global__ __launch_bounds__(256) void k_i4row_idot(const int8_t* __restrict__ xq, const float* __restrict__ sx,
                                                    const uint8_t* __restrict__ q4, const float* __restrict__ scale,
                                                    float* __restrict__ y, int S, int I, int O) {
  const int lane = threadIdx.x % MOTY_WAVE;
  const int o = blockIdx.x * 4 + threadIdx.x / MOTY_WAVE;
  if (o >= O) return;
  const uint8_t* wr = q4 + (int64_t)o * (I / 2);
  const float so = scale[o];
  for (int s0 = 0; s0 < S; s0 += 4) {
    int acc[4] = {0, 0, 0, 0};
    for (int k = lane * 16; k < I; k += 1024) {
      const int4 w = i4row_expand16(*(const uint2*)(wr + k / 2));
#pragma unroll
      for (int j = 0; j < 4; j++)
        if (s0 + j < S) acc[j] = dot16(w, *(const int4*)(xq + (int64_t)(s0 + j) * I + k), acc[j]);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int a = wave_sum_i32(acc[j]);
      if (lane == 0 && s0 + j < S) y[(int64_t)(s0 + j) * O + o] = so * sx[s0 + j] * (float)a;
    }
  }
}

int launch_i4row_idot(const int8_t* xq, const float* sx, const uint8_t* q4, const float* scale, float* y, int S,
                      int I, int O, hipStream_t st) {
  if (S <= 0 || O <= 0) return MOTY_OK;
  if (I % 16 || (((uintptr_t)q4) & 7) || (((uintptr_t)xq) & 15)) return MOTY_EUNSUP;
  hipLaunchKernelGGL(k_i4row_idot, dim3((unsigned)((O + 3) / 4)), dim3(256), 0, st, xq, sx, q4, scale, y, S, I, O);
  LAUNCH_TRY("k_i4row_idot");
  return MOTY_OK;
}

int launch_quantize_rows(const float* w, int8_t* q, float* scale, int O, int I, int bits, hipStream_t st) {
  if (O <= 0) return MOTY_OK;
  if ((I % 4) == 0 && I <= 16384 && !(((uintptr_t)w) & 15) && !(((uintptr_t)q) & 3)) {
    // one pass in registers: float4 units per thread as the row needs
    const int nv = (I / 4 + 255) / 256;
#define QV(NV)                                                                                             \
  if (nv <= NV) {                                                                                           \
    hipLaunchKernelGGL((k_quantize_rows_v<256, NV>), dim3(O), dim3(256), 0, st, w, q, scale, I, bits);       \
    LAUNCH_TRY("k_quantize_rows_v");                                                                        \
    return MOTY_OK;                                                                                         \
  }
    QV(1) QV(2) QV(4) QV(8) QV(16)
#undef QV
  }
  hipLaunchKernelGGL(k_quantize_rows<256>, dim3(O), dim3(256), 0, st, w, q, scale, I, bits);
  LAUNCH_TRY("k_quantize_rows");
  return MOTY_OK;
}

int launch_pack_i4g(const float* w, uint8_t* q4, float* scale, int O, int I, int gs, hipStream_t st) {
  const int ng = (I + gs - 1) / gs;
  const int64_t n = (int64_t)O * ng;
  if (n <= 0) return MOTY_OK;
  if (gs == 32 && (I % 32) == 0 && !(((uintptr_t)w) & 15) && !(((uintptr_t)q4) & 15)) {
    // rows are whole groups: the groups of the matrix are consecutive 128-byte runs of w
    hipLaunchKernelGGL(k_pack_i4g32<256>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, q4, scale, n);
    LAUNCH_TRY("k_pack_i4g32");
    return MOTY_OK;
  }
  hipLaunchKernelGGL(k_pack_i4g, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, q4, scale, O, I, gs);
  LAUNCH_TRY("k_pack_i4g");
  return MOTY_OK;
}

}  // namespace moty
