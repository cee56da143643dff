// ops.hip -- the f32 router matmul and the SiLU row op as standalone kernels.
//
//  k_matmul_f32  moty_matmul (nn/matmul.c:15-27) with dot_f32 in the AVX512
//                lane order (hw/hw_avx512.h:231-243): one 32-lane half-wave
//                per output, 32 FMA chains, the reduce_add tree, FMA tail.
//  k_silu_mul    g = (g / (1 + expf(-g))) * u   (hw/hw_ops.h:19-21)
#include "common.h"
#include "kernels.h"

namespace moty {

constexpr int MF_NT = 256;

__global__ __launch_bounds__(MF_NT) void k_matmul_f32(const float* __restrict__ x, const float* __restrict__ W,
                                                      float* __restrict__ y, int S, int I, int O) {
  const int64_t h = (int64_t)blockIdx.x * (MF_NT / 32) + threadIdx.x / 32;  // one output per half-wave
  const bool live = h < (int64_t)S * O;
  const int64_t hh = live ? h : 0;
  const int s = (int)(hh / O), o = (int)(hh % O);
  const float r = dot_f32_half(x + (int64_t)s * I, W + (int64_t)o * I, I);
  if (live && (threadIdx.x % 32) == 0) y[(int64_t)s * O + o] = r;
}

__global__ void k_silu_mul(float* __restrict__ g, const float* __restrict__ u, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) g[i] = ref_silu_mul(g[i], u[i]);
}

// silu_rows over a row-fused gate_up output (nn/ffn.c:8-24): h [S][I] =
// silu(gu[s][i]) * gu[s][I + i]
__global__ void k_silu_rows(float* __restrict__ h, const float* __restrict__ gu, int S, int I) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)S * I) return;
  const int64_t s = i / I, c = i % I;
  h[i] = ref_silu_mul(gu[s * 2 * I + c], gu[s * 2 * I + I + c]);
}

__global__ void k_expf(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = ref_expf(x[i]);
}

// moty_softmax_row (nn/norm.c:10 -> hw/hw_ops.h:22-26) over S rows of n:
// max (order-free), expf(x - m), serial sum in one lane, divide.
__global__ void k_softmax_rows(float* __restrict__ x, int n) {
  float* r = x + (int64_t)blockIdx.x * n;
  const int lane = threadIdx.x;
  float m = -1e30f;
  for (int i = lane; i < n; i += MOTY_WAVE) m = r[i] > m ? r[i] : m;
  m = wave_max_f32(m);
  for (int i = lane; i < n; i += MOTY_WAVE) r[i] = ref_expf(r[i] - m);
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  float s = 0.f;
  if (lane == 0)
    for (int i = 0; i < n; i++) s += r[i];
  s = __shfl(s, 0, 64);
  for (int i = lane; i < n; i += MOTY_WAVE) r[i] = r[i] / s;
}

int launch_expf(const float* x, float* y, int64_t n, hipStream_t st) {
  if (n <= 0) return MOTY_OK;
  hipLaunchKernelGGL(k_expf, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, y, n);
  LAUNCH_TRY("k_expf");
  return MOTY_OK;
}

int launch_softmax_rows(float* x, int S, int n, hipStream_t st) {
  if (S <= 0 || n <= 0) return MOTY_OK;
  hipLaunchKernelGGL(k_softmax_rows, dim3(S), dim3(MOTY_WAVE), 0, st, x, n);
  LAUNCH_TRY("k_softmax_rows");
  return MOTY_OK;
}

int launch_matmul_f32(const float* x, const float* W, float* y, int S, int I, int O, hipStream_t st) {
  const int64_t n = (int64_t)S * O;
  if (n <= 0) return MOTY_OK;
  const int64_t nb = (n + MF_NT / 32 - 1) / (MF_NT / 32);
  hipLaunchKernelGGL(k_matmul_f32, dim3((unsigned)nb), dim3(MF_NT), 0, st, x, W, y, S, I, O);
  LAUNCH_TRY("k_matmul_f32");
  return MOTY_OK;
}

int launch_silu_rows(float* h, const float* gu, int S, int I, hipStream_t st) {
  const int64_t n = (int64_t)S * I;
  if (n <= 0) return MOTY_OK;
  hipLaunchKernelGGL(k_silu_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, h, gu, S, I);
  LAUNCH_TRY("k_silu_rows");
  return MOTY_OK;
}

int launch_silu_mul(float* g, const float* u, int64_t n, hipStream_t st) {
  if (n <= 0) return MOTY_OK;
  hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, u, n);
  LAUNCH_TRY("k_silu_mul");
  return MOTY_OK;
}

}  // namespace moty
