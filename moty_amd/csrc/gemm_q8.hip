// gemm_q8.hip -- Q8_0 prefill GEMM on int8 MFMA (v_mfma_i32_16x16x64_i8).
//
// Reference: moty_matmul_q_s (nn/matmul.c:51-66) for S > 1 token rows:
//     y[s*O+o] = (scale[o]*sx[s]) * (float)sum_i W[o][i]*xq[s][i]
// The int32 accumulation is exact in any order, so the MFMA result equals
// the reference's VPDPBUSD chains bit for bit; the epilogue keeps the
// reference's two multiplies.
//
// Both operands are K-contiguous (xq [S][I] token-major, W [O][I] row-major),
// which is exactly the MFMA operand layout: lane l of a 16x16x64 step holds
// 16 consecutive k-bytes of row (l % 16) at k offset 16*(l / 16), for A
// (tokens) and B (weight rows) alike.  Fragments load straight from global
// memory (16 B per lane, 64 B contiguous per row) with the next K step
// prefetched while the current one runs on the matrix cores.
#include "common.h"
#include "kernels.h"

namespace moty {

constexpr int GM_NT = 256;  // 4 waves, 2x2 over the block tile
constexpr int GM_BM = 64, GM_BN = 64, GM_BK = 64;

__device__ __forceinline__ int4 ld16(const int8_t* p, bool ok) {
  return ok ? *(const int4*)p : int4{0, 0, 0, 0};
}

// One problem: y[M][O] from xq[M][K] (ld = K), W[O][K]; K % 16 == 0.
__global__ __launch_bounds__(GM_NT) void k_gemm_q8(const int8_t* __restrict__ xq, const float* __restrict__ sx,
                                                   const int8_t* __restrict__ W, const float* __restrict__ scale,
                                                   float* __restrict__ y, int M, int K, int O) {
  const int lane = threadIdx.x % MOTY_WAVE, wv = threadIdx.x / MOTY_WAVE;
  const int wm = wv >> 1, wn = wv & 1;
  // blockIdx.x walks N tiles fastest so consecutive blocks share the same
  // activation rows (hot in L2) while streaming different weight rows
  const int m0 = blockIdx.y * GM_BM + wm * 32;
  const int n0 = blockIdx.x * GM_BN + wn * 32;
  const int r16 = lane & 15, kq = (lane >> 4) * 16;

  const int8_t* ap[2];
  const int8_t* bp[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    int m = m0 + i * 16 + r16;
    m = m < M ? m : M - 1;
    ap[i] = xq + (int64_t)m * K + kq;
    int n = n0 + i * 16 + r16;
    n = n < O ? n : O - 1;
    bp[i] = W + (int64_t)n * K + kq;
  }
  v4i acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = v4i{0, 0, 0, 0};

  int4 a[2], b[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    a[i] = ld16(ap[i], kq < K);
    b[i] = ld16(bp[i], kq < K);
  }
  for (int k0 = 0; k0 < K; k0 += GM_BK) {
    int4 an[2], bn[2];
    const int kn = k0 + GM_BK;
    const bool ok = (kn + kq) < K;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      an[i] = ld16(ap[i] + kn, ok);
      bn[i] = ld16(bp[i] + kn, ok);
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(*(v4i*)&a[i], *(v4i*)&b[j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; i++) {
      a[i] = an[i];
      b[i] = bn[i];
    }
  }
  // D layout: lane l holds column (l % 16), rows 4*(l / 16) + r
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int n = n0 + j * 16 + r16;
    if (n >= O) continue;
    const float sc = scale[n];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + i * 16 + (lane >> 4) * 4 + r;
        if (m < M) y[(int64_t)m * O + n] = (sc * sx[m]) * (float)acc[i][j][r];
      }
  }
}

int launch_gemm_q8(const int8_t* xq, const float* sx, const int8_t* W, const float* scale, float* y, int M,
                   int K, int O, hipStream_t st) {
  if (K % 16) return MOTY_EUNSUP;
  if (M <= 0 || O <= 0) return MOTY_OK;
  dim3 grid((O + GM_BN - 1) / GM_BN, (M + GM_BM - 1) / GM_BM);
  hipLaunchKernelGGL(k_gemm_q8, grid, dim3(GM_NT), 0, st, xq, sx, W, scale, y, M, K, O);
  LAUNCH_TRY("k_gemm_q8");
  return MOTY_OK;
}

}  // namespace moty
