// gemv_q8.hip -- Q8_0 GEMV for decode (S <= 4 token rows).
//
// Reference: moty_matmul_q_s (nn/matmul.c:51-66) -> q8_idot_rows (:29-36)
// -> dot_i8i8 (hw/hw_avx512.h:24-54):
//     xq[s] = qrow_i8(x[s]);  y[s*O+o] = (scale[o]*sx[s]) * (float)dot(W[o], xq[s])
//
// MI355X design (HBM-bound, one pass over W).  S = 1 with I <= 4096 takes
// k_gemv1_q8 (activations quantized per wave in registers) or, for large
// matrices, k_gemv1_q8_lds (quantized once per workgroup into LDS); otherwise:
//  * a wave owns RPW weight rows; each lane streams 16 contiguous bytes per
//    1 KiB chunk of a row (global_load_dwordx4, fully coalesced), up to four
//    chunks per row in flight;
//  * the block issues its first weight loads, then quantizes the S
//    activation rows into LDS while those loads are in flight (every block
//    re-derives the same int8 activations: the quantization is a pure
//    function of x, so this is bit-identical to quantizing once);
//  * int8 dot products on v_dot4_i32_i8, int32 wave reduction (exact);
//  * epilogue: (scale*sx)*float(acc), two plain multiplies, as the reference.
// PAIR mode (decode FFN gate+up): the wave reads row o of W and of W2 and
// writes silu(g)*u (hw/hw_ops.h:19-21) -- the SwiGLU of nn/ffn.c:26-55.
#include "common.h"
#include "kernels.h"

namespace moty {

constexpr int GEMV_NT = 256;
constexpr int GEMV_WAVES = GEMV_NT / MOTY_WAVE;
constexpr int CHUNK = 16 * MOTY_WAVE;  // bytes of a row one wave-load covers
constexpr int CB = 4;                  // chunks in flight per row

__device__ __forceinline__ int4 ldnt16(const int8_t* p) {
  const v4i v = __builtin_nontemporal_load((const v4i*)p);
  return int4{v.x, v.y, v.z, v.w};
}

// qrow_i8 of a row held across a wave (lane l: 16 values per 1 KiB chunk):
// the wave-max is the row's amax; returns the scale, int8 values in place.
template <int NC>
__device__ __forceinline__ float wave_qrow(const float4 (&v)[NC][4], int4 (&q)[NC]) {
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < NC; c++)
#pragma unroll
    for (int j = 0; j < 4; j++)
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[c][j].x), fabsf(v[c][j].y)), fmaxf(fabsf(v[c][j].z), fabsf(v[c][j].w))));
  amax = wave_max_f32(amax);
  float s = amax / 127.f;
  if (s < 1e-12f) s = 1e-12f;
  const float inv = 1.f / s;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    int* qp = (int*)&q[c];
#pragma unroll
    for (int j = 0; j < 4; j++)
      qp[j] = (int)((uint32_t)(rne_int(v[c][j].x * inv) & 0xff) | ((uint32_t)(rne_int(v[c][j].y * inv) & 0xff) << 8) |
                    ((uint32_t)(rne_int(v[c][j].z * inv) & 0xff) << 16) |
                    ((uint32_t)(rne_int(v[c][j].w * inv) & 0xff) << 24));
  }
  return s;
}

template <int S_, int RPW, bool PAIR>
__global__ __launch_bounds__(GEMV_NT) void k_gemv_q8(const float* __restrict__ x, const int8_t* __restrict__ W,
                                                     const float* __restrict__ scale,
                                                     const int8_t* __restrict__ W2,
                                                     const float* __restrict__ scale2, float* __restrict__ y,
                                                     int I, int O) {
  extern __shared__ __align__(16) int8_t xq_s[];  // [S_][Ipad]
  __shared__ float red[GEMV_WAVES][S_];
  __shared__ float sx_s[S_];
  const int lane = threadIdx.x % MOTY_WAVE, wv = threadIdx.x / MOTY_WAVE;
  const int Ipad = (I + CHUNK - 1) / CHUNK * CHUNK;
  const int nch = Ipad / CHUNK;
  const int o0 = (blockIdx.x * GEMV_WAVES + wv) * RPW;

  int acc[RPW][S_];
  int acc2[RPW][S_];
#pragma unroll
  for (int r = 0; r < RPW; r++)
#pragma unroll
    for (int s = 0; s < S_; s++) acc[r][s] = acc2[r][s] = 0;

  for (int cb = 0; cb < nch; cb += CB) {
    int4 wq[RPW][CB], wq2[RPW][CB];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      // clamped addresses, unconditional loads (no waits at branch joins):
      // rows past O are never stored, columns past I meet zero activations
      // in LDS, chunks past the row end are never consumed
      const int o = o0 + r < O ? o0 + r : O - 1;
#pragma unroll
      for (int j = 0; j < CB; j++) {
        const int k = (cb + j) * CHUNK + lane * 16;
        const int kc = k < I ? k : 0;
        wq[r][j] = ldnt16(W + (int64_t)o * I + kc);
        if (PAIR) wq2[r][j] = ldnt16(W2 + (int64_t)o * I + kc);
      }
    }
    if (cb == 0) {
      // quantize the activation rows into LDS while the loads above fly
#pragma unroll
      for (int s = 0; s < S_; s++) {
        const float* xr = x + (int64_t)s * I;
        float amax = 0.f;
        for (int i = threadIdx.x * 4; i < I; i += GEMV_NT * 4) {
          float4 v = *(const float4*)(xr + i);
          amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        amax = wave_max_f32(amax);
        if (lane == 0) red[wv][s] = amax;
      }
      __syncthreads();
#pragma unroll
      for (int s = 0; s < S_; s++) {
        float amax = red[0][s];
#pragma unroll
        for (int i = 1; i < GEMV_WAVES; i++) amax = fmaxf(amax, red[i][s]);
        float sc = amax / 127.f;
        if (sc < 1e-12f) sc = 1e-12f;
        const float inv = 1.f / sc;
        if (threadIdx.x == 0) sx_s[s] = sc;
        const float* xr = x + (int64_t)s * I;
        for (int i = threadIdx.x * 4; i < Ipad; i += GEMV_NT * 4) {
          uint32_t p = 0;
          if (i < I) {
            float4 v = *(const float4*)(xr + i);
            p = (uint32_t)(rne_int(v.x * inv) & 0xff) | ((uint32_t)(rne_int(v.y * inv) & 0xff) << 8) |
                ((uint32_t)(rne_int(v.z * inv) & 0xff) << 16) | ((uint32_t)(rne_int(v.w * inv) & 0xff) << 24);
          }
          *(uint32_t*)(xq_s + s * Ipad + i) = p;
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < CB; j++) {
      if (cb + j >= nch) break;
#pragma unroll
      for (int s = 0; s < S_; s++) {
        const int4 xv = *(const int4*)(xq_s + s * Ipad + (cb + j) * CHUNK + lane * 16);
#pragma unroll
        for (int r = 0; r < RPW; r++) {
          acc[r][s] = dot16(wq[r][j], xv, acc[r][s]);
          if (PAIR) acc2[r][s] = dot16(wq2[r][j], xv, acc2[r][s]);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; r++)
#pragma unroll
    for (int s = 0; s < S_; s++) {
      acc[r][s] = wave_sum_i32(acc[r][s]);
      if (PAIR) acc2[r][s] = wave_sum_i32(acc2[r][s]);
    }
  // lane (r*S_ + s) writes element (r, s)
#pragma unroll
  for (int r = 0; r < RPW; r++)
#pragma unroll
    for (int s = 0; s < S_; s++) {
      const int o = o0 + r;
      if (lane == r * S_ + s && o < O) {
        const float sxv = sx_s[s];
        float v = (scale[o] * sxv) * (float)acc[r][s];
        if (PAIR) {
          const float u = (scale2[o] * sxv) * (float)acc2[r][s];
          v = ref_silu_mul(v, u);
        }
        y[(int64_t)s * O + o] = v;
      }
    }
}

// S = 1, I <= 4096, small matrices: the activation row never touches LDS.  Lane l of every
// wave loads elements [c*1024 + 16l, +16) of each 1 KiB chunk c -- exactly
// its dot inputs -- so a wave-max gives the row's amax and each wave
// quantizes in registers (qrow_i8 bit for bit), with no workgroup barrier.
// The activation loads are issued before the weight loads, so waiting for
// them does not wait for the weights.  Weights stream with non-temporal
// loads (read once, kept out of the caches' way).
template <int NC, int RPW, bool PAIR, int NW = GEMV_WAVES>
__global__ __launch_bounds__(NW * MOTY_WAVE) void k_gemv1_q8(const float* __restrict__ x, const int8_t* __restrict__ W,
                                                      const float* __restrict__ scale,
                                                      const int8_t* __restrict__ W2,
                                                      const float* __restrict__ scale2, float* __restrict__ y,
                                                      int I, int O) {
  const int lane = threadIdx.x % MOTY_WAVE;
  const int o0 = (blockIdx.x * NW + threadIdx.x / MOTY_WAVE) * RPW;
  float4 xv[NC][4];
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const int k = c * CHUNK + lane * 16;
#pragma unroll
    for (int j = 0; j < 4; j++) xv[c][j] = *(const float4*)(x + (k < I ? k : 0) + 4 * j);
  }
  int4 wq[RPW][NC], wq2[RPW][NC];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const int o = o0 + r < O ? o0 + r : O - 1;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const int k = c * CHUNK + lane * 16;
      const int kc = k < I ? k : 0;
      wq[r][c] = ldnt16(W + (int64_t)o * I + kc);
      if (PAIR) wq2[r][c] = ldnt16(W2 + (int64_t)o * I + kc);
    }
  }
  // each lane loads the scales of the row whose sum it will hold
  // (wave_sum_row), with the weights, so the epilogue waits on no further
  // memory latency
  const int rl = wave_sum_row<RPW>(lane);
  float sc = 0.f, sc2 = 0.f;
  {
    const int o = o0 + rl;
    sc = scale[o < O ? o : O - 1];
    if (PAIR) sc2 = scale2[o < O ? o : O - 1];
  }
  // keep the scheduler from sinking weight loads below the first use of x
  __builtin_amdgcn_sched_barrier(0);
  // past the row end x was read from a clamped address: zero it (the
  // weights there are multiplied by these zeros)
#pragma unroll
  for (int c = 0; c < NC; c++)
#pragma unroll
    for (int j = 0; j < 4; j++) xv[c][j] = sel4(c * CHUNK + lane * 16 < I, xv[c][j]);
  int4 xq[NC];
  const float sx = wave_qrow<NC>(xv, xq);
  int acc[RPW], acc2[RPW];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    acc[r] = 0;
    acc2[r] = 0;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      acc[r] = dot16(wq[r][c], xq[c], acc[r]);
      if (PAIR) acc2[r] = dot16(wq2[r][c], xq[c], acc2[r]);
    }
  }
  // the RPW row sums at once: lane l ends with row rl's; the first lane of
  // each group holding a row finishes it (computed on every lane, so the
  // scale loads above stay where they were issued)
  const int a = wave_sum_multi_i32<RPW>(acc);
  const int a2 = PAIR ? wave_sum_multi_i32<RPW>(acc2) : 0;
  float v = (sc * sx) * (float)a;
  if (PAIR) v = ref_silu_mul(v, (sc2 * sx) * (float)a2);
  const int o = o0 + rl;
  if ((lane & (MOTY_WAVE / RPW - 1)) == 0 && o < O) y[o] = v;
}

// S = 1, I <= 4096: large matrices, and plain rows of 3-4 KiB whose
// activation row is as large as a wave's weights (C1's down: 12 KiB of h
// against 3 KiB per row), so better loaded once per workgroup than once per
// wave.  The workgroup loads the activation row once (thread t takes float4
// units t, t + NT, ...); wave w owns RPW rows, lane l reads bytes
// [c*1024 + 16l, +16) of each 1 KiB chunk c, with non-temporal loads (read
// once, kept out of the caches' way).  While they fly the row is quantized
// (qrow_i8 bit for bit: the row's amax from a wave max and an LDS exchange
// across the waves) into LDS, from where each lane takes exactly the 16
// codes per chunk its dot needs.
// XF (every launch below): the weight loads are issued right behind the
// activation loads.  Without it the workgroup waits for the row first,
// which an earlier one-row-per-wave form needed (its row, queued behind the
// weight stream, arrived 3.5 us into a 10 us kernel) and which measured
// slower for every launch shape used now.
template <int NC, int RPW, bool PAIR, int NW, bool XF = false>
__global__ __launch_bounds__(NW * MOTY_WAVE) void k_gemv1_q8_lds(const float* __restrict__ x, const int8_t* __restrict__ W,
                                                      const float* __restrict__ scale,
                                                      const int8_t* __restrict__ W2,
                                                      const float* __restrict__ scale2, float* __restrict__ y,
                                                      int I, int O) {
  constexpr int NU = NC * CHUNK / 4;                         // float4 units of the row
  constexpr int XV = (NU + NW * MOTY_WAVE - 1) / (NW * MOTY_WAVE);  // per thread (unit t + j*NT)
  __shared__ __align__(16) int8_t xq_s[NC * CHUNK];
  __shared__ float red[NW];
  const int lane = threadIdx.x % MOTY_WAVE, wv = threadIdx.x / MOTY_WAVE;
  const int o0 = (blockIdx.x * NW + wv) * RPW;
  float4 xv[XV];
#pragma unroll
  for (int j = 0; j < XV; j++) {
    const int k = (threadIdx.x + j * NW * MOTY_WAVE) * 4;
    xv[j] = *(const float4*)(x + (k < I ? k : 0));
  }
  if (!XF) {
    MOTY_WAIT_VMCNT(0);
    __builtin_amdgcn_s_barrier();
  }
  int4 wq[RPW][NC], wq2[RPW][NC];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const int o = o0 + r < O ? o0 + r : O - 1;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const int k = c * CHUNK + lane * 16;
      const int kc = k < I ? k : 0;
      wq[r][c] = ldnt16(W + (int64_t)o * I + kc);
      if (PAIR) wq2[r][c] = ldnt16(W2 + (int64_t)o * I + kc);
    }
  }
  // each lane loads the scales of the row whose sum it will hold
  // (wave_sum_row), with the weights, so the epilogue waits on no further
  // memory latency
  const int rl = wave_sum_row<RPW>(lane);
  float sc = 0.f, sc2 = 0.f;
  {
    const int o = o0 + rl;
    sc = scale[o < O ? o : O - 1];
    if (PAIR) sc2 = scale2[o < O ? o : O - 1];
  }
  // keep the scheduler from sinking weight loads below the quantization
  __builtin_amdgcn_sched_barrier(0);
  // past the row end x was read from a clamped address: zero it (the
  // weights there are multiplied by these zeros)
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < XV; j++) {
    xv[j] = sel4((threadIdx.x + j * NW * MOTY_WAVE) * 4 < I, xv[j]);
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(xv[j].x), fabsf(xv[j].y)), fmaxf(fabsf(xv[j].z), fabsf(xv[j].w))));
  }
  amax = wave_max_f32(amax);
  if (NW > 1) {
    if (lane == 0) red[wv] = amax;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NW; i++) amax = fmaxf(amax, red[i]);
  }
  float sx = amax / 127.f;
  if (sx < 1e-12f) sx = 1e-12f;
  const float inv = 1.f / sx;
#pragma unroll
  for (int j = 0; j < XV; j++) {
    const int k = (threadIdx.x + j * NW * MOTY_WAVE) * 4;
    if (k < NC * CHUNK)
      *(uint32_t*)(xq_s + k) =
          (uint32_t)(rne_int(xv[j].x * inv) & 0xff) | ((uint32_t)(rne_int(xv[j].y * inv) & 0xff) << 8) |
          ((uint32_t)(rne_int(xv[j].z * inv) & 0xff) << 16) | ((uint32_t)(rne_int(xv[j].w * inv) & 0xff) << 24);
  }
  __syncthreads();
  int4 xq[NC];
#pragma unroll
  for (int c = 0; c < NC; c++) xq[c] = *(const int4*)(xq_s + c * CHUNK + lane * 16);
  int acc[RPW], acc2[RPW];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    acc[r] = 0;
    acc2[r] = 0;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      acc[r] = dot16(wq[r][c], xq[c], acc[r]);
      if (PAIR) acc2[r] = dot16(wq2[r][c], xq[c], acc2[r]);
    }
  }
  // the RPW row sums at once: lane l ends with row rl's; the first lane of
  // each group holding a row finishes it (computed on every lane, so the
  // scale loads above stay where they were issued)
  const int a = wave_sum_multi_i32<RPW>(acc);
  const int a2 = PAIR ? wave_sum_multi_i32<RPW>(acc2) : 0;
  float v = (sc * sx) * (float)a;
  if (PAIR) v = ref_silu_mul(v, (sc2 * sx) * (float)a2);
  const int o = o0 + rl;
  if ((lane & (MOTY_WAVE / RPW - 1)) == 0 && o < O) y[o] = v;
}

template <int NC, bool PAIR>
static int launch_1(const float* x, const int8_t* W, const float* scale, const int8_t* W2, const float* scale2,
                    float* y, int I, int O, hipStream_t st) {
  // Launch shape from a sweep of rows/wave x waves/workgroup on MI355X over
  // decode shapes (O 1024..12288, I 1024..4096, plain and PAIR): four rows
  // per wave (fewer when that leaves < 256 waves), then enough waves per
  // workgroup to bring the grid near one workgroup per CU.
  int rpw = 4;
  while (rpw > 1 && (O + rpw - 1) / rpw < 256) rpw >>= 1;
  const int waves = (O + rpw - 1) / rpw;
  // up to one workgroup per CU, of up to 4 waves; from 768 waves on, 4
  // (C1's gate/up, 768 waves: FFN step 5.85 us against 5.90 with 3-wave
  // workgroups on every CU, 5.96 with 2, 5.90 with 1)
  const int nw = waves >= 768 ? 4 : (waves + 255) / 256;
  const unsigned nb = (unsigned)((waves + nw - 1) / nw);
  // a long weight stream: the shared-activation kernel (activation row
  // quantized once per workgroup into LDS, fewer registers per wave), the
  // weight loads issued before the activation row lands: two rows per wave
  // for plain matrices, one for the fused gate/up pair; 8-wave workgroups
  // from 4096 waves on, else 4.  From a sweep of rows/wave x waves/workgroup
  // x issue order on MI355X (graph replays over rotating weights): 4096 x
  // 4096 4.26 us against 4.64 for 8 waves of one row with the row awaited
  // first, 12288 x 4096 9.65 against 10.06 (2 rows, 8 waves, awaited), the
  // fused 2 x 12288 x 4096 17.2 against 17.7
  if ((int64_t)O * I * (PAIR ? 2 : 1) >= ((int64_t)16 << 20)) {
    constexpr int NWL = (4 * NC) % 8 == 0 ? 8 : 4;  // whole float4 of the row per thread
    const int lwaves = PAIR ? O : (O + 1) / 2;
    const bool wide = lwaves >= 4096;
    const unsigned nbl = (unsigned)((lwaves + (wide ? NWL : 4) - 1) / (wide ? NWL : 4));
    constexpr int R = PAIR ? 1 : 2;
    if (wide)
      hipLaunchKernelGGL((k_gemv1_q8_lds<NC, R, PAIR, NWL, true>), dim3(nbl), dim3(NWL * MOTY_WAVE), 0, st, x, W,
                         scale, W2, scale2, y, I, O);
    else
      hipLaunchKernelGGL((k_gemv1_q8_lds<NC, R, PAIR, 4, true>), dim3(nbl), dim3(4 * MOTY_WAVE), 0, st, x, W, scale,
                         W2, scale2, y, I, O);
    LAUNCH_TRY("k_gemv1_q8_lds");
    return MOTY_OK;
  }
  // plain rows of 3-4 KiB with at least 1024 of them: the shared-activation
  // kernel in 4-wave workgroups, weight loads issued before the row lands
  // (C1's down, 1024 x 3072: FFN step 5.63 against 5.95 us for the per-wave
  // kernel; waiting for the row first 5.94; 2 rows x 2 waves 5.65)
  if (!PAIR && NC >= 3 && O >= 1024) {
    if (O >= 2048)
      hipLaunchKernelGGL((k_gemv1_q8_lds<NC, 2, false, 4, true>), dim3((O + 7) / 8), dim3(4 * MOTY_WAVE), 0, st, x, W,
                         scale, W2, scale2, y, I, O);
    else
      hipLaunchKernelGGL((k_gemv1_q8_lds<NC, 1, false, 4, true>), dim3((O + 3) / 4), dim3(4 * MOTY_WAVE), 0, st, x, W,
                         scale, W2, scale2, y, I, O);
    LAUNCH_TRY("k_gemv1_q8_lds");
    return MOTY_OK;
  }
#define L1(R, N)                                                                                              \
  if (rpw == R && nw == N) {                                                                                 \
    hipLaunchKernelGGL((k_gemv1_q8<NC, R, PAIR, N>), dim3(nb), dim3(N * MOTY_WAVE), 0, st, x, W, scale, W2,   \
                       scale2, y, I, O);                                                                     \
    LAUNCH_TRY("k_gemv1_q8");                                                                                \
    return MOTY_OK;                                                                                          \
  }
  L1(4, 4) L1(4, 3) L1(4, 2) L1(4, 1) L1(2, 2) L1(2, 1) L1(1, 2) L1(1, 1)
#undef L1
  return MOTY_EUNSUP;
}

template <int S_, bool PAIR>
static int launch_s(const float* x, const int8_t* W, const float* scale, const int8_t* W2, const float* scale2,
                    float* y, int S, int I, int O, hipStream_t st) {
  const int Ipad = (I + CHUNK - 1) / CHUNK * CHUNK;
  const size_t lds = (size_t)S_ * Ipad;
  // rows per wave: keep >= ~2 blocks per CU on the 256-CU part
  const int rpw = (O >= 32768) ? 4 : (O >= 8192 ? 2 : 1);
  auto go = [&](auto kern, int r) {
    const int rows_per_block = GEMV_WAVES * r;
    const unsigned nb = (unsigned)((O + rows_per_block - 1) / rows_per_block);
    hipLaunchKernelGGL(kern, dim3(nb), dim3(GEMV_NT), lds, st, x, W, scale, W2, scale2, y, I, O);
  };
  if (rpw == 4) go(k_gemv_q8<S_, 4, PAIR>, 4);
  else if (rpw == 2) go(k_gemv_q8<S_, 2, PAIR>, 2);
  else go(k_gemv_q8<S_, 1, PAIR>, 1);
  LAUNCH_TRY("k_gemv_q8");
  return MOTY_OK;
}

// y [S][O] = Q8 GEMV of x [S][I]; PAIR: y = silu(x.W^T) * (x.W2^T)
int launch_gemv_q8(const float* x, const int8_t* W, const float* scale, const int8_t* W2, const float* scale2,
                   float* y, int S, int I, int O, hipStream_t st) {
  if (S < 1 || S > GEMV_MAX_S || (I % 16) || I > 16384) return MOTY_EUNSUP;
  if (O <= 0) return MOTY_OK;
  const bool pair = (W2 != nullptr);
  if (S == 1 && I <= 4 * CHUNK) {
    const int nc = (I + CHUNK - 1) / CHUNK;
#define CASE1(n)                                                                                             \
  case n:                                                                                                    \
    return pair ? launch_1<n, true>(x, W, scale, W2, scale2, y, I, O, st)                                    \
                : launch_1<n, false>(x, W, scale, W2, scale2, y, I, O, st);
    switch (nc) {
      CASE1(1)
      CASE1(2)
      CASE1(3)
      CASE1(4)
    }
#undef CASE1
  }
#define CASE(n)                                                                              \
  case n:                                                                                    \
    return pair ? launch_s<n, true>(x, W, scale, W2, scale2, y, S, I, O, st)                 \
                : launch_s<n, false>(x, W, scale, W2, scale2, y, S, I, O, st);
  switch (S) {
    CASE(1)
    CASE(2)
    CASE(3)
    CASE(4)
  }
#undef CASE
  return MOTY_EUNSUP;
}

}  // namespace moty
