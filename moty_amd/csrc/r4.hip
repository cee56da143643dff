// r4.hip -- Q4R4 / Q8R4 matmuls: 4-row blocks, groups of 32, f16 group
// scales, group-32 int8 activations.
//
// Reference: hw/hw_q4r4.h (format, kernels), nn/quant.c:110-179 (packers),
// nn/matmul.c:365-466 (moty_matmul_q4r4_s / moty_matmul_q8r4_s).
//
// Layout (unchanged from the reference): weight rows in blocks of 4; per
// (block, group) Q4R4 stores 64 bytes = 4 rows x 16 bytes, row byte j =
// c[j] | c[j+16] << 4 with codes c = v + 8 in 0..15; Q8R4 stores 128 bytes =
// 4 rows x 32 signed codes.  Scales: f16 [block][group][4].
//
// Activations: per group of 32, s = amax/127 (clamped at 1e-30), q =
// rint(x/s) and the code sum xsum (hw/hw_q4r4.h:36-46).
//
// Arithmetic, as the reference's x86 build evaluates it (its portable
// kernels are the scalar references): per output, groups in order,
//   tokens t < 4*floor(S/4) (the 4-token tile kernel):
//       s = sum c*x;  acc = fma(s, dd*xs, acc);  acc = fma(-dd, (8*xsum)*xs, acc)
//   the remaining tokens (the per-token kernel):
//       s = sum c*x - 8*xsum;  acc = fma(s, dd*xs, acc)
//   Q8R4 (no offset): acc = fma(sum c*x, dd*xs, acc).
// The integer group sums are exact, so only the float chain's order is
// fixed; the kernels below keep it.
#include "common.h"
#include "kernels.h"

namespace moty {

// ---------------------------------------------------------------------------
// Group-32 activation quantization: a lane pair per group, 16 elements
// (4 float4) per lane.  Each lane reduces its half in registers; one
// exchange with the partner lane joins amax and the code sum, so the scale's
// two divisions run once per half group.  The arithmetic per element is the
// reference's: s = amax/127 (at least 1e-30), q = rint(x * (1/s)).
// Returns the group's code sum; q gets the lane's 16 codes, s the scale.
__device__ __forceinline__ int quant_half_g32(const float4 (&v)[4], uint4& q, float& s) {
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++)
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  s = amax / 127.f;
  if (s < 1e-30f) s = 1e-30f;
  const float inv = 1.f / s;
  int sum = 0;
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int a = rne_int(v[j].x * inv), b = rne_int(v[j].y * inv), c = rne_int(v[j].z * inv),
              d = rne_int(v[j].w * inv);
    sum += a + b + c + d;
    w[j] = (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
  }
  q = make_uint4(w[0], w[1], w[2], w[3]);
  return sum + __shfl_xor(sum, 1, 64);
}

// One lane per 16 elements of a row: lanes 2i, 2i+1 share group i.
__global__ __launch_bounds__(256) void k_quant_g32(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                   float* __restrict__ xs, int32_t* __restrict__ xm, int I) {
  const int64_t row = blockIdx.y;
  const int e = (blockIdx.x * 256 + threadIdx.x) * 16;
  const bool ok = e < I;
  const float4* src = (const float4*)(x + row * I + (ok ? e : 0));
  float4 v[4];
#pragma unroll
  for (int j = 0; j < 4; j++) v[j] = sel4(ok, src[j]);
  uint4 q;
  float s;
  const int sum = quant_half_g32(v, q, s);
  if (!ok) return;
  *(uint4*)(xq + row * I + e) = q;
  if ((threadIdx.x & 1) == 0) {
    const int nb = I / 32;
    xs[row * nb + e / 32] = s;
    xm[row * nb + e / 32] = sum;
  }
}

int launch_quant_g32(const float* x, int8_t* xq, float* xs, int32_t* xm, int S, int I, hipStream_t st) {
  if (S <= 0) return MOTY_OK;
  if (I % 32) return MOTY_EUNSUP;
  hipLaunchKernelGGL(k_quant_g32, dim3((I + 4095) / 4096, S), dim3(256), 0, st, x, xq, xs, xm, I);
  LAUNCH_TRY("k_quant_g32");
  return MOTY_OK;
}

// low / high nibbles of 16 packed Q4R4 bytes as 16 + 16 unsigned int8 codes
__device__ __forceinline__ int4 r4_lo(int4 w) {
  return int4{w.x & 0x0f0f0f0f, w.y & 0x0f0f0f0f, w.z & 0x0f0f0f0f, w.w & 0x0f0f0f0f};
}
__device__ __forceinline__ int4 r4_hi(int4 w) {
  return int4{(w.x >> 4) & 0x0f0f0f0f, (w.y >> 4) & 0x0f0f0f0f, (w.z >> 4) & 0x0f0f0f0f, (w.w >> 4) & 0x0f0f0f0f};
}

// ---------------------------------------------------------------------------
// Decode GEMV, S_ <= 3 tokens (all in the per-token kernel's form), I <=
// 1024*IC.  KS waves share one 4-row block, split along K: chunk index kk
// (64 lanes x 16 bytes, GPC groups) belongs to part kk % KS, so a block
// count near the SIMD count still puts several waves on every SIMD.  The
// activation rows are loaded and land first; the weight chunks of the part
// (each load instruction reads 1 KiB of the contiguous block) and the f16
// scale of each chunk's (row, group) are then kept PD chunks ahead of the
// one being consumed.  The workgroup quantizes the activation rows into LDS
// from registers (every workgroup derives the same codes).  Each lane forms
// the exact integer group sums of its chunks (Q8R4: half a row per chunk,
// the halves joined across the lane pair) and parks the two operands of the
// chain step, (s - 8*xsum, dd*xs), in the block's LDS slice
// ([row][token][group]); after its k-th chunk a part raises its progress
// flag to k+1.  One lane per (row, token) of part 0 runs acc = fma(a, b,
// acc) over the groups in order, chunk index by chunk index, each one as
// soon as its part's flag says it is parked.  Only part 0 ever waits, on
// flags that every other part raises unconditionally, so every wait ends.
template <bool Q8, int S_, int IC, int NT, bool PAIR = false, int KS = 1>
__global__ __launch_bounds__(NT) void k_r4_gemv(const float* __restrict__ x, const uint8_t* __restrict__ W,
                                                const uint16_t* __restrict__ d16, float* __restrict__ y, int S,
                                                int I, int O) {
  static_assert(!PAIR || S_ == 1, "the fused gate/up form serves one token");
  constexpr int NM = PAIR ? 2 : 1;  // matrices: gate (and up)
  constexpr int GB = Q8 ? 128 : 64;        // bytes per (block, group)
  constexpr int NCH = IC * (Q8 ? 4 : 2);   // chunk indices per block
  static_assert(NCH % KS == 0, "K parts of whole chunks");
  constexpr int NCW = NCH / KS;            // chunks per lane per wave
  // chunks in flight ahead of the one consumed: one for a single token (the
  // C3 shapes on MI355X: 4096 x 12288 9.5 us against 10.9 with four ahead,
  // the fused 2 x 12288 x 4096 gate_up 11.6 against 13.7 -- each row's chain
  // then keeps pace with its data), four for more tokens
  constexpr int PD = S_ == 1 ? 1 : (NCW < 4 ? NCW : 4);
  constexpr int P0 = PD < 2 ? PD : 2;      // of them issued before the quantization
  constexpr int GPC = Q8 ? 8 : 16;         // groups per chunk index
  constexpr int WAVES = NT / MOTY_WAVE;
  static_assert(WAVES % KS == 0, "whole blocks per workgroup");
  constexpr int BPW = WAVES / KS;          // blocks per workgroup
  constexpr int XU = (IC * 64 + NT - 1) / NT;  // activation half groups (16 floats) per thread per row
  extern __shared__ __align__(16) int8_t lds[];
  __shared__ int flag_s[BPW * KS];
  const int nb = I / 32, O4 = (O + 3) / 4;
  const int lane = threadIdx.x % MOTY_WAVE, wv = threadIdx.x / MOTY_WAVE;
  const int part = wv % KS, bw = wv / KS;
  // LDS: xq [S_][I] | xs [S_][nb] | xm [S_][nb] | per block: operands [NM*4][S_][nb] float2
  int8_t* xq_s = lds;
  float* xs_s = (float*)(lds + S_ * I);
  int* xm_s = (int*)(xs_s + S_ * nb);
  // operand rows padded to an even length past nb: the four rows of a
  // block that lanes 4g..4g+3 write land in distinct banks (rows nb apart
  // shared banks: 8-16 % of LDS cycles in bank conflicts)
  const int ldo = nb + 2 - (nb & 1);
  float2* op_s = (float2*)(xm_s + S_ * nb) + (size_t)bw * (4 * NM * S_ * ldo);
  int blk = blockIdx.x * BPW + bw;
  const bool live = blk < O4;
  blk = live ? blk : O4 - 1;

  // 1. activation rows
  float4 xr[S_][XU][4];
#pragma unroll
  for (int t = 0; t < S_; t++)
#pragma unroll
    for (int c = 0; c < XU; c++) {
      const int e = (c * NT + threadIdx.x) * 16;
      const float4* src = (const float4*)(x + (size_t)(t < S ? t : 0) * I + (e < I ? e : 0));
#pragma unroll
      for (int j = 0; j < 4; j++) xr[t][c][j] = src[j];
    }
  if (KS > 1 && threadIdx.x < BPW * KS) flag_s[threadIdx.x] = 0;

  // 2. weight chunks of the part and their scales, PD chunks ahead: chunk
  // k + PD is issued just before chunk k is consumed, so the integer dots
  // and the chain run while the stream is still arriving (a wave that
  // issued all of its loads first would sit in the issue stall until the
  // memory path had taken them all).  The activation rows land first (the
  // wait and the bare barrier: queued behind the weight stream in the CU's
  // load path and in L2 they would arrive with it), then the first P0
  // chunks go out before the quantization, the rest of the PD after it.
  // PAIR: W is the row-fused [gate; up] matrix (moty_mat_fuse_rows), the up
  // rows' blocks start O/4 blocks after the gate rows'
  const int nchunk = nb * GB / 16;
  int4 wc[NM][NCW];
  uint16_t dc[NM][NCW];
  auto issue = [&](int k) {
#pragma unroll
    for (int m = 0; m < NM; m++) {
      const int ci = lane + 64 * (k * KS + part);
      const int cc = ci < nchunk ? ci : 0;
      {
        const v4i t = __builtin_nontemporal_load((const v4i*)(W + ((size_t)(blk + m * O4) * nb * GB + (size_t)cc * 16)));
        wc[m][k] = int4{t.x, t.y, t.z, t.w};
      }
      // chunk ci: group ci/4, row ci%4 (Q8R4: group ci/8, row (ci/2)%4)
      dc[m][k] = __builtin_nontemporal_load(d16 + (size_t)(blk + m * O4) * nb * 4 + (Q8 ? (cc >> 3) * 4 + ((cc >> 1) & 3) : cc));
    }
  };
  MOTY_WAIT_VMCNT(0);
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int k = 0; k < P0; k++) issue(k);
  __builtin_amdgcn_sched_barrier(0);

  // 3. group-32 quantization of the activation rows into LDS (k_quant_g32's
  // arithmetic)
#pragma unroll
  for (int t = 0; t < S_; t++)
#pragma unroll
    for (int c = 0; c < XU; c++) {
      const int e = (c * NT + threadIdx.x) * 16;
      const bool ok = e < I;
      float4 v[4];
#pragma unroll
      for (int j = 0; j < 4; j++) v[j] = sel4(ok, xr[t][c][j]);
      uint4 q;
      float sc;
      const int sum = quant_half_g32(v, q, sc);
      if (ok) {
        *(uint4*)(xq_s + t * I + e) = q;
        if ((threadIdx.x & 1) == 0) {
          xs_s[t * nb + e / 32] = sc;
          xm_s[t * nb + e / 32] = sum;
        }
      }
    }
  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (int k = P0; k < PD; k++) issue(k);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();

  // 4. per chunk: the exact integer group sum and the chain step's
  // operands; then part 0's lane (m*4 + r)*S_ + t continues row r's chain
  // for token t (PAIR: m = 1 is the up row) over chunk indices k*KS ..
  // k*KS + KS-1 in order, while later chunks may still be in flight.
  // part 0 carries the serial chain: its wave gets the SIMD's issue
  // priority over the parts that only form group sums
  if (KS > 1 && part == 0) __builtin_amdgcn_s_setprio(3);
  const bool chain = part == 0 && lane < 4 * NM * S_;
  const float2* opc = op_s + (lane < 4 * NM * S_ ? lane : 0) * ldo;  // lane = (m*4 + r)*S_ + t
  const bool even = (nb & 1) == 0;  // 16-byte reads of two groups' operands stay aligned
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < NCW; k++) {
    if (k + PD < NCW) issue(k + PD);
    __builtin_amdgcn_sched_barrier(0);
    const int ci = lane + 64 * (k * KS + part);
    const int g = Q8 ? (ci >> 3) : (ci >> 2), r = Q8 ? ((ci >> 1) & 3) : (ci & 3), h = Q8 ? (ci & 1) : 0;
    const bool ok = ci < nchunk;
    const int gc = ok ? g : 0;
#pragma unroll
    for (int m = 0; m < NM; m++) {
      const float dd = f16_to_f32(dc[m][k]);
#pragma unroll
      for (int t = 0; t < S_; t++) {
        const int8_t* xg = xq_s + t * I + gc * 32;
        int sacc;
        if (Q8) {
          sacc = dot16(wc[m][k], *(const int4*)(xg + 16 * h), 0);
          sacc += __shfl_xor(sacc, 1, 64);  // the row's other half: lanes 2i, 2i+1 hold (g, r, h = 0/1)
        } else {
          sacc = dot16(r4_lo(wc[m][k]), *(const int4*)xg, dot16(r4_hi(wc[m][k]), *(const int4*)(xg + 16), 0));
          sacc -= 8 * xm_s[t * nb + gc];
        }
        if (ok && h == 0) op_s[((m * 4 + r) * S_ + t) * ldo + g] = float2{(float)sacc, dd * xs_s[t * nb + gc]};
      }
    }
    if (KS > 1 && part != 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (lane == 0) __hip_atomic_store(&flag_s[bw * KS + part], k + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      continue;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (chain) {
#pragma unroll
      for (int p = 0; p < KS; p++) {
        if (p > 0) {
          while (__hip_atomic_load(&flag_s[bw * KS + p], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) <= k)
            __builtin_amdgcn_s_sleep(1);
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        }
        const int g0 = (k * KS + p) * GPC, g1 = nb < g0 + GPC ? nb : g0 + GPC;
        if (g1 - g0 == GPC && even) {
          const float4* p4 = (const float4*)(opc + g0);
          float4 v[GPC / 2];
#pragma unroll
          for (int u = 0; u < GPC / 2; u++) v[u] = p4[u];
#pragma unroll
          for (int u = 0; u < GPC / 2; u++) {
            acc = __fmaf_rn(v[u].x, v[u].y, acc);
            acc = __fmaf_rn(v[u].z, v[u].w, acc);
          }
        } else {
          for (int gg = g0; gg < g1; gg++) acc = __fmaf_rn(opc[gg].x, opc[gg].y, acc);
        }
      }
    }
  }
  if (part != 0) return;
  if (PAIR) {
    const float u = __shfl(acc, (lane + 4) & 63, 64);
    const int o = blk * 4 + lane;
    if (live && lane < 4 && o < O) y[o] = ref_silu_mul(acc, u);
  } else if (lane < 4 * S_) {
    // lane = r*S_ + t
    const int r = lane / S_, t = lane % S_;
    const int o = blk * 4 + r;
    if (live && t < S && o < O) y[(size_t)t * O + o] = acc;
  }
}

template <int S_, int NT, bool PAIR, int KS>
static size_t r4_gemv_lds(int I) {
  const int nb = I / 32;
  const int ldo = nb + 2 - (nb & 1);
  return (size_t)S_ * I + (size_t)S_ * nb * 8 + (size_t)(NT / MOTY_WAVE / KS) * 4 * (PAIR ? 2 : 1) * S_ * ldo * 8;
}

template <bool Q8, int S_, int IC, int NT, bool PAIR, int KS>
static int go_r4_gemv(const float* x, const uint8_t* W, const uint16_t* d16, float* y, int S, int I, int O,
                      hipStream_t st) {
  const int O4 = (O + 3) / 4, bpw = NT / MOTY_WAVE / KS;
  const size_t lds = r4_gemv_lds<S_, NT, PAIR, KS>(I);
  if (lds + 256 > 64 * 1024) return MOTY_EUNSUP;  // 256: the static progress flags
  hipLaunchKernelGGL((k_r4_gemv<Q8, S_, IC, NT, PAIR, KS>), dim3((unsigned)((O4 + bpw - 1) / bpw)), dim3(NT), lds,
                     st, x, W, d16, y, S, I, O);
  LAUNCH_TRY("k_r4_gemv");
  return MOTY_OK;
}

// Waves per block: K is split until the blocks give every SIMD (1024 on the
// chip) about four waves, within the chunks a lane holds.  Workgroups of
// 4 * KS... waves as the LDS allows.
template <bool Q8, int S_, int IC, bool PAIR>
static int go_r4_gemv_nt(const float* x, const uint8_t* W, const uint16_t* d16, float* y, int S, int I, int O,
                         hipStream_t st) {
  constexpr int NCH = IC * (Q8 ? 4 : 2);
  const int O4 = (O + 3) / 4;
  if constexpr (NCH % 4 == 0 && NCH >= 8) {
    if (O4 <= 1024) {
      int rc = go_r4_gemv<Q8, S_, IC, 1024, PAIR, 4>(x, W, d16, y, S, I, O, st);
      if (rc != MOTY_EUNSUP) return rc;
      rc = go_r4_gemv<Q8, S_, IC, 512, PAIR, 4>(x, W, d16, y, S, I, O, st);
      if (rc != MOTY_EUNSUP) return rc;
    }
  }
  if constexpr (NCH % 2 == 0 && NCH >= 4) {
    if (O4 <= 2048) {
      int rc = go_r4_gemv<Q8, S_, IC, 512, PAIR, 2>(x, W, d16, y, S, I, O, st);
      if (rc != MOTY_EUNSUP) return rc;
      rc = go_r4_gemv<Q8, S_, IC, 256, PAIR, 2>(x, W, d16, y, S, I, O, st);
      if (rc != MOTY_EUNSUP) return rc;
    }
  }
  int rc = go_r4_gemv<Q8, S_, IC, 256, PAIR, 1>(x, W, d16, y, S, I, O, st);
  if (rc != MOTY_EUNSUP) return rc;
  return go_r4_gemv<Q8, S_, IC, 128, PAIR, 1>(x, W, d16, y, S, I, O, st);
}

// instances: activation float4 per thread and weight chunks per lane stay
// within a register budget (S_ * IC <= 16, Q8R4 IC <= 8; PAIR IC <= 8)
template <bool Q8, int S_, bool PAIR = false>
static int go_r4_gemv_ic(const float* x, const uint8_t* W, const uint16_t* d16, float* y, int S, int I, int O,
                         hipStream_t st) {
  const int ic = (I + 1023) / 1024;
  if (ic <= 1) return go_r4_gemv_nt<Q8, S_, 1, PAIR>(x, W, d16, y, S, I, O, st);
  if (ic <= 2) return go_r4_gemv_nt<Q8, S_, 2, PAIR>(x, W, d16, y, S, I, O, st);
  if (ic <= 4) return go_r4_gemv_nt<Q8, S_, 4, PAIR>(x, W, d16, y, S, I, O, st);
  if constexpr (S_ <= 2 && !(Q8 && PAIR)) {
    if (ic <= 8) return go_r4_gemv_nt<Q8, S_, 8, PAIR>(x, W, d16, y, S, I, O, st);
  }
  if constexpr (!Q8 && !PAIR && S_ == 1) {
    if (ic <= 12) return go_r4_gemv_nt<Q8, S_, 12, PAIR>(x, W, d16, y, S, I, O, st);
    if (ic <= 16) return go_r4_gemv_nt<Q8, S_, 16, PAIR>(x, W, d16, y, S, I, O, st);
  }
  return MOTY_EUNSUP;
}

template <bool Q8>
static int launch_r4_gemv(const float* x, const uint8_t* W, const uint16_t* d16, float* y, int S, int I, int O,
                          hipStream_t st) {
  switch (S) {
    case 1: return go_r4_gemv_ic<Q8, 1>(x, W, d16, y, S, I, O, st);
    case 2: return go_r4_gemv_ic<Q8, 2>(x, W, d16, y, S, I, O, st);
    case 3: return go_r4_gemv_ic<Q8, 3>(x, W, d16, y, S, I, O, st);
  }
  return MOTY_EUNSUP;  // S = 4 is the reference's 4-token tile: the GEMM path
}

// ---------------------------------------------------------------------------
// Prefill GEMM on v_mfma_i32_32x32x32_i8: one MFMA per group (K = 32 = the
// group), so each group's integer sum comes out separately and is folded
// into the float chain per output in group order.  Block tile 64 tokens x 64
// weight rows, 4 waves as 2 x 2 (32 x 32 each).  Per K block of 4 groups the
// workgroup stages in LDS, by whole-line loads: the tokens' int8 codes, the
// weight codes (Q4R4: 16 packed bytes per row and group, unpacked to low /
// high nibbles for the two MFMA halves; Q8R4: 32 codes), the decoded f16
// scales per (row, group), and per (group, token) the activation scale xs,
// the integer offset m8 = -8*xsum for per-token-kernel tokens (else 0) and
// the tile kernel's offset term xct = (8*xsum)*xs (0 for per-token tokens):
//   acc = fma(float(s + m8), dd*xs, acc);  acc = fma(-dd, xct, acc)
// reproduces both reference forms (the second FMA adds -dd*0 to a nonzero-
// signed or +0 accumulator: exactly nothing).  Q8R4 runs the first FMA only.
// WV = 8 / 16: eight waves of 16 tokens x 32 rows each (two
// v_mfma_i32_16x16x32_i8 per group) or sixteen of 16 x 16, over the same block tile and staging (done by the first four
// waves), for grids that give one workgroup per CU: two waves per SIMD
// instead of one.  Lane l's fragments: A = codes [8(l/16), +8) of token row
// l % 16; B = the same k of weight row l % 16 -- for Q4R4 the low (k < 16)
// or high nibbles of bytes [8(l/16 % 2), +8) of the row's 16 group bytes,
// byte j holding codes j and j + 16.
constexpr int R4M_NT = 256;
constexpr int R4M_KG = 4;                 // groups per K block
constexpr int R4M_AS = R4M_KG * 32 + 16;  // A row stride (bytes)

// PAIR (WV = 4): W is a row-fused [gate; up] matrix of 2*O rows; the tile's
// first 32 weight rows are gate rows 32*bx + [0, 32), the last 32 the up rows
// O + 32*bx + [0, 32), and the epilogue writes y [S][O] = silu(gate) * up
// (the gate_up + silu_rows of nn/ffn.c:28-37; the up waves hand their sums
// over through LDS).
template <bool Q8, bool TILE = false, int WV = 4, bool PAIR = false>
__global__ __launch_bounds__(64 * WV, WV <= 8 ? 8 / WV : 1) void k_r4_gemm(const int8_t* __restrict__ xq, const float* __restrict__ xs,
                                                       const int32_t* __restrict__ xm,
                                                       const uint8_t* __restrict__ W,
                                                       const uint16_t* __restrict__ d16, float* __restrict__ y,
                                                       int S, int I, int O) {
  constexpr int GB = Q8 ? 128 : 64;
  constexpr int RB = Q8 ? 32 : 16;          // bytes per (row, group)
  constexpr int BS = R4M_KG * RB + 16;      // B row stride (bytes)
  constexpr int NBC = Q8 ? 2 : 1;           // B chunks per thread
  constexpr int NWN = WV / 4, JN = 4 / NWN;  // WV >= 8: waves along the rows, 16-row tiles per wave
  static_assert(WV == 4 || WV == 8 || WV == 16, "waves");
  static_assert(!PAIR || WV == 4, "PAIR runs the 32 x 32 waves");
  __shared__ __align__(16) int8_t sA[64 * R4M_AS];
  __shared__ __align__(16) uint8_t sB[64 * BS];
  __shared__ float sD[64 * R4M_KG];         // [row][group]
  __shared__ __align__(16) float sX[R4M_KG * 64], sC[R4M_KG * 64];  // [group][token]
  __shared__ __align__(16) int sM[R4M_KG * 64];
  const int tid = threadIdx.x, lane = tid % MOTY_WAVE, wv = tid / MOTY_WAVE;
  const int wm = wv >> 1, wn = wv & 1;
  const int r32 = lane & 31, hk = lane >> 5;
  const int mb = blockIdx.y * 64, nb0 = blockIdx.x * (PAIR ? 32 : 64);
  const int nb = I / 32, S4 = S / 4 * 4;
  const int O4 = ((PAIR ? 2 * O : O) + 3) / 4;

  // copy assignments
  const int8_t* srcA[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int q = tid + i * R4M_NT;
    int m = mb + (q >> 3);
    m = m < S ? m : S - 1;
    srcA[i] = xq + (int64_t)m * I + (q & 7) * 16;
  }
  // B: thread -> (row tid/4, group tid%4), Q8R4 two 16-byte halves
  const int trow = tid >> 2;
  int orow = !PAIR ? nb0 + trow : trow < 32 ? nb0 + trow : O + nb0 + trow - 32;
  int ob = orow / 4;
  ob = ob < O4 ? ob : O4 - 1;
  const uint8_t* srcB = W + (size_t)ob * nb * GB + (size_t)(orow & 3) * RB;
  const uint16_t* srcD = d16 + (size_t)ob * nb * 4 + (orow & 3);
  // token scales: thread -> (group tid/64, token tid%64)
  const int st_t = mb + (tid & 63), st_g = tid >> 6;
  const int st_tc = st_t < S ? st_t : S - 1;
  const bool st_tile = st_t < S4;

  struct Set {
    int4 a[2];
    int4 b[NBC];
    uint32_t d;
    float x;
    int m;
  };
  Set s0, s1;
  const bool stager = WV == 4 || tid < R4M_NT;  // wave-uniform
  const int glast = (nb - 1) / R4M_KG * R4M_KG;
  auto gload = [&](int g0, Set& sv) {
    if (!stager) return;
    const int gc = g0 < nb ? g0 : glast;
    const int kb = gc * 32;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int q = tid + i * R4M_NT;
      sv.a[i] = *(const int4*)(srcA[i] + (kb + (q & 7) * 16 < I ? kb : -(q & 7) * 16));
    }
    const int g = gc + (tid & 3) < nb ? gc + (tid & 3) : 0;
#pragma unroll
    for (int i = 0; i < NBC; i++) sv.b[i] = *(const int4*)(srcB + (size_t)g * GB + 16 * i);
    sv.d = srcD[(size_t)g * 4];
    const int gt = gc + st_g < nb ? gc + st_g : 0;
    sv.x = xs[(size_t)st_tc * nb + gt];
    sv.m = xm[(size_t)st_tc * nb + gt];
    __builtin_amdgcn_sched_barrier(0);
  };
  float accf[16];
#pragma unroll
  for (int r = 0; r < 16; r++) accf[r] = 0.f;
  auto stage = [&](int g0, Set& sv) {
    const int kb = g0 * 32;
    if (stager) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int q = tid + i * R4M_NT;
      *(int4*)(sA + (q >> 3) * R4M_AS + (q & 7) * 16) = sel4(kb + (q & 7) * 16 < I, sv.a[i]);
    }
    const bool gok = g0 + (tid & 3) < nb;
#pragma unroll
    for (int i = 0; i < NBC; i++) *(int4*)(sB + (tid >> 2) * BS + (tid & 3) * RB + 16 * i) = sel4(gok, sv.b[i]);
    sD[(tid >> 2) * R4M_KG + (tid & 3)] = gok ? f16_to_f32(sv.d) : 0.f;
    {
      const bool ok = g0 + st_g < nb;
      const float xv = ok ? sv.x : 0.f;
      sX[st_g * 64 + (tid & 63)] = xv;
      sM[st_g * 64 + (tid & 63)] = (ok && !st_tile) ? -8 * sv.m : 0;
      sC[st_g * 64 + (tid & 63)] = (ok && st_tile) ? (8.f * (float)sv.m) * xv : 0.f;
    }
    }
    __syncthreads();
    gload(g0 + 2 * R4M_KG, sv);
    if constexpr (WV >= 8) {
      // wave: tokens wm16 * 16 + [0, 16) x rows wn16 * 16 * JN + [0, 16 * JN)
      const int wm16 = wv / NWN, wn16 = wv % NWN, r16 = lane & 15, q4 = lane >> 4;
      const int ngk = (nb - g0) < R4M_KG ? (nb - g0) : R4M_KG;
      const int tb = wm16 * 16 + 4 * q4;  // this lane's 4 tokens (D rows)
#pragma unroll
      for (int gg = 0; gg < R4M_KG; gg++) {
        if (gg >= ngk) break;  // wave-uniform
        const long a = *(const long*)(sA + (wm16 * 16 + r16) * R4M_AS + gg * 32 + q4 * 8);
        const float4 xv = *(const float4*)(sX + gg * 64 + tb);
        const int4 mv = (Q8 || TILE) ? int4{0, 0, 0, 0} : *(const int4*)(sM + gg * 64 + tb);
        const float4 cv = Q8 ? float4{0.f, 0.f, 0.f, 0.f} : *(const float4*)(sC + gg * 64 + tb);
#pragma unroll
        for (int jn = 0; jn < JN; jn++) {
          const int row = wn16 * 16 * JN + jn * 16 + r16;
          long b;
          if (Q8) {
            b = *(const long*)(sB + row * BS + gg * RB + q4 * 8);
          } else {
            const uint2 w = *(const uint2*)(sB + row * BS + gg * RB + (q4 & 1) * 8);
            const int sh = (q4 >> 1) * 4;
            b = (long)(((w.x >> sh) & 0x0f0f0f0fu) | ((uint64_t)((w.y >> sh) & 0x0f0f0f0fu) << 32));
          }
          const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, v4i{0, 0, 0, 0}, 0, 0, 0);
          const float dd = sD[row * R4M_KG + gg];
          float* ac = accf + 4 * jn;
          if (Q8) {
            ac[0] = __fmaf_rn((float)d[0], dd * xv.x, ac[0]);
            ac[1] = __fmaf_rn((float)d[1], dd * xv.y, ac[1]);
            ac[2] = __fmaf_rn((float)d[2], dd * xv.z, ac[2]);
            ac[3] = __fmaf_rn((float)d[3], dd * xv.w, ac[3]);
          } else {
            ac[0] = __fmaf_rn(-dd, cv.x, __fmaf_rn((float)(d[0] + mv.x), dd * xv.x, ac[0]));
            ac[1] = __fmaf_rn(-dd, cv.y, __fmaf_rn((float)(d[1] + mv.y), dd * xv.y, ac[1]));
            ac[2] = __fmaf_rn(-dd, cv.z, __fmaf_rn((float)(d[2] + mv.z), dd * xv.z, ac[2]));
            ac[3] = __fmaf_rn(-dd, cv.w, __fmaf_rn((float)(d[3] + mv.w), dd * xv.w, ac[3]));
          }
        }
      }
    } else if constexpr (Q8) {
      // Straight-line over the block's groups -- fragments, the MFMAs, then
      // the epilogues in group order -- so the MFMAs overlap.  Groups past
      // the row end hold zero codes and scales: their steps add exactly
      // nothing (fma(0, 0, acc) = acc; acc is never -0).
      if (g0 < nb) {
        v4i af[R4M_KG], bf[R4M_KG];
#pragma unroll
        for (int gg = 0; gg < R4M_KG; gg++) {
          af[gg] = *(const v4i*)(sA + (wm * 32 + r32) * R4M_AS + gg * 32 + hk * 16);
          bf[gg] = *(const v4i*)(sB + (wn * 32 + r32) * BS + gg * RB + hk * 16);
        }
        v16i dsum[R4M_KG];
#pragma unroll
        for (int gg = 0; gg < R4M_KG; gg++)
          dsum[gg] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[gg], bf[gg], v16i{}, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);  // all MFMAs issue before the epilogues
#pragma unroll
        for (int gg = 0; gg < R4M_KG; gg++) {
          const float dd = sD[(wn * 32 + r32) * R4M_KG + gg];
          // D layout: lane l, register r -> token 8*(r/4) + 4*(l/32) + r%4, row l%32
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const float4 xv = *(const float4*)(sX + gg * 64 + wm * 32 + 8 * q + 4 * hk);
            accf[4 * q + 0] = __fmaf_rn((float)dsum[gg][4 * q + 0], dd * xv.x, accf[4 * q + 0]);
            accf[4 * q + 1] = __fmaf_rn((float)dsum[gg][4 * q + 1], dd * xv.y, accf[4 * q + 1]);
            accf[4 * q + 2] = __fmaf_rn((float)dsum[gg][4 * q + 2], dd * xv.z, accf[4 * q + 2]);
            accf[4 * q + 3] = __fmaf_rn((float)dsum[gg][4 * q + 3], dd * xv.w, accf[4 * q + 3]);
          }
        }
      }
    } else {
      // Q4R4 (a heavier epilogue): group by group, within the register budget
      const int ngk = (nb - g0) < R4M_KG ? (nb - g0) : R4M_KG;
#pragma unroll
      for (int gg = 0; gg < R4M_KG; gg++) {
        if (gg >= ngk) break;  // wave-uniform
        const v4i a = *(const v4i*)(sA + (wm * 32 + r32) * R4M_AS + gg * 32 + hk * 16);
        const int4 w = *(const int4*)(sB + (wn * 32 + r32) * BS + gg * RB);
        // this half's nibbles (low for hk = 0, high for hk = 1): one shift
        // and one mask per word in every lane, no divergent branch
        const int sh = 4 * hk;
        const int4 u = int4{(w.x >> sh) & 0x0f0f0f0f, (w.y >> sh) & 0x0f0f0f0f, (w.z >> sh) & 0x0f0f0f0f,
                            (w.w >> sh) & 0x0f0f0f0f};
        v16i dsum = {};
        dsum = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, v4i{u.x, u.y, u.z, u.w}, dsum, 0, 0, 0);
        const float dd = sD[(wn * 32 + r32) * R4M_KG + gg];
        // D layout: lane l, register r -> token 8*(r/4) + 4*(l/32) + r%4, row l%32
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int tb = wm * 32 + 8 * q + 4 * hk;
          const float4 xv = *(const float4*)(sX + gg * 64 + tb);
          // every token in the tile kernel's form (S % 4 == 0): m8 is 0 throughout
          const int4 mv = TILE ? int4{0, 0, 0, 0} : *(const int4*)(sM + gg * 64 + tb);
          const float4 cv = *(const float4*)(sC + gg * 64 + tb);
          accf[4 * q + 0] = __fmaf_rn(-dd, cv.x, __fmaf_rn((float)(dsum[4 * q + 0] + mv.x), dd * xv.x, accf[4 * q + 0]));
          accf[4 * q + 1] = __fmaf_rn(-dd, cv.y, __fmaf_rn((float)(dsum[4 * q + 1] + mv.y), dd * xv.y, accf[4 * q + 1]));
          accf[4 * q + 2] = __fmaf_rn(-dd, cv.z, __fmaf_rn((float)(dsum[4 * q + 2] + mv.z), dd * xv.z, accf[4 * q + 2]));
          accf[4 * q + 3] = __fmaf_rn(-dd, cv.w, __fmaf_rn((float)(dsum[4 * q + 3] + mv.w), dd * xv.w, accf[4 * q + 3]));
        }
      }
    }
    __syncthreads();
  };
  gload(0, s0);
  gload(R4M_KG, s1);
  for (int g0 = 0; g0 < nb; g0 += 2 * R4M_KG) {
    stage(g0, s0);
    stage(g0 + R4M_KG, s1);
  }
  // retire the clamped prefetches once before the conditional stores
  __builtin_amdgcn_s_waitcnt(0);
  if constexpr (WV >= 8) {
    const int wm16 = wv / NWN, wn16 = wv % NWN, r16 = lane & 15, q4 = lane >> 4;
#pragma unroll
    for (int jn = 0; jn < JN; jn++) {
      const int col = nb0 + wn16 * 16 * JN + jn * 16 + r16;
      if (col >= O) continue;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int t = mb + wm16 * 16 + 4 * q4 + r;
        if (t < S) y[(int64_t)t * O + col] = accf[4 * jn + r];
      }
    }
    return;
  }
  if constexpr (PAIR) {
    // up sums (wn = 1) to the gate waves through LDS, [r][wm][lane]
    float* xch = (float*)sA;
    __syncthreads();
    if (wn == 1) {
#pragma unroll
      for (int r = 0; r < 16; r++) xch[r * 128 + wm * 64 + lane] = accf[r];
    }
    __syncthreads();
    const int col = nb0 + r32;
    if (wn == 1 || col >= O) return;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int t = mb + wm * 32 + 8 * (r >> 2) + 4 * hk + (r & 3);
      if (t < S) y[(int64_t)t * O + col] = ref_silu_mul(accf[r], xch[r * 128 + wm * 64 + lane]);
    }
    return;
  }
  const int col = nb0 + wn * 32 + r32;
  if (col >= O) return;
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const int t = mb + wm * 32 + 8 * (r >> 2) + 4 * hk + (r & 3);
    if (t < S) y[(int64_t)t * O + col] = accf[r];
  }
}

// y [S][O] = R4 matmul of x [S][I]; xq/xs/xm: scratch for the activation
// codes (S*I bytes, S*(I/32) floats and ints)
int launch_r4_matmul(bool q8, const float* x, const uint8_t* W, const uint16_t* d16, float* y, int S, int I, int O,
                     int8_t* xq, float* xs, int32_t* xm, hipStream_t st) {
  if (I % 32 || I <= 0) return MOTY_EUNSUP;
  if (S <= 0 || O <= 0) return MOTY_OK;
  if (S <= 3) {
    const int rc = q8 ? launch_r4_gemv<true>(x, W, d16, y, S, I, O, st) : launch_r4_gemv<false>(x, W, d16, y, S, I, O, st);
    if (rc != MOTY_EUNSUP) return rc;
  }
  if (!xq || !xs || !xm) return MOTY_EINVAL;  // the GEMM path needs the activation scratch
  int rc = launch_quant_g32(x, xq, xs, xm, S, I, st);
  if (rc) return rc;
  dim3 grid((O + 63) / 64, (S + 63) / 64);
  // at most one workgroup per CU: sixteen waves of 16 x 16 (four per SIMD
  // instead of one); measured on MI355X at S = 256, 4096 x 12288: Q4R4 92.7
  // us against 132 with four waves (eight: 112), Q8R4 95.9 against 104.  The
  // wider grids keep four waves of 32 x 32 (24576 x 4096: 147 us; eight or
  // sixteen waves 179 / 191).
  const bool few = (int64_t)grid.x * grid.y <= 256;
#define R4G(Q, T, WV) \
  hipLaunchKernelGGL((k_r4_gemm<Q, T, WV>), grid, dim3(64 * WV), 0, st, xq, xs, xm, W, d16, y, S, I, O)
  if (q8) {
    if (few) R4G(true, false, 16);
    else R4G(true, false, 4);
  } else if (S % 4 == 0) {  // every token in the tile kernel's form
    if (few) R4G(false, true, 16);
    else R4G(false, true, 4);
  } else {
    if (few) R4G(false, false, 16);
    else R4G(false, false, 4);
  }
#undef R4G
  LAUNCH_TRY("k_r4_gemm");
  return MOTY_OK;
}

// gate/up + SiLU over a row-fused [gate; up] R4 matrix (2*I rows) for S > 3
// tokens: h [S][I] = silu(x.gate^T) * (x.up^T) in one GEMM pass (PAIR tiles)
int launch_r4_gate_up_gemm(bool q8, const float* x, const uint8_t* W, const uint16_t* d16, float* h, int S, int D,
                           int I, int8_t* xq, float* xs, int32_t* xm, hipStream_t st) {
  if (D % 32 || D <= 0 || I % 4 || I <= 0) return MOTY_EUNSUP;
  if (S <= 0) return MOTY_OK;
  int rc = launch_quant_g32(x, xq, xs, xm, S, D, st);
  if (rc) return rc;
  dim3 grid((I + 31) / 32, (S + 63) / 64);
#define R4P(Q, T) hipLaunchKernelGGL((k_r4_gemm<Q, T, 4, true>), grid, dim3(R4M_NT), 0, st, xq, xs, xm, W, d16, h, S, D, I)
  if (q8) R4P(true, false);
  else if (S % 4 == 0) R4P(false, true);
  else R4P(false, false);
#undef R4P
  LAUNCH_TRY("k_r4_gemm<pair>");
  return MOTY_OK;
}

// Decode gate/up + SiLU over a row-fused [gate; up] R4 matrix (2*I rows,
// the gate_up of nn/ffn.c:28-37): h [I] = silu(x.gate^T) * (x.up^T), one token.
int launch_r4_gate_up_silu(bool q8, const float* x, const uint8_t* W, const uint16_t* d16, float* h, int D, int I,
                           hipStream_t st) {
  if (D % 32 || D <= 0 || I % 4 || I <= 0) return MOTY_EUNSUP;
  return q8 ? go_r4_gemv_ic<true, 1, true>(x, W, d16, h, 1, D, I, st)
            : go_r4_gemv_ic<false, 1, true>(x, W, d16, h, 1, D, I, st);
}

// ---------------------------------------------------------------------------
// Packers (nn/quant.c:130-177): thread per (block, group, row).  The group
// scale is the "no-clip Q4_0" rule: mx = the largest-magnitude weight (the
// first one on ties), opp = the largest |w| of the other sign, d =
// -sign(mx) * max(|mx|/lo, opp/hi) rounded to f16 (nearest even), codes
// rint(w / d) via the reciprocal of the rounded scale, clipped.

// float -> IEEE half, round to nearest even (nn/quant.c:111-128)
__device__ __forceinline__ uint32_t f32_to_f16(float f) {
  const uint32_t x = __float_as_uint(f);
  const uint32_t sign = (x >> 16) & 0x8000u, e = (x >> 23) & 0xffu;
  uint32_t m = x & 0x7fffffu;
  if (e == 0xffu) return sign | 0x7c00u | (m ? 0x200u : 0u);
  const int ne = (int)e - 127 + 15;
  if (ne >= 31) return sign | 0x7c00u;
  if (ne <= 0) {
    if (ne < -10) return sign;
    m |= 0x800000u;
    const int sh = 14 - ne;
    uint32_t h = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (h & 1))) h++;
    return sign | h;
  }
  uint32_t h = ((uint32_t)ne << 10) | (m >> 13);
  const uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
  return sign | h;
}

template <bool Q8>
__global__ __launch_bounds__(256) void k_pack_r4(const float* __restrict__ w, uint8_t* __restrict__ q,
                                                 uint16_t* __restrict__ d16, int O, int I) {
  const int nb = I / 32, O4 = (O + 3) / 4;
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (block, group, row)
  if (id >= (int64_t)O4 * nb * 4) return;
  const int r = (int)(id & 3);
  const int64_t bg = id >> 2;
  const int g = (int)(bg % nb), b = (int)(bg / nb);
  const int row = b * 4 + r;
  constexpr int GB = Q8 ? 128 : 64;
  uint8_t* dst = q + (size_t)bg * GB + r * (Q8 ? 32 : 16);
  if (row >= O) {
#pragma unroll
    for (int j = 0; j < (Q8 ? 32 : 16); j += 4) *(uint32_t*)(dst + j) = Q8 ? 0u : 0x88888888u;
    d16[(size_t)bg * 4 + r] = 0;
    return;
  }
  const float* wg = w + (size_t)row * I + g * 32;
  float v[32];
#pragma unroll
  for (int j = 0; j < 32; j += 4) *(float4*)(v + j) = *(const float4*)(wg + j);
  float mx = 0.f;
#pragma unroll
  for (int j = 0; j < 32; j++) mx = fabsf(v[j]) > fabsf(mx) ? v[j] : mx;
  float opp = 0.f;
#pragma unroll
  for (int j = 0; j < 32; j++) opp = ((v[j] > 0) != (mx > 0) && fabsf(v[j]) > opp) ? fabsf(v[j]) : opp;
  const float lo = Q8 ? 128.f : 8.f, hi = Q8 ? 127.f : 7.f;
  const float dm = fmaxf(fabsf(mx) / lo, opp / hi);
  const uint32_t h = f32_to_f16(mx > 0 ? -dm : dm);
  const float dd = f16_to_f32(h), inv = dd != 0.f ? 1.f / dd : 0.f;
  d16[(size_t)bg * 4 + r] = (uint16_t)h;
  int c[32];
#pragma unroll
  for (int j = 0; j < 32; j++) {
    int t = rne_int(v[j] * inv);
    t = t < (Q8 ? -128 : -8) ? (Q8 ? -128 : -8) : t;
    t = t > (Q8 ? 127 : 7) ? (Q8 ? 127 : 7) : t;
    c[j] = t;
  }
  if (Q8) {
#pragma unroll
    for (int j = 0; j < 32; j += 4)
      *(uint32_t*)(dst + j) = (uint32_t)(c[j] & 0xff) | ((uint32_t)(c[j + 1] & 0xff) << 8) |
                              ((uint32_t)(c[j + 2] & 0xff) << 16) | ((uint32_t)(c[j + 3] & 0xff) << 24);
  } else {
#pragma unroll
    for (int j = 0; j < 16; j += 4) {
      uint32_t p = 0;
#pragma unroll
      for (int u = 0; u < 4; u++)
        p |= ((uint32_t)(c[j + u] + 8) | ((uint32_t)(c[j + u + 16] + 8) << 4)) << (8 * u);
      *(uint32_t*)(dst + j) = p;
    }
  }
}

int launch_pack_r4(bool q8, const float* w, uint8_t* q, uint16_t* d16, int O, int I, hipStream_t st) {
  if (I % 32 || I <= 0) return MOTY_EUNSUP;
  if (O <= 0) return MOTY_OK;
  const int64_t n = (int64_t)((O + 3) / 4) * (I / 32) * 4;
  const unsigned nbk = (unsigned)((n + 255) / 256);
  if (q8)
    hipLaunchKernelGGL(k_pack_r4<true>, dim3(nbk), dim3(256), 0, st, w, q, d16, O, I);
  else
    hipLaunchKernelGGL(k_pack_r4<false>, dim3(nbk), dim3(256), 0, st, w, q, d16, O, I);
  LAUNCH_TRY("k_pack_r4");
  return MOTY_OK;
}

}  // namespace moty
