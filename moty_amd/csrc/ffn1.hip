// ffn1.hip -- the Q8 decode FFN (S = 1) in one launch.
//
// Reference: moty_ffn (nn/ffn.c:26-55) over moty_matmul_q_s (nn/matmul.c:51-66):
//     xq = qrow_i8(x);  g = (gs*sx)*dot(G, xq);  u = (us*sx)*dot(U, xq)
//     h = silu(g)*u  (hw/hw_ops.h:19-21);  hq = qrow_i8(h)
//     y = (ds*sh)*dot(Dn, hq)
//
// Two dependent GEMV launches pay the launch and drain latency twice, and
// the down weights cannot start streaming before the gate/up launch ends.
// This form does the whole FFN in one grid of exactly one workgroup per CU
// (all co-resident), handing h between workgroups through device memory.
// Every exchanged word is {tag, value} in 64 bits, written and read with
// agent-scope atomics (single-copy atomic, coherent across the XCDs' L2s),
// re-read until its tag is this call's: no flag, counter, fence or cache
// write-back stands between h and its readers.  The tag is a per-workgroup
// call counter kept in device memory (every call runs the same grid, so the
// counters stay equal), so graph replays need no new kernel arguments.
// Every wait is bounded: a wait that runs out sets a device error flag
// (moty_hip_wait_errors) and that call's output is invalid, but every wave
// still exits.
//
// Measured on MI355X at C1's shape (D = 1024, I = 3072) it is bit-exact and
// slower than the two launches (6.8 against 5.7 us per FFN), so it is off
// unless moty_hip_set_ffn1(1) selects it: a cross-XCD hand-off costs about
// 0.5 us one way, the last workgroup's h is ready 1.2 us after the first's,
// and the chain from the last h to y (fetch, gather, amax, quantize, dots)
// adds more than a kernel boundary saves.
#include "common.h"
#include "kernels.h"

namespace moty {

constexpr int F1_CHUNK = 16 * MOTY_WAVE;  // bytes of a row one wave-load covers
constexpr int F1_SPIN = 1 << 18;          // bound on re-reads of one word

// the XCD (accelerator complex) this wave runs on
__device__ __forceinline__ unsigned xcc_id() {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(v));
  return v;
}

__device__ __forceinline__ int4 f1_ldnt16(const int8_t* p) {
  const v4i v = __builtin_nontemporal_load((const v4i*)p);
  return int4{v.x, v.y, v.z, v.w};
}

// ---------------------------------------------------------------------------
// XCD-hierarchical form (256 workgroups; I % 1024 == 0, I <= 4096,
// D % 1024 == 0, D <= 2048).  Workgroup b computes h rows [b*I/256, +I/256)
// (four per gate/up wave) and the full down rows [b*D/256, +D/256) (four per
// down wave).  Every workgroup needs all of h, so h crosses the chip once per
// XCD, not once per workgroup:
//  1. a gate/up wave writes its h words through to memory (agent scope);
//  2. fetch: workgroup b reads words [(b/8)*I/32, +I/32) from there and
//     re-publishes them with plain stores into its XCD's copy of h, which
//     stay in that XCD's L2 (the 32 workgroups on an XCD together fetch all
//     I words: workgroups are dispatched round-robin over the 8 XCDs);
//  3. gather: every workgroup reads its XCD's copy (device-scope loads, which
//     find the plain stores of the same XCD in its L2), takes the row's amax,
//     quantizes h into LDS (qrow_i8) and finishes its down rows.
// A workgroup that finds itself on an unexpected XCD still fetches into the
// copy of the XCD it runs on, and a gather that finds a word missing from its
// copy for long reads it from the written-through words instead, so results
// never depend on the dispatch order (only the speed does).
// The down wave issues its weight loads once the gate/up rows have landed,
// so the inputs of h lead the weight stream.
template <int NC, int KC, int DWV>
__global__ __launch_bounds__((KC + DWV) * MOTY_WAVE) void k_ffn1h_q8(
    const float* __restrict__ x, const int8_t* __restrict__ G, const float* __restrict__ gs,
    const int8_t* __restrict__ U, const float* __restrict__ us, const int8_t* __restrict__ Dn,
    const float* __restrict__ ds, float* __restrict__ y, int D, int I, unsigned long long* __restrict__ xh,
    unsigned* __restrict__ epoch, unsigned* __restrict__ err) {
  constexpr int GW = KC;                  // gate/up waves: I/256 rows, 4 per wave
  constexpr int NW = GW + DWV;
  constexpr int NT = NW * MOTY_WAVE;
  constexpr int NI = KC * F1_CHUNK;       // I
  constexpr int NJ = (NI + NT - 1) / NT;  // gathered words per thread
  constexpr int NF = NI / 32;             // fetched words per workgroup
  constexpr int LOCAL_SPIN = 4096;        // local rounds before reading the written-through words
  __shared__ __align__(16) int8_t hq_s[NI];
  __shared__ float red[NW];
  __shared__ int g_in;                    // the gate/up rows have landed
  unsigned long long* const Hx = xh;                               // [I] written-through h words
  const int lane = threadIdx.x % MOTY_WAVE, wv = threadIdx.x / MOTY_WAVE;
  const int b = blockIdx.x;
  const unsigned xcc = xcc_id();
  unsigned long long* const Lx = xh + 4096 + (size_t)(xcc & 7) * 4096;  // this XCD's copy
  const int rl = wave_sum_row<4>(lane);
  if (threadIdx.x == 0) g_in = 0;
  __syncthreads();
  unsigned tag;
  int4 wd[4][KC];
  float dsc = 0.f;
  int orow = 0;
  if (wv < GW) {
    tag = __hip_atomic_load(epoch + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    const int grow0 = b * (NI / 256) + wv * 4;
    float4 xv[NC][4];
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const int k = c * F1_CHUNK + lane * 16;
#pragma unroll
      for (int j = 0; j < 4; j++) xv[c][j] = *(const float4*)(x + (k < D ? k : 0) + 4 * j);
    }
    int4 wgt[4][NC], wup[4][NC];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const int k = c * F1_CHUNK + lane * 16;
        const int kc = k < D ? k : 0;
        wgt[r][c] = f1_ldnt16(G + (int64_t)(grow0 + r) * D + kc);
        wup[r][c] = f1_ldnt16(U + (int64_t)(grow0 + r) * D + kc);
      }
    const float sg = gs[grow0 + rl], su = us[grow0 + rl];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
      for (int j = 0; j < 4; j++) xv[c][j] = sel4(c * F1_CHUNK + lane * 16 < D, xv[c][j]);
    float amax = 0.f;
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
      for (int j = 0; j < 4; j++)
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(xv[c][j].x), fabsf(xv[c][j].y)),
                                 fmaxf(fabsf(xv[c][j].z), fabsf(xv[c][j].w))));
    amax = wave_max_f32(amax);
    float sx = amax / 127.f;
    if (sx < 1e-12f) sx = 1e-12f;
    const float inv = 1.f / sx;
    int4 q[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
      int* qp = (int*)&q[c];
#pragma unroll
      for (int j = 0; j < 4; j++)
        qp[j] = (int)((uint32_t)(rne_int(xv[c][j].x * inv) & 0xff) |
                      ((uint32_t)(rne_int(xv[c][j].y * inv) & 0xff) << 8) |
                      ((uint32_t)(rne_int(xv[c][j].z * inv) & 0xff) << 16) |
                      ((uint32_t)(rne_int(xv[c][j].w * inv) & 0xff) << 24));
    }
    int ag[4], au[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      ag[r] = 0;
      au[r] = 0;
#pragma unroll
      for (int c = 0; c < NC; c++) {
        ag[r] = dot16(wgt[r][c], q[c], ag[r]);
        au[r] = dot16(wup[r][c], q[c], au[r]);
      }
    }
    // the weights of this wave are in (the dots above used them): let the
    // down wave start its stream
    asm volatile("" ::"v"(ag[0]), "v"(au[0]) : "memory");
    if (wv == 0 && lane == 0) __hip_atomic_store(&g_in, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const int a = wave_sum_multi_i32<4>(ag);
    const int a2 = wave_sum_multi_i32<4>(au);
    const float h = ref_silu_mul((sg * sx) * (float)a, (su * sx) * (float)a2);
    if ((lane & 15) == 0)
      __hip_atomic_store(Hx + grow0 + rl, ((unsigned long long)tag << 32) | __float_as_uint(h), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    // fetch this workgroup's share of h into the XCD's copy
    if (threadIdx.x < NF) {
      const int i = (b / 8) * NF + threadIdx.x;
      unsigned long long v = 0;
      for (int spin = 0;; spin++) {
        v = __hip_atomic_load(Hx + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((unsigned)(v >> 32) == tag) break;
        if (spin == F1_SPIN) {
          __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      Lx[i] = v;
    }
  } else {
    // down wave: start its weight stream once the gate/up rows are in
    tag = __hip_atomic_load(epoch + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    for (int spin = 0; spin < F1_SPIN && !__hip_atomic_load(&g_in, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
         spin++)
      __builtin_amdgcn_s_sleep(2);
    const int o0 = b * (D / 256) + (wv - GW) * 4;
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int c = 0; c < KC; c++) wd[r][c] = f1_ldnt16(Dn + (int64_t)(o0 + r) * I + c * F1_CHUNK + lane * 16);
    orow = o0 + rl;
    dsc = ds[orow];
  }

  // gather all of h from the XCD's copy
  unsigned long long w[NJ];
  for (int spin = 0;; spin++) {
    unsigned long long* const src = spin < LOCAL_SPIN ? Lx : Hx;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const int i = threadIdx.x + j * NT;
      const unsigned long long v = __hip_atomic_load(src + (i < NI ? i : 0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      w[j] = i < NI ? v : (unsigned long long)tag << 32;
    }
    bool ok = true;
#pragma unroll
    for (int j = 0; j < NJ; j++) ok = ok && (unsigned)(w[j] >> 32) == tag;
    if (ok) break;
    if (spin == LOCAL_SPIN + F1_SPIN) {
      __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; j++) amax = fmaxf(amax, fabsf(__uint_as_float((unsigned)w[j])));
  amax = wave_max_f32(amax);
  if (lane == 0) red[wv] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int i = 1; i < NW; i++) amax = fmaxf(amax, red[i]);
  float sh = amax / 127.f;
  if (sh < 1e-12f) sh = 1e-12f;
  const float inv = 1.f / sh;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int i = threadIdx.x + j * NT;
    if (i < NI) hq_s[i] = (int8_t)rne_int(__uint_as_float((unsigned)w[j]) * inv);
  }
  __syncthreads();
  if (wv >= GW) {
    int4 hq[KC];
#pragma unroll
    for (int c = 0; c < KC; c++) hq[c] = *(const int4*)(hq_s + c * F1_CHUNK + lane * 16);
    int acc[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      acc[r] = 0;
#pragma unroll
      for (int c = 0; c < KC; c++) acc[r] = dot16(wd[r][c], hq[c], acc[r]);
    }
    const int a = wave_sum_multi_i32<4>(acc);
    if ((lane & 15) == 0) y[orow] = (dsc * sh) * (float)a;
  }
  if (threadIdx.x == 0) __hip_atomic_store(epoch + b, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int ffn1h_q8_fits(int D, int I, int nwg) {
  return nwg == 256 && I % 1024 == 0 && I <= 4096 && D % 1024 == 0 && D <= 2048;
}

int launch_ffn1h_q8(const float* x, const int8_t* G, const float* gs, const int8_t* U, const float* us,
                    const int8_t* Dn, const float* ds, float* y, int D, int I, int nwg, unsigned long long* xh,
                    unsigned* epoch, unsigned* err, hipStream_t st) {
  if (!ffn1h_q8_fits(D, I, nwg)) return MOTY_EUNSUP;
  const int kc = I / 1024, dwv = D / 1024;
#define FH(A, B, C)                                                                                           \
  if (D / 1024 == A && kc == B && dwv == C) {                                                                 \
    hipLaunchKernelGGL((k_ffn1h_q8<A, B, C>), dim3(256), dim3((B + C) * MOTY_WAVE), 0, st, x, G, gs, U, us,    \
                       Dn, ds, y, D, I, xh, epoch, err);                                                      \
    LAUNCH_TRY("k_ffn1h_q8");                                                                                 \
    return MOTY_OK;                                                                                           \
  }
  FH(1, 1, 1) FH(1, 2, 1) FH(1, 3, 1) FH(1, 4, 1) FH(2, 1, 2) FH(2, 2, 2) FH(2, 3, 2) FH(2, 4, 2)
#undef FH
  return MOTY_EUNSUP;
}

}  // namespace moty
