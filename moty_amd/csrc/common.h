// common.h -- shared device helpers for libmoty-hw-hip (gfx950, wave64).
//
// Everything in this library is compiled with -ffp-contract=off: every FMA
// is written explicitly where the reference's x86-64 build forms one, so
// the float results match the reference bit for bit.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define MOTY_WAVE 64

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// expf, bit-identical to glibc 2.35 expf on x86-64 (hw/hw_ops.h:20 calls it).
// Method: ARM optimized-routines expf (Szabolcs Nagy), as glibc builds it with
// FMA contraction: k = round(x*32/ln2), r = x*32/ln2 - k,
// exp(x) = 2^(k/32) * (1 + C2 r + C1 r^2 + C0 r^3) in double, rounded once
// to float.  T2[i] = bits(2^(i/32)) - (i << 47).  The same steps, checked on
// every one of the 2^32 float inputs against libm, are the test oracle.
__constant__ static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};

__device__ __forceinline__ float ref_expf(float x) {
  const double kC0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  const double kC1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  const double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
  const double kShift = 0x1.8p+52;
  uint32_t ux = __float_as_uint(x);
  uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= 0x42b) {                 // |x| >= 88, inf or nan
    if (ux == 0xff800000u) return 0.f;   // -inf
    if (abstop >= 0x7f8) return x + x;   // inf / nan
    if (x > 0x1.62e42ep6f) return __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.f;
  }
  double xd = (double)x;
  double kd = __fma_rn(kInvLn2N, xd, kShift);
  uint64_t ki = (uint64_t)__double_as_longlong(kd);
  kd = kd - kShift;
  double r = __fma_rn(kInvLn2N, xd, -kd);
  uint64_t t = kExp2Tab[ki & 31] + (ki << 47);
  double s = __longlong_as_double((long long)t);
  double z = __fma_rn(kC0, r, kC1);
  double r2 = r * r;
  double y = __fma_rn(kC2, r, 1.0);
  y = __fma_rn(z, r2, y);
  y = y * s;
  return (float)y;
}

// g / (1 + expf(-g)) * u  (hw/hw_ops.h:19-21); division correctly rounded.
__device__ __forceinline__ float ref_silu_mul(float g, float u) {
  return (g / (1.f + ref_expf(-g))) * u;
}

// Branch-free "ok ? v : 0" for a value loaded from a clamped (always valid)
// address: a predicated load would split the wave's loads into branches and
// force a wait for every load in flight at the join.
__device__ __forceinline__ int4 sel4(bool ok, int4 v) {
  return int4{ok ? v.x : 0, ok ? v.y : 0, ok ? v.z : 0, ok ? v.w : 0};
}
__device__ __forceinline__ float4 sel4(bool ok, float4 v) {
  return float4{ok ? v.x : 0.f, ok ? v.y : 0.f, ok ? v.z : 0.f, ok ? v.w : 0.f};
}
// lrintf under the default round-to-nearest-even mode, as an int.
__device__ __forceinline__ int rne_int(float v) { return (int)__builtin_rintf(v); }

// IEEE half (bits) -> float, exact for every half (hw/hw_q4r4.h:22-33):
// normals and inf/nan by re-biasing, subnormals as m * 2^-24 (exact: m has
// 10 bits and the product is a normal float).
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  const uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  const uint32_t un = s | ((e + 112u) << 23) | (m << 13);
  const uint32_t ui = s | 0x7f800000u | (m << 13);
  const uint32_t us = s | __float_as_uint((float)m * 5.9604644775390625e-8f);
  return __uint_as_float(e == 0u ? us : (e == 31u ? ui : un));
}

// ---------------------------------------------------------------------------
// 16 bytes per lane from global memory straight into LDS, at lds_base +
// 16*lane (global_load_lds_dwordx4; lds_base must be wave-uniform).  Written
// as inline asm so that the compiler's wait insertion does not see an LDS
// write in flight -- it would wait for every outstanding load before each
// LDS read -- callers order it themselves with vmcnt waits and barriers.
// m0 (the LDS base register) is saved and restored around the load.
__device__ __forceinline__ void dma16_to_lds(const void* g, uint32_t lds_base) {
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(g), "s"(lds_base));
}

// Buffer resource over `bytes` bytes at p (raw, stride 0): loads past the
// end return zeros instead of faulting.
__device__ __forceinline__ v4i buf_rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  return v4i{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
             __builtin_amdgcn_readfirstlane((int)(uint32_t)((a >> 32) & 0xffffu)),
             __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
}

// 16 bytes per lane from buffer offset voff + soff straight into LDS at
// lds_base + 16*lane (buffer_load_dwordx4 ... lds); as dma16_to_lds, the
// caller orders it with vmcnt waits and barriers.
__device__ __forceinline__ void bdma16_to_lds(v4i rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base) {
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "buffer_load_dwordx4 %1, %2, %4 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(voff), "s"(rsrc), "s"(lds_base), "s"(soff));
}

// s_waitcnt vmcnt(n) alone (expcnt and lgkmcnt left at their maxima)
#define MOTY_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

// ---------------------------------------------------------------------------
// Cross-lane moves without LDS: DPP within 16-lane rows and the gfx950
// permlane swaps across rows / halves (VALU latency, where ds_bpermute
// behind __shfl costs an LDS round trip per step).
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
#define MOTY_DPP_QXOR1 0xB1   // quad_perm [1,0,3,2]: lane ^ 1
#define MOTY_DPP_QXOR2 0x4E   // quad_perm [2,3,0,1]: lane ^ 2
#define MOTY_DPP_ROR4 0x124   // row_ror:4: lane i of a row takes lane (i - 4) & 15
#define MOTY_DPP_ROR8 0x128   // row_ror:8: lane ^ 8 within the row
#define MOTY_DPP_ROR12 0x12C  // row_ror:12: lane i takes lane (i + 4) & 15
__device__ __forceinline__ int xor16_i(int v) {  // value of lane ^ 16
  const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
  return (int)((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ int xor32_i(int v) {  // value of lane ^ 32
  const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
  return (int)((threadIdx.x & 32) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor16_f(float v) { return __int_as_float(xor16_i(__float_as_int(v))); }
__device__ __forceinline__ float xor32_f(float v) { return __int_as_float(xor32_i(__float_as_int(v))); }

// wave64 all-reductions (order-free operations: every lane gets the result)
__device__ __forceinline__ int wave_sum_i32(int v) {
  v += dpp_i<MOTY_DPP_QXOR1>(v);
  v += dpp_i<MOTY_DPP_QXOR2>(v);
  v += dpp_i<MOTY_DPP_ROR4>(v);
  v += dpp_i<MOTY_DPP_ROR8>(v);
  v += xor16_i(v);
  return v + xor32_i(v);
}
// Integer wave sums of RPW = 1, 2 or 4 values at once (exact: integer adds
// in any order).  Pairs of registers are folded by permlane swaps, each
// swap + add halving the lanes a value spans while packing two values into
// one register, then each 16-lane row by DPP: 4 values cost 10 VALU
// operations instead of 4 x 8.  Lane l then holds the total of value
// wave_sum_row<RPW>(l): RPW 4: value [0, 2, 1, 3][l / 16]; RPW 2: l / 32.
template <int RPW>
__device__ __forceinline__ int wave_sum_row(int lane) {
  return RPW == 4 ? (((lane >> 4) & 1) << 1) | (lane >> 5) : RPW == 2 ? lane >> 5 : 0;
}
__device__ __forceinline__ int fold32_i(int a, int b) {  // lanes 0-31: a's halves, 32-63: b's
  const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)a, (uint32_t)b, false, false);
  return (int)r[0] + (int)r[1];
}
__device__ __forceinline__ int fold16_i(int a, int b) {  // per 32-lane half: rows a, b
  const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)a, (uint32_t)b, false, false);
  return (int)r[0] + (int)r[1];
}
__device__ __forceinline__ int row_sum_i32(int v) {
  v += dpp_i<MOTY_DPP_QXOR1>(v);
  v += dpp_i<MOTY_DPP_QXOR2>(v);
  v += dpp_i<MOTY_DPP_ROR4>(v);
  return v + dpp_i<MOTY_DPP_ROR8>(v);
}
template <int RPW>
__device__ __forceinline__ int wave_sum_multi_i32(const int (&v)[RPW]) {
  static_assert(RPW == 1 || RPW == 2 || RPW == 4, "1, 2 or 4 values");
  if constexpr (RPW == 4) return row_sum_i32(fold16_i(fold32_i(v[0], v[1]), fold32_i(v[2], v[3])));
  else if constexpr (RPW == 2) {
    const int t = fold32_i(v[0], v[1]);
    return row_sum_i32(fold16_i(t, t));
  } else {
    return wave_sum_i32(v[0]);
  }
}
// inclusive prefix sum over the wave's lanes: row_shr steps within each
// 16-lane row (lanes shifted in from before the row read 0), then the
// totals of the rows below
__device__ __forceinline__ int wave_incl_scan_i32(int v) {
  v += dpp_i<0x111>(v);  // row_shr:1
  v += dpp_i<0x112>(v);  // row_shr:2
  v += dpp_i<0x114>(v);  // row_shr:4
  v += dpp_i<0x118>(v);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31);
  const int r2 = __builtin_amdgcn_readlane(v, 47);
  const int row = (threadIdx.x % 64) >> 4;
  return v + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}
__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, dpp_f<MOTY_DPP_QXOR1>(v));
  v = fmaxf(v, dpp_f<MOTY_DPP_QXOR2>(v));
  v = fmaxf(v, dpp_f<MOTY_DPP_ROR4>(v));
  v = fmaxf(v, dpp_f<MOTY_DPP_ROR8>(v));
  v = fmaxf(v, xor16_f(v));
  return fmaxf(v, xor32_f(v));
}

// 4 signed int8 x 4 signed int8 -> int32 accumulate (v_dot4_i32_i8)
__device__ __forceinline__ int dot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}
__device__ __forceinline__ int dot16(const int4 a, const int4 b, int c) {
  c = dot4(a.x, b.x, c);
  c = dot4(a.y, b.y, c);
  c = dot4(a.z, b.z, c);
  c = dot4(a.w, b.w, c);
  return c;
}

// 8 packed int4 bytes (16 nibbles, even element in the low nibble, value
// n in 0..15 standing for n-8) -> 16 signed int8 (n-8) in element order.
// Per input word: low and high nibbles masked out as bytes, interleaved
// back into element order by two byte permutes, then n-8 per byte without
// carries between bytes: n + 0x78 stays below 0x100, and flipping bit 7
// turns it into n - 8 in two's complement.
__device__ __forceinline__ uint32_t nib_minus8(uint32_t t) { return (t + 0x78787878u) ^ 0x80808080u; }
__device__ __forceinline__ int4 unpack_nib16(uint2 w) {
  const uint32_t l0 = w.x & 0x0f0f0f0fu, h0 = (w.x >> 4) & 0x0f0f0f0fu;
  const uint32_t l1 = w.y & 0x0f0f0f0fu, h1 = (w.y >> 4) & 0x0f0f0f0fu;
  // perm(hi, lo, sel): byte k of the result = byte sel_k of {hi:lo} (lo = bytes 0..3)
  int4 r;
  r.x = (int)nib_minus8(__builtin_amdgcn_perm(h0, l0, 0x05010400u));  // elements 0..3
  r.y = (int)nib_minus8(__builtin_amdgcn_perm(h0, l0, 0x07030602u));  // 4..7
  r.z = (int)nib_minus8(__builtin_amdgcn_perm(h1, l1, 0x05010400u));  // 8..11
  r.w = (int)nib_minus8(__builtin_amdgcn_perm(h1, l1, 0x07030602u));  // 12..15
  return r;
}

// The same 16 codes as unsigned bytes n (0..15), for dots whose -8*sum(x)
// term is added separately (its accumulator starts there).
__device__ __forceinline__ int4 unpack_nib16_u(uint2 w) {
  const uint32_t l0 = w.x & 0x0f0f0f0fu, h0 = (w.x >> 4) & 0x0f0f0f0fu;
  const uint32_t l1 = w.y & 0x0f0f0f0fu, h1 = (w.y >> 4) & 0x0f0f0f0fu;
  int4 r;
  r.x = (int)__builtin_amdgcn_perm(h0, l0, 0x05010400u);
  r.y = (int)__builtin_amdgcn_perm(h0, l0, 0x07030602u);
  r.z = (int)__builtin_amdgcn_perm(h1, l1, 0x05010400u);
  r.w = (int)__builtin_amdgcn_perm(h1, l1, 0x07030602u);
  return r;
}

// ---------------------------------------------------------------------------
// 16-lane horizontal sum with gcc's _mm512_reduce_add_ps association:
// v[j+8]+v[j], then [j+4]+[j], then (b0+b2)+(b1+b3).  `v` is lane c's value
// for c in 0..15 of a 32-lane half (lanes 16..31 unused).  Returns the sum
// in every lane of the half.
__device__ __forceinline__ float hsum16_half(float v, int base) {
  const int c = threadIdx.x % 32;
  float a = __shfl(v, base + ((c + 8) & 15), 64) + v;  // valid for c < 8
  float b = __shfl(a, base + ((c + 4) & 7), 64) + a;   // valid for c < 4
  float b2 = __shfl(b, base + 2, 64), b0 = __shfl(b, base + 0, 64);
  float b3 = __shfl(b, base + 3, 64), b1 = __shfl(b, base + 1, 64);
  return (b0 + b2) + (b1 + b3);
}

// exact dot_f32 (AVX512 order) of x with a W row, computed by a 32-lane
// half-wave; returns the dot in every lane of the half.  Lane c owns chain c
// (s0[c] for c < 16, s1[c-16] for c >= 16); loads are batched 16 steps ahead
// of the FMA chain, which keeps the reference's order.
__device__ __forceinline__ float dot_f32_half(const float* __restrict__ xs, const float* __restrict__ wr, int n) {
  const int c = threadIdx.x % 32;
  const int base = (threadIdx.x % MOTY_WAVE) & 32;
  float s = 0.f;
  int i = 0;
  for (; i + 32 * 16 <= n; i += 32 * 16) {
    float w[16], x[16];
#pragma unroll
    for (int u = 0; u < 16; u++) {
      w[u] = wr[i + 32 * u + c];
      x[u] = xs[i + 32 * u + c];
    }
#pragma unroll
    for (int u = 0; u < 16; u++) s = __fmaf_rn(x[u], w[u], s);
  }
  for (; i + 32 <= n; i += 32) s = __fmaf_rn(xs[i + c], wr[i + c], s);
  if (i + 16 <= n) {
    if (c < 16) s = __fmaf_rn(xs[i + c], wr[i + c], s);
    i += 16;
  }
  const float t = s + __shfl(s, base + ((c + 16) & 31), 64);  // s0[c] + s1[c]
  float r = hsum16_half(t, base);
  for (; i < n; i++) r = __fmaf_rn(xs[i], wr[i], r);
  return r;
}

// ---------------------------------------------------------------------------
// host-side plumbing shared by the translation units
namespace moty {
void set_error(const char* fmt, ...);
int check_hip(hipError_t e, const char* what);
}  // namespace moty

#define MOTY_OK 0
#define MOTY_EINVAL 1   // bad argument / shape
#define MOTY_EHIP 2     // HIP runtime error
#define MOTY_ENOMEM 3   // device allocation failed
#define MOTY_EUNSUP 4   // shape/format not supported by this backend

#define HIP_TRY(call)                                           \
  do {                                                          \
    hipError_t _e = (call);                                     \
    if (_e != hipSuccess) return moty::check_hip(_e, #call);    \
  } while (0)

#define LAUNCH_TRY(what)                                        \
  do {                                                          \
    hipError_t _e = hipGetLastError();                          \
    if (_e != hipSuccess) return moty::check_hip(_e, what);     \
  } while (0)
