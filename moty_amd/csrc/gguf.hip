// gguf.hip -- GGUF block formats to the device layouts, on the device.
//
// Reference: io/gguf.h:231-330 (block dequantisers behind st_read_f32),
// io/gguf.h:335-357 (gguf_repack_q4_0, the lossless Q4_0 -> grouped int4
// repack used by runtime/rt_model_load.h:26-34), io/st.h:74-80 (type ids,
// block sizes).
//
// Every format is an array of fixed-size blocks, and both outputs are linear
// in the block index: block b dequantizes to floats [b*E, (b+1)*E), and
// repacks to bytes [16b, 16b+16) of the int4 matrix plus scale b.  A
// workgroup takes a run of whole blocks, stages their bytes through LDS with
// 16-byte loads (the runs are multiples of 16 bytes), then each thread builds
// float4 (or 16-byte) outputs whose stores are contiguous across the wave.
// The work is a byte stream: HBM-bound, no matrix cores.
//
// Arithmetic, as the reference's x86 build evaluates it:
//   Q8_0  d*q                 Q4_0  d*(nib-8)
//   Q4_K / Q5_K  fma(d*sc, q, -(dmin*mn))   (d*sc*q is exact in f32: an
//                                            f16 mantissa times 6 + 5 bits)
//   Q6_K  (d*sc)*(q-32)
#include "common.h"
#include "kernels.h"

namespace moty {

constexpr int GG_TPB = 256;

template <int DT>
struct GG;
template <>
struct GG<GG_Q8_0> { static constexpr int E = 32, B = 34, NBW = 256; };
template <>
struct GG<GG_Q4_0> { static constexpr int E = 32, B = 18, NBW = 256; };
template <>
struct GG<GG_Q4_K> { static constexpr int E = 256, B = 144, NBW = 32; };
template <>
struct GG<GG_Q5_K> { static constexpr int E = 256, B = 176, NBW = 32; };
template <>
struct GG<GG_Q6_K> { static constexpr int E = 256, B = 210, NBW = 32; };

// Bytes [src, src+n) of global memory into LDS; ALIGNED: src is 16-byte
// aligned (n is then a multiple of 16 for every run but the last).
template <bool ALIGNED>
__device__ __forceinline__ void gg_stage(uint8_t* lds, const uint8_t* __restrict__ src, int n) {
  if (ALIGNED) {
    const int n16 = n >> 4;
    for (int i = threadIdx.x; i < n16; i += GG_TPB)
      reinterpret_cast<uint4*>(lds)[i] = reinterpret_cast<const uint4*>(src)[i];
    for (int i = (n16 << 4) + threadIdx.x; i < n; i += GG_TPB) lds[i] = src[i];
  } else {
    for (int i = threadIdx.x; i < n; i += GG_TPB) lds[i] = src[i];
  }
}

__device__ __forceinline__ float gg_f16(const uint8_t* p) { return f16_to_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

// The 6-bit scale and min of K-quant sub-block j (io/gguf.h:253-260).
__device__ __forceinline__ void gg_k4(const uint8_t* s, int j, int& sc, int& mn) {
  if (j < 4) {
    sc = s[j] & 63;
    mn = s[j + 4] & 63;
  } else {
    sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
    mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

// Four consecutive elements [pos, pos+4) of the block at `p` (pos % 4 == 0).
template <int DT>
__device__ __forceinline__ float4 gg_decode4(const uint8_t* p, int pos) {
  float v[4];
  if constexpr (DT == GG_Q8_0) {
    const float d = gg_f16(p);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = d * (float)(int8_t)p[2 + pos + i];
  } else if constexpr (DT == GG_Q4_0) {
    // element i < 16: low nibble of byte i; element i >= 16: high nibble of byte i-16
    const float d = gg_f16(p);
    const int hi = pos >> 4, b0 = 2 + (pos & 15);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = d * (float)((int)((p[b0 + i] >> (4 * hi)) & 15) - 8);
  } else if constexpr (DT == GG_Q4_K || DT == GG_Q5_K) {
    // chunk c of 64: low nibbles of ql[32c .. 32c+31] (sub-block 2c), then
    // their high nibbles (sub-block 2c+1); Q5_K adds 16 when bit j of qh[l] is set
    constexpr bool Q5 = DT == GG_Q5_K;
    const int c = pos >> 6, h = (pos >> 5) & 1, l = pos & 31, j = 2 * c + h;
    int sci, mni;
    gg_k4(p + 4, j, sci, mni);
    const float sc = gg_f16(p) * (float)sci, mn = gg_f16(p + 2) * (float)mni;
    const uint8_t* ql = p + (Q5 ? 48 : 16) + 32 * c + l;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int q = (ql[i] >> (4 * h)) & 15;
      if (Q5) q += ((p[16 + l + i] >> j) & 1) << 4;
      v[i] = __builtin_fmaf(sc, (float)q, -mn);
    }
  } else {
    // Q6_K: half n of 128, quarter r of 32; low four bits from
    // ql[64n + l + 32(r&1)] (nibble r>>1), top two from bits 2r of qh[32n + l],
    // int8 scale sc[8n + l/16 + 2r], d (f16) at byte 208
    const int n = pos >> 7, r = (pos >> 5) & 3, l = pos & 31;
    const float ds = gg_f16(p + 208) * (float)(int8_t)p[192 + 8 * n + (l >> 4) + 2 * r];
    const uint8_t* ql = p + 64 * n + l + 32 * (r & 1);
    const uint8_t* qh = p + 128 + 32 * n + l;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int q = ((ql[i] >> (4 * (r >> 1))) & 15) | (((qh[i] >> (2 * r)) & 3) << 4);
      v[i] = ds * (float)(q - 32);
    }
  }
  return make_float4(v[0], v[1], v[2], v[3]);
}

// One workgroup per NBW blocks (8192 elements): stage, then float4 stores,
// nontemporal: the f32 output (four times the input bytes or more) is not
// read again by this kernel and would only crowd L2 (12288 x 4096 Q8_0:
// 48.2 -> 41.3 us, Q4_K 45 -> 35).
template <int DT, bool ALIGNED>
__global__ __launch_bounds__(GG_TPB) void k_gguf_dequant(const uint8_t* __restrict__ raw, float* __restrict__ out,
                                                         int64_t nblk) {
  using F = GG<DT>;
  __shared__ __align__(16) uint8_t lds[F::NBW * F::B];
  const int64_t b0 = (int64_t)blockIdx.x * F::NBW;
  const int nb = (int)min((int64_t)F::NBW, nblk - b0);
  gg_stage<ALIGNED>(lds, raw + b0 * F::B, nb * F::B);
  __syncthreads();
  float4* o = reinterpret_cast<float4*>(out + b0 * F::E);
  const int n4 = nb * (F::E / 4);
  for (int f = threadIdx.x; f < n4; f += GG_TPB) {
    const int e = 4 * f, b = e / F::E;
    const float4 v = gg_decode4<DT>(lds + b * F::B, e - b * F::E);
    typedef float f4v __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(f4v{v.x, v.y, v.z, v.w}, reinterpret_cast<f4v*>(o + f));
  }
}

// Q4_0 -> grouped int4 (gs = 32): one thread per block.  Output byte k holds
// elements 2k (low) and 2k+1 (high); the source nibble of element i is the
// low nibble of byte i (i < 16) or the high nibble of byte i-16.
template <bool ALIGNED>
__global__ __launch_bounds__(GG_TPB) void k_gguf_repack_q4_0(const uint8_t* __restrict__ raw,
                                                             uint8_t* __restrict__ q4, float* __restrict__ qs,
                                                             int64_t nblk) {
  __shared__ __align__(16) uint8_t lds[GG_TPB * 18];
  const int64_t b0 = (int64_t)blockIdx.x * GG_TPB;
  const int nb = (int)min((int64_t)GG_TPB, nblk - b0);
  gg_stage<ALIGNED>(lds, raw + b0 * 18, nb * 18);
  __syncthreads();
  const int t = threadIdx.x;
  if (t >= nb) return;
  const uint8_t* p = lds + t * 18;
  uint32_t w[4];
#pragma unroll
  for (int m = 0; m < 4; m++) {
    // output bytes 4m..4m+3 = elements 8m..8m+7 = nibble half (m >= 2) of
    // source bytes 8(m&1) .. 8(m&1)+7
    const uint8_t* s = p + 2 + 8 * (m & 1);
    const int sh = 4 * (m >> 1);
    uint32_t acc = 0;
#pragma unroll
    for (int k = 0; k < 4; k++)
      acc |= ((uint32_t)((s[2 * k] >> sh) & 15) | ((uint32_t)((s[2 * k + 1] >> sh) & 15) << 4)) << (8 * k);
    w[m] = acc;
  }
  const int64_t b = b0 + t;
  reinterpret_cast<uint4*>(q4)[b] = make_uint4(w[0], w[1], w[2], w[3]);
  qs[b] = gg_f16(p);
}

template <int DT>
static void go_dequant(const uint8_t* raw, float* out, int64_t nblk, bool al, hipStream_t st) {
  const unsigned g = (unsigned)((nblk + GG<DT>::NBW - 1) / GG<DT>::NBW);
  if (al)
    hipLaunchKernelGGL((k_gguf_dequant<DT, true>), dim3(g), dim3(GG_TPB), 0, st, raw, out, nblk);
  else
    hipLaunchKernelGGL((k_gguf_dequant<DT, false>), dim3(g), dim3(GG_TPB), 0, st, raw, out, nblk);
}

int gguf_block(int dtype, int* elems, int* bytes) {
  switch (dtype) {
    case GG_Q8_0: *elems = 32, *bytes = 34; return 1;
    case GG_Q4_0: *elems = 32, *bytes = 18; return 1;
    case GG_Q4_K: *elems = 256, *bytes = 144; return 1;
    case GG_Q5_K: *elems = 256, *bytes = 176; return 1;
    case GG_Q6_K: *elems = 256, *bytes = 210; return 1;
  }
  return 0;
}

int launch_gguf_dequant(int dtype, const void* raw, float* out, int64_t numel, hipStream_t st) {
  int E, B;
  if (!gguf_block(dtype, &E, &B) || numel % E) return MOTY_EUNSUP;
  if (numel == 0) return MOTY_OK;
  const int64_t nblk = numel / E;
  if ((uintptr_t)out & 15) return MOTY_EUNSUP;
  const uint8_t* r = (const uint8_t*)raw;
  const bool al = ((uintptr_t)r & 15) == 0;
  switch (dtype) {
    case GG_Q8_0: go_dequant<GG_Q8_0>(r, out, nblk, al, st); break;
    case GG_Q4_0: go_dequant<GG_Q4_0>(r, out, nblk, al, st); break;
    case GG_Q4_K: go_dequant<GG_Q4_K>(r, out, nblk, al, st); break;
    case GG_Q5_K: go_dequant<GG_Q5_K>(r, out, nblk, al, st); break;
    default: go_dequant<GG_Q6_K>(r, out, nblk, al, st); break;
  }
  LAUNCH_TRY("k_gguf_dequant");
  return MOTY_OK;
}

int launch_gguf_repack_q4_0(const void* raw, uint8_t* q4, float* qs, int64_t nblk, hipStream_t st) {
  if (nblk <= 0) return MOTY_OK;
  if ((uintptr_t)q4 & 15 || (uintptr_t)qs & 3) return MOTY_EUNSUP;
  const uint8_t* r = (const uint8_t*)raw;
  const unsigned g = (unsigned)((nblk + GG_TPB - 1) / GG_TPB);
  if (((uintptr_t)r & 15) == 0)
    hipLaunchKernelGGL(k_gguf_repack_q4_0<true>, dim3(g), dim3(GG_TPB), 0, st, r, q4, qs, nblk);
  else
    hipLaunchKernelGGL(k_gguf_repack_q4_0<false>, dim3(g), dim3(GG_TPB), 0, st, r, q4, qs, nblk);
  LAUNCH_TRY("k_gguf_repack_q4_0");
  return MOTY_OK;
}

}  // namespace moty
