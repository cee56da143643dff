// moe.hip -- MoE layer: router top-k, ragged per-expert grouping, grouped
// int8 GEMMs over the active experts only, top-k weighted combine.
//
// Reference:
//   router    moty_matmul -> dot_f32 (nn/matmul.c:15-27, hw/hw_avx512.h:231-243)
//   softmax   moty_softmax_row (nn/norm.c:10 -> hw/hw_ops.h:22-26)
//   top-k     moty_moe_topk (runtime/moecache.c:97-111)
//   experts   matmul_q_s gate/up, silu*up, matmul_q_s down (nn/moe.c:186-203,
//             engines/olmoe.c:230-240)
//   combine   out[t] += w * hh, fused multiply-add (nn/moe.c:200-202 in
//             ascending expert id; engines/olmoe.c:241-242 in top-k order)
//
// Pipeline (5 launches, no host synchronisation):
//   k_route        one workgroup per token: f32 router logits in the exact
//                  AVX512 lane order, optional logit bias, softmax, greedy
//                  top-k, and the token's int8 activation row (qrow_i8)
//   k_group        one workgroup: per-expert histogram, exclusive scan, slot
//                  scatter (pairs grouped by expert), M-tile list
//   k_moe_gateup   grouped GEMM, v_mfma_i32_32x32x32_i8, gate and up rows of
//                  one expert per workgroup, epilogue silu(g)*u -> h (f32)
//   k_qrow_i8      h rows -> int8 (the down projection's activation quant)
//   k_moe_down     grouped GEMM over the same slots -> per-pair rows y
//   k_moe_combine  per token, its K rows in the reference's order, FMA
// A slot's position inside its expert's segment depends on atomic order,
// but every slot row is computed independently of the others and the
// combine reads rows through the pair->slot map in a fixed order, so the
// output is the same bit for bit on every run.
#include "common.h"
#include "kernels.h"

namespace moty {

constexpr int RT_NT = 256;

// One workgroup per token.  Writes idx[t][K], w[t][K], xq[t][D], sx[t].
__global__ __launch_bounds__(RT_NT) void k_route(const float* __restrict__ x, const float* __restrict__ Wr,
                                                 const float* __restrict__ bias, int D, int E, int K, int norm,
                                                 int* __restrict__ idx, float* __restrict__ wout,
                                                 int8_t* __restrict__ xq, float* __restrict__ sx,
                                                 float* __restrict__ probs_out) {
  extern __shared__ __align__(16) float sm[];
  float* xs = sm;           // [D]
  float* pr = sm + D;       // [E]
  __shared__ float red[RT_NT / MOTY_WAVE];
  __shared__ int sel[64];
  __shared__ float selw[64];
  const int t = blockIdx.x;
  const int lane = threadIdx.x % MOTY_WAVE, wv = threadIdx.x / MOTY_WAVE;
  const float* xr = x + (int64_t)t * D;
  float amax = 0.f;
  for (int i = threadIdx.x; i < D; i += RT_NT) {
    const float v = xr[i];
    xs[i] = v;
    amax = fmaxf(amax, fabsf(v));
  }
  amax = wave_max_f32(amax);
  if (lane == 0) red[wv] = amax;
  __syncthreads();
  // activation row for the expert GEMMs: qrow_i8 (hw/hw_quant.h:9-16)
  {
    float m = red[0];
    for (int i = 1; i < RT_NT / MOTY_WAVE; i++) m = fmaxf(m, red[i]);
    float s = m / 127.f;
    if (s < 1e-12f) s = 1e-12f;
    const float inv = 1.f / s;
    if (threadIdx.x == 0) sx[t] = s;
    for (int i = threadIdx.x; i < D; i += RT_NT) xq[(int64_t)t * D + i] = (int8_t)rne_int(xs[i] * inv);
  }
  // router logits: each half-wave owns one expert at a time
  const int half = threadIdx.x / 32, nhalf = RT_NT / 32;
  for (int e = half; e < E; e += nhalf) {
    float l = dot_f32_half(xs, Wr + (int64_t)e * D, D);
    if (bias) l = l + bias[e];
    if ((threadIdx.x % 32) == 0) pr[e] = l;
  }
  __syncthreads();
  // softmax (wave 0): max is order-free; the sum runs serially in lane 0.
  // The other waves stay alive for the workgroup barriers below.
  float m = -1e30f;
  if (wv == 0) {
    for (int e = lane; e < E; e += MOTY_WAVE) m = pr[e] > m ? pr[e] : m;
    m = wave_max_f32(m);
    for (int e = lane; e < E; e += MOTY_WAVE) pr[e] = ref_expf(pr[e] - m);
  }
  __syncthreads();
  if (wv == 0) {
    float ssum = 0.f;
    if (lane == 0)
      for (int e = 0; e < E; e++) ssum += pr[e];
    ssum = __shfl(ssum, 0, 64);
    for (int e = lane; e < E; e += MOTY_WAVE) pr[e] = pr[e] / ssum;
  }
  __syncthreads();
  if (probs_out)
    for (int e = threadIdx.x; e < E; e += RT_NT) probs_out[(int64_t)t * E + e] = pr[e];
  // greedy top-k: largest value, lowest index on ties (the strict '>' scan)
  for (int kk = 0; kk < K; kk++) {
    if (wv == 0) {
      float bv = -1e30f;
      int be = -1;
      for (int e = lane; e < E; e += MOTY_WAVE) {
        bool taken = false;
        for (int j = 0; j < kk; j++) taken |= (sel[j] == e);
        const float v = pr[e];
        if (!taken && v > bv) { bv = v; be = e; }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oe = __shfl_xor(be, o, 64);
        if (oe >= 0 && (ov > bv || (ov == bv && (be < 0 || oe < be)))) { bv = ov; be = oe; }
      }
      if (lane == 0) { sel[kk] = be; selw[kk] = bv; }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (norm) {
      float s = 0.f;
      for (int kk = 0; kk < K; kk++) s += selw[kk];
      if (s > 0)
        for (int kk = 0; kk < K; kk++) selw[kk] = selw[kk] / s;
    }
    for (int kk = 0; kk < K; kk++) {
      idx[(int64_t)t * K + kk] = sel[kk];
      wout[(int64_t)t * K + kk] = selw[kk];
    }
  }
}

// ---------------------------------------------------------------------------
constexpr int GR_NT = 1024;

// Single workgroup.  offs[E+1]: expert segment starts; slot_tok[P]: token of
// each slot; pair_slot[P]: slot of pair (t,k); tiles[]: (expert, m0) M-tiles
// of MOE_BM slots; ntiles[0]: their count.
__global__ __launch_bounds__(GR_NT) void k_group(const int* __restrict__ idx, int P, int K, int E,
                                                 int* __restrict__ offs, int* __restrict__ slot_tok,
                                                 int* __restrict__ pair_slot, int2* __restrict__ tiles,
                                                 int* __restrict__ ntiles, int* __restrict__ counts_out) {
  extern __shared__ int gs[];
  int* cnt = gs;          // [E]
  int* cur = gs + E;      // [E]
  int* tstart = gs + 2 * E;  // [E+1]
  for (int e = threadIdx.x; e < E; e += GR_NT) cnt[e] = 0;
  __syncthreads();
  for (int p = threadIdx.x; p < P; p += GR_NT) {
    const int e = idx[p];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int o = 0, tl = 0;
    for (int e = 0; e < E; e++) {
      cur[e] = o;
      offs[e] = o;
      tstart[e] = tl;
      o += cnt[e];
      tl += (cnt[e] + MOE_BM - 1) / MOE_BM;
    }
    offs[E] = o;
    tstart[E] = tl;
    ntiles[0] = tl;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += GR_NT) {
    if (counts_out) counts_out[e] = cnt[e];
    const int nt = tstart[e + 1] - tstart[e];
    for (int j = 0; j < nt; j++) tiles[tstart[e] + j] = int2{e, j * MOE_BM};
  }
  for (int p = threadIdx.x; p < P; p += GR_NT) {
    const int e = idx[p];
    if (e < 0 || e >= E) { pair_slot[p] = -1; continue; }
    const int s = atomicAdd(&cur[e], 1);
    slot_tok[s] = p / K;
    pair_slot[p] = s;
  }
}

// ---------------------------------------------------------------------------
// Grouped GEMMs.  Workgroup = 4 waves; each wave computes a 32 (slots) x 32
// (weight rows) tile with v_mfma_i32_32x32x32_i8; the workgroup covers
// MOE_BM slots x 128 weight rows of one expert.  Lane l holds A row l%32 and
// B row l%32, 16 k-bytes at offset 16*(l/32) of each 32-byte K step.
// D layout: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, column l%32.
constexpr int MG_NT = 256;
constexpr int MG_BN = 128;

__device__ __forceinline__ int4 ldg16(const int8_t* p) { return *(const int4*)p; }

template <bool GATEUP>
__global__ __launch_bounds__(MG_NT) void k_moe_gemm(
    const int2* __restrict__ tiles, const int* __restrict__ ntiles, const int* __restrict__ offs,
    const int* __restrict__ slot_tok,
    const int8_t* __restrict__ act, const float* __restrict__ act_s,  // GATEUP: xq[T][K], sx[T]; else hq[P][K], sh[P]
    const int8_t* __restrict__ W1, const float* __restrict__ S1,      // [E][N][K], [E][N]
    const int8_t* __restrict__ W2, const float* __restrict__ S2,      // up (GATEUP only)
    float* __restrict__ out,                                          // [P][N]
    int N, int Kd) {
  const int tile = blockIdx.y;
  if (tile >= ntiles[0]) return;
  const int2 tm = tiles[tile];
  const int e = tm.x, mb = tm.y;
  const int seg0 = offs[e], nseg = offs[e + 1] - seg0;
  const int lane = threadIdx.x % MOTY_WAVE, wv = threadIdx.x / MOTY_WAVE;
  const int r32 = lane & 31, kq = (lane >> 5) * 16;
  const int n0 = blockIdx.x * MG_BN + wv * 32;
  // A row of this lane (clamped inside the segment; extra rows are not stored)
  int mrow = mb + r32;
  mrow = mrow < nseg ? mrow : nseg - 1;
  const int slot = seg0 + mrow;
  const int64_t arow = GATEUP ? (int64_t)slot_tok[slot] : (int64_t)slot;
  const int8_t* ap = act + arow * Kd + kq;
  int nrow = n0 + r32;
  nrow = nrow < N ? nrow : N - 1;
  const int8_t* b1 = W1 + ((int64_t)e * N + nrow) * Kd + kq;
  const int8_t* b2 = GATEUP ? W2 + ((int64_t)e * N + nrow) * Kd + kq : nullptr;

  v16i acc1 = {}, acc2 = {};
  int4 a = ldg16(ap), w1 = ldg16(b1), w2 = GATEUP ? ldg16(b2) : int4{0, 0, 0, 0};
  for (int k0 = 32; k0 <= Kd; k0 += 32) {
    int4 an = a, w1n = w1, w2n = w2;
    if (k0 < Kd) {
      an = ldg16(ap + k0);
      w1n = ldg16(b1 + k0);
      if (GATEUP) w2n = ldg16(b2 + k0);
    }
    acc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(*(v4i*)&a, *(v4i*)&w1, acc1, 0, 0, 0);
    if (GATEUP) acc2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(*(v4i*)&a, *(v4i*)&w2, acc2, 0, 0, 0);
    a = an; w1 = w1n; w2 = w2n;
  }
  const int ncol = n0 + r32;
  if (ncol >= N) return;
  const float s1 = S1[(int64_t)e * N + ncol];
  const float s2 = GATEUP ? S2[(int64_t)e * N + ncol] : 0.f;
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const int m = mb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    if (m >= nseg) continue;
    const int sl = seg0 + m;
    if (GATEUP) {
      const float sxv = act_s[slot_tok[sl]];
      const float g = (s1 * sxv) * (float)acc1[r];
      const float u = (s2 * sxv) * (float)acc2[r];
      out[(int64_t)sl * N + ncol] = ref_silu_mul(g, u);
    } else {
      out[(int64_t)sl * N + ncol] = (s1 * act_s[sl]) * (float)acc1[r];
    }
  }
}

// ---------------------------------------------------------------------------
// out[t][d] = sum over the token's K rows, FMA in the reference's order:
// order 0 = top-k order (engines/olmoe.c), 1 = ascending expert id (nn/moe.c).
__global__ void k_moe_combine(const float* __restrict__ y, const int* __restrict__ idx,
                              const float* __restrict__ w, const int* __restrict__ pair_slot,
                              float* __restrict__ out, int D, int K, int order) {
  __shared__ int slot_s[64];
  __shared__ float w_s[64];
  const int t = blockIdx.x;
  if (threadIdx.x == 0) {
    int ord[64];
    for (int k = 0; k < K; k++) ord[k] = k;
    if (order == 1)
      for (int a = 1; a < K; a++)
        for (int b = a; b > 0 && idx[t * K + ord[b]] < idx[t * K + ord[b - 1]]; b--) {
          const int tmp = ord[b]; ord[b] = ord[b - 1]; ord[b - 1] = tmp;
        }
    for (int j = 0; j < K; j++) {
      slot_s[j] = pair_slot[t * K + ord[j]];
      w_s[j] = w[t * K + ord[j]];
    }
  }
  __syncthreads();
  for (int d = threadIdx.x * 4; d < D; d += blockDim.x * 4) {
    float4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < K; j++) {
      const int sl = slot_s[j];
      if (sl < 0) continue;
      const float wk = w_s[j];
      const float4 v = *(const float4*)(y + (int64_t)sl * D + d);
      acc.x = __fmaf_rn(wk, v.x, acc.x);
      acc.y = __fmaf_rn(wk, v.y, acc.y);
      acc.z = __fmaf_rn(wk, v.z, acc.z);
      acc.w = __fmaf_rn(wk, v.w, acc.w);
    }
    *(float4*)(out + (int64_t)t * D + d) = acc;
  }
}

// ---------------------------------------------------------------------------
size_t moe_scratch_size(int T, int D, int E, int K, int I, size_t* offsets) {
  const int64_t P = (int64_t)T * K;
  const int64_t maxt = P / MOE_BM + E + 1;
  size_t sz[MOE_NBUF] = {(size_t)T * D,       (size_t)T * 4,     (size_t)P * 4, (size_t)P * 4,
                         (size_t)(E + 1) * 4, (size_t)P * 4,     (size_t)P * 4, (size_t)maxt * 8,
                         16,                  (size_t)P * I * 4, (size_t)P * I, (size_t)P * 4,
                         (size_t)P * D * 4,   (size_t)E * 4};
  size_t o = 0;
  for (int i = 0; i < MOE_NBUF; i++) {
    offsets[i] = o;
    o += (sz[i] + 255) / 256 * 256;
  }
  return o;
}

int launch_moe(const MoeArgs& a, void* scratch, hipStream_t st) {
  const int T = a.T, D = a.D, E = a.E, K = a.K, I = a.I;
  if (T <= 0) return MOTY_OK;
  if (K < 1 || K > 64 || K > E || E > 4096 || (D % 32) || (I % 32) || (D % 4)) return MOTY_EUNSUP;
  size_t off[MOE_NBUF];
  moe_scratch_size(T, D, E, K, I, off);
  char* b = (char*)scratch;
  int8_t* xq = (int8_t*)(b + off[0]);
  float* sx = (float*)(b + off[1]);
  int* idx = (int*)(b + off[2]);
  float* w = (float*)(b + off[3]);
  int* offs = (int*)(b + off[4]);
  int* slot_tok = (int*)(b + off[5]);
  int* pair_slot = (int*)(b + off[6]);
  int2* tiles = (int2*)(b + off[7]);
  int* ntiles = (int*)(b + off[8]);
  float* h = (float*)(b + off[9]);
  int8_t* hq = (int8_t*)(b + off[10]);
  float* sh = (float*)(b + off[11]);
  float* y = (float*)(b + off[12]);
  int* counts = (int*)(b + off[13]);
  const int P = T * K;
  const int maxt = P / MOE_BM + E + 1;

  const size_t lds_route = (size_t)(D + E) * 4;
  if (lds_route > 64 * 1024) return MOTY_EUNSUP;
  hipLaunchKernelGGL(k_route, dim3(T), dim3(RT_NT), lds_route, st, a.x, a.Wr, a.bias, D, E, K, a.norm, idx, w,
                     xq, sx, a.probs_out);
  LAUNCH_TRY("k_route");
  hipLaunchKernelGGL(k_group, dim3(1), dim3(GR_NT), (size_t)(3 * E + 1) * 4, st, idx, P, K, E, offs, slot_tok,
                     pair_slot, tiles, ntiles, counts);
  LAUNCH_TRY("k_group");
  hipLaunchKernelGGL(k_moe_gemm<true>, dim3((I + MG_BN - 1) / MG_BN, maxt), dim3(MG_NT), 0, st, tiles, ntiles,
                     offs, slot_tok, xq, sx, a.G, a.GS, a.U, a.US, h, I, D);
  LAUNCH_TRY("k_moe_gemm<gateup>");
  int rc = launch_qrow_i8(h, hq, sh, nullptr, P, I, I, I, st);
  if (rc) return rc;
  hipLaunchKernelGGL(k_moe_gemm<false>, dim3((D + MG_BN - 1) / MG_BN, maxt), dim3(MG_NT), 0, st, tiles, ntiles,
                     offs, slot_tok, hq, sh, a.Dn, a.DS, nullptr, nullptr, y, D, I);
  LAUNCH_TRY("k_moe_gemm<down>");
  hipLaunchKernelGGL(k_moe_combine, dim3(T), dim3(256), 0, st, y, idx, w, pair_slot, a.out, D, K, a.order);
  LAUNCH_TRY("k_moe_combine");
  if (a.idx_out) HIP_TRY(hipMemcpyAsync(a.idx_out, idx, (size_t)P * 4, hipMemcpyDeviceToDevice, st));
  if (a.w_out) HIP_TRY(hipMemcpyAsync(a.w_out, w, (size_t)P * 4, hipMemcpyDeviceToDevice, st));
  if (a.counts_out) HIP_TRY(hipMemcpyAsync(a.counts_out, counts, (size_t)E * 4, hipMemcpyDeviceToDevice, st));
  return MOTY_OK;
}

}  // namespace moty
