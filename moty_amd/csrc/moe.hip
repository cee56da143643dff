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
// Pipeline (7 launches, no host synchronisation):
//   k_router       router logits on f32 MFMA in dot_f32's AVX512 chain
//                  order, plus logit bias (token tile x expert slice per
//                  workgroup)
//   k_route_topk   wave per token: softmax and greedy top-k; another wave:
//                  the token's int8 row (qrow_i8)
//   k_group        per-expert histogram, exclusive scan, slot scatter (pairs
//                  grouped by expert; each workgroup places one chunk), M-tiles
//   k_moe_gemm<true>   grouped GEMM, v_mfma_i32_32x32x32_i8, gate and up
//                  rows of one expert per workgroup, epilogue silu(g)*u -> h
//                  (f32)
//   k_qrow_wave    h rows -> int8 (the down projection's activation quant)
//   k_moe_gemm<false>  grouped GEMM over the same slots -> per-pair rows y
//   k_moe_combine  per token, its K rows in the reference's order, FMA
// A slot's position inside its expert's segment depends on atomic order,
// but every slot row is computed independently of the others and the
// combine reads rows through the pair->slot map in a fixed order, so the
// output is the same bit for bit on every run.
#include "common.h"
#include "kernels.h"

namespace moty {

// ---------------------------------------------------------------------------
// Routing.
//
// Router logits keep dot_f32's AVX512 order (nn/matmul.c:15-27 ->
// hw/hw_avx512.h:231-243): each (token, expert) dot is 32 FMA chains --
// chain c takes elements c, c+32, c+64, ... in order (s0[c] for c < 16,
// s1[c-16] else) -- then s0+s1 and gcc's _mm512_reduce_add_ps tree.  The
// chains run on v_mfma_f32_4x4x1_16b_f32: one instruction is 16 independent
// 4x4 outer products with k = 1, each output a single fused multiply-add
// (checked bit for bit against v_fma_f32 on MI355X, denormals and all bit
// patterns included).  Block b of instruction q carries chain q*16 + b of a
// 4-token x 4-expert sub-tile: lane l = 4b + i feeds token i's element
// u*32 + q*16 + b (A) and expert i's (B), and holds the 4 tokens' sums for
// expert l%4 (output rows in its 4 registers).
//
// x and router rows stream through an S-stage LDS ring of 64-element chunks
// by buffer_load ... lds DMA (1 KiB per instruction = 4 rows x 64 floats);
// a row's 16-byte column slot c is stored at c ^ ((row & 3) << 1), so the 4
// rows x 16 chains one read touches fall in distinct banks.  A CU streams
// (experts + tokens of its tile) x D floats at about 50 B per clock, so
// tiles are near-square in tokens x experts rather than all experts of a
// token: the per-token steps run in a second kernel.
//
// Per token, one wave: softmax (nn/norm.c:10 -> hw/hw_ops.h:22-26: max
// order-free, exp, sum serial in expert order, per-element divide) and the
// greedy top-k of runtime/moecache.c:97-111 as K rounds of a wave argmax
// under (p desc, index asc) over the experts not yet taken (the reference's
// first strict '>' over ascending e; values not above -1e30, NaN included,
// are never taken, and a round without a candidate gives id -1 and weight
// -1e30 as there); normalisation sum serial over k.  Another wave writes the
// token's int8 row (qrow_i8, hw/hw_quant.h:9-16).

// qrow_i8 of one row by one wave (hw/hw_quant.h:9-16): amax, scale =
// max(amax/127, 1e-12), RNE of x/scale, as bytes.
__device__ __forceinline__ void qrow_row_wave(const float* __restrict__ xr, int D, int8_t* __restrict__ q,
                                              float* __restrict__ sxo) {
  const int lane = threadIdx.x % MOTY_WAVE;
  auto pack = [](float4 v, float inv) {
    return (uint32_t)(rne_int(v.x * inv) & 0xff) | ((uint32_t)(rne_int(v.y * inv) & 0xff) << 8) |
           ((uint32_t)(rne_int(v.z * inv) & 0xff) << 16) | ((uint32_t)(rne_int(v.w * inv) & 0xff) << 24);
  };
  if (D <= 4096) {
    // the row held in registers: lane l owns [c*1024 + 16l, +16) of each
    // 1 KiB chunk c (clamped loads past the end, zeroed)
    float4 v[4][4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int k = c * 1024 + lane * 16;
#pragma unroll
      for (int j = 0; j < 4; j++) v[c][j] = *(const float4*)(xr + (k < D ? k : 0) + 4 * j);
    }
    float amax = 0.f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const bool ok = c * 1024 + lane * 16 < D;
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
    if (lane == 0) *sxo = s;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int k = c * 1024 + lane * 16;
      if (k >= D) continue;
      int4 o;
#pragma unroll
      for (int j = 0; j < 4; j++) ((int*)&o)[j] = (int)pack(v[c][j], inv);
      *(int4*)(q + k) = o;
    }
    return;
  }
  float amax = 0.f;
  for (int i = lane * 4; i < D; i += MOTY_WAVE * 4) {
    const float4 v = *(const float4*)(xr + i);
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  amax = wave_max_f32(amax);
  float s = amax / 127.f;
  if (s < 1e-12f) s = 1e-12f;
  const float inv = 1.f / s;
  if (lane == 0) *sxo = s;
  for (int i = lane * 4; i < D; i += MOTY_WAVE * 4) *(uint32_t*)(q + i) = pack(*(const float4*)(xr + i), inv);
}

// Softmax and greedy top-k of one token's logits lg[0..E) (LDS, 16-byte
// aligned, overwritten with the exponentials) by one wave; lane kk < K
// ends with pick kk (*e, *w: expert id and routing weight); probs[0..E)
// written if non-null.
__device__ __forceinline__ void route_token_regs(float* lg, int E, int K, int norm, int* e_out, float* w_out,
                                                 float* __restrict__ probs) {
  constexpr int PV = 4;  // E <= 256
  const int lane = threadIdx.x % MOTY_WAVE;
  float pv[PV];
#pragma unroll
  for (int j = 0; j < PV; j++) pv[j] = (lane + 64 * j < E) ? lg[lane + 64 * j] : -1e30f;
  float m = -1e30f;
#pragma unroll
  for (int j = 0; j < PV; j++) m = pv[j] > m ? pv[j] : m;
  m = wave_max_f32(m);
#pragma unroll
  for (int j = 0; j < PV; j++) {
    pv[j] = ref_expf(pv[j] - m);
    if (lane + 64 * j < E) lg[lane + 64 * j] = pv[j];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float ssum = 0.f;  // serial in expert order (every lane runs it; reads batched)
  {
    int e = 0;
    for (; e + 32 <= E; e += 32) {
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) v[u] = *(const float4*)(lg + e + 4 * u);
#pragma unroll
      for (int u = 0; u < 8; u++) ssum = (((ssum + v[u].x) + v[u].y) + v[u].z) + v[u].w;
    }
    for (; e < E; e++) ssum += lg[e];
  }
  // candidates: this lane's probabilities, -inf where not one (past E, or
  // not above -1e30 as the reference's scan requires, NaN included)
#pragma unroll
  for (int j = 0; j < PV; j++) {
    const bool in = lane + 64 * j < E;
    const float p = in ? pv[j] / ssum : 0.f;
    if (probs && in) probs[lane + 64 * j] = p;
    pv[j] = (in && p > -1e30f) ? p : -__builtin_inff();
  }
  // K rounds: the wave maximum, then the lowest expert id holding it (first
  // candidate set with a lane at the maximum, its lowest lane), taken out
  int my_e = -1;
  float my_w = -1e30f, ws = 0.f;
  for (int kk = 0; kk < K; kk++) {
    float lm = pv[0];
#pragma unroll
    for (int j = 1; j < PV; j++) lm = fmaxf(lm, pv[j]);
    const float bv = wave_max_f32(lm);
    int be = -1;
#pragma unroll
    for (int j = PV - 1; j >= 0; j--) {
      const uint64_t hit = __ballot(pv[j] == bv);
      if (hit) be = 64 * j + (int)__builtin_ctzll(hit);
    }
    const bool none = !(bv > -__builtin_inff());
    const float wk = none ? -1e30f : bv;
    be = none ? -1 : be;
#pragma unroll
    for (int j = 0; j < PV; j++) pv[j] = (be == lane + 64 * j) ? -__builtin_inff() : pv[j];
    my_e = lane == kk ? be : my_e;
    my_w = lane == kk ? wk : my_w;
    ws += wk;  // the normalisation sum, serial over k
  }
  *e_out = my_e;
  *w_out = (norm && ws > 0) ? my_w / ws : my_w;
}

// route_token_regs, then idx/w[0..K) written
__device__ __forceinline__ void route_token_wave(float* lg, int E, int K, int norm, int* __restrict__ idx,
                                                 float* __restrict__ wout, float* __restrict__ probs) {
  int e;
  float w;
  route_token_regs(lg, E, K, norm, &e, &w, probs);
  const int lane = threadIdx.x % MOTY_WAVE;
  if (lane < K) {
    idx[lane] = e;
    wout[lane] = w;
  }
}

typedef float v4f __attribute__((ext_vector_type(4)));

// Router logits, one workgroup per (token tile, expert slice): WT x WE waves,
// each TWW tokens x EWW experts; the tile is TW = WT*TWW tokens by EG =
// WE*EWW experts.  S ring stages of KS 32-element steps; every wave issues
// NJ DMA instructions per stage.  Workgroup ids are decoded so that all the
// slices of a token tile run on one XCD (workgroups go to the 8 XCDs
// round-robin by linear id): its x rows come from that XCD's L2 after the
// first read.
template <int TWW, int EWW, int WT, int WE, int S, int KS, int NJ>
__global__ __launch_bounds__(WT * WE * 64) void k_router(const float* __restrict__ x, const float* __restrict__ Wr,
                                                         const float* __restrict__ bias, int T, int D, int E,
                                                         float* __restrict__ logits) {
  constexpr int TW = WT * TWW, EG = WE * EWW, NW = WT * WE, ROWS = EG + TW;
  constexpr int RT = TWW / 4, CT = EWW / 4;  // 4 x 4 sub-tiles per wave
  constexpr int KC = KS * 32;                // chunk elements per row
  constexpr int ROWB = KC * 4;               // bytes per staged row
  constexpr int RPI = 1024 / ROWB;           // rows per 1 KiB DMA instruction
  constexpr int NSL = KC / 4;                // 16-byte slots per row
  constexpr int J = ROWS / RPI;              // DMA instructions per stage
  constexpr int STAGE = ROWS * ROWB + 1024;  // the rows, then 1 KiB for idle DMA slots
  static_assert(RPI >= 1 && 4 % RPI == 0 && ROWS % 4 == 0 && J <= NJ * NW, "stage layout");
  __shared__ __align__(1024) uint8_t lds[S * STAGE];
  int tb, eb;
  {
    const int nsl = (E + EG - 1) / EG;
    const int xcd = blockIdx.x % 8, j = blockIdx.x / 8;
    tb = ((j / nsl) * 8 + xcd) * TW;
    eb = (j % nsl) * EG;
    if (tb >= T) return;  // padding of the tile count to a multiple of 8
  }
  const int lane = threadIdx.x % MOTY_WAVE;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / MOTY_WAVE);
  const int wi = wv / WE, wj = wv % WE;
  const v4i rW = buf_rsrc(Wr, (uint32_t)E * (uint32_t)D * 4u);
  const v4i rX = buf_rsrc(x, (uint32_t)T * (uint32_t)D * 4u);
  // stage rows: EG router rows (clamped past E), then TW x rows (clamped
  // past T).  This wave's DMA slots: instruction j*NW + wv of each stage;
  // slots past J load from past the buffer end (no memory traffic) into the
  // stage's spare KiB.
  uint32_t vo[NJ], ldo[NJ];
  bool isx[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int jb = j * NW + wv;
    const int row = jb * RPI + lane / NSL;
    const int c = (lane % NSL) ^ ((row & 3) << 1);
    isx[j] = jb * RPI >= EG;  // whole instructions: EG is a multiple of 4
    const int r = isx[j] ? (tb + row - EG < T ? tb + row - EG : T - 1) : (eb + row < E ? eb + row : E - 1);
    vo[j] = jb < J ? (uint32_t)r * (uint32_t)D * 4u + (uint32_t)c * 16u : 0x80000000u;
    ldo[j] = jb < J ? (uint32_t)jb * 1024u : (uint32_t)(STAGE - 1024);
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
  auto issue = [&](int kb) {
    const uint32_t st0 = lds0 + (uint32_t)(kb % S) * (uint32_t)STAGE;
#pragma unroll
    for (int j = 0; j < NJ; j++) bdma16_to_lds(isx[j] ? rX : rW, vo[j], (uint32_t)kb * (uint32_t)ROWB, st0 + ldo[j]);
  };
  v4f acc[RT][CT][2];
#pragma unroll
  for (int r = 0; r < RT; r++)
#pragma unroll
    for (int c = 0; c < CT; c++) acc[r][c][0] = acc[r][c][1] = v4f{0.f, 0.f, 0.f, 0.f};
  const int b = lane >> 2, i4 = lane & 3;
  // LDS float offset of this lane's operand in a stage, chain q*16 + b of
  // step u: row*KC + ((col/4) ^ ((row&3)<<1))*4 + col%4, with row&3 == i4
  auto off = [&](int row, int u, int q) {
    const int col = u * 32 + q * 16 + b;
    return row * KC + (((col >> 2) ^ (i4 << 1)) << 2) + (col & 3);
  };
  // a chunk's operands in registers: read while the previous chunk's
  // MFMAs run
  struct Frags {
    float a[KS][2][RT], w[KS][2][CT];
  };
  auto read = [&](int kb, Frags& f) {
    const float* st = (const float*)(lds + (kb % S) * STAGE);
#pragma unroll
    for (int u = 0; u < KS; u++)
#pragma unroll
      for (int q = 0; q < 2; q++) {
#pragma unroll
        for (int r = 0; r < RT; r++) f.a[u][q][r] = st[off(EG + wi * TWW + r * 4 + i4, u, q)];
#pragma unroll
        for (int c = 0; c < CT; c++) f.w[u][q][c] = st[off(wj * EWW + c * 4 + i4, u, q)];
      }
  };
  const int nsteps = D / 32, nk = (nsteps + KS - 1) / KS;
  auto compute = [&](int kb, const Frags& f) {
#pragma unroll
    for (int u = 0; u < KS; u++) {
      if (kb * KS + u >= nsteps) break;  // the last chunk's row end (wave-uniform)
#pragma unroll
      for (int q = 0; q < 2; q++)
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
          for (int c = 0; c < CT; c++)
            acc[r][c][q] = __builtin_amdgcn_mfma_f32_4x4x1f32(f.a[u][q][r], f.w[u][q][c], acc[r][c][q], 0, 0, 0);
    }
  };
  // every stage of the ring in flight, then chunk 0's operands to registers
#pragma unroll
  for (int s = 0; s < S; s++) issue(s);
  MOTY_WAIT_VMCNT((S - 1) * NJ);
  __syncthreads();
  Frags f0, f1;
  read(0, f0);
  for (int kb = 0; kb < nk; kb += 2) {
    // chunk kb + 1 has landed (S - 2 later ones may still fly); the barrier
    // also retires every wave's reads of chunk kb's stage, which the next
    // DMA overwrites.  Chunks past the end are loaded and never used.
    MOTY_WAIT_VMCNT((S - 2) * NJ);
    __syncthreads();
    issue(kb + S);
    read(kb + 1, f1);
    compute(kb, f0);
    if (kb + 1 >= nk) break;
    MOTY_WAIT_VMCNT((S - 2) * NJ);
    __syncthreads();
    issue(kb + 1 + S);
    read(kb + 2, f0);
    compute(kb + 1, f1);
  }
  __builtin_amdgcn_s_waitcnt(0);
  // s0[c] + s1[c] (same lane), then the reduce tree over the 16 blocks
  // (block k in lanes 4k..4k+3): t[k+8] + t[k] (lane ^ 32), a[k+4] + a[k]
  // (lane ^ 16), then (b0 + b2) + (b1 + b3) from lanes j, j+8, j+4, j+12
#pragma unroll
  for (int c = 0; c < CT; c++) {
    const int e = eb + wj * EWW + c * 4 + i4;
    const float bv = (bias && e < E) ? bias[e] : 0.f;
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float t = acc[r][c][0][i] + acc[r][c][1][i];
        const float a8 = xor32_f(t) + t;
        const float b4 = xor16_f(a8) + a8;
        const float s2 = dpp_f<MOTY_DPP_ROR8>(b4) + b4;  // lane j: b2 + b0, lane j+4: b3 + b1
        float v = dpp_f<MOTY_DPP_ROR12>(s2) + s2;        // lane j: (b1 + b3) + (b0 + b2)
        if (bias) v = v + bv;
        const int tk = tb + wi * TWW + r * 4 + i;
        if (lane < 4 && e < E && tk < T) logits[(int64_t)tk * E + e] = v;
      }
  }
}

// Per token, two waves: one routes (softmax, greedy top-k), the other writes
// the token's int8 row; TK_TOK tokens per workgroup.
constexpr int TK_TOK = 4;
__global__ __launch_bounds__(TK_TOK * 128) void k_route_topk(const float* __restrict__ x,
                                                            const float* __restrict__ logits, int T, int D, int E,
                                                            int K, int norm, int* __restrict__ idx,
                                                            float* __restrict__ wout, int8_t* __restrict__ xq,
                                                            float* __restrict__ sx, float* __restrict__ probs_out) {
  __shared__ float lg[TK_TOK][256];
  const int lane = threadIdx.x % MOTY_WAVE, wv = threadIdx.x / MOTY_WAVE;
  const int tl = wv % TK_TOK, t = blockIdx.x * TK_TOK + tl;
  if (t >= T) return;  // whole waves; no workgroup barrier in this kernel
  if (wv >= TK_TOK) {
    qrow_row_wave(x + (int64_t)t * D, D, xq + (int64_t)t * D, sx + t);
    return;
  }
  for (int e = lane; e < E; e += MOTY_WAVE) lg[tl][e] = logits[(int64_t)t * E + e];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  route_token_wave(lg[tl], E, K, norm, idx + (int64_t)t * K, wout + (int64_t)t * K,
                   probs_out ? probs_out + (int64_t)t * E : nullptr);
}

// ---------------------------------------------------------------------------
constexpr int GR_NT = 1024;
constexpr int GR_CHUNK = 256;  // pairs placed per workgroup (at most 32 workgroups)
constexpr int GR_U = 8;        // expert ids loaded ahead in the counting pass

// Grouping over G workgroups, with no hand-off between them: every
// workgroup counts all P expert ids (the histogram, and the part of it from
// pairs before its own chunk), scans the counts itself and places only its
// chunk's pairs, at offs[e] + (pairs of e in earlier chunks) + its rank
// among its chunk's pairs of e.  offs[E+1]: expert segment starts;
// slot_tok[P]: token of each slot; pair_slot[P]: slot of pair (t,k);
// tiles[]: (expert, m0) M-tiles of bm slots; ntiles[0]: their count (these
// three and counts_out from workgroup 0).  Within an expert's segment the
// slot order is free: every GEMM row is computed on its own and the combine
// finds each pair through pair_slot.
__global__ __launch_bounds__(GR_NT) void k_group(const int* __restrict__ idx, int P, int K, int E, int bm, int chunk,
                                                 int* __restrict__ offs, int* __restrict__ slot_tok,
                                                 int* __restrict__ pair_slot, int2* __restrict__ tiles,
                                                 int* __restrict__ ntiles, int* __restrict__ counts_out) {
  __shared__ int cnt[256], pre[256], cur[256], base[256], tstart[257];
  const int tid = threadIdx.x;
  const int c0 = blockIdx.x * chunk, c1 = c0 + chunk < P ? c0 + chunk : P;
  // this thread's first pair of the chunk, loaded with the counting pass's
  // ids rather than after the scan
  const int eo = c0 + tid < c1 ? idx[c0 + tid] : -1;
  if (tid < E) {
    cnt[tid] = 0;
    pre[tid] = 0;
    cur[tid] = 0;
  }
  __syncthreads();
  for (int p0 = 0; p0 < P; p0 += GR_U * GR_NT) {
    int ev[GR_U];
#pragma unroll
    for (int u = 0; u < GR_U; u++) {
      const int p = p0 + u * GR_NT + tid;
      ev[u] = p < P ? idx[p] : -1;
    }
#pragma unroll
    for (int u = 0; u < GR_U; u++) {
      const int p = p0 + u * GR_NT + tid;
      if (ev[u] >= 0 && ev[u] < E) {
        atomicAdd(&cnt[ev[u]], 1);
        if (p < c0) atomicAdd(&pre[ev[u]], 1);
      }
    }
  }
  __syncthreads();
  if (tid < MOTY_WAVE) {
    // exclusive scans of the counts and of the M-tile counts by one wave:
    // lane l owns experts 4l..4l+3 (E <= 256)
    const int l = tid;
    const bool w0 = blockIdx.x == 0;
    int c[4], t[4], so = 0, st = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int e = 4 * l + j;
      c[j] = e < E ? cnt[e] : 0;
      t[j] = (c[j] + bm - 1) / bm;
      so += c[j];
      st += t[j];
    }
    int o = wave_incl_scan_i32(so) - so, tl = wave_incl_scan_i32(st) - st;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int e = 4 * l + j;
      if (e < E) {
        base[e] = o + pre[e];
        tstart[e] = tl;
        if (w0) {
          offs[e] = o;
          if (counts_out) counts_out[e] = c[j];
        }
      }
      o += c[j];
      tl += t[j];
    }
    if (l == MOTY_WAVE - 1) {
      tstart[E] = tl;
      if (w0) {
        offs[E] = o;
        ntiles[0] = tl;
      }
    }
  }
  __syncthreads();
  if (blockIdx.x == 0 && tid < E) {
    const int nt = tstart[tid + 1] - tstart[tid];
    for (int j = 0; j < nt; j++) tiles[tstart[tid] + j] = int2{tid, j * bm};
  }
  for (int p = c0 + tid; p < c1; p += GR_NT) {
    const int e = p == c0 + tid ? eo : idx[p];
    if (e < 0 || e >= E) {
      pair_slot[p] = -1;
      continue;
    }
    const int s = base[e] + atomicAdd(&cur[e], 1);
    slot_tok[s] = p / K;
    pair_slot[p] = s;
  }
}

// ---------------------------------------------------------------------------
// Grouped GEMMs.  Workgroup = MT groups of 4 waves over one (expert,
// 64*MT-slot M-tile, 128-row N-tile); MT = 2 when experts average more than
// 48 slots, so that an expert's weight tile is read once for up to 128 slots
// instead of once per 64.  Per 128-byte K block the workgroup stages the
// tile in LDS: every global load instruction reads whole 128 B lines (8
// lanes per row, 16 B each) -- activation rows gathered through slot ->
// token for the gate/up GEMM -- into rows padded to 144 B.  Each wave then
// owns 32 weight rows (of gate and up, or of down) for both 32-slot halves
// of its group's 64-slot sub-tile and runs v_mfma_i32_32x32x32_i8 on
// fragments read back from LDS.  Two register sets keep the next two K
// blocks' global loads in flight during the MFMAs.
//
// Fragment k-order: MFMA step j of a K block takes, in lane l, bytes
// [64*(l/32) + 16j, +16) of row (l % 32).  An integer dot is order-free, so
// this k-permutation, shared by A and B, gives the exact sum.
// D layout: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, column l%32.
constexpr int MG_KB = 128;   // K bytes per stage
constexpr int MG_LS = 144;   // padded LDS row stride

__device__ __forceinline__ int4 ldg16(const int8_t* p) { return *(const int4*)p; }
// expert weights, streamed past the caches in the 64-slot form (experts
// averaging at most 48 slots: one M-tile each, the weights read once), so
// that the activation rows every N-tile shares stay in L2: C4 122-125 ->
// 118-120 us per layer.  The 128-slot form keeps them cacheable: at C5 the
// streamed form was no faster uniform and 13 us slower skewed (hot experts
// span several M-tiles that share each weight tile).
__device__ __forceinline__ int4 ldg16_nt(const int8_t* p) {
  const v4i t = __builtin_nontemporal_load((const v4i*)p);
  return int4{t.x, t.y, t.z, t.w};
}

template <bool GATEUP, int MT, int NW>
__global__ __launch_bounds__(MOTY_WAVE * MT * NW) void k_moe_gemm(
    const int2* __restrict__ tiles, const int* __restrict__ ntiles, const int* __restrict__ offs,
    const int* __restrict__ slot_tok,
    const int8_t* __restrict__ act, const float* __restrict__ act_s,  // GATEUP: xq[T][K], sx[T]; else hq[P][K], sh[P]
    const int8_t* __restrict__ W1, const float* __restrict__ S1,      // [E][N][K], [E][N]
    const int8_t* __restrict__ W2, const float* __restrict__ S2,      // up (GATEUP only)
    float* __restrict__ out,                                          // [P][N]
    int N, int Kd, const int* __restrict__ eslot) {                  // expert -> weight slot, or null
  constexpr int NTH = MOTY_WAVE * MT * NW;  // MT groups of NW waves, one group per 64-slot sub-tile
  constexpr int BM = 64 * MT;               // slots per M-tile
  constexpr int BN = 32 * NW;               // weight rows per N-tile (32 per wave)
  constexpr int BROWS = GATEUP ? 2 * BN : BN;  // staged weight rows
  constexpr int NA = BM * 8 / NTH;                   // 16 B chunks per thread: A
  constexpr int NBW = BROWS * 8 / NTH;               // and B
  __shared__ __align__(16) int8_t sA[BM * MG_LS];
  __shared__ __align__(16) int8_t sB[BROWS * MG_LS];
  __shared__ float s_act[BM];
  // XCD-aware placement (workgroups go round-robin over the 8 XCDs): the
  // N-tiles of one M-tile share an XCD, so its activation rows are pulled
  // into one L2 instead of eight.  Workgroup L runs M-tile 8*(j / nn) + L%8,
  // N-tile j % nn, with j = L / 8 and nn N-tiles.
  const int nn = (N + 32 * NW - 1) / (32 * NW);
  const int jx = blockIdx.x >> 3;
  const int tile = 8 * (jx / nn) + (blockIdx.x & 7);
  const int ntile = jx % nn;
  if (tile >= ntiles[0]) return;
  const int2 tm = tiles[tile];
  const int e = tm.x, mb = tm.y;
  // weight slot of the expert: itself, or its expert-cache slot (-1: not in
  // this pass, the workgroup has nothing to do)
  const int ws = eslot ? eslot[e] : e;
  if (ws < 0) return;
  const int seg0 = offs[e], nseg = offs[e + 1] - seg0;
  const int tid = threadIdx.x, lane = tid % MOTY_WAVE, wv = tid / MOTY_WAVE;
  const int sub = wv / NW, wn = wv % NW;  // this wave: sub-tile, 32-row N slice
  const int r32 = lane & 31, h = lane >> 5;
  const int nb0 = ntile * BN;
  const int msub = mb + 64 * sub;
  const bool one = (nseg - msub) > 0;   // the sub-tile's halves have rows (wave-uniform)
  const bool two = (nseg - msub) > 32;

  // epilogue scales, loaded before the K loop so their latency hides behind
  // it: the activation scale of M-tile row tid % BM (to LDS after the loop)
  // and this lane's weight-row scales
  float srow;
  {
    int m = mb + (tid % BM);
    m = m < nseg ? m : nseg - 1;
    const int sl = seg0 + m;
    srow = act_s[GATEUP ? slot_tok[sl] : sl];
  }
  const int ncol = nb0 + wn * 32 + r32;
  const int ncl = ncol < N ? ncol : N - 1;
  const float s1 = S1[(int64_t)ws * N + ncl];
  const float s2 = GATEUP ? S2[(int64_t)ws * N + ncl] : 0.f;
  // this thread's copy assignments: chunk q -> (row q/8, 16 B column q%8)
  const int8_t* srcA[NA];
  const int8_t* srcB[NBW];
  const int col = (tid & 7) * 16;
#pragma unroll
  for (int i = 0; i < NA; i++) {
    const int row = (tid + i * NTH) >> 3;
    int m = mb + row;
    m = m < nseg ? m : nseg - 1;
    const int slot = seg0 + m;
    const int64_t arow = GATEUP ? (int64_t)slot_tok[slot] : (int64_t)slot;
    srcA[i] = act + arow * Kd + col;
  }
#pragma unroll
  for (int i = 0; i < NBW; i++) {
    const int row = (tid + i * NTH) >> 3;
    const int8_t* W = (GATEUP && row >= BN) ? W2 : W1;
    int n = nb0 + (GATEUP && row >= BN ? row - BN : row);
    n = n < N ? n : N - 1;
    srcB[i] = W + ((int64_t)ws * N + n) * Kd + col;
  }
  // Two register sets: while one K block is consumed from LDS, the next two
  // are in flight from HBM.  Every load is unconditional, from a clamped
  // address (a K chunk past the row end re-reads the row start; a K block
  // past the end re-reads the last block, an L2 hit), and chunks past the
  // end are zeroed when written to LDS: with no branch around a load, the
  // compiler waits only for the register set about to be consumed.
  int4 ra0[NA], rb0[NBW], ra1[NA], rb1[NBW];
  const int klast = (Kd - 1) / MG_KB * MG_KB;
  auto gload = [&](int k0, int4(&ra)[NA], int4(&rb)[NBW]) {
    const int kc = k0 < Kd ? k0 : klast;
    const int off = kc + col < Kd ? kc : -col;  // K % 16 == 0: a chunk is all in or all out
#pragma unroll
    for (int i = 0; i < NA; i++) ra[i] = ldg16(srcA[i] + off);
#pragma unroll
    for (int i = 0; i < NBW; i++) rb[i] = MT == 1 ? ldg16_nt(srcB[i] + off) : ldg16(srcB[i] + off);
    // keep each set's loads together and in issue order
    __builtin_amdgcn_sched_barrier(0);
  };
  v16i acc1[2] = {}, acc2[2] = {};
  auto stage = [&](int k0, int4(&ra)[NA], int4(&rb)[NBW]) {
    const bool ok = k0 + col < Kd;
#pragma unroll
    for (int i = 0; i < NA; i++) *(int4*)(sA + ((tid + i * NTH) >> 3) * MG_LS + col) = sel4(ok, ra[i]);
#pragma unroll
    for (int i = 0; i < NBW; i++) *(int4*)(sB + ((tid + i * NTH) >> 3) * MG_LS + col) = sel4(ok, rb[i]);
    __syncthreads();
    gload(k0 + 2 * MG_KB, ra, rb);
    const int8_t* a0 = sA + (64 * sub + r32) * MG_LS + h * 64;
    const int8_t* a1 = a0 + 32 * MG_LS;
    const int8_t* bg = sB + (wn * 32 + r32) * MG_LS + h * 64;
    const int8_t* bu = bg + BN * MG_LS;
    if (one) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const v4i fa0 = *(const v4i*)(a0 + 16 * j);
        const v4i fg = *(const v4i*)(bg + 16 * j);
        acc1[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa0, fg, acc1[0], 0, 0, 0);
        v4i fu = {};
        if (GATEUP) {
          fu = *(const v4i*)(bu + 16 * j);
          acc2[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa0, fu, acc2[0], 0, 0, 0);
        }
        if (two) {
          const v4i fa1 = *(const v4i*)(a1 + 16 * j);
          acc1[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa1, fg, acc1[1], 0, 0, 0);
          if (GATEUP) acc2[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa1, fu, acc2[1], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  };
  gload(0, ra0, rb0);
  gload(MG_KB, ra1, rb1);
  // an odd number of K blocks runs one all-zero block (adds exactly 0)
  for (int k0 = 0; k0 < Kd; k0 += 2 * MG_KB) {
    stage(k0, ra0, rb0);
    stage(k0 + MG_KB, ra1, rb1);
  }
  // retire every load still in flight (the clamped prefetches past the end)
  // once, here: otherwise the compiler waits for all memory operations --
  // each previous store included -- before every conditional store below
  __builtin_amdgcn_s_waitcnt(0);
  if (tid < BM) s_act[tid] = srow;
  __syncthreads();
  if (ncol >= N || !one) return;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    if (i == 1 && !two) break;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int ml = 64 * sub + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);  // row within the M-tile
      if (mb + ml >= nseg) continue;
      const int sl = seg0 + mb + ml;
      if (GATEUP) {
        const float sxv = s_act[ml];
        const float g = (s1 * sxv) * (float)acc1[i][r];
        const float u = (s2 * sxv) * (float)acc2[i][r];
        out[(int64_t)sl * N + ncol] = ref_silu_mul(g, u);
      } else {
        out[(int64_t)sl * N + ncol] = (s1 * s_act[ml]) * (float)acc1[i][r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// out[t][d] = sum over the token's K rows, FMA in the reference's order:
// order 0 = top-k order (engines/olmoe.c), 1 = ascending expert id (nn/moe.c).
__global__ __launch_bounds__(256) void k_moe_combine(const float* __restrict__ y, const int* __restrict__ idx,
                                                     const float* __restrict__ w, const int* __restrict__ pair_slot,
                                                     float* __restrict__ out, int D, int K, int order) {
  __shared__ int slot_s[64];
  __shared__ float w_s[64];
  const int t = blockIdx.x;
  if (threadIdx.x < MOTY_WAVE) {
    // lane k < K places pair k at its rank: k itself (top-k order) or the
    // number of the token's experts with a smaller id (ascending id; the K
    // ids of a token are distinct)
    const int k = threadIdx.x;
    const int e = k < K ? idx[t * K + k] : 0x7fffffff;
    int rank = k;
    if (order == 1) {
      rank = 0;
      for (int j = 0; j < K; j++) rank += (__shfl(e, j, 64) < e) ? 1 : 0;
    }
    if (k < K) {
      slot_s[rank] = pair_slot[t * K + k];
      w_s[rank] = w[t * K + k];
    }
  }
  __syncthreads();
  const int d = (blockIdx.y * 256 + threadIdx.x) * 4;
  if (d >= D) return;
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < K; j0 += 8) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      // unconditional loads (clamped slot; skipped pairs are not used): a
      // branch around each load would serialize their latencies
      const int sl = (j0 + u < K) ? slot_s[j0 + u] : -1;
      // nontemporal: every row is read once (C5: 70 MB; 220 -> 216 us per layer)
      const v4f t = __builtin_nontemporal_load((const v4f*)(y + (int64_t)(sl >= 0 ? sl : 0) * D + d));
      v[u] = float4{t.x, t.y, t.z, t.w};
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
      if (j0 + u >= K || slot_s[j0 + u] < 0) continue;
      const float wk = w_s[j0 + u];
      acc.x = __fmaf_rn(wk, v[u].x, acc.x);
      acc.y = __fmaf_rn(wk, v[u].y, acc.y);
      acc.z = __fmaf_rn(wk, v[u].z, acc.z);
      acc.w = __fmaf_rn(wk, v[u].w, acc.w);
    }
  }
  *(float4*)(out + (int64_t)t * D + d) = acc;
}

// ---------------------------------------------------------------------------
// Decode (T = 1): moty_nn_moe_topk_d1 (nn/moe.c:33-153).  With one token the
// K routed experts' FFNs are GEMVs over rows nobody else reads, so after the
// routing (k_router, k_route_topk: the token's int8 row and its K experts)
// two launches replace the grouping, the two tile GEMMs, the h quantization
// and the combine:
//   k_moe_d1_gateup  wave per 4 rows of one routed expert: gate and up rows
//                    against the token's int8 row, (s*sx)*acc, silu(g)*u
//                    (nn/moe.c:99-127) -> h [K][I] f32
//   k_moe_d1_down_ew a wave per routed expert and RPW output rows: the
//                    expert's h row quantized in registers (qrow_i8,
//                    nn/moe.c:129-139), its down dots, (ds*sh)*acc
//                    (nn/moe.c:146-152); then the weighted sum in the
//                    reference's order (out = fma(w_k, v_k, out), k in top-k
//                    order; ascending expert id for nn/moe.c's batch order),
//                    written once (no per-pair rows, no combine pass).
constexpr int D1_NW = 4;  // waves per workgroup

__device__ __forceinline__ int4 d1_ldnt16(const int8_t* p) {
  const v4i v = __builtin_nontemporal_load((const v4i*)p);
  return int4{v.x, v.y, v.z, v.w};
}

// Router logits of one token (nn/matmul.c:15-27 -> hw/hw_avx512.h:231-243):
// a half-wave per expert, lane c carrying FMA chain c (elements c, c+32, ...,
// s0 for c < 16, s1 for c >= 16), then s0 + s1 and the _mm512_reduce_add_ps
// tree; plus the logit bias.  A workgroup per two experts (E/2 of them,
// spread over as many CUs): its NWV waves stage x and the two router rows
// in LDS by 16-byte loads (a quarter of the load instructions of 4-byte
// loads per chain element: decode MoE 21.4 -> 21.2 us at the C4 shape; 8
// waves sharing them instead of one: 21.4 -> 20.6 us), then the first wave
// runs the chains, lane c reading its chain's elements back.  NPL >= D/32.
template <int NPL, int NWV>
__global__ __launch_bounds__(NWV * MOTY_WAVE) void k_router_t1v(const float* __restrict__ x, const float* __restrict__ Wr,
                                                          const float* __restrict__ bias, int D, int E,
                                                          float* __restrict__ logits) {
  __shared__ __align__(16) float xs[32 * NPL];
  __shared__ __align__(16) float ws[2][32 * NPL];
  const int lane = threadIdx.x % MOTY_WAVE, c = lane & 31, hf = lane >> 5;
  const int e = blockIdx.x * 2 + hf;
  const int e0 = blockIdx.x * 2 < E ? blockIdx.x * 2 : E - 1, e1 = e0 + 1 < E ? e0 + 1 : E - 1;
  for (int i = threadIdx.x * 4; i < D; i += NWV * MOTY_WAVE * 4) {
    *(float4*)(xs + i) = *(const float4*)(x + i);
    *(float4*)(ws[0] + i) = *(const float4*)(Wr + (int64_t)e0 * D + i);
    *(float4*)(ws[1] + i) = *(const float4*)(Wr + (int64_t)e1 * D + i);
  }
  const float bv = bias ? bias[hf ? e1 : e0] : 0.f;
  __syncthreads();
  if (threadIdx.x >= MOTY_WAVE) return;  // the other waves only helped load
  const float* wr = ws[hf];
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NPL; j++)
    if (j * 32 < D) acc = __fmaf_rn(xs[j * 32 + c], wr[j * 32 + c], acc);
  const float t = acc + __shfl(acc, (lane & 32) + ((c + 16) & 31), 64);  // s0[c] + s1[c]
  float r = hsum16_half(t, lane & 32);
  if (bias) r = r + bv;
  if (c == 0 && e < E) logits[e] = r;
}

// NC: 1 KiB chunks of a gate/up row (D); lane l takes bytes [c*1024 + 16l, +16).
// Every wave routes the token itself from the logits (softmax, greedy top-k:
// the same steps as k_route_topk, a few microseconds less than a launch of its
// own) and quantizes x in registers (qrow_i8); then the 4 rows of its expert.
// Workgroup 0's first wave writes idx, w (and the probabilities).
template <int NC>
__global__ __launch_bounds__(D1_NW * MOTY_WAVE) void k_moe_d1_gateup(
    const float* __restrict__ x, const float* __restrict__ logits, int E, int K, int norm,
    int* __restrict__ idx, float* __restrict__ wout, float* __restrict__ probs,
    const int8_t* __restrict__ G, const float* __restrict__ GS, const int8_t* __restrict__ U,
    const float* __restrict__ US, float* __restrict__ h, int D, int I) {
  __shared__ __align__(16) float lg[D1_NW][256];
  const int lane = threadIdx.x % MOTY_WAVE, wv = threadIdx.x / MOTY_WAVE;
  const int gw = blockIdx.x * D1_NW + wv;  // 4-row group over K*I rows
  const int rpk = (I + 3) / 4;
  if (gw >= K * rpk) return;  // whole waves; no workgroup barrier in this kernel
  const int k = gw / rpk, i0 = (gw % rpk) * 4;
  float4 xv[NC][4];
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const int kk = c * 1024 + lane * 16;
#pragma unroll
    for (int j = 0; j < 4; j++) xv[c][j] = *(const float4*)(x + (kk < D ? kk : 0) + 4 * j);
  }
  for (int e = lane; e < E; e += MOTY_WAVE) lg[wv][e] = logits[e];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  int pe;
  float pw;
  const bool first = blockIdx.x == 0 && wv == 0;
  route_token_regs(lg[wv], E, K, norm, &pe, &pw, first ? probs : nullptr);
  if (first && lane < K) {
    idx[lane] = pe;
    wout[lane] = pw;
  }
  const int e0 = __builtin_amdgcn_readlane(pe, k);
  const int e = e0 < 0 ? 0 : e0;  // a round without a candidate: its rows are not used
  int4 wg[4][NC], wu[4][NC];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int i = i0 + r < I ? i0 + r : I - 1;
    const int8_t* gr = G + ((int64_t)e * I + i) * D;
    const int8_t* ur = U + ((int64_t)e * I + i) * D;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const int kk = c * 1024 + lane * 16;
      wg[r][c] = d1_ldnt16(gr + (kk < D ? kk : 0));
      wu[r][c] = d1_ldnt16(ur + (kk < D ? kk : 0));
    }
  }
  const int rl = wave_sum_row<4>(lane);
  const int ir = i0 + rl < I ? i0 + rl : I - 1;
  const float sg = GS[(int64_t)e * I + ir], su = US[(int64_t)e * I + ir];
  __builtin_amdgcn_sched_barrier(0);
  // qrow_i8 of x while the weights fly
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < NC; c++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      xv[c][j] = sel4(c * 1024 + lane * 16 < D, xv[c][j]);
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(xv[c][j].x), fabsf(xv[c][j].y)), fmaxf(fabsf(xv[c][j].z), fabsf(xv[c][j].w))));
    }
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
      qp[j] = (int)((uint32_t)(rne_int(xv[c][j].x * inv) & 0xff) | ((uint32_t)(rne_int(xv[c][j].y * inv) & 0xff) << 8) |
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
      ag[r] = dot16(wg[r][c], q[c], ag[r]);
      au[r] = dot16(wu[r][c], q[c], au[r]);
    }
  }
  const int a = wave_sum_multi_i32<4>(ag);
  const int a2 = wave_sum_multi_i32<4>(au);
  const float v = ref_silu_mul((sg * sx) * (float)a, (su * sx) * (float)a2);
  if ((lane & 15) == 0 && i0 + rl < I) h[(int64_t)k * I + i0 + rl] = v;
}

// The decode down projection, one wave per routed expert: workgroup = K <= KM
// waves over RPW output rows; wave j takes the expert of combine rank j,
// loads that expert's h row and its RPW down rows, quantizes the h row in
// registers (a wave max is the row's amax: qrow_i8 with no workgroup
// barrier), forms its RPW dots and (ds*sh)*acc, and parks them in LDS; after
// one barrier the first wave runs the ordered weighted sum per row.  A wave
// thus holds one h row and RPW weight rows in flight, not every expert's:
// against one workgroup quantizing all K rows of h for 2 rows per wave, the
// decode MoE at the C4 shape 23.8 -> 21.4 us per token (RPW 8; 4: 22.0,
// 16: 22.3).
template <int KC, int RPW, int KM>
__global__ __launch_bounds__(KM * MOTY_WAVE) void k_moe_d1_down_ew(
    const int* __restrict__ idx, const float* __restrict__ w, const float* __restrict__ h,
    const int8_t* __restrict__ Dn, const float* __restrict__ DS, float* __restrict__ out, int D, int I, int K, int E,
    int order, int* __restrict__ counts) {
  __shared__ float val_s[KM][RPW];
  const int lane = threadIdx.x % MOTY_WAVE, j = threadIdx.x / MOTY_WAVE;
  const int d0 = blockIdx.x * RPW;
  // the expert of combine rank j: rank k = k (top-k order) or the number of
  // smaller expert ids (ascending order; a token's K ids are distinct)
  const int ek = lane < K ? idx[lane] : 0x7fffffff;
  int rank = lane;
  if (order == 1) {
    rank = 0;
    for (int q = 0; q < K; q++) rank += (__shfl(ek, q, 64) < ek) ? 1 : 0;
  }
  const unsigned long long hit = __ballot(lane < K && rank == j);
  const bool live = j < K && hit != 0ull;
  const int kj = live ? (int)__builtin_ctzll(hit) : 0;  // h row of this rank
  const int e0 = __shfl(ek, kj, 64);
  const bool use = live && e0 >= 0;
  const int e = use ? e0 : 0;
  const float wj = w[kj];
  // loads: the h row, then the RPW down rows and their scales
  float4 hv[KC][4];
#pragma unroll
  for (int c = 0; c < KC; c++) {
    const int kk = c * 1024 + lane * 16;
#pragma unroll
    for (int q = 0; q < 4; q++) hv[c][q] = *(const float4*)(h + (int64_t)kj * I + (kk < I ? kk : 0) + 4 * q);
  }
  int4 wd[RPW][KC];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const int d = d0 + r < D ? d0 + r : D - 1;
    const int8_t* dr = Dn + ((int64_t)e * D + d) * I;
#pragma unroll
    for (int c = 0; c < KC; c++) {
      const int kk = c * 1024 + lane * 16;
      wd[r][c] = d1_ldnt16(dr + (kk < I ? kk : 0));
    }
  }
  constexpr int RS = RPW < 4 ? RPW : 4;  // rows per wave sum
  const int rl = wave_sum_row<RS>(lane);
  float dsc[RPW / RS];
#pragma unroll
  for (int t = 0; t < RPW / RS; t++) dsc[t] = DS[(int64_t)e * D + (d0 + t * RS + rl < D ? d0 + t * RS + rl : D - 1)];
  __builtin_amdgcn_sched_barrier(0);
  // qrow_i8 of the h row in registers (fmaxf drops NaN as the reference's
  // `a > amax` does)
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < KC; c++)
#pragma unroll
    for (int q = 0; q < 4; q++) {
      hv[c][q] = sel4(c * 1024 + lane * 16 < I, hv[c][q]);
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(hv[c][q].x), fabsf(hv[c][q].y)), fmaxf(fabsf(hv[c][q].z), fabsf(hv[c][q].w))));
    }
  amax = wave_max_f32(amax);
  float sh = amax / 127.f;
  if (sh < 1e-12f) sh = 1e-12f;
  const float inv = 1.f / sh;
  int4 hq[KC];
#pragma unroll
  for (int c = 0; c < KC; c++) {
    int* qp = (int*)&hq[c];
#pragma unroll
    for (int q = 0; q < 4; q++)
      qp[q] = (int)((uint32_t)(rne_int(hv[c][q].x * inv) & 0xff) | ((uint32_t)(rne_int(hv[c][q].y * inv) & 0xff) << 8) |
                    ((uint32_t)(rne_int(hv[c][q].z * inv) & 0xff) << 16) |
                    ((uint32_t)(rne_int(hv[c][q].w * inv) & 0xff) << 24));
  }
  int acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    acc[r] = 0;
#pragma unroll
    for (int c = 0; c < KC; c++) acc[r] = dot16(wd[r][c], hq[c], acc[r]);
  }
#pragma unroll
  for (int t = 0; t < RPW / RS; t++) {
    int part[RS];
#pragma unroll
    for (int q = 0; q < RS; q++) part[q] = acc[t * RS + q];
    const int a = wave_sum_multi_i32<RS>(part);
    if ((lane & (MOTY_WAVE / RS - 1)) == 0) val_s[j][t * RS + rl] = (dsc[t] * sh) * (float)a;
  }
  if (blockIdx.x == 0 && j == 0 && counts) {
    for (int x = lane; x < E; x += MOTY_WAVE) {
      int cnt = 0;
      for (int q = 0; q < K; q++) cnt += __shfl(ek, q, 64) == x;
      counts[x] = cnt;
    }
  }
  // each wave's weight of its rank, for the combine
  __shared__ float w_s[KM];
  __shared__ int u_s[KM];
  if (lane == 0) {
    w_s[j] = wj;
    u_s[j] = use ? 1 : 0;
  }
  __syncthreads();
  // the ordered weighted sum out = fma(w, v, out) from 0 (nn/moe.c:146-152
  // and 200-202), one lane per row
  if (j == 0 && lane < RPW && d0 + lane < D) {
    float o = 0.f;
#pragma unroll
    for (int q = 0; q < KM; q++)
      if (q < K && u_s[q]) o = __fmaf_rn(w_s[q], val_s[q][lane], o);
    out[d0 + lane] = o;
  }
}

// ---------------------------------------------------------------------------
size_t moe_scratch_size(int T, int D, int E, int K, int I, size_t* offsets) {
  const int64_t P = (int64_t)T * K;
  const int64_t maxt = P / MOE_BM + E + 1;
  size_t sz[MOE_NBUF] = {(size_t)T * D,       (size_t)T * 4,     (size_t)P * 4, (size_t)P * 4,
                         (size_t)(E + 1) * 4, (size_t)P * 4,     (size_t)P * 4, (size_t)maxt * 8,
                         16,                  (size_t)P * I * 4, (size_t)P * I, (size_t)P * 4,
                         (size_t)P * D * 4,   (size_t)E * 4,     (size_t)T * E * 4};
  size_t o = 0;
  for (int i = 0; i < MOE_NBUF; i++) {
    offsets[i] = o;
    o += (sz[i] + 255) / 256 * 256;
  }
  return o;
}

struct MoeBufs {
  int8_t* xq;
  float *sx, *w, *h, *sh, *y, *logits;
  int *idx, *offs, *slot_tok, *pair_slot, *ntiles, *counts;
  int2* tiles;
  int8_t* hq;
};

static MoeBufs moe_bufs(const MoeArgs& a, void* scratch) {
  size_t off[MOE_NBUF];
  moe_scratch_size(a.T, a.D, a.E, a.K, a.I, off);
  char* b = (char*)scratch;
  MoeBufs m;
  m.xq = (int8_t*)(b + off[0]);
  m.sx = (float*)(b + off[1]);
  m.idx = (int*)(b + off[2]);
  m.w = (float*)(b + off[3]);
  m.offs = (int*)(b + off[4]);
  m.slot_tok = (int*)(b + off[5]);
  m.pair_slot = (int*)(b + off[6]);
  m.tiles = (int2*)(b + off[7]);
  m.ntiles = (int*)(b + off[8]);
  m.h = (float*)(b + off[9]);
  m.hq = (int8_t*)(b + off[10]);
  m.sh = (float*)(b + off[11]);
  m.y = (float*)(b + off[12]);
  m.counts = (int*)(b + off[13]);
  m.logits = (float*)(b + off[14]);
  return m;
}

// 128-slot M-tiles when experts average more than 48 slots (one pass over
// an expert's weights for up to 128 slots), 64-slot tiles otherwise
static int moe_mt(const MoeArgs& a) { return ((int64_t)a.T * a.K > 48 * (int64_t)a.E) ? 2 : 1; }

void moe_routing(const MoeArgs& a, void* scratch, const int** idx, const int** counts) {
  const MoeBufs m = moe_bufs(a, scratch);
  *idx = m.idx;
  *counts = m.counts;
}

int launch_moe_route(const MoeArgs& a, void* scratch, hipStream_t st, bool group) {
  const int T = a.T, D = a.D, E = a.E, K = a.K, I = a.I;
  if (K < 1 || K > 64 || K > E || E > 256 || (D % 32) || (I % 32) || (D % 4)) return MOTY_EUNSUP;
  const MoeBufs m = moe_bufs(a, scratch);
  const int P = T * K;
  // router tiles, from a sweep on MI355X (graph replays, rotating x): 8
  // tokens x 8 experts of 4 waves with a 4-stage ring for small layers
  // (T = 256, E = 64: 7.0 us against 7.9 with 8 stages, 9.1 for 8 x 16),
  // 24 tokens x 32 experts of 12 waves otherwise (T = 1072, E = 128: 20.0
  // us; 16 x 16: 23.5, 8 x 16: 21.3, 16 x 32: 28.0); token slices keep every
  // buffer offset below 2^31 bytes
  const bool small = E <= 64 && T <= 1024;
  const int tw = small ? 8 : 24, eg = small ? 8 : 32, nsl = (E + eg - 1) / eg;
  const int tmax = (int)(((int64_t)1 << 31) / ((int64_t)D * 4)) / tw * tw;
  if (tmax < tw) return MOTY_EUNSUP;
  for (int t0 = 0; t0 < T; t0 += tmax) {
    const int ts = T - t0 < tmax ? T - t0 : tmax;
    const float* x = a.x + (int64_t)t0 * D;
    const dim3 grid((unsigned)((((ts + tw - 1) / tw + 7) / 8) * 8 * nsl));
    if (small)
      hipLaunchKernelGGL((k_router<4, 4, 2, 2, 4, 8, 4>), grid, dim3(256), 0, st, x, a.Wr, a.bias, ts, D, E,
                         m.logits + (int64_t)t0 * E);
    else
      hipLaunchKernelGGL((k_router<8, 8, 3, 4, 4, 4, 3>), grid, dim3(768), 0, st, x, a.Wr, a.bias, ts, D, E,
                         m.logits + (int64_t)t0 * E);
    LAUNCH_TRY("k_router");
  }
  hipLaunchKernelGGL(k_route_topk, dim3((T + TK_TOK - 1) / TK_TOK), dim3(TK_TOK * 128), 0, st, a.x, m.logits, T, D, E,
                     K, a.norm, m.idx, m.w, m.xq, m.sx, a.probs_out);
  LAUNCH_TRY("k_route_topk");
  if (!group) return MOTY_OK;
  const int mt = moe_mt(a);
  {
    // one workgroup per GR_CHUNK pairs, at most 32 (each one reads all P
    // ids, so more would only add L2 reads): C5's 8576 pairs take 32
    const int nch = (P + GR_CHUNK - 1) / GR_CHUNK;
    const int g = nch < 1 ? 1 : nch < 32 ? nch : 32;
    const int chunk = (P + g - 1) / g;
    hipLaunchKernelGGL(k_group, dim3(g), dim3(GR_NT), 0, st, m.idx, P, K, E, 64 * mt, chunk, m.offs, m.slot_tok,
                       m.pair_slot, m.tiles, m.ntiles, m.counts);
  }
  LAUNCH_TRY("k_group");
  return MOTY_OK;
}

int launch_moe_experts(const MoeArgs& a, void* scratch, const int* eslot, hipStream_t st) {
  const int D = a.D, E = a.E, I = a.I;
  const MoeBufs m = moe_bufs(a, scratch);
  const int P = a.T * a.K, mt = moe_mt(a);
  const int maxt = P / (64 * mt) + E + 1;
  // one workgroup per (M-tile, 128-row N-tile), M-tiles padded to a
  // multiple of the 8 XCDs (the kernel maps workgroup -> tile XCD-aware)
  const int maxt8 = (maxt + 7) / 8 * 8;
  if (mt == 2)
    hipLaunchKernelGGL((k_moe_gemm<true, 2, 4>), dim3((unsigned)(((I + 127) / 128) * maxt8)), dim3(512), 0, st,
                       m.tiles, m.ntiles, m.offs, m.slot_tok, m.xq, m.sx, a.G, a.GS, a.U, a.US, m.h, I, D, eslot);
  else
    hipLaunchKernelGGL((k_moe_gemm<true, 1, 4>), dim3((unsigned)(((I + 127) / 128) * maxt8)), dim3(256), 0, st,
                       m.tiles, m.ntiles, m.offs, m.slot_tok, m.xq, m.sx, a.G, a.GS, a.U, a.US, m.h, I, D, eslot);
  LAUNCH_TRY("k_moe_gemm<gateup>");
  int rc = launch_qrow_i8(m.h, m.hq, m.sh, nullptr, P, I, I, I, st);
  if (rc) return rc;
  if (mt == 2)
    hipLaunchKernelGGL((k_moe_gemm<false, 2, 4>), dim3((unsigned)(((D + 127) / 128) * maxt8)), dim3(512), 0, st,
                       m.tiles, m.ntiles, m.offs, m.slot_tok, m.hq, m.sh, a.Dn, a.DS, nullptr, nullptr, m.y, D, I, eslot);
  else
    hipLaunchKernelGGL((k_moe_gemm<false, 1, 4>), dim3((unsigned)(((D + 127) / 128) * maxt8)), dim3(256), 0, st,
                       m.tiles, m.ntiles, m.offs, m.slot_tok, m.hq, m.sh, a.Dn, a.DS, nullptr, nullptr, m.y, D, I, eslot);
  LAUNCH_TRY("k_moe_gemm<down>");
  return MOTY_OK;
}

int launch_moe_combine(const MoeArgs& a, void* scratch, hipStream_t st) {
  const int T = a.T, D = a.D, K = a.K, P = a.T * a.K;
  const MoeBufs m = moe_bufs(a, scratch);
  hipLaunchKernelGGL(k_moe_combine, dim3(T, (D / 4 + 255) / 256), dim3(256), 0, st, m.y, m.idx, m.w, m.pair_slot,
                     a.out, D, K, a.order);
  LAUNCH_TRY("k_moe_combine");
  if (a.idx_out) HIP_TRY(hipMemcpyAsync(a.idx_out, m.idx, (size_t)P * 4, hipMemcpyDeviceToDevice, st));
  if (a.w_out) HIP_TRY(hipMemcpyAsync(a.w_out, m.w, (size_t)P * 4, hipMemcpyDeviceToDevice, st));
  if (a.counts_out) HIP_TRY(hipMemcpyAsync(a.counts_out, m.counts, (size_t)a.E * 4, hipMemcpyDeviceToDevice, st));
  return MOTY_OK;
}

// the decode path's shapes: one token, K <= 8 experts of E <= 256, D and I
// <= 4 KiB rows (D % 32 == 0 as the routing requires)
static bool moe_d1(const MoeArgs& a) {
  return a.T == 1 && a.K >= 1 && a.K <= 8 && a.K <= a.E && a.E <= 256 && a.D <= 4096 && a.I <= 4096 &&
         a.D % 32 == 0 && a.I % 32 == 0;
}

static int launch_moe_d1(const MoeArgs& a, void* scratch, hipStream_t st) {
  const MoeBufs m = moe_bufs(a, scratch);
  const int D = a.D, I = a.I, K = a.K, E = a.E;
#define RT(N)                                                                                                \
  case N:                                                                                                    \
    hipLaunchKernelGGL((k_router_t1v<N, 8>), dim3((E + 1) / 2), dim3(8 * MOTY_WAVE), 0, st, a.x, a.Wr, a.bias, D, E,    \
                       m.logits);                                                                            \
    break;
  switch ((D / 32 + 15) / 16 * 16) {
    RT(16) RT(32) RT(48) RT(64) RT(80) RT(96) RT(112) RT(128)
    default: return MOTY_EUNSUP;
  }
#undef RT
  LAUNCH_TRY("k_router_t1v");
  const int nc = (D + 1023) / 1024, kc = (I + 1023) / 1024;
  const unsigned gu_blocks = (unsigned)((K * ((I + 3) / 4) + D1_NW - 1) / D1_NW);
#define GU(N)                                                                                                  \
  case N:                                                                                                      \
    hipLaunchKernelGGL((k_moe_d1_gateup<N>), dim3(gu_blocks), dim3(D1_NW * MOTY_WAVE), 0, st, a.x, m.logits, E, K, \
                       a.norm, m.idx, m.w, a.probs_out, a.G, a.GS, a.U, a.US, m.h, D, I);                    \
    break;
  switch (nc) {
    GU(1) GU(2) GU(3) GU(4)
    default: return MOTY_EUNSUP;
  }
#undef GU
  LAUNCH_TRY("k_moe_d1_gateup");
  // eight output rows per workgroup of one wave per routed expert (four
  // for rows of 3-4 KiB)
  const int rpw = kc <= 2 ? 8 : 4;
#define DE(KC, R)                                                                                             \
  if (kc == KC && rpw == R) {                                                                                 \
    hipLaunchKernelGGL((k_moe_d1_down_ew<KC, R, 8>), dim3((D + R - 1) / R), dim3(K * MOTY_WAVE), 0, st, m.idx, m.w, \
                       m.h, a.Dn, a.DS, a.out, D, I, K, a.E, a.order, m.counts);                               \
    LAUNCH_TRY("k_moe_d1_down_ew");                                                                            \
  }
  DE(1, 8) DE(2, 8) DE(3, 4) DE(4, 4)
#undef DE
  if (a.idx_out) HIP_TRY(hipMemcpyAsync(a.idx_out, m.idx, (size_t)K * 4, hipMemcpyDeviceToDevice, st));
  if (a.w_out) HIP_TRY(hipMemcpyAsync(a.w_out, m.w, (size_t)K * 4, hipMemcpyDeviceToDevice, st));
  if (a.counts_out) HIP_TRY(hipMemcpyAsync(a.counts_out, m.counts, (size_t)a.E * 4, hipMemcpyDeviceToDevice, st));
  return MOTY_OK;
}

int launch_moe(const MoeArgs& a, void* scratch, hipStream_t st) {
  if (a.T <= 0) return MOTY_OK;
  if (moe_d1(a)) return launch_moe_d1(a, scratch, st);
  int rc = launch_moe_route(a, scratch, st);
  if (!rc) rc = launch_moe_experts(a, scratch, nullptr, st);
  if (!rc) rc = launch_moe_combine(a, scratch, st);
  return rc;
}

}  // namespace moty
