// gemm_q8.hip -- Q8_0 prefill GEMM on int8 MFMA (v_mfma_i32_32x32x32_i8).
//
// Reference: moty_matmul_q_s (nn/matmul.c:51-66) for S > 1 token rows:
//     y[s*O+o] = (scale[o]*sx[s]) * (float)sum_i W[o][i]*xq[s][i]
// The int32 accumulation is exact in any order, so the MFMA result equals
// the reference's VPDPBUSD chains bit for bit; the epilogue keeps the
// reference's two multiplies.
//
// Both operands are K-contiguous (xq [S][I] token-major, W [O][I] row-major),
// so both stage into LDS the same way and feed the matrix cores alike.
#include "common.h"
#include "kernels.h"
#include <stdlib.h>

namespace moty {

constexpr int GM_NT = 256;  // 4 waves, 2 x 2 over the block tile
constexpr int GM_KB = 128;  // K bytes per stage
constexpr int GM_LS = 144;  // padded LDS row stride

// y[M][O] from xq[M][K], W[O][K]; K % 16 == 0.  Block tile BM x BN with
// BM = 64*WM, BN = 64*WN; wave (wm, wn) owns (32*WM) x (32*WN) outputs as
// WM x WN v_mfma_i32_32x32x32_i8 tiles.  Per 128-byte K block the tile is
// staged in LDS by whole-line loads (8 lanes x 16 B per row); NS register
// sets keep the next K blocks' loads in flight during the MFMAs.  MFMA step
// j takes, in lane l, bytes [64*(l/32) + 16j, +16) of row (l % 32): a
// k-permutation shared by both operands, exact for integer dots.
template <int WM, int WN, int NS = 2>
__global__ __launch_bounds__(GM_NT, 2) void k_gemm_q8(const int8_t* __restrict__ xq, const float* __restrict__ sx,
                                                      const int8_t* __restrict__ W, const float* __restrict__ scale,
                                                      float* __restrict__ y, int M, int K, int O) {
  constexpr int BM = 64 * WM, BN = 64 * WN;
  constexpr int NA = BM * 8 / GM_NT, NB = BN * 8 / GM_NT;
  __shared__ __align__(16) int8_t sA[BM * GM_LS];
  __shared__ __align__(16) int8_t sB[BN * GM_LS];
  const int tid = threadIdx.x, lane = tid % MOTY_WAVE, wv = tid / MOTY_WAVE;
  const int wm = wv >> 1, wn = wv & 1;
  const int r32 = lane & 31, h = lane >> 5;
  // blockIdx.x walks N tiles fastest: consecutive workgroups share activation rows
  const int mb = blockIdx.y * BM, nb = blockIdx.x * BN;
  const int col = (tid & 7) * 16;
  const int8_t* srcA[NA];
  const int8_t* srcB[NB];
#pragma unroll
  for (int i = 0; i < NA; i++) {
    int m = mb + ((tid + i * GM_NT) >> 3);
    m = m < M ? m : M - 1;
    srcA[i] = xq + (int64_t)m * K + col;
  }
#pragma unroll
  for (int i = 0; i < NB; i++) {
    int n = nb + ((tid + i * GM_NT) >> 3);
    n = n < O ? n : O - 1;
    srcB[i] = W + (int64_t)n * K + col;
  }
  // NS register sets: while one K block is consumed from LDS, the next NS
  // are in flight from HBM.  Every load is unconditional, from a clamped
  // address (a chunk past the row end re-reads the row start; a K block past
  // the end re-reads the last block, an L2 hit), and chunks past the end are
  // zeroed when written to LDS: with no branch around a load, the compiler
  // waits only for the register set about to be consumed.
  int4 setA[NS][NA], setB[NS][NB];
  const int klast = (K - 1) / GM_KB * GM_KB;
  auto gload = [&](int k0, int4(&ra)[NA], int4(&rb)[NB]) {
    const int kc = k0 < K ? k0 : klast;
    const int off = kc + col < K ? kc : -col;
#pragma unroll
    for (int i = 0; i < NA; i++) ra[i] = *(const int4*)(srcA[i] + off);
#pragma unroll
    for (int i = 0; i < NB; i++) rb[i] = *(const int4*)(srcB[i] + off);
    // keep each set's loads together and in issue order
    __builtin_amdgcn_sched_barrier(0);
  };
  // epilogue scales, loaded before the K loop so that their latency hides
  // behind it: the tile's activation-row scales (to LDS after the loop) and
  // this lane's weight-row scales
  __shared__ float s_sx[BM];
  float sxr;
  {
    const int m = mb + tid % BM;
    sxr = sx[m < M ? m : M - 1];
  }
  float scn[WN];
#pragma unroll
  for (int j = 0; j < WN; j++) {
    const int n = nb + wn * 32 * WN + j * 32 + r32;
    scn[j] = scale[n < O ? n : O - 1];
  }
  v16i acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; i++)
#pragma unroll
    for (int j = 0; j < WN; j++) acc[i][j] = v16i{};
  auto stage = [&](int k0, int4(&ra)[NA], int4(&rb)[NB]) {
    const bool ok = k0 + col < K;
#pragma unroll
    for (int i = 0; i < NA; i++) *(int4*)(sA + ((tid + i * GM_NT) >> 3) * GM_LS + col) = sel4(ok, ra[i]);
#pragma unroll
    for (int i = 0; i < NB; i++) *(int4*)(sB + ((tid + i * GM_NT) >> 3) * GM_LS + col) = sel4(ok, rb[i]);
    __syncthreads();
    gload(k0 + NS * GM_KB, ra, rb);
    if (k0 < K) {  // a trailing block past the end adds nothing: skip it
#pragma unroll
    for (int st = 0; st < 4; st++) {
      v4i fa[WM], fb[WN];
#pragma unroll
      for (int i = 0; i < WM; i++)
        fa[i] = *(const v4i*)(sA + (wm * 32 * WM + i * 32 + r32) * GM_LS + h * 64 + 16 * st);
#pragma unroll
      for (int j = 0; j < WN; j++)
        fb[j] = *(const v4i*)(sB + (wn * 32 * WN + j * 32 + r32) * GM_LS + h * 64 + 16 * st);
#pragma unroll
      for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    }
    __syncthreads();
  };
#pragma unroll
  for (int i = 0; i < NS; i++) gload(i * GM_KB, setA[i], setB[i]);
  for (int k0 = 0; k0 < K; k0 += NS * GM_KB) {
#pragma unroll
    for (int i = 0; i < NS; i++) stage(k0 + i * GM_KB, setA[i], setB[i]);
  }
  // retire every load still in flight (the clamped prefetches past the end)
  // once, here: otherwise the compiler waits for all memory operations --
  // each previous store included -- before every conditional store below
  __builtin_amdgcn_s_waitcnt(0);
  if (tid < BM) s_sx[tid] = sxr;
  __syncthreads();
  // D layout: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, column l%32
#pragma unroll
  for (int j = 0; j < WN; j++) {
    const int n = nb + wn * 32 * WN + j * 32 + r32;
    if (n >= O) continue;
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int ml = wm * 32 * WM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (mb + ml < M) __builtin_nontemporal_store((scn[j] * s_sx[ml]) * (float)acc[i][j][r], y + (int64_t)(mb + ml) * O + n);
      }
  }
}

// The same GEMM for K % 128 == 0 with the operand tiles moved by DMA:
// global_load_lds writes each 16-byte chunk straight into LDS (no register
// staging), S - 1 K blocks ahead of the MFMAs.  A stage holds the BM
// activation rows then the BN weight rows, 128 bytes each, dense; chunk c of
// row r sits in 16-byte slot c ^ ((r >> 1) & 7), so the 16 lanes that one
// ds_read_b128 cycle serves (rows r..r+15, one chunk) hit 16 distinct
// 16-byte bank groups.  A DMA instruction fills 8 rows (1 KiB): lane l loads
// row l/8's chunk (l%8) ^ ((row >> 1) & 7) into slot l%8.
// WGM x WGN waves over the block tile (each wave TM x TN outputs).  KS = 2
// runs two such groups of waves on alternate K blocks (the int32 partial
// sums are added at the end: exact), doubling the loads and MFMAs in flight
// per workgroup where the grid has few tiles.
template <int BM, int BN, int S, int WGM = 2, int WGN = 2, int KS = 1>
__global__ __launch_bounds__(64 * WGM * WGN * KS) void k_gemm_q8_dma(const int8_t* __restrict__ xq,
                                                                     const float* __restrict__ sx,
                                                                     const int8_t* __restrict__ W,
                                                                     const float* __restrict__ scale,
                                                                     float* __restrict__ y, int M, int K, int O) {
  constexpr int NW = WGM * WGN;              // waves per K group
  constexpr int STAGE = (BM + BN) * GM_KB;   // one K group's share of a stage
  constexpr int NI = (BM + BN) / (8 * NW);   // DMA instructions per wave per stage
  constexpr int TM = BM / WGM, TN = BN / WGN, FM = TM / 32, FN = TN / 32;
  static_assert((BM + BN) % (8 * NW) == 0 && FM >= 1 && FN >= 1, "tile shape");
  static_assert(KS == 1 || KS * STAGE * S >= (KS - 1) * NW * 64 * FM * FN * 64, "room for the partial sums");
  __shared__ __align__(1024) int8_t lds[S * KS * STAGE];
  __shared__ float s_sx[BM];
  const int tid = threadIdx.x, lane = tid % MOTY_WAVE, wv = tid / MOTY_WAVE;
  const int kg = wv / NW, w = wv % NW;
  const int wm = w / WGN, wn = w % WGN;
  const int r32 = lane & 31, h = lane >> 5;
  int bx = blockIdx.x, by = blockIdx.y;
  {
    // workgroups go round-robin over the 8 XCDs by linear id: give XCD x a
    // (gy/2) x (gx/4) block of tiles, so its L2 pulls in half the
    // activation rows and a quarter of the weight rows (row-major order
    // gave each XCD every activation row and an eighth of the weights)
    const int gx = gridDim.x, gy = gridDim.y;
    if (gx % 4 == 0 && gy % 2 == 0) {
      const int lin = by * gx + bx, x = lin & 7, j = lin >> 3;
      const int bw = gx / 4;
      bx = (x & 3) * bw + j % bw;
      by = (x >> 2) * (gy / 2) + j / bw;
    }
  }
  const int mb = by * BM, nb = bx * BN;
  const int8_t* src[NI];
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int row = (i * NW + w) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((row >> 1) & 7);
    if (row < BM) {
      const int m = mb + row < M ? mb + row : M - 1;  // rows past the end: loaded, never stored
      src[i] = xq + (int64_t)m * K + c * 16;
    } else {
      const int n = nb + row - BM < O ? nb + row - BM : O - 1;
      src[i] = W + (int64_t)n * K + c * 16;
    }
  }
  const int nk = K / GM_KB;
  const int nsb = (nk + KS - 1) / KS;  // iterations: KS K blocks each
  // iteration sb brings K block sb*KS + kg into this group's part of stage
  // sb % S; blocks past the end reload the last one (their stage is never
  // read), so every iteration issues the same count
  auto issue = [&](int sb) {
    const int kb = sb * KS + kg;
    const int kc = (kb < nk ? kb : nk - 1) * GM_KB;
    const uint32_t base = (uint32_t)(uintptr_t)lds + ((sb % S) * KS + kg) * STAGE + w * 1024;
#pragma unroll
    for (int i = 0; i < NI; i++) dma16_to_lds(src[i] + kc, __builtin_amdgcn_readfirstlane(base + i * NW * 1024));
  };
  // epilogue scales first: their loads are the oldest, so the vmcnt waits
  // below (which count only the DMAs after them) also cover them
  float sxr;
  {
    const int m = mb + tid % BM;
    sxr = sx[m < M ? m : M - 1];
  }
  float scn[FN];
#pragma unroll
  for (int j = 0; j < FN; j++) {
    const int n = nb + wn * TN + j * 32 + r32;
    scn[j] = scale[n < O ? n : O - 1];
  }
#pragma unroll
  for (int s = 0; s < S - 1; s++) issue(s);
  v16i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = v16i{};
  for (int sb = 0; sb < nsb; sb++) {
    // this wave's DMAs of iteration sb have landed (the S-2 later ones may
    // still fly); the barrier makes every wave's share visible and retires
    // the reads of iteration sb-1, whose stage the next DMA overwrites
    MOTY_WAIT_VMCNT((S - 2) * NI);
    __syncthreads();
    issue(sb + S - 1);
    if (KS > 1 && sb * KS + kg >= nk) continue;  // the group's block is past the end (wave-uniform)
    const int8_t* st = lds + ((sb % S) * KS + kg) * STAGE;
#pragma unroll
    for (int j4 = 0; j4 < 4; j4++) {
      // MFMA step j4 takes chunk 4h + j4 of row r32 (a k-permutation shared
      // by both operands: exact for integer dots)
      const int sw = ((h * 4 + j4) ^ ((r32 >> 1) & 7)) * 16;
      v4i fa[FM], fb[FN];
#pragma unroll
      for (int i = 0; i < FM; i++) fa[i] = *(const v4i*)(st + (wm * TM + i * 32 + r32) * GM_KB + sw);
#pragma unroll
      for (int j = 0; j < FN; j++) fb[j] = *(const v4i*)(st + (BM + wn * TN + j * 32 + r32) * GM_KB + sw);
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  }
  // every DMA (including the reloads past the end) lands before the
  // workgroup's LDS can be released or reused
  __builtin_amdgcn_s_waitcnt(0);
  if (KS > 1) {
    // the other groups' partial sums through LDS, added by the first (int32:
    // exact in any order)
    __syncthreads();
    constexpr int PW = FM * FN * 16;  // ints per lane
    if (kg > 0) {
      int* part = (int*)lds + (((kg - 1) * NW + w) * 64 + lane) * PW;
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) *(v16i*)(part + (i * FN + j) * 16) = acc[i][j];
    }
    __syncthreads();
    if (kg == 0) {
#pragma unroll
      for (int q = 1; q < KS; q++) {
        const int* part = (const int*)lds + (((q - 1) * NW + w) * 64 + lane) * PW;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++) acc[i][j] += *(const v16i*)(part + (i * FN + j) * 16);
      }
    }
  }
  if (tid < BM) s_sx[tid] = sxr;
  __syncthreads();
  if (kg) return;
#pragma unroll
  for (int j = 0; j < FN; j++) {
    const int n = nb + wn * TN + j * 32 + r32;
    if (n >= O) continue;
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int ml = wm * TM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (mb + ml < M) __builtin_nontemporal_store((scn[j] * s_sx[ml]) * (float)acc[i][j][r], y + (int64_t)(mb + ml) * O + n);
      }
  }
}

int launch_gemm_q8(const int8_t* xq, const float* sx, const int8_t* W, const float* scale, float* y, int M,
                   int K, int O, hipStream_t st) {
  if (K % 16) return MOTY_EUNSUP;
  if (M <= 0 || O <= 0) return MOTY_OK;
  if (K % GM_KB == 0) {
    // 64 x 64 tiles (several workgroups per CU hide the DMA latency); three
    // stages for K <= 1024, four for longer rows.  Measured on MI355X, M =
    // 512: N=10240, K=1024: 17.3 us vs 18.8 register-staged; K=2048, N=1024:
    // 7.7 vs 9.6; K=3072: 10.0 vs 12.5.
    // Tiles from a sweep on MI355X at M = 512 (the C2 projections): 64 x 64
    // tiles of 4 waves while the grid holds at least 256 of them (N = 10240,
    // K = 1024: 15.2 us); below that 64 x 32 tiles with two groups of 2 waves
    // on alternate K blocks (N = 1024, K = 2048: 7.1 us vs 7.4; K = 3072: 8.7
    // vs 9.3) -- these GEMMs are bound by each workgroup's K-loop latency,
    // not by the grid's width.  Four groups of 2 waves (three stages) where
    // K holds at least 4 blocks: 6.3 / 7.3 us against 6.9 / 8.5 with two,
    // timed back to back on rotating weights (inside the C2 layer step, after
    // the wide GEMM, both forms average 8.0 us).  Grids of at least 512
    // tiles of 64 x 128 with K <= 1024 (C2's fused N = 10240): those tiles,
    // 8 waves, two stages, 13.3 us against 15.0 (median 14.2 against 16.8)
    // for 64 x 64 in three; 128 x 64 13.5, 128 x 128 13.8-14.1, three stages
    // of 64 x 128 16.2.  Both GEMMs write y with nontemporal stores: the
    // output (21 MB for C2's fused GEMM) then does not sit dirty in L2 to be
    // evicted under the next kernels' reads (C2 step 42.7 -> 40.8 us).
#define QD(BM, BN, S, WM, WN, KS)                                                                             \
  hipLaunchKernelGGL((k_gemm_q8_dma<BM, BN, S, WM, WN, KS>), dim3((O + BN - 1) / BN, (M + BM - 1) / BM),       \
                     dim3(64 * WM * WN * KS), 0, st, xq, sx, W, scale, y, M, K, O)
    const bool narrow = (int64_t)((M + 63) / 64) * ((O + 63) / 64) < 256;
    if (narrow && K >= 4 * GM_KB) QD(64, 32, 3, 2, 1, 4);
    else if (narrow && K >= 2 * GM_KB) QD(64, 32, 4, 2, 1, 2);
    else if (K <= 1024 && (int64_t)((M + 63) / 64) * ((O + 127) / 128) >= 512) QD(64, 128, 2, 2, 4, 1);
    else if (K <= 1024) QD(64, 64, 3, 2, 2, 1);
    else QD(64, 64, 4, 2, 2, 1);
#undef QD
    LAUNCH_TRY("k_gemm_q8_dma");
    return MOTY_OK;
  }
  // Tiles and prefetch depth from a sweep on MI355X (M = 512, the C2
  // projections): 64 x 64 tiles beat 128 x 128 until the grid holds several
  // workgroups per CU (N=10240, K=1024: 17.1 us vs 18.5); long K rows keep
  // four K blocks in flight (K=2048: 9.6 us vs 10.1, K=3072: 12.5 vs 13.5).
  auto nblk = [&](int bm, int bn) { return (int64_t)((M + bm - 1) / bm) * ((O + bn - 1) / bn); };
  if (nblk(128, 128) >= 1024) {
    hipLaunchKernelGGL((k_gemm_q8<2, 2>), dim3((O + 127) / 128, (M + 127) / 128), dim3(GM_NT), 0, st, xq, sx, W,
                       scale, y, M, K, O);
  } else if (K >= 2048) {
    hipLaunchKernelGGL((k_gemm_q8<1, 1, 4>), dim3((O + 63) / 64, (M + 63) / 64), dim3(GM_NT), 0, st, xq, sx, W,
                       scale, y, M, K, O);
  } else {
    hipLaunchKernelGGL((k_gemm_q8<1, 1>), dim3((O + 63) / 64, (M + 63) / 64), dim3(GM_NT), 0, st, xq, sx, W, scale,
                       y, M, K, O);
  }
  LAUNCH_TRY("k_gemm_q8");
  return MOTY_OK;
}

}  // namespace moty
