// kernels.h -- launchers shared between the kernel translation units and the
// C-ABI layer (api.cpp).  Every launcher is asynchronous on `st` and returns
// MOTY_OK or an error code; none allocates.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace moty {

constexpr int GEMV_MAX_S = 4;  // token rows served by the decode GEMVs
constexpr int MOE_BM = 64;     // slots per M-tile of the grouped MoE GEMMs
constexpr int MOE_NBUF = 15;   // MoE scratch sub-buffers

// several qrow_i8 jobs (dense rows, I <= 4096, I % 16 == 0) in one launch
constexpr int QROW_MAX_JOBS = 4;
struct QrowJobs {
  const float* x[QROW_MAX_JOBS];
  int8_t* q[QROW_MAX_JOBS];
  float* sx[QROW_MAX_JOBS];
  int S[QROW_MAX_JOBS], I[QROW_MAX_JOBS];
  int b0[QROW_MAX_JOBS + 1];  // first workgroup of each job (set by the launcher)
  int n;
};
int launch_qrow_multi(QrowJobs jb, hipStream_t st);
int launch_qrow_i8(const float* x, int8_t* q, float* sx, int32_t* xg, int S, int I, int64_t ldx, int64_t ldq,
                   hipStream_t st);
// qrow_i8 with f16 codes in the k-permuted fragment order of the f16-MFMA
// grouped-int4 GEMM (f8: its 16 x 16 form, see gemm_i4g_h_f8); I % 16 == 0,
// I <= 16384, x and xh 16-byte aligned
int launch_qrow_f16p(const float* x, uint16_t* xh, float* sx, int S, int I, int f8, hipStream_t st);
// per-row int4 weights (WF_I4, nn/quant.c:34-55) and their expansion to
// int8 codes n - 8 (I % 16 == 0; n = O * I codes)
int launch_pack_i4row(const float* w, uint8_t* q4, float* scale, int O, int I, hipStream_t st);
int launch_i4row_idot(const int8_t* xq, const float* sx, const uint8_t* q4, const float* scale, float* y, int S,
                      int I, int O, hipStream_t st);
// the exact f32 path of moty_matmul_i4_s (I % 16 == 0)
int launch_i4row_f32(const float* x, const uint8_t* q4, const float* scale, float* y, int S, int I, int O,
                     hipStream_t st);
int launch_quantize_rows(const float* w, int8_t* q, float* scale, int O, int I, int bits, hipStream_t st);
int launch_pack_i4g(const float* w, uint8_t* q4, float* scale, int O, int I, int gs, hipStream_t st);

int launch_gemv_q8(const float* x, const int8_t* W, const float* scale, const int8_t* W2, const float* scale2,
                   float* y, int S, int I, int O, hipStream_t st);
// the S = 1 Q8 FFN in one launch of 256 co-resident workgroups (one per CU;
// nwg must be 256); xh holds 9 * 4096 words and epoch nwg counters, both
// zeroed once and owned by this launcher from then on
int ffn1h_q8_fits(int D, int I, int nwg);
int launch_ffn1h_q8(const float* x, const int8_t* G, const float* gs, const int8_t* U, const float* us,
                    const int8_t* Dn, const float* ds, float* y, int D, int I, int nwg, unsigned long long* xh,
                    unsigned* epoch, unsigned* err, hipStream_t st);
int launch_gemm_q8(const int8_t* xq, const float* sx, const int8_t* W, const float* scale, float* y, int M, int K,
                   int O, hipStream_t st);

// q4b/sclb non-null: PAIR mode (S = 1), y = silu(x.q4^T) * (x.q4b^T)
int launch_gemv_i4g(const float* x, const uint8_t* q4, const float* scl, const uint8_t* q4b, const float* sclb,
                    float* y, int S, int I, int O, hipStream_t st);
// the exact-f32 path (IDOT4 unset), many tokens (tiled); q4b/sclb non-null: PAIR
int launch_gemm_i4g_xf(const float* x, const uint8_t* q4, const float* scl, const uint8_t* q4b, const float* sclb,
                       float* y, int M, int I, int O, hipStream_t st);
// the exact-f32 path (IDOT4 unset), one token; q4b/sclb non-null: PAIR
// Exact-f32 grouped int4, S tokens through an O x I matrix: the one-token
// GEMV once per token, or the 64-token tiled GEMM?  The tiled GEMM's time
// follows its K loop, not the token or row count (about 66 ns per element
// of I: 69 us at I = 1024, 270-280 us at 4096 for 256 to 12288 rows); the
// GEMV's is about 4 us plus the matrix bytes at 5 TB/s per token (measured
// on MI355X: 4.2 us at 1024 x 1024, 10.3 at 12288 x 4096).
inline bool xf_gemv_per_token(int S, int I, int O) {
  const double gemv_us = 4.0 + ((double)O * I * 0.625) / 5.0e6, gemm_us = 0.066 * I;
  return S <= 64 && S * gemv_us < gemm_us;
}
int launch_gemv_i4g_xf(const float* x, const uint8_t* q4, const float* scl, const uint8_t* q4b, const float* sclb,
                       float* y, int I, int O, hipStream_t st);
int launch_gemm_i4g(const int8_t* xq, const float* sx, const uint8_t* q4, const float* scl, float* y, int M, int I,
                    int O, hipStream_t st);
// the same GEMM on f16 MFMA over activations from launch_qrow_f16p;
// q4b/sclb non-null: PAIR, y = silu(x.q4^T) * (x.q4b^T).  MOTY_EUNSUP when
// I % 128 != 0 or a pointer is not 16-byte aligned
bool gemm_i4g_h_fits(int M, int I, int O);
int launch_gemm_i4g_h(const uint16_t* xh, const float* sx, const uint8_t* q4, const float* scl, const uint8_t* q4b,
                      const float* sclb, float* y, int M, int I, int O, hipStream_t st);
// 1 when launch_gemm_i4g_h runs its 16 x 16 form at this shape: its
// activations then come from launch_qrow_f16p with f8 = 1
int gemm_i4g_h_f8(int M, int O, bool pair);
int launch_i4g_f32(const float* x, const uint8_t* q4, const float* scl, float* y, int S, int I, int O,
                   hipStream_t st);

// Q4R4 / Q8R4 (f16 group scales, 4-row blocks): group-32 activation
// quantization, the matmul (xq/xs/xm: activation scratch of S*I bytes and
// S*(I/32) floats and ints, used when S > 4) and the packers
int launch_quant_g32(const float* x, int8_t* xq, float* xs, int32_t* xm, int S, int I, hipStream_t st);
int launch_r4_matmul(bool q8, const float* x, const uint8_t* W, const uint16_t* d16, float* y, int S, int I, int O,
                     int8_t* xq, float* xs, int32_t* xm, hipStream_t st);
// the same for S > 3 (GEMM, xq/xs/xm: activation scratch for S*D codes)
int launch_r4_gate_up_gemm(bool q8, const float* x, const uint8_t* W, const uint16_t* d16, float* h, int S, int D,
                           int I, int8_t* xq, float* xs, int32_t* xm, hipStream_t st);
int launch_r4_gate_up_silu(bool q8, const float* x, const uint8_t* W, const uint16_t* d16, float* h, int D, int I,
                           hipStream_t st);
int launch_pack_r4(bool q8, const float* w, uint8_t* q, uint16_t* d16, int O, int I, hipStream_t st);

// GGUF block formats (type ids of io/st.h:74): block dequantization to f32
// and the lossless Q4_0 -> grouped-int4 (gs = 32) repack
enum { GG_Q8_0 = 4, GG_Q4_0 = 5, GG_Q4_K = 6, GG_Q5_K = 7, GG_Q6_K = 8 };
int gguf_block(int dtype, int* elems, int* bytes);
int launch_gguf_dequant(int dtype, const void* raw, float* out, int64_t numel, hipStream_t st);
int launch_gguf_repack_q4_0(const void* raw, uint8_t* q4, float* qs, int64_t nblk, hipStream_t st);

int launch_matmul_f32(const float* x, const float* W, float* y, int S, int I, int O, hipStream_t st);
int launch_silu_mul(float* g, const float* u, int64_t n, hipStream_t st);
int launch_silu_rows(float* h, const float* gu, int S, int I, hipStream_t st);
int launch_expf(const float* x, float* y, int64_t n, hipStream_t st);
int launch_softmax_rows(float* x, int S, int n, hipStream_t st);

struct MoeArgs {
  const float* x;
  const float* Wr;
  const float* bias;
  const int8_t *G, *U, *Dn;
  const float *GS, *US, *DS;
  float* out;
  int T, D, E, K, I;
  int norm, order;
  int* idx_out;
  float* w_out;
  int* counts_out;
  float* probs_out;
};
size_t moe_scratch_size(int T, int D, int E, int K, int I, size_t* offsets);
// T = 1 with K <= 8 and D, I <= 4096 takes the decode path (routing, then a
// gate/up GEMV over the routed experts and a down GEMV that combines)
int launch_moe(const MoeArgs& a, void* scratch, hipStream_t st);
// The layer in three phases, for callers that act between them (the expert
// cache): router + top-k + grouping; the expert GEMMs (eslot: expert ->
// weight slot in a.G/U/Dn and their scales, -1 = skip; null = identity);
// the combine.  moe_routing gives the device idx [T*K] and counts [E].
int launch_moe_route(const MoeArgs& a, void* scratch, hipStream_t st, bool group = true);
int launch_moe_experts(const MoeArgs& a, void* scratch, const int* eslot, hipStream_t st);
int launch_moe_combine(const MoeArgs& a, void* scratch, hipStream_t st);
void moe_routing(const MoeArgs& a, void* scratch, const int** idx, const int** counts);

}  // namespace moty
