// api.cpp -- the C ABI of libmoty-hw-hip (include/moty_hw_hip.h).
//
// Owns, per device: one HIP stream for the synchronous host-pointer calls,
// a growable scratch arena (activation quantization, MoE intermediates),
// a transfer arena for host x/y, and the weight cache keyed by host pointer.
// Device entry points only validate, carve scratch and queue kernels.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <unordered_map>

#include "../../include/moty_hw_hip.h"
#include "common.h"
#include "dev.h"
#include "kernels.h"

namespace moty {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

int check_hip(hipError_t e, const char* what) {
  set_error("%s: %s", what, hipGetErrorString(e));
  return e == hipErrorOutOfMemory ? MOTY_ENOMEM : MOTY_EHIP;
}

constexpr int MAX_DEV = 16;
static Dev g_dev[MAX_DEV];

// Fixed scratch of the no-allocation entry point: a file-scope device array,
// one copy per GPU the library runs on, held until the process ends.  Host
// code never uses its name as an address (that is a host-side stand-in);
// each device's address comes from hipGetSymbolAddress at set-up.
constexpr size_t FIXED_SCRATCH_BYTES = (size_t)64 << 20;
static __device__ __align__(256) char scratch[FIXED_SCRATCH_BYTES];
static std::mutex g_mu;  // guards g_dev[*] set-up and the weight caches
static thread_local int t_dev = -1;

static int dev_init(int d) {
  int n = 0;
  HIP_TRY(hipGetDeviceCount(&n));
  if (d < 0 || d >= n || d >= MAX_DEV) {
    set_error("moty_hip_init: device %d not present (%d visible)", d, n);
    return MOTY_EINVAL;
  }
  HIP_TRY(hipSetDevice(d));
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_dev[d].ready) {
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, d));
    g_dev[d].cus = prop.multiProcessorCount;
    void* fp = nullptr;
    HIP_TRY(hipGetSymbolAddress(&fp, HIP_SYMBOL(scratch)));
    g_dev[d].fixed_scratch = fp;
    HIP_TRY(hipEventCreateWithFlags(&g_dev[d].fx_ev, hipEventDisableTiming));
    {
      // the one-launch FFN's exchange words (9 copies of I <= 4096 words),
      // per-workgroup call counters and wait-error flag, zeroed once
      const size_t xb = (9 * 4096) * 8, eb = al256((size_t)g_dev[d].cus * 4);
      void* p = nullptr;
      HIP_TRY(hipMalloc(&p, xb + eb + 256));
      HIP_TRY(hipMemset(p, 0, xb + eb + 256));
      HIP_TRY(hipDeviceSynchronize());
      g_dev[d].f1_xh = (unsigned long long*)p;
      g_dev[d].f1_epoch = (unsigned*)((char*)p + xb);
      g_dev[d].f1_err = (unsigned*)((char*)p + xb + eb);
      const char* e = getenv("MOTY_FFN1");
      g_dev[d].f1_on = e && e[0] == '1';
    }
    HIP_TRY(hipStreamCreateWithFlags(&g_dev[d].stream, hipStreamNonBlocking));
    g_dev[d].ready = true;
  }
  t_dev = d;
  return MOTY_OK;
}

int cur(Dev** out) {
  g_err[0] = 0;  // an entry point that succeeds leaves no stale message
  if (t_dev < 0) {
    int rc = dev_init(0);
    if (rc) return rc;
  } else {
    HIP_TRY(hipSetDevice(t_dev));
  }
  *out = &g_dev[t_dev];
  return MOTY_OK;
}

// Grow an arena to at least `bytes`.  Waits for queued work that may still
// read the old buffer before releasing it.
int arena_get(Arena& a, size_t bytes, void** p) {
  if (bytes == 0) bytes = 256;
  if (a.cap < bytes) {
    if (a.p) {
      HIP_TRY(hipDeviceSynchronize());
      HIP_TRY(hipFree(a.p));
      a.p = nullptr;
      a.cap = 0;
    }
    size_t nb = bytes + bytes / 4;
    nb = (nb + (1 << 20) - 1) & ~(size_t)((1 << 20) - 1);
    hipError_t e = hipMalloc(&a.p, nb);
    if (e != hipSuccess) {
      a.p = nullptr;
      return check_hip(e, "scratch hipMalloc");
    }
    a.cap = nb;
  }
  *p = a.p;
  return MOTY_OK;
}

static bool capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

int scratch_get(Dev* d, size_t bytes, hipStream_t st, void** p) {
  if (d->scr_used && d->scr_stream != st && d->scr_ev_ok && !capturing(st))
    HIP_TRY(hipStreamWaitEvent(st, d->scr_ev, 0));
  int rc = arena_get(d->scratch, bytes, p);
  if (rc) return rc;
  d->scr_stream = st;
  d->scr_used = true;
  d->scr_pend = true;
  return MOTY_OK;
}

void scratch_mark(Dev* d) {
  d->scr_pend = false;
  d->scr_ev_ok = false;
  if (capturing(d->scr_stream)) return;
  if (!d->scr_ev && hipEventCreateWithFlags(&d->scr_ev, hipEventDisableTiming) != hipSuccess) {
    d->scr_ev = nullptr;
    return;
  }
  // a failed record leaves scr_ev_ok false: the next call on another stream
  // then runs unordered, so synchronise here instead
  if (hipEventRecord(d->scr_ev, d->scr_stream) == hipSuccess)
    d->scr_ev_ok = true;
  else
    (void)hipDeviceSynchronize();
}

// Fingerprint of a host buffer from 64 evenly spaced 16-byte samples (the
// first and last bytes included): FNV-1a over the sampled bytes.  A few
// hundred nanoseconds per call, independent of the buffer's size.
static uint64_t host_fp(const void* host, size_t bytes) {
  const uint8_t* p = (const uint8_t*)host;
  uint64_t h = 1469598103934665603ull ^ bytes;
  constexpr int NS = 64, SB = 16;
  if (bytes <= (size_t)NS * SB) {
    for (size_t i = 0; i < bytes; i++) h = (h ^ p[i]) * 1099511628211ull;
    return h;
  }
  const size_t span = bytes - SB;
  for (int k = 0; k < NS; k++) {
    const uint8_t* q = p + span * k / (NS - 1);
    for (int i = 0; i < SB; i++) h = (h ^ q[i]) * 1099511628211ull;
  }
  return h;
}

// Device copy of a persistent host weight buffer, keyed by its address.  A
// hit also needs the same sampled fingerprint: a different buffer that got
// the address of a freed one is uploaded afresh.  An in-place rewrite that
// leaves every sampled byte alone is not detected (moty_hip_weight_forget
// is the caller's way to announce one).
static int weight(Dev* d, const void* host, size_t bytes, const void** dev) {
  std::lock_guard<std::mutex> lk(g_mu);
  const uint64_t fp = host_fp(host, bytes);
  auto it = d->wcache.find(host);
  if (it != d->wcache.end() && it->second.bytes == bytes && it->second.fp == fp) {
    *dev = it->second.dev;
    return MOTY_OK;
  }
  if (it != d->wcache.end()) {
    HIP_TRY(hipStreamSynchronize(d->stream));
    HIP_TRY(hipFree(it->second.dev));
    d->wcache.erase(it);
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
  if (e != hipSuccess) return check_hip(e, "weight hipMalloc");
  // on the library's stream, ahead of every kernel that reads the copy: a
  // plain hipMemcpy from pageable memory may return before its DMA lands,
  // and the library's (non-blocking) stream does not wait for the null stream
  e = hipMemcpyAsync(p, host, bytes, hipMemcpyHostToDevice, d->stream);
  if (e != hipSuccess) {
    hipFree(p);
    return check_hip(e, "weight upload");
  }
  d->wcache[host] = WEntry{p, bytes, fp};
  *dev = p;
  return MOTY_OK;
}

static int env_int(const char* name, int dflt) {
  const char* e = getenv(name);
  return e ? atoi(e) : dflt;
}

// Stage host x into the transfer arena; returns device x and y pointers.
int stage_io(Dev* d, const void* x, size_t xbytes, size_t ybytes, void** dx, void** dy) {
  void* p;
  int rc = arena_get(d->io, al256(xbytes) + al256(ybytes), &p);
  if (rc) return rc;
  *dx = p;
  *dy = (char*)p + al256(xbytes);
  HIP_TRY(hipMemcpyAsync(*dx, x, xbytes, hipMemcpyHostToDevice, d->stream));
  return MOTY_OK;
}

int finish_io(Dev* d, void* y, const void* dy, size_t ybytes) {
  HIP_TRY(hipMemcpyAsync(y, dy, ybytes, hipMemcpyDeviceToHost, d->stream));
  HIP_TRY(hipStreamSynchronize(d->stream));
  return MOTY_OK;
}

}  // namespace moty

using namespace moty;


extern "C" {

int moty_hip_init(int device) { return dev_init(device); }

int moty_hip_shutdown(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (int i = 0; i < MAX_DEV; i++) {
    Dev& d = g_dev[i];
    if (!d.ready) continue;
    HIP_TRY(hipSetDevice(i));
    HIP_TRY(hipDeviceSynchronize());
    for (auto& kv : d.wcache) hipFree(kv.second.dev);
    d.wcache.clear();
    if (d.scratch.p) hipFree(d.scratch.p);
    if (d.io.p) hipFree(d.io.p);
    d.scratch = Arena();
    d.io = Arena();
    hipStreamDestroy(d.stream);
    d.stream = nullptr;
    if (d.scr_ev) hipEventDestroy(d.scr_ev);
    d.scr_ev = nullptr;
    d.scr_used = d.scr_pend = d.scr_ev_ok = false;
    if (d.fx_ev) hipEventDestroy(d.fx_ev);
    d.fx_ev = nullptr;
    d.fx_used = d.fx_ev_ok = false;
    d.fx_stream = nullptr;
    d.scr_stream = nullptr;
    if (d.f1_xh) hipFree(d.f1_xh);  // one block: exchange words, counters, flag
    d.f1_xh = nullptr;
    d.f1_epoch = d.f1_err = nullptr;
    d.ready = false;
  }
  t_dev = -1;
  return MOTY_OK;
}

const char* moty_hip_last_error(void) { return g_err; }
const char* moty_hip_kernel_tier(void) { return "gfx950-mfma-i8/gfx950-f32"; }

int moty_hip_wait_errors(int* count) {
  CUR(d);
  if (!count) return set_error("wait_errors: count is NULL"), MOTY_EINVAL;
  unsigned v = 0;
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMemcpy(&v, d->f1_err, 4, hipMemcpyDeviceToHost));
  if (v) HIP_TRY(hipMemset(d->f1_err, 0, 4));
  HIP_TRY(hipDeviceSynchronize());
  *count = (int)v;
  return MOTY_OK;
}

int moty_hip_set_ffn1(int on) {
  CUR(d);
  d->f1_on = on != 0;
  return MOTY_OK;
}

// ---------------- device-pointer entry points ----------------

// the kernels move activations and weight rows in 16-byte units: pointers
// that are not 16-byte aligned are refused rather than read out of line
static int need_al16(const char* what, const void* a, const void* b, const void* c = nullptr,
                     const void* e = nullptr) {
  if ((((uintptr_t)a) | ((uintptr_t)b) | ((uintptr_t)c) | ((uintptr_t)e)) & 15) {
    set_error("%s: activations and weights must be 16-byte aligned", what);
    return MOTY_EUNSUP;
  }
  return MOTY_OK;
}

int moty_hip_qrow_i8_multi_dev(int n, const float* const* x, int8_t* const* q, float* const* sx, const int* S,
                               const int* I, void* stream) {
  CUR(d);
  if (n < 1 || n > QROW_MAX_JOBS || !x || !q || !sx || !S || !I)
    return set_error("qrow_i8_multi: bad arguments (1 <= n <= %d)", QROW_MAX_JOBS), MOTY_EINVAL;
  QrowJobs jb = {};
  jb.n = n;
  for (int j = 0; j < n; j++) {
    if (S[j] < 0 || I[j] <= 0 || (S[j] > 0 && (!x[j] || !q[j] || !sx[j])))
      return set_error("qrow_i8_multi: bad job %d", j), MOTY_EINVAL;
    jb.x[j] = x[j];
    jb.q[j] = q[j];
    jb.sx[j] = sx[j];
    jb.S[j] = S[j];
    jb.I[j] = I[j];
  }
  const int rc = launch_qrow_multi(jb, STREAM(stream));
  if (rc == MOTY_EUNSUP)
    set_error("qrow_i8_multi: every job needs I <= 4096, I %% 16 == 0 and 16-byte aligned x and q");
  return rc;
}

int moty_hip_qrow_i8_dev(const float* x, int8_t* q, float* sx, int32_t* xg, int S, int I, void* stream) {
  CUR(d);
  if (S < 0 || I <= 0 || !x || !q || !sx) return set_error("qrow_i8: bad arguments"), MOTY_EINVAL;
  return launch_qrow_i8(x, q, sx, xg, S, I, I, I, STREAM(stream));
}

int moty_hip_quantize_rows_dev(const float* w, int8_t* q, float* scale, int O, int I, int bits, void* stream) {
  CUR(d);
  if (O < 0 || I <= 0 || bits < 2 || bits > 8 || !w || !q || !scale)
    return set_error("quantize_rows: bad arguments"), MOTY_EINVAL;
  return launch_quantize_rows(w, q, scale, O, I, bits, STREAM(stream));
}

int moty_hip_pack_int4_grouped_dev(const float* w, uint8_t* q4, float* scale, int O, int I, int gs,
                                   void* stream) {
  CUR(d);
  if (gs <= 0 || gs % 16) return set_error("pack_int4_grouped: gs=%d not a multiple of 16", gs), MOTY_EINVAL;
  if (O < 0 || I <= 0 || !w || !q4 || !scale) return set_error("pack_int4_grouped: bad arguments"), MOTY_EINVAL;
  return launch_pack_i4g(w, q4, scale, O, I, gs, STREAM(stream));
}

int moty_hip_matmul_q8_preq_dev(float* y, const int8_t* xq, const float* sx, const int8_t* q, const float* scale,
                                int S, int I, int O, void* stream) {
  CUR(d);
  if (S < 0 || I <= 0 || O < 0) return set_error("matmul_q8_preq: bad shape"), MOTY_EINVAL;
  if (S > 0 && O > 0 && need_al16("matmul_q8_preq", xq, q)) return MOTY_EUNSUP;
  int rc = launch_gemm_q8(xq, sx, q, scale, y, S, I, O, STREAM(stream));
  if (rc == MOTY_EUNSUP) set_error("matmul_q8_preq: I=%d must be a multiple of 16", I);
  return rc;
}

int moty_hip_matmul_q_s_dev(float* y, const float* x, const int8_t* q, const float* scale, int S, int I, int O,
                            void* stream) {
  CUR(d);
  if (S < 0 || I <= 0 || O < 0 || !y || !x || !q || !scale) return set_error("matmul_q_s: bad arguments"), MOTY_EINVAL;
  if (S == 0 || O == 0) return MOTY_OK;
  if (need_al16("matmul_q_s", x, q)) return MOTY_EUNSUP;
  if (I > 16384 || (I % 16)) {
    set_error("matmul_q_s: I=%d unsupported (needs I %% 16 == 0, I <= 16384)", I);
    return MOTY_EUNSUP;
  }
  hipStream_t st = STREAM(stream);
  if (S <= GEMV_MAX_S) return launch_gemv_q8(x, q, scale, nullptr, nullptr, y, S, I, O, st);
  void* sp;
  const size_t xb = al256((size_t)S * I);
  int rc = scratch_get(d, xb + al256((size_t)S * 4), st, &sp);
  if (rc) return rc;
  int8_t* xq = (int8_t*)sp;
  float* sx = (float*)((char*)sp + xb);
  rc = launch_qrow_i8(x, xq, sx, nullptr, S, I, I, I, st);
  if (rc) return rc;
  return launch_gemm_q8(xq, sx, q, scale, y, S, I, O, st);
}

int moty_hip_matmul_i4_grouped_s_dev(float* y, const float* x, const uint8_t* q4, const float* scale, int S,
                                     int I, int O, int gs, int idot4, void* stream) {
  CUR(d);
  if (S < 0 || I <= 0 || O < 0 || gs <= 0 || !y || !x || !q4 || !scale)
    return set_error("matmul_i4_grouped_s: bad arguments"), MOTY_EINVAL;
  if (S == 0 || O == 0) return MOTY_OK;
  hipStream_t st = STREAM(stream);
  if (idot4 && gs == 32 && (I % 64) == 0 && I <= 16384) {
    if (need_al16("matmul_i4_grouped_s", x, q4)) return MOTY_EUNSUP;
    if (S <= 4) return launch_gemv_i4g(x, q4, scale, nullptr, nullptr, y, S, I, O, st);
    void* sp;
    if (gemm_i4g_h_fits(S, I, O) && !(((uintptr_t)x | (uintptr_t)q4 | (uintptr_t)scale) & 15)) {
      // f16 codes + f16 MFMA: one FMA per output and group in the epilogue
      const size_t hb = al256((size_t)S * I * 2);
      int rc = scratch_get(d, hb + al256((size_t)S * 4), st, &sp);
      if (rc) return rc;
      uint16_t* xh = (uint16_t*)sp;
      float* sx = (float*)((char*)sp + hb);
      if ((rc = launch_qrow_f16p(x, xh, sx, S, I, gemm_i4g_h_f8(S, O, false), st))) return rc;
      return launch_gemm_i4g_h(xh, sx, q4, scale, nullptr, nullptr, y, S, I, O, st);
    }
    const size_t xb = al256((size_t)S * I);
    int rc = scratch_get(d, xb + al256((size_t)S * 4), st, &sp);
    if (rc) return rc;
    int8_t* xq = (int8_t*)sp;
    float* sx = (float*)((char*)sp + xb);
    rc = launch_qrow_i8(x, xq, sx, nullptr, S, I, I, I, st);
    if (rc) return rc;
    return launch_gemm_i4g(xq, sx, q4, scale, y, S, I, O, st);
  }
  const bool per_token = S <= 4 || xf_gemv_per_token(S, I, O);
  if (gs == 32 && per_token) {
    // a few tokens: the one-token GEMV per token
    int rc = MOTY_OK;
    for (int s = 0; s < S && rc == MOTY_OK; s++)
      rc = launch_gemv_i4g_xf(x + (int64_t)s * I, q4, scale, nullptr, nullptr, y + (int64_t)s * O, I, O, st);
    if (rc != MOTY_EUNSUP) return rc;
  }
  if (gs == 32 && S > 4) {
    const int rc = launch_gemm_i4g_xf(x, q4, scale, nullptr, nullptr, y, S, I, O, st);
    if (rc != MOTY_EUNSUP) return rc;
  }
  if (gs == 32 && (I % 32) == 0) return launch_i4g_f32(x, q4, scale, y, S, I, O, st);
  set_error("matmul_i4_grouped_s: gs=%d I=%d unsupported (exact path needs gs == 32, I %% 32 == 0)", gs, I);
  return MOTY_EUNSUP;
}

int moty_hip_pack_int4_dev(const float* w, uint8_t* q4, float* scale, int O, int I, void* stream) {
  CUR(d);
  if (O < 0 || I <= 0 || !w || !q4 || !scale) return set_error("pack_int4: bad arguments"), MOTY_EINVAL;
  return launch_pack_i4row(w, q4, scale, O, I, STREAM(stream));
}

// moty_matmul_i4_s (nn/matmul.c:75-145), per-row int4 weights.  IDOT4:
// x is quantized per row (qrow_i8) into scratch and k_i4row_idot runs the
// integer dot straight from the nibbles with the (scale*sx)*acc epilogue;
// otherwise the exact f32 path.  I % 16 == 0 (the AVX2 step of the f32 path;
// other widths stay on the CPU); q4 8-byte and x 16-byte aligned.
int moty_hip_matmul_i4_s_dev(float* y, const float* x, const uint8_t* q4, const float* scale, int S, int I, int O,
                             int idot4, void* stream) {
  CUR(d);
  if (S < 0 || I <= 0 || O < 0 || !y || !x || !q4 || !scale) return set_error("matmul_i4_s: bad arguments"), MOTY_EINVAL;
  if (S == 0 || O == 0) return MOTY_OK;
  if (I % 16) return set_error("matmul_i4_s: I=%d unsupported (I %% 16 == 0)", I), MOTY_EUNSUP;
  if ((((uintptr_t)q4) & 7) || (((uintptr_t)x) & 15))
    return set_error("matmul_i4_s: q4 must be 8-byte and x 16-byte aligned"), MOTY_EUNSUP;
  hipStream_t st = STREAM(stream);
  if (!idot4 || I > 16384) return launch_i4row_f32(x, q4, scale, y, S, I, O, st);
  const size_t bx = al256((size_t)S * I);
  void* sp;
  int rc = scratch_get(d, bx + al256((size_t)S * 4), st, &sp);
  if (rc) return rc;
  int8_t* xq = (int8_t*)sp;
  float* sx = (float*)((char*)sp + bx);
  if ((rc = launch_qrow_i8(x, xq, sx, nullptr, S, I, I, I, st))) return rc;
  return launch_i4row_idot(xq, sx, q4, scale, y, S, I, O, st);
}

int moty_hip_matmul_dev(float* y, const float* x, const float* W, int S, int I, int O, void* stream) {
  CUR(d);
  if (S < 0 || I <= 0 || O < 0 || !y || !x || !W) return set_error("matmul: bad arguments"), MOTY_EINVAL;
  return launch_matmul_f32(x, W, y, S, I, O, STREAM(stream));
}

int moty_hip_silu_mul_dev(float* g, const float* u, int64_t n, void* stream) {
  CUR(d);
  if (n < 0 || !g || !u) return set_error("silu_mul: bad arguments"), MOTY_EINVAL;
  return launch_silu_mul(g, u, n, STREAM(stream));
}

int moty_hip_softmax_rows_dev(float* x, int S, int n, void* stream) {
  CUR(d);
  if (S < 0 || n <= 0 || !x) return set_error("softmax_rows: bad arguments"), MOTY_EINVAL;
  return launch_softmax_rows(x, S, n, STREAM(stream));
}

int moty_hip_expf_dev(const float* x, float* y, int64_t n, void* stream) {
  CUR(d);
  if (n < 0 || !x || !y) return set_error("expf: bad arguments"), MOTY_EINVAL;
  return launch_expf(x, y, n, STREAM(stream));
}

int moty_hip_gate_up_silu_q8_dev(float* h, const float* x, int S, const int8_t* gate, const float* gs,
                                 const int8_t* up, const float* us, int D, int I, void* stream) {
  CUR(d);
  if (S < 0 || D <= 0 || I <= 0 || !h || !x || !gate || !gs || !up || !us)
    return set_error("gate_up_silu_q8: bad arguments"), MOTY_EINVAL;
  if (S == 0) return MOTY_OK;
  if (S > GEMV_MAX_S || (D % 16) || D > 16384) {
    set_error("gate_up_silu_q8: S=%d D=%d unsupported (S <= %d, D %% 16 == 0)", S, D, GEMV_MAX_S);
    return MOTY_EUNSUP;
  }
  if (need_al16("gate_up_silu_q8", x, gate, up)) return MOTY_EUNSUP;
  return launch_gemv_q8(x, gate, gs, up, us, h, S, D, I, STREAM(stream));
}

int moty_hip_gate_up_silu_i4g_dev(float* h, const float* x, const uint8_t* gate, const float* gs,
                                  const uint8_t* up, const float* us, int D, int I, void* stream) {
  CUR(d);
  if (D <= 0 || I <= 0 || !h || !x || !gate || !gs || !up || !us)
    return set_error("gate_up_silu_i4g: bad arguments"), MOTY_EINVAL;
  if (need_al16("gate_up_silu_i4g", x, gate, up)) return MOTY_EUNSUP;
  int rc = launch_gemv_i4g(x, gate, gs, up, us, h, 1, D, I, STREAM(stream));
  if (rc == MOTY_EUNSUP) set_error("gate_up_silu_i4g: D=%d unsupported (D %% 64 == 0, D <= 16384)", D);
  return rc;
}

int moty_hip_dense_ffn_q8_dev(float* out, const float* x, int S, const int8_t* gate, const float* gs,
                              const int8_t* up, const float* us, const int8_t* down, const float* ds, int D, int I,
                              void* stream) {
  CUR(d);
  if (S < 0 || D <= 0 || I <= 0) return set_error("dense_ffn_q8: bad shape"), MOTY_EINVAL;
  if (S == 0) return MOTY_OK;
  if (need_al16("dense_ffn_q8", x, gate, up, down)) return MOTY_EUNSUP;
  if ((D % 16) || (I % 16) || D > 16384 || I > 16384) {
    set_error("dense_ffn_q8: D=%d I=%d unsupported", D, I);
    return MOTY_EUNSUP;
  }
  hipStream_t st = STREAM(stream);
  void* sp;
  if (S == 1 && d->f1_on && ffn1h_q8_fits(D, I, d->cus)) {
    // the exchange words and call counters are per-device state shared by
    // every call: the scratch ordering keeps calls on two streams apart
    int rc = scratch_get(d, 256, st, &sp);
    if (rc) return rc;
    return launch_ffn1h_q8(x, gate, gs, up, us, down, ds, out, D, I, d->cus, d->f1_xh, d->f1_epoch, d->f1_err, st);
  }
  if (S <= GEMV_MAX_S) {
    int rc = scratch_get(d, al256((size_t)S * I * 4), st, &sp);
    if (rc) return rc;
    float* h = (float*)sp;
    rc = launch_gemv_q8(x, gate, gs, up, us, h, S, D, I, st);
    if (rc) return rc;
    return launch_gemv_q8(h, down, ds, nullptr, nullptr, out, S, I, D, st);
  }
  const size_t b_xq = al256((size_t)S * (D > I ? D : I)), b_sx = al256((size_t)S * 4);
  const size_t b_g = al256((size_t)S * I * 4);
  int rc = scratch_get(d, b_xq + b_sx + 2 * b_g, st, &sp);
  if (rc) return rc;
  int8_t* xq = (int8_t*)sp;
  float* sx = (float*)((char*)sp + b_xq);
  float* g = (float*)((char*)sp + b_xq + b_sx);
  float* u = (float*)((char*)sp + b_xq + b_sx + b_g);
  if ((rc = launch_qrow_i8(x, xq, sx, nullptr, S, D, D, D, st))) return rc;
  if ((rc = launch_gemm_q8(xq, sx, gate, gs, g, S, D, I, st))) return rc;
  if ((rc = launch_gemm_q8(xq, sx, up, us, u, S, D, I, st))) return rc;
  if ((rc = launch_silu_mul(g, u, (int64_t)S * I, st))) return rc;
  if ((rc = launch_qrow_i8(g, xq, sx, nullptr, S, I, I, I, st))) return rc;
  return launch_gemm_q8(xq, sx, down, ds, out, S, I, D, st);
}

static int moe_check(const MotyHipMoe* m, const float* x, float* out, int S, const char* what) {
  if (!m || !x || !out || S < 0) return set_error("%s: bad arguments", what), MOTY_EINVAL;
  if (m->E <= 0 || m->K <= 0 || m->K > m->E || m->K > 64 || m->I <= 0 || m->D <= 0)
    return set_error("%s: bad shape E=%d K=%d I=%d D=%d", what, m->E, m->K, m->I, m->D), MOTY_EINVAL;
  if (S > 0 && ((m->D % 32) || (m->I % 32) || m->E > 256)) {
    set_error("%s: D=%d I=%d E=%d unsupported (D, I multiples of 32, E <= 256)", what, m->D, m->I, m->E);
    return MOTY_EUNSUP;
  }
  // the kernels move x, out, the router and the expert rows in 16-byte units
  if (S > 0 && ((((uintptr_t)x) | ((uintptr_t)out) | ((uintptr_t)m->router) | ((uintptr_t)m->g) |
                 ((uintptr_t)m->u) | ((uintptr_t)m->d)) & 15)) {
    set_error("%s: x, out, router and the g/u/d expert tensors must be 16-byte aligned", what);
    return MOTY_EUNSUP;
  }
  return MOTY_OK;
}

static MoeArgs moe_args(const MotyHipMoe* m, const float* x, int S, float* out) {
  MoeArgs a;
  a.x = x;
  a.Wr = m->router;
  a.bias = m->logit_bias;
  a.G = m->g;
  a.U = m->u;
  a.Dn = m->d;
  a.GS = m->gs;
  a.US = m->us;
  a.DS = m->ds;
  a.out = out;
  a.T = S;
  a.D = m->D;
  a.E = m->E;
  a.K = m->K;
  a.I = m->I;
  a.norm = m->norm_topk;
  a.order = m->combine_order;
  a.idx_out = m->idx_out;
  a.w_out = m->w_out;
  a.counts_out = m->counts_out;
  a.probs_out = nullptr;
  return a;
}

// moty_nn_dense_ffn (nn/ffn.c:26-55) over grouped-int4 gate/up/down Mats
// (WF_I4G, gs = 32): gate and up in one pass with the SiLU epilogue, then
// down.  idot4 selects the int8-activation path (nn/matmul.c:171), else the
// exact f32 path.
int moty_hip_dense_ffn_i4g_dev(float* out, const float* x, int S, const uint8_t* gate, const float* gs,
                               const uint8_t* up, const float* us, const uint8_t* down, const float* ds, int D,
                               int I, int idot4, void* stream) {
  CUR(d);
  if (S < 0 || D <= 0 || I <= 0 || !out || !x || !gate || !gs || !up || !us || !down || !ds)
    return set_error("dense_ffn_i4g: bad arguments"), MOTY_EINVAL;
  if (S == 0) return MOTY_OK;
  if ((D % 32) || (I % 32)) return set_error("dense_ffn_i4g: D=%d I=%d must be multiples of 32", D, I), MOTY_EUNSUP;
  // the exact-f32 path falls back to byte-granular kernels; IDOT4 needs alignment
  if (idot4 && need_al16("dense_ffn_i4g", x, gate, up, down)) return MOTY_EUNSUP;
  hipStream_t st = STREAM(stream);
  const bool vec = idot4 && (D % 64) == 0 && (I % 64) == 0 && D <= 16384 && I <= 16384;  // both matrices
  const bool h16 = vec && S > 4 && gemm_i4g_h_fits(S, D, I) && gemm_i4g_h_fits(S, I, D) &&
                   !(((uintptr_t)x | (uintptr_t)gate | (uintptr_t)gs | (uintptr_t)up | (uintptr_t)us |
                      (uintptr_t)down | (uintptr_t)ds) & 15);
  const int W = D > I ? D : I;
  // scratch: h [S][I] f32 | u [S][I] f32 (paths without the fused pass) |
  // activation codes [S][W] (f16 or int8) | row scales [S]
  const size_t bh = al256((size_t)S * I * 4), bq = al256((size_t)S * W * 2), bs = al256((size_t)S * 4);
  void* sp;
  int rc = scratch_get(d, 2 * bh + bq + bs, st, &sp);
  if (rc) return rc;
  float* h = (float*)sp;
  float* u = (float*)((char*)sp + bh);
  void* xq = (char*)sp + 2 * bh;
  float* sx = (float*)((char*)sp + 2 * bh + bq);
  if (h16) {
    if ((rc = launch_qrow_f16p(x, (uint16_t*)xq, sx, S, D, gemm_i4g_h_f8(S, I, true), st))) return rc;
    if ((rc = launch_gemm_i4g_h((const uint16_t*)xq, sx, gate, gs, up, us, h, S, D, I, st))) return rc;
    if ((rc = launch_qrow_f16p(h, (uint16_t*)xq, sx, S, I, gemm_i4g_h_f8(S, D, false), st))) return rc;
    return launch_gemm_i4g_h((const uint16_t*)xq, sx, down, ds, nullptr, nullptr, out, S, I, D, st);
  }
  if (vec && S == 1) {
    if ((rc = launch_gemv_i4g(x, gate, gs, up, us, h, 1, D, I, st))) return rc;
    return launch_gemv_i4g(h, down, ds, nullptr, nullptr, out, 1, I, D, st);
  }
  const bool xf_tok = S <= 4 || (xf_gemv_per_token(S, D, 2 * I) && xf_gemv_per_token(S, I, D));
  if (!idot4 && xf_tok && D <= 16384 && I <= 16384 &&
      !(((uintptr_t)x | (uintptr_t)gate | (uintptr_t)up | (uintptr_t)down | (uintptr_t)h) & 15)) {
    // exact f32, per token: gate + up + SiLU in one pass, then down (the
    // shapes fit, so no launch is refused after the first)
    for (int s = 0; s < S; s++) {
      if ((rc = launch_gemv_i4g_xf(x + (int64_t)s * D, gate, gs, up, us, h + (int64_t)s * I, D, I, st))) return rc;
      if ((rc = launch_gemv_i4g_xf(h + (int64_t)s * I, down, ds, nullptr, nullptr, out + (int64_t)s * D, I, D, st)))
        return rc;
    }
    return MOTY_OK;
  }
  // one matmul_i4_grouped_s each, the path chosen per matrix as the
  // reference does (IDOT4 needs the row length a multiple of 64, <= 16384)
  auto mm = [&](const float* a, const uint8_t* w, const float* ws, float* o, int K, int N) -> int {
    if (idot4 && (K % 64) == 0 && K <= 16384) {
      if (S <= 4) return launch_gemv_i4g(a, w, ws, nullptr, nullptr, o, S, K, N, st);
      int r = launch_qrow_i8(a, (int8_t*)xq, sx, nullptr, S, K, K, K, st);
      return r ? r : launch_gemm_i4g((const int8_t*)xq, sx, w, ws, o, S, K, N, st);
    }
    const bool tok = S <= 4 || xf_gemv_per_token(S, K, N);
    if (!tok && launch_gemm_i4g_xf(a, w, ws, nullptr, nullptr, o, S, K, N, st) == MOTY_OK) return MOTY_OK;
    if (tok) {
      // exact f32, a few tokens: the one-token GEMV per token (it refuses
      // what it cannot take before launching anything)
      int r = MOTY_OK;
      for (int s = 0; s < S && r == MOTY_OK; s++)
        r = launch_gemv_i4g_xf(a + (int64_t)s * K, w, ws, nullptr, nullptr, o + (int64_t)s * N, K, N, st);
      if (r != MOTY_EUNSUP) return r;
    }
    return launch_i4g_f32(a, w, ws, o, S, K, N, st);
  };
  if (!idot4 && !xf_tok && S > 4 && (D % 64) == 0 && !(((uintptr_t)x) & 15) &&
      !(((uintptr_t)gate | (uintptr_t)up) & 7)) {
    // exact f32, many tokens: gate + up + SiLU in one tiled pass, then down
    if ((rc = launch_gemm_i4g_xf(x, gate, gs, up, us, h, S, D, I, st))) return rc;
    return mm(h, down, ds, out, I, D);
  }
  if ((rc = mm(x, gate, gs, h, D, I))) return rc;
  if ((rc = mm(x, up, us, u, D, I))) return rc;
  if ((rc = launch_silu_mul(h, u, (int64_t)S * I, st))) return rc;
  return mm(h, down, ds, out, I, D);
}

int moty_hip_moe_topk_dev(const MotyHipMoe* m, const float* x, int S, float* out, void* stream) {
  CUR(d);
  int rc = moe_check(m, x, out, S, "moe_topk");
  if (rc || S == 0) return rc;
  size_t offs[MOE_NBUF];
  const size_t need = moe_scratch_size(S, m->D, m->E, m->K, m->I, offs);
  void* sp;
  if ((rc = scratch_get(d, need, STREAM(stream), &sp))) return rc;
  rc = launch_moe(moe_args(m, x, S, out), sp, STREAM(stream));
  if (rc == MOTY_EUNSUP) set_error("moe_topk: unsupported shape");
  return rc;
}

// The MoE layer of moty_hip_moe_topk_dev on the fixed device scratch array:
// no allocation of any kind, for callers that cannot allocate.  The device
// must have been set up on this thread by moty_hip_init (which allocates);
// a call on another stream than the previous one first waits, on the device,
// for the previous call's work (an event recorded after each call), so
// sequential calls on different streams do not race.
int moty_hip_moe_topk_noalloc_dev(const MotyHipMoe* m, const float* x, int S, float* out, void* stream) {
  if (t_dev < 0 || !g_dev[t_dev].ready)
    return set_error("moe_topk_noalloc: call moty_hip_init on this thread first (it does the set-up that allocates)"),
           MOTY_EINVAL;
  CUR(d);
  int rc = moe_check(m, x, out, S, "moe_topk_noalloc");
  if (rc || S == 0) return rc;
  size_t offs[MOE_NBUF];
  const size_t need = moe_scratch_size(S, m->D, m->E, m->K, m->I, offs);
  if (need > FIXED_SCRATCH_BYTES) {
    set_error("moe_topk_noalloc: S=%d E=%d K=%d I=%d D=%d needs %zu bytes of scratch, above the fixed %zu", S,
              m->E, m->K, m->I, m->D, need, FIXED_SCRATCH_BYTES);
    return MOTY_EINVAL;
  }
  if (!d->fixed_scratch || !d->fx_ev)
    return set_error("moe_topk_noalloc: fixed scratch has no device address"), MOTY_EHIP;
  hipStream_t st = STREAM(stream);
  const bool cap = capturing(st);
  if (d->fx_used && d->fx_stream != st && d->fx_ev_ok && !cap) HIP_TRY(hipStreamWaitEvent(st, d->fx_ev, 0));
  rc = launch_moe(moe_args(m, x, S, out), d->fixed_scratch, st);
  if (rc == MOTY_EUNSUP) set_error("moe_topk_noalloc: unsupported shape");
  d->fx_used = true;
  d->fx_stream = st;
  d->fx_ev_ok = !cap && hipEventRecord(d->fx_ev, st) == hipSuccess;
  return rc;
}

// ---------------- host-pointer drop-ins ----------------


int moty_hip_matmul_q_s(float* y, const float* x, const int8_t* q, const float* scale, int S, int I, int O) {
  CUR(d);
  if (S < 0 || I <= 0 || O < 0 || !y || !x || !q || !scale) return set_error("matmul_q_s: bad arguments"), MOTY_EINVAL;
  static const int idot = [] {
    const char* e = getenv("IDOT");
    return !(e && *e == '0');
  }();
  if (!idot) return set_error("matmul_q_s: IDOT=0 (f32 x int8) is served by the CPU path"), MOTY_EUNSUP;
  if (S == 0 || O == 0) return MOTY_OK;
  const void *dq, *ds;
  int rc;
  if ((rc = weight(d, q, (size_t)O * I, &dq))) return rc;
  if ((rc = weight(d, scale, (size_t)O * 4, &ds))) return rc;
  void *dx, *dy;
  if ((rc = stage_io(d, x, (size_t)S * I * 4, (size_t)S * O * 4, &dx, &dy))) return rc;
  if ((rc = moty_hip_matmul_q_s_dev((float*)dy, (const float*)dx, (const int8_t*)dq, (const float*)ds, S, I, O,
                                    d->stream)))
    return rc;
  return finish_io(d, y, dy, (size_t)S * O * 4);
}

// ---- Q4R4 / Q8R4 (nn/matmul.c:365-466) ----
static int r4_check(const char* what, int S, int I, int O, const void* y, const void* x, const void* q,
                    const void* s16) {
  if (S < 0 || I <= 0 || O < 0 || !y || !x || !q || !s16) return set_error("%s: bad arguments", what), MOTY_EINVAL;
  if (I % 32) return set_error("%s: I=%d must be a multiple of 32", what, I), MOTY_EINVAL;
  return MOTY_OK;
}

static int r4_dev(bool q8, const char* what, float* y, const float* x, const uint8_t* q, const uint16_t* s16, int S,
                  int I, int O, void* stream) {
  CUR(d);
  int rc = r4_check(what, S, I, O, y, x, q, s16);
  if (rc || S == 0 || O == 0) return rc;
  if (need_al16(what, x, q)) return MOTY_EUNSUP;
  void* sp = nullptr;
  int8_t* xq = nullptr;
  float* xs = nullptr;
  int32_t* xm = nullptr;
  {  // activation scratch for the GEMM path (also taken by S <= 3 when the
     // decode GEMV does not serve the shape)
    const size_t bq = al256((size_t)S * I), bs = al256((size_t)S * (I / 32) * 4);
    if ((rc = scratch_get(d, bq + 2 * bs, STREAM(stream), &sp))) return rc;
    xq = (int8_t*)sp;
    xs = (float*)((char*)sp + bq);
    xm = (int32_t*)((char*)sp + bq + bs);
  }
  rc = launch_r4_matmul(q8, x, q, s16, y, S, I, O, xq, xs, xm, STREAM(stream));
  if (rc == MOTY_EUNSUP) set_error("%s: shape S=%d I=%d O=%d unsupported", what, S, I, O);
  return rc;
}

int moty_hip_matmul_q4r4_s_dev(float* y, const float* x, const uint8_t* q4, const uint16_t* s16, int S, int I, int O,
                               void* stream) {
  return r4_dev(false, "matmul_q4r4_s", y, x, q4, s16, S, I, O, stream);
}

int moty_hip_matmul_q8r4_s_dev(float* y, const float* x, const int8_t* q8, const uint16_t* s16, int S, int I, int O,
                               void* stream) {
  return r4_dev(true, "matmul_q8r4_s", y, x, (const uint8_t*)q8, s16, S, I, O, stream);
}

static int r4_host(bool q8, const char* what, float* y, const float* x, const void* q, const uint16_t* s16, int S,
                   int I, int O) {
  CUR(d);
  int rc = r4_check(what, S, I, O, y, x, q, s16);
  if (rc || S == 0 || O == 0) return rc;
  const size_t blocks = (size_t)((O + 3) / 4) * (I / 32);
  const void *dq, *ds;
  if ((rc = weight(d, q, blocks * (q8 ? 128 : 64), &dq))) return rc;
  if ((rc = weight(d, s16, blocks * 8, &ds))) return rc;
  void *dx, *dy;
  if ((rc = stage_io(d, x, (size_t)S * I * 4, (size_t)S * O * 4, &dx, &dy))) return rc;
  if ((rc = r4_dev(q8, what, (float*)dy, (const float*)dx, (const uint8_t*)dq, (const uint16_t*)ds, S, I, O,
                   d->stream)))
    return rc;
  return finish_io(d, y, dy, (size_t)S * O * 4);
}

int moty_hip_matmul_q4r4_s(float* y, const float* x, const uint8_t* q4, const uint16_t* s16, int S, int I, int O) {
  return r4_host(false, "matmul_q4r4_s", y, x, q4, s16, S, I, O);
}

int moty_hip_matmul_q8r4_s(float* y, const float* x, const int8_t* q8, const uint16_t* s16, int S, int I, int O) {
  return r4_host(true, "matmul_q8r4_s", y, x, q8, s16, S, I, O);
}

static int r4_gate_up(bool q8, const char* what, float* h, const float* x, const uint8_t* gu, const uint16_t* s16,
                      int D, int I, void* stream) {
  CUR(d);
  if (D <= 0 || I <= 0 || !h || !x || !gu || !s16) return set_error("%s: bad arguments", what), MOTY_EINVAL;
  if (D % 32 || I % 4) return set_error("%s: D=%d (multiple of 32), I=%d (multiple of 4)", what, D, I), MOTY_EINVAL;
  if (need_al16(what, x, gu)) return MOTY_EUNSUP;
  hipStream_t st = STREAM(stream);
  int rc = launch_r4_gate_up_silu(q8, x, gu, s16, h, D, I, st);
  if (rc != MOTY_EUNSUP) return rc;
  // widths the fused GEMV does not hold in registers (Q8R4 past D = 4096):
  // the plain R4 matmul over all 2I rows into scratch, then SiLU(g)*u --
  // the same results, one more pass over 2I floats
  const size_t bgu = al256((size_t)2 * I * 4), bq = al256((size_t)D), bs = al256((size_t)(D / 32) * 4);
  void* sp;
  if ((rc = scratch_get(d, bgu + bq + 2 * bs, st, &sp))) return rc;
  float* g2 = (float*)sp;
  int8_t* xq = (int8_t*)((char*)sp + bgu);
  float* xs = (float*)((char*)sp + bgu + bq);
  int32_t* xm = (int32_t*)((char*)sp + bgu + bq + bs);
  if ((rc = launch_r4_matmul(q8, x, gu, s16, g2, 1, D, 2 * I, xq, xs, xm, st)) == MOTY_OK)
    rc = launch_silu_rows(h, g2, 1, I, st);
  if (rc == MOTY_EUNSUP) set_error("%s: D=%d unsupported", what, D);
  return rc;
}

int moty_hip_gate_up_silu_q4r4_dev(float* h, const float* x, const uint8_t* gate_up, const uint16_t* s16, int D,
                                   int I, void* stream) {
  return r4_gate_up(false, "gate_up_silu_q4r4", h, x, gate_up, s16, D, I, stream);
}

int moty_hip_gate_up_silu_q8r4_dev(float* h, const float* x, const int8_t* gate_up, const uint16_t* s16, int D,
                                   int I, void* stream) {
  return r4_gate_up(true, "gate_up_silu_q8r4", h, x, (const uint8_t*)gate_up, s16, D, I, stream);
}

// moty_nn_dense_ffn with a row-fused R4 gate_up (nn/ffn.c:26-41)
static int r4_ffn(bool q8, const char* what, float* out, const float* x, int S, const uint8_t* gu,
                  const uint16_t* gs16, const uint8_t* dn, const uint16_t* ds16, int D, int I, void* stream) {
  CUR(d);
  if (S < 0 || D <= 0 || I <= 0 || !out || !x || !gu || !gs16 || !dn || !ds16)
    return set_error("%s: bad arguments", what), MOTY_EINVAL;
  if (D % 32 || I % 32) return set_error("%s: D=%d, I=%d must be multiples of 32", what, D, I), MOTY_EINVAL;
  if (S == 0) return MOTY_OK;
  if (need_al16(what, x, gu, dn)) return MOTY_EUNSUP;
  hipStream_t st = STREAM(stream);
  // scratch: h [S][I] | gu [S][2I] | activation codes for the GEMMs
  const int W = D > I ? D : I;
  const size_t bh = al256((size_t)S * I * 4), bgu = al256((size_t)S * 2 * I * 4);
  const size_t bq = al256((size_t)S * W), bs = al256((size_t)S * (W / 32) * 4);
  void* sp;
  int rc = scratch_get(d, bh + bgu + bq + 2 * bs, st, &sp);
  if (rc) return rc;
  float* h = (float*)sp;
  float* g2 = (float*)((char*)sp + bh);
  int8_t* xq = (int8_t*)((char*)sp + bh + bgu);
  float* xs = (float*)((char*)sp + bh + bgu + bq);
  int32_t* xm = (int32_t*)((char*)sp + bh + bgu + bq + bs);
  // S = 1: the decode GEMV with its SiLU epilogue; S > 3: one GEMM pass over
  // gate and up tiles with the SiLU epilogue; else the GEMV then silu_rows
  rc = S == 1 ? launch_r4_gate_up_silu(q8, x, gu, gs16, h, D, I, st)
       : S > 3 ? launch_r4_gate_up_gemm(q8, x, gu, gs16, h, S, D, I, xq, xs, xm, st)
               : MOTY_EUNSUP;
  if (rc == MOTY_EUNSUP) {
    if ((rc = launch_r4_matmul(q8, x, gu, gs16, g2, S, D, 2 * I, xq, xs, xm, st))) return rc;
    rc = launch_silu_rows(h, g2, S, I, st);
  }
  if (rc) return rc;
  rc = launch_r4_matmul(q8, h, dn, ds16, out, S, I, D, xq, xs, xm, st);
  if (rc == MOTY_EUNSUP) set_error("%s: shape S=%d D=%d I=%d unsupported", what, S, D, I);
  return rc;
}

int moty_hip_dense_ffn_q4r4_dev(float* out, const float* x, int S, const uint8_t* gate_up, const uint16_t* gus16,
                                const uint8_t* down, const uint16_t* ds16, int D, int I, void* stream) {
  return r4_ffn(false, "dense_ffn_q4r4", out, x, S, gate_up, gus16, down, ds16, D, I, stream);
}

int moty_hip_dense_ffn_q8r4_dev(float* out, const float* x, int S, const int8_t* gate_up, const uint16_t* gus16,
                                const int8_t* down, const uint16_t* ds16, int D, int I, void* stream) {
  return r4_ffn(true, "dense_ffn_q8r4", out, x, S, (const uint8_t*)gate_up, gus16, (const uint8_t*)down, ds16, D, I,
                stream);
}

int moty_hip_quant_g32_dev(const float* x, int8_t* xq, float* xs, int32_t* xsum, int S, int I, void* stream) {
  CUR(d);
  if (S < 0 || I <= 0 || !x || !xq || !xs || !xsum) return set_error("quant_g32: bad arguments"), MOTY_EINVAL;
  if (I % 32) return set_error("quant_g32: I=%d must be a multiple of 32", I), MOTY_EINVAL;
  return launch_quant_g32(x, xq, xs, xsum, S, I, STREAM(stream));
}

int moty_hip_pack_q4r4_dev(const float* w, uint8_t* q4, uint16_t* s16, int O, int I, void* stream) {
  CUR(d);
  if (O < 0 || I <= 0 || !w || !q4 || !s16) return set_error("pack_q4r4: bad arguments"), MOTY_EINVAL;
  if (I % 32) return set_error("pack_q4r4: I=%d must be a multiple of 32", I), MOTY_EINVAL;
  return launch_pack_r4(false, w, q4, s16, O, I, STREAM(stream));
}

int moty_hip_pack_q8r4_dev(const float* w, int8_t* q8, uint16_t* s16, int O, int I, void* stream) {
  CUR(d);
  if (O < 0 || I <= 0 || !w || !q8 || !s16) return set_error("pack_q8r4: bad arguments"), MOTY_EINVAL;
  if (I % 32) return set_error("pack_q8r4: I=%d must be a multiple of 32", I), MOTY_EINVAL;
  return launch_pack_r4(true, w, (uint8_t*)q8, s16, O, I, STREAM(stream));
}

// ---- GGUF block formats (io/gguf.h:231-357) ----
static int gguf_check(int dtype, int64_t numel, const void* raw, const void* out, const char* what) {
  int E, B;
  if (numel < 0 || (numel && (!raw || !out))) return set_error("%s: bad arguments", what), MOTY_EINVAL;
  if (!gguf_block(dtype, &E, &B)) return set_error("%s: GGUF type %d not supported", what, dtype), MOTY_EUNSUP;
  if (numel % E) return set_error("%s: numel=%lld is not a multiple of %d", what, (long long)numel, E), MOTY_EINVAL;
  return MOTY_OK;
}

int moty_hip_gguf_dequant_dev(int dtype, const void* raw, int64_t numel, float* out, void* stream) {
  CUR(d);
  int rc = gguf_check(dtype, numel, raw, out, "gguf_dequant");
  if (rc) return rc;
  if ((uintptr_t)out & 15) return set_error("gguf_dequant: out must be 16-byte aligned"), MOTY_EINVAL;
  return launch_gguf_dequant(dtype, raw, out, numel, STREAM(stream));
}

static int q40_check(const void* blocks, const void* q4, const void* qs, int64_t O, int64_t I) {
  if (O < 0 || I <= 0 || (O && (!blocks || !q4 || !qs))) return set_error("gguf_repack_q4_0: bad arguments"), MOTY_EINVAL;
  if (I % 32) return set_error("gguf_repack_q4_0: I=%lld must be a multiple of 32", (long long)I), MOTY_EINVAL;
  return MOTY_OK;
}

int moty_hip_gguf_repack_q4_0_dev(const uint8_t* blocks, uint8_t* q4, float* qs, int64_t O, int64_t I,
                                  void* stream) {
  CUR(d);
  int rc = q40_check(blocks, q4, qs, O, I);
  if (rc) return rc;
  if ((uintptr_t)q4 & 15 || (uintptr_t)qs & 3)
    return set_error("gguf_repack_q4_0: q4 must be 16-byte and qs 4-byte aligned"), MOTY_EINVAL;
  return launch_gguf_repack_q4_0(blocks, q4, qs, O * (I / 32), STREAM(stream));
}

int moty_hip_gguf_dequant(int dtype, const void* raw, int64_t numel, float* out) {
  CUR(d);
  int rc = gguf_check(dtype, numel, raw, out, "gguf_dequant");
  if (rc || numel == 0) return rc;
  int E, B;
  gguf_block(dtype, &E, &B);
  void *dr, *dy;
  if ((rc = stage_io(d, raw, (size_t)(numel / E) * B, (size_t)numel * 4, &dr, &dy))) return rc;
  if ((rc = launch_gguf_dequant(dtype, dr, (float*)dy, numel, d->stream))) return rc;
  return finish_io(d, out, dy, (size_t)numel * 4);
}

int moty_hip_gguf_repack_q4_0(const uint8_t* blocks, uint8_t* q4, float* qs, int64_t O, int64_t I) {
  CUR(d);
  int rc = q40_check(blocks, q4, qs, O, I);
  if (rc || O == 0) return rc;
  const int64_t nblk = O * (I / 32);
  void *dr, *dy;
  if ((rc = stage_io(d, blocks, (size_t)nblk * 18, (size_t)nblk * 20, &dr, &dy))) return rc;
  uint8_t* dq = (uint8_t*)dy;
  float* ds = (float*)(dq + nblk * 16);
  if ((rc = launch_gguf_repack_q4_0(dr, dq, ds, nblk, d->stream))) return rc;
  HIP_TRY(hipMemcpyAsync(q4, dq, (size_t)nblk * 16, hipMemcpyDeviceToHost, d->stream));
  return finish_io(d, qs, ds, (size_t)nblk * 4);
}

// The slot returns void: a failed call must not leave y looking valid, so
// every output becomes a quiet NaN (and the message stays for
// moty_hip_last_error()).
void moty_hip_hw_matmul_i8(float* y, const float* x, const int8_t* q, const float* scale, int S, int I, int O) {
  if (moty_hip_matmul_q_s(y, x, q, scale, S, I, O) != MOTY_OK && y && S > 0 && O > 0) {
    const float nan = __builtin_nanf("");
    for (int64_t i = 0; i < (int64_t)S * O; i++) y[i] = nan;
  }
}

int moty_hip_matmul_i4_grouped_s(float* y, const float* x, const uint8_t* q4, const float* scale, int S, int I,
                                 int O, int gs) {
  CUR(d);
  if (S < 0 || I <= 0 || O < 0 || gs <= 0 || !y || !x || !q4 || !scale)
    return set_error("matmul_i4_grouped_s: bad arguments"), MOTY_EINVAL;
  static const int idot4 = env_int("IDOT4", 0);
  if (S == 0 || O == 0) return MOTY_OK;
  const int ng = (I + gs - 1) / gs;
  const void *dq, *ds;
  int rc;
  if ((rc = weight(d, q4, (size_t)O * ((I + 1) / 2), &dq))) return rc;
  if ((rc = weight(d, scale, (size_t)O * ng * 4, &ds))) return rc;
  void *dx, *dy;
  if ((rc = stage_io(d, x, (size_t)S * I * 4, (size_t)S * O * 4, &dx, &dy))) return rc;
  if ((rc = moty_hip_matmul_i4_grouped_s_dev((float*)dy, (const float*)dx, (const uint8_t*)dq, (const float*)ds, S,
                                             I, O, gs, idot4, d->stream)))
    return rc;
  return finish_io(d, y, dy, (size_t)S * O * 4);
}

// moty_matmul_i4_s on host pointers; IDOT4 read from the environment once
// (nn/matmul.c:76-77)
int moty_hip_matmul_i4_s(float* y, const float* x, const uint8_t* q4, const float* scale, int S, int I, int O) {
  CUR(d);
  if (S < 0 || I <= 0 || O < 0 || !y || !x || !q4 || !scale) return set_error("matmul_i4_s: bad arguments"), MOTY_EINVAL;
  static const int idot4 = env_int("IDOT4", 0);
  if (S == 0 || O == 0) return MOTY_OK;
  if (I % 16) return set_error("matmul_i4_s: I=%d unsupported (I %% 16 == 0)", I), MOTY_EUNSUP;
  const void *dq, *ds;
  int rc;
  if ((rc = weight(d, q4, (size_t)O * ((I + 1) / 2), &dq))) return rc;
  if ((rc = weight(d, scale, (size_t)O * 4, &ds))) return rc;
  void *dx, *dy;
  if ((rc = stage_io(d, x, (size_t)S * I * 4, (size_t)S * O * 4, &dx, &dy))) return rc;
  if ((rc = moty_hip_matmul_i4_s_dev((float*)dy, (const float*)dx, (const uint8_t*)dq, (const float*)ds, S, I, O,
                                     idot4, d->stream)))
    return rc;
  return finish_io(d, y, dy, (size_t)S * O * 4);
}

// HwBackend.matmul_i4 (hw/hw_backend.h:59-60), void like matmul_i8: a
// failed call leaves every y a quiet NaN and its message.
void moty_hip_hw_matmul_i4(float* y, const float* x, const uint8_t* q4, const float* scale, int S, int I, int O) {
  if (moty_hip_matmul_i4_s(y, x, q4, scale, S, I, O) != MOTY_OK && y && S > 0 && O > 0) {
    const float nan = __builtin_nanf("");
    for (int64_t i = 0; i < (int64_t)S * O; i++) y[i] = nan;
  }
}

int moty_hip_matmul(float* y, const float* x, const float* W, int S, int I, int O) {
  CUR(d);
  if (S < 0 || I <= 0 || O < 0 || !y || !x || !W) return set_error("matmul: bad arguments"), MOTY_EINVAL;
  if (S == 0 || O == 0) return MOTY_OK;
  const void* dw;
  int rc;
  if ((rc = weight(d, W, (size_t)O * I * 4, &dw))) return rc;
  void *dx, *dy;
  if ((rc = stage_io(d, x, (size_t)S * I * 4, (size_t)S * O * 4, &dx, &dy))) return rc;
  if ((rc = moty_hip_matmul_dev((float*)dy, (const float*)dx, (const float*)dw, S, I, O, d->stream))) return rc;
  return finish_io(d, y, dy, (size_t)S * O * 4);
}

// Host-pointer MoE layer: router, bias and (uncached) the stacked experts go
// to the device through the weight cache; with an expert cache the experts
// come from its loader instead.
static int moe_host(const MotyHipMoe* m, MotyHipExpertCache* c, void* ctx, int layer, MotyHipLoadExpertFn fn,
                    const float* x, int S, float* out) {
  CUR(d);
  if (!m || !x || !out || S < 0 || m->E <= 0 || m->K <= 0 || m->I <= 0 || m->D <= 0)
    return set_error("moe_topk: bad arguments"), MOTY_EINVAL;
  if (S == 0) return MOTY_OK;
  const int E = m->E, I = m->I, D = m->D, K = m->K;
  const size_t ne = (size_t)E * I * D;
  MotyHipMoe dm = *m;
  const void* p;
  int rc;
  if ((rc = weight(d, m->router, (size_t)E * D * 4, &p))) return rc;
  dm.router = (const float*)p;
  if (m->logit_bias) {
    if ((rc = weight(d, m->logit_bias, (size_t)E * 4, &p))) return rc;
    dm.logit_bias = (const float*)p;
  }
  if (!c) {
    if ((rc = weight(d, m->g, ne, &p))) return rc;
    dm.g = (const int8_t*)p;
    if ((rc = weight(d, m->u, ne, &p))) return rc;
    dm.u = (const int8_t*)p;
    if ((rc = weight(d, m->d, ne, &p))) return rc;
    dm.d = (const int8_t*)p;
    if ((rc = weight(d, m->gs, (size_t)E * I * 4, &p))) return rc;
    dm.gs = (const float*)p;
    if ((rc = weight(d, m->us, (size_t)E * I * 4, &p))) return rc;
    dm.us = (const float*)p;
    if ((rc = weight(d, m->ds, (size_t)E * D * 4, &p))) return rc;
    dm.ds = (const float*)p;
  }
  // outputs: out, then optional idx/w/counts after it in the transfer arena
  const size_t b_out = al256((size_t)S * D * 4), b_kw = al256((size_t)S * K * 4), b_c = al256((size_t)E * 4);
  void *dx, *dy;
  if ((rc = stage_io(d, x, (size_t)S * D * 4, b_out + 2 * b_kw + b_c, &dx, &dy))) return rc;
  char* extra = (char*)dy + b_out;
  dm.idx_out = m->idx_out ? (int32_t*)extra : nullptr;
  dm.w_out = m->w_out ? (float*)(extra + b_kw) : nullptr;
  dm.counts_out = m->counts_out ? (int32_t*)(extra + 2 * b_kw) : nullptr;
  rc = c ? moty_hip_moe_topk_cached_dev(&dm, c, ctx, layer, fn, (const float*)dx, S, (float*)dy, d->stream)
         : moty_hip_moe_topk_dev(&dm, (const float*)dx, S, (float*)dy, d->stream);
  if (rc) return rc;
  if (m->idx_out) HIP_TRY(hipMemcpyAsync(m->idx_out, dm.idx_out, (size_t)S * K * 4, hipMemcpyDeviceToHost, d->stream));
  if (m->w_out) HIP_TRY(hipMemcpyAsync(m->w_out, dm.w_out, (size_t)S * K * 4, hipMemcpyDeviceToHost, d->stream));
  if (m->counts_out)
    HIP_TRY(hipMemcpyAsync(m->counts_out, dm.counts_out, (size_t)E * 4, hipMemcpyDeviceToHost, d->stream));
  return finish_io(d, out, dy, (size_t)S * D * 4);
}

int moty_hip_moe_topk(const MotyHipMoe* m, const float* x, int S, float* out) {
  return moe_host(m, nullptr, nullptr, 0, nullptr, x, S, out);
}

int moty_hip_moe_topk_cached(const MotyHipMoe* m, MotyHipExpertCache* c, void* ctx, int layer,
                             MotyHipLoadExpertFn fn, const float* x, int S, float* out) {
  if (!c || !fn) return set_error("moe_topk_cached: bad arguments"), MOTY_EINVAL;
  return moe_host(m, c, ctx, layer, fn, x, S, out);
}

int moty_hip_weight_forget(const void* host_ptr) {
  CUR(d);
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = d->wcache.find(host_ptr);
  if (it == d->wcache.end()) return MOTY_OK;
  HIP_TRY(hipStreamSynchronize(d->stream));
  HIP_TRY(hipFree(it->second.dev));
  d->wcache.erase(it);
  return MOTY_OK;
}

}  // extern "C"
