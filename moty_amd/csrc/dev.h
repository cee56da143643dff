// dev.h -- per-device state of libmoty-hw-hip shared by the C-ABI files
// (api.cpp, expert_cache.cpp): the library stream, the growable scratch and
// transfer arenas, and the weight cache keyed by host pointer.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

#include <unordered_map>

namespace moty {

struct WEntry {
  void* dev;
  size_t bytes;
  uint64_t fp;  // sampled content fingerprint of the host buffer at upload
};

struct Arena {
  void* p = nullptr;
  size_t cap = 0;
};

struct Dev {
  bool ready = false;
  int cus = 0;  // compute units
  hipStream_t stream = nullptr;
  Arena scratch, io;
  // the stream whose queued work last used `scratch`, and an event recorded
  // on it when that call returned (after its work was queued) that orders a
  // later call on another stream behind that work; scr_pend: a call took the
  // arena and has not returned yet; scr_ev_ok: scr_ev marks the last use
  // (false when that use was under graph capture)
  hipStream_t scr_stream = nullptr;
  bool scr_used = false, scr_pend = false, scr_ev_ok = false;
  hipEvent_t scr_ev = nullptr;
  // device address of this device's copy of the fixed no-allocation
  // scratch array (api.cpp), taken once at set-up, and the same ordering
  // state for it (event created at set-up)
  void* fixed_scratch = nullptr;
  hipStream_t fx_stream = nullptr;
  bool fx_used = false, fx_ev_ok = false;
  hipEvent_t fx_ev = nullptr;
  // one-launch decode FFN: the h exchange words, one call counter per
  // workgroup of its grid (which is always `cus` workgroups) and the
  // bounded-wait error flag; allocated and zeroed at set-up
  unsigned long long* f1_xh = nullptr;
  unsigned* f1_epoch = nullptr;
  unsigned* f1_err = nullptr;
  bool f1_on = true;
  std::unordered_map<const void*, WEntry> wcache;
};

// The calling thread's device (device 0 on first use), made current.
int cur(Dev** out);
// Grow an arena to at least `bytes`; waits for queued work before freeing.
int arena_get(Arena& a, size_t bytes, void** p);
// The device's scratch arena for work about to be queued on `st`: when the
// previous user queued on another stream, `st` first waits for that work
// (calls on one device share the arena, so two streams must not overlap in
// it).  Streams under graph capture are left unordered.
int scratch_get(Dev* d, size_t bytes, hipStream_t st, void** p);
// Called as an entry point returns (ScrGuard): when it took the scratch
// arena, record scr_ev on its stream, behind the work it queued.
void scratch_mark(Dev* d);
struct ScrGuard {
  Dev* d;
  ~ScrGuard() {
    if (d && d->scr_pend) scratch_mark(d);
  }
};
// Stage host x into the transfer arena (device x and y returned), and copy
// y back and synchronise.
int stage_io(Dev* d, const void* x, size_t xbytes, size_t ybytes, void** dx, void** dy);
int finish_io(Dev* d, void* y, const void* dy, size_t ybytes);

inline size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

}  // namespace moty

#define CUR(d)           \
  moty::Dev* d = nullptr; \
  {                      \
    int _rc = moty::cur(&d); \
    if (_rc) return _rc; \
  }                      \
  moty::ScrGuard _scr_guard{d};
#define STREAM(s) ((hipStream_t)(s))
