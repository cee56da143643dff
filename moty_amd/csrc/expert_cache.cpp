// expert_cache.cpp -- the expert residency manager on the device: the
// reference's per-layer ExpertCache (runtime/moecache.c:4-89, LFRU score of
// io/tier.c:23-26) with its slots in HBM, and the MoE layer over it.
//
// Bookkeeping is the reference's, decision for decision: the same slot
// receives the same expert, heat/recency/clock and the hit/miss counters
// move identically, so a caller's statistics and eviction behaviour do not
// change when the cache moves to the device.  A load calls the caller's
// loader (the reference's LoadExpertFn contract, runtime/moe.h:54-56) on a
// pinned host staging slot, then copies it into the device slot; two staging
// slots alternate so the loader fills one while the other's copy runs.
//
// The cached MoE layer routes on the device, reads the routing back (one
// small copy and a host wait, the point where the reference walks its
// experts), replays the reference's expert_get sequence -- ascending expert
// id once per active expert (nn/moe.c:186-203), or per token in top-k order
// (engines/olmoe.c:230-233) -- and runs the grouped GEMMs in passes: a pass
// holds experts loaded and not yet computed, and is flushed (its GEMMs
// queued) just before a load would overwrite one of them.  With cap >= the
// active experts that is one pass.  Results do not depend on the passes:
// every expert's rows are computed once from the same weights, and the
// combine runs after the last pass.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <vector>

#include "../../include/moty_hw_hip.h"
#include "common.h"
#include "dev.h"
#include "kernels.h"

struct MotyHipExpertCache {
  int cap = 1, n = 0, n_experts = 0;
  uint32_t clock = 0;
  long long hits = 0, misses = 0;
  std::vector<int> eid;  // [cap]
  std::vector<uint32_t> heat, last;
  std::vector<uint8_t> pinned;
  // device slots, sized by the first load's inter / hidden
  int I = 0, D = 0, dev = -1;
  int8_t *g = nullptr, *u = nullptr, *d = nullptr;
  float *gs = nullptr, *us = nullptr, *ds = nullptr;
  std::vector<MotyHipExpertSlot> dslot;  // [cap] device pointers
  // pinned host staging (two slots) and the event of each one's last copy
  MotyHipExpertSlot stage[2] = {}, stage_base[2] = {};
  hipEvent_t staged[2] = {nullptr, nullptr};
  int next_stage = 0;
  // the cached layer: pass tables (pinned host, one row per pass), routing
  // read-back, and the event that ends the previous call's use of them
  int* ptab_h = nullptr;
  size_t ptab_rows = 0;
  int* route_h = nullptr;
  size_t route_cap = 0;
  hipEvent_t call_done = nullptr;
};

namespace moty {

static uint64_t lfru_score(uint32_t heat, uint32_t last, uint32_t clock) {
  const uint32_t age = clock - last;
  return ((uint64_t)heat << 8) | (age < 255 ? 255 - age : 0);
}

static bool ec_pinned(const MotyHipExpertCache* c, int e) {
  return !c->pinned.empty() && e >= 0 && e < c->n_experts && c->pinned[e];
}

// expert_get's bookkeeping (runtime/moecache.c:48-88): the slot, whether it
// must be (re)loaded, and the expert it held before.
static int ec_get(MotyHipExpertCache* c, int eid, bool* load, int* prev) {
  if (!c->heat.empty() && eid >= 0 && eid < c->n_experts) {
    if (c->heat[eid] < 0xFFFFFFFFu) c->heat[eid]++;
    c->last[eid] = c->clock++;
  }
  for (int i = 0; i < c->n; i++)
    if (c->eid[i] == eid) {
      c->hits++;
      *load = false;
      *prev = eid;
      return i;
    }
  c->misses++;
  int v = 0;
  if (c->n < c->cap) {
    v = c->n++;
  } else if (!c->heat.empty()) {
    uint64_t worst = UINT64_MAX;
    for (int i = 0; i < c->n; i++) {
      const int e = c->eid[i];
      if (ec_pinned(c, e)) continue;
      // a slot left empty by a failed load scores lowest: refill it first
      const uint64_t s = e < 0 || e >= c->n_experts ? 0 : lfru_score(c->heat[e], c->last[e], c->clock);
      if (s < worst) {
        worst = s;
        v = i;
      }
    }
  } else {
    // no heat tracking (n_experts = 0): the reference's LRU-by-fill stand-in
    for (int i = 1; i < c->n; i++)
      if (!ec_pinned(c, c->eid[i])) {
        v = i;
        break;
      }
  }
  *prev = c->eid[v];
  c->eid[v] = eid;
  *load = true;
  return v;
}

// expert_pin's bookkeeping (runtime/moecache.c:24-46): always a load.
static int ec_pin(MotyHipExpertCache* c, int eid, int* prev) {
  if (!c->pinned.empty() && eid >= 0 && eid < c->n_experts) c->pinned[eid] = 1;
  int v;
  if (c->n < c->cap) {
    v = c->n++;
  } else {
    v = -1;
    for (int i = 0; i < c->n; i++)
      if (!ec_pinned(c, c->eid[i])) {
        v = i;
        break;
      }
    if (v < 0) v = 0;
  }
  *prev = c->eid[v];
  c->eid[v] = eid;
  return v;
}

static void ec_release(MotyHipExpertCache* c) {
  for (void* p : {(void*)c->g, (void*)c->u, (void*)c->d, (void*)c->gs, (void*)c->us, (void*)c->ds})
    if (p) hipFree(p);
  c->g = c->u = c->d = nullptr;
  c->gs = c->us = c->ds = nullptr;
  for (int k = 0; k < 2; k++) {
    if (c->stage_base[k].g) hipHostFree(c->stage_base[k].g);
    if (c->staged[k]) hipEventDestroy(c->staged[k]);
    c->stage_base[k] = c->stage[k] = MotyHipExpertSlot{};
    c->staged[k] = nullptr;
  }
  c->dslot.clear();
}

// Device and staging storage, on the first load; all or nothing.
static int ec_alloc(MotyHipExpertCache* c, int inter, int hidden) {
  if (c->g) {
    if (inter != c->I || hidden != c->D)
      return set_error("expert cache: inter/hidden %d/%d differ from the first load's %d/%d", inter, hidden, c->I,
                       c->D),
             MOTY_EINVAL;
    return MOTY_OK;
  }
  if (inter <= 0 || hidden <= 0) return set_error("expert cache: bad inter/hidden"), MOTY_EINVAL;
  HIP_TRY(hipGetDevice(&c->dev));
  const size_t ng = (size_t)inter * hidden, cap = (size_t)c->cap;
  void* p[6] = {};
  const size_t sz[6] = {cap * ng, cap * ng, cap * ng, cap * inter * 4, cap * inter * 4, cap * hidden * 4};
  hipError_t e = hipSuccess;
  for (int i = 0; i < 6 && e == hipSuccess; i++) e = hipMalloc(&p[i], sz[i]);
  c->g = (int8_t*)p[0];
  c->u = (int8_t*)p[1];
  c->d = (int8_t*)p[2];
  c->gs = (float*)p[3];
  c->us = (float*)p[4];
  c->ds = (float*)p[5];
  for (int k = 0; k < 2 && e == hipSuccess; k++) {
    void* h = nullptr;
    e = hipHostMalloc(&h, 3 * ng + (2 * (size_t)inter + hidden) * 4, hipHostMallocDefault);
    if (e != hipSuccess) break;
    char* b = (char*)h;
    c->stage_base[k] = MotyHipExpertSlot{-1,
                                         (int8_t*)b,
                                         (int8_t*)(b + ng),
                                         (int8_t*)(b + 2 * ng),
                                         (float*)(b + 3 * ng),
                                         (float*)(b + 3 * ng + inter * 4),
                                         (float*)(b + 3 * ng + 2 * (size_t)inter * 4)};
    c->stage[k] = c->stage_base[k];
    e = hipEventCreateWithFlags(&c->staged[k], hipEventDisableTiming);
  }
  if (e != hipSuccess) {
    ec_release(c);
    return check_hip(e, "expert cache allocation");
  }
  c->I = inter;
  c->D = hidden;
  c->dslot.resize(c->cap);
  for (int s = 0; s < c->cap; s++)
    c->dslot[s] = MotyHipExpertSlot{c->eid[s],         c->g + s * ng,     c->u + s * ng,     c->d + s * ng,
                                    c->gs + s * inter, c->us + s * inter, c->ds + s * hidden};
  return MOTY_OK;
}

// Fill device slot `s` with expert `eid` through the loader, on `st`.  On
// failure the slot is marked empty, so a later get reloads it instead of
// taking stale weights for a hit.
static int ec_load_(MotyHipExpertCache* c, void* ctx, int layer, int eid, MotyHipLoadExpertFn fn, int s,
                    hipStream_t st);
static int ec_load(MotyHipExpertCache* c, void* ctx, int layer, int eid, MotyHipLoadExpertFn fn, int s,
                   hipStream_t st) {
  const int rc = ec_load_(c, ctx, layer, eid, fn, s, st);
  if (rc) {
    c->eid[s] = -1;
    c->dslot[s].eid = -1;
  }
  return rc;
}
static int ec_load_(MotyHipExpertCache* c, void* ctx, int layer, int eid, MotyHipLoadExpertFn fn, int s,
                    hipStream_t st) {
  const int k = c->next_stage;
  c->next_stage ^= 1;
  HIP_TRY(hipEventSynchronize(c->staged[k]));  // its previous copy has left the staging slot
  MotyHipExpertSlot* h = &c->stage[k];
  *h = c->stage_base[k];  // the loader fills these buffers (it may not keep the pointers)
  h->eid = eid;
  fn(ctx, layer, eid, h, c->I, c->D);
  const size_t ng = (size_t)c->I * c->D;
  MotyHipExpertSlot& ds = c->dslot[s];
  HIP_TRY(hipMemcpyAsync(ds.g, h->g, ng, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(ds.u, h->u, ng, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(ds.d, h->d, ng, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(ds.gs, h->gs, (size_t)c->I * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(ds.us, h->us, (size_t)c->I * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(ds.ds, h->ds, (size_t)c->D * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(hipEventRecord(c->staged[k], st));
  ds.eid = eid;
  return MOTY_OK;
}

static int ec_check(MotyHipExpertCache* c, int eid, MotyHipLoadExpertFn fn, const char* what) {
  if (!c || !fn) return set_error("%s: bad arguments", what), MOTY_EINVAL;
  if (c->n_experts > 0 && (eid < 0 || eid >= c->n_experts))
    return set_error("%s: expert %d outside [0, %d)", what, eid, c->n_experts), MOTY_EINVAL;
  if (c->dev >= 0) {
    int cd;
    HIP_TRY(hipGetDevice(&cd));
    if (cd != c->dev) return set_error("%s: cache lives on device %d, current is %d", what, c->dev, cd), MOTY_EINVAL;
  }
  return MOTY_OK;
}

// Standalone get / pin: the slot is loaded on the library stream and ready
// when the call returns.
static int ec_fetch(bool pin, MotyHipExpertCache* c, void* ctx, int layer, int eid, MotyHipLoadExpertFn fn,
                    int inter, int hidden, MotyHipExpertSlot** out, const char* what) {
  CUR(dv);
  int rc = ec_check(c, eid, fn, what);
  if (rc) return rc;
  if ((rc = ec_alloc(c, inter, hidden))) return rc;
  bool load = true;
  int prev;
  const int s = pin ? ec_pin(c, eid, &prev) : ec_get(c, eid, &load, &prev);
  if (load) {
    // a cached MoE call queued on a caller's stream may still read the slot
    if (c->call_done) HIP_TRY(hipEventSynchronize(c->call_done));
    // work queued earlier on the library stream may still read the slot
    if ((rc = ec_load(c, ctx, layer, eid, fn, s, dv->stream))) return rc;
    HIP_TRY(hipStreamSynchronize(dv->stream));
  }
  if (out) *out = &c->dslot[s];
  return MOTY_OK;
}

}  // namespace moty

using namespace moty;

extern "C" {

int moty_hip_expert_cache_init(MotyHipExpertCache** lc, int cap, int n_experts) {
  if (!lc) return set_error("expert_cache_init: bad arguments"), MOTY_EINVAL;
  MotyHipExpertCache* c = new MotyHipExpertCache();
  c->cap = cap < 1 ? 1 : cap;
  c->n_experts = n_experts > 0 ? n_experts : 0;
  c->eid.assign(c->cap, -1);
  if (c->n_experts) {
    c->heat.assign(c->n_experts, 0);
    c->last.assign(c->n_experts, 0);
    c->pinned.assign(c->n_experts, 0);
  }
  *lc = c;
  return MOTY_OK;
}

int moty_hip_expert_cache_free(MotyHipExpertCache* c) {
  if (!c) return MOTY_OK;
  if (c->dev >= 0) {
    HIP_TRY(hipSetDevice(c->dev));
    HIP_TRY(hipDeviceSynchronize());
  }
  ec_release(c);
  if (c->ptab_h) hipHostFree(c->ptab_h);
  if (c->route_h) hipHostFree(c->route_h);
  if (c->call_done) hipEventDestroy(c->call_done);
  delete c;
  return MOTY_OK;
}

int moty_hip_expert_get(MotyHipExpertCache* c, void* ctx, int layer, int eid, MotyHipLoadExpertFn fn, int inter,
                        int hidden, MotyHipExpertSlot** slot) {
  return ec_fetch(false, c, ctx, layer, eid, fn, inter, hidden, slot, "expert_get");
}

int moty_hip_expert_pin(MotyHipExpertCache* c, void* ctx, int layer, int eid, MotyHipLoadExpertFn fn, int inter,
                        int hidden, MotyHipExpertSlot** slot) {
  return ec_fetch(true, c, ctx, layer, eid, fn, inter, hidden, slot, "expert_pin");
}

int moty_hip_expert_cache_stats(const MotyHipExpertCache* c, int* n, int* slot_eids, uint32_t* heat, uint32_t* last,
                                uint32_t* clock, long long* hits, long long* misses) {
  if (!c) return set_error("expert_cache_stats: bad arguments"), MOTY_EINVAL;
  if (n) *n = c->n;
  if (slot_eids) memcpy(slot_eids, c->eid.data(), sizeof(int) * c->cap);
  if (heat && c->n_experts) memcpy(heat, c->heat.data(), 4 * (size_t)c->n_experts);
  if (last && c->n_experts) memcpy(last, c->last.data(), 4 * (size_t)c->n_experts);
  if (clock) *clock = c->clock;
  if (hits) *hits = c->hits;
  if (misses) *misses = c->misses;
  return MOTY_OK;
}

void moty_hip_moe_route_bias(float* logits, const MotyHipExpertCache* c, float bias) {
  if (bias <= 0 || !c || !logits) return;
  for (int i = 0; i < c->n; i++)
    if (c->eid[i] >= 0) logits[c->eid[i]] += bias;
}

int moty_hip_moe_topk_cached_dev(const MotyHipMoe* m, MotyHipExpertCache* c, void* ctx, int layer,
                                 MotyHipLoadExpertFn fn, const float* x, int S, float* out, void* stream) {
  CUR(dv);
  if (!m || !c || !fn || !x || !out || S < 0) return set_error("moe_topk_cached: bad arguments"), MOTY_EINVAL;
  const int E = m->E, K = m->K, I = m->I, D = m->D;
  if (E <= 0 || K <= 0 || K > E || K > 64 || I <= 0 || D <= 0)
    return set_error("moe_topk_cached: bad shape E=%d K=%d I=%d D=%d", E, K, I, D), MOTY_EINVAL;
  if (c->n_experts > 0 && c->n_experts != E)
    return set_error("moe_topk_cached: cache tracks %d experts, layer has %d", c->n_experts, E), MOTY_EINVAL;
  if (S == 0) return MOTY_OK;
  if ((D % 32) || (I % 32) || E > 256)
    return set_error("moe_topk_cached: D=%d I=%d E=%d unsupported (D, I multiples of 32, E <= 256)", D, I, E),
           MOTY_EUNSUP;
  // the kernels move x, out and the router rows in 16-byte units
  if ((((uintptr_t)x) | ((uintptr_t)out) | ((uintptr_t)m->router)) & 15)
    return set_error("moe_topk_cached: x, out and router must be 16-byte aligned"), MOTY_EUNSUP;
  int rc = ec_check(c, 0, fn, "moe_topk_cached");
  if (rc) return rc;
  if ((rc = ec_alloc(c, I, D))) return rc;
  hipStream_t st = STREAM(stream);
  if (!c->call_done) HIP_TRY(hipEventCreateWithFlags(&c->call_done, hipEventDisableTiming));
  HIP_TRY(hipEventSynchronize(c->call_done));  // the previous call's host tables are free

  const int P = S * K;
  const bool topk = m->combine_order == MOTY_MOE_ORDER_TOPK;
  // at most one pass per expert_get of the sequence, plus the last
  const size_t max_pass = (size_t)(topk ? P : E) + 1;
  size_t offs[MOE_NBUF];
  const size_t need = al256(moe_scratch_size(S, D, E, K, I, offs));
  void* sp;
  if ((rc = scratch_get(dv, need + max_pass * E * 4, st, &sp))) return rc;
  int* ptab_d = (int*)((char*)sp + need);
  if (c->ptab_rows < max_pass) {
    if (c->ptab_h) HIP_TRY(hipHostFree(c->ptab_h));
    c->ptab_h = nullptr;
    HIP_TRY(hipHostMalloc((void**)&c->ptab_h, max_pass * E * 4, hipHostMallocDefault));
    c->ptab_rows = max_pass;
  }
  MoeArgs a;
  a.x = x;
  a.Wr = m->router;
  a.bias = m->logit_bias;
  a.G = c->g;
  a.U = c->u;
  a.Dn = c->d;
  a.GS = c->gs;
  a.US = c->us;
  a.DS = c->ds;
  a.out = out;
  a.T = S;
  a.D = D;
  a.E = E;
  a.K = K;
  a.I = I;
  a.norm = m->norm_topk;
  a.order = m->combine_order;
  a.idx_out = m->idx_out;
  a.w_out = m->w_out;
  a.counts_out = m->counts_out;
  a.probs_out = nullptr;
  if ((rc = launch_moe_route(a, sp, st))) {
    if (rc == MOTY_EUNSUP) set_error("moe_topk_cached: unsupported shape");
    return rc;
  }
  // routing back to the host: counts [E] and, for the top-k order, idx [P]
  const size_t rn = (size_t)E + (topk ? P : 0);
  if (c->route_cap < rn) {
    if (c->route_h) HIP_TRY(hipHostFree(c->route_h));
    c->route_h = nullptr;
    HIP_TRY(hipHostMalloc((void**)&c->route_h, rn * 4, hipHostMallocDefault));
    c->route_cap = rn;
  }
  const int *didx, *dcnt;
  moe_routing(a, sp, &didx, &dcnt);
  HIP_TRY(hipMemcpyAsync(c->route_h, dcnt, (size_t)E * 4, hipMemcpyDeviceToHost, st));
  if (topk) HIP_TRY(hipMemcpyAsync(c->route_h + E, didx, (size_t)P * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  std::vector<int> seq;
  if (topk) {
    seq.assign(c->route_h + E, c->route_h + E + P);
  } else {
    for (int e = 0; e < E; e++)
      if (c->route_h[e] > 0) seq.push_back(e);
  }

  std::vector<char> inpass(E, 0), done(E, 0);
  int npass = 0, pending = 0;
  int* row = c->ptab_h;
  for (int e = 0; e < E; e++) row[e] = -1;
  auto flush = [&]() -> int {
    if (!pending) return MOTY_OK;
    int* drow = ptab_d + (size_t)npass * E;
    HIP_TRY(hipMemcpyAsync(drow, row, (size_t)E * 4, hipMemcpyHostToDevice, st));
    int r = launch_moe_experts(a, sp, drow, st);
    if (r) return r;
    for (int e = 0; e < E; e++)
      if (inpass[e]) {
        inpass[e] = 0;
        done[e] = 1;
      }
    pending = 0;
    npass++;
    row = c->ptab_h + (size_t)npass * E;
    for (int e = 0; e < E; e++) row[e] = -1;
    return MOTY_OK;
  };
  for (const int eid : seq) {
    if (eid < 0 || eid >= E) continue;
    bool load;
    int prev;
    const int s = ec_get(c, eid, &load, &prev);
    if (load) {
      if (prev >= 0 && prev < E && inpass[prev] && (rc = flush())) return rc;
      if ((rc = ec_load(c, ctx, layer, eid, fn, s, st))) return rc;
    }
    if (!done[eid] && !inpass[eid]) {
      inpass[eid] = 1;
      pending++;
    }
    if (inpass[eid]) row[eid] = s;
  }
  if ((rc = flush())) return rc;
  if ((rc = launch_moe_combine(a, sp, st))) return rc;
  HIP_TRY(hipEventRecord(c->call_done, st));
  return MOTY_OK;
}

}  // extern "C"
