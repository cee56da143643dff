"""bench.py -- one-GPU benchmark of libmoty-hw-hip on BASELINE.json's configs.

Headline (`value`): C1, the Qwen3-0.6B-shaped decode FFN through the Q8_0
path (fused gate/up GEMV with the SiLU epilogue, then the down GEMV), as
whole-FFN algorithmic GB/s.  The MoE metric (C4, OLMoE-shaped layer at
T=256, tokens/s) is the `moe` object; C2, C3 and C5 are under `extra`.
Every figure is kernel work on inputs already resident in HBM: weights
rotate over distinct copies totalling more than the 256 MB Infinity Cache,
so each step streams its weights from HBM, and steps replay from HIP graphs.
The reference's CPU path (oracle/_ref, built from the reference's sources)
is timed on the host cores beside it (`cpu_baseline`).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

# the reference engines' own OpenMP tuning (runtime/env.c:43-78), for the
# CPU baseline; set before any OpenMP runtime loads
for _k, _v in (("OMP_WAIT_POLICY", "active"), ("OMP_PROC_BIND", "close"), ("GOMP_SPINCOUNT", "200000")):
    os.environ.setdefault(_k, _v)

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # dense int8 MFMA
F16_PEAK_TFLOPS = 2500.0  # dense f16 MFMA
F32_PEAK_TFLOPS = 157.3  # f32
METRIC = "Q8 GEMV HBM GB/s (% peak); MoE layer tokens/s at T=256 (1 GPU)"
HIDDEN = ("x", "Wr", "layer0", "_cpu", "w0")  # inputs kept for the CPU baseline, never printed


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--quick", action="store_true", help="C1 and C4 only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU reference baseline")
    ap.add_argument("--cpu-seconds", type=float, default=6.0, help="bound on each CPU baseline sample")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="only launch the dominant kernel on distinct weights and a 64 MiB copy (for rocprofv3 --pmc)")
    ap.add_argument("--only", choices=["c1", "c2", "c3", "c3r4", "c4", "c5", "c5s", "q8gemv", "floor", "d1"],
                    help="run one config alone and print its JSON object (for rocprofv3 runs of a single config)")
    return ap.parse_args()


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def roofline(bound, achieved, peak, unit, traffic=None):
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


class Ctx:
    def __init__(self, torch, ops):
        import moty_amd
        self.torch, self.ops, self.ops_mod = torch, ops, moty_amd

    def gen(self, cfg, tensor):
        return self.torch.Generator(device="cuda:0").manual_seed(0x4D4F5459 ^ (cfg << 8) ^ tensor)

    def randn(self, shape, g, std=1.0):
        return self.torch.randn(shape, generator=g, device="cuda:0", dtype=self.torch.float32) * std

    def q8(self, shape, g):
        """W ~ N(0, 0.02) on the device, quantized by the library's
        moty_quantize_rows kernel (QBITS=8)."""
        w = self.randn(shape, g, 0.02)
        q, s = self.ops.quantize_rows(w.reshape(-1, shape[-1]))
        return q.reshape(shape), s.reshape(shape[:-1])

    def q4(self, shape, g):
        w = self.randn(shape, g, 0.02)
        return self.ops.pack_int4_grouped(w, 32)

    def time_steps(self, fns, steps, warmup, replays=7):
        """Time exactly `steps` steps, `replays` times: step k of a run
        calls one fns[i] (each fn a step over its own weight copy).  Every
        round r captures three HIP graphs over consecutive copies: warm-up A
        (`warmup` steps), warm-up B (`warmup` steps) and the K timed steps;
        round r starts where round r-1 ended, so with enough copies no copy
        is touched twice within the Infinity Cache's reach.  After one
        untimed replay of every graph (the first replay uploads it), each
        round times A alone between two HIP events, then B followed by the
        timed graph between two more: B's graph is queued behind the events
        while the GPU is still busy, and A and B do the same work on cold
        copies, so the difference is the time the K steps add, with the fixed
        cost of an event pair around a graph launch (about 9 us on MI355X,
        0.45 us per C1 step at the driver's K = 20) cancelled.  The result is
        the median round's seconds per step (self.last holds the round count,
        the spread and the raw B + timed figure).  Returns (seconds per step,
        steps timed)."""
        torch = self.torch
        n = len(fns)
        steps = max(1, int(steps))
        warmup = max(1, int(warmup))
        replays = max(1, int(replays))
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for f in fns:  # eager pass sizes the library's scratch before capture
                f()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()

        def capture(first, count):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for k in range(count):
                    fns[(first + k) % n]()
            return g
        rounds = []
        per = 2 * warmup + steps
        for r in range(replays):
            b = r * per
            rounds.append((capture(b, warmup), capture(b + warmup, warmup), capture(b + 2 * warmup, steps)))
        ts, raw = [], []
        with torch.cuda.stream(s):
            for gs in rounds:
                for g in gs:
                    g.replay()
            torch.cuda.synchronize()
            for wa, wb, timed in rounds:
                ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
                ev[0].record(s)
                wa.replay()
                ev[1].record(s)
                ev[2].record(s)
                wb.replay()
                timed.replay()
                ev[3].record(s)
                torch.cuda.synchronize()
                tw = ev[0].elapsed_time(ev[1]) / 1e3
                twk = ev[2].elapsed_time(ev[3]) / 1e3
                ts.append((twk - tw) / steps)
                raw.append(twk)
        del rounds
        ts.sort()
        raw.sort()
        med = ts[len(ts) // 2]
        self.last = {"replays": len(ts), "spread_us": [round(ts[0] * 1e6, 3), round(ts[-1] * 1e6, 3)],
                     "method": "per round: (warm-up B + K steps) - (warm-up A), each between HIP events, over "
                               "copies no earlier round touched when the copies allow; median over rounds",
                     "warm_plus_timed_us_median": round(raw[len(raw) // 2] * 1e6, 1)}
        return med, steps


C5_SKEW_LABEL = "skewed (+2.0 on 8 hot experts)"


def c5_skew_bias():
    """C5's skewed routing: +2.0 on the router logits of every 16th of the 128 experts."""
    import torch
    bias = torch.zeros(128, device="cuda:0")
    bias[torch.arange(0, 128, 16, device="cuda:0")] = 2.0
    return bias


def pmc_traffic(name, key=None):
    """HBM bytes per launch of a kernel from its committed rocprofv3 PMC
    summary (profiles/<name>.md, line `traffic_bytes_per_launch: N`, or
    `traffic_bytes_per_launch[key]: N` for one of several kernels)."""
    tag = "traffic_bytes_per_launch%s:" % ("[%s]" % key if key else "")
    try:
        for line in open(os.path.join(ROOT, "profiles", name + ".md")):
            if line.startswith(tag):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def n_copies(bytes_per_copy, target=1200 << 20, lo=2):
    return max(lo, -(-target // bytes_per_copy))


# --------------------------------------------------------------------------
def bench_c1(c, steps, warmup):
    """Qwen3-0.6B FFN decode: D=1024, I=3072, S=1 (configs[0] shape)."""
    torch, ops = c.torch, c.ops
    D, I = 1024, 3072
    wbytes = 3 * D * I + (2 * I + D) * 4           # int8 weights + f32 row scales
    algo = wbytes + 2 * D * 4                      # + x in, out
    # 4.8 GB of copies: the Infinity Cache keeps some lines of the copies
    # written last at set-up, so a 1.2 GB rotation (133 copies) read part of
    # its bytes from there (5.59 against 5.92 us per step at 266 copies and
    # 5.88 at 532)
    ncopy = n_copies(wbytes, target=4800 << 20)
    g = c.gen(0, 1)
    copies = [c.q8((I, D), g) + c.q8((I, D), g) + c.q8((D, I), g) for _ in range(ncopy)]
    x = c.randn((1, D), c.gen(0, 2))
    out = torch.empty((1, D), device="cuda:0")
    h = torch.empty((1, I), device="cuda:0")
    t, n = c.time_steps([lambda w=w: ops.dense_ffn_q8(x, *w, out=out) for w in copies], steps, warmup)
    rep = dict(c.last)
    # dominant kernel alone: the fused gate+up GEMV (k_gemv_q8 PAIR mode)
    gu = [lambda w=w: ops.gate_up_silu_q8(x, w[0], w[1], w[2], w[3], out=h) for w in copies]
    tg, _ = c.time_steps(gu, steps, warmup)
    gu_algo = 2 * I * D + 2 * I * 4 + D * 4 + I * 4
    # the one-launch form of the same FFN (workgroups exchanging h through
    # device memory; bit-exact, off by default), timed alike
    ops.set_ffn1(1)
    try:
        t1, _ = c.time_steps([lambda w=w: ops.dense_ffn_q8(x, *w, out=out) for w in copies], steps, warmup)
    finally:
        ops.set_ffn1(0)
    torch.cuda.synchronize()
    return {
        "workload": "C1 Qwen3-0.6B FFN decode, Q8_0 (fused gate/up GEMV + SiLU, down GEMV), S=1, D=1024, I=3072",
        "gbs": algo / t / 1e9, "ms_per_step": t * 1e3, "steps": n, "algo_bytes": algo,
        "weight_copies": ncopy, "x": x, "w0": copies[0], "timing": rep,
        "kernel": {"name": "k_gemv1_q8<1,4,PAIR,4> gate+up+SiLU", "us": tg * 1e6, "algo_bytes": gu_algo,
                   "gbs": gu_algo / tg / 1e9},
        "one_launch_us": round(t1 * 1e6, 3),
    }


def floor_probe():
    """Launch and pure-read floors and hand-off latencies of this GPU
    (libmoty_probe.so, built from moty_amd/csrc/floor_probe.hip)."""
    import ctypes as C
    try:
        L = C.CDLL(os.path.join(ROOT, "moty_amd", "libmoty_probe.so"))
        L.moty_probe_floor_names.restype = C.c_char_p
        names = L.moty_probe_floor_names().decode().split(",")
        out = (C.c_float * len(names))()
        rc = L.moty_probe_floor(out)
        if rc:
            return {"error": "hip error %d" % rc}
        return {k: round(float(v), 3) for k, v in zip(names, out)}
    except OSError as e:
        return {"error": str(e)[:160]}


def moe_weights(c, cfg, E, I, D):
    g = c.gen(cfg, 10)
    G, GS = c.q8((E, I, D), g)
    U, US = c.q8((E, I, D), g)
    Dn, DS = c.q8((E, D, I), g)
    return G, GS, U, US, Dn, DS


def bench_moe(c, cfg, T, E, K, I, D, norm, order, steps, warmup, bias=None, label="", traffic_key=None):
    torch, ops = c.torch, c.ops
    from moty_amd.ops import MoeLayer
    ebytes = 3 * E * I * D + E * (2 * I + D) * 4
    ncopy = n_copies(ebytes, lo=2)
    Wr = c.randn((E, D), c.gen(cfg, 1), 0.02)
    x = c.randn((T, D), c.gen(cfg, 2))
    layers = [MoeLayer(Wr, *moe_weights(c, cfg + 16 * k, E, I, D), K, norm_topk=norm, order=order,
                       logit_bias=bias) for k in range(ncopy)]
    out = torch.empty((T, D), device="cuda:0")
    # routing statistics (same router for every copy)
    _, idx, w, cnt = layers[0](x, want_routing=True)
    cnt = cnt.cpu()
    active = int((cnt > 0).sum())
    algo = 3 * active * I * D + active * (2 * I + D) * 4 + E * D * 4 + 2 * T * D * 4
    ops_int = 2 * T * K * 3 * I * D
    t, n = c.time_steps([lambda L=L: L(x, out=out) for L in layers], max(16, steps // 16), max(4, warmup // 16))
    gbs = algo / t / 1e9
    return {
        "workload": label, "tokens_per_s": T / t, "ms_per_layer": t * 1e3, "steps": n, "timing": dict(c.last),
        "weight_copies": ncopy,
        "active_experts": active, "load_max": int(cnt.max()), "load_mean": round(float(cnt.float().mean()), 2),
        "roofline": roofline("hbm", gbs, HBM_PEAK_GBS, "GB/s",
                             pmc_traffic("hbm_traffic_pmc", traffic_key) if traffic_key else None),
        "int_tops": round(ops_int / t / 1e12, 2),
        "x": x, "Wr": Wr, "layer0": layers[0],
    }


def bench_moe_d1(c, cfg, E, K, I, D, steps, warmup, label):
    """Decode MoE, S = 1: moty_nn_moe_topk_d1 (nn/moe.c:33-153) -- router,
    softmax top-k (normalised), the K active experts' FFNs, combine in top-k
    order.  Only the K routed experts' weights move, so the weight copies
    rotate until the touched bytes exceed the Infinity Cache."""
    torch = c.torch
    from moty_amd.ops import MoeLayer
    ebytes = 3 * I * D + (2 * I + D) * 4  # one expert
    algo = K * ebytes + E * D * 4 + 2 * D * 4
    ncopy = n_copies(K * ebytes, lo=2)
    Wr = c.randn((E, D), c.gen(cfg, 1), 0.02)
    x = c.randn((1, D), c.gen(cfg, 2))
    layers = [MoeLayer(Wr, *moe_weights(c, cfg + 32 * k, E, I, D), K, norm_topk=1, order=c.ops_mod.ORDER_TOPK)
              for k in range(ncopy)]
    out = torch.empty((1, D), device="cuda:0")
    t, n = c.time_steps([lambda L=L: L(x, out=out) for L in layers], steps, warmup)
    rep = dict(c.last)
    return {"workload": label, "us_per_token": round(t * 1e6, 3), "tokens_per_s": round(1 / t, 1), "steps": n,
            "timing": rep, "weight_copies": ncopy, "algo_bytes": algo,
            "roofline": roofline("hbm", algo / t / 1e9, HBM_PEAK_GBS, "GB/s"),
            "x": x, "Wr": Wr, "layer0": layers[0]}


def bench_moe_cached(c, steps):
    """The C4 layer shape through the device expert cache (runtime/moecache.c
    on HBM slots) in nn/moe.c's batch order: cap = 64 (every expert resident
    after the first call: the cost over the uncached layer is the routing
    read-back) and cap = 32 (half the experts stream from host memory each
    call; bound by the host-to-device copies).  Eager calls: the cached layer
    waits for its routing mid-call, so it is not graph-captured."""
    import ctypes as C
    import time
    import numpy as np
    import moty_amd
    from moty_amd import LOAD_EXPERT_FN, MotyHipMoe, ORDER_EXPERT, lib
    torch = c.torch
    T, E, K, I, D = 256, 64, 8, 1024, 2048
    G, GS, U, US, Dn, DS = (t.cpu().numpy() for t in moe_weights(c, 3, E, I, D))
    host = {"g": G, "u": U, "d": Dn, "gs": GS, "us": US, "ds": DS}
    ebytes = 3 * I * D + (2 * I + D) * 4

    def load(ctx, layer, eid, slot, inter, hidden):
        s = slot.contents
        for k in host:
            a = host[k][eid]
            C.memmove(getattr(s, k), a.ctypes.data, a.nbytes)

    fn = LOAD_EXPERT_FN(load)
    Wr = c.randn((E, D), c.gen(3, 1), 0.02)
    x = c.randn((T, D), c.gen(3, 2))
    out = torch.empty((T, D), device="cuda:0")
    m = MotyHipMoe()
    m.router = C.c_void_p(Wr.data_ptr())
    m.E, m.K, m.I, m.D = E, K, I, D
    m.norm_topk, m.combine_order = 1, ORDER_EXPERT
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    res = {}
    for cap, n in ((64, max(10, steps // 16)), (32, 5)):
        cache = C.c_void_p()
        moty_amd.check(lib().moty_hip_expert_cache_init(C.byref(cache), cap, E), "cache init")

        def call():
            moty_amd.check(lib().moty_hip_moe_topk_cached_dev(C.byref(m), cache, None, 0, fn, C.c_void_p(x.data_ptr()),
                                                              T, C.c_void_p(out.data_ptr()), st), "moe cached")
        for _ in range(3):
            call()
        torch.cuda.synchronize()
        miss0 = C.c_longlong()
        lib().moty_hip_expert_cache_stats(cache, None, None, None, None, None, None, C.byref(miss0))
        t0 = time.perf_counter()
        for _ in range(n):
            call()
        torch.cuda.synchronize()
        t = (time.perf_counter() - t0) / n
        miss = C.c_longlong()
        lib().moty_hip_expert_cache_stats(cache, None, None, None, None, None, None, C.byref(miss))
        loads = (miss.value - miss0.value) / n
        res["cap%d" % cap] = {"ms_per_layer": round(t * 1e3, 4), "tokens_per_s": round(T / t, 1),
                              "loads_per_call": loads, "h2d_gbs": round(loads * ebytes / t / 1e9, 2)}
        moty_amd.check(lib().moty_hip_expert_cache_free(cache), "cache free")
    return {"workload": "C4 MoE layer shape through the device expert cache (batch order), T=256, E=64, top-8, "
                        "cap=64 resident / cap=32 streaming from host memory", **res}


def bench_c2(c, steps, warmup):
    """Qwen3-0.6B layer, the seven projections as Q8 prefill GEMMs, M=512.
    q, k, v, gate and up share their input, so their rows are stored
    concatenated (the fused-rows layout of moty_mat_fuse_rows,
    nn/mat.c:32-68, and of the fused gate_up of nn/ffn.c:28-37) and run as
    one GEMM; o and down run on their own inputs.  The three distinct
    inputs are quantized in one launch (moty_hip_qrow_i8_multi_dev)."""
    torch, ops = c.torch, c.ops
    M = 512
    shapes = [("q", 2048, 1024), ("k", 1024, 1024), ("v", 1024, 1024), ("gate", 3072, 1024), ("up", 3072, 1024),
              ("o", 1024, 2048), ("down", 1024, 3072)]
    fused_o = sum(O for _, O, I in shapes if I == 1024)
    wbytes = sum(O * I + O * 4 for _, O, I in shapes)
    ncopy = n_copies(wbytes, target=1100 << 20)
    g = c.gen(1, 1)
    copies = [[c.q8((fused_o, 1024), g), c.q8((1024, 2048), g), c.q8((1024, 3072), g)] for _ in range(ncopy)]
    xs = {I: c.randn((M, I), c.gen(1, 2 + I)) for I in (1024, 2048, 3072)}
    ys = {1024: torch.empty((M, fused_o), device="cuda:0"), 2048: torch.empty((M, 1024), device="cuda:0"),
          3072: torch.empty((M, 1024), device="cuda:0")}
    xq = {I: torch.empty((M, I), dtype=torch.int8, device="cuda:0") for I in xs}
    sx = {I: torch.empty(M, device="cuda:0") for I in xs}
    lib = ops.lib()
    import ctypes as C
    keys = (1024, 2048, 3072)
    arr = lambda vals: (C.c_void_p * 3)(*vals)
    qjobs = (arr([xs[I].data_ptr() for I in keys]), arr([xq[I].data_ptr() for I in keys]),
             arr([sx[I].data_ptr() for I in keys]), (C.c_int * 3)(M, M, M), (C.c_int * 3)(*keys))

    def step(ws):
        def f():
            # the three distinct inputs quantized in one launch
            ops.check(lib.moty_hip_qrow_i8_multi_dev(3, *qjobs, ops._stream()), "qrow_multi")
            for I, (q, s) in zip((1024, 2048, 3072), ws):
                ops.matmul_q8_preq(xq[I], sx[I], q, s, out=ys[I])
        return f
    t, n = c.time_steps([step(w) for w in copies], max(16, steps // 8), max(4, warmup // 8))
    rep = dict(c.last)
    ops_int = 2 * M * sum(O * I for _, O, I in shapes)

    # the three GEMMs alone, and the platform library's int8 GEMM
    # (torch._int_mm: hipBLASLt, int32 out, no scale epilogue) on the same
    # operands, timed alike: a yardstick for the MFMA fraction above
    def gemms(ws):
        return lambda: [ops.matmul_q8_preq(xq[I], sx[I], q, s, out=ys[I]) for I, (q, s) in zip((1024, 2048, 3072), ws)]

    def lib_gemms(ws):
        return lambda: [torch._int_mm(xq[I], q.t()) for I, (q, _) in zip((1024, 2048, 3072), ws)]
    nt, nw = max(16, steps // 8), max(4, warmup // 8)
    tg, _ = c.time_steps([gemms(w) for w in copies], nt, nw)
    try:
        tl, _ = c.time_steps([lib_gemms(w) for w in copies], nt, nw)
        lib_ref = {"ms_per_step": tl * 1e3, "tops": round(ops_int / tl / 1e12, 1)}
    except Exception as e:  # the library may not take a shape
        lib_ref = {"error": str(e)[:160]}
    algo = wbytes + M * (1024 + 2048 + 3072) * 4 + sum(M * O * 4 for _, O, _ in shapes)
    return {"workload": "C2 Qwen3-0.6B layer, 7 Q8 projections as prefill GEMMs, M=512 "
                        "(q/k/v/gate/up fused by rows: one GEMM N=10240, K=1024; o; down)",
            "ms_per_step": t * 1e3, "steps": n, "timing": rep,
            "roofline": roofline("mfma", ops_int / t / 1e12, INT8_PEAK_TOPS, "TOP/s",
                                 pmc_traffic("hbm_traffic_pmc", "c2_step")),
            "hbm_gbs": round(algo / t / 1e9, 1),
            "gemms_only": {"ms_per_step": tg * 1e3, "tops": round(ops_int / tg / 1e12, 1)},
            "library_int_mm": lib_ref,
            "_cpu": {"x": xs, "w": copies[0], "ops_int": ops_int}}


def bench_c3(c, steps, warmup):
    """8B-dense FFN in grouped int4 (Q4FMT=g, IDOT4=1): M=1 GEMV and M=256 GEMM."""
    torch, ops = c.torch, c.ops
    D, I = 4096, 12288
    wbytes = 3 * (I * D // 2 + I * D // 32 * 4)
    ncopy = n_copies(wbytes)
    g = c.gen(2, 1)
    copies = [(c.q4((I, D), g), c.q4((I, D), g), c.q4((D, I), g)) for _ in range(ncopy)]
    res = {"_cpu": {"w": copies[0], "x": {}}}
    for M in (1, 256):
        x = c.randn((M, D), c.gen(2, 2))
        res["_cpu"]["x"][M] = x
        y = torch.empty((M, D), device="cuda:0")

        def step(w):
            # moty_nn_dense_ffn over WF_I4G Mats: gate + up + SiLU in one
            # pass (a GEMV at M = 1, the f16-MFMA GEMM at M = 256), then down
            return lambda: ops.dense_ffn_i4g(x, w[0][0], w[0][1], w[1][0], w[1][1], w[2][0], w[2][1], out=y)
        t, n = c.time_steps([step(w) for w in copies], max(32 if M == 1 else 8, steps // (8 if M == 1 else 16)), 8)
        ops_int = 2 * M * 3 * I * D
        algo = wbytes + M * (D + I + I + D) * 4
        tr = pmc_traffic("hbm_traffic_pmc", "c3_M%d_step" % M)
        res["M%d" % M] = {"ms_per_step": t * 1e3, "steps": n, "timing": dict(c.last),
                          "hbm": roofline("hbm", algo / t / 1e9, HBM_PEAK_GBS, "GB/s", tr),
                          "mfma": roofline("mfma", ops_int / t / 1e12, INT8_PEAK_TOPS, "TOP/s", tr)}
        if M > 1:
            # the M = 256 GEMMs multiply on f16 MFMA (exact for these
            # integers), whose dense peak is half the int8 one
            res["M%d" % M]["mfma_f16"] = roofline("mfma", ops_int / t / 1e12, F16_PEAK_TFLOPS, "TFLOP/s")

        # the reference's default path (IDOT4 unset: exact f32 activations,
        # nn/matmul.c:199-253), same weights and inputs
        def step_f32(w):
            return lambda: ops.dense_ffn_i4g(x, w[0][0], w[0][1], w[1][0], w[1][1], w[2][0], w[2][1], idot4=False,
                                             out=y)
        t, n = c.time_steps([step_f32(w) for w in copies], max(32 if M == 1 else 4, steps // (8 if M == 1 else 64)), 4)
        res["M%d_exact_f32" % M] = {"ms_per_step": t * 1e3, "steps": n, "timing": dict(c.last),
                                    "hbm": roofline("hbm", algo / t / 1e9, HBM_PEAK_GBS, "GB/s",
                                                    pmc_traffic("hbm_traffic_pmc", "c3_M%d_exact_f32_step" % M)),
                                    "vector_f32": roofline("valu", 2 * M * 3 * I * D / t / 1e12, F32_PEAK_TFLOPS,
                                                           "TFLOP/s")}
    return {"workload": "C3 8B-dense FFN, grouped int4 g32, D=4096, I=12288, M=1 and M=256: IDOT4=1 (int8 "
                        "activations) and, as M*_exact_f32, the reference default IDOT4 unset (exact f32)", **res}


def bench_q8_gemv_sizes(c, steps, warmup):
    """The C1 decode kernels at larger weight matrices, where the launch
    floor no longer dominates: the Q8 GEMV (k_gemv1_q8, S = 1) on the
    reference's own matmul_q_s benchmark shape 4096 x 4096
    (docs/performance.md:45) and on the 8B FFN's 12288 x 4096, and the fused
    gate/up + SiLU GEMV over the 8B gate and up matrices.  Weights rotate
    past the Infinity Cache like C1's."""
    torch, ops = c.torch, c.ops
    res = {"_cpu": {}}
    for O, I in ((4096, 4096), (12288, 4096)):
        wbytes = O * I + O * 4
        g = c.gen(7, O)
        copies = [c.q8((O, I), g) for _ in range(n_copies(wbytes, target=4800 << 20))]
        x = c.randn((1, I), c.gen(7, 1))
        res["_cpu"]["gemv_%dx%d" % (O, I)] = (x, copies[0], wbytes + (I + O) * 4)
        y = torch.empty((1, O), device="cuda:0")
        t, n = c.time_steps([lambda w=w: ops.matmul_q_s(x, w[0], w[1], out=y) for w in copies], steps, warmup)
        algo = wbytes + (I + O) * 4
        key = "gemv_%dx%d" % (O, I)
        res[key] = {"us": round(t * 1e6, 3),
                    **roofline("hbm", algo / t / 1e9, HBM_PEAK_GBS, "GB/s", pmc_traffic("q8_gemv_large_pmc", key))}
    D, I = 4096, 12288
    wbytes = 2 * (I * D + I * 4)
    g = c.gen(7, 2)
    copies = [c.q8((I, D), g) + c.q8((I, D), g) for _ in range(n_copies(wbytes, target=4800 << 20))]
    x = c.randn((1, D), c.gen(7, 3))
    h = torch.empty((1, I), device="cuda:0")
    t, n = c.time_steps([lambda w=w: ops.gate_up_silu_q8(x, w[0], w[1], w[2], w[3], out=h) for w in copies],
                        steps, warmup)
    algo = wbytes + (D + I) * 4
    res["gate_up_silu_8B"] = {"us": round(t * 1e6, 3),
                              **roofline("hbm", algo / t / 1e9, HBM_PEAK_GBS, "GB/s",
                                         pmc_traffic("q8_gemv_large_pmc", "gate_up_silu_8B"))}
    return {"workload": "Q8 decode GEMV at larger shapes (S = 1): 4096 x 4096, 12288 x 4096, fused gate/up + SiLU "
                        "over 2 x 12288 x 4096", **res}


def bench_c3_r4(c, steps, warmup):
    """The C3 8B-dense FFN shapes in the Q4R4 format (nn/matmul.c:395-431:
    f16 group scales, 4-row blocks, group-32 int8 activations), gate and up
    row-fused as moty_mat_fuse_rows stores them (nn/ffn.c:26-41): M=1
    decode (fused gate/up + SiLU GEMV, down GEMV) and M=256 prefill."""
    torch, ops = c.torch, c.ops
    D, I = 4096, 12288
    wbytes = 3 * (I * D // 2 + I * D // 32 * 2)
    ncopy = n_copies(wbytes)
    g = c.gen(2, 5)
    copies = [ops.pack_r4(c.randn((2 * I, D), g, 0.02)) + ops.pack_r4(c.randn((D, I), g, 0.02))
              for _ in range(ncopy)]
    res = {"_cpu": {"w": copies[0], "x": {}, "I": I}}
    for M in (1, 256):
        x = c.randn((M, D), c.gen(2, 6))
        res["_cpu"]["x"][M] = x
        y = torch.empty((M, D), device="cuda:0")
        t, n = c.time_steps([lambda w=w: ops.dense_ffn_r4(x, w[0], w[1], w[2], w[3], I, out=y) for w in copies],
                            max(32 if M == 1 else 8, steps // (8 if M == 1 else 16)), 8)
        ops_int = 2 * M * 3 * I * D
        algo = wbytes + M * (D + D) * 4
        tr = pmc_traffic("hbm_traffic_pmc", "c3r4_M%d_step" % M)
        res["M%d" % M] = {"ms_per_step": t * 1e3, "steps": n,
                          "hbm": roofline("hbm", algo / t / 1e9, HBM_PEAK_GBS, "GB/s", tr),
                          "mfma": roofline("mfma", ops_int / t / 1e12, INT8_PEAK_TOPS, "TOP/s", tr)}
    return {"workload": "C3 shapes in Q4R4 (f16 group-32 scales, 4-row blocks, gate/up row-fused), D=4096, "
                        "I=12288, M=1 and M=256", **res}


def bench_gguf(c, steps, warmup):
    """Loading GGUF weights on the device (io/gguf.h): the lossless Q4_0 ->
    grouped-int4 repack (runtime/rt_model_load.h:26-34) and the block
    dequantisers, on one 8B-model FFN matrix (12288 x 4096).  Pure byte
    streams: algorithmic bytes = block bytes read + output bytes written."""
    torch, ops = c.torch, c.ops
    O, I = 12288, 4096
    n = O * I
    blk = {4: (32, 34), 5: (32, 18), 6: (256, 144), 7: (256, 176), 8: (256, 210)}
    names = {4: "Q8_0", 5: "Q4_0", 6: "Q4_K", 7: "Q5_K", 8: "Q6_K"}
    g = c.gen(6, 1)
    res = {}

    def raws(dt):
        E, B = blk[dt]
        nb = n // E * B
        return [torch.randint(0, 256, (nb,), generator=g, device="cuda:0", dtype=torch.uint8)
                for _ in range(n_copies(nb + n * 4, lo=3))]

    rs = raws(5)
    res["_cpu"] = {"O": O, "I": I, "raw": {"repack_Q4_0": (5, rs[0])}}
    q4 = [torch.empty((O, I // 2), dtype=torch.uint8, device="cuda:0") for _ in range(2)]
    qs = [torch.empty((O, I // 32), device="cuda:0") for _ in range(2)]
    lib, P = ops.lib(), ops._p  # raw entry points: no output allocation per call
    fns = [lambda r=r, k=k: ops.check(lib.moty_hip_gguf_repack_q4_0_dev(P(r), P(q4[k % 2]), P(qs[k % 2]), O, I,
                                                                        ops._stream()), "repack")
           for k, r in enumerate(rs)]
    t, _ = c.time_steps(fns, steps, warmup)
    algo = n // 32 * (18 + 16 + 4)
    res["repack_Q4_0"] = {"us": round(t * 1e6, 2), "algo_bytes": algo,
                          **roofline("hbm", algo / t / 1e9, HBM_PEAK_GBS, "GB/s")}
    outs = [torch.empty(n, device="cuda:0") for _ in range(2)]
    for dt in sorted(blk):
        rs = raws(dt)
        fns = [lambda r=r, k=k, dt=dt: ops.check(lib.moty_hip_gguf_dequant_dev(dt, P(r), n, P(outs[k % 2]),
                                                                               ops._stream()), "dequant")
               for k, r in enumerate(rs)]
        t, _ = c.time_steps(fns, steps, warmup)
        E, B = blk[dt]
        algo = n // E * B + n * 4
        res["dequant_" + names[dt]] = {"us": round(t * 1e6, 2), "algo_bytes": algo,
                                       **roofline("hbm", algo / t / 1e9, HBM_PEAK_GBS, "GB/s")}
        res["_cpu"]["raw"]["dequant_" + names[dt]] = (dt, rs[0])
        del rs
    return {"workload": "GGUF -> device layouts on a 12288 x 4096 matrix (Q4_0 repack to grouped int4; "
                        "Q8_0/Q4_0/Q4_K/Q5_K/Q6_K dequant to f32)", **res}


def pmc_probe(c):
    """For the rocprofv3 --pmc runs behind roofline.traffic: the C1 gate+up
    GEMV on 8 distinct weight copies (3 rounds), then a plain 64 MiB
    device-to-device copy whose FETCH_SIZE/WRITE_SIZE calibrate the
    counters (64 MiB read, 64 MiB written)."""
    torch, ops = c.torch, c.ops
    D, I = 1024, 3072
    g = c.gen(0, 1)
    copies = [c.q8((I, D), g) + c.q8((I, D), g) for _ in range(8)]
    x = c.randn((1, D), c.gen(0, 2))
    h = torch.empty((1, I), device="cuda:0")
    src = torch.randint(0, 255, (64 << 20,), dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        for w in copies:
            ops.gate_up_silu_q8(x, w[0], w[1], w[2], w[3], out=h)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("pmc probe done")


# --------------------------------------------------------------------------
def cpu_med(fn, budget, nmin=20, warm=3):
    """Median wall time of fn over at least nmin runs after `warm` warm-ups
    (CLOCK_MONOTONIC around the call, as c/tests/bench.c), stopping early
    only past `budget` seconds with 3 runs done; returns (seconds, runs)."""
    import numpy as np
    for _ in range(warm):
        fn()
    ts = []
    t0 = time.perf_counter()
    while len(ts) < nmin:
        a = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - a)
        if time.perf_counter() - t0 > budget and len(ts) >= 3:
            break
    return float(np.median(ts)), len(ts)


class CpuRef:
    """The reference's own kernels (oracle/_ref, built from the reference's
    sources, kind 'reference': the int8-activation library and the exact
    IDOT4=0 one), or the oracle restatement ('port') where that build is
    absent, timed on the host cores with moty's OpenMP tuning."""

    def __init__(self):
        import numpy as np
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import cpu_libs as cl
        self.np, self.cl = np, cl
        self.r = cl.ref(True)
        self.r32 = cl.ref(False)
        self.kind = "reference" if self.r is not None else "port"
        self.cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))

    def out(self, value, unit, sample, runs, cores=None, warm=3):
        return {"value": value, "unit": unit, "cores": cores or self.cores, "kind": self.kind,
                "sample": "%s; median of %d runs after %d warm-up%s" % (sample, runs, warm, "" if warm == 1 else "s")}

    def q_s(self, y, x, q, s):
        S, I = x.shape
        O = q.shape[0]
        if self.r is not None:
            self.r.ref_matmul_q_s(self.cl.ptr(y), self.cl.ptr(x), self.cl.ptr(q), self.cl.ptr(s), S, I, O)
        else:
            y[...] = self.cl.o_matmul_q_s(x, q, s)

    def i4g(self, y, x, q4, s, idot4):
        S, I = x.shape
        O = q4.shape[0]
        r = self.r if idot4 else self.r32
        if r is not None:
            r.ref_matmul_i4_grouped_s(self.cl.ptr(y), self.cl.ptr(x), self.cl.ptr(q4), self.cl.ptr(s), S, I, O, 32)
        else:
            y[...] = self.cl.o_matmul_i4g(x, q4, s, idot4)

    def silu(self, g, u):
        if self.r is not None:
            self.r.ref_silu_mul(self.cl.ptr(g), self.cl.ptr(u), g.size)
        else:
            self.cl.oracle().o_silu_mul(self.cl.ptr(g), self.cl.ptr(u), g.size)

    def moe(self, out, x, Wr, ws, E, K, I, D, order, norm, cap=0):
        cl, T = self.cl, x.shape[0]
        if self.r is not None:
            if order == "batch":
                self.r.ref_moe_batch_cap(cl.ptr(out), cl.ptr(x), T, cl.ptr(Wr), *[cl.ptr(a) for a in ws], E, K, I,
                                         D, cap or E)
            else:
                i2 = self.np.empty((T, K), self.np.int32)
                self.r.ref_moe_olmoe(cl.ptr(out), cl.ptr(x), T, cl.ptr(Wr), *[cl.ptr(a) for a in ws], E, K, I, D,
                                     norm, cl.ptr(i2))
        else:
            out[...] = cl.o_moe(x, Wr, dict(zip(("G", "GS", "U", "US", "Dn", "DS"), ws)), K, order, norm=norm)[0]


def cpu_c1(cr, c1, budget):
    np = cr.np
    x = c1["x"].cpu().numpy()
    G, GS, U, US, Dn, DS = [t.cpu().numpy() for t in c1["w0"]]
    D, I = 1024, 3072
    g, u, y = np.empty((1, I), np.float32), np.empty((1, I), np.float32), np.empty((1, D), np.float32)

    def ffn():
        cr.q_s(g, x, G, GS)
        cr.q_s(u, x, U, US)
        cr.silu(g, u)
        cr.q_s(y, g, Dn, DS)
    t, n = cpu_med(ffn, budget)
    return cr.out(round(c1["algo_bytes"] / t / 1e9, 2), "GB/s", "C1 decode FFN (3 matmul_q_s + silu_mul)", n)


MOE_WARM = 1  # warm-up runs of a CPU MoE layer (each is a whole layer)


def cpu_moe(cr, r, T_sample, order, norm, budget, nmin=20, skew=None, cap=0):
    """r: a bench_moe result (its first weight copy and inputs); skew: hot
    expert ids whose logits the inputs lift by +2.0 (the reference's batch
    layer takes no logit bias: cpu_libs.skew_inputs expresses it in x and
    the router); cap: expert-cache slots (0: every expert resident)."""
    np = cr.np
    lay = r["layer0"]
    xs = np.ascontiguousarray(r["x"].cpu().numpy()[:T_sample])
    Wr = r["Wr"].cpu().numpy()
    if skew is not None:
        xs, Wr = cr.cl.skew_inputs(xs, Wr, skew)
    ws = [t.cpu().numpy() for t in lay.keep[1:7]]
    out = np.empty((T_sample, lay.D), np.float32)
    t, n = cpu_med(lambda: cr.moe(out, xs, Wr, ws, lay.E, lay.K, lay.I, lay.D, order, norm, cap), budget,
                   nmin=nmin, warm=MOE_WARM)
    return T_sample / t, n


def cpu_moe_d1(cr, r, budget):
    np, cl = cr.np, cr.cl
    lay = r["layer0"]
    x = np.ascontiguousarray(r["x"].cpu().numpy())
    Wr = r["Wr"].cpu().numpy()
    ws = [t.cpu().numpy() for t in lay.keep[1:7]]
    out = np.empty((1, lay.D), np.float32)
    if cr.r is not None:
        fn = lambda: cr.r.ref_moe_d1(cl.ptr(out), cl.ptr(x), cl.ptr(Wr), *[cl.ptr(a) for a in ws], lay.E, lay.K,
                                     lay.I, lay.D)
    else:
        fn = lambda: cl.o_moe(x, Wr, dict(zip(("G", "GS", "U", "US", "Dn", "DS"), ws)), lay.K, "olmoe", norm=1)
    t, n = cpu_med(fn, budget)
    return cr.out(round(t * 1e6, 1), "us/token", "moty_nn_moe_topk_d1 (nn/moe.c:33-153), one token", n)


def cpu_c2(cr, c2, budget):
    np = cr.np
    d = c2["_cpu"]
    xs = {I: d["x"][I].cpu().numpy() for I in d["x"]}
    ws = [(q.cpu().numpy(), s.cpu().numpy()) for q, s in d["w"]]
    ys = [np.empty((x.shape[0], q.shape[0]), np.float32) for x, (q, _) in zip(xs.values(), ws)]

    def step():  # the same three calls (fused q/k/v/gate/up rows, o, down)
        for (I, x), (q, s), y in zip(xs.items(), ws, ys):
            cr.q_s(y, x, q, s)
    t, n = cpu_med(step, budget)
    return cr.out(round(d["ops_int"] / t / 1e12, 4), "TOP/s", "C2 seven projections at M=512 (3 matmul_q_s calls)", n)


def cpu_c3(cr, c3, budget):
    np = cr.np
    d = c3["_cpu"]
    (gq, gs), (uq, us), (dq, ds) = [(q.cpu().numpy(), s.cpu().numpy()) for q, s in d["w"]]
    res = {}
    for M, xt in d["x"].items():
        x = xt.cpu().numpy()
        D, I = x.shape[1], gq.shape[0]
        g, u, y = np.empty((M, I), np.float32), np.empty((M, I), np.float32), np.empty((M, D), np.float32)
        for idot4 in (True, False):
            def ffn():
                cr.i4g(g, x, gq, gs, idot4)
                cr.i4g(u, x, uq, us, idot4)
                cr.silu(g, u)
                cr.i4g(y, g, dq, ds, idot4)
            t, n = cpu_med(ffn, budget / 4)
            res["M%d_%s" % (M, "idot4" if idot4 else "exact_f32")] = cr.out(
                round(t * 1e3, 3), "ms/step", "C3 FFN M=%d (matmul_i4_grouped_s x3 + silu_mul, IDOT4=%d)" % (
                    M, int(idot4)), n)
    return res


def cpu_q8_sizes(cr, r, budget):
    np = cr.np
    res = {}
    for key, (x, (q, s), algo) in r["_cpu"].items():
        xh, qh, sh = x.cpu().numpy(), q.cpu().numpy(), s.cpu().numpy()
        y = np.empty((1, qh.shape[0]), np.float32)
        t, n = cpu_med(lambda: cr.q_s(y, xh, qh, sh), budget / 2)
        res[key] = cr.out(round(algo / t / 1e9, 2), "GB/s", "matmul_q_s S=1 " + key, n)
    return res


def cpu_r4(cr, r, budget):
    """moty_matmul_q4r4_s over the row-fused gate_up, silu_rows, down (the
    reference's dense FFN with a fused gate_up, nn/ffn.c:26-41)."""
    np, cl = cr.np, cr.cl
    d = r["_cpu"]
    gu, gus, dn, dns = [t.cpu().numpy() for t in d["w"]]
    I = d["I"]
    res = {}
    for M, xt in d["x"].items():
        x = xt.cpu().numpy()
        D = x.shape[1]
        g = np.empty((M, 2 * I), np.float32)
        h = np.empty((M, I), np.float32)
        y = np.empty((M, D), np.float32)

        def ffn():
            if cr.r is not None:
                cr.r.moty_matmul_q4r4_s(cl.ptr(g), cl.ptr(x), cl.ptr(gu), cl.ptr(gus), M, D, 2 * I)
            else:
                g[...] = cl.o_matmul_r4(x, gu, gus, 2 * I)
            h[...] = g[:, :I]
            cr.silu(h, np.ascontiguousarray(g[:, I:]))
            if cr.r is not None:
                cr.r.moty_matmul_q4r4_s(cl.ptr(y), cl.ptr(h), cl.ptr(dn), cl.ptr(dns), M, I, D)
            else:
                y[...] = cl.o_matmul_r4(h, dn, dns, D)
        t, n = cpu_med(ffn, budget / 2)
        res["M%d" % M] = cr.out(round(t * 1e3, 3), "ms/step", "Q4R4 FFN M=%d (moty_matmul_q4r4_s x2 over the fused "
                                "gate_up and down, silu_mul)" % M, n)
    return res


def cpu_gguf(cr, r, budget):
    """io/gguf.h's gguf_repack_q4_0 / gguf_dequant (compiled into oracle/_ref
    from the reference tree) on the same blocks; GB/s of block bytes read +
    output bytes written, as the GPU lines."""
    np, cl = cr.np, cr.cl
    d = r["_cpu"]
    O, I = d["O"], d["I"]
    n = O * I
    res = {}
    for key, (dt, raw) in d["raw"].items():
        rh = raw.cpu().numpy()
        if dt == 5 and key.startswith("repack"):
            q4, qs = np.empty(n // 2, np.uint8), np.empty(n // 32, np.float32)
            fn = (lambda: cr.r.ref_gguf_repack_q4_0(cl.ptr(rh), cl.ptr(q4), cl.ptr(qs), O, I)) if cr.r else (
                lambda: cl.o_gguf_repack_q4_0(rh, O, I))
        else:
            out = np.empty(n, np.float32)
            fn = (lambda: cr.r.ref_gguf_dequant(dt, cl.ptr(rh), n, cl.ptr(out))) if cr.r else (
                lambda: cl.o_gguf_dequant(dt, rh, n))
        t, runs = cpu_med(fn, budget / 6, nmin=5, warm=1)
        res[key] = cr.out(round(r[key]["algo_bytes"] / t / 1e9, 2), "GB/s", "io/gguf.h %s, one thread" % key, runs,
                          cores=1)
    return res


def cpu_baseline(c1, c4, extra, budget):
    """Every config's reference CPU path on the host cores; returns the C1
    object and attaches the others to their lines."""
    import numpy as np
    cr = CpuRef()
    out = cpu_c1(cr, c1, min(3.0, budget))
    if c4 is not None:
        tpo, n1 = cpu_moe(cr, c4, 256, "olmoe", 0, budget, nmin=3)
        tpb, n2 = cpu_moe(cr, c4, 256, "batch", 1, budget)
        out["moe"] = cr.out(round(tpb, 1), "tokens/s", "C4 OLMoE layer through moe_batch_core (nn/moe.c:159-205), "
                            "all 256 tokens", n2, warm=MOE_WARM)
        out["moe"]["olmoe_per_token"] = cr.out(round(tpo, 1), "tokens/s", "the olmoe engine's per-token moe() "
                                               "(engines/olmoe.c:219-244), all 256 tokens", n1, warm=MOE_WARM)
    for r in extra:
        w = r.get("workload", "")
        try:
            if w.startswith("C2"):
                r["cpu_baseline"] = cpu_c2(cr, r, budget)
            elif w.startswith("C3 8B"):
                r["cpu_baseline"] = cpu_c3(cr, r, budget)
            elif w.startswith("C3 shapes in Q4R4"):
                r["cpu_baseline"] = cpu_r4(cr, r, budget)
            elif w.startswith("Q8 decode GEMV"):
                r["cpu_baseline"] = cpu_q8_sizes(cr, r, budget)
            elif w.startswith("GGUF"):
                r["cpu_baseline"] = cpu_gguf(cr, r, budget)
            elif w.startswith("Decode MoE"):
                r["cpu_baseline"] = cpu_moe_d1(cr, r, budget)
            elif w.startswith("C5"):
                sk = "skewed" in w
                tp, n = cpu_moe(cr, r, 1072, "batch", 1, budget, nmin=3,
                                skew=np.arange(0, 128, 16) if sk else None)
                r["cpu_baseline"] = cr.out(round(tp, 1), "tokens/s", "C5 layer through moe_batch_core, all 1072 "
                                           "tokens of the batch%s" % (
                                               "; skew as +2.0 on the hot experts' logits through x and the router"
                                               if sk else ""), n, warm=MOE_WARM)
            elif w.startswith("C4 MoE layer shape through the device expert cache") and c4 is not None:
                res = {}
                for cap in (64, 32):
                    tp, n = cpu_moe(cr, c4, 256, "batch", 1, budget / 2, cap=cap, nmin=5)
                    res["cap%d" % cap] = cr.out(round(tp, 1), "tokens/s", "C4 batch layer over the reference's "
                                                "ExpertCache (runtime/moecache.c) with %d slots, all 256 tokens" % cap, n,
                                                warm=MOE_WARM)
                r["cpu_baseline"] = res
        except Exception as e:  # the baseline is reported, never required
            log("cpu baseline for %s failed: %s" % (w[:20], e))
    return out


# --------------------------------------------------------------------------
def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU: every box in this pool has a single MI355X, so --gpus %d is not "
              "supported. Run with --gpus 1." % args.gpus, file=sys.stderr)
        sys.exit(2)
    import torch
    import moty_amd
    from moty_amd import ops
    moty_amd.lib()
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    c = Ctx(torch, ops)
    if args.pmc_probe:
        pmc_probe(c)
        return
    if args.only:
        one = {"c1": lambda: bench_c1(c, args.steps, args.warmup),
               "floor": floor_probe,
               "d1": lambda: bench_moe_d1(c, 5, 64, 8, 1024, 2048, args.steps, args.warmup, "Decode MoE S=1, C4 shape"),
               "c2": lambda: bench_c2(c, args.steps, args.warmup),
               "c3": lambda: bench_c3(c, args.steps, args.warmup),
               "c3r4": lambda: bench_c3_r4(c, args.steps, args.warmup),
               "q8gemv": lambda: bench_q8_gemv_sizes(c, args.steps, args.warmup),
               "c4": lambda: bench_moe(c, 3, 256, 64, 8, 1024, 2048, 0, moty_amd.ORDER_TOPK, args.steps,
                                       args.warmup, label="C4 OLMoE MoE layer Q8, T=256", traffic_key="c4_layer"),
               "c5": lambda: bench_moe(c, 4, 1072, 128, 8, 768, 2048, 1, moty_amd.ORDER_EXPERT, args.steps,
                                       args.warmup, label="C5 Qwen3-30B-A3B MoE layer Q8, T=1072, uniform",
                                       traffic_key="c5_layer"),
               "c5s": lambda: bench_moe(c, 4, 1072, 128, 8, 768, 2048, 1, moty_amd.ORDER_EXPERT, args.steps,
                                        args.warmup, bias=c5_skew_bias(),
                                        label="C5 Qwen3-30B-A3B MoE layer Q8, T=1072, " + C5_SKEW_LABEL,
                                        traffic_key="c5s_layer")}[args.only]()
        print(json.dumps({k2: v for k2, v in one.items() if k2 not in HIDDEN}), flush=True)
        return

    log("C1 decode FFN")
    c1 = bench_c1(c, args.steps, args.warmup)
    log("C1: %.1f GB/s, %.2f us/step; gate/up kernel %.2f us (%.1f GB/s)" % (
        c1["gbs"], c1["ms_per_step"] * 1e3, c1["kernel"]["us"], c1["kernel"]["gbs"]))
    log("C4 OLMoE MoE T=256")
    c4 = bench_moe(c, 3, 256, 64, 8, 1024, 2048, 0, moty_amd.ORDER_TOPK, args.steps, args.warmup,
                   label="C4 OLMoE MoE layer Q8, T=256, E=64, top-8 softmax (norm_topk_prob=false), I=1024, D=2048",
                   traffic_key="c4_layer")
    log("C4: %.0f tokens/s, %.3f ms/layer" % (c4["tokens_per_s"], c4["ms_per_layer"]))
    extra = []
    if not args.quick:
        log("Q8 GEMV at larger shapes")
        extra.append(bench_q8_gemv_sizes(c, args.steps, args.warmup))
        log("C2")
        extra.append(bench_c2(c, args.steps, args.warmup))
        log("C3")
        extra.append(bench_c3(c, args.steps, args.warmup))
        log("C3 in Q4R4")
        extra.append(bench_c3_r4(c, args.steps, args.warmup))
        log("decode MoE (S = 1)")
        extra.append(bench_moe_d1(c, 5, 64, 8, 1024, 2048, args.steps, args.warmup,
                                  "Decode MoE S=1 (moty_nn_moe_topk_d1), C4 expert shape: E=64, top-8, I=1024, D=2048"))
        extra.append(bench_moe_d1(c, 6, 128, 8, 768, 2048, args.steps, args.warmup,
                                  "Decode MoE S=1 (moty_nn_moe_topk_d1), C5 expert shape: E=128, top-8, I=768, D=2048"))
        log("C4 through the expert cache")
        extra.append(bench_moe_cached(c, args.steps))
        log("GGUF loading")
        extra.append(bench_gguf(c, args.steps, args.warmup))
        log("C5")
        for b, lab in ((None, "uniform"), (c5_skew_bias(), C5_SKEW_LABEL)):
            r5 = bench_moe(c, 4, 1072, 128, 8, 768, 2048, 1, moty_amd.ORDER_EXPERT, args.steps, args.warmup, bias=b,
                           label="C5 Qwen3-30B-A3B MoE layer Q8, T=1072 ragged batch (48 decode + 1024 prefill), "
                                 "E=128, top-8, I=768, D=2048, " + lab, traffic_key="c5_layer" if b is None else "c5s_layer")
            extra.append(r5)
    cpu = None
    if not args.no_cpu:
        log("CPU baseline")
        try:
            cpu = cpu_baseline(c1, c4, extra, args.cpu_seconds)
        except Exception as e:  # the baseline is reported, never required
            log("cpu baseline failed:", e)
    for r in extra:
        for k in HIDDEN:
            r.pop(k, None)
    k = c1["kernel"]
    fl = floor_probe()
    moe = {k2: v for k2, v in c4.items() if k2 not in HIDDEN}
    moe["metric"] = "MoE layer tokens/s at T=256 (1 GPU)"
    moe["value"] = round(moe.pop("tokens_per_s"), 1)
    moe["unit"] = "tokens/s"
    if cpu and "moe" in cpu:
        moe["cpu_baseline"] = cpu.pop("moe")
    line = {
        "metric": METRIC, "value": round(c1["gbs"], 2), "unit": "GB/s", "n_gpus": 1,
        "steps": c1["steps"], "warmup": args.warmup, "ms_per_step": round(c1["ms_per_step"], 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (W ~ N(0,0.02) quantized by the library's QBITS=8 kernels, x ~ N(0,1)); "
                "weights rotate over %d copies" % c1["weight_copies"],
        "config": {"workload": c1["workload"]},
        "roofline": dict(roofline("hbm", k["gbs"], HBM_PEAK_GBS, "GB/s", pmc_traffic("hbm_traffic_pmc", "c1_gate_up")),
                         kernel=k["name"], kernel_us=round(k["us"], 3), algo_bytes=k["algo_bytes"],
                         timing="HIP events around graph replays of the kernel alone (weights rotating "
                                "over the copies), elapsed / launches, median of the replays",
                         floor_us=fl.get("read_6332416B_us")),
        "whole_ffn_roofline": dict(roofline("hbm", c1["gbs"], HBM_PEAK_GBS, "GB/s",
                                            pmc_traffic("hbm_traffic_pmc", "c1_step")),
                                   floor_us=fl.get("read_pair_6332416B_3170304B_us"),
                                   one_launch_floor_us=fl.get("read_9474048B_us")),
        "timing": c1["timing"],
        "one_launch_us": c1["one_launch_us"],
        "floors": fl,
        "cpu_baseline": cpu,
        "moe": moe,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
