#!/usr/bin/env python3
"""Benchmark of the resident-weight matmul hot path on one MI355X, through the drop-in C-ABI.

Metric: "w8a8 M=1 GEMV HBM GB/s (% peak); M=512 int8 GEMM TOPS (% MFMA peak)".
Workload (BASELINE config 1 shape): W f32[6144][2048] ~ N(0,0.02) seeded, packed once with
ork_i8_mm_pack_f32 (per-channel int8); A int8 ~ U[-127,127]; C int32. A step is one ork_i8_mm_run
call (M=1 for the headline value). The weight is packed into R=64 resident copies (64 x 12.6 MB =
805 MB > 3 x the 256 MB MALL) and consecutive steps rotate through them; when fewer steps than copies
are timed, the copies outside the timed set are streamed by the same kernel just before the timed
replay. Either way every timed step reads a weight that was last read more than 2 x MALL (512 MB) of
other weights earlier, so it streams from HBM. A and C live in HBM (ork_dev_alloc); the steps are
captured into one HIP graph and timed with HIP events on the library's stream, bracketed by device
synchronisation.

Also reported on the same line: the M=512 int8 GEMM (TOPS, % of dense int8 MFMA peak) as "m512",
the eager (non-graph) launch rate, the reference's own calling convention (host A and C, one
synchronous call per step, PCIe and sync included) as "host_api", and the CPU baseline: the reference's own CPU GEMM
(orki_cpu_gemm_i32, compiled from its sources into oracle/_ref) timed on the host, single-threaded
as the reference builds it, on a bounded sample of the same workload.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ork-driver_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

K, N = 2048, 6144
R = 64                          # rotated resident weight copies (64 x 12.6 MB = 805 MB)
MALL_BYTES = 256 << 20          # MI355X Infinity Cache
HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, GB/s
INT8_PEAK_TOPS = 5000.0         # MI355X dense int8 MFMA, TOP/s
WARM_S = 0.05                   # untimed replays of a timed graph before its timed replay (steady state)
EAGER_ONLY = False              # --eager-only: no graphs, events or other HIP calls from Python (profiler runs)
FP16_PEAK_TFLOPS = 2500.0       # MI355X dense fp16 MFMA, TFLOP/s


def algo_bytes(M):
    return K * N + M * K + 4 * M * N


def algo_ops(M):
    return 2 * M * N * K


class Hip:
    """The few HIP runtime calls the timing needs (graph capture, events), via ctypes."""

    def __init__(self):
        self.L = C.CDLL("libamdhip64.so")
        for n in ("hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate", "hipGraphLaunch",
                  "hipEventCreate", "hipEventRecord", "hipEventSynchronize", "hipEventElapsedTime",
                  "hipDeviceSynchronize", "hipGraphExecDestroy", "hipGraphDestroy", "hipEventDestroy"):
            getattr(self.L, n).restype = C.c_int

    def ck(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: {rc}")

    def event(self):
        e = C.c_void_p()
        self.ck(self.L.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e

    def capture(self, stream, fn):
        g = C.c_void_p()
        ex = C.c_void_p()
        self.ck(self.L.hipStreamBeginCapture(C.c_void_p(stream), 0), "hipStreamBeginCapture")
        fn()
        self.ck(self.L.hipStreamEndCapture(C.c_void_p(stream), C.byref(g)), "hipStreamEndCapture")
        self.ck(self.L.hipGraphInstantiate(C.byref(ex), g, None, None, C.c_size_t(0)), "hipGraphInstantiate")
        return g, ex

    def time_ms(self, stream, launch):
        e0, e1 = self.event(), self.event()
        self.ck(self.L.hipDeviceSynchronize(), "sync")
        self.ck(self.L.hipEventRecord(e0, C.c_void_p(stream)), "record")
        launch()
        self.ck(self.L.hipEventRecord(e1, C.c_void_p(stream)), "record")
        self.ck(self.L.hipEventSynchronize(e1), "event sync")
        self.ck(self.L.hipDeviceSynchronize(), "sync")
        ms = C.c_float()
        self.ck(self.L.hipEventElapsedTime(C.byref(ms), e0, e1), "elapsed")
        self.L.hipEventDestroy(e0)
        self.L.hipEventDestroy(e1)
        return ms.value


def measure(npu, hip, ws, M, dA, dC, steps, warmup, entry="ork_i8_mm_run", scales=None, outer=None, call=None):
    """Returns (graph ms/step, eager ms/step). Step i runs weight ws[i % len(ws)] through `entry` (or, given
    `call`, runs call(ws[i % len(ws)])); the
    grouped entry points also take the device scale buffers `scales` = (aScale, bScale). With fewer timed
    steps than weights, a second graph streams the weights outside the timed set (ws[steps:]) right before
    the timed replay, so the timed weights are as cold as in a full rotation.
    Before the timed replay the graph is replayed untimed for WARM_S seconds (steady state).
    The graph ms/step is timed on the device: the graph's first and last nodes write the GPU wall clock
    (ork_npu_mark), so the timed region is exactly the `steps` steps; the host's submission of the graph (one per
    replay) falls outside it. The same replay is also timed by events recorded around the graph launch; that
    launch-inclusive ms/step goes to outer[0] when a list is given."""
    import ork

    L = ork.lib()
    stream = L.ork_npu_stream(npu.h)
    fn = getattr(L, entry)
    mid = tuple(scales) if scales else ()

    def run(i):
        rc = call(ws[i % len(ws)]) if call else fn(npu.h, ws[i % len(ws)], M, dA, *mid, dC)
        if rc:
            raise RuntimeError(f"{entry} rc={rc}")

    # eager: warmup, then steps individually launched (host launch rate included)
    for i in range(warmup):
        run(i)
    if EAGER_ONLY:
        # profiler runs: only the library's own calls reach the HIP runtime (host clock around the launches and
        # the library's stream sync); the profiler's per-dispatch durations are what such a run is for
        assert L.ork_npu_sync(npu.h) == 0
        t0 = time.perf_counter()
        for i in range(steps):
            run(i)
        assert L.ork_npu_sync(npu.h) == 0
        ms = (time.perf_counter() - t0) * 1e3 / steps
        return ms, ms
    eager = hip.time_ms(stream, lambda: [run(i) for i in range(steps)]) / steps
    # graph: timestamp node, exactly `steps` launches, timestamp node; warm it, stream the other weights, then time
    # one replay
    ts = L.ork_dev_alloc(npu.h, 16)
    assert ts

    def body():
        if L.ork_npu_mark(npu.h, ts) or any(run(i) for i in range(steps)) or L.ork_npu_mark(npu.h, ts + 8):
            raise RuntimeError("ork_npu_mark failed")

    g, ex = hip.capture(stream, body)
    hip.ck(hip.L.hipGraphLaunch(ex, C.c_void_p(stream)), "hipGraphLaunch")
    # untimed replays until the GPU has run this step for WARM_S: the first milliseconds of a step after other
    # work (or idle) run slower than its steady state (int8 M=512: 14.2-14.9 us/step on a first replay, 13.5 from
    # the second on; the M=1 GEMV is steady at once). The stream-out of the other weights below still comes last.
    t_end = time.perf_counter() + WARM_S
    while time.perf_counter() < t_end:
        hip.ck(hip.L.hipGraphLaunch(ex, C.c_void_p(stream)), "hipGraphLaunch")
        hip.ck(hip.L.hipDeviceSynchronize(), "sync")
    flush = None
    if steps < len(ws):
        flush = hip.capture(stream, lambda: [run(i) for i in range(steps, len(ws))])
        hip.ck(hip.L.hipGraphLaunch(flush[1], C.c_void_p(stream)), "hipGraphLaunch")
    launch_incl = hip.time_ms(stream, lambda: hip.ck(hip.L.hipGraphLaunch(ex, C.c_void_p(stream)), "hipGraphLaunch"))
    inner = graph_stamps_ms(npu, L, ts)
    if not (0.0 < inner <= launch_incl * 1.001):
        raise RuntimeError(f"in-graph timing {inner} ms outside (0, {launch_incl}] ms")
    for gg, ee in [(g, ex)] + ([flush] if flush else []):
        hip.L.hipGraphExecDestroy(ee)
        hip.L.hipGraphDestroy(gg)
    L.ork_dev_free(npu.h, ts)
    if outer is not None:
        outer.append(launch_incl / steps)
    return inner / steps, eager


def measure_marks(npu, hip, L, dA, dC, steps, warmup):
    """ms per step of measure()'s graph harness around ork_npu_mark alone (one one-thread kernel writing the wall
    clock): the per-dispatch floor of a launch that does no work, beside the K=32, N=32 GEMV's."""
    slot = L.ork_dev_alloc(npu.h, 256)
    assert slot
    ms, _ = measure(npu, hip, [slot], 1, dA, dC, steps, warmup, call=lambda p: L.ork_npu_mark(npu.h, p))
    L.ork_dev_free(npu.h, slot)
    return ms


def graph_stamps_ms(npu, L, ts):
    """ms between the two wall-clock stamps (ork_npu_mark) the timed graph wrote to ts[0], ts[1]."""
    import ork

    t = np.zeros(2, np.uint64)
    assert L.ork_dev_download(npu.h, ork.ptr(t), ts, 16) == 0
    khz = L.ork_npu_wallclock_khz(npu.h)
    if khz <= 0 or t[1] <= t[0]:
        raise RuntimeError(f"bad wall-clock stamps {t} at {khz} kHz")
    return float(t[1] - t[0]) / khz


def cold_distance(ws_bytes, n_ws, steps):
    """Bytes of other weights read between a timed weight's previous read and its timed read."""
    return (n_ws - 1) * ws_bytes if steps >= n_ws else (n_ws - steps) * ws_bytes


def measure_copy(hip, L, npu, nbytes, steps, warmup=8):
    """ms per device-to-device copy of nbytes (hipMemcpyAsync: the runtime's copy kernel, nbytes read + nbytes
    written), graph-timed like measure() over R rotated source buffers: the data-movement reference beside the
    GEMV, which reads the same nbytes of weight."""
    stream = L.ork_npu_stream(npu.h)
    bufs = [L.ork_dev_alloc(npu.h, nbytes) for _ in range(R)]
    dst = L.ork_dev_alloc(npu.h, nbytes)
    assert all(bufs) and dst
    hip.L.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]

    def run(i):
        hip.ck(hip.L.hipMemcpyAsync(C.c_void_p(dst), C.c_void_p(bufs[i % R]), nbytes, 3, C.c_void_p(stream)),
               "hipMemcpyAsync")

    for i in range(warmup):
        run(i)
    g, ex = hip.capture(stream, lambda: [run(i) for i in range(steps)])
    hip.ck(hip.L.hipGraphLaunch(ex, C.c_void_p(stream)), "hipGraphLaunch")
    if steps < R:
        fl = hip.capture(stream, lambda: [run(i) for i in range(steps, R)])
        hip.ck(hip.L.hipGraphLaunch(fl[1], C.c_void_p(stream)), "hipGraphLaunch")
    ms = hip.time_ms(stream, lambda: hip.ck(hip.L.hipGraphLaunch(ex, C.c_void_p(stream)), "hipGraphLaunch")) / steps
    hip.L.hipGraphExecDestroy(ex)
    hip.L.hipGraphDestroy(g)
    for b in bufs + [dst]:
        L.ork_dev_free(npu.h, b)
    return ms


def measure_read(npu, hip, L, ws, dA, dC, steps, warmup):
    """ms per plain streaming read of a weight's panel bytes (ork_npu_read_probe: the M = 1 GEMV's loads without its
    arithmetic), in measure()'s graph harness over the same rotation: what reading the bytes alone costs per launch.
    The probe's XOR words of the first weight are checked against the host's XOR of its panel bytes."""
    import ork

    sink = L.ork_dev_alloc(npu.h, 1 << 20)
    assert sink
    pan = []
    for w in ws:
        p, kb, kind, lut = C.c_void_p(), C.c_int(), C.c_int(), (C.c_uint32 * 4)()
        kk, nn = C.c_int(), C.c_int()
        L.ork_w_dims(w, C.byref(kk), C.byref(nn))
        assert L.ork_w_device_panels(w, C.byref(p), C.byref(kb), C.byref(kind), lut) == 0
        pan.append((p.value, (nn.value // 16) * kb.value * 1024))
    nb = pan[0][1]
    host = np.empty(nb, np.uint8)
    assert L.ork_dev_download(npu.h, ork.ptr(host), pan[0][0], nb) == 0
    n = L.ork_npu_read_probe(npu.h, pan[0][0], nb, sink)
    assert n > 0 and L.ork_npu_sync(npu.h) == 0
    words = np.empty(n, np.uint32)
    assert L.ork_dev_download(npu.h, ork.ptr(words), sink, 4 * n) == 0
    assert np.bitwise_xor.reduce(words) == np.bitwise_xor.reduce(host.view(np.uint32)), "read probe missed bytes"
    ms, _ = measure(npu, hip, pan, 1, dA, dC, steps, warmup, call=lambda pb: 0 if L.ork_npu_read_probe(
        npu.h, pb[0], pb[1], sink) > 0 else 1)
    L.ork_dev_free(npu.h, sink)
    return ms


def cpu_rows_baseline(fn_rows, M, nbytes, ops, bound, kind, what, budget_s):
    """One config's CPU baseline in the config's own unit: fn_rows(r) runs the CPU GEMM on the first r rows of
    the config's A. The reference's CPU GEMMs treat rows independently (a k-outer AXPY per row, or a row loop), so
    a bounded sample of min(M, 16) rows is timed for ~budget_s seconds and scaled to M rows."""
    r = min(M, 16)
    dt, n = _time_calls(lambda: fn_rows(r), budget_s)
    full = dt * M / r
    if bound == "hbm":
        value, unit = nbytes / full / 1e9, "GB/s"
    else:
        value, unit = ops / full / 1e12, ("TOP/s" if bound == "mfma_int8" else "TFLOP/s")
    scaled = f", scaled to M={M}" if r != M else ""
    return {"value": round(value, 6), "unit": unit, "cores": 1, "kind": kind,
            "sample": f"{n} calls of {r} row(s): {what}, 1 thread, {dt * 1e3:.2f} ms/call{scaled}; host {cpu_model()}"}


def sweep_configs(npu, hip, L, ws_c1, dA, dC, codes1, A512, cpu_s, only=None):
    """BASELINE configs 1-4 at their stated shapes, measured like the headline (one HIP graph of
    rotating resident weights, >= 2x the 256 MB MALL, A and C in HBM): throughput and roofline fraction
    per config. Each result is spot-checked against the oracle on a few rows. With cpu_s > 0 each config
    also carries its CPU baseline (cpu_rows_baseline, ~cpu_s seconds): the reference's own orki_cpu_gemm_i32 /
    orki_cpu_gemm_grouped from oracle/_ref for the integer kinds, the oracle's restatement of the reference's
    fp32-accumulate loop (examples/test_matmul.c:37) for fp16."""
    import ork
    import oracle as O

    rng = np.random.default_rng(0x6F726B00 + (9 << 8))
    out = []

    def want(name):
        """Sections to run (profiling runs select some); the grouped section reuses config 4's operands."""
        return only is None or name in only or (name == "c4" and "grouped" in only)
    have_ref = O.ref_available()
    gemm = O.ref_gemm_i32 if have_ref else O.gemm_i32
    gkind = "reference" if have_ref else "port"
    gwhat = "orki_cpu_gemm_i32 as built (-O2)" if have_ref else "oracle restatement of orki_cpu_gemm_i32"

    def rec(name, plan, M, ms, nbytes, ops, bound, cpu=None):
        us = ms * 1e3
        if bound == "hbm":
            val, unit, peak = nbytes / (ms * 1e-3) / 1e9, "GB/s", HBM_PEAK_GBS
        else:
            val, unit, peak = ops / (ms * 1e-3) / 1e12, "TOP/s" if bound == "mfma_int8" else "TFLOP/s", \
                (INT8_PEAK_TOPS if bound == "mfma_int8" else FP16_PEAK_TFLOPS)
        out.append({"config": name, "M": M, "kernel": plan, "us_per_call": round(us, 3), "value": round(val, 1),
                    "unit": unit, "roofline": {"bound": "hbm" if bound == "hbm" else "mfma", "peak": peak,
                                               "frac": round(val / peak, 4)}})
        print(f"[bench] {name} M={M}: {us:.2f} us ({val:.1f} {unit}, {val / peak:.1%} of peak) {plan}",
              file=sys.stderr, flush=True)
        if cpu is not None and cpu_s > 0:
            fn_rows, kind, what = cpu
            out[-1]["cpu_baseline"] = cpu_rows_baseline(fn_rows, M, nbytes, ops, bound, kind, what, cpu_s)
            cb = out[-1]["cpu_baseline"]
            print(f"[bench]   CPU: {cb['value']:.4g} {cb['unit']} ({cb['kind']}, {cb['sample']})", file=sys.stderr,
                  flush=True)

    def steps_for(ms_guess):
        return max(64, min(2400, int(400.0 / max(ms_guess * 1e3, 1.0))))

    if want("c1"):
        # ---- config 1, M=16 (the headline weights)
        g, _ = measure(npu, hip, ws_c1, 16, dA, dC, 960, 48)
        rec("C1 w8a8 K=2048 N=6144", npu.plan_name(ws_c1[0], 16), 16, g, K * N + 16 * K + 4 * 16 * N, 2 * 16 * N * K, "hbm",
            (lambda r: gemm(A512[:r], codes1), gkind, gwhat))

    if only is not None and "m512" in only:
        # ---- the metric's M=512 GEMM on the headline weights, for profiler runs only (--eager-only passes its
        # kernel to the counters with no graph or event calls from Python; the bench line's m512 entry times it in
        # a graph)
        g, _ = measure(npu, hip, ws_c1, 512, dA, dC, 480, 48)
        rec("int8 GEMM M=512 K=2048 N=6144", npu.plan_name(ws_c1[0], 512), 512, g, K * N + 512 * K + 4 * 512 * N,
            2 * 512 * N * K, "mfma_int8")

    if want("shard"):
        # ---- one GPU's share of config 1 split 8 ways over N (output channels), the natural split of the path
        # across GPUs: K=2048, N=768, M=1 and 16. 336 rotated copies of the 1.57 MB share (528 MB > 2x the MALL).
        NS = N // 8
        Ws = np.ascontiguousarray(codes1[:, :NS])
        wss = [npu.pack_i8(Ws) for _ in range(336)]
        assert all(wss)
        for M in (1, 16):
            g, _ = measure(npu, hip, wss, M, dA, dC, steps_for(0.002), 64)
            rec("C1 one-GPU share of an 8-way N split, K=2048 N=768", npu.plan_name(wss[0], M), M, g,
                K * NS + M * K + 4 * M * NS, 2 * M * NS * K, "hbm",
                (lambda r: gemm(A512[:r], Ws), gkind, gwhat))
        L.ork_npu_set_async(npu.h, 0)
        A1 = np.empty((16, K), np.int8)
        assert L.ork_dev_download(npu.h, ork.ptr(A1), dA, A1.nbytes) == 0
        Cs = np.empty((16, NS), np.int32)
        assert L.ork_dev_download(npu.h, ork.ptr(Cs), dC, Cs.nbytes) == 0   # the timed M=16 launches wrote it
        assert np.array_equal(Cs, O.gemm_i32(A1, Ws)), "N-split share spot check"
        L.ork_npu_set_async(npu.h, 1)
        for w in wss:
            L.ork_mm_free(npu.h, w)

    if want("c2"):
        # ---- config 2: fp16, K = N = 2048, M in {1, 16, 128, 512}
        K2 = N2 = 2048
        B2 = (rng.standard_normal((K2, N2)) * 0.02).astype(np.float16)
        A2 = rng.standard_normal((512, K2)).astype(np.float16)
        ws2 = [npu.pack_f16(B2) for _ in range(64)]   # 64 x 8 MB
        dA2 = L.ork_dev_alloc(npu.h, A2.nbytes)
        assert all(ws2) and dA2 and L.ork_dev_upload(npu.h, dA2, ork.ptr(A2), A2.nbytes) == 0
        for M in (1, 16, 128, 512):
            n = steps_for(0.006 if M < 512 else 0.012)
            g, _ = measure(npu, hip, ws2, M, dA2, dC, n, 16, "ork_f16_mm_run")
            rec("C2 fp16 K=N=2048", npu.plan_name(ws2[0], M), M, g, 2 * M * K2 + 2 * K2 * N2 + 4 * M * N2,
                2 * M * N2 * K2, "hbm" if M <= 128 else "mfma_fp16",
                (lambda r: O.gemm_f16_f32acc(A2[:r], B2), "port",
                 "oracle restatement of the reference's fp32-accumulate fp16 loop (examples/test_matmul.c:37)"))
        L.ork_npu_set_async(npu.h, 0)
        C2 = np.empty((4, N2), np.float32)
        assert L.ork_f16_mm_run(npu.h, ws2[0], 4, dA2, dC) == 0
        assert L.ork_dev_download(npu.h, ork.ptr(C2), dC, C2.nbytes) == 0
        assert O.fp16_err(C2, O.gemm_f16_f64acc(A2[:4], B2)) <= 2e-3, "fp16 spot check"
        L.ork_npu_set_async(npu.h, 1)
        for w in ws2:
            L.ork_mm_free(npu.h, w)
        L.ork_dev_free(npu.h, dA2)

    if want("c3"):
        # ---- config 3: w4a8, K=2048, N=6144, importance vector, uniform and NF4, M in {1, 64}
        W3 = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        im3 = rng.uniform(0.5, 2.0, K).astype(np.float32)
        for nf4 in (0, 1):
            if nf4:
                os.environ["ORK_NF4"] = "1"
            try:
                w0, _ = npu.pack_i4a8(W3, im3)
            finally:
                os.environ.pop("ORK_NF4", None)
            blob = ork.dump_i4a8(w0)
            ws3 = [w0] + [npu.load_i4a8(K, N, blob) for _ in range(83)]   # 84 x 6.3 MB
            assert all(ws3)
            _, codes3 = O.o4n1_decode(K, N, blob)   # the reference's CPU path: inflate at load, then the int8 GEMM
            name = "C3 w4a8 %s K=2048 N=6144" % ("nf4" if nf4 else "uniform")
            for M in (1, 64):
                g, _ = measure(npu, hip, ws3, M, dA, dC, steps_for(0.003), 32)
                rec(name, npu.plan_name(ws3[0], M), M, g, K * N // 2 + M * K + 4 * M * N, 2 * M * N * K, "hbm",
                    (lambda r, c3=codes3: gemm(A512[:r], c3), gkind, gwhat + " on the inflated codes"))
            L.ork_npu_set_async(npu.h, 0)
            A3 = np.empty((2, K), np.int8)
            assert L.ork_dev_download(npu.h, ork.ptr(A3), dA, A3.nbytes) == 0
            C3 = np.empty((2, N), np.int32)
            assert L.ork_i8_mm_run(npu.h, ws3[-1], 2, dA, dC) == 0
            assert L.ork_dev_download(npu.h, ork.ptr(C3), dC, C3.nbytes) == 0
            assert np.array_equal(C3, O.gemm_i32(A3, codes3)), "w4a8 spot check"
            L.ork_npu_set_async(npu.h, 1)
            for w in ws3:
                L.ork_mm_free(npu.h, w)

    if want("c4"):
        # ---- config 4: W4A4, M=256, K=N=4096, values in [-8, 7]
        K4 = N4 = 4096
        B4 = rng.integers(-8, 8, size=(K4, N4), dtype=np.int8)
        A4 = rng.integers(-8, 8, size=(256, K4), dtype=np.int8)
        ws4 = [npu.pack_i4(B4) for _ in range(64)]   # 64 x 8 MB of nibbles
        dA4 = L.ork_dev_alloc(npu.h, A4.nbytes)
        assert all(ws4) and dA4 and L.ork_dev_upload(npu.h, dA4, ork.ptr(A4), A4.nbytes) == 0
        g, _ = measure(npu, hip, ws4, 256, dA4, dC, steps_for(0.01), 16, "ork_i4_mm_run")
        rec("C4 W4A4 K=N=4096", npu.plan_name(ws4[0], 256), 256, g, 256 * K4 + K4 * N4 // 2 + 4 * 256 * N4,
            2 * 256 * N4 * K4, "mfma_int8",
            (lambda r: gemm(A4[:r], B4), gkind, gwhat + " on the int8 containers (ork_i4_mm_run's offline branch)"))
        L.ork_npu_set_async(npu.h, 0)
        C4 = np.empty((256, N4), np.int32)
        assert L.ork_dev_download(npu.h, ork.ptr(C4), dC, C4.nbytes) == 0
        assert np.array_equal(C4[:2], O.gemm_i32(A4[:2], B4)) and np.array_equal(C4[-2:], O.gemm_i32(A4[-2:], B4)), \
            "W4A4 spot check"
        L.ork_npu_set_async(npu.h, 1)
        for w in ws4:
            L.ork_mm_free(npu.h, w)
        if not want("grouped"):
            L.ork_dev_free(npu.h, dA4)

    if want("grouped"):
        # ---- grouped scales (not a BASELINE config): W4A4 K=N=4096 with G=128 scales, M in {1, 256}; and the
        # grouped int8 shape of examples/test_grouped_i8.c (W4A4 pack loaded as int8, K=2048, N=16384, G=512)
        G4 = 128
        Sk4 = K4 // G4
        ggemm = O.ref_gemm_grouped if have_ref else O.gemm_grouped
        ggwhat = "orki_cpu_gemm_grouped as built (-O2)" if have_ref else "oracle restatement of orki_cpu_gemm_grouped"
        aS4 = rng.uniform(1e-3, 1e-2, size=(256, Sk4)).astype(np.float32)
        bS4 = rng.uniform(1e-3, 1e-2, size=(Sk4, N4)).astype(np.float32)
        dS4 = [L.ork_dev_alloc(npu.h, a.nbytes) for a in (aS4, bS4)]
        assert all(dS4) and all(L.ork_dev_upload(npu.h, d, ork.ptr(a), a.nbytes) == 0 for d, a in zip(dS4, (aS4, bS4)))
        wg4 = [L.ork_i4_mm_pack_grouped(npu.h, K4, N4, ork.ptr(B4), G4) for _ in range(64)]
        assert all(wg4)
        for M in (1, 256):
            g, _ = measure(npu, hip, wg4, M, dA4, dC, steps_for(0.01), 16, "ork_i4_mm_run_grouped", dS4)
            nbytes = K4 * N4 // 2 + M * K4 + 4 * (M * Sk4 + Sk4 * N4) + 4 * M * N4
            rec("grouped W4A4 K=N=4096 G=128", npu.grouped_plan_name(wg4[0], M), M, g, nbytes, 2 * M * N4 * K4,
                "hbm" if M <= 16 else "mfma_int8",
                (lambda r: ggemm(A4[:r], B4, aS4[:r], bS4, G4), gkind, ggwhat))
        L.ork_npu_set_async(npu.h, 0)
        Cg = np.empty((256, N4), np.float32)  # what the timed M=256 launches wrote (every copy holds B4)
        assert L.ork_dev_download(npu.h, ork.ptr(Cg), dC, Cg.nbytes) == 0
        rows = np.r_[0:2, 254:256]
        assert np.array_equal(Cg[rows], O.gemm_grouped(A4[rows], B4, aS4[rows], bS4, G4)), "grouped W4A4 M=256 spot check"
        Cg = np.empty((4, N4), np.float32)
        assert L.ork_i4_mm_run_grouped(npu.h, wg4[0], 4, dA4, dS4[0], dS4[1], dC) == 0
        assert L.ork_dev_download(npu.h, ork.ptr(Cg), dC, Cg.nbytes) == 0
        assert np.array_equal(Cg, O.gemm_grouped(A4[:4], B4, aS4[:4], bS4, G4)), "grouped W4A4 spot check"
        L.ork_npu_set_async(npu.h, 1)
        for w in wg4:
            L.ork_mm_free(npu.h, w)
        L.ork_dev_free(npu.h, dA4)
        K8, N8, G8, M8 = 2048, 16384, 512, 8
        B8 = rng.integers(-8, 8, size=(K8, N8), dtype=np.int8)
        blob8 = ork.dump_cpu(npu.h, B8, w4a4=True)
        wg8 = [L.ork_i4a8_mm_load_tiled(npu.h, K8, N8, ork.ptr(blob8), blob8.nbytes, G8) for _ in range(40)]
        aS8 = rng.uniform(1e-3, 1e-2, size=(M8, K8 // G8)).astype(np.float32)
        bS8 = rng.uniform(1e-3, 1e-2, size=(K8 // G8, N8)).astype(np.float32)
        dS8 = [L.ork_dev_alloc(npu.h, a.nbytes) for a in (aS8, bS8)]
        assert all(wg8) and all(dS8)
        assert all(L.ork_dev_upload(npu.h, d, ork.ptr(a), a.nbytes) == 0 for d, a in zip(dS8, (aS8, bS8)))
        g, _ = measure(npu, hip, wg8, M8, dA, dC, steps_for(0.01), 16, "ork_i8_mm_run_grouped", dS8)
        rec("grouped int8 (W4A4 pack) K=2048 N=16384 G=512", npu.grouped_plan_name(wg8[0], M8), M8, g,
            K8 * N8 // 2 + M8 * K8 + 4 * (M8 * 4 + 4 * N8) + 4 * M8 * N8, 2 * M8 * N8 * K8, "hbm",
            (lambda r: ggemm(A512[:r], B8, aS8[:r], bS8, G8), gkind, ggwhat))
        for w in wg8:
            L.ork_mm_free(npu.h, w)
        for d in dS4 + dS8:
            L.ork_dev_free(npu.h, d)
    return out


def measure_chain(npu, hip, L, ws, dA, dC, S, steps):
    """ms per ork_i8_mm_run_chain call of S M=1 GEMVs (the multi-matmul submit), graph-timed like
    measure(): call i runs weights ws[(i*S + j) % len(ws)], one shared activation row, S output rows."""
    import ork

    stream = L.ork_npu_stream(npu.h)
    nsets = len(ws) // S
    sets = [ork.tasks(ork.TaskI8, [(ws[(k * S + j) % len(ws)], 1, dA, dC + j * N * 4, 0) for j in range(S)])
            for k in range(nsets)]

    def run(i):
        rc = L.ork_i8_mm_run_chain(npu.h, S, sets[i % nsets])
        if rc:
            raise RuntimeError(f"ork_i8_mm_run_chain rc={rc}")

    for i in range(2 * nsets):
        run(i)
    ts = L.ork_dev_alloc(npu.h, 16)
    assert ts

    def body():
        if L.ork_npu_mark(npu.h, ts):
            raise RuntimeError("ork_npu_mark failed")
        for i in range(steps):
            run(i)
        if L.ork_npu_mark(npu.h, ts + 8):
            raise RuntimeError("ork_npu_mark failed")

    g, ex = hip.capture(stream, body)
    hip.ck(hip.L.hipGraphLaunch(ex, C.c_void_p(stream)), "hipGraphLaunch")
    hip.time_ms(stream, lambda: hip.ck(hip.L.hipGraphLaunch(ex, C.c_void_p(stream)), "hipGraphLaunch"))
    ms = graph_stamps_ms(npu, L, ts)
    hip.L.hipGraphExecDestroy(ex)
    hip.L.hipGraphDestroy(g)
    L.ork_dev_free(npu.h, ts)
    return ms / steps


def measure_decoder(npu, nf4, prompt_len=128, decode_len=256, graph=True):
    """the Qwen3-1.7B-shaped decoder (28 layers, hidden 2048, 16 Q / 8 KV heads,
    head_dim 128, SwiGLU 6144, vocab 151936), seeded N(0, 0.02) weights packed w8a8 per channel (NF4 w4a8
    FFNs when nf4), prefill of 128 seeded tokens, then 256 greedy decode steps (context <= 512). Every
    projection and the LM head run through the public matmul API; one decode step is a replayed HIP
    graph. Decode tokens/s is wall-clock over the 256 steps, enqueue to completion; prefill tokens/s is the
    median of five timed prefills. Checked: finite
    logits, tokens in range, and an eager (non-graph) replay of the first steps reproduces the tokens."""
    import qwen3 as Q

    cfg = Q.make_cfg(max_ctx=512, max_rows=prompt_len, ffn_nf4=nf4, **Q.QWEN3_1P7B)
    m = Q.Model(npu, cfg)
    try:
        t0 = time.perf_counter()
        assert m.init_random(0x6F726B00 + (5 << 8)) == 0
        init_s = time.perf_counter() - t0
        prompt = np.random.default_rng(0x6F726B05).integers(0, cfg.vocab, prompt_len).astype(np.int32)
        assert m.prefill(prompt) == 0 and m.decode(4, graph=graph) == 0   # warm-up and graph capture
        pre = []
        for _ in range(5):   # eager launches timed from the host: the median of five prefills
            t0 = time.perf_counter()
            assert m.prefill(prompt) == 0
            pre.append(time.perf_counter() - t0)
        pre_s = float(np.median(pre))
        t0 = time.perf_counter()
        assert m.decode(decode_len, graph=graph) == 0
        dec_s = time.perf_counter() - t0
        toks = m.tokens()
        logits = m.last_logits()
        assert np.all(np.isfinite(logits)) and toks.min() >= 0 and toks.max() < cfg.vocab
        assert m.prefill(prompt) == 0 and m.decode(16, graph=False) == 0
        assert np.array_equal(m.tokens(), toks[:prompt_len + 17]), "eager decode differs from the graph replay"
        wbytes = m.weight_bytes()
    finally:
        m.close()
    kvd = cfg.kv_heads * cfg.head_dim
    mean_keys = prompt_len + (decode_len + 1) / 2.0
    kv_bytes = cfg.layers * mean_keys * kvd * 4 * 2          # K and V (fp32) read per token
    per_tok = wbytes + kv_bytes
    tps = decode_len / dec_s
    gbs = per_tok * tps / 1e9
    name = "C5 qwen3-1.7b decoder %s" % ("w8a8 + NF4 FFN" if nf4 else "w8a8")
    print(f"[bench] {name}: decode {tps:.1f} tok/s ({dec_s / decode_len * 1e3:.3f} ms/token, {gbs:.0f} GB/s), "
          f"prefill {prompt_len / pre_s:.0f} tok/s; weights {wbytes / 1e9:.3f} GB (init+pack {init_s:.1f} s)",
          file=sys.stderr, flush=True)
    return {"config": name, "value": round(tps, 1), "unit": "tokens/s",
            "ms_per_token": round(dec_s / decode_len * 1e3, 4),
            "prefill_tokens_per_s": round(prompt_len / pre_s, 1), "prefill_ms": round(pre_s * 1e3, 3),
            "bytes_per_token": int(per_tok),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)},
            "note": "prefill 128 seeded tokens, 256 greedy decode steps (HIP graph per step), batch 1; bytes per "
                    "token = resident weights + scales + fp32 KV cache read at the mean context"}


def cpu_decoder_baseline(budget_s):
    """Config 5's CPU counterpart on a bounded sample: the per-token matmuls of the Qwen3-1.7B shape (28 layers of
    q, k, v, o, gate, up, down GEMVs and the LM head) through the reference's own orki_cpu_gemm_i32 at M = 1, each
    distinct shape timed for ~budget_s / 5 seconds. Attention, norms and sampling are left out, so the tokens/s
    is an upper bound for a CPU decode. The NF4-FFN variant runs the same GEMMs on the CPU (its codes are
    inflated to int8 at load), so one number serves both."""
    import oracle as O

    have_ref = O.ref_available()
    gemm = O.ref_gemm_i32 if have_ref else O.gemm_i32
    rng = np.random.default_rng(0x6F726B05)
    H, KV, F, V, layers = 2048, 8 * 128, 6144, 151936, 28
    per_layer = [((H, H), 2), ((H, KV), 2), ((H, F), 2), ((F, H), 1)]   # (q, o), (k, v), (gate, up), down
    ms_tok, parts = 0.0, []
    for (k, n), cnt in per_layer + [((H, V), None)]:
        B = np.frombuffer(rng.bytes(k * n), np.int8).reshape(k, n)
        A = rng.integers(-127, 128, size=(1, k), dtype=np.int8)
        dt, _ = _time_calls(lambda: gemm(A, B), budget_s / 5)
        ms_tok += dt * 1e3 * (layers * cnt if cnt else 1)
        parts.append(f"{k}x{n} {dt * 1e3:.2f} ms")
        del B
    return {"value": round(1e3 / ms_tok, 3), "unit": "tokens/s", "cores": 1,
            "kind": "reference" if have_ref else "port",
            "sample": f"per-token matmuls only (28 layers x q,k,v,o,gate,up,down + LM head) with "
                      f"{'orki_cpu_gemm_i32 as built (-O2)' if have_ref else 'the oracle restatement'}, M=1, 1 thread, "
                      f"each distinct shape timed separately ({'; '.join(parts)}) = {ms_tok:.1f} ms/token; attention and glue left "
                      f"out (an upper bound); host {cpu_model()}"}


def copy_calibration(hip, L, reps=96):
    """Device-to-device copies of K*N bytes (hipMemcpyAsync D2D: the runtime's copy kernel) between
    rotated buffers, so rocprofv3's FETCH_SIZE / WRITE_SIZE for a kernel of known traffic can be read."""
    import ork

    nbytes = K * N
    with ork.Npu() as npu:
        bufs = [L.ork_dev_alloc(npu.h, nbytes) for _ in range(R)]
        dst = L.ork_dev_alloc(npu.h, nbytes)
        stream = L.ork_npu_stream(npu.h)
        hip.L.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
        for i in range(reps):
            hip.ck(hip.L.hipMemcpyAsync(C.c_void_p(dst), C.c_void_p(bufs[i % R]), nbytes, 3, C.c_void_p(stream)),
                   "hipMemcpyAsync")
        hip.ck(hip.L.hipDeviceSynchronize(), "sync")
        print(f"[bench] copy calibration: {reps} device copies of {nbytes} bytes", file=sys.stderr, flush=True)


def cpu_model():
    """The host CPU's model name and logical CPU count (reported beside every CPU number)."""
    name = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return f"{name}, {os.cpu_count()} logical CPUs"


def _time_calls(fn, budget_s):
    fn()
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        fn()
        n += 1
    return (time.perf_counter() - t0) / n, n


def cpu_baseline(W_codes, A_row, budget_s):
    """The reference's own CPU GEMM (orki_cpu_gemm_i32 from oracle/_ref) single-threaded on M=1 calls of
    the same workload, for ~budget_s seconds. Falls back to the oracle restatement if _ref is absent.
    M = 1 is single-threaded in the reference whatever the build (its pragma is `if(M>1)`)."""
    import oracle as O

    kind = "reference" if O.ref_available() else "port"
    fn = O.ref_gemm_i32 if kind == "reference" else O.gemm_i32
    dt, n = _time_calls(lambda: fn(A_row, W_codes), budget_s)
    return {"value": round(algo_bytes(1) / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{n} M=1 calls of the K=2048,N=6144 int8 GEMM (orki_cpu_gemm_i32 as built, -O2, 1 thread), "
                      f"{dt * 1e3:.2f} ms/call; host {cpu_model()}"}


def cpu_baseline_m512(W_codes, A512, budget_s):
    """The M=512 GEMM on the host with the reference's own orki_cpu_gemm_i32: one thread (the library as the
    reference builds it) on a 16-row sample of the same A -- its rows are independent k-outer AXPY passes, so
    the time scales by 512/16 -- and, from the -fopenmp build of the same sources, full M=512 calls with the
    row-parallel pragma (src/npu/core/buf.c:438) on every host thread. ~budget_s seconds each."""
    import oracle as O

    if not O.ref_available():
        dt, n = _time_calls(lambda: O.gemm_i32(A512[:16], W_codes), budget_s)
        return {"value": round(algo_ops(512) / (dt * 32) / 1e12, 5), "unit": "TOP/s", "cores": 1, "kind": "port",
                "sample": f"{n} calls of 16 rows of the M=512 GEMM (oracle restatement, 1 thread), x32 rows"}
    dt1, n1 = _time_calls(lambda: O.ref_gemm_i32(A512[:16], W_codes), budget_s)
    out = {"value": round(algo_ops(512) / (dt1 * 32) / 1e12, 5), "unit": "TOP/s", "cores": 1, "kind": "reference",
           "sample": f"{n1} calls of 16 rows of the M=512 K=2048 N=6144 GEMM (orki_cpu_gemm_i32 as built, -O2, "
                     f"1 thread), {dt1 * 1e3:.1f} ms per 16 rows, scaled to 512 rows; host {cpu_model()}"}
    if O.ref_omp_available():
        threads = O.ref_omp().ref_threads()
        dtm, nm = _time_calls(lambda: O.ref_gemm_i32(A512, W_codes, omp=True), budget_s)
        out["all_cores"] = {"value": round(algo_ops(512) / dtm / 1e12, 5), "unit": "TOP/s", "cores": threads,
                            "kind": "reference",
                            "sample": f"{nm} full M=512 calls, orki_cpu_gemm_i32 built with -fopenmp (its row-parallel "
                                      f"pragma live), {threads} threads, {dtm * 1e3:.1f} ms/call"}
    return out


def trace_from_profiles(kernel_tag):
    """The rocprofv3 kernel-trace summary of the dominant kernel (profiles/*_trace.json): its traced per-dispatch
    duration, the tracer's per-dispatch overhead measured in the same traced run on the K=32, N=32 GEMV and the
    one-thread wall-clock kernel against their untraced graph steps, and the step time and roofline fraction that
    follow from them; or None."""
    p = os.path.join(ROOT, "profiles", f"{kernel_tag}_trace.json")
    if not os.path.exists(p):
        return None
    try:
        return json.load(open(p)).get("roofline_from_trace")
    except Exception:
        return None


def traffic_from_profiles(kernel_tag):
    """HBM bytes per launch from committed rocprofv3 --pmc summaries (profiles/*_pmc.json), or None."""
    p = os.path.join(ROOT, "profiles", f"{kernel_tag}_pmc.json")
    if not os.path.exists(p):
        return None
    try:
        return json.load(open(p)).get("hbm_bytes_per_launch")
    except Exception:
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2400)
    ap.add_argument("--warmup", type=int, default=240)
    ap.add_argument("--m512-steps", type=int, default=480)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the sweep over BASELINE configs 1-4")
    ap.add_argument("--no-decoder", action="store_true", help="skip BASELINE config 5 (the Qwen3-shaped decoder)")
    ap.add_argument("--eager-decoder", action="store_true",
                    help="profiling: launch the decode steps eagerly instead of replaying the captured graph (same kernels)")
    ap.add_argument("--only", choices=["gemv", "m512", "chain", "decoder", "configs"],
                    help="profiling: time only one kernel (decoder: only BASELINE config 5, w8a8; configs: the "
                         "config sweep's sections named by --configs)")
    ap.add_argument("--configs", default="c1,shard,c2,c3,c4,grouped",
                    help="with --only configs: comma-separated sections of the config sweep (c1 shard c2 c3 c4 "
                         "grouped; shard = one GPU's share of config 1 split 8 ways over N; m512, only when named: "
                         "the M=512 int8 GEMM of the bench line, for profiler runs)")
    ap.add_argument("--eager-only", action="store_true",
                    help="profiling: time eager launches by the host clock only (no graphs, events or HIP calls "
                         "from Python); with --only configs")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="profiling: run device-to-device copies of one weight's bytes (a plain copy kernel of "
                         "known size) instead of the bench, to scale rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the resident-weight matmul has no collective; "
              "N-sharding across GPUs is designed but not run in this build). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import ork
    import oracle as O

    L = ork.lib()
    global EAGER_ONLY
    EAGER_ONLY = args.eager_only
    if EAGER_ONLY and args.only != "configs":
        ap.error("--eager-only goes with --only configs")
    hip = None if EAGER_ONLY else Hip()
    if args.copy_calibration:
        copy_calibration(hip, L)
        return
    if args.only == "decoder":
        with ork.Npu() as npu:
            print(json.dumps(measure_decoder(npu, 0, graph=not args.eager_decoder)), flush=True)
        return
    rng = np.random.default_rng(0x6F726B00 + (1 << 8))
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)   # f32[N][K]
    A512 = rng.integers(-127, 128, size=(512, K), dtype=np.int8)
    with ork.Npu() as npu:
        t0 = time.perf_counter()
        ws = []
        for _ in range(R):
            w, bs = npu.pack_i8_f32(W)
            if not w:
                raise RuntimeError("ork_i8_mm_pack_f32 failed")
            ws.append(w)
        pack_s = (time.perf_counter() - t0) / R
        codes, bs_ref = O.pack_i8_f32(W)
        assert np.array_equal(bs, bs_ref)
        dA = L.ork_dev_alloc(npu.h, A512.nbytes)
        dC = L.ork_dev_alloc(npu.h, 512 * N * 4)
        assert dA and dC
        assert L.ork_dev_upload(npu.h, dA, ork.ptr(A512), A512.nbytes) == 0
        L.ork_npu_set_async(npu.h, 1)
        if args.only == "configs":
            sel = set(x.strip() for x in args.configs.split(",") if x.strip())
            print(json.dumps(sweep_configs(npu, hip, L, ws, dA, dC, codes, A512,
                                           0.0 if args.no_cpu else min(2.0, args.cpu_seconds / 5), only=sel)),
                  flush=True)
            for w in ws:
                ork.lib().ork_mm_free(npu.h, w)
            return
        gemv_plan = npu.plan_name(ws[0], 1)
        gemm_plan = npu.plan_name(ws[0], 512)
        print(f"[bench] packed {R} x {K}x{N} int8 weights ({pack_s * 1e3:.1f} ms/pack); plans M=1 {gemv_plan}, "
              f"M=512 {gemm_plan}", file=sys.stderr, flush=True)

        g1 = e1 = g512 = e512 = floor_ms = copy_ms = read_ms = mark_ms = float("nan")
        if args.only == "chain":
            ms = measure_chain(npu, hip, L, ws, dA, dC, 8, 300)
            print(f"[bench] chain of 8: {ms * 1e3:.2f} us/call", file=sys.stderr, flush=True)
            for w in ws:
                ork.lib().ork_mm_free(npu.h, w)
            return
        o1, o512 = [], []
        if args.only not in ("m512",):
            g1, e1 = measure(npu, hip, ws, 1, dA, dC, args.steps, args.warmup, outer=o1)
            print(f"[bench] M=1: graph {g1 * 1e3:.2f} us/step, eager {e1 * 1e3:.2f} us/step", file=sys.stderr, flush=True)
        if args.only in (None, "gemv", "m512"):
            # the same graph harness around a launch that moves almost nothing (K=32, N=32) and around the one-thread
            # wall-clock kernel alone: what one launch costs on this box before any data (in a traced run, the
            # tracer's own cost per dispatch beside the GEMV's)
            tiny = npu.pack_i8(np.ones((32, 32), np.int8))
            floor_ms, _ = measure(npu, hip, [tiny], 1, dA, dC, args.steps, args.warmup)
            ork.lib().ork_mm_free(npu.h, tiny)
            mark_ms = measure_marks(npu, hip, L, dA, dC, args.steps, args.warmup)
            print(f"[bench] K=32 N=32 GEMV: {floor_ms * 1e3:.3f} us/step; wall-clock mark alone: {mark_ms * 1e3:.3f} "
                  f"us/step", file=sys.stderr, flush=True)
        if not args.only:
            # and around the runtime's copy kernel moving the weight's bytes, and a plain read of them
            copy_ms = measure_copy(hip, L, npu, K * N, args.steps)
            read_ms = measure_read(npu, hip, L, ws, dA, dC, args.steps, args.warmup)
            print(f"[bench] launch floor (K=32 N=32 GEMV): {floor_ms * 1e3:.2f} us/step; D2D copy of {K * N} B: "
                  f"{copy_ms * 1e3:.2f} us ({2 * K * N / (copy_ms * 1e-3) / 1e9:.0f} GB/s read+write); plain read of "
                  f"the weight's panels: {read_ms * 1e3:.2f} us ({K * N / (read_ms * 1e-3) / 1e9:.0f} GB/s)",
                  file=sys.stderr, flush=True)
        if args.only != "gemv":
            g512, e512 = measure(npu, hip, ws, 512, dA, dC, args.m512_steps, max(args.warmup // 8, 8), outer=o512)
            print(f"[bench] M=512: graph {g512 * 1e3:.2f} us/step, eager {e512 * 1e3:.2f} us/step",
                  file=sys.stderr, flush=True)
        if args.only:
            for w in ws:
                ork.lib().ork_mm_free(npu.h, w)
            return

        # correctness of what was timed: the last M=512 and an M=1 launch vs the oracle
        L.ork_npu_set_async(npu.h, 0)
        C512 = np.empty((512, N), np.int32)
        assert L.ork_dev_download(npu.h, ork.ptr(C512), dC, C512.nbytes) == 0
        rows = np.r_[0:4, 508:512]
        assert np.array_equal(C512[rows], O.gemm_i32(A512[rows], codes)), "M=512 result differs from the oracle"
        assert L.ork_i8_mm_run(npu.h, ws[1], 1, dA, dC) == 0
        C1 = np.empty((1, N), np.int32)
        assert L.ork_dev_download(npu.h, ork.ptr(C1), dC, C1.nbytes) == 0
        assert np.array_equal(C1, O.gemm_i32(A512[:1], codes)), "M=1 result differs from the oracle"

        # the reference's calling convention: host A and C, synchronous (PCIe-inclusive; not `value`)
        Ah = np.ascontiguousarray(A512[:1])
        Ch = np.empty((1, N), np.int32)
        for i in range(20):
            assert L.ork_i8_mm_run(npu.h, ws[i % R], 1, ork.ptr(Ah), ork.ptr(Ch)) == 0
        nh = 2000
        t0 = time.perf_counter()
        for i in range(nh):
            L.ork_i8_mm_run(npu.h, ws[i % R], 1, ork.ptr(Ah), ork.ptr(Ch))
        host_us = (time.perf_counter() - t0) / nh * 1e6
        assert np.array_equal(Ch, O.gemm_i32(Ah, codes)), "host-pointer M=1 result differs from the oracle"
        print(f"[bench] M=1 host pointers, synchronous: {host_us:.2f} us/call", file=sys.stderr, flush=True)

        # the multi-matmul submit: 8 GEMVs of the same shape per call, one grouped launch
        L.ork_npu_set_async(npu.h, 1)
        S8 = 8
        chain_ms = measure_chain(npu, hip, L, ws, dA, dC, S8, 300)
        L.ork_npu_set_async(npu.h, 0)
        Cch = np.empty((S8, N), np.int32)
        assert L.ork_dev_download(npu.h, ork.ptr(Cch), dC, Cch.nbytes) == 0
        assert np.array_equal(Cch, np.repeat(O.gemm_i32(A512[:1], codes), S8, axis=0)), "chain result differs"
        chain_gbs = S8 * algo_bytes(1) / (chain_ms * 1e-3) / 1e9
        print(f"[bench] ork_i8_mm_run_chain of {S8} M=1 GEMVs: {chain_ms * 1e3:.2f} us/call "
              f"({chain_gbs:.0f} GB/s aggregate)", file=sys.stderr, flush=True)

        # the same GEMV kernel on a weight large enough to amortise the launch: an LM head's shape
        L.ork_npu_set_async(npu.h, 1)
        NL = 151936
        BL = np.frombuffer(np.random.default_rng(0x6F726B4C).bytes(K * NL), np.int8).reshape(K, NL)
        wl = [npu.pack_i8(BL) for _ in range(3)]
        dCl = L.ork_dev_alloc(npu.h, NL * 4)
        assert all(wl) and dCl
        lm_ms, _ = measure(npu, hip, wl, 1, dA, dCl, 60, 6)
        L.ork_npu_set_async(npu.h, 0)
        Cl = np.empty((1, NL), np.int32)
        assert L.ork_dev_download(npu.h, ork.ptr(Cl), dCl, Cl.nbytes) == 0
        assert np.array_equal(Cl, O.gemm_i32(A512[:1], BL)), "large-N GEMV result differs"
        lm_plan = npu.plan_name(wl[0], 1)
        lm_gbs = (K * NL + K + 4 * NL) / (lm_ms * 1e-3) / 1e9
        for w in wl:
            ork.lib().ork_mm_free(npu.h, w)
        L.ork_dev_free(npu.h, dCl)
        del BL
        print(f"[bench] M=1 GEMV K={K} N={NL}: {lm_ms * 1e3:.2f} us/step ({lm_gbs:.0f} GB/s, "
              f"{lm_gbs / HBM_PEAK_GBS:.1%} of HBM) {lm_plan}", file=sys.stderr, flush=True)

        # the LDS-ring kernel on a large square GEMM, where each CU's operand bytes per MAC are small enough for the
        # MFMA work to dominate: what the kernel reaches when operand delivery to the CUs is not the bound
        L.ork_npu_set_async(npu.h, 1)
        SQ = 4096
        rq = np.random.default_rng(0x6F726B51)
        Bq = np.frombuffer(rq.bytes(SQ * SQ), np.int8).reshape(SQ, SQ)
        Aq = np.frombuffer(rq.bytes(SQ * SQ), np.int8).reshape(SQ, SQ)
        wq = [npu.pack_i8(Bq) for _ in range(40)]
        dAq, dCq = L.ork_dev_alloc(npu.h, SQ * SQ), L.ork_dev_alloc(npu.h, SQ * SQ * 4)
        assert all(wq) and dAq and dCq
        assert L.ork_dev_upload(npu.h, dAq, ork.ptr(Aq), Aq.nbytes) == 0
        sq_ms, _ = measure(npu, hip, wq, SQ, dAq, dCq, 40, 4)
        L.ork_npu_set_async(npu.h, 0)
        Cq = np.empty((SQ, SQ), np.int32)
        assert L.ork_dev_download(npu.h, ork.ptr(Cq), dCq, Cq.nbytes) == 0
        rows = np.r_[0:4, 2045:2051, SQ - 4:SQ]
        assert np.array_equal(Cq[rows], O.gemm_i32(Aq[rows], Bq)), "large GEMM result differs"
        sq_plan = npu.plan_name(wq[0], SQ)
        sq_tops = 2.0 * SQ ** 3 / (sq_ms * 1e-3) / 1e12
        for w in wq:
            ork.lib().ork_mm_free(npu.h, w)
        L.ork_dev_free(npu.h, dAq)
        L.ork_dev_free(npu.h, dCq)
        del Aq, Bq, Cq
        print(f"[bench] int8 GEMM M=K=N={SQ}: {sq_ms * 1e3:.2f} us/step ({sq_tops:.0f} TOP/s, "
              f"{sq_tops / INT8_PEAK_TOPS:.1%} of MFMA) {sq_plan}", file=sys.stderr, flush=True)

        configs = None
        if not args.no_configs:
            L.ork_npu_set_async(npu.h, 1)
            configs = sweep_configs(npu, hip, L, ws, dA, dC, codes, A512,
                                    0.0 if args.no_cpu else min(2.0, args.cpu_seconds / 5))
            L.ork_npu_set_async(npu.h, 0)

        for w in ws:
            ork.lib().ork_mm_free(npu.h, w)
        L.ork_dev_free(npu.h, dA)
        L.ork_dev_free(npu.h, dC)

        if not args.no_decoder:
            dec = [measure_decoder(npu, 0), measure_decoder(npu, 1)]
            if not args.no_cpu:
                cb = cpu_decoder_baseline(min(3.0, args.cpu_seconds / 3))
                print(f"[bench]   CPU decoder: {cb['value']:.3g} tokens/s ({cb['sample']})", file=sys.stderr, flush=True)
                for d in dec:
                    d["cpu_baseline"] = cb
            configs = (configs or []) + dec

    gbs = algo_bytes(1) / (g1 * 1e-3) / 1e9
    tops = algo_ops(512) / (g512 * 1e-3) / 1e12
    out = {
        "metric": "w8a8 M=1 GEMV HBM GB/s (% peak); M=512 int8 GEMM TOPS (% MFMA peak)",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g1, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": f"synthetic (seeded N(0,0.02) weights, U[-127,127] activations); {R} rotated resident weight copies: "
                f"each timed step reads a weight last read {cold_distance(K * N, R, args.steps) / 1e6:.0f} MB of other "
                f"weights earlier (> 2 x the 256 MB MALL)",
        "config": {"workload": "w8a8 GEMV ork_i8_mm_run M=1 K=2048 N=6144 (BASELINE config 1)",
                   "kernel": gemv_plan,
                   "timing": "one HIP graph of `steps` launches between two device wall-clock stamps written by its "
                             "first and last nodes (ork_npu_mark: the timed region is exactly the steps on the device), "
                             "device-synchronised before and after; replayed untimed for 50 ms first (steady state), "
                             "then the other weights streamed, then the timed replay"},
        "graph_launch_inclusive": {"ms_per_step": round(o1[0], 6) if o1 else None,
                                   "value": round(algo_bytes(1) / (o1[0] * 1e-3) / 1e9, 1) if o1 else None,
                                   "note": "the same replay timed by events recorded around hipGraphLaunch: adds the "
                                           "host's one submission of the graph, spread over `steps`"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles("gemv_i8_m1"),
                     "rocprof": trace_from_profiles("gemv_i8_m1")},
        "eager_value": round(algo_bytes(1) / (e1 * 1e-3) / 1e9, 1),
        "launch_floor": {"gemv_k32_n32_us": round(floor_ms * 1e3, 3),
                         "mark_us": round(mark_ms * 1e3, 3),
                         "d2d_copy_us": round(copy_ms * 1e3, 3),
                         "d2d_copy_gbs": round(2 * K * N / (copy_ms * 1e-3) / 1e9, 1),
                         "read_us": round(read_ms * 1e3, 3),
                         "read_gbs": round(K * N / (read_ms * 1e-3) / 1e9, 1),
                         "note": "same HIP-graph harness and step count as `value`: ork_i8_mm_run on a K=32, N=32 weight "
                                 "(a launch that moves almost nothing), ork_npu_mark alone (a one-thread kernel), "
                                 "hipMemcpyAsync device-to-device of the "
                                 "weight's 12,582,912 bytes from the same rotation (read + write counted), and "
                                 "ork_npu_read_probe reading those panel bytes alone (the GEMV's loads without its "
                                 "arithmetic: 1,536 workgroups of 4 waves, 2 loads of 16 bytes per lane, the fastest of 1-4 KiB per wave)"},
        "gemv_large_n": {"workload": f"ork_i8_mm_run M=1 K={K} N={NL} (an LM head's shape, 3 rotated copies of 311 MB)",
                         "kernel": lm_plan, "us_per_step": round(lm_ms * 1e3, 3), "value": round(lm_gbs, 1),
                         "unit": "GB/s", "frac": round(lm_gbs / HBM_PEAK_GBS, 4),
                         "note": "the same kernel as `value` in the same HIP-graph harness, on a weight large enough "
                                 "that the ~1.6 us launch no longer dominates; checked against the oracle"},
        "gemm_large": {"workload": f"int8 GEMM ork_i8_mm_run M=K=N={SQ} (40 rotated resident weights)", "kernel": sq_plan,
                       "us_per_step": round(sq_ms * 1e3, 3), "value": round(sq_tops, 1), "unit": "TOP/s",
                       "frac": round(sq_tops / INT8_PEAK_TOPS, 4),
                       "note": "the M=512 kernel family in the same HIP-graph harness on a shape with far more "
                               "multiply-accumulates per operand byte a CU receives; rows spot-checked against the oracle"},
        "chain8": {"value": round(chain_gbs, 1), "unit": "GB/s", "us_per_call": round(chain_ms * 1e3, 3),
                   "frac": round(chain_gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles("chain8_i8_m1"),
                   "note": "ork_i8_mm_run_chain: 8 M=1 GEMVs of the same shape (distinct resident weights) per call, "
                           "one grouped launch; A and C in HBM; HIP graph of 300 calls timed by in-graph wall-clock stamps"},
        "host_api": {"value": round(algo_bytes(1) / (host_us * 1e-6) / 1e9, 1), "unit": "GB/s",
                     "us_per_call": round(host_us, 2),
                     "note": "ork_i8_mm_run(M=1) with host A and C: H2D of A, launch, D2H of C, stream sync"},
        "m512": {"workload": "int8 GEMM ork_i8_mm_run M=512 K=2048 N=6144", "kernel": gemm_plan,
                 "value": round(tops, 1), "unit": "TOP/s", "ms_per_step": round(g512, 6), "steps": args.m512_steps,
                 "graph_launch_inclusive_ms_per_step": round(o512[0], 6) if o512 else None,
                 "roofline": {"bound": "mfma", "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                              "frac": round(tops / INT8_PEAK_TOPS, 4), "traffic": traffic_from_profiles("gemm_i8_m512"),
                              "rocprof": trace_from_profiles("gemm_i8_m512")},
                 "hbm_gbs": round(algo_bytes(512) / (g512 * 1e-3) / 1e9, 1),
                 "eager_value": round(algo_ops(512) / (e512 * 1e-3) / 1e12, 1)},
    }
    if configs is not None:
        out["configs"] = configs
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(codes, A512[:1], args.cpu_seconds)
        out["m512"]["cpu_baseline"] = cpu_baseline_m512(codes, A512, args.cpu_seconds / 2)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
