#!/usr/bin/env python3
"""Benchmark of the opcode-15 W8A8 linear on one MI355X.

A step is one full opcode-15 computation on HBM-resident inputs: per-token
activation quantization + INT8 MFMA GEMM + scale epilogue, at the headline
shape M=4096, K=1536, N=6144 (MLP-up layer).  Six
independent activation / weight / output sets rotate across steps so the
working set (about 0.8 GB) exceeds the 256 MB MALL.  Weights are prepacked
once at load, outside the timed region.

Printed: one JSON line with the headline TOPS, the GEMM kernel's roofline
(per-kernel averages from graph replays of back-to-back launches), the M=1 decode
HBM bandwidth (K=4096, N=14336) and a CPU baseline (the oracle, multithreaded,
on a bounded row sample of the same workload).

    python bench.py [--steps 200] [--warmup 20] [--config headline|all] [--no-cpu]

Profiling helpers (their output is what profiles/ holds):
    python bench.py --traffic-probe        a plain 256 MiB copy, then 12 headline
                                           GEMM launches: the workload of the
                                           FETCH_SIZE / WRITE_SIZE rocprofv3 passes
    python bench.py --profile-summary DIR  markdown summary of the rocprofv3 CSV
                                           output under DIR (kernel stats and/or
                                           per-dispatch counters)
"""
import argparse
import csv
import glob
import json
import os
import platform
import re
import statistics
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "htp-ops-lib-sd.cpp_amd"))

import htp_ops as hip  # noqa: E402

METRIC = "W8A8 INT8 TOPS & %MFMA peak (M=4096,K=1536,N=6144); M=1 decode HBM GB/s"
PEAK_INT8_TOPS = 5000.0   # MI355X dense INT8 MFMA
PEAK_HBM_GBPS = 8000.0    # MI355X HBM3E
PEAK_F16_TFLOPS = 2500.0  # MI355X dense FP16 MFMA
HEADLINE = (4096, 1536, 6144)
SETTLE_MS = 80.0          # untimed GPU time before each timed sequence (clock ramp)
TRAFFIC_FILE = os.path.join(REPO, "profiles", "w8a8_gemm_stream_4096x1536x6144_traffic.md")
COPY_PROBE_BYTES = 256 << 20
CHUNKS = 20               # chunks of the separate median pass (run only when every chunk has >= 10 steps)
USE_GRAPHS = True         # --no-graph: no graph capture or replay anywhere (for traced runs)


def progress(msg):
    """One progress line on stderr per finished case, so a failing run names its case."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _us(ms, digits=3):
    """ms -> us rounded, None stays None."""
    return None if ms is None else round(ms * 1e3, digits)


def w8a8_bytes(m, k, n):
    """Algorithmic HBM bytes of one opcode-15 call: activations f32, weights
    int8, scales/sums f32/i32, smoothing f32, blob header, output f32."""
    return 4 * m * k + n * k + 8 * n + 4 * k + 128 + 4 * m * n


def gemm_bytes(m, k, n):
    """Algorithmic bytes of the GEMM kernel alone: q int8, W int8, per-column
    scale + correction, row scales, f32 output."""
    return m * k + n * k + 8 * n + 4 * m + 4 * m * n


class W8A8Set:
    """One rotated copy: activations, packed weights, output, workspace."""

    def __init__(self, m, k, n, seed, outliers, scale_lo, scale_hi):
        rng = np.random.default_rng(seed)
        x = rng.standard_normal((m, k), dtype=np.float32)
        if outliers:
            chans = rng.choice(k, max(1, int(outliers * k)), replace=False)
            x[:, chans] *= 20.0
        w = rng.integers(-127, 128, (n, k), dtype=np.int8)
        sw = rng.uniform(scale_lo, scale_hi, n).astype(np.float32)
        blob = hip.pack_constants(w, sw)
        blob_dev = hip.DeviceBuffer.from_array(blob)
        self.packed = hip.w8a8_prepack(blob_dev, k, n)
        blob_dev.free()
        self.x = hip.DeviceBuffer.from_array(x)
        self.y = hip.DeviceBuffer(m * n * 4)
        mp = (m + 15) // 16 * 16
        # workspace of hb_w8a8_linear: q (mp x kp int8) then the row scales
        self.ws = hip.DeviceBuffer(hip.w8a8_workspace_bytes(m, k))
        self.q_ptr = self.ws.ptr
        self.s_ptr = self.ws.ptr + (mp * hip.kp_of(k) + 255) // 256 * 256
        self.inv_ptr = self.packed.ptr + hip.w8a8_packed_offset(k, n, hip.SECTION_INV)
        self.host_x, self.host_blob = (x, blob) if seed == 0 else (None, None)


def run_w8a8(m, k, n, steps, warmup, rotate, outliers=0.0, scale=(1e-4, 1e-3), settle_ms=SETTLE_MS,
             epilogue=None):
    """Times `steps` opcode-15 steps launched in stream order (the library's
    own launches, as a caller issues them; the host enqueues ahead of the
    GPU), then the same number of GEMM-only and quantize-only launches, for
    per-kernel averages (HIP events on the library stream that runs the
    kernels).  The same three sequences are also replayed from HIP graphs
    and reported beside them.  Each timed sequence starts after at least
    settle_ms of untimed load (the GPU clocks ramp over tens of ms)."""
    lib = hip.lib()
    stream = hip.default_stream()
    sets = [W8A8Set(m, k, n, seed, outliers, *scale) for seed in range(rotate)]

    epi = hip.EPI_SCALE if epilogue is None else epilogue

    def quant(st):
        hip.check(lib.hb_w8a8_quantize(st.q_ptr, st.s_ptr, st.x.ptr, st.inv_ptr, m, k, stream), "quantize")

    def gemm(st):
        hip.check(lib.hb_w8a8_gemm(st.y.ptr, n, st.q_ptr, st.s_ptr, st.packed.ptr, m, k, n, epi,
                                   stream), "gemm")

    def step(st):
        # the full op as the library runs it: quantize + GEMM, or for one row
        # the fused decode kernel
        hip.check(lib.hb_w8a8_linear(st.y.ptr, st.x.ptr, st.packed.ptr, m, k, n, epi, st.ws.ptr,
                                     st.ws.nbytes, stream), "linear")

    def capture(fn, count):
        with hip.Graph.capture(stream) as g:
            for i in range(count):
                fn(sets[i % rotate])
        return g

    def synced():
        hip.check(lib.hb_stream_sync(stream), "sync")
        hip.sync()

    def timed_stream(fn, count):
        """ms of `count` stream-ordered launches between ONE pair of HIP events
        (no event inside the timed region: each record costs GPU time), and
        the host's enqueue ms per launch.  `count` untimed launches (at least
        200) are queued first without a sync, so the GPU is still busy with
        them while the host enqueues the timed ones: the timed launches never
        wait for the host as long as one enqueue is shorter than one launch's
        GPU time (the host figure says whether it was)."""
        a, b = hip.Event(), hip.Event()
        synced()
        lead = max(count, 200)
        for i in range(lead):
            fn(sets[i % rotate])
        t0 = time.perf_counter()
        a.record(stream)
        for i in range(count):
            fn(sets[i % rotate])
        b.record(stream)
        host_ms = (time.perf_counter() - t0) * 1e3 / count
        synced()
        return a.elapsed_ms(b), host_ms

    def chunk_median(fn, count):
        """Median over CHUNKS event-bracketed chunks of the per-launch ms, in a
        pass of its own (the chunk events cost GPU time, so they never share
        a run with the mean); None unless every chunk has at least 10 launches."""
        if count < 10 * CHUNKS:
            return None
        bounds = [count * c // CHUNKS for c in range(CHUNKS + 1)]
        events = [hip.Event() for _ in range(CHUNKS + 1)]
        synced()
        for i in range(max(count, 200)):
            fn(sets[i % rotate])
        events[0].record(stream)
        for c in range(CHUNKS):
            for i in range(bounds[c], bounds[c + 1]):
                fn(sets[i % rotate])
            events[c + 1].record(stream)
        synced()
        return statistics.median(events[c].elapsed_ms(events[c + 1]) / (bounds[c + 1] - bounds[c])
                                 for c in range(CHUNKS))

    def timed_graph(graph):
        """ms of one replay queued behind an untimed replay of the same graph,
        so the timed one does not include the GPU's idle wait for the host's
        first submission after a sync."""
        a, b = hip.Event(), hip.Event()
        synced()
        graph.launch(stream)
        a.record(stream)
        graph.launch(stream)
        b.record(stream)
        synced()
        return a.elapsed_ms(b)

    def settle(min_steps):
        # GPU clocks ramp up over tens of milliseconds of load: run at least
        # min_steps untimed steps and keep going, 100 at a time, until 80 ms
        # of GPU time has passed.
        done, gpu_ms = 0, 0.0
        while done < min_steps or gpu_ms < settle_ms:
            a, b = hip.Event(), hip.Event()
            a.record(stream)
            for i in range(100):
                step(sets[(done + i) % rotate])
            b.record(stream)
            synced()
            done, gpu_ms = done + 100, gpu_ms + a.elapsed_ms(b)

    for st in sets:  # eager pass: every set quantized once
        quant(st)
        step(st)
    synced()
    settle(warmup)
    total_ms, host_ms = timed_stream(step, steps)
    gemm_total, _ = timed_stream(gemm, steps)
    quant_total, _ = timed_stream(quant, steps)
    step_median = chunk_median(step, steps)
    gemm_median = chunk_median(gemm, steps)
    graph_ms = {"step": None, "gemm": None, "quant": None}
    if USE_GRAPHS:
        for name, fn in (("step", step), ("gemm", gemm), ("quant", quant)):
            g = capture(fn, steps)
            settle(0)
            graph_ms[name] = timed_graph(g) / steps
            g.destroy()
    return {"ms_per_step": total_ms / steps, "ms_per_step_median": step_median, "host_enqueue_ms": host_ms,
            "gemm_ms_mean": gemm_total / steps, "gemm_ms_median": gemm_median, "quant_ms_mean": quant_total / steps,
            "graph_ms_per_step": graph_ms["step"],
            "graph_gemm_ms_mean": graph_ms["gemm"], "graph_quant_ms_mean": graph_ms["quant"], "sets": sets}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(m, k, n, target_s=12.0, min_reps=5):
    """Oracle (portable C11, pthreads, -O2 -march=x86-64-v3 -ffp-contract=off)
    on the same workload: the full opcode-15 semantics (quantize, int32
    accumulate, scale epilogue).  Rows are sampled only if one full pass would
    exceed target_s / min_reps; the median over the repetitions is reported."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle

    online = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or online
    threads = max(1, min(threads, online))
    rng = np.random.default_rng(1234)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    blob = oracle.pack_blob(w, rng.uniform(1e-4, 1e-3, n).astype(np.float32))

    def timed(x):
        t0 = time.perf_counter()
        oracle.linear(x, blob, k, n, nthreads=threads)
        return time.perf_counter() - t0

    probe_rows = min(m, max(threads, 16))
    t_probe = timed(rng.standard_normal((probe_rows, k), dtype=np.float32))
    per_row = max(t_probe / probe_rows, 1e-9)
    rows = int(min(m, max(probe_rows, target_s / min_reps / per_row)))
    x = rng.standard_normal((rows, k), dtype=np.float32)
    # the probe carries fixed costs (thread start-up): re-estimate once at size
    t_first = timed(x)
    grown = int(min(m, rows * (target_s / min_reps) / max(t_first, 1e-9)))
    if grown > rows * 1.2:
        rows = grown
        x = rng.standard_normal((rows, k), dtype=np.float32)
    times = []
    t_start = time.perf_counter()
    while len(times) < min_reps or (time.perf_counter() - t_start < target_s and len(times) < 200):
        times.append(timed(x))
    med = statistics.median(times)
    tops = 2.0 * rows * n * k / med / 1e12
    return {"value": round(tops, 4), "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"{rows} of {m} rows x K={k} x N={n} (full opcode-15 semantics), median of {len(times)} "
                      f"reps, {med * 1e3:.1f} ms each, {time.perf_counter() - t_start:.1f} s total",
            "cpu_model": cpu_model(), "online_cores": online}


def e2e_opcode15(m, k, n, reps=10):
    """Opcode 15 through execute_op_simple (the executor's validation, weight
    cache lookup, launch and stream sync), on rpcmem buffers in HBM and on
    pinned host buffers (the latter adds the H2D of x and the D2H of y)."""
    rng = np.random.default_rng(99)
    x = rng.standard_normal((m, k), dtype=np.float32)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    blob = hip.pack_constants(w, rng.uniform(1e-4, 1e-3, n).astype(np.float32))
    out = {}
    for where, device in (("device_rpcmem", True), ("host_rpcmem", False)):
        bufs = [hip.RpcBuffer(m * n * 4, device=device), hip.RpcBuffer(m * k * 4, device=device),
                hip.RpcBuffer(blob.nbytes, device=device)]
        bufs[1].write(x)
        bufs[2].write(blob)
        payload = hip.w8a8_params((bufs[0].fd, 0), (bufs[1].fd, 0), (bufs[2].fd, 0), m, k, n)
        times = []
        for i in range(reps + 2):
            t0 = time.perf_counter()
            rc, after = hip.execute(hip.OP_MAT_MUL_NATIVE_W8A8, payload)
            if rc != 0:
                raise RuntimeError(f"opcode 15 returned {rc}: {hip.last_error()}")
            if i >= 2:
                times.append(time.perf_counter() - t0)
        elapsed_us = int.from_bytes(after[36:40], "little", signed=True)
        out[where] = {"ms_median": round(statistics.median(times) * 1e3, 4), "elapsed_us_field": elapsed_us}
        for b in bufs:
            b.free()
    return out


def e2e_mailbox(cases, reps=20):
    """Opcode 15 through the message channel, as sd.cpp drives it: the request
    is written into the channel buffer, the state word's v0 is raised, and the
    caller spins until the executor's polling thread publishes v1 (after the
    request's kernels have completed).  One single-request message per rep on
    rpcmem buffers in HBM; the median over `reps` after 3 untimed reps."""
    lib = hip.lib()
    if lib.open_dsp_session(3, 1) != 0:
        raise RuntimeError("open_dsp_session failed: " + hip.last_error())
    lib.init_htp_backend()
    cap = 4096
    chan = hip.RpcBuffer(cap)
    if lib.create_htp_message_channel(chan.fd, cap) != 0:
        raise RuntimeError("create_htp_message_channel failed: " + hip.last_error())
    view = chan.host_view()
    rng = np.random.default_rng(98)
    out = {}
    try:
        for name, (m, k, n) in cases.items():
            x = rng.standard_normal((m, k), dtype=np.float32)
            w = rng.integers(-127, 128, (n, k), dtype=np.int8)
            blob = hip.pack_constants(w, rng.uniform(1e-4, 1e-3, n).astype(np.float32))
            bufs = [hip.RpcBuffer(m * n * 4, device=True), hip.RpcBuffer(m * k * 4, device=True),
                    hip.RpcBuffer(blob.nbytes, device=True)]
            bufs[1].write(x)
            bufs[2].write(blob)
            req = hip.compute_request(hip.OP_MAT_MUL_NATIVE_W8A8,
                                      hip.w8a8_params((bufs[0].fd, 0), (bufs[1].fd, 0), (bufs[2].fd, 0), m, k, n))
            msg, offs = hip.build_message([(hip.REQUEST_TYPE_OP_COMPUTE, req)], cap)
            body = np.frombuffer(bytes(msg[8:offs[-1]]), np.uint8)
            times = []
            for i in range(reps + 3):
                view[8:offs[-1]] = body
                view[:8] = 0
                t0 = time.perf_counter()
                view[0] = 1
                deadline = t0 + 10.0
                while view[1] != 1:
                    if time.perf_counter() > deadline:
                        raise RuntimeError(f"mailbox request {name} did not complete")
                t1 = time.perf_counter()
                if i >= 3:
                    times.append(t1 - t0)
            done = bytes(view[:offs[-1]].tobytes())
            state = hip.request_state(done, offs, 0)
            if state != 0:
                raise RuntimeError(f"mailbox request {name} returned {state}")
            elapsed_us = int.from_bytes(hip.request_data(done, offs, 0)[4 + 36:4 + 40], "little", signed=True)
            out[name] = {"shape": f"M={m} K={k} N={n}", "us_median": round(statistics.median(times) * 1e6, 1),
                         "us_min": round(min(times) * 1e6, 1), "elapsed_us_field": elapsed_us, "reps": reps}
            for b in bufs:
                b.free()
    finally:
        lib.destroy_htp_message_channel()
        lib.close_dsp_session()
        chan.free()
    return out


KERNEL_SOURCE = os.path.join(REPO, "htp-ops-lib-sd.cpp_amd", "csrc", "hip", "w8a8.hip")


def kernel_source_sha16():
    """First 16 hex digits of the SHA-256 of the W8A8 kernel source: the
    provenance key of the committed counter summary."""
    import hashlib
    with open(KERNEL_SOURCE, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def read_traffic():
    """HBM bytes per headline GEMM launch from the committed PMC summary, and
    whether that summary is stale: it records the kernel source hash it was
    measured on (`kernel_source_sha16:`), and a different hash now (or none)
    means the kernel changed since, so the figure is reported as stale
    instead of silently reused."""
    try:
        with open(TRAFFIC_FILE) as f:
            text = f.read()
    except OSError:
        return None, None
    match = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", text, re.M)
    src = re.search(r"^kernel_source_sha16:\s*([0-9a-f]{16})", text, re.M)
    stale = src is None or src.group(1) != kernel_source_sha16()
    return (int(match.group(1)) if match else None), stale


def decode_case(m, k, n, steps, warmup, rotate):
    r = run_w8a8(m, k, n, steps, warmup, rotate, scale=(5e-5, 5e-4))
    op_bytes = w8a8_bytes(m, k, n)
    # the path hb_w8a8_linear takes at these shapes (k % 32 == 0, n % 16 == 0)
    kp = (k + 63) // 64 * 64
    if m == 1 and kp <= 32 * 512:
        path = "fused quantize+GEMM kernel"
    elif 2 <= m <= 4 and kp <= 8 * 8 * 64:
        path = "fused few-row quantize+GEMM kernel"
    else:
        path = "quantize, GEMM"
    return {"shape": f"M={m} K={k} N={n}", "path": path,
            "us_per_call": round(r["ms_per_step"] * 1e3, 3),
            "gbps": round(op_bytes / (r["ms_per_step"] * 1e-3) / 1e9, 1),
            "frac_hbm": round(op_bytes / (r["ms_per_step"] * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
            "gemm_us": round(r["gemm_ms_mean"] * 1e3, 3),
            "gemm_gbps": round(gemm_bytes(m, k, n) / (r["gemm_ms_mean"] * 1e-3) / 1e9, 1),
            "quant_us": round(r["quant_ms_mean"] * 1e3, 3), "rotated_sets": rotate,
            "us_per_call_median": _us(r["ms_per_step_median"]),
            "host_enqueue_us": _us(r["host_enqueue_ms"]),
            "graph_us_per_call": None if r["graph_ms_per_step"] is None else round(r["graph_ms_per_step"] * 1e3, 3)}


def all_configs(steps, warmup, with_cpu=False, only=None):
    """Every BASELINE configuration; `only`: a set of case names to run alone."""
    def wanted(name):
        return only is None or name in only

    out = {}
    for name, (m, k, n, outl, sc) in {
            "C1_77x768x3072": (77, 768, 3072, 0.0, (1e-4, 1e-3)),
            "C3_qkv_4096x1536x4608": (4096, 1536, 4608, 0.01, (1e-4, 1e-3)),
            "C3_up_gelu_4096x1536x6144": (4096, 1536, 6144, 0.01, (1e-4, 1e-3)),
            "C3_down_4096x6144x1536": (4096, 6144, 1536, 0.01, (1e-4, 1e-3)),
            "C4_qkv_2048x4096x6144": (2048, 4096, 6144, 0.0, (5e-5, 5e-4)),
            "C4_o_2048x4096x4096": (2048, 4096, 4096, 0.0, (5e-5, 5e-4))}.items():
        if not wanted(name):
            continue
        progress(f"start {name}")
        r = run_w8a8(m, k, n, steps, warmup, 4, outliers=outl, scale=sc,
                     epilogue=hip.EPI_SCALE_GELU if "gelu" in name else None)
        out[name] = {"us": round(r["ms_per_step"] * 1e3, 2), "us_median": _us(r["ms_per_step_median"]),
                     "tops": round(2 * m * n * k / (r["ms_per_step"] * 1e-3) / 1e12, 1),
                     "gemm_us": round(r["gemm_ms_mean"] * 1e3, 2)}
        del r
        progress(f"done {name}: {out[name]['us']} us")
    for m in (1, 4, 16):
        for k, n in ((4096, 14336), (14336, 4096)):
            if not wanted(f"C5_M{m}_{k}x{n}"):
                continue
            progress(f"start C5 M={m} {k}x{n}")
            out[f"C5_M{m}_{k}x{n}"] = decode_case(m, k, n, steps, warmup, 6)
            progress(f"done C5 M={m} {k}x{n}: {out[f'C5_M{m}_{k}x{n}']['us_per_call']} us")
    if wanted("C2_f16_text_mlp_77x768x3072x768"):
        progress("start C2")
        out["C2_f16_text_mlp_77x768x3072x768"] = f16_mlp_case(steps, warmup)
    if wanted("f16_vae_mode3"):
        progress("start F16 VAE convolutions")
        out["f16_vae_mode3"] = f16_vae_cases(steps, warmup)
    if wanted("f16_unet_mode3"):
        progress("start F16 UNet convolutions")
        out["f16_unet_mode3"] = f16_vae_cases(steps, warmup, cases=UNET_CASES, workspace=True)
    if wanted("opcode19_aux"):
        progress("start opcode 19")
        out["opcode19_aux"] = aux_cases(steps, warmup, with_cpu=with_cpu)
    if wanted("opcodes_2_3_4_qk0"):
        progress("start opcodes 2/3/4")
        out["opcodes_2_3_4_qk0"] = qk0_cases(steps, warmup)
    progress("done all configs")
    return out


def _timed_graph_us(launch, steps, warmup, stream):
    """Settles the clock with stream-ordered launches, then the mean of one
    graph replay of `steps` launches (µs per launch); with --no-graph, the
    mean of `steps` stream-ordered launches instead."""
    lib = hip.lib()
    done, gpu_ms = 0, 0.0
    while done < max(warmup, 1) or gpu_ms < SETTLE_MS:
        a, b = hip.Event(), hip.Event()
        a.record(stream)
        for i in range(50):
            launch(done + i)
        b.record(stream)
        hip.check(lib.hb_stream_sync(stream), "sync")
        done, gpu_ms = done + 50, gpu_ms + a.elapsed_ms(b)
    a, b = hip.Event(), hip.Event()
    if not USE_GRAPHS:
        a.record(stream)
        for i in range(steps):
            launch(i)
        b.record(stream)
        hip.check(lib.hb_stream_sync(stream), "sync")
        return a.elapsed_ms(b) * 1e3 / steps
    with hip.Graph.capture(stream) as g:
        for i in range(steps):
            launch(i)
    hip.check(lib.hb_stream_sync(stream), "sync")
    g.launch(stream)  # untimed replay ahead of the timed one (no idle wait for the host inside it)
    a.record(stream)
    g.launch(stream)
    b.record(stream)
    hip.check(lib.hb_stream_sync(stream), "sync")
    g.destroy()
    return a.elapsed_ms(b) * 1e3 / steps


def qk0_cases(steps, warmup, rotate=4):
    """Opcodes 2/3/4 (Q4_0 / Q8_0 / IQ4_NL weights) at BASELINE C5's gate/up
    shape (K=4096, N=14336).  m <= 16 multiplies the super-blocks directly
    (`direct_*`: algorithmic bytes 4MK + K*N*block/256 + 4MN, the quantized
    weights read once); larger m runs the F16 GEMM on the dequantized image
    (`f16_image_*`, identical for the three formats; the one-time
    dequantizing prepack is `prepack_us`).  Graph-replayed means over
    `rotate` weight sets."""
    lib = hip.lib()
    stream = hip.default_stream()
    rng = np.random.default_rng(4)
    k, n = 4096, 14336
    out = {"prepack_us": {}}
    block_bytes = {hip.GGML_Q4_0: 144, hip.GGML_Q8_0: 272, hip.GGML_IQ4_NL: 144}
    names = {hip.GGML_Q4_0: "q4_0", hip.GGML_Q8_0: "q8_0", hip.GGML_IQ4_NL: "iq4_nl"}
    image_sets = []
    for wtype, bb in block_bytes.items():
        nb = k * n // 256
        sets = []
        for _ in range(rotate):
            blocks = rng.integers(0, 256, nb * bb, dtype=np.uint8).reshape(nb, bb)
            blocks[:, :16] = (rng.uniform(1e-3, 2e-3, nb * 8).astype(np.float16)).view(np.uint8).reshape(nb, 16)
            sets.append(hip.DeviceBuffer.from_array(blocks.ravel()))
        packed = hip.DeviceBuffer(lib.hb_f16_packed_bytes(k, n))
        for _ in range(3):  # the first call pays module load; report the third
            a, b = hip.Event(), hip.Event()
            a.record(stream)
            hip.check(lib.hb_qk0_prepack(packed.ptr, sets[0].ptr, k, n, wtype, stream), "hb_qk0_prepack")
            b.record(stream)
            hip.check(lib.hb_stream_sync(stream), "sync")
        out["prepack_us"][names[wtype]] = round(a.elapsed_ms(b) * 1e3, 1)
        if wtype == hip.GGML_Q4_0:
            image_sets.append(packed)
        else:
            packed.free()
        for m in (1, 4, 16):
            x = hip.DeviceBuffer.from_array(rng.standard_normal((m, k), dtype=np.float32))
            y = hip.DeviceBuffer(m * n * 4)
            ws = hip.DeviceBuffer(hip.f16_workspace_bytes(m, k, n))

            def launch(i):
                hip.check(lib.hb_qk0_gemm_ws(y.ptr, x.ptr, sets[i % rotate].ptr, m, k, n, wtype, ws.ptr, ws.nbytes,
                                             stream), "hb_qk0_gemm_ws")

            us = _timed_graph_us(launch, steps, warmup, stream)
            nbytes = 4 * m * k + k * n // 256 * bb + 4 * m * n
            out[f"direct_{names[wtype]}_M{m}_{k}x{n}"] = {
                "us": round(us, 2), "gbps": round(nbytes / us * 1e-3, 1),
                "frac_hbm": round(nbytes / us * 1e-3 / PEAK_HBM_GBPS, 4)}
            for buf in (x, y, ws):
                buf.free()
        for buf in sets:
            buf.free()
    while len(image_sets) < rotate:
        image_sets.append(hip.DeviceBuffer(lib.hb_f16_packed_bytes(k, n)))
        hip.check(lib.hb_memcpy_d2d(image_sets[-1].ptr, image_sets[0].ptr, image_sets[0].nbytes, stream), "copy")
    for m in (77, 2048):
        x = hip.DeviceBuffer.from_array(rng.standard_normal((m, k), dtype=np.float32))
        y = hip.DeviceBuffer(m * n * 4)
        ws = hip.DeviceBuffer(max(hip.f16_workspace_bytes(m, k, n), 256))

        def launch(i):
            hip.check(lib.hb_f16_gemm_ws(y.ptr, x.ptr, image_sets[i % rotate].ptr, None, m, k, n, n, 0, ws.ptr,
                                         ws.nbytes, stream), "hb_f16_gemm_ws")

        us = _timed_graph_us(launch, steps if m < 2048 else max(steps // 10, 20), warmup, stream)
        nbytes = 4 * m * k + 2 * n * k + 4 * m * n  # the fp16 image read per call
        out[f"f16_image_M{m}_{k}x{n}"] = {"us": round(us, 2), "tflops": round(2 * m * n * k / us * 1e-6, 2),
                                          "gbps": round(nbytes / us * 1e-3, 1),
                                          "frac_hbm": round(nbytes / us * 1e-3 / PEAK_HBM_GBPS, 4)}
        for buf in (x, y, ws):
            buf.free()
    for p in image_sets:
        p.free()
    return out


def aux_cases(steps, warmup, rotate=4, with_cpu=True):
    """Opcode-19 model auxiliary ops at DiT/VAE shapes (hb_model_aux on HBM
    tensors, rotated copies, stream-ordered after clock settling).  Bytes are
    the algorithmic ones: every input value read once, every output written
    once."""
    lib = hip.lib()
    stream = hip.default_stream()
    rng = np.random.default_rng(5)
    tok, width, ff, heads, dim = 4096, 1536, 6144, 24, 64
    cases = {
        # name: (kw, input floats, weight floats, bias floats, output floats)
        "ln_modulation_4096x1536": (dict(mode=9, count=tok * width, width=width, spatial=tok, batch=1,
                                         other_count=width, eps=1e-6), tok * width, width, width, tok * width),
        "rms_norm_4096x1536": (dict(mode=1, count=tok * width, width=width, other_count=width, eps=1e-6),
                               tok * width, width, 0, tok * width),
        "group_norm_512ch_64x64": (dict(mode=2, count=512 * 4096, width=4096, channels=512, spatial=4096, groups=32,
                                        batch=1, other_count=512, eps=1e-6), 512 * 4096, 512, 512, 512 * 4096),
        "group_norm_128ch_512x512": (dict(mode=2, count=128 * 262144, width=262144, channels=128, spatial=262144,
                                          groups=32, batch=1, other_count=128, eps=1e-6), 128 * 262144, 128, 128,
                                     128 * 262144),
        "swiglu_4096x6144": (dict(mode=12, count=tok * ff, width=ff, channels=2 * ff, spatial=tok, activation=1),
                             tok * 2 * ff, 0, 0, tok * ff),
        "gelu_4096x6144": (dict(mode=6, count=tok * ff, width=ff), tok * ff, 0, 0, tok * ff),
        "rope_4096tok_24x64": (dict(mode=11, count=tok * heads * dim, width=dim, channels=heads, spatial=tok,
                                    groups=1, batch=1, other_count=2 * dim * tok), tok * heads * dim, 2 * dim * tok, 0,
                               tok * heads * dim),
        "transpose_512x4096": (dict(mode=8, count=512 * 4096, width=512, spatial=4096, batch=1), 512 * 4096, 0, 0,
                               512 * 4096),
    }
    out = {}
    for name, (kw, nx, nw, nb, ny) in cases.items():
        sets = []
        for r in range(rotate):
            hx = rng.standard_normal(nx, dtype=np.float32)
            hw = rng.standard_normal(nw, dtype=np.float32) * 0.1 if nw else None
            hb = rng.standard_normal(nb, dtype=np.float32) * 0.1 if nb else None
            if r == 0:
                host = (hx, hw, hb)
            x = hip.DeviceBuffer.from_array(hx)
            w = hip.DeviceBuffer.from_array(hw) if nw else None
            b = hip.DeviceBuffer.from_array(hb) if nb else None
            y = hip.DeviceBuffer(ny * 4)
            sets.append((x, w, b, y))

        wsb = hip.model_aux_workspace_bytes(kw["mode"], kw.get("channels", 1), kw.get("spatial", 1),
                                            kw.get("groups", 1), kw.get("batch", 1))
        ws = hip.DeviceBuffer(wsb) if wsb else None

        def launch(i):
            x, w, b, y = sets[i % rotate]
            hip.model_aux(y, x, w, b, stream=stream, workspace=ws, **kw)

        done, gpu_ms = 0, 0.0
        while done < max(warmup, 1) or gpu_ms < SETTLE_MS:
            a, e = hip.Event(), hip.Event()
            a.record(stream)
            for i in range(100):
                launch(done + i)
            e.record(stream)
            hip.check(lib.hb_stream_sync(stream), "sync")
            done, gpu_ms = done + 100, gpu_ms + a.elapsed_ms(e)
        a, e = hip.Event(), hip.Event()
        a.record(stream)
        for i in range(steps):
            launch(i)
        e.record(stream)
        hip.check(lib.hb_stream_sync(stream), "sync")
        us = a.elapsed_ms(e) * 1e3 / steps
        nbytes = 4 * (nx + nw + nb + ny)
        out[name] = {"mode": kw["mode"], "us": round(us, 2), "gbps": round(nbytes / us * 1e-3, 1),
                     "frac_hbm": round(nbytes / us * 1e-3 / PEAK_HBM_GBPS, 4)}
        if with_cpu:
            # the oracle's single-threaded restatement on the same values, once
            sys.path.insert(0, os.path.join(REPO, "oracle"))
            import oracle
            t0 = time.perf_counter()
            oracle.model_aux(*host, **kw)
            cpu_us = (time.perf_counter() - t0) * 1e6
            out[name]["cpu_baseline"] = {"us": round(cpu_us, 1), "gbps": round(nbytes / cpu_us * 1e-3, 2),
                                         "cores": 1, "kind": "port"}
        for st in sets:
            for buf in st:
                if buf is not None:
                    buf.free()
    return out


def qkv_cases(steps, warmup, with_cpu=True):
    """Opcode 12 (dual fused QKV + RMS norm + RoPE, packed fp16 outputs) at
    joint-attention shapes: image 256 + text 4096 tokens, input 1536.  The
    request runs through execute_op_simple on HBM-resident rpcmem buffers
    (mean over `steps` requests after `warmup`); its two kernels are timed
    alone on the text part (HIP events around `steps` launches each).
    Post-processing bytes are algorithmic: the GEMM output read once (f32),
    the rotary matrices of the rows read once, three packed fp16 images
    written once."""
    import struct
    lib = hip.lib()
    stream = hip.default_stream()
    rng = np.random.default_rng(12)
    out = {}
    for n_heads, hd in ((24, 64), (24, 128)):
        image, text, k = 256, 4096, 1536
        tokens = image + text
        cols = 3 * n_heads * hd
        tiles = (tokens + 31) // 32
        name = f"qkv_dual_rope_{image}+{text}x{k}_{n_heads}x{hd}"
        act = rng.standard_normal((tokens, k), dtype=np.float32)
        w = (rng.standard_normal((k, cols), dtype=np.float32) * 0.03).astype(np.float16)
        perm = hip.permute_f16(w.view(np.uint16))
        bias = rng.standard_normal(cols, dtype=np.float32) * 0.1
        qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
        kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
        ang = rng.uniform(-3, 3, (tokens, hd // 2))
        pe = np.stack([np.cos(ang), -np.sin(ang), np.sin(ang), np.cos(ang)], -1).astype(np.float32).ravel()
        qkv_bytes = n_heads * tiles * (hd // 32) * 1024 * 2
        pieces = [("act", act), ("w", perm), ("bias", bias), ("qn", qn), ("kn", kn), ("pe", pe)]
        offs, pos = {}, 0
        for key, arr in pieces:
            offs[key] = pos
            pos = (pos + arr.nbytes + 255) // 256 * 256
        for key in ("q", "k", "v"):
            offs[key] = pos
            pos = (pos + qkv_bytes + 255) // 256 * 256
        buf = hip.RpcBuffer(pos, device=True)
        for key, arr in pieces:
            buf.write(arr, offs[key])
        a = {key: (buf.fd, o) for key, o in offs.items()}
        img = (a["act"], a["w"], a["bias"], a["qn"], a["kn"])
        txt = ((buf.fd, offs["act"] + image * k * 4), a["w"], a["bias"], a["qn"], a["kn"])
        payload = hip.qkv_dual_rope_params(a["q"], a["k"], a["v"], img, txt, a["pe"], image, text, k, n_heads, hd,
                                           0, image)
        for _ in range(max(warmup // 10, 3)):
            rc, _ = hip.execute(12, payload)
            assert rc == 0, hip.last_error()
        hip.sync()
        n_req = max(steps // 10, 10)
        elapsed = []
        t0 = time.perf_counter()
        for _ in range(n_req):
            rc, after = hip.execute(12, payload)
            elapsed.append(struct.unpack_from("<i", after, len(after) - 4)[0])
        hip.sync()
        wall_us = (time.perf_counter() - t0) / n_req * 1e6
        # the two kernels alone on the text part
        m = text
        packed = hip.f16_prepack(hip.DeviceBuffer.from_array(perm), k, cols)
        x = hip.DeviceBuffer.from_array(act[image:])
        y = hip.DeviceBuffer(m * cols * 4)
        ws = hip.DeviceBuffer(max(hip.f16_workspace_bytes(m, k, cols), 1))
        outs = [hip.DeviceBuffer(qkv_bytes) for _ in range(3)]
        bd, qd, kd, ped = (hip.DeviceBuffer.from_array(v) for v in (bias, qn, kn, pe))

        def gemm(i):
            hip.f16_gemm(y, x, packed, None, m, k, cols, cols, 0, stream=stream, workspace=ws)

        def post(i):
            hip.qkv_post(*outs, y, bd, qd, kd, ped, image, tokens, m, n_heads, hd, tiles, image, stream=stream)

        fws = hip.DeviceBuffer(hip.qkv_gemm_workspace_bytes(m, k))
        xt = hip.DeviceBuffer.from_array(act[image:])

        def fused(i):
            hip.qkv_gemm(*outs, xt, packed, bd, qd, kd, ped, image, tokens, m, k, n_heads, hd, tiles, image, fws,
                         stream=stream)

        gemm_us = _timed_graph_us(gemm, steps, warmup, stream)
        post_us = _timed_graph_us(post, steps, warmup, stream)
        fused_us = _timed_graph_us(fused, steps, warmup, stream)
        post_bytes = m * cols * 4 + m * (hd // 2) * 16 + 3 * ((m + 31) // 32 * 32) * n_heads * hd * 2
        flops = 2.0 * m * k * cols
        out[name] = {
            "op12_us_wall": round(wall_us, 1), "op12_elapsed_us_median": int(np.median(elapsed)),
            "gemm_us": round(gemm_us, 2), "gemm_tflops": round(flops / gemm_us * 1e-6, 1),
            "gemm_frac_fp16_mfma": round(flops / gemm_us * 1e-6 / PEAK_F16_TFLOPS, 4),
            "post_us": round(post_us, 2), "post_gbps": round(post_bytes / post_us * 1e-3, 1),
            "post_frac_hbm": round(post_bytes / post_us * 1e-3 / PEAK_HBM_GBPS, 4),
            "post_algorithmic_bytes": post_bytes, "fused_gemm_post_us": round(fused_us, 2)}
        if with_cpu and n_heads == 24 and hd == 64:
            # the oracle's restatement (GEMM + post-processing) of the image
            # part, single-threaded
            sys.path.insert(0, os.path.join(REPO, "oracle"))
            import oracle
            t0 = time.perf_counter()
            raw = oracle.f16_gemm_epilogue(act[:image], perm, None, image, k, cols, cols, 0, nthreads=1)
            oracle.qkv_post(raw, bias, qn, kn, pe, 0, tokens, image, n_heads, hd, tiles)
            cpu_s = time.perf_counter() - t0
            out[name]["cpu_baseline"] = {"us_per_token": round(cpu_s / image * 1e6, 1), "cores": 1, "kind": "port",
                                         "sample": f"image part: {image} tokens (GEMM {image}x{k}x{cols} + "
                                                   f"post-processing)",
                                         "gpu_us_per_token": round(wall_us / tokens, 3)}
        for b in (packed, x, y, ws, *outs, bd, qd, kd, ped, fws, xt):
            b.free()
        buf.free()
    return out


def f16_mlp_case(steps, warmup, m=77, k=768, n=3072, rotate=6):
    """opcode-16 F16 GEMM 77x768 -> 3072 with bias +
    QuickGELU, then 3072 -> 768 with bias (text-encoder MLP block); FP32
    activations, FP16 weights prepacked once, HBM-resident.  Each layer's
    graph-replayed mean is reported with its algorithmic bytes
    (4MK + 2NK + 4N + 4MN) and flops (2MNK)."""
    lib = hip.lib()
    stream = hip.default_stream()
    rng = np.random.default_rng(2)
    layers = []
    for (kk, nn, mode) in ((k, n, 2), (n, k, 0)):
        sets = []
        for _ in range(rotate):
            w = (rng.standard_normal((kk, nn), dtype=np.float32) * 0.02).astype(np.float16)
            perm = hip.permute_f16(w.view(np.uint16))
            pd = hip.DeviceBuffer.from_array(perm)
            packed = hip.f16_prepack(pd, kk, nn)
            pd.free()
            bias = hip.DeviceBuffer.from_array((rng.standard_normal(nn, dtype=np.float32) * 0.02))
            sets.append((packed, bias))
        layers.append((kk, nn, mode, sets))
    x = hip.DeviceBuffer.from_array(rng.standard_normal((m, k), dtype=np.float32))
    h = hip.DeviceBuffer(m * n * 4)
    y = hip.DeviceBuffer(m * k * 4)
    ios = [(x, h), (h, y)]
    out = {}
    for li, (kk, nn, mode, sets) in enumerate(layers):
        src, dst = ios[li]
        ws = hip.DeviceBuffer(max(hip.f16_workspace_bytes(m, kk, nn), 256))

        def launch(i):
            packed, bias = sets[i % rotate]
            hip.check(lib.hb_f16_gemm_ws(dst.ptr, src.ptr, packed.ptr, bias.ptr, m, kk, nn, nn, mode, ws.ptr,
                                         ws.nbytes, stream), "hb_f16_gemm_ws")

        done, gpu_ms = 0, 0.0
        while done < max(warmup, 1) or gpu_ms < SETTLE_MS:  # clock settling, as in run_w8a8
            a, b = hip.Event(), hip.Event()
            a.record(stream)
            for i in range(200):
                launch(done + i)
            b.record(stream)
            hip.check(lib.hb_stream_sync(stream), "sync")
            done, gpu_ms = done + 200, gpu_ms + a.elapsed_ms(b)
        us = _timed_graph_us(launch, steps, 0, stream)
        nbytes = 4 * m * kk + 2 * nn * kk + 4 * nn + 4 * m * nn
        out["layer1_quickgelu" if li == 0 else "layer2_bias"] = {
            "shape": f"M={m} K={kk} N={nn} mode={mode}", "us": round(us, 3),
            "tflops": round(2 * m * nn * kk / us * 1e-6, 2), "gbps": round(nbytes / us * 1e-3, 1),
            "frac_hbm": round(nbytes / us * 1e-3 / PEAK_HBM_GBPS, 4)}
    return out


VAE_CASES = {  # im2col GEMMs of a VAE decoder's 3x3 convolutions (512x512 output): M pixels, K = 9 x in-channels
    "vae_conv_128x128_512ch": (16384, 4608, 512),
    "vae_conv_256x256_256ch": (65536, 2304, 256),
    "vae_conv_512x512_128ch": (262144, 1152, 128),
}

UNET_CASES = {  # the same for a 512x512 UNet's 3x3 convolutions (64x64 latent), with the F16 workspace
    "unet_conv_16x16_1280ch": (256, 11520, 1280),
    "unet_conv_32x32_640ch": (1024, 5760, 640),
    "unet_conv_64x64_320ch": (4096, 2880, 320),
}


def f16_vae_cases(steps, warmup, rotate=2, cases=None, workspace=False):
    """Opcode 16 mode 3 (bias, channel-major [channels][M] output) at the
    VAE decoder's convolution shapes: FP32 activations read once by the
    activation-streaming kernel (no workspace); with workspace=True and
    UNET_CASES the UNet's (the ring kernel and the split-K ring path).
    Graph-replayed mean per call with its algorithmic bytes (4MK + 2NK + 4N
    + 4MN) and flops (2MNK)."""
    lib = hip.lib()
    stream = hip.default_stream()
    rng = np.random.default_rng(5)
    out = {}
    for name, (m, k, n) in (VAE_CASES if cases is None else cases).items():
        sets = []
        for _ in range(rotate):
            w = (rng.standard_normal((k, n), dtype=np.float32) * 0.02).astype(np.float16)
            pd = hip.DeviceBuffer.from_array(hip.permute_f16(w.view(np.uint16)))
            packed = hip.f16_prepack(pd, k, n)
            pd.free()
            sets.append((packed, hip.DeviceBuffer.from_array(rng.standard_normal(n, dtype=np.float32) * 0.02)))
        x = hip.DeviceBuffer.from_array(rng.standard_normal((m, k), dtype=np.float32))
        y = hip.DeviceBuffer(m * n * 4)
        ws = hip.DeviceBuffer(max(hip.f16_workspace_bytes(m, k, n), 256)) if workspace else None
        ws_ptr, ws_bytes = (ws.ptr, ws.nbytes) if ws else (None, 0)

        def launch(i):
            packed, bias = sets[i % rotate]
            hip.check(lib.hb_f16_gemm_ws(y.ptr, x.ptr, packed.ptr, bias.ptr, m, k, n, n, 3, ws_ptr, ws_bytes, stream),
                      "hb_f16_gemm_ws")

        for i in range(max(warmup, 3)):
            launch(i)
        hip.check(lib.hb_stream_sync(stream), "sync")
        us = _timed_graph_us(launch, max(steps // 10, 20), 0, stream)
        nbytes = 4 * m * k + 2 * n * k + 4 * n + 4 * m * n
        out[name] = {"shape": f"M={m} K={k} N={n} mode=3", "us": round(us, 2),
                     "tflops": round(2 * m * n * k / us * 1e-6, 1), "gbps": round(nbytes / us * 1e-3, 1),
                     "frac_hbm": round(nbytes / us * 1e-3 / PEAK_HBM_GBPS, 4)}
        progress(f"done {name}: {out[name]['us']} us")
        for b in (x, y) + ((ws,) if ws else ()):
            b.free()
        for st in sets:
            for b in st:
                b.free()
    return out


def traffic_probe(steps=12, configs=False, only=None):
    """Workload of the counter passes (FETCH_SIZE, WRITE_SIZE, MFMA busy
    cycles): a plain elementwise copy of COPY_PROBE_BYTES (torch's unary
    kernel, reads and writes each byte once) for calibration, then the
    headline opcode-15 steps and the M=1 decode calls on rotated sets, without
    the clock-settling runs (every dispatch is serialized under counters).
    With configs: then the C3 chain's three layers, the C4 QKV and O layers,
    C5's M=1 down projection, the C2 F16 text MLP and the F16 MLP at DiT size
    (4096x1536x6144, the ring kernel), `steps` calls each;
    `only`: a set of those case names (the headline and decode runs are then
    skipped too)."""
    import torch

    src = torch.empty(COPY_PROBE_BYTES // 4, dtype=torch.float32, device="cuda:0").normal_()
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()
    hip.init(0)
    if only is None:
        m, k, n = HEADLINE
        r = run_w8a8(m, k, n, steps, 2, 6, outliers=0.01, settle_ms=0.0)
        del r
        r = run_w8a8(1, 4096, 14336, steps, 2, 6, scale=(5e-5, 5e-4), settle_ms=0.0)
        print(f"counter probe: decode {r['ms_per_step'] * 1e3:.2f} us", flush=True)
    if configs or only is not None:
        for name, (m, k, n, outl, sc, epi) in {
                "C3_qkv_4096x1536x4608": (4096, 1536, 4608, 0.01, (1e-4, 1e-3), None),
                "C3_up_gelu_4096x1536x6144": (4096, 1536, 6144, 0.01, (1e-4, 1e-3), hip.EPI_SCALE_GELU),
                "C3_down_4096x6144x1536": (4096, 6144, 1536, 0.01, (1e-4, 1e-3), None),
                "C4_qkv_2048x4096x6144": (2048, 4096, 6144, 0.0, (5e-5, 5e-4), None),
                "C4_o_2048x4096x4096": (2048, 4096, 4096, 0.0, (5e-5, 5e-4), None),
                "C5_M1_14336x4096": (1, 14336, 4096, 0.0, (5e-5, 5e-4), None)}.items():
            if only is not None and name not in only:
                continue
            r = run_w8a8(m, k, n, steps, 2, 4, outliers=outl, scale=sc, settle_ms=0.0, epilogue=epi)
            print(f"counter probe: {name} ({hip.w8a8_gemm_kernel(m, k, n)}) {r['ms_per_step'] * 1e3:.2f} us",
                  flush=True)
            del r
        if only is None or "C2_f16_text_mlp_77x768x3072x768" in only:
            r = f16_mlp_case(steps, 2)
            print(f"counter probe: C2 f16 text MLP {r}", flush=True)
        if only is None or "F16_mlp_4096x1536x6144" in only:
            # the F16 driver at DiT MLP size: the ring kernel (f16_gemm_ring)
            r = f16_mlp_case(steps, 2, m=4096, k=1536, n=6144, rotate=2)
            print(f"counter probe: F16 MLP 4096x1536x6144 {r}", flush=True)
    print("counter probe done", flush=True)


def _short(name):
    name = name.replace("(anonymous namespace)::", "")
    return name if len(name) <= 110 else name[:107] + "..."


def profile_summary(directory):
    """Markdown summary of the rocprofv3 CSV files under directory: kernel
    stats, per-dispatch durations grouped by kernel and grid (one group per
    shape a kernel ran at), and counters grouped the same way."""
    lines = []
    for path in sorted(glob.glob(os.path.join(directory, "**", "*kernel_stats.csv"), recursive=True)):
        lines.append(f"### kernel stats ({os.path.relpath(path, directory)})\n")
        lines.append("| kernel | calls | average us | min us | max us | % time |")
        lines.append("|---|---|---|---|---|---|")
        with open(path) as f:
            for row in csv.DictReader(f):
                lines.append(f"| `{_short(row['Name'])}` | {row['Calls']} | {float(row['AverageNs']) / 1e3:.3f} | "
                             f"{float(row['MinNs']) / 1e3:.3f} | {float(row['MaxNs']) / 1e3:.3f} | "
                             f"{float(row['Percentage']):.2f} |")
        lines.append("")
    for path in sorted(glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True)):
        groups = {}
        with open(path) as f:
            for row in csv.DictReader(f):
                key = (_short(row["Kernel_Name"]), int(row["Grid_Size_X"]), int(row["Workgroup_Size_X"]))
                groups.setdefault(key, []).append((int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3)
        lines.append(f"### dispatches by kernel and grid ({os.path.relpath(path, directory)})\n")
        lines.append("| kernel | grid (threads) | workgroup | calls | mean us | median us |")
        lines.append("|---|---|---|---|---|---|")
        for (kernel, grid, wg), durs in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
            lines.append(f"| `{kernel}` | {grid} | {wg} | {len(durs)} | {statistics.fmean(durs):.3f} | "
                         f"{statistics.median(durs):.3f} |")
        lines.append("")
    counters = {}
    for path in sorted(glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)):
        with open(path) as f:
            for row in csv.DictReader(f):
                key = (_short(row["Kernel_Name"]), int(row["Grid_Size"]), row["Counter_Name"])
                counters.setdefault(key, []).append(float(row["Counter_Value"]))
    if counters:
        lines.append("### counters, mean per dispatch, by kernel and grid\n")
        lines.append("| kernel | grid (threads) | counter | mean | dispatches |")
        lines.append("|---|---|---|---|---|")
        for (kernel, grid, counter), vals in sorted(counters.items()):
            lines.append(f"| `{kernel}` | {grid} | {counter} | {statistics.fmean(vals):.1f} | {len(vals)} |")
        lines.append("")
    print("\n".join(lines))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--rotate", type=int, default=6)
    ap.add_argument("--config", default="headline", choices=["headline", "all", "small", "aux", "qk0", "qkv", "vae"],
                    help="small / aux / qk0 / qkv / vae: only the C1 W8A8 and C2 F16 text-MLP cases / the opcode-19 "
                         "cases / the opcode-2/3/4 cases / the opcode-12 fused QKV cases / the F16 mode-3 VAE "
                         "convolution cases (print those cases alone)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="no HIP graph capture or replay (every timing stream-ordered); for profiler-traced runs")
    ap.add_argument("--traffic-probe", action="store_true")
    ap.add_argument("--probe-configs", action="store_true",
                    help="with --traffic-probe: also the C3/C4 layers, C5 M=1 down and the C2 F16 MLP")
    ap.add_argument("--only", metavar="NAMES",
                    help="comma-separated case names: with --config all, run and print only those cases (e.g. "
                         "C3_qkv_4096x1536x4608,C5_M4_14336x4096); with --traffic-probe, only those probe cases "
                         "(the same names)")
    ap.add_argument("--profile-summary", metavar="DIR")
    args = ap.parse_args()
    if args.profile_summary:
        profile_summary(args.profile_summary)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the path is single-GPU; "
              "multi-GPU sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))
    global USE_GRAPHS
    USE_GRAPHS = not args.no_graph
    if args.traffic_probe:
        traffic_probe(configs=args.probe_configs, only=None if not args.only else set(args.only.split(",")))
        return

    hip.init(0)
    if args.config == "small":
        r = run_w8a8(77, 768, 3072, args.steps, args.warmup, 4, scale=(1e-4, 1e-3))
        print(json.dumps({"C1_77x768x3072_us": round(r["ms_per_step"] * 1e3, 2),
                          "C2_f16_text_mlp_77x768x3072x768": f16_mlp_case(args.steps, args.warmup)}), flush=True)
        return
    if args.config == "aux":
        print(json.dumps({"opcode19_aux": aux_cases(args.steps, args.warmup, with_cpu=not args.no_cpu)}), flush=True)
        return
    if args.config == "qk0":
        print(json.dumps({"opcodes_2_3_4_qk0": qk0_cases(args.steps, args.warmup)}), flush=True)
        return
    if args.config == "vae":
        print(json.dumps({"f16_vae_mode3": f16_vae_cases(args.steps, args.warmup),
                          "f16_unet_mode3": f16_vae_cases(args.steps, args.warmup, cases=UNET_CASES,
                                                          workspace=True)}), flush=True)
        return
    if args.config == "qkv":
        print(json.dumps({"opcodes_8_10_11_12_qkv": qkv_cases(args.steps, args.warmup, with_cpu=not args.no_cpu)}),
              flush=True)
        return
    if args.config == "all" and args.only:
        print(json.dumps({"configs": all_configs(args.steps, args.warmup, with_cpu=not args.no_cpu,
                                                 only=set(args.only.split(",")))}), flush=True)
        return
    m, k, n = HEADLINE
    traffic, traffic_stale = read_traffic()
    r = run_w8a8(m, k, n, args.steps, args.warmup, args.rotate, outliers=0.01)
    ops = 2.0 * m * n * k
    tops = ops / (r["ms_per_step"] * 1e-3) / 1e12
    gemm_tops = ops / (r["gemm_ms_mean"] * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "opcode-15 W8A8 linear, M=4096 K=1536 N=6144 (quantize + INT8 MFMA GEMM + "
                               "scale epilogue), HBM-resident inputs, 1% outlier channels x20",
                   "m": m, "k": k, "n": n, "rotated_sets": args.rotate},
        "mfma_frac_full_op": round(tops / PEAK_INT8_TOPS, 4),
        "hbm_gbps_full_op": round(w8a8_bytes(m, k, n) / (r["ms_per_step"] * 1e-3) / 1e9, 1),
        "quant_us": round(r["quant_ms_mean"] * 1e3, 3),
        "us_per_step_median": _us(r["ms_per_step_median"]),
        "host_enqueue_us": _us(r["host_enqueue_ms"]),
        "timing": f"{args.steps} stream-ordered launches between one pair of HIP events on the library stream, "
                  f"queued behind {max(args.steps, 200)} untimed launches (value: their mean" +
                  (f"; median over {CHUNKS} event-bracketed chunks in a separate pass beside it)"
                   if r["ms_per_step_median"] is not None else ")") +
                  ("" if r["graph_ms_per_step"] is None else
                   f"; graph replay of the same steps: {r['graph_ms_per_step'] * 1e3:.3f} us/step, "
                   f"GEMM {r['graph_gemm_ms_mean'] * 1e3:.3f} us"),
        "roofline": {"kernel": hip.w8a8_gemm_kernel(m, k, n), "bound": "mfma", "achieved": round(gemm_tops, 2),
                     "peak": PEAK_INT8_TOPS, "unit": "TOPS", "frac": round(gemm_tops / PEAK_INT8_TOPS, 4),
                     "traffic": traffic, "traffic_stale": traffic_stale,
                     "gemm_us": round(r["gemm_ms_mean"] * 1e3, 3),
                     "gemm_gbps": round(gemm_bytes(m, k, n) / (r["gemm_ms_mean"] * 1e-3) / 1e9, 1),
                     "algorithmic_ops_per_launch": ops,
                     "algorithmic_bytes_per_launch": gemm_bytes(m, k, n)},
    }
    line["roofline"]["gemm_us_median"] = _us(r["gemm_ms_median"])
    if r["graph_gemm_ms_mean"] is not None:
        line["roofline"]["gemm_us_graph"] = _us(r["graph_gemm_ms_mean"])
    del r
    progress(f"headline {line['ms_per_step'] * 1e3:.2f} us/step")
    line["decode_m1"] = decode_case(1, 4096, 14336, args.steps, args.warmup, 6)
    progress(f"decode M=1 {line['decode_m1']['us_per_call']} us")
    line["e2e_opcode15"] = e2e_opcode15(m, k, n)
    line["e2e_mailbox"] = e2e_mailbox({"headline": (m, k, n), "decode_m1": (1, 4096, 14336)})
    progress(f"mailbox e2e {line['e2e_mailbox']['headline']['us_median']} us / "
             f"{line['e2e_mailbox']['decode_m1']['us_median']} us")
    if args.config == "all":
        line["configs"] = all_configs(args.steps, args.warmup, with_cpu=not args.no_cpu)
    if not args.no_cpu and rank == 0:
        line["cpu_baseline"] = cpu_baseline(m, k, n)
    else:
        line["cpu_baseline"] = None
    if rank == 0:
        print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
