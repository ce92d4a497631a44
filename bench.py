"""Benchmark: greedy decode tokens/s of the MiniCPM-2B-shaped int8 decoder
on one MI355X, with the q8 GEMV roofline and the CPU
oracle's rate on the host beside it.

    python bench.py [--gpus 1] [--steps 64] [--warmup 8] [--batch 16]

A step is one greedy decode step of every sequence in the batch (40 layers,
LM head, argmax fed back), replayed as one HIP graph; inputs and weights are
resident in HBM before timing starts. Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
VALU_MAC_PEAK_T = 256 * 64 * 2.4e9 / 2 / 1e12  # non-FMA multiply + add per lane


def log(msg):
    print(msg, file=sys.stderr, flush=True)


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "ks_gemv_decode_minicpm2b_b16_traffic.md")
TRAFFIC_PROFILE_FULLK = os.path.join(ROOT, "profiles", "fq_gemv_decode_minicpm2b_b16_traffic.md")
TRAFFIC_PROFILE_FUSED = os.path.join(ROOT, "profiles", "fk_gemv_decode_minicpm2b_b1_traffic.md")


def traffic_profile(dec):
    """The committed counter summary of the program the session runs."""
    if dec.fused:
        return TRAFFIC_PROFILE_FUSED
    return TRAFFIC_PROFILE_FULLK if dec.program == dec.FULLK else TRAFFIC_PROFILE


SUITE_KERNELS_PROFILE = os.path.join(ROOT, "profiles", "suite_device_api_kernels.md")


def profiled_kernel_us(*names):
    """Kernel-only mean and minimum duration (us) of the named kernels, summed,
    from the rocprofv3 trace of the suite (profiles/suite_device_api_kernels.md),
    or None when the file or a kernel is missing."""
    try:
        rows = {}
        for line in open(SUITE_KERNELS_PROFILE):
            parts = [x.strip() for x in line.strip().strip("|").split("|")]
            if len(parts) == 4 and parts[0].startswith("`"):
                rows[parts[0].strip("`")] = (float(parts[2]), float(parts[3]))
        mean = sum(rows[n][0] for n in names)
        mn = sum(rows[n][1] for n in names)
    except (OSError, KeyError, ValueError):
        return None
    return {"mean_us": round(mean, 2), "min_us": round(mn, 2), "kernels": list(names),
            "source": "profiles/suite_device_api_kernels.md (rocprofv3 per-dispatch durations, "
                      "profiler overhead included)"}


def measured_traffic(path=TRAFFIC_PROFILE):
    """HBM bytes per launch of the decode GEMV from the committed counter
    summary (two rocprofv3 --pmc passes, FETCH_SIZE and WRITE_SIZE, scaled by
    a plain copy's reading; the command is in the file), or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch_mean:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def gemv_roofline(dec, iters):
    """q8 GEMV (the int8 projections of a decode step): mean launch duration
    per shape from HIP events on the session stream, and the step-mix
    achieved bandwidth = sum(bytes) / sum(time) over one launch of each.
    At batch 16 (the full-K program) q/k/v and gate/up are full-K kernels
    (fq_gemv_kernel: rows out, SiLU * up in the gate/up epilogue) and o and
    down k-slice kernels (ks_gemv_kernel on bf16 terms, ks_gemv_i8_kernel on
    f32 rows quantized while staged) whose partials a residual kernel
    reduces; at batch <= 5 the fused full-K kernels (fk_gemv_kernel, with
    their RMSNorm, residual and SiLU work)."""
    per = {}
    tot_b = tot_t = 0.0
    rd_b = rd_t = 0.0
    for which, name in ((0, "qkv"), (1, "o"), (2, "gate_up"), (3, "down")):
        us, nbytes = dec.time_gemv(which, iters)
        per[name] = {"us": round(us, 3), "bytes": int(nbytes),
                     "GBps": round(nbytes / us / 1e3, 1)}
        tot_b += nbytes
        tot_t += us
        # the same shape's weights read by a plain streaming kernel, launched
        # the same way: what one launch of these bytes can reach at best
        r_us, r_b = dec.time_gemv(8 + which, iters)
        per[name]["read_floor"] = {"us": round(r_us, 3), "weight_bytes": int(r_b),
                                   "GBps": round(r_b / r_us / 1e3, 1)}
        rd_b += r_b
        rd_t += r_us
    lm_us, lm_b = dec.time_gemv(4, max(4, iters // 10))
    per["lm_head_bf16"] = {"us": round(lm_us, 3), "bytes": int(lm_b),
                           "GBps": round(lm_b / lm_us / 1e3, 1)}
    # 40 layers of o weights (212 MB) fit the 256 MB Infinity Cache, so its
    # loop may read them warm; the other shapes' 40-layer sets do not fit
    per["o"]["cache"] = "212 MB of o weights fit the 256 MB Infinity Cache: may read warm"
    with_red = None
    if not dec.fused:
        # each projection with the kernel that reduces its partials (o:
        # residual RMSNorm into int8 rows, down: residual RMSNorm; gate/up: on
        # the full-K program none, SiLU * up is in its epilogue, on the k-slice
        # program SiLU * up); q/k/v needs none on the full-K program (its
        # k-slice form's partials are reduced inside the attention kernel)
        with_red = {}
        rb = rt = 0.0
        fullk = dec.program == dec.FULLK
        pairs = ((0, "qkv"), (5, "o+resid_q8"), (6, "gate_up_silu"), (7, "down+resid_q8")) \
            if fullk else ((5, "o+resid_q8"), (6, "gate_up+silu_q8"), (7, "down+resid_q8"))
        for which, name in pairs:
            us, nbytes = dec.time_gemv(which, iters)
            with_red[name] = {"us": round(us, 3), "bytes": int(nbytes),
                              "GBps": round(nbytes / us / 1e3, 1)}
            rb += nbytes
            rt += us
        with_red["frac"] = round(rb / rt / 1e3 / HBM_PEAK_GBS, 4)
        with_red["note"] = ("each projection with the kernel that reduces its partials (none for "
                            "the full-K ones); frac = sum bytes / sum time over them")
    achieved = tot_b / tot_t / 1e3  # GB/s
    gap_us, _ = dec.time_gemv(13, iters)
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(traffic_profile(dec)),
            "traffic_source": os.path.relpath(traffic_profile(dec), ROOT),
            "kernel": ("fk_gemv_kernel (full-K, fused RMSNorm / residual / SiLU epilogues; "
                       "at batch 1 the o projection also merges the attention's four "
                       "position-range partials per head)"
                       if dec.fused else
                       "fq_gemv_kernel (q/k/v and gate/up with SiLU * up; full-K over blocked "
                       "int8 rows), ks_gemv_kernel (o; bf16 terms, k-slice partials) and "
                       "ks_gemv_i8_kernel (down; f32 rows quantized while staged, k-slice "
                       "partials)"
                       if dec.program == dec.FULLK else
                       "ks_gemv_i8_kernel (q/k/v, gate+up, down; int8 rows) and "
                       "ks_gemv_kernel (o; bf16 terms); k-slice partials"),
            "bytes_per_launch_mean": int(tot_b / 4), "us_per_launch_mean": round(tot_t / 4, 3),
            "timing": "graph replay of back-to-back launches (launch gaps included)",
            "read_floor_frac": round(rd_b / rd_t / 1e3 / HBM_PEAK_GBS, 4),
            "empty_kernel_us": round(gap_us, 3),
            "frac_excl_empty_kernel": round(tot_b / (tot_t - 4 * gap_us) / 1e3 / HBM_PEAK_GBS, 4),
            "per_shape": per, "with_reduction": with_red}


def decode_attention(dec, iters):
    """The session's decode attention (one launch per layer, every layer in
    turn, graph-replayed): K and V rows of the cached positions plus the new
    row, against HBM."""
    us, nbytes = dec.time_gemv(12, iters)
    return {"us": round(us, 3), "bytes": int(nbytes), "GBps": round(nbytes / us / 1e3, 1),
            "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "position": dec.position()}


def cpu_baseline(cfg, W, steps, threads):
    """The oracle (C restatement of the reference kernels) decoding on the
    host, at positions 129.. of a KV cache whose first 128 positions hold
    synthetic values (the step cost does not depend on them):
      - 1 thread, batch 1: the reference engine's execution model (a single
        thread, core/src/lib.rs:2); this is `value`;
      - `threads` OpenMP threads (rows split like par_for), batch 1;
      - `threads` threads, batch 16: 16 sequences, one step each per batch
        step (the oracle, like the reference's program, steps one sequence
        at a time; each step appends its row at the same position of one
        cache, which costs what 16 caches would)."""
    from oracle import oracle
    n1 = max(2, steps // 2)
    ref = oracle.DecoderOracle(W, cfg, cap=128 + max(steps, n1) + 2)
    rng = np.random.default_rng(0)
    ref.kcache[:, :, :128, :] = rng.standard_normal(ref.kcache[:, :, :128, :].shape,
                                                    dtype=np.float32)
    ref.vcache[:, :, :128, :] = rng.standard_normal(ref.vcache[:, :, :128, :].shape,
                                                    dtype=np.float32)

    def rate(nthreads, nsteps, batch):
        oracle.set_threads(nthreads)
        ref.step(1, 128)  # warm-up (page in weights)
        t = time.perf_counter()
        tok = 2
        for s in range(nsteps):
            for b in range(batch):
                logits, _ = ref.step((tok + 7919 * b) % cfg["vocab"], 129 + s)
            tok = int(np.argmax(logits))
        return nsteps * batch / (time.perf_counter() - t)

    one = rate(1, n1, 1)
    many = rate(threads, steps, 1)
    many16 = rate(threads, max(1, steps // 8), 16)
    model, physical, logical = host_cpu()
    src = "oracle/vmlm_oracle.c (AVX2 restatement of ops/src/kernels.rs)"
    return {"value": round(one, 3), "unit": "tokens/s", "cores": 1, "kind": "port", "batch": 1,
            "cpu_model": model, "host_physical_cores": physical, "host_logical_cpus": logical,
            "sample": f"{n1} greedy decode steps, batch 1, 1 thread (the reference engine is "
                      f"single-threaded), all 40 layers + LM head at the MiniCPM-2B shape, "
                      f"positions 129..{128 + n1}; {src} on {model}",
            "threads": {
                "batch1": {"value": round(many, 3), "unit": "tokens/s", "cores": threads,
                           "sample": f"{steps} steps, batch 1, {threads} OpenMP threads"},
                "batch16": {"value": round(many16, 3), "unit": "tokens/s", "cores": threads,
                            "sample": f"{max(1, steps // 8)} steps of 16 sequences, one "
                                      f"sequence at a time, {threads} OpenMP threads"}}}


def host_cpu():
    """The host's CPU model name, physical core count and logical CPU count
    (from /proc/cpuinfo; None where unreadable)."""
    model, cores, logical = None, set(), 0
    try:
        phys = core = None
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "processor":
                    logical += 1
                elif k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                    cores.add((phys, core))
    except OSError:
        pass
    return model, (len(cores) or None), (logical or os.cpu_count())


PEAK_BF16_TFLOPS = 2500.0   # dense MFMA bf16
PEAK_FP32_TFLOPS = 157.3    # FP32
PEAK_INT8_TOPS = 5000.0     # dense MFMA int8
Q8_TERMS = 3                # int8 terms per f32 activation in the int8-row path (Q8_T)


_LAST = ["eager"]  # how the last _timed call measured the GPU time


INFINITY_CACHE = 256 << 20  # MI355X last-level (Infinity) cache


def n_sets(set_bytes, iters):
    """Buffer sets an HBM-bound row cycles through: enough that one graph
    replay of `iters` calls streams more than twice the Infinity Cache, so
    each call reads memory the previous ones did not leave cached (capped at
    one set per call)."""
    return max(1, min(iters, -(-2 * INFINITY_CACHE // max(1, set_bytes))))


def cache_note(set_bytes, sets):
    """How an HBM row was timed: cold (its calls cycle through more bytes
    than the Infinity Cache holds, so a set is gone before its next use) or
    warm (what it reads fits that cache)."""
    tot = set_bytes * sets
    if tot > INFINITY_CACHE:
        return f"cold: calls cycle through {sets} buffer sets ({tot / 2**20:.0f} MiB)"
    return (f"warm: {sets} buffer set(s), {tot / 2**20:.1f} MiB in all, fit the 256 MiB "
            f"Infinity Cache")


_EAGER = [False]  # --eager: no graph replay (kernel traces of the suite)


def _timed(L, fn, iters):
    """Mean GPU time per call and host wall time per call. `fn(i)` issues
    call i (HBM-bound rows pick their buffer set from i).

    GPU time: `iters` calls captured into one HIP graph (after 3 warm-up
    calls, so every workspace is in place), the graph replayed for about
    30 ms of warm-up, then 5 times between HIP events on the library stream;
    consecutive kernels keep their in-graph launch gap. When a call's work
    cannot be captured as kernels only, the GPU time is the event time around
    `iters` eager calls instead (then bounded below by the host issue rate).
    Host time: the wall time per eager call."""
    import ctypes as C
    from sparrow_amd import check
    for i in range(3):
        check(fn(i))
    check(L.vmlm_hip_sync())
    e0, e1 = C.c_int(), C.c_int()
    check(L.vmlm_hip_event_record(None, C.byref(e0)))
    t = time.perf_counter()
    for i in range(iters):
        check(fn(i))
    check(L.vmlm_hip_event_record(None, C.byref(e1)))
    check(L.vmlm_hip_sync())
    wall = (time.perf_counter() - t) / iters * 1e6
    ms = C.c_float()
    check(L.vmlm_hip_event_elapsed_ms(e0.value, e1.value, C.byref(ms)))
    eager = ms.value * 1e3 / iters
    graph = C.c_void_p()
    _LAST[0] = "eager (host-issue bound)"
    L.vmlm_hip_event_release_all()
    if _EAGER[0] or L.vmlm_hip_capture_begin(None) != 0:
        return eager, wall
    rc = 0
    for i in range(iters):
        rc = rc or fn(i)
    if L.vmlm_hip_capture_end(None, C.byref(graph)) != 0 or rc or not graph.value:
        return eager, wall
    try:
        # warm-up replays, about 30 ms of GPU work (the clocks settle), then the
        # timed ones
        check(L.vmlm_hip_event_record(None, C.byref(e0)))
        check(L.vmlm_hip_graph_launch(graph, None))
        check(L.vmlm_hip_event_record(None, C.byref(e1)))
        check(L.vmlm_hip_sync())
        check(L.vmlm_hip_event_elapsed_ms(e0.value, e1.value, C.byref(ms)))
        for _ in range(min(200, int(30.0 / max(ms.value, 1e-3)))):
            check(L.vmlm_hip_graph_launch(graph, None))
        check(L.vmlm_hip_sync())
        check(L.vmlm_hip_event_record(None, C.byref(e0)))
        for _ in range(5):
            check(L.vmlm_hip_graph_launch(graph, None))
        check(L.vmlm_hip_event_record(None, C.byref(e1)))
        check(L.vmlm_hip_sync())
        check(L.vmlm_hip_event_elapsed_ms(e0.value, e1.value, C.byref(ms)))
    finally:
        L.vmlm_hip_graph_destroy(graph)
        L.vmlm_hip_event_release_all()
    _LAST[0] = "graph replay"
    return ms.value * 1e3 / (5 * iters), wall


def _cpu_us(fn, budget_s=0.5):
    """Mean host time of the oracle call `fn` (reported beside the GPU figure,
    never the product path): at least one call, more while under budget_s."""
    t = time.perf_counter()
    fn()
    n, el = 1, time.perf_counter() - t
    while el < budget_s and n < 20:
        fn()
        n += 1
        el = time.perf_counter() - t
    return round(el / n * 1e6, 1)


def run_suite(iters, cpu=True):
    """The other BASELINE configs through the device-pointer API, inputs
    resident in HBM: per-call time and the achieved fraction of the roofline
    that bounds each (HBM 8 TB/s, bf16 MFMA 2.5 PF, FP32 157.3 TF). With
    `cpu`, the oracle (C restatement of the reference kernels, OpenMP) is timed
    on the same inputs on the host and reported as cpu_us."""
    import ctypes as C
    from sparrow_amd import check, conn, lib
    L = lib()
    ptrs = []
    orc = None
    if cpu:
        from oracle import oracle as orc
        orc.lib()

    def up(a):
        a = np.ascontiguousarray(a)
        p = C.c_void_p()
        check(L.vmlm_hip_malloc(C.byref(p), a.nbytes))
        check(L.vmlm_hip_memcpy_h2d(p, a.ctypes.data, a.nbytes))
        ptrs.append(p)
        return p

    def zeros(nbytes):
        p = C.c_void_p()
        check(L.vmlm_hip_malloc(C.byref(p), nbytes))
        check(L.vmlm_hip_memset(p, 0, nbytes))
        ptrs.append(p)
        return p

    def bf16(x):
        u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)

    def copies(p, nbytes, n):
        """p and n - 1 device copies of its nbytes (the buffer sets an HBM
        row cycles through)."""
        out = [p]
        for _ in range(n - 1):
            q = C.c_void_p()
            check(L.vmlm_hip_malloc(C.byref(q), nbytes))
            check(L.vmlm_hip_memcpy_d2d(q, p, nbytes))
            ptrs.append(q)
            out.append(q)
        return out

    out = {}
    # config 0: q8 GEMM X f32[16,2304] . (W i8[2304,2304] * scale)^T (+ the M=1 GEMV)
    rng = np.random.default_rng(0)
    n = k = 2304
    x = rng.standard_normal((16, k), dtype=np.float32)
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sc = (np.abs(rng.normal(0, 0.02, n)) / 127 + 1e-6).astype(np.float32)
    cfg0 = {}
    set0 = x.nbytes + q.nbytes + sc.nbytes + 16 * n * 4
    ns0 = n_sets(set0, 10**9)
    dx, dq, ds = copies(up(x), x.nbytes, ns0), copies(up(q), q.nbytes, ns0), \
        copies(up(sc), sc.nbytes, ns0)
    dy = [zeros(16 * n * 4) for _ in range(ns0)]
    for m, nbytes in ((16, 5612544), (1, 5336064)):
        us, wall = _timed(L, lambda i: L.vmlm_hip_gemm_nt_int8(dx[i % ns0], dq[i % ns0],
                                                               ds[i % ns0], dy[i % ns0], m, n, k,
                                                               None), max(iters, ns0))
        gbs = nbytes / us / 1e3
        cfg0[f"M{m}"] = {"us": round(us, 2), "host_us": round(wall, 2), "timing": _LAST[0], "bytes": nbytes,
                         "GBps": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                         "cache": cache_note(set0, ns0)}
    if orc:
        cfg0["cpu_us_M16"] = _cpu_us(lambda: orc.gemm_nt_int8(x, q, sc))
        cfg0["cpu_threads"] = orc.get_threads()
    cfg0["M16"]["kernel_only"] = profiled_kernel_us("gemv_wide_kernel<3, false, 2, 8, true>",
                                                    "gemv_reduce_kernel")
    cfg0["M1"]["kernel_only"] = profiled_kernel_us("fx_gemv_kernel<4, 9, 1, true, false>")
    out["cfg0_q8_gemm"] = cfg0
    # config 1: bf16 A[1024,512] . B[512,2048] (B passed as its [2048,512] transpose)
    rng = np.random.default_rng(1)
    a = bf16(rng.standard_normal((1024, 512), dtype=np.float32))
    bt = bf16((rng.standard_normal((512, 2048), dtype=np.float32) / np.sqrt(512)).T)
    da, db, dc = up(a), up(bt), zeros(1024 * 2048 * 4)
    us, wall = _timed(L, lambda i: L.vmlm_hip_gemm_nt_bf16bf16(da, db, dc, 1024, 2048, 512, None),
                      iters)
    tf = 2147483648 / us / 1e6
    out["cfg1_bf16_gemm"] = {"us": round(us, 2), "host_us": round(wall, 2), "timing": _LAST[0],
                             "TFLOPs": round(tf, 1), "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4),
                             "kernel_only": profiled_kernel_us("gemm_dma_kernel<false, 1, 64, 64, 2>")}
    # config 1's M = 1 variant (the GEMV path of the same entry point)
    b1 = 2048 * 512 * 2 + 512 * 2 + 2048 * 4
    ns1 = n_sets(b1, 10**9)
    db1 = copies(db, bt.nbytes, ns1)
    dc1 = [zeros(2048 * 4) for _ in range(ns1)]
    us1, wall1 = _timed(L, lambda i: L.vmlm_hip_gemm_nt_bf16bf16(da, db1[i % ns1], dc1[i % ns1], 1,
                                                                 2048, 512, None),
                        max(iters, ns1))
    out["cfg1_bf16_gemm"]["M1"] = {"us": round(us1, 2), "host_us": round(wall1, 2),
                                   "timing": _LAST[0], "bytes": b1,
                                   "GBps": round(b1 / us1 / 1e3, 1),
                                   "frac_hbm": round(b1 / us1 / 1e3 / HBM_PEAK_GBS, 4),
                                   "cache": cache_note(b1, ns1)}
    # the decoder's prefill projections at batch 16 (M = 2048 rows of f32
    # activations) through the device API: rows_q8 (the int8 terms of the
    # rows), the int8 x int8 MFMA GEMM and the non-finite-row check, per call
    xp = up(rng.standard_normal((2048, 5760), dtype=np.float32))
    pre = {}
    for name, n, k in (("qkv", 6912, 2304), ("o", 2304, 2304), ("gate_up", 11520, 2304),
                       ("down", 2304, 5760)):
        wq = up(rng.integers(-127, 128, (n, k), dtype=np.int8))
        sq = up(np.full(n, 1e-3, np.float32))
        yq = zeros(2048 * n * 4)
        usp, wallp = _timed(L, lambda i: L.vmlm_hip_gemm_nt_int8(xp, wq, sq, yq, 2048, n, k, None),
                            max(8, iters // 10))
        useful = 2 * 2048 * n * k / usp / 1e6
        pre[name] = {"us": round(usp, 2), "host_us": round(wallp, 2), "timing": _LAST[0],
                     "useful_TOPs": round(useful, 1),
                     "frac_int8_peak_useful": round(useful / PEAK_INT8_TOPS, 4),
                     "frac_bf16_peak_useful": round(useful / (PEAK_BF16_TFLOPS), 4),
                     "frac_int8_peak_issued": round(Q8_TERMS * useful / PEAK_INT8_TOPS, 4)}
    pre["note"] = (f"per call: rows_q8 + gemm_dma_i8_kernel + non-finite-row check; issued = "
                   f"{Q8_TERMS} int8 MFMAs per product ({Q8_TERMS} int8 terms per activation), so "
                   f"useful work is at most 1/{Q8_TERMS} of the int8 peak "
                   f"({PEAK_INT8_TOPS / Q8_TERMS / PEAK_BF16_TFLOPS:.3f} of the bf16 peak)")
    out["cfg3_prefill_gemm"] = pre
    if orc:
        af = orc.bf16_to_f32(a)
        out["cfg1_bf16_gemm"]["cpu_us"] = _cpu_us(lambda: orc.gemm_nt_bf16(af, bt))
    # config 2: causal attention prefill [512, 36, 64] and one decode token vs 1024 positions
    rng = np.random.default_rng(2)
    S, H = 512, 36
    qkv_h = [rng.standard_normal((S, H * 64), dtype=np.float32) for _ in range(3)]
    qkv = [up(t) for t in qkv_h]
    do = zeros(S * H * 64 * 4)
    us, wall = _timed(L, lambda i: L.vmlm_hip_attention_prefill(qkv[0], qkv[1], qkv[2], do, S, H, 64,
                                                             C.c_float(10000.0), 0,
                                                             C.c_float(0.125), True, None),
                      max(8, iters // 4))
    tf = 1210318848 / us / 1e6
    tm_prefill = _LAST[0]
    cap = 1024
    kvb = H * cap * 64 * 4
    ns2 = n_sets(2 * kvb, 10**9)
    kc = copies(up(rng.standard_normal((H, cap, 64), dtype=np.float32)), kvb, ns2)
    vc = copies(up(rng.standard_normal((H, cap, 64), dtype=np.float32)), kvb, ns2)
    qd, kd, vd = (up(rng.standard_normal(H * 64, dtype=np.float32)) for _ in range(3))
    dod = zeros(H * 64 * 4)
    usd, walld = _timed(L, lambda i: L.vmlm_hip_attention_decode(qd, kd, vd, kc[i % ns2],
                                                              vc[i % ns2], dod, H, 64, cap,
                                                              cap - 1, C.c_float(10000.0),
                                                              C.c_float(0.125), None),
                        max(iters, ns2))
    gbs = (18874368 + 18432) / usd / 1e3
    out["cfg2_attention"] = {
        "prefill": {"us": round(us, 2), "host_us": round(wall, 2), "timing": tm_prefill,
                    "TFLOPs": round(tf, 2),
                    "frac_fp32_peak": round(tf / PEAK_FP32_TFLOPS, 4)},
        "decode": {"us": round(usd, 2), "host_us": round(walld, 2), "timing": _LAST[0],
                   "GBps": round(gbs, 1),
                   "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                   "cache": cache_note(2 * kvb, ns2)}}
    if orc:
        out["cfg2_attention"]["prefill"]["cpu_us"] = _cpu_us(
            lambda: orc.attention_prefill(qkv_h[0], qkv_h[1], qkv_h[2], H, 10000.0, 0, 0.125,
                                          True))
    # config 4: B1 stack, 8 layers, d = 1536, k0 = 32, 1024 tokens, tanh
    rng = np.random.default_rng(4)
    d, k0, T = 1536, 32, 1024
    layers = []
    for li in range(8):
        w, src = conn.make_block_aligned(rng, d, k0)
        layers.append(conn.DeviceConn(w, src, layer=li))
    xb = up(rng.standard_normal((T, d), dtype=np.float32))
    yb = zeros(T * d * 4)
    arr = (type(layers[0].struct) * 8)(*[l.struct for l in layers])
    us_fwd, wall_fwd = _timed(L, lambda i: L.vmlm_b1_stack_forward(arr, 8, xb, yb, T, 4, None),
                              max(8, iters // 4))
    tm_fwd = _LAST[0]
    # the plan built once (vmlm_b1_stack_create): one kernel per forward,
    # captured and replayed
    plan = conn.StackPlan(layers)
    us, wall = _timed(L, lambda i: L.vmlm_b1_stack_run(plan._h, xb, yb, T, 4, None),
                      max(8, iters // 4))
    plan.close()
    layer_bytes = 12976128
    gbs = 8 * layer_bytes / us / 1e3
    # the t8 contract sums without FMA: one multiply and one add per
    # connection and token, so the vector ALU bound is 64 lanes x 2.4 GHz x
    # 256 CUs / 2 ops = 19.66 T connection-tokens/s (tanh_f comes on top)
    macs = 8 * d * k0 * T
    tmac = macs / us / 1e6
    out["cfg4_b1_stack"] = {"us": round(us, 2), "host_us": round(wall, 2), "timing": _LAST[0],
                            "us_per_layer": round(us / 8, 2), "GBps_unique": round(gbs, 1),
                            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                            "T_mac_per_s": round(tmac, 3),
                            "frac_valu_mac": round(tmac / VALU_MAC_PEAK_T, 4),
                            "note": "one kernel for all 8 layers over a plan built once "
                                    "(vmlm_b1_stack_create), x and y [T][d]",
                            "cache": "warm: one buffer set replayed (x, y, 8 layers of w and "
                                     "src, the plan: about 27 MB, within the Infinity Cache); "
                                     "frac_hbm is over the unique bytes",
                            "per_call_forward": {"us": round(us_fwd, 2),
                                                 "host_us": round(wall_fwd, 2),
                                                 "timing": tm_fwd,
                                                 "note": "vmlm_b1_stack_forward: plan kernel "
                                                         "+ stack kernel on every call"}}
    if orc:  # one layer of the stack on the host (the t8 contract), per layer
        w0, s0 = conn.make_block_aligned(np.random.default_rng(4), d, k0)
        xt_h = orc.transpose_t8(np.random.default_rng(5).standard_normal((T, d), dtype=np.float32),
                                T)
        out["cfg4_b1_stack"]["cpu_us_per_layer"] = _cpu_us(
            lambda: orc.b1_forward_t8(w0, s0, xt_h, T))
    out["ops"] = run_ops(L, up, zeros, copies, iters, orc)
    for l in layers:
        l.free()
    for p in ptrs:
        L.vmlm_hip_free(p)
    return out


def run_ops(L, up, zeros, copies, iters, orc):
    """The per-op kernels of the VM path (RMSNorm, softmax, RoPE, activation,
    elementwise, scale, EMB, TOPK_IDX, f32 GEMM NT / NN) through the device
    API at decoder-sized shapes: time per call, algorithmic bytes (or flops)
    and the fraction of the roofline that bounds each; the oracle on the same
    inputs beside it. The HBM rows cycle through buffer sets larger than the
    Infinity Cache (`cache` says how each was timed)."""
    import ctypes as C
    rng = np.random.default_rng(7)
    ops = {}

    def rec(name, us, wall, nbytes=None, flops=None, cpu=None, cache=None):
        e = {"us": round(us, 2), "host_us": round(wall, 2), "timing": _LAST[0]}
        if nbytes is not None:
            gbs = nbytes / us / 1e3
            e.update({"bytes": int(nbytes), "GBps": round(gbs, 1),
                      "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)})
        if flops is not None:
            tf = flops / us / 1e6
            e.update({"flops": int(flops), "TFLOPs": round(tf, 2),
                      "frac_fp32_peak": round(tf / PEAK_FP32_TFLOPS, 4)})
        if cache is not None:
            e["cache"] = cache
        if cpu is not None:
            e["cpu_us"] = cpu
        ops[name] = e

    def sets(*arrays_or_bytes):
        """(buffer sets, bytes per set) of a row whose calls touch these."""
        nb = sum(a if isinstance(a, int) else a.nbytes for a in arrays_or_bytes)
        return n_sets(nb, 10**9), nb

    R, Hd = 2048, 2304  # prefill activations: 16 sequences x 128 tokens
    x = rng.standard_normal((R, Hd), dtype=np.float32)
    y = rng.standard_normal((R, Hd), dtype=np.float32)
    g = rng.standard_normal(Hd, dtype=np.float32)
    dg = up(g)
    n, sb = sets(x, x)
    dx, dd = copies(up(x), x.nbytes, n), [zeros(x.nbytes) for _ in range(n)]
    us, wall = _timed(L, lambda i: L.vmlm_hip_rmsnorm(dd[i % n], dx[i % n], dg, R, Hd,
                                                      C.c_float(1e-5), None), max(iters, n))
    rec("rmsnorm_2048x2304", us, wall, nbytes=2 * x.nbytes + g.nbytes,
        cpu=_cpu_us(lambda: orc.rmsnorm(x, g, 1e-5)) if orc else None, cache=cache_note(sb, n))
    EWADD, SILU = 20, 2  # VMLM_OP_EWADD, VMLM_ACT_SILU
    n3, sb3 = sets(x, y, x)
    dx3 = copies(dx[0], x.nbytes, n3)
    dy3 = copies(up(y), y.nbytes, n3)
    dd3 = [zeros(x.nbytes) for _ in range(n3)]
    us, wall = _timed(L, lambda i: L.vmlm_hip_ew_op(dd3[i % n3], dx3[i % n3], dy3[i % n3], R * Hd,
                                                    EWADD, None), max(iters, n3))
    rec("ew_add_2048x2304", us, wall, nbytes=3 * x.nbytes,
        cpu=_cpu_us(lambda: orc.ew_op(x, y, EWADD)) if orc else None, cache=cache_note(sb3, n3))
    us, wall = _timed(L, lambda i: L.vmlm_hip_scale(dd[i % n], dx[i % n], R * Hd,
                                                    C.c_float(0.125), None), max(iters, n))
    rec("scale_2048x2304", us, wall, nbytes=2 * x.nbytes,
        cpu=_cpu_us(lambda: orc.scale(x, 0.125)) if orc else None, cache=cache_note(sb, n))
    a = rng.standard_normal((R, 5760), dtype=np.float32)
    na, sba = sets(a)  # in place
    da = copies(up(a), a.nbytes, na)
    us, wall = _timed(L, lambda i: L.vmlm_hip_act(da[i % na], R * 5760, SILU, None),
                      max(iters, na))
    rec("act_silu_2048x5760", us, wall, nbytes=2 * a.nbytes,
        cpu=_cpu_us(lambda: orc.act(a, SILU)) if orc else None, cache=cache_note(sba, na))
    # softmax over the scores of 36 heads x 512 queries (rows of 512), in place
    p = rng.standard_normal((36 * 512, 512), dtype=np.float32)
    npp, sbp = sets(p)
    dp = copies(up(p), p.nbytes, npp)
    us, wall = _timed(L, lambda i: L.vmlm_hip_softmax(dp[i % npp], 36 * 512, 512, False, None),
                      max(iters, npp))
    rec("softmax_18432x512", us, wall, nbytes=2 * p.nbytes,
        cpu=_cpu_us(lambda: orc.softmax(p, False)) if orc else None, cache=cache_note(sbp, npp))
    # RoPE of 512 positions x 36 heads (rows of 64)
    r = rng.standard_normal((512 * 36, 64), dtype=np.float32)
    nr, sbr = sets(r, r)
    dr, dro = copies(up(r), r.nbytes, nr), [zeros(r.nbytes) for _ in range(nr)]
    us, wall = _timed(L, lambda i: L.vmlm_hip_rope(dro[i % nr], dr[i % nr], 512 * 36, 64,
                                                   C.c_float(10000.0), 0, None), max(iters, nr))
    rec("rope_18432x64", us, wall, nbytes=2 * r.nbytes,
        cpu=_cpu_us(lambda: orc.rope(r, 10000.0, 0)) if orc else None, cache=cache_note(sbr, nr))
    # TOPK_IDX over one row of LM-head logits (the op scans the first row)
    lg = rng.standard_normal((1, 122753), dtype=np.float32)
    nl, sbl = sets(lg)
    nl = min(nl, 1024)
    dl, di = copies(up(lg), lg.nbytes, nl), zeros(4)
    us, wall = _timed(L, lambda i: L.vmlm_hip_topk_idx(dl[i % nl], 1, 122753, di, None),
                      max(iters, nl))
    rec("topk_idx_122753", us, wall, nbytes=lg.nbytes,
        cpu=_cpu_us(lambda: orc.topk_idx(lg)) if orc else None, cache=cache_note(sbl, nl))
    # f32 GEMMs of the VM's attention composition (one head): scores Q K^T
    # 512x512x64 (NT) and P V 512x64x512 (NN)
    qh = rng.standard_normal((512, 64), dtype=np.float32)
    kh = rng.standard_normal((512, 64), dtype=np.float32)
    ph = rng.standard_normal((512, 512), dtype=np.float32)
    dq, dk, dph, ds_, do_ = up(qh), up(kh), up(ph), zeros(512 * 512 * 4), zeros(512 * 64 * 4)
    us, wall = _timed(L, lambda i: L.vmlm_hip_gemm_nt(dq, dk, ds_, 512, 512, 64, False, None), iters)
    rec("gemm_nt_f32_512x512x64", us, wall, flops=2 * 512 * 512 * 64,
        cpu=_cpu_us(lambda: orc.gemm_nt(qh, kh)) if orc else None)
    us, wall = _timed(L, lambda i: L.vmlm_hip_gemm(dph, dk, do_, 512, 64, 512, False, None), iters)
    rec("gemm_nn_f32_512x64x512", us, wall, flops=2 * 512 * 64 * 512,
        cpu=_cpu_us(lambda: orc.gemm(ph, kh)) if orc else None)
    return ops


def run_decode(cfg, W, batch, steps, warmup, prompt_len=128, cap=1024):
    from sparrow_amd import model as M
    from sparrow_amd.decoder import Decoder
    prompts = M.make_prompts(cfg, batch, prompt_len, seed=3)
    dec = Decoder(cfg, batch=batch, cap=cap)
    dec.load(W)
    dec.prefill(prompts)  # first call: one-time set-up (workspaces, code objects)
    ts = []
    for _ in range(3):  # timed prefills (each restarts the session at position S)
        t = time.perf_counter()
        t0, _ = dec.prefill(prompts)
        ts.append(time.perf_counter() - t)
    dec.prefill_s = sorted(ts)[1]
    if warmup:
        dec.decode(warmup, want_tokens=False)
    from sparrow_amd import lib
    L = lib()
    import ctypes as C
    st = dec.stream()
    e0, e1 = C.c_int(), C.c_int()
    L.vmlm_hip_event_record(st, C.byref(e0))
    t = time.perf_counter()
    toks, _ = dec.decode(steps)
    wall = time.perf_counter() - t
    L.vmlm_hip_event_record(st, C.byref(e1))
    ms = C.c_float()
    L.vmlm_hip_event_elapsed_ms(e0.value, e1.value, C.byref(ms))
    L.vmlm_hip_event_release_all()
    return dec, wall, ms.value / 1e3, t0, toks


def vm_step_loop(cfg, W, steps, base=2, prompt_len=128):
    """The step-looped decoder program (config 3 at batch 1) on the device
    VM: one LOOP_CNT body per greedy step. Two programs of base and base +
    steps steps are loaded; each is run once (first run: code objects,
    workspaces), then timed as the fastest of three runs, and the decode
    rate is steps / (t(base + steps) - t(base)). Its
    greedy chain (st_gen, fed the session's first token) is compared with
    the batch-1 session's over the same steps."""
    from sparrow_amd import model as M
    from sparrow_amd import programs, vmb
    from sparrow_amd import vm as gvm
    from sparrow_amd.decoder import Decoder
    prompts = M.make_prompts(cfg, 1, prompt_len, seed=3)
    dec = Decoder(cfg, batch=1, cap=1024)
    dec.load(W)
    chain = dec.generate(prompts, base + steps)[0]
    dec.close()
    times, gen, info = {}, None, {}
    for G in (base, base + steps):
        t = time.perf_counter()
        P = programs.minicpm_program(cfg, W, prompt_len, G, step_loop=True, print_prefill=False)
        loop = [i for i, ins in enumerate(P.text) if ins[0] == vmb.OP["LOOP_CNT"]][-1]
        info["instructions_per_step"] = loop - P.text[loop][3] + 1  # LOOP_CNT jumps to dst
        img = P.build()
        del P
        info["build_s"] = round(time.perf_counter() - t, 2)
        t = time.perf_counter()
        with gvm.Vm(img) as v:
            del img
            info["load_s"] = round(time.perf_counter() - t, 2)
            info["swizzled_int8_consts"] = v.swizzled_consts()
            info["fused_runs"] = v.fused_runs()
            v.write("st_tok", np.float32(prompts[0]))
            v.write("st_gen", np.float32([chain[0]]))
            v.run()
            ts = []
            for _ in range(3):  # the prefill's host dispatch varies by tenths of a second
                v.clear_output()
                t = time.perf_counter()
                v.run()
                ts.append(time.perf_counter() - t)
            times[G] = min(ts)
            info["graph_segments"] = v.graph_segments()
            gen = v.read("st_gen")[0].astype(np.int64)
    dt = times[base + steps] - times[base]
    same = np.array_equal(gen, chain.astype(np.int64))
    diff = np.nonzero(gen != chain)[0]
    return {
        "tokens_per_s": round(steps / dt, 2),
        "ms_per_step": round(dt / steps * 1e3, 3),
        "run_s": {str(k): round(v, 3) for k, v in times.items()},
        "chain_equal_to_session": bool(same),
        "first_difference": None if same else int(diff[0]),
        "steps": steps,
        "load": info,
        "note": "step-looped program (programs.minicpm_program step_loop=True): prefill of the "
                "128-token prompt, then a LOOP_CNT body per step (per layer: RMSNORM, q/k/v "
                "GEMMs, per head SLICE/ROPE/TRANSPOSE/WRITECOL and GEMM/SCALE/SOFTMAX/GEMM, "
                "then o, gate/up, ACT, EWMUL, down). The executor dispatches opcode by opcode, "
                "except the runs it matched at load (fused_runs: per layer the cache append and "
                "the attention over all heads in one launch; q/k/v, and gate/up with ACT and "
                "EWMUL, one launch each with the RMSNORM before them; per layer and head the "
                "prompt's column-by-column K/V cache writes, two strided copies; o and down with "
                "their residual EWADD, one launch each). The "
                "loop body up to its PRINT is captured into a HIP graph on its second step and "
                "replayed after (graph_segments). The rate is the difference of two programs' "
                "run times",
    }


def traffic_probe(iters, batches=(16, 1)):
    """For `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE` runs: a plain device copy
    of 256 MiB (the calibration: its bytes are known) three times, then the
    four decode GEMV shapes of the batch-16 session and of the batch-1 session
    (or only the sessions in `batches`) `iters` times each (after a warm-up
    pass over the 40 layers)."""
    import ctypes as C
    from sparrow_amd import check, lib
    from sparrow_amd import model as M
    from sparrow_amd.decoder import Decoder
    L = lib()
    nbytes = 256 << 20
    a, b = C.c_void_p(), C.c_void_p()
    check(L.vmlm_hip_malloc(C.byref(a), nbytes))
    check(L.vmlm_hip_malloc(C.byref(b), nbytes))
    check(L.vmlm_hip_memset(a, 1, nbytes))
    for _ in range(3):
        check(L.vmlm_hip_memcpy_d2d(b, a, nbytes))
    check(L.vmlm_hip_free(a))
    check(L.vmlm_hip_free(b))
    cfg = M.minicpm_2b_config()
    W = M.make_weights(cfg, seed=3, threads=16)
    for batch in batches:  # the k-slice GEMVs (batch 16), then the fused ones (batch 1)
        dec = Decoder(cfg, batch=batch, cap=1024)
        dec.load(W)
        dec.prefill(M.make_prompts(cfg, batch, 128, seed=3))
        for which in range(4):
            dec.time_gemv(which, iters)
        dec.close()
    print(json.dumps({"probe": "traffic", "copy_bytes": nbytes, "gemv_iters": iters}))


def mfma_probe(reps):
    """For `rocprofv3 --pmc` runs of the MFMA kernels: config 1 (bf16 GEMM
    1024 x 512 x 2048) and the four prefill projections of the decoder at
    batch 16 (M = 2048 rows of f32 activations through the int8-row path:
    q/k/v 6912 x 2304, o 2304 x 2304, gate/up 11520 x 2304, down 2304 x 5760),
    `reps` eager calls each after one warm-up call."""
    import ctypes as C
    from sparrow_amd import check, lib
    L = lib()
    rng = np.random.default_rng(1)
    bufs = []

    def dev(a):
        a = np.ascontiguousarray(a)
        p = C.c_void_p()
        check(L.vmlm_hip_malloc(C.byref(p), a.nbytes))
        check(L.vmlm_hip_memcpy_h2d(p, a.ctypes.data, a.nbytes))
        bufs.append(p)
        return p

    def out(nbytes):
        p = C.c_void_p()
        check(L.vmlm_hip_malloc(C.byref(p), nbytes))
        bufs.append(p)
        return p

    a = dev(rng.integers(0, 65535, (1024, 512)).astype(np.uint16) & 0xBFFF)
    bt = dev(rng.integers(0, 65535, (2048, 512)).astype(np.uint16) & 0xBFFF)
    c = out(1024 * 2048 * 4)
    for _ in range(reps + 1):
        check(L.vmlm_hip_gemm_nt_bf16bf16(a, bt, c, 1024, 2048, 512, None))
    x = dev(rng.standard_normal((2048, 5760), dtype=np.float32))
    for n, k in ((6912, 2304), (2304, 2304), (11520, 2304), (2304, 5760)):
        w = dev(rng.integers(-127, 128, (n, k), dtype=np.int8))
        sc = dev(np.full(n, 1e-3, np.float32))
        y = out(2048 * n * 4)
        for _ in range(reps + 1):
            check(L.vmlm_hip_gemm_nt_int8(x, w, sc, y, 2048, n, k, None))
    check(L.vmlm_hip_sync())
    for p in bufs:
        L.vmlm_hip_free(p)
    print(json.dumps({"probe": "mfma", "reps": reps}))


def b1_probe(reps):
    """For `rocprofv3` runs of the B1 stack kernel: config 4 (8 layers,
    d = 1536, k0 = 32, 1024 tokens, tanh) over a plan built once, `reps` + 1
    forwards."""
    import ctypes as C
    from sparrow_amd import check, conn, lib
    L = lib()
    rng = np.random.default_rng(4)
    d, k0, T = 1536, 32, 1024
    layers = []
    for li in range(8):
        w, src = conn.make_block_aligned(rng, d, k0)
        layers.append(conn.DeviceConn(w, src, layer=li))
    x = np.ascontiguousarray(rng.standard_normal((T, d), dtype=np.float32))
    xb, yb = C.c_void_p(), C.c_void_p()
    check(L.vmlm_hip_malloc(C.byref(xb), x.nbytes))
    check(L.vmlm_hip_memcpy_h2d(xb, x.ctypes.data, x.nbytes))
    check(L.vmlm_hip_malloc(C.byref(yb), x.nbytes))
    plan = conn.StackPlan(layers)
    for _ in range(reps + 1):
        check(L.vmlm_b1_stack_run(plan._h, xb, yb, T, 4, None))
    check(L.vmlm_hip_sync())
    plan.close()
    for l in layers:
        l.free()
    L.vmlm_hip_free(xb)
    L.vmlm_hip_free(yb)
    print(json.dumps({"probe": "b1", "reps": reps}))


def prefill_probe(reps, batch=16):
    """For `rocprofv3 --kernel-trace` runs of the prefill: the session
    (`batch` x 128 prompt tokens; batch 16: M = 2048 rows) prefilled once,
    then `reps` more times; no decode."""
    from sparrow_amd import model as M
    from sparrow_amd.decoder import Decoder
    cfg = M.minicpm_2b_config()
    W = M.make_weights(cfg, seed=3, threads=16)
    dec = Decoder(cfg, batch=batch, cap=1024)
    dec.load(W)
    prompts = M.make_prompts(cfg, batch, 128, seed=3)
    ts = []
    for _ in range(reps + 1):
        t = time.perf_counter()
        dec.prefill(prompts)
        ts.append(time.perf_counter() - t)
    dec.close()
    print(json.dumps({"probe": "prefill", "batch": batch, "ms": [round(x * 1e3, 3) for x in ts]}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--cpu-steps", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--gemv-iters", type=int, default=400)
    ap.add_argument("--suite-iters", type=int, default=100)
    ap.add_argument("--no-suite", action="store_true")
    ap.add_argument("--suite-only", action="store_true",
                    help="only configs 0, 1, 2, 4 and the op timings (no decoder, no CPU)")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="only config 1 and the prefill GEMMs, for the MFMA counter runs")
    ap.add_argument("--b1-probe", action="store_true",
                    help="only config 4's stack kernel (plan built once), for counter runs")
    ap.add_argument("--prefill-probe", action="store_true",
                    help="only the prefill at --batch (a first call, then more), for kernel traces")
    ap.add_argument("--no-batch1", action="store_true",
                    help="only the --batch session (no batch-1 session): for kernel traces "
                         "and traffic counters of the batch-16 program")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only the copy + GEMV launches that the counter runs measure")
    ap.add_argument("--eager", action="store_true",
                    help="suite rows timed from eager launches only (no HIP graph replay): "
                         "for rocprofv3 kernel traces of the suite's kernels")
    ap.add_argument("--no-vm", action="store_true",
                    help="skip the device VM's step-looped decoder program")
    ap.add_argument("--vm-steps", type=int, default=64)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)
    if 128 + args.warmup + args.steps > 1024:
        sys.exit("prompt (128) + warmup + steps must fit the 1024-position KV cache")

    import sparrow_amd
    from sparrow_amd import model as M
    sparrow_amd.init(0)
    _EAGER[0] = args.eager
    if args.traffic_probe:
        traffic_probe(20, (16,) if args.no_batch1 else (16, 1))
        return
    if args.mfma_probe:
        mfma_probe(3)
        return
    if args.prefill_probe:
        prefill_probe(4, args.batch)
        return
    if args.b1_probe:
        b1_probe(3)
        return
    if args.suite_only:
        print(json.dumps({"suite": run_suite(args.suite_iters, cpu=False)}))
        return
    cfg = M.minicpm_2b_config()
    t = time.time()
    W = M.make_weights(cfg, seed=3, threads=16)
    log(f"weights generated in {time.time() - t:.1f}s")

    dec, wall, ev_s, _, toks = run_decode(cfg, W, args.batch, args.steps, args.warmup)
    log(f"batch {args.batch}: {args.steps} steps in {wall * 1e3:.1f} ms wall "
        f"({ev_s * 1e3:.1f} ms events); prefill {dec.prefill_s * 1e3:.2f} ms")
    prefill = {f"batch{args.batch}_ms": round(dec.prefill_s * 1e3, 3)}
    roof = gemv_roofline(dec, args.gemv_iters)
    log(f"q8 GEMV: {roof['achieved']} GB/s ({roof['frac'] * 100:.1f}% of peak)")
    attn = {f"batch{args.batch}": decode_attention(dec, args.gemv_iters)}
    dec.close()
    if args.no_batch1:
        print(json.dumps({"probe": "decode", "batch": args.batch,
                          "tokens_per_s": round(args.batch * args.steps / wall, 2),
                          "roofline_frac": roof["frac"],
                          "gemv_us": {k: v["us"] for k, v in roof["per_shape"].items()},
                          "decode_attention": attn, "prefill": prefill}))
        return

    if args.batch == 1:
        wall1, roof1 = wall, roof
    else:
        dec1, wall1, _, _, _ = run_decode(cfg, W, 1, args.steps, args.warmup)
        prefill["batch1_ms"] = round(dec1.prefill_s * 1e3, 3)
        roof1 = gemv_roofline(dec1, args.gemv_iters)
        log(f"batch 1 q8 GEMV: {roof1['achieved']} GB/s ({roof1['frac'] * 100:.1f}% of peak)")
        attn["batch1"] = decode_attention(dec1, args.gemv_iters)
        dec1.close()
        log(f"batch 1: {args.steps} steps in {wall1 * 1e3:.1f} ms wall")

    vm = None
    if not args.no_vm:
        vm = vm_step_loop(cfg, W, args.vm_steps)
        log(f"device VM step loop: {vm['tokens_per_s']} tokens/s at batch 1 "
            f"({vm['load']['instructions_per_step']} opcodes per step), chain equal to the "
            f"session's: {vm['chain_equal_to_session']}")

    suite = None
    if not args.no_suite:
        suite = run_suite(args.suite_iters, cpu=not args.no_cpu)
        log(f"suite: {json.dumps(suite)}")

    cpu = None
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        cpu = cpu_baseline(cfg, W, args.cpu_steps, threads)
        log(f"cpu oracle: {cpu['value']} tokens/s on 1 thread, "
            f"{cpu['threads']['batch1']['value']} on {threads} (batch 16: "
            f"{cpu['threads']['batch16']['value']})")

    value = args.steps * args.batch / wall
    out = {
        "metric": "decode tokens/s at MiniCPM-2B int8 shape; q8 GEMV GB/s vs HBM peak",
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("int8 weights; batch 16: each f32 activation as three int8 terms with "
                  "power-of-two factors per row segment (int32 sums, f32 combine); batch <= 5: "
                  "three bf16 terms (f32 accumulate)"),
        "data": "synthetic (seeded random-init weights and prompts)",
        "config": {
            "workload": "config 3: MiniCPM-2B-shaped int8 decoder, greedy decode",
            "batch": args.batch, "prompt_len": 128, "kv_capacity": 1024,
            "layers": cfg["n_layers"], "hidden": cfg["hidden"], "heads": cfg["n_heads"],
            "head_dim": cfg["head_dim"], "inter": cfg["inter"], "vocab": cfg["vocab"],
            "lm_head": "bf16", "parallelism": "single GPU",
        },
        "batch1_tokens_per_s": round(args.steps / wall1, 2),
        "batch1_ms_per_step": round(wall1 / args.steps * 1e3, 4),
        "batch1_roofline": roof1,
        "vm_step_loop_batch1": vm,
        "prefill": dict(prefill, prompt_len=128,
                        note="wall time of one prefill call (128 prompt tokens per sequence, "
                             "40 layers, LM head and first argmax): median of three "
                             "calls after a first"),
        "event_ms_per_step": round(ev_s / args.steps * 1e3, 4),
        "roofline": roof,
        "decode_attention": dict(attn, note="attn_decode_kernel per layer after the timed "
                                            "steps (position: the row being appended)"),
        "cpu_baseline": cpu,
        "other_configs": suite,
        "tokens_checksum": int(np.asarray(toks, np.int64).sum()),
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
