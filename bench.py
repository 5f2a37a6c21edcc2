"""Decode benchmark: SmolLM3-3B architecture, random-init Q4 weights, batch 1.

Workload: a 64-token random-ID prompt (seed 0) is prefilled, then greedy
decode runs token by token through the C ABI (qora_hip_decode: one captured
HIP graph per token, argmax read back to the host each step). W untimed
warmup tokens, then exactly K timed tokens. `value` is decode tokens/s with
the weights resident in HBM.

Also reported on the same JSON line:
  roofline     - the dominant kernel (fused gate/up Q4 GEMV, 2048 -> 2x11008)
                 timed with HIP events on the stream it is launched on, over
                 a graph of launches that rotate through >= 768 MB of distinct
                 weight copies (so the 256 MB Infinity Cache cannot serve
                 them); achieved = algorithmic bytes / average launch time.
  cpu_baseline - the reference CPU algorithm (the C oracle: AVX-512 LUT
                 GEMV, k-split into T partials) timed on this host's cores on
                 a bounded sample of the same workload.
  gemv_gbps    - every per-layer GEMV shape and the tied lm_head, same method.
  tok_s_ctx2048 - decode rate with the KV cache at ~2048 positions.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import __graft_entry__ as entry  # noqa: E402

HBM_PEAK_GBS = 8000.0
PUBLISHED_GPU_TOK_S = 4.1   # reference README.md:43,157 (GTX 1660 SUPER, Vulkan)


class Hip:
    """The few HIP runtime calls the harness needs (events, D2D copies)."""

    def __init__(self):
        self.h = ctypes.CDLL("libamdhip64.so")
        self.h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.h.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]

    def event(self):
        e = ctypes.c_void_p()
        assert self.h.hipEventCreate(ctypes.byref(e)) == 0
        return e.value

    def record(self, e, stream):
        assert self.h.hipEventRecord(e, stream) == 0

    def elapsed_ms(self, a, b):
        assert self.h.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.h.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value

    def d2d(self, dst, src, n):
        assert self.h.hipMemcpy(dst, src, n, 3) == 0


def q4_bytes(k, n):
    """Algorithmic bytes of one Q4 GEMV: nibbles + f16 scales + f32 x + f32 y."""
    return k * n // 2 + k * n // 16 + 4 * k + 4 * n


EAGER = False   # --eager: no HIP graphs (rocprofv3 does not follow graph launches)


def time_graph(ctx, hip, launch_fns, reps=3):
    """Capture one launch per entry of launch_fns into a graph, replay it
    `reps` times between HIP events on the context stream; return average
    milliseconds per launch. With --eager the launches are issued directly."""
    for f in launch_fns[:2]:
        f()          # eager calls size the scratch before capture
    ctx.synchronize()
    if EAGER:
        a, b = hip.event(), hip.event()
        hip.record(a, ctx.stream)
        for _ in range(reps):
            for f in launch_fns:
                f()
        hip.record(b, ctx.stream)
        return hip.elapsed_ms(a, b) / (reps * len(launch_fns))
    ctx.capture_begin()
    for f in launch_fns:
        f()
    g = ctx.capture_end()
    try:
        ctx.graph_launch(g, 1)
        ctx.synchronize()
        a, b = hip.event(), hip.event()
        hip.record(a, ctx.stream)
        ctx.graph_launch(g, reps)
        hip.record(b, ctx.stream)
        ms = hip.elapsed_ms(a, b)
    finally:
        ctx.graph_destroy(g)
    return ms / (reps * len(launch_fns))


def prepared_time(ctx, hip, wid, wid_up, paired, nbytes, x, acc):
    """Average ms per launch of the decode step's GEMV kernel (tile layout,
    qora_hip_gemv_run) over >= 768 MB of distinct packed copies."""
    copies = max(4, math.ceil((768 << 20) / nbytes))
    gids = [ctx.gemv_prepare(wid, wid_up, paired) for _ in range(copies)]
    try:
        fns = [(lambda g=g: ctx.check(ctx.lib.qora_hip_gemv_run(ctx.h, g, x, acc, None), "gemv_run")) for g in gids]
        return time_graph(ctx, hip, fns)
    finally:
        for g in gids:
            ctx.gemv_release(g)


def f16_bytes(k, n):
    """Algorithmic bytes of one F16 GEMV: binary16 weights + f32 x + f32 y."""
    return 2 * k * n + 4 * k + 4 * n


def device_copies(ctx, hip, srcs, min_bytes=768 << 20, min_copies=2):
    """Distinct device copies of the device buffers `srcs` [(ptr, nbytes)],
    enough copies that together they span >= min_bytes. Returns the list of
    per-copy pointer tuples and the allocations to free."""
    per = sum(nb for _, nb in srcs)
    copies = max(min_copies, math.ceil(min_bytes / per))
    sets, allocs = [], []
    try:
        for _ in range(copies):
            ptrs = []
            for p, nb in srcs:
                d = ctx.malloc(nb)
                allocs.append(d)
                hip.d2d(d, p, nb)
                ptrs.append(d)
            sets.append(tuple(ptrs))
    except Exception:
        for d in allocs:
            ctx.free(d)
        raise
    return sets, allocs


def copies_time(ctx, hip, srcs, launch):
    """Average ms per launch of launch(ptr_tuple) over distinct copies of srcs."""
    sets, allocs = device_copies(ctx, hip, srcs)
    try:
        return time_graph(ctx, hip, [(lambda s=s: launch(s)) for s in sets])
    finally:
        ctx.synchronize()
        for d in allocs:
            ctx.free(d)


def valu_q4_roofline(ctx, hip, be, pkg):
    """The VALU Q4 GEMV (gemv_kernel, the reference weight layout, one
    launch through qora_hip_gemv_q4_accumulate / _gate_up_q4_accumulate)
    and the VALU row-dot lm_head (qora_hip_gemv_q4_rowdot) on the shapes the
    matrix-core kernels are timed on, for the comparison of the two."""
    c = be.config
    lib, h = ctx.lib, ctx.h
    x = ctx.malloc(4 * c.intermediate)
    acc = ctx.malloc(8 * 2 * c.intermediate)
    ctx.h2d(x, pkg.synth_f32(0, 77, c.intermediate))
    shapes = c.weight_shapes()
    res = {}
    try:
        for j, label in ((0, "q/o 2048x2048"), (1, "k/v 2048x512"), (6, "down 11008x2048")):
            k, n = shapes[j]
            p, s = ctx.weight_ptrs(int(be.wids[0, j]))
            ms = copies_time(ctx, hip, [(p, k * n // 2), (s, k * n // 16)],
                             lambda t, k=k, n=n: ctx.check(
                                 lib.qora_hip_gemv_q4_accumulate(h, t[0], t[1], x, acc, k, n, None), "q4_acc"))
            res[label] = {"us": ms * 1e3, "gbps": q4_bytes(k, n) / (ms * 1e-3) / 1e9}
        k, n = shapes[4]
        gp, gs = ctx.weight_ptrs(int(be.wids[0, 4]))
        up, us = ctx.weight_ptrs(int(be.wids[0, 5]))
        ms = copies_time(ctx, hip, [(gp, k * n // 2), (gs, k * n // 16), (up, k * n // 2), (us, k * n // 16)],
                         lambda t: ctx.check(lib.qora_hip_gate_up_q4_accumulate(h, t[0], t[1], t[2], t[3], x, acc,
                                                                                 k, n, None), "gate_up_acc"))
        gu_bytes = 2 * (k * n // 2 + k * n // 16) + 4 * k + 8 * n
        res["gate+up 2048x(2x11008)"] = {"us": ms * 1e3, "gbps": gu_bytes / (ms * 1e-3) / 1e9}
        V, Hd = c.vocab, c.hidden
        ep, es = ctx.weight_ptrs(be.embed_wid)
        lm = ctx.malloc(4 * V)
        try:
            ms = copies_time(ctx, hip, [(ep, V * Hd // 2), (es, V * Hd // 16)],
                             lambda t: ctx.check(lib.qora_hip_gemv_q4_rowdot(h, t[0], t[1], x, lm, V, Hd, None),
                                                 "q4_rowdot"))
        finally:
            ctx.free(lm)
        res["lm_head 128256x2048"] = {"us": ms * 1e3, "gbps": q4_bytes(V, Hd) / (ms * 1e-3) / 1e9}
    finally:
        ctx.free(x)
        ctx.free(acc)
    return res


def f16_measurements(pkg, hip, cfg, prompt, steps, warmup):
    """The F16 weight path on its own context: decode tok/s of the
    SmolLM3-3B architecture with seeded N(0, 0.02) binary16 weights (same
    prompt, f32 KV cache of 2048 positions), and GB/s of its decode-step
    GEMV (the VALU kernel on the tile layout) and row-dot lm_head on the
    per-layer shapes, each over >= 768 MB of distinct copies."""
    t0 = time.perf_counter()
    w16 = pkg.synthetic_model(cfg, seed=0, fmt=pkg.FORMAT_F16, rope_positions=2048)
    print(f"# F16 synthetic model ready in {time.perf_counter() - t0:.1f}s", file=sys.stderr, flush=True)
    ctx = pkg.HipContext(0)
    try:
        be = pkg.HipBackend(ctx, w16, kv_capacity=2048, kv_dtype=pkg.KV_F32)
        _, tok = be.raw_prefill(prompt, want_logits=False)
        for _ in range(warmup):
            _, tok = be.forward_decode_raw(tok, want_logits=False)
        ctx.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            _, tok = be.forward_decode_raw(tok, want_logits=False)
        ctx.synchronize()
        tok_s = steps / (time.perf_counter() - t0)
        wbytes = w16.weight_bytes_per_token()
        roof = HBM_PEAK_GBS * 1e9 / wbytes
        print(f"# F16 decode {tok_s:.1f} tok/s (weight roofline {roof:.0f})", file=sys.stderr, flush=True)
        lib, h = ctx.lib, ctx.h
        x = ctx.malloc(4 * cfg.intermediate)
        acc = ctx.malloc(8 * 2 * cfg.intermediate)
        ctx.h2d(x, pkg.synth_f32(0, 77, cfg.intermediate))
        shapes = cfg.weight_shapes()
        gemv = {}
        try:
            for j, label in ((0, "q/o 2048x2048"), (1, "k/v 2048x512"), (6, "down 11008x2048")):
                k, n = shapes[j]
                ms = prepared_time(ctx, hip, int(be.wids[0, j]), 0, False, 2 * k * n, x, acc)
                gemv[label] = {"us": ms * 1e3, "gbps": f16_bytes(k, n) / (ms * 1e-3) / 1e9}
            k, n = shapes[4]
            ms = prepared_time(ctx, hip, int(be.wids[0, 4]), int(be.wids[0, 5]), True, 4 * k * n, x, acc)
            gu_bytes = 4 * k * n + 4 * k + 8 * n
            gemv["gate+up 2048x(2x11008)"] = {"us": ms * 1e3, "gbps": gu_bytes / (ms * 1e-3) / 1e9}
            V, Hd = cfg.vocab, cfg.hidden
            ep, _ = ctx.weight_ptrs(be.embed_wid)
            lm = ctx.malloc(4 * V)
            try:
                ms = copies_time(ctx, hip, [(ep, 2 * V * Hd)],
                                 lambda t: ctx.check(lib.qora_hip_gemv_f16_rowdot(h, t[0], x, lm, V, Hd, None),
                                                     "f16_rowdot"))
            finally:
                ctx.free(lm)
            gemv["lm_head 128256x2048"] = {"us": ms * 1e3, "gbps": f16_bytes(V, Hd) / (ms * 1e-3) / 1e9}
        finally:
            ctx.free(x)
            ctx.free(acc)
        for kname, v in gemv.items():
            print(f"# F16 {kname}: {v['us']:.2f} us, {v['gbps']:.0f} GB/s", file=sys.stderr, flush=True)
    finally:
        ctx.close()
    return {"tok_s": round(tok_s, 2), "weight_bytes_per_token": wbytes, "weight_roofline_tok_s": round(roof, 1),
            "frac_of_weight_roofline": round(tok_s / roof, 4),
            "gemv_gbps": {k2: round(v["gbps"], 1) for k2, v in gemv.items()},
            "gemv_us": {k2: round(v["us"], 3) for k2, v in gemv.items()}}


def gemv_roofline(ctx, hip, be, pkg):
    """Per-shape GB/s of the decode step's Q4 GEMV kernel on the model's own
    weights (tile layout, qora_hip_gemv_prepare / qora_hip_gemv_run), and of
    the tied lm_head row-dot kernel."""
    c = be.config
    lib, h = ctx.lib, ctx.h
    x = ctx.malloc(4 * c.intermediate)
    acc = ctx.malloc(8 * 2 * c.intermediate)
    ctx.h2d(x, pkg.synth_f32(0, 77, c.intermediate))
    results = {}
    shapes = c.weight_shapes()
    for j, label in ((0, "q/o 2048x2048"), (1, "k/v 2048x512"), (6, "down 11008x2048")):
        k, n = shapes[j]
        ms = prepared_time(ctx, hip, int(be.wids[0, j]), 0, False, k * n // 2 + k * n // 16, x, acc)
        results[label] = {"us": ms * 1e3, "gbps": q4_bytes(k, n) / (ms * 1e-3) / 1e9}
    # the single 2048 -> 11008 gate projection (the one-GEMV workload's shape)
    k, n = shapes[4]
    ms = prepared_time(ctx, hip, int(be.wids[0, 4]), 0, False, k * n // 2 + k * n // 16, x, acc)
    results["gate 2048x11008"] = {"us": ms * 1e3, "gbps": q4_bytes(k, n) / (ms * 1e-3) / 1e9}
    # fused gate+up (the dominant kernel)
    gu_w = 2 * (k * n // 2 + k * n // 16)
    ms = prepared_time(ctx, hip, int(be.wids[0, 4]), int(be.wids[0, 5]), True, gu_w, x, acc)
    gu_bytes = gu_w + 4 * k + 8 * n
    results["gate+up 2048x(2x11008)"] = {"us": ms * 1e3, "gbps": gu_bytes / (ms * 1e-3) / 1e9, "bytes": gu_bytes}
    # tied lm_head: the decode step's matrix-core kernel (qora_hip_lm_head_run,
    # logits only) on distinct packed copies of the embedding
    V, Hd = c.vocab, c.hidden
    copies = max(4, math.ceil((768 << 20) / (V * Hd // 2 + V * Hd // 16)))
    lids = [ctx.lm_head_prepare(be.embed_wid) for _ in range(copies)]
    lm = ctx.malloc(4 * V)
    try:
        fns = [(lambda i=i: ctx.check(lib.qora_hip_lm_head_run(h, i, x, lm, None, None), "lm_head_run")) for i in lids]
        ms = time_graph(ctx, hip, fns)
    finally:
        for i in lids:
            ctx.gemv_release(i)
        ctx.free(lm)
    results["lm_head 128256x2048"] = {"us": ms * 1e3, "gbps": q4_bytes(V, Hd) / (ms * 1e-3) / 1e9}
    ctx.free(x)
    ctx.free(acc)
    return results


CPU_THREADS = 16   # host threads a one-GPU job of this benchmark is given


def host_cpu():
    """Model name and counts of the host CPU, from /proc/cpuinfo (what lscpu
    reports as Model name, CPU(s), Socket(s) and Core(s) per socket)."""
    info = {"model": None, "logical_cpus": os.cpu_count(), "sockets": None, "cores_per_socket": None}
    try:
        info["available_cpus"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        info["available_cpus"] = os.cpu_count()
    try:
        sockets, cores = set(), None
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key, val = key.strip(), val.strip()
                if key == "model name" and info["model"] is None:
                    info["model"] = val
                elif key == "physical id":
                    sockets.add(val)
                elif key == "cpu cores" and cores is None:
                    cores = int(val)
        info["sockets"] = len(sockets) or None
        info["cores_per_socket"] = cores
    except (OSError, ValueError):
        pass
    return info


def cpu_threads():
    """Threads for the multi-threaded CPU baseline: every CPU this process
    may run on, at most CPU_THREADS."""
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    return max(1, min(CPU_THREADS, avail))


def cpu_gemv_rates(pkg, orc, threads_list, min_bytes=1 << 30):
    """GB/s of the reference CPU GEMVs (the oracle's AVX-512 LUT Q4 GEMV,
    gemv.rs:646-675 / simd.rs:44-83, and the row-dot lm_head,
    gemv.rs:825-864) on the 2048 -> 11008 gate shape (seed 0, x ~ N(0,1))
    and the 128256 x 2048 tied lm_head, each pass over >= min_bytes of
    distinct weight copies so the host caches cannot serve them."""
    out = {}
    k, n = 2048, 11008
    p, s = pkg.synth_q4(0, 4, k, n)
    x = pkg.synth_f32(0, 77, k)
    copies = max(2, math.ceil(min_bytes / (p.nbytes + s.nbytes)))
    ps = [(p.copy(), s.copy()) for _ in range(copies)]
    for T in threads_list:
        orc.set_threads(T)
        orc.gemv_q4(x, ps[0][0], ps[0][1], k, n, T)
        t0 = time.perf_counter()
        for pp, ss in ps:
            orc.gemv_q4(x, pp, ss, k, n, T)
        dt = (time.perf_counter() - t0) / copies
        out[f"gate 2048x11008 T={T}"] = {"us": round(dt * 1e6, 1), "gbps": round(q4_bytes(k, n) / dt / 1e9, 2)}
    del ps
    V, Hd = pkg.SMOLLM3_3B.vocab, pkg.SMOLLM3_3B.hidden
    p, s = pkg.synth_q4(0, 1000, V, Hd)
    x = pkg.synth_f32(0, 78, Hd)
    copies = max(2, math.ceil(min_bytes / (p.nbytes + s.nbytes)))
    ps = [(p, s)] + [(p.copy(), s.copy()) for _ in range(copies - 1)]
    for T in threads_list:
        orc.set_threads(T)
        orc.lm_head_q4(x, ps[0][0], ps[0][1], V, Hd)
        t0 = time.perf_counter()
        for pp, ss in ps:
            orc.lm_head_q4(x, pp, ss, V, Hd)
        dt = (time.perf_counter() - t0) / copies
        out[f"lm_head 128256x2048 T={T}"] = {"us": round(dt * 1e6, 1), "gbps": round(q4_bytes(V, Hd) / dt / 1e9, 2)}
    return out


def cpu_baseline(pkg, orc, w, prompt, seconds=15.0, threads=16):
    """Reference CPU algorithm (oracle) on this host: prefill 8 prompt tokens,
    then decode tokens until `seconds` of decode time have passed."""
    threads = max(1, threads)
    orc.set_threads(threads)
    om = orc.OracleModel(w, kv_capacity=1024, T=threads)
    logits = om.prefill(prompt[:8])
    tok = orc.argmax(logits)
    n = 0
    t0 = time.perf_counter()
    while True:
        logits = om.forward_decode(tok)
        tok = orc.argmax(logits)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 1000:
            break
    return {"value": n / el, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"C restatement of the reference CPU path (AVX-512 LUT GEMV, k-split T={threads}); "
                      f"8-token prefill then {n} greedy decode tokens of the same model, {el:.1f} s"}


def read_traffic(path):
    """HBM bytes per launch of the dominant kernel from a committed rocprofv3
    --pmc summary (line 'traffic_bytes_per_launch: N'), else None."""
    try:
        with open(path) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def extra_decode_rates(be, ctx, pkg, cfg, prompt, cap, steps):
    """Device-chained greedy loop (no host round trip per token), and the
    host-driven decode rate with the KV cache at ~2048 positions."""
    be.kv_reset()
    _, tok = be.raw_prefill(prompt, want_logits=False)
    ctx.synchronize()
    t0 = time.perf_counter()
    be.generate_greedy(tok, steps)
    chained = steps / (time.perf_counter() - t0)
    # prefill 1920 positions, then time 120 tokens
    long_prompt = pkg.synth_tokens(0, 2002, cap - 128, cfg.vocab)
    _, tok = be.raw_prefill(long_prompt, want_logits=False)
    ctx.synchronize()
    n_long = 120
    t0 = time.perf_counter()
    for _ in range(n_long):
        _, tok = be.forward_decode_raw(tok, want_logits=False)
    ctx.synchronize()
    tok_s_2048 = n_long / (time.perf_counter() - t0)
    print(f"# decode at ctx ~2048: {tok_s_2048:.1f} tok/s", file=sys.stderr, flush=True)
    # sampled decode (main.rs defaults: T 0.7, top-p 0.95, top-k 20, penalties 1.1 / 1.5) on the device
    be.kv_reset()
    _, tok = be.raw_prefill(prompt, want_logits=False)
    params = pkg.SampleParams(**pkg.DEFAULT_SAMPLING)
    hist, st = [tok], 0x9E3779B97F4A7C15
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        _, tok, st = be.decode_sample(hist[-1], hist, params, st)
        hist.append(tok)
    sampled = steps / (time.perf_counter() - t0)
    print(f"# sampled decode (device top-k/top-p + penalties): {sampled:.1f} tok/s", file=sys.stderr, flush=True)
    # top_k 0 (every token a candidate, sample_token_top_k's k = vocab): the
    # full device sort and the sequential scan over all 128256 probabilities
    params0 = pkg.SampleParams(**dict(pkg.DEFAULT_SAMPLING, top_k=0))
    n0 = 16
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(n0):
        _, tok, st = be.decode_sample(hist[-1], hist, params0, st)
        hist.append(tok)
    sampled_k0 = n0 / (time.perf_counter() - t0)
    print(f"# sampled decode, top_k 0 (full sort): {sampled_k0:.1f} tok/s", file=sys.stderr, flush=True)
    return chained, tok_s_2048, sampled, sampled_k0


def prefill_rate(be, ctx, pkg, cfg, n=512, reps=3):
    """Batched prefill of n seeded random token ids (seed 1): ms per prompt,
    tokens/s, and the projection GEMMs' useful rate (2 * weights * n flops,
    lm_head and attention excluded) in TFLOP/s."""
    ids = pkg.synth_tokens(1, 2500, n, cfg.vocab)
    be.kv_reset()
    be.raw_prefill(ids, want_logits=False)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        be.kv_reset()
        be.raw_prefill(ids, want_logits=False)
    ctx.synchronize()
    dt = (time.perf_counter() - t0) / reps
    params = sum(k * n_ for (k, n_) in cfg.weight_shapes()) * cfg.num_layers
    tflops = 2.0 * params * n / dt / 1e12
    print(f"# prefill {n} tokens: {dt * 1e3:.2f} ms ({n / dt:.0f} tok/s, projections {tflops:.1f} TFLOP/s)",
          file=sys.stderr, flush=True)
    return {"tokens": n, "ms": round(dt * 1e3, 3), "tok_s": round(n / dt, 1), "gemm_tflops": round(tflops, 2)}


def long_context_rate(ctx, pkg, w, n_ctx=32768, n_tok=64):
    """Host-driven decode with an f16 KV cache holding ~n_ctx positions: every
    layer's cache is filled with seeded random K/V through qora_hip_kv_upload
    (the caller-built RawKvCache path), then n_tok tokens are timed."""
    import dataclasses
    cfg = w.config
    cos_t, sin_t = pkg.rope_tables(n_ctx, cfg.rope_half_dim, cfg.rope_theta)
    wl = dataclasses.replace(w, rope_cos=cos_t, rope_sin=sin_t)
    be = pkg.HipBackend(ctx, wl, kv_capacity=n_ctx, kv_dtype=pkg.KV_F16)
    fill = n_ctx - n_tok - 8
    kvd = cfg.num_kv_heads * cfg.head_dim
    r = np.random.default_rng(7)
    k = r.standard_normal((fill, kvd), dtype=np.float32)
    v = r.standard_normal((fill, kvd), dtype=np.float32)
    for layer in range(cfg.num_layers):
        be.kv_upload(layer, k, v)
    del k, v
    tok = 1
    for _ in range(4):
        _, tok = be.forward_decode_raw(tok, want_logits=False)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(n_tok):
        _, tok = be.forward_decode_raw(tok, want_logits=False)
    ctx.synchronize()
    rate = n_tok / (time.perf_counter() - t0)
    kv_bytes = 2 * cfg.num_layers * (fill + 4 + n_tok // 2) * kvd * 2
    print(f"# decode at ctx ~{n_ctx} (f16 KV): {rate:.1f} tok/s", file=sys.stderr, flush=True)
    return rate, w.weight_bytes_per_token() + kv_bytes


COPY_BYTES = 64 << 20


def calibration_copies(ctx, hip):
    """Three device copies of COPY_BYTES (hipMemcpy's blit kernel reads and
    writes COPY_BYTES each): the known-size dispatches that scale the
    FETCH_SIZE / WRITE_SIZE counters of a --pmc run to bytes."""
    src, dst = ctx.malloc(COPY_BYTES), ctx.malloc(COPY_BYTES)
    for _ in range(3):
        hip.d2d(dst, src, COPY_BYTES)
    ctx.synchronize()
    ctx.free(src)
    ctx.free(dst)


def profile_decode(steps=16, prompt_len=64):
    """The decode step's kernels, launched eagerly, for rocprofv3 --pmc
    runs: the calibration copies, then the prompt's prefill (64 tokens, or
    the 2048-context workload's 1920) and `steps` greedy decode tokens of the
    SmolLM3-3B Q4 model (seed 0, f32 KV cache of 2048 positions). Every
    layer's weights are distinct, so each decode GEMV reads its weights from
    HBM."""
    pkg = entry.load_package()
    cfg = pkg.SMOLLM3_3B
    w = pkg.synthetic_model(cfg, seed=0, rope_positions=2048)
    prompt = (pkg.synth_tokens(0, 2000, 64, cfg.vocab) if prompt_len == 64
              else pkg.synth_tokens(0, 2002, prompt_len, cfg.vocab))
    hip = Hip()
    ctx = pkg.HipContext(0)
    be = pkg.HipBackend(ctx, w, kv_capacity=2048, kv_dtype=pkg.KV_F32)
    calibration_copies(ctx, hip)
    _, tok = be.raw_prefill(prompt, want_logits=False)
    for _ in range(steps):
        _, tok = be.forward_decode_raw(tok, want_logits=False)
    ctx.synchronize()
    print(json.dumps({"profile_decode": {"prompt_tokens": len(prompt), "steps": steps, "copy_bytes": COPY_BYTES,
                                         "last_token": int(tok)}}), flush=True)
    ctx.close()


def profile_kernel(launches=8, shape="gate_up"):
    """The dominant kernel alone, for rocprofv3 --pmc runs: three device
    copies of COPY_BYTES (hipMemcpy's blit kernel: reads and writes
    COPY_BYTES each, the counter calibration), then `launches` launches of
    the gate|up GEMV (2048 -> 2 x 11008, SmolLM3-3B layer 0 weights), or of
    the single gate GEMV (shape "gate": 2048 -> 11008), on distinct packed
    copies, so each launch reads its weights from HBM."""
    pkg = entry.load_package()
    cfg = pkg.SMOLLM3_3B
    hip = Hip()
    ctx = pkg.HipContext(0)
    k, n = cfg.hidden, cfg.intermediate
    gp, gs = pkg.synth_q4(0, 4, k, n)
    up, us = pkg.synth_q4(0, 5, k, n)
    wg = ctx.upload(pkg.Weight(k=k, n=n, packed=gp, scales=gs))
    wu = ctx.upload(pkg.Weight(k=k, n=n, packed=up, scales=us))
    x = ctx.malloc(4 * k)
    acc = ctx.malloc(8 * 2 * n)
    ctx.h2d(x, pkg.synth_f32(0, 77, k))
    calibration_copies(ctx, hip)
    paired = shape == "gate_up"
    gids = [ctx.gemv_prepare(wg, wu if paired else 0, paired) for _ in range(launches)]
    ctx.synchronize()
    for g in gids:
        ctx.check(ctx.lib.qora_hip_gemv_run(ctx.h, g, x, acc, None), "gemv_run")
    ctx.synchronize()
    nbytes = 2 * (k * n // 2 + k * n // 16) + 4 * k + 8 * n if paired else q4_bytes(k, n)
    print(json.dumps({"profile_kernel": "gemv_q4m4_kernel " + ("gate|up 2048x(2x11008)" if paired else
                                                               "gate 2048x11008"),
                      "launches": launches, "algorithmic_bytes_per_launch": nbytes, "copy_bytes": COPY_BYTES}),
          flush=True)
    for g in gids:
        ctx.gemv_release(g)


def probe_context(pkg, cfg, n_tok=32):
    """Host-driven greedy decode rate against the KV cache length: every layer's
    cache is filled with seeded random K/V rows (qora_hip_kv_upload) up to the
    context, then n_tok tokens are timed. An f32 cache of 2048 positions (the
    fused attention + o step below 256 positions, the chunked step below 512,
    the split attention above), and an f16 cache of 32768 positions."""
    import dataclasses
    out = {}
    kvd = cfg.num_kv_heads * cfg.head_dim
    r = np.random.default_rng(7)
    for cap, kv_dtype, label, ctxs in ((2048, pkg.KV_F32, "f32 cache, capacity 2048",
                                        (64, 128, 192, 256, 320, 448, 512, 768, 1024, 1536, 2000)),
                                       (32768, pkg.KV_F16, "f16 cache, capacity 32768",
                                        (512, 1024, 2000, 2048, 3000, 4096, 8192, 16384, 24576, 32700))):
        cos_t, sin_t = pkg.rope_tables(cap, cfg.rope_half_dim, cfg.rope_theta)
        w = dataclasses.replace(pkg.synthetic_model(cfg, seed=0, rope_positions=64), rope_cos=cos_t, rope_sin=sin_t)
        ctx = pkg.HipContext(0)
        try:
            be = pkg.HipBackend(ctx, w, kv_capacity=cap, kv_dtype=kv_dtype)
            per = {}
            for n_ctx in ctxs:
                fill = n_ctx - 4
                k = r.standard_normal((fill, kvd), dtype=np.float32)
                v = r.standard_normal((fill, kvd), dtype=np.float32)
                for layer in range(cfg.num_layers):
                    be.kv_upload(layer, k, v)
                del k, v
                tok = 1
                for _ in range(4):
                    _, tok = be.forward_decode_raw(tok, want_logits=False)
                ctx.synchronize()
                t0 = time.perf_counter()
                for _ in range(n_tok):
                    _, tok = be.forward_decode_raw(tok, want_logits=False)
                ctx.synchronize()
                per[f"{n_ctx}..{n_ctx + n_tok - 1}"] = round(n_tok / (time.perf_counter() - t0), 1)
                print(f"# {label}: positions {n_ctx}..{n_ctx + n_tok - 1}: {per[f'{n_ctx}..{n_ctx + n_tok - 1}']} tok/s",
                      file=sys.stderr, flush=True)
            out[label] = {"attn_o_limit": be.attn_o_limit(), "attn_chunk_limit": be.attn_chunk_limit(), "tok_s": per}
        finally:
            ctx.close()
    return out


def probe_overlap(pkg, hip, cfg, stream_counts=(1, 2, 4, 8)):
    """The decode step's GEMV kernel with its launch boundaries overlapped:
    independent launches over >= 768 MB of distinct packed copies, spread
    round-robin over N streams forked from the context stream inside one
    captured graph (streams and events are created before the capture), so
    a launch's ramp and tail can overlap the next one's. Average microseconds
    per launch and GB/s of algorithmic bytes, per shape and N."""
    import dataclasses
    h = hip.h
    h.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    h.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    h.hipStreamWaitEvent.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint]
    w = pkg.synthetic_model(dataclasses.replace(cfg, num_layers=1, vocab=1000), seed=0, rope_positions=2048)
    ctx = pkg.HipContext(0)
    out = {}
    try:
        be = pkg.HipBackend(ctx, w, kv_capacity=2048, kv_dtype=pkg.KV_F32)
        c = be.config
        x = ctx.malloc(4 * c.intermediate)
        acc = ctx.malloc(8 * 2 * c.intermediate)
        ctx.h2d(x, pkg.synth_f32(0, 77, c.intermediate))
        shapes = c.weight_shapes()
        for label, j, paired in (("down 11008x2048", 6, False), ("gate 2048x11008", 4, False),
                                 ("gate+up 2048x(2x11008)", 4, True)):
            k, n = shapes[j]
            nb = (k * n // 2 + k * n // 16) * (2 if paired else 1)
            algo = nb + 4 * k + (8 if paired else 4) * n
            per = {}
            for ns in stream_counts:
                gids = [ctx.gemv_prepare(int(be.wids[0, j]), int(be.wids[0, 5]) if paired else 0, paired)
                        for _ in range(max(8, math.ceil((768 << 20) / nb)))]
                streams = []
                for _ in range(ns):
                    s = ctypes.c_void_p()
                    assert h.hipStreamCreate(ctypes.byref(s)) == 0
                    streams.append(s.value)
                fork, joins = hip.event(), [hip.event() for _ in streams]
                try:
                    for g in gids[:2]:
                        ctx.check(ctx.lib.qora_hip_gemv_run(ctx.h, g, x, acc, None), "gemv_run")
                    ctx.synchronize()
                    ctx.capture_begin()
                    hip.record(fork, ctx.stream)
                    for s in streams:
                        assert h.hipStreamWaitEvent(s, fork, 0) == 0
                    for i, g in enumerate(gids):
                        ctx.check(ctx.lib.qora_hip_gemv_run(ctx.h, g, x, acc, ctypes.c_void_p(streams[i % ns])),
                                  "gemv_run")
                    for s, e in zip(streams, joins):
                        hip.record(e, s)
                        assert h.hipStreamWaitEvent(ctx.stream, e, 0) == 0
                    gr = ctx.capture_end()
                    try:
                        ctx.graph_launch(gr, 1)
                        ctx.synchronize()
                        a, b, reps = hip.event(), hip.event(), 3
                        hip.record(a, ctx.stream)
                        ctx.graph_launch(gr, reps)
                        hip.record(b, ctx.stream)
                        ms = hip.elapsed_ms(a, b) / (reps * len(gids))
                    finally:
                        ctx.graph_destroy(gr)
                finally:
                    ctx.synchronize()
                    for s in streams:
                        h.hipStreamDestroy(s)
                    for g in gids:
                        ctx.gemv_release(g)
                per[f"{ns} streams"] = {"us": round(ms * 1e3, 3), "gbps": round(algo / (ms * 1e-3) / 1e9, 1)}
            out[label] = per
        ctx.free(x)
        ctx.free(acc)
    finally:
        ctx.close()
    return out


def probe_residency(pkg, hip, cfg, prompt, steps=128, warmup=8):
    """What bounds the decode step besides HBM bandwidth: the per-launch floor
    of a captured graph of dependent launches (the smallest GEMV, 256 -> 128),
    one GEMV launched on a single prepared copy (L2- and Infinity-Cache-resident)
    against 8 and 64 rotating copies, and decode with every layer on layer 0's
    weights (44 MB resident) against the model's own 1.7 GB."""
    out = {}
    w = pkg.synthetic_model(cfg, seed=0, rope_positions=2048)
    ctx = pkg.HipContext(0)
    try:
        be = pkg.HipBackend(ctx, w, kv_capacity=2048, kv_dtype=pkg.KV_F32)
        c = be.config
        x = ctx.malloc(4 * c.intermediate)
        acc = ctx.malloc(8 * 2 * c.intermediate)
        ctx.h2d(x, pkg.synth_f32(0, 77, c.intermediate))
        packed, scales = pkg.synth_q4(0, 99, 256, 128)
        tiny = ctx.upload(pkg.Weight(k=256, n=128, packed=packed, scales=scales))
        g = ctx.gemv_prepare(tiny)
        run = lambda g=g: ctx.check(ctx.lib.qora_hip_gemv_run(ctx.h, g, x, acc, None), "gemv_run")
        out["launch_floor_us_gemv_256x128"] = round(time_graph(ctx, hip, [run] * 200) * 1e3, 3)
        ctx.gemv_release(g)
        shapes = c.weight_shapes()
        res = {}
        for label, j, paired in (("q/o 2048x2048", 0, False), ("down 11008x2048", 6, False),
                                 ("gate+up 2048x(2x11008)", 4, True)):
            k, n = shapes[j]
            nb = (k * n // 2 + k * n // 16) * (2 if paired else 1)
            per = {}
            for copies in (1, 8, 64):
                gids = [ctx.gemv_prepare(int(be.wids[0, j]), int(be.wids[0, 5]) if paired else 0, paired)
                        for _ in range(copies)]
                fns = [(lambda g=g: ctx.check(ctx.lib.qora_hip_gemv_run(ctx.h, g, x, acc, None), "gemv_run"))
                       for g in gids] * max(1, 64 // copies)
                ms = time_graph(ctx, hip, fns)
                for g in gids:
                    ctx.gemv_release(g)
                per[f"{copies} copies ({copies * nb / 2**20:.0f} MiB)"] = round(ms * 1e3, 3)
            res[label] = per
        out["gemv_us_by_copies"] = res
        ctx.free(x)
        ctx.free(acc)
    finally:
        ctx.close()

    def decode_rate(shared):
        ctx = pkg.HipContext(0)
        try:
            be = pkg.HipBackend(ctx, w, kv_capacity=2048, kv_dtype=pkg.KV_F32, shared_layers=shared)
            _, tok = be.raw_prefill(prompt, want_logits=False)
            for _ in range(warmup):
                _, tok = be.forward_decode_raw(tok, want_logits=False)
            ctx.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                _, tok = be.forward_decode_raw(tok, want_logits=False)
            ctx.synchronize()
            return steps / (time.perf_counter() - t0)
        finally:
            ctx.close()

    out["decode_tok_s_own_weights"] = round(decode_rate(False), 1)
    out["decode_tok_s_layer0_weights_everywhere"] = round(decode_rate(True), 1)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-gemv", action="store_true")
    ap.add_argument("--no-f16", action="store_true", help="skip the F16-weight decode and GEMV figures")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--decode-only", action="store_true",
                    help="time only the host-driven decode (skips the chained loop and the ~2048-context run)")
    ap.add_argument("--eager", action="store_true",
                    help="launch every kernel directly instead of replaying HIP graphs (for rocprofv3)")
    ap.add_argument("--profile-prefill", action="store_true",
                    help="only the 512-token batched prefill of the SmolLM3-3B model (for rocprofv3)")
    ap.add_argument("--profile-long", action="store_true",
                    help="only the decode at ~32768 positions with an f16 KV cache (for rocprofv3)")
    ap.add_argument("--profile-decode", action="store_true",
                    help="only the 64-token prefill and 16 decode tokens, launched eagerly after device copies "
                         "of known size, for hardware-counter runs")
    ap.add_argument("--profile-shape", default="gate_up", choices=["gate_up", "gate"],
                    help="GEMV of --profile-kernel: the paired gate|up (default) or the single gate projection")
    ap.add_argument("--profile-prompt", type=int, default=64, choices=[64, 1920],
                    help="prompt length of --profile-decode: 64, or 1920 for the 2048-context workload")
    ap.add_argument("--probe-residency", action="store_true",
                    help="only the launch-floor and cache-residency probes of the decode step")
    ap.add_argument("--probe-context", action="store_true",
                    help="only the decode rate against the KV cache length (f32 up to 2048, f16 up to 32768)")
    ap.add_argument("--probe-overlap", action="store_true",
                    help="only the GEMV kernel with independent launches overlapped on 1, 2, 4 and 8 streams")
    ap.add_argument("--profile-kernel", action="store_true",
                    help="only launch the dominant kernel (gate|up GEMV) eagerly, after a device copy of "
                         "known size, for hardware-counter runs")
    args = ap.parse_args()
    if args.eager:
        global EAGER
        EAGER = True
        os.environ["QORA_HIP_EAGER"] = "1"
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU scaling is not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.profile_kernel:
        profile_kernel(shape=args.profile_shape)
        return
    if args.probe_context:
        pkg = entry.load_package()
        print(json.dumps({"probe_context": probe_context(pkg, pkg.SMOLLM3_3B)}), flush=True)
        return
    if args.probe_overlap:
        pkg = entry.load_package()
        print(json.dumps({"probe_overlap": probe_overlap(pkg, Hip(), pkg.SMOLLM3_3B)}), flush=True)
        return
    if args.probe_residency:
        pkg = entry.load_package()
        cfg = pkg.SMOLLM3_3B
        prompt = pkg.synth_tokens(0, 2000, 64, cfg.vocab)
        print(json.dumps({"probe_residency": probe_residency(pkg, Hip(), cfg, prompt)}), flush=True)
        return
    if args.profile_decode:
        os.environ["QORA_HIP_EAGER"] = "1"
        profile_decode(prompt_len=args.profile_prompt)
        return
    if args.profile_prefill or args.profile_long:
        pkg = entry.load_package()
        cfg = pkg.SMOLLM3_3B
        w = pkg.synthetic_model(cfg, seed=0, rope_positions=2048)
        ctx = pkg.HipContext(0)
        if args.profile_prefill:
            be = pkg.HipBackend(ctx, w, kv_capacity=2048, kv_dtype=pkg.KV_F32)
            print(json.dumps({"profile_prefill": prefill_rate(be, ctx, pkg, cfg)}), flush=True)
        else:
            calibration_copies(ctx, Hip())
            rate, _ = long_context_rate(ctx, pkg, w)
            print(json.dumps({"profile_long_tok_s": round(rate, 2)}), flush=True)
        ctx.close()
        return
    prompt_len, cap = 64, 2048
    if prompt_len + args.warmup + args.steps > cap:
        sys.exit("warmup + steps exceed the 2048-position KV cache")
    cpu_host = host_cpu()

    pkg = entry.load_package()
    cfg = pkg.SMOLLM3_3B
    t0 = time.perf_counter()
    w = pkg.synthetic_model(cfg, seed=0, rope_positions=cap)
    prompt = pkg.synth_tokens(0, 2000, prompt_len, cfg.vocab)
    print(f"# synthetic model ready in {time.perf_counter() - t0:.1f}s", file=sys.stderr, flush=True)
    hip = Hip()
    ctx = pkg.HipContext(0)
    be = pkg.HipBackend(ctx, w, kv_capacity=cap, kv_dtype=pkg.KV_F32)
    print(f"# model on device ({ctx.cus} CUs)", file=sys.stderr, flush=True)

    _, tok = be.raw_prefill(prompt, want_logits=False)
    for _ in range(args.warmup):
        _, tok = be.forward_decode_raw(tok, want_logits=False)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        _, tok = be.forward_decode_raw(tok, want_logits=False)
    ctx.synchronize()
    dt = time.perf_counter() - t0
    tok_s = args.steps / dt
    print(f"# decode {tok_s:.1f} tok/s ({dt / args.steps * 1e3:.3f} ms/token)", file=sys.stderr, flush=True)

    chained = tok_s_2048 = sampled = sampled_k0 = None
    if not args.decode_only:
        chained, tok_s_2048, sampled, sampled_k0 = extra_decode_rates(be, ctx, pkg, cfg, prompt, cap, args.steps)

    prefill = None if args.decode_only else prefill_rate(be, ctx, pkg, cfg)

    gemv = {} if args.no_gemv else gemv_roofline(ctx, hip, be, pkg)
    for kname, v in gemv.items():
        print(f"# {kname}: {v['us']:.2f} us, {v['gbps']:.0f} GB/s", file=sys.stderr, flush=True)

    valu = {} if args.no_gemv else valu_q4_roofline(ctx, hip, be, pkg)
    for kname, v in valu.items():
        print(f"# VALU Q4 {kname}: {v['us']:.2f} us, {v['gbps']:.0f} GB/s", file=sys.stderr, flush=True)

    long_rate = long_bytes = None
    if not args.decode_only:
        long_rate, long_bytes = long_context_rate(ctx, pkg, w)

    roofline = None
    if gemv:
        gu = gemv["gate+up 2048x(2x11008)"]
        roofline = {"bound": "hbm", "achieved": round(gu["gbps"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(gu["gbps"] / HBM_PEAK_GBS, 4),
                    "traffic": read_traffic(os.path.join(ROOT, "profiles", "gate_up_q4_2048x11008_pmc.md")),
                    "kernel": "gemv_q4m4_kernel<GW=1,KW=256,PRO_PLAIN> paired gate|up 2048->2x11008 (qora_hip_gemv_run)",
                    "algorithmic_bytes_per_launch": gu["bytes"], "avg_launch_us": round(gu["us"], 3)}

    weight_bytes = w.weight_bytes_per_token()
    ctx.close()
    f16 = None
    if not args.decode_only and not args.no_f16:
        f16 = f16_measurements(pkg, hip, cfg, prompt, min(args.steps, 128), args.warmup)

    cpu = cpu_t1 = cpu_gemv = None
    if not args.no_cpu_baseline:
        orc = entry.load_oracle()
        T = cpu_threads()
        cpu = cpu_baseline(pkg, orc, w, prompt, seconds=args.cpu_seconds, threads=T)
        print(f"# cpu baseline {cpu['value']:.2f} tok/s on {cpu['cores']} threads", file=sys.stderr, flush=True)
        if not args.decode_only:
            cpu_t1 = cpu_baseline(pkg, orc, w, prompt, seconds=min(args.cpu_seconds, 10.0), threads=1)
            print(f"# cpu baseline {cpu_t1['value']:.2f} tok/s on 1 thread", file=sys.stderr, flush=True)
            cpu_gemv = cpu_gemv_rates(pkg, orc, sorted({T, 1}, reverse=True))
            for kname, v in cpu_gemv.items():
                print(f"# cpu {kname}: {v['us']:.0f} us, {v['gbps']:.2f} GB/s", file=sys.stderr, flush=True)

    out = {
        "metric": "decode tok/s (SmolLM3-3B Q4, bs=1) + Q4 GEMV HBM GB/s vs ~8 TB/s peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(tok_s / PUBLISHED_GPU_TOK_S, 1),
        "dtype": "int8 MFMA + f32",
        "data": "synthetic (seeded random-init weights and token ids)",
        "config": {"workload": "SmolLM3-3B architecture (36 layers, hidden 2048, 16q/4kv heads, hd 128, "
                               "inter 11008, vocab 128256 tied), Q4 g32 weights, 64-token prompt then greedy "
                               "decode, f32 KV cache of 2048 positions, host-driven one token per call",
                   "prompt_tokens": prompt_len, "kv_capacity": cap, "kv_dtype": "f32", "batch": 1, "seed": 0},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "weight_roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / weight_bytes, 1),
        "frac_of_weight_roofline": round(tok_s * weight_bytes / (HBM_PEAK_GBS * 1e9), 4),
        "tok_s_device_chained": round(chained, 2) if chained else None,
        "tok_s_ctx2048": round(tok_s_2048, 2) if tok_s_2048 else None,
        "tok_s_sampled": round(sampled, 2) if sampled else None,
        "tok_s_sampled_top_k0": round(sampled_k0, 2) if sampled_k0 else None,
        "tok_s_ctx32768_f16kv": round(long_rate, 2) if long_rate else None,
        "prefill_512": prefill,
        "frac_of_roofline_ctx32768": (round(long_rate * long_bytes / (HBM_PEAK_GBS * 1e9), 4)
                                      if long_rate else None),
        "gemv_gbps": {k2: round(v["gbps"], 1) for k2, v in gemv.items()},
        "gemv_us": {k2: round(v["us"], 3) for k2, v in gemv.items()},
        "gemv_gbps_valu_q4": {k2: round(v["gbps"], 1) for k2, v in valu.items()},
        "f16": f16,
        "cpu_host": cpu_host,
        "cpu_baseline_t1": cpu_t1,
        "cpu_gemv_gbps": cpu_gemv,
        "vs_baseline_ref": "reference GPU decode ~4.1 tok/s (README.md:43,157, GTX 1660 SUPER)",
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
