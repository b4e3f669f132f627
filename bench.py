#!/usr/bin/env python3
"""Decode throughput of the 4B-class TQ1_0 model on one MI355X.

Prints one JSON line:
  value      greedy decode tok/s of the 4B-class dense decoder (36 layers,
             d_model 2560, 32/8 heads x 128, SwiGLU 9728, vocab 151936, TQ1_0
             linear weights, f16 embedding and output), fully HBM-resident,
             batch 1, KV cache pre-filled with 2048 positions of f16 N(0,1)
             values; exact attention (logits bit-identical to RustFox's).
  roofline   the fused TQ1_0 GEMV kernel (gemv_fused, 14336 x 4096, one
             token): algorithmic bytes per launch / its mean launch time from
             HIP events on the stream it runs on, against 8 TB/s.  traffic is
             the HBM bytes per launch that rocprofv3 counts (FETCH_SIZE and
             WRITE_SIZE, two runs of --gemv-only made before this process
             touches the GPU), each counter scaled by its reading for a plain
             256 MiB device copy.
  cpu_baseline  the CPU restatement of RustFox's decode path (the oracle,
             oracle/liboracle.so) on the same workload: the same model file,
             the same 2048 injected cache rows, greedy steps at positions
             2048+, its GEMVs and attention heads split over a pool of
             threads as RustFox splits them.  Beside it: RustFox itself
             (compiled from its sources into oracle/_ref) decoding the same
             file at short context (its cache cannot be pre-filled), both at
             the pool size and on one thread, and the host's CPU model, core
             count and NUMA layout.
  extra      the 8B-class Q4_K/Q6_K model after 4096 cached positions and the
             27B-class TQ1_0 model after 8192 cached positions (batch-1
             decode and the 8-token verify pass), each with its HBM GB/s.

A step is one token through all 36 layers, the output head and the greedy
pick.  Inputs are resident in HBM before the timed region starts.
"""
from __future__ import annotations

import argparse
import ctypes
import csv
import glob
import json
import os
import shutil
import statistics
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import rustfox_amd as rf  # noqa: E402
from rustfox_amd import synth  # noqa: E402

HBM_PEAK_GBS = 8000.0
PREFILL = 2048


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ decode

def kv_rows(spec, n, seed, layer):
    rng = np.random.default_rng([seed, 0xCAC4E, layer])
    kvd = spec.n_head_kv * spec.head_dim
    k = rng.standard_normal((n, kvd), dtype=np.float32).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((n, kvd), dtype=np.float32).astype(np.float16).astype(np.float32)
    return k, v


def prefill_cache(set_kv, set_pos, spec, n, seed=11, shared=False):
    """f16 N(0,1) rows 0..n-1 of every layer's K and V cache; shared: the
    same rows in every layer (the larger models, where drawing
    n_layer distinct caches would dominate the run)."""
    kv = kv_rows(spec, n, seed, 0) if shared else None
    for layer in range(spec.n_layer):
        k, v = kv if shared else kv_rows(spec, n, seed, layer)
        set_kv(layer, k, v)
    set_pos(n)


def time_decode(ctx, prefill, steps, warmup, exact):
    """Seconds of `steps` greedy steps after `warmup` untimed ones, from
    token 1 at position `prefill`; returns (seconds, timed ids, warmup ids +
    timed ids)."""
    ctx.set_attention(exact)
    ctx.set_position(prefill)
    tok = 1
    first = []
    if warmup:
        first = [int(i) for i in ctx.decode_greedy(tok, warmup)]
        tok = first[-1]
    t0 = time.perf_counter()
    ids = ctx.decode_greedy(tok, steps)
    dt = time.perf_counter() - t0
    return dt, ids, first + [int(i) for i in ids]


def first_logits(ctx, prefill, exact):
    """The logits of token 1 at position `prefill` (fox_eval)."""
    ctx.set_attention(exact)
    ctx.set_position(prefill)
    return ctx.eval([1]).copy()


def token_bytes(spec, mean_pos):
    """Algorithmic HBM bytes of one decode token: every linear weight and the
    output head in their GGUF bytes, the norm vectors, one embedding row and
    the K and V cache rows attention reads (f32)."""
    b = 0
    for name, ne0, ne1, gt in synth.tensor_list(spec):
        rb = synth.row_bytes(gt, ne0)
        b += rb if name == "token_embd.weight" else max(ne1, 1) * rb
    return b + 2 * spec.n_layer * int(mean_pos) * spec.n_head_kv * spec.head_dim * 4


def model_file(workdir, spec):
    path = synth.path_in(workdir, spec)
    if not os.path.exists(path):
        t0 = time.perf_counter()
        synth.write_gguf(path, spec)
        log(f"bench: wrote {path} ({os.path.getsize(path) / 1e9:.2f} GB) in "
            f"{time.perf_counter() - t0:.1f} s")
    return path


def extra_case(workdir, name, prefill, steps, warmup, verify):
    """Greedy decode of one of the larger models after `prefill` cached
    positions (and, with verify, the 8-token pass: fox_eval of 8 drafted
    tokens, the last position's logits)."""
    spec = synth.spec(name, n_ctx=prefill + warmup + steps + 16)
    path = model_file(workdir, spec)
    t0 = time.perf_counter()
    model = rf.Model(path, mode=rf.WEIGHTS_DEVICE)
    ctx = model.context(spec.n_ctx, n_batch=8)
    prefill_cache(lambda l, k, v: ctx.set_kv(l, 0, k, v), ctx.set_position, spec, prefill,
                  shared=True)
    log(f"bench: {name} HBM load + cache prefill {time.perf_counter() - t0:.1f} s")
    dt, ids, _ = time_decode(ctx, prefill, steps, warmup, exact=True)
    tok_s = steps / dt
    gbs = token_bytes(spec, prefill + warmup + steps / 2) * tok_s / 1e9
    out = {"workload": f"{name}-class dense decoder ({spec.n_layer} layers, d_model "
                       f"{spec.n_embd}, {spec.n_head}/{spec.n_head_kv} heads x {spec.head_dim}, "
                       f"ffn {spec.n_ff}, vocab {spec.n_vocab}), batch 1, greedy decode after "
                       f"{prefill} cached positions (f16 N(0,1) rows, the same in every layer)",
           "tok_s": round(tok_s, 2), "ms_per_token": round(dt * 1e3 / steps, 3),
           "steps": steps, "decode_hbm_gbs": round(gbs, 1),
           "frac_of_hbm": round(gbs / HBM_PEAK_GBS, 4),
           "greedy_ids_head": [int(i) for i in ids[:4]]}
    log(f"bench: {name} decode {tok_s:.1f} tok/s, {gbs:.0f} GB/s")
    if verify:
        reps = 8
        draft = np.array(ids[:8], np.uint32)
        times = []
        for _ in range(reps):
            ctx.set_position(prefill)
            t0 = time.perf_counter()
            ctx.eval(draft)
            times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        gbs8 = token_bytes(spec, prefill + 4) / med / 1e9
        out["verify8"] = {"tokens_per_pass": 8, "ms_per_pass": round(med * 1e3, 3),
                          "tok_s": round(8 / med, 2), "weight_and_kv_gbs": round(gbs8, 1),
                          "passes": reps,
                          "note": "fox_eval of 8 drafted tokens at position " + str(prefill) +
                                  ": one pass over the weights for all 8 (int8 MFMA columns), "
                                  "last position's logits copied to the host"}
        log(f"bench: {name} 8-token verify {8 / med:.1f} tok/s ({med * 1e3:.2f} ms per pass)")
    ctx.close()
    model.close()
    os.remove(path)
    return out


def stream_case(path, spec, warmup, slots=8, steps=8):
    """The same 4B model through the streaming backend with HBM for `slots`
    of its 36 layers: every token reads the other layers from the file into
    pinned host memory and uploads them on the copy stream, one layer ahead
    of the compute."""
    layer = outside = 0
    for name, ne0, ne1, gt in synth.tensor_list(spec):
        b = max(ne1, 1) * synth.row_bytes(gt, ne0)
        if name.startswith("blk.0."):
            layer += b
        elif not name.startswith("blk."):
            outside += b
    model = rf.Model(path, mode=rf.WEIGHTS_STREAM, budget=outside + slots * layer)
    ctx = model.context(spec.n_ctx, n_batch=8)
    prefill_cache(lambda l, k, v: ctx.set_kv(l, 0, k, v), ctx.set_position, spec, PREFILL)
    dt, ids, _ = time_decode(ctx, PREFILL, steps, 2, exact=True)
    w = model.weights()
    ev = model.lib.fox_weights_evictions(w)
    ctx.close()
    model.close()
    tok_s = steps / dt
    moved = (spec.n_layer - slots) * layer * tok_s / 1e9
    log(f"bench: 4b streamed ({slots} of {spec.n_layer} layer slots) {tok_s:.2f} tok/s")
    return {"workload": f"4B-class model, FOX_WEIGHTS_STREAM with HBM for the tensors outside "
                        f"the layers and {slots} of the {spec.n_layer} layers; every token "
                        f"re-reads the other layers from the file (page cache) into pinned "
                        f"host memory and uploads them on the copy stream",
            "tok_s": round(tok_s, 3), "steps": steps,
            "layer_bytes_streamed_gbs": round(moved, 2), "tensor_evictions": int(ev),
            "greedy_ids_head": [int(i) for i in ids[:4]]}


# --------------------------------------------------------------- GEMV bench

def gemv_bytes(gtype, N, K, M):
    """Algorithmic bytes of one launch of fox_gpu_gemv (f32 activations in,
    quantised inside the kernel): packed weights + f32 activations + f32
    outputs."""
    wb = N * synth.row_bytes(gtype, K)
    return wb + 4 * M * K + 4 * M * N


def gemv_case(gpu, gtype, N, K, M, rotate_bytes=1 << 30, min_launches=400):
    rng = np.random.default_rng([N, K, gtype])
    if gtype == rf.TQ1_0:
        w = synth.tq1_random(rng, N * K // 256).reshape(-1)
    else:
        w = synth.tq2_random(rng, N * K // 256).reshape(-1)
    n_copies = max(2, -(-rotate_bytes // w.nbytes))
    ts = [gpu.tensor(gtype, K, N, w) for _ in range(n_copies)]
    x = gpu.array(rng.standard_normal((M, K)).astype(np.float32))
    out = gpu.empty((M, N), np.float32)
    for i in range(min(n_copies, 32)):
        gpu.gemv(ts[i], x, M, out)
    gpu.sync()
    launches = max(min_launches, 2 * n_copies)
    e0, e1 = gpu.event(), gpu.event()
    gpu.record(e0)
    for i in range(launches):
        gpu.gemv(ts[i % n_copies], x, M, out)
    gpu.record(e1)
    ms = gpu.elapsed_ms(e0, e1)
    for t in ts:
        t.free()
    us = ms * 1e3 / launches
    b = gemv_bytes(gtype, N, K, M)
    return dict(type=synth.TYPE_NAMES[gtype], rows=N, cols=K, tokens=M, us_per_launch=round(us, 3),
                bytes_per_launch=b, gbs=round(b / us / 1e3, 1),
                frac_of_hbm=round(b / us / 1e3 / HBM_PEAK_GBS, 4), weight_copies=n_copies)


COPY_BYTES = 256 << 20


def gemv_only():
    """The roofline case (TQ1_0 14336 x 4096, one token) and a plain device
    copy of COPY_BYTES, whose counter readings scale the GEMV's."""
    gpu = rf.Gpu(0)
    r = gemv_case(gpu, rf.TQ1_0, 14336, 4096, 1, min_launches=100)
    src = gpu.empty(COPY_BYTES, np.uint8)
    dst = gpu.empty(COPY_BYTES, np.uint8)
    gpu.copy(dst, src, COPY_BYTES)
    gpu.sync()
    gpu.copy(dst, src, COPY_BYTES)
    gpu.sync()
    src.free()
    dst.free()
    gpu.close()
    log(f"bench: gemv-only {r['us_per_launch']} us per launch; copied {COPY_BYTES} bytes twice")


def gemv_counters():
    """Fixed launches for instruction counters: the TQ1_0 14336 x 4096 GEMV
    at one and at eight tokens, and the 27B-class gate/up + SwiGLU (2 x 21504
    x 5376) at eight tokens, six launches each on the same inputs."""
    gpu = rf.Gpu(0)
    rng = np.random.default_rng(3)

    def tensor(N, K):
        return gpu.tensor(rf.TQ1_0, K, N, synth.tq1_random(rng, N * K // 256).reshape(-1))

    w = tensor(14336, 4096)
    for M in (1, 8):
        x = gpu.array(rng.standard_normal((M, 4096)).astype(np.float32))
        out = gpu.empty((M, 14336), np.float32)
        for _ in range(6):
            gpu.gemv(w, x, M, out)
    gpu.sync()
    wg, wu = tensor(21504, 5376), tensor(21504, 5376)
    x = gpu.array(rng.standard_normal((8, 5376)).astype(np.float32))
    nw = gpu.array(np.ones(5376, np.float32))
    h = gpu.empty((8, 21504), np.float32)
    for _ in range(6):
        gpu.gate_up_silu(wg, wu, x, 8, nw, 1e-6, h)
    gpu.sync()
    gpu.close()
    log("bench: gemv-counters launches done")


READ_PROBE_BYTES = 1 << 30


def read_probe():
    """The HBM read ceiling: a 1 GiB streaming read (fox_gpu_read_probe,
    workgroups reading contiguous chunks) with 1 to 16 16-byte loads in flight
    per thread and 1024 to 8192 workgroups of 256 threads, beside a device
    copy of the same size; mean of 10 timed
    launches after 2 untimed ones, HIP events on the launching stream.  Then
    single launches reading 3 to 64 MB (a decode kernel's share), and the
    cost of an empty kernel launched back to back and as a graph node.  One
    JSON line per case on stdout."""
    gpu = rf.Gpu(0)
    src = gpu.empty(READ_PROBE_BYTES, np.uint8)
    dst = gpu.empty(READ_PROBE_BYTES, np.uint8)
    src.fill(0x5a)
    sink = gpu.array(np.zeros(1, np.uint32))
    e0, e1 = gpu.event(), gpu.event()

    def timed(run):
        for _ in range(2):
            run()
        gpu.record(e0)
        for _ in range(10):
            run()
        gpu.record(e1)
        return gpu.elapsed_ms(e0, e1) / 10
    for loads in (1, 2, 4, 8, 16):
        for grid in (1024, 2048, 4096, 8192):
            ms = timed(lambda: gpu.read_probe(src, READ_PROBE_BYTES, loads, grid, sink))
            print(json.dumps({"probe": "read", "loads_in_flight": loads, "workgroups": grid,
                              "us": round(ms * 1e3, 1),
                              "gbs": round(READ_PROBE_BYTES / ms / 1e6, 1)}), flush=True)
    ms = timed(lambda: gpu.copy(dst, src, READ_PROBE_BYTES))
    print(json.dumps({"probe": "copy", "us": round(ms * 1e3, 1),
                      "gbs_read": round(READ_PROBE_BYTES / ms / 1e6, 1),
                      "gbs_read_plus_write": round(2 * READ_PROBE_BYTES / ms / 1e6, 1)}),
          flush=True)
    # one launch at the sizes of a decode step's kernels (2 loads in flight,
    # 1024 workgroups): a new region of the buffer each launch (cold), or
    # the same region every time (warm: the infinity cache and L2 hold it)
    for n in (3 << 20, 15138816 // 4096 * 4096, 27 << 20, 64 << 20):
        nreg = READ_PROBE_BYTES // n
        for mode in ("cold", "warm"):
            offs = [(i % nreg) * n if mode == "cold" else 0 for i in range(64)]
            run = lambda o: rf._check(gpu.lib.fox_gpu_read_probe(gpu.ctx, src.ptr + o, n, 2,
                                                                  1024, sink.ptr))
            for o in offs[:4]:
                run(o)
            gpu.record(e0)
            for o in offs:
                run(o)
            gpu.record(e1)
            us = gpu.elapsed_ms(e0, e1) * 1e3 / len(offs)
            print(json.dumps({"probe": "read_one_launch", "bytes": n, "mode": mode,
                              "us": round(us, 2), "gbs": round(n / us / 1e3, 1)}), flush=True)
    # the fixed cost of a kernel: empty launches back to back on the stream,
    # and as the nodes of one captured graph (the decode replays one graph
    # per token)
    for grid in (1, 256, 1024):
        for _ in range(50):
            gpu.empty_probe(grid, sink)
        gpu.record(e0)
        for _ in range(2000):
            gpu.empty_probe(grid, sink)
        gpu.record(e1)
        us_stream = gpu.elapsed_ms(e0, e1) * 1e3 / 2000
        rf._check(gpu.lib.fox_gpu_graph_begin(gpu.ctx))
        for _ in range(100):
            gpu.empty_probe(grid, sink)
        g = ctypes.c_void_p()
        rf._check(gpu.lib.fox_gpu_graph_end(gpu.ctx, ctypes.byref(g)))
        for _ in range(3):
            rf._check(gpu.lib.fox_gpu_graph_launch(gpu.ctx, g))
        gpu.record(e0)
        for _ in range(20):
            rf._check(gpu.lib.fox_gpu_graph_launch(gpu.ctx, g))
        gpu.record(e1)
        us_node = gpu.elapsed_ms(e0, e1) * 1e3 / 2000
        gpu.lib.fox_gpu_graph_free(g)
        print(json.dumps({"probe": "empty_kernel", "workgroups": grid,
                          "us_per_stream_launch": round(us_stream, 2),
                          "us_per_graph_node": round(us_node, 2)}), flush=True)
    gpu.close()


def pmc_run(counter, timeout):
    """Per-dispatch readings of one counter over a --gemv-only run:
    (mean of the fused GEMV's, largest of the device copy's), in KiB."""
    exe = shutil.which("rocprofv3")
    if not exe:
        return None
    d = tempfile.mkdtemp(prefix="foxpmc-", dir="/tmp")
    try:
        cmd = [exe, "--pmc", counter, "--kernel-trace", "-d", d, "-o", "pmc", "-f", "csv",
               "--", sys.executable, os.path.abspath(__file__), "--gemv-only"]
        subprocess.run(cmd, timeout=timeout, stdout=subprocess.DEVNULL,
                       stderr=subprocess.DEVNULL, check=True)
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        gemv, copy = [], []
        for r in csv.DictReader(open(files[0])):
            if r["Counter_Name"] != counter:
                continue
            if "gemv_fused" in r["Kernel_Name"]:
                gemv.append(float(r["Counter_Value"]))
            elif "copyBuffer" in r["Kernel_Name"]:
                copy.append(float(r["Counter_Value"]))
        return statistics.mean(gemv), max(copy)
    finally:
        shutil.rmtree(d, ignore_errors=True)


def measure_traffic(timeout=180):
    """HBM bytes per launch of the roofline GEMV: FETCH_SIZE + WRITE_SIZE,
    each scaled so that the COPY_BYTES copy reads (or writes) COPY_BYTES."""
    try:
        total = 0.0
        scales = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            log(f"bench: rocprofv3 --pmc {counter} over the roofline GEMV and a copy")
            r = pmc_run(counter, timeout)
            if r is None:
                return None
            g, c = r
            scales[counter] = COPY_BYTES / (c * 1024)
            total += g * 1024 * scales[counter]
        log(f"bench: counted traffic {total / 1e6:.3f} MB per launch (scales: fetch "
            f"{scales['FETCH_SIZE']:.3f}, write {scales['WRITE_SIZE']:.3f})")
        return int(round(total))
    except Exception as e:  # the roofline stands without it
        log(f"bench: traffic counters unavailable: {e}")
        return None


# ------------------------------------------------------------ CPU baseline

def cpu_threads():
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit():
        n = min(n, int(cap))
    return max(1, min(n, 256))


def host_info():
    """CPU model, logical CPUs, sockets/cores and NUMA layout (lscpu)."""
    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k in ("Model name", "CPU(s)", "Socket(s)", "Core(s) per socket",
                     "Thread(s) per core", "NUMA node(s)") or k.startswith("NUMA node") and "CPU" in k:
                info[k] = v
    except Exception as e:  # the baseline stands without it
        info["error"] = str(e)
    info["affinity_cpus"] = len(os.sched_getaffinity(0))
    return info


def timed_tokens(step, budget_s, max_tokens, min_tokens=2, warm=True):
    """Median seconds per call of step() (after one untimed call when warm),
    as many calls as fit the budget (between min_tokens and max_tokens)."""
    if warm:
        step()
    times = []
    t_start = time.perf_counter()
    while len(times) < max_tokens and (len(times) < min_tokens or
                                       time.perf_counter() - t_start < budget_s):
        times.append(step())
    return statistics.median(times), len(times)


def cpu_port(path, spec, threads, budget_s, max_tokens, min_tokens=2, warm=True,
             prefill=PREFILL):
    """The oracle (oracle/liboracle.so, the C restatement of RustFox's path)
    decoding the same file after the same injected cache rows, greedy from
    token 1 at position `prefill` (0: an empty cache, as RustFox itself is
    timed).  Returns the median step time, the number of timed steps, the
    greedy ids of every step (the untimed first one included) and the first
    step's logits."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_libs import Oracle  # test infrastructure: the oracle, timed as the CPU baseline
    om = Oracle().model(spec, synth.map_tensors(path, spec))
    ctx = om.context(prefill + max_tokens + 8, n_batch=8, n_threads=threads)
    if prefill:
        prefill_cache(lambda l, k, v: ctx.set_kv(l, 0, k, v), ctx.set_pos, spec, prefill)
    state = {"tok": 1, "ids": [], "first": None}

    def step():
        t0 = time.perf_counter()
        lg = ctx.eval(np.array([state["tok"]], np.uint32))
        dt = time.perf_counter() - t0
        if state["first"] is None:
            state["first"] = lg.copy()
        state["tok"] = int(np.argmax(lg))
        state["ids"].append(state["tok"])
        return dt
    med, n = timed_tokens(step, budget_s, max_tokens, min_tokens, warm)
    ctx.close()
    return med, n, state["ids"], state["first"]


def cpu_reference(path, threads, budget_s, max_tokens, min_tokens=2):
    """RustFox itself (oracle/_ref, built from its sources) decoding the same
    file from position 1 (its cache cannot be pre-filled)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_libs import REF_FAST_SO, Ref  # test infrastructure: the reference
    if not os.path.exists(REF_FAST_SO):
        return None
    ref = Ref(REF_FAST_SO)
    m = ref.open_model(path)
    ctx = m.context(64, n_batch=32, n_threads=threads)
    state = {"tok": 1}

    def step():
        lg = ctx.eval(np.array([state["tok"]], np.uint32))
        state["tok"] = int(np.argmax(lg))
        return ctx.last_seconds()
    med, n = timed_tokens(step, budget_s, max_tokens, min_tokens)
    ctx.close()
    m.close()
    return med, n


PARITY_STEPS = 64


def parity(gpu_ids, gpu_first, cpu_ids, cpu_first):
    """The GPU decode against the oracle's on the same model and state:
    greedy ids over the steps both ran, and the first step's logits."""
    n = min(len(gpu_ids), len(cpu_ids))
    d = np.asarray(gpu_first, np.float64) - np.asarray(cpu_first, np.float64)
    rel = float(np.linalg.norm(d) / np.linalg.norm(np.asarray(cpu_first, np.float64)))
    diff = [i for i in range(n) if int(gpu_ids[i]) != int(cpu_ids[i])]
    return {"steps_compared": n, "ids_equal": not diff,
            "first_differing_step": diff[0] if diff else None,
            "first_logits_bit_identical": bool(np.array_equal(
                np.asarray(gpu_first, np.float32).view(np.uint32),
                np.asarray(cpu_first, np.float32).view(np.uint32))),
            "rel_l2": rel}


def cpu_baseline(path, spec, budget_s):
    threads = cpu_threads()
    # the parity run: PARITY_STEPS greedy steps (the first untimed), every
    # one's id kept; the median step time is the baseline
    med, n, ids, first = cpu_port(path, spec, threads, 1e9, PARITY_STEPS - 1,
                                  min_tokens=PARITY_STEPS - 1)
    log(f"bench: cpu port {1 / med:.3f} tok/s on {threads} threads ({n} tokens)")
    # one token on one thread (its pages are already in from the run above)
    med1, n1, _, _ = cpu_port(path, spec, 1, 0.0, 1, min_tokens=1, warm=False)
    log(f"bench: cpu port {1 / med1:.3f} tok/s on 1 thread ({n1} tokens)")
    out = {"value": round(1.0 / med, 3), "unit": "tok/s", "cores": threads, "kind": "port",
           "sample": (f"the oracle (oracle/liboracle.so, the C restatement of RustFox's decode "
                      f"path, -O2, GEMV rows and attention heads split over a pool of {threads} "
                      f"threads as RustFox splits them) decoding the same 4B TQ1_0 GGUF after "
                      f"the same {PREFILL} injected f16 N(0,1) cache rows: median of {n} "
                      f"single-token steps at positions {PREFILL + 1}..{PREFILL + n} (one "
                      f"untimed step first); the same run's greedy ids and first logits are "
                      f"the parity check of the GPU decode"),
           "one_thread": {"value": round(1.0 / med1, 4), "unit": "tok/s", "tokens": n1,
                          "note": "one step at position " + str(PREFILL + 1)},
           "host": host_info(),
           "_parity": (ids, first)}
    try:
        r = cpu_reference(path, threads, budget_s * 0.15, 16)
        r1 = cpu_reference(path, 1, 0.0, 1, min_tokens=1) if r else None
        if r:
            # the port at the same short context, same threads, same run:
            # the fidelity of the port-based figure
            ps, pn, _, _ = cpu_port(path, spec, threads, budget_s * 0.15, 16, prefill=0)
            out["port_vs_reference"] = {
                "port_tok_s": round(1.0 / ps, 3), "reference_tok_s": round(1.0 / r[0], 3),
                "port_tok_s_over_reference": round(r[0] / ps, 3), "cores": threads,
                "sample": (f"both decode the same file greedy from token 1 with an empty "
                           f"cache on {threads} threads: medians of {pn} (port) and {r[1]} "
                           f"(RustFox) steps at positions 2..17; RustFox's own time per "
                           f"step, the port's around its eval call")}
            log(f"bench: cpu port {1 / ps:.3f} tok/s vs reference {1 / r[0]:.3f} tok/s at "
                f"short context ({r[0] / ps:.3f}x)")
            out["reference_short_context"] = {
                "value": round(1.0 / r[0], 3), "unit": "tok/s", "cores": threads,
                "one_thread": round(1.0 / r1[0], 4) if r1 else None,
                "sample": (f"RustFox's own fox_eval (built from its sources, -O3 "
                           f"-march=x86-64-v3) on the same file, threadpool of {threads}: "
                           f"median of {r[1]} steps at positions 2..{r[1] + 1}; its cache "
                           f"cannot be pre-filled, so attention reads at most {r[1] + 2} "
                           f"rows instead of {PREFILL}+")}
            log(f"bench: cpu reference {1 / r[0]:.3f} tok/s on {threads} threads at short "
                f"context")
    except Exception as e:  # the port's figure stands without it
        log(f"bench: reference timing failed: {e}")
    return out


# --------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=40.0)
    ap.add_argument("--extra-steps", type=int, default=32,
                    help="decode steps of the 8B- and 27B-class runs")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the 8B- and 27B-class runs")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemv", action="store_true")
    ap.add_argument("--workdir", default=None)
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc runs behind roofline.traffic")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only the roofline GEMV case and a 256 MB device copy (the runs "
                         "that rocprofv3 --pmc counts for the traffic figure)")
    ap.add_argument("--gemv-counters", action="store_true",
                    help="only six launches each of the TQ1_0 14336 x 4096 GEMV at 1 and 8 "
                         "tokens and the 27B-class gate/up + SwiGLU at 8 (for rocprofv3 "
                         "instruction counters)")
    ap.add_argument("--read-probe", action="store_true",
                    help="only the HBM read-ceiling probes (1 GiB streaming reads with 1-16 "
                         "loads in flight per thread, a device copy, single launches at "
                         "decode-step sizes, the cost of an empty launch and graph node), "
                         "one JSON line per case")
    a = ap.parse_args()

    if a.gpus != 1:
        print(f"bench.py: rustfox_amd runs on one GPU; --gpus {a.gpus} is not supported "
              "(sharding is designed but not built)", file=sys.stderr)
        sys.exit(2)

    if a.gemv_only:
        gemv_only()
        return
    if a.gemv_counters:
        gemv_counters()
        return
    if a.read_probe:
        read_probe()
        return
    # (child processes: they run before this process initialises the GPU)
    traffic = None if (a.no_traffic or a.no_gemv) else measure_traffic()

    spec = synth.spec("4b", n_ctx=PREFILL + a.warmup + a.steps)
    workdir = a.workdir or tempfile.mkdtemp(prefix="foxbench-", dir="/tmp")
    path = model_file(workdir, spec)

    t0 = time.perf_counter()
    model = rf.Model(path, mode=rf.WEIGHTS_DEVICE)
    ctx = model.context(spec.n_ctx, n_batch=8)
    prefill_cache(lambda l, k, v: ctx.set_kv(l, 0, k, v), ctx.set_position, spec, PREFILL)
    log(f"bench: HBM load + cache prefill {time.perf_counter() - t0:.1f} s")

    dt, ids, all_ids = time_decode(ctx, PREFILL, a.steps, a.warmup, exact=True)
    tok_s = a.steps / dt
    log(f"bench: exact attention  {tok_s:.1f} tok/s ({dt * 1e3 / a.steps:.3f} ms/token)")
    dt_split, ids_split, all_split = time_decode(ctx, PREFILL, a.steps, a.warmup, exact=False)
    log(f"bench: split attention  {a.steps / dt_split:.1f} tok/s")
    lg_exact = first_logits(ctx, PREFILL, True)
    lg_split = first_logits(ctx, PREFILL, False)
    ctx.close()
    model.close()

    extra = {}
    if not a.no_extra:
        try:
            extra["4b_stream"] = stream_case(path, spec, a.warmup)
        except Exception as e:  # the headline stands without it
            log(f"bench: streaming run failed: {e}")
            extra["4b_stream"] = {"error": str(e)}
        for name, pre, verify in (("8b", 4096, False), ("27b", 8192, True)):
            try:
                extra[name] = extra_case(workdir, name, pre, a.extra_steps, 4, verify)
            except Exception as e:  # the headline stands without it
                log(f"bench: {name} run failed: {e}")
                extra[name] = {"error": str(e)}

    gemv = []
    roof = None
    if not a.no_gemv:
        gpu = rf.Gpu(0)
        for gtype in (rf.TQ1_0, rf.TQ2_0):
            for (N, K) in ((4096, 4096), (14336, 4096)):
                for M in (1, 8):
                    r = gemv_case(gpu, gtype, N, K, M)
                    gemv.append(r)
                    log(f"bench: gemv {r['type']} {N}x{K} M={M}: {r['us_per_launch']} us, "
                        f"{r['gbs']} GB/s ({100 * r['frac_of_hbm']:.1f}% of 8 TB/s)")
        gpu.close()
        main_case = [g for g in gemv if g["type"] == "TQ1_0" and g["rows"] == 14336
                     and g["tokens"] == 1][0]
        roof = {"bound": "hbm", "achieved": main_case["gbs"], "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(main_case["gbs"] / HBM_PEAK_GBS, 4),
                "traffic": traffic,
                "kernel": "gemv_fused<TQ1_0, f32 in, store>, 14336x4096, 1 token",
                "bytes_per_launch": main_case["bytes_per_launch"],
                "us_per_launch": main_case["us_per_launch"]}

    cpu = None
    par = par_split = None
    if not a.no_cpu:
        try:
            cpu = cpu_baseline(path, spec, a.cpu_seconds)
            if cpu:
                log(f"bench: cpu baseline ({cpu['kind']}) {cpu['value']} tok/s on {cpu['cores']} threads")
                cpu_ids, cpu_first = cpu.pop("_parity")
                par = parity(all_ids, lg_exact, cpu_ids, cpu_first)
                par_split = parity(all_split, lg_split, cpu_ids, cpu_first)
                log(f"bench: parity against the oracle: {par}")
                log(f"bench: split attention against the oracle: {par_split}")
        except Exception as e:  # the GPU number stands without it
            log(f"bench: cpu baseline failed: {e}")

    if not a.workdir:
        try:
            os.remove(path)
            os.rmdir(workdir)
        except OSError:
            pass

    per_token_bytes = token_bytes(spec, PREFILL + a.warmup + a.steps / 2)
    line = {
        "metric": "decode tok/s on 1 MI355X; quantized-GEMV HBM GB/s as % of peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(dt * 1e3 / a.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x ternary (int32 block sums), f32 combine",
        "data": "synthetic (seeded ternary weights, f16 N(0,0.02) embeddings, f16 N(0,1) cache)",
        "config": {"workload": "4B-class dense decoder, TQ1_0, HBM-resident, batch 1, "
                               "greedy decode after a 2048-position pre-filled cache",
                   "layers": spec.n_layer, "d_model": spec.n_embd, "heads": spec.n_head,
                   "kv_heads": spec.n_head_kv, "head_dim": spec.head_dim, "ffn": spec.n_ff,
                   "vocab": spec.n_vocab, "kv_context": PREFILL, "kv_dtype": "f32",
                   "attention": "exact (reference summation order)"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "parity": par,
        "split_attention": {"tok_s": round(a.steps / dt_split, 2), "parity": par_split,
                            "note": "positions split over workgroups with a merge of partial "
                                    "softmaxes (float reassociation); not the headline"},
        "decode_hbm_gbs": round(per_token_bytes * tok_s / 1e9, 1),
        "decode_frac_of_hbm": round(per_token_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4),
        "extra": extra,
        "gemv": gemv,
        "greedy_ids_head": [int(i) for i in ids[:8]],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
