"""The benchmark's own model at full depth against the oracle.

The 4B-class TQ1_0 model of the headline benchmark (36 layers, d_model 2560,
32/8 heads x 128, ffn 9728, vocab 151936), every layer's K and V cache
pre-filled with 2048 rows of f16 N(0,1) values on both sides: the first
step's logits bit-identical to the oracle's, then 64 greedy steps through
the captured-graph decode with the oracle's ids (north star: identical
greedy sequences over 64 steps; src/forward.c:295-438, src/sample.c:147-153).
"""
import os

import numpy as np
import pytest

import rustfox_amd as rf
from rustfox_amd import synth

pytestmark = pytest.mark.gpu

PREFILL = 2048
STEPS = 64
THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def kv_rows(spec, layer):
    rng = np.random.default_rng([11, 0xCAC4E, layer])
    kvd = spec.n_head_kv * spec.head_dim
    k = rng.standard_normal((PREFILL, kvd), dtype=np.float32).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((PREFILL, kvd), dtype=np.float32).astype(np.float16).astype(np.float32)
    return k, v


def test_4b_full_depth_64_greedy_steps(tmp_path, oracle):
    spec = synth.spec("4b", n_ctx=PREFILL + STEPS + 16)
    path = str(tmp_path / "4b.gguf")
    print("case full-depth 4b: writing the 36-layer GGUF", flush=True)
    synth.write_gguf(path, spec)
    kv = [kv_rows(spec, l) for l in range(spec.n_layer)]

    print(f"case full-depth 4b: oracle, {STEPS} steps on {THREADS} threads", flush=True)
    octx = oracle.model(spec, synth.map_tensors(path, spec)).context(
        spec.n_ctx, n_batch=8, n_threads=THREADS)
    for l, (k, v) in enumerate(kv):
        octx.set_kv(l, 0, k, v)
    octx.set_pos(PREFILL)
    want_ids, tok, first = [], 1, None
    for _ in range(STEPS):
        lg = octx.eval(np.array([tok], np.uint32))
        if first is None:
            first = lg.copy()
        tok = int(np.argmax(lg))
        want_ids.append(tok)
    octx.close()

    print("case full-depth 4b: device", flush=True)
    with rf.Model(path) as m:
        ctx = m.context(spec.n_ctx, n_batch=8)
        for l, (k, v) in enumerate(kv):
            ctx.set_kv(l, 0, k, v)
        ctx.set_position(PREFILL)
        got = ctx.eval([1])
        ctx.set_position(PREFILL)
        ids = [int(i) for i in ctx.decode_greedy(1, STEPS)]
        ctx.close()
    d = np.flatnonzero(got.view(np.uint32) != first.view(np.uint32))
    assert d.size == 0, f"{d.size} first-step logits differ, first at {d[:4]}"
    diff = [i for i in range(STEPS) if ids[i] != want_ids[i]]
    assert not diff, f"greedy ids differ from step {diff[0]}: {ids[diff[0]]} != {want_ids[diff[0]]}"
