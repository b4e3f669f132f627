"""End-to-end decode at the benchmark models' own dimensions, against the
oracle (bit-identical logits at every step, identical greedy ids).

Each model keeps every dimension of its benchmark configuration but has two
layers instead of 36, 32 or 62 (the layers are identical in shape, so two
exercise every kernel at its benchmark size, including a layer's input
arriving from the previous layer):

  4B-class   d_model 2560, 32/8 heads x 128, ffn 9728, vocab 151936, RoPE
             base 1e6, TQ1_0 linear weights, f16 embedding and output;
             2048 cached positions;
  8B-class   d_model 4096, 32/8 x 128, ffn 14336, vocab 128256, Q4_K
             attn_q/k/o, ffn_gate/up, Q6_K attn_v, ffn_down and output;
             4096 cached positions;
  27B-class  d_model 5376, 32/16 x 128, ffn 21504, vocab 262144, TQ1_0;
             8192 cached positions, then an 8-token verify pass.

The caches are pre-filled with the same f16 N(0,1) rows on both sides
(fox_context_set_kv and the oracle's or_context_set_kv).  Greedy decoding
runs 8 steps through fox_eval (logits compared every step) and again
through fox_decode_greedy (the captured-graph loop, ids compared).  The
4B-class model also decodes with the fused GEMVs' persistent grid capped
to 3 workgroups (FOX_MAX_WORKGROUPS), where every workgroup walks
hundreds of row tiles.
"""
import os

import numpy as np
import pytest

import rustfox_amd as rf
from rustfox_amd import synth

pytestmark = pytest.mark.gpu

STEPS = 8
THREADS = max(1, min(16, len(os.sched_getaffinity(0))))
MODELS = {"4b": 2048, "8b": 4096, "27b": 8192}


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def prefill(n_layer, n, kvd, seed):
    rng = np.random.default_rng([seed, 0xCAC4E])
    return [(rng.standard_normal((n, kvd), dtype=np.float32).astype(np.float16).astype(np.float32),
             rng.standard_normal((n, kvd), dtype=np.float32).astype(np.float16).astype(np.float32))
            for _ in range(n_layer)]


def load_kv(ctx, kv, setter, pos_setter):
    for layer, (k, v) in enumerate(kv):
        setter(ctx, layer, k, v)
    pos_setter(ctx, kv[0][0].shape[0])


def device_steps(path, n_ctx, kv, tok, steps, want=None, env=None):
    """Logits of `steps` single-token evals (greedy inputs from `want` when
    given, else from the device's own argmax) and the greedy ids of
    fox_decode_greedy from the same start."""
    old = {}
    for k, v in (env or {}).items():
        old[k] = os.environ.get(k)
        os.environ[k] = v
    try:
        with rf.Model(path) as m:
            ctx = m.context(n_ctx, n_batch=8)
            load_kv(ctx, kv, lambda c, l, k, v: c.set_kv(l, 0, k, v),
                    lambda c, p: c.set_position(p))
            logits, t = [], tok
            for s in range(steps):
                lg = ctx.eval([t])
                logits.append(lg)
                t = int(np.argmax(lg)) if want is None else int(want[s])
            ctx.close()
            g = m.context(n_ctx, n_batch=8)
            load_kv(g, kv, lambda c, l, k, v: c.set_kv(l, 0, k, v),
                    lambda c, p: c.set_position(p))
            ids = g.decode_greedy(tok, steps)
            g.close()
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    return logits, ids


@pytest.mark.parametrize("name", list(MODELS))
def test_benchmark_dims_decode_bit_identical(tmp_path, oracle, name):
    pre = MODELS[name]
    s = synth.spec(name, n_layer=2, n_ctx=pre + 64)
    path = str(tmp_path / f"{name}.gguf")
    tensors = {}
    print(f"case model {name}: writing the 2-layer GGUF", flush=True)
    synth.write_gguf(path, s, tensors=tensors)
    kvd = s.n_head_kv * s.head_dim
    kv = prefill(s.n_layer, pre, kvd, 11)
    n_ctx = pre + 2 * STEPS + 16

    print(f"case model {name}: oracle, {STEPS} steps after {pre} cached rows", flush=True)
    octx = oracle.model(s, tensors).context(n_ctx, n_batch=8, n_threads=THREADS)
    load_kv(octx, kv, lambda c, l, k, v: c.set_kv(l, 0, k, v), lambda c, p: c.set_pos(p))
    want, ids, tok = [], [], 1
    for _ in range(STEPS):
        lg = octx.eval(np.array([tok], np.uint32))
        want.append(lg)
        tok = int(np.argmax(lg))
        ids.append(tok)

    print(f"case model {name}: device", flush=True)
    got, gids = device_steps(path, n_ctx, kv, 1, STEPS, want=ids)
    for step, (g, w) in enumerate(zip(got, want)):
        d = np.flatnonzero(bits(g) != bits(w))
        assert d.size == 0, (f"{name} step {step}: {d.size} logits differ, first {d[:4]} "
                             f"got {g[d[:4]]} want {w[d[:4]]}")
    assert list(gids) == ids, f"{name}: graph greedy ids {list(gids)} != oracle {ids}"

    if name == "4b":
        print(f"case model {name}: device, grid capped to 3 workgroups", flush=True)
        got3, gids3 = device_steps(path, n_ctx, kv, 1, STEPS, want=ids,
                                   env={"FOX_MAX_WORKGROUPS": "3"})
        for step, (g, w) in enumerate(zip(got3, want)):
            assert np.array_equal(bits(g), bits(w)), f"capped grid, step {step}"
        assert list(gids3) == ids

    if name == "27b":
        # the 8-token verify pass: fox_eval over 8 drafted tokens at once
        # gives the last position's logits of the stepped evaluation
        print(f"case model {name}: 8-token pass", flush=True)
        draft = np.array([1] + ids[:7], np.uint32)
        with rf.Model(path) as m:
            ctx = m.context(n_ctx, n_batch=8)
            load_kv(ctx, kv, lambda c, l, k, v: c.set_kv(l, 0, k, v),
                    lambda c, p: c.set_position(p))
            rows = ctx.eval_all(draft)
            ctx.close()
        for i in range(8):
            assert np.array_equal(bits(rows[i]), bits(want[i])), f"verify row {i}"
    octx.close()
