"""The streaming weight backend (FOX_WEIGHTS_STREAM): layers go through a
ring of HBM slots, reloaded from the file through pinned host memory on a
copy stream, one layer ahead of the compute stream.

tests/test_forward.c:277-300 on the device: the same model opened with a
budget far below its size (two layer slots besides the tensors outside the
layers) gives bit-identical logits to the HBM-resident backend, and the
budget was tight enough that layers really were evicted and re-read.  Also
the lease contract in streaming mode and the budget's lower limit.
"""
import ctypes as C

import numpy as np
import pytest

import rustfox_amd as rf
from rustfox_amd import synth

pytestmark = pytest.mark.gpu


def split_bytes(s):
    """(GGUF bytes of one layer, bytes of the tensors outside the layers)."""
    layer = outside = 0
    for name, ne0, ne1, gt in synth.tensor_list(s):
        b = max(ne1, 1) * synth.row_bytes(gt, ne0)
        if name.startswith("blk.0."):
            layer += b
        elif not name.startswith("blk."):
            outside += b
    return layer, outside


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("stream")
    out = {}
    for name in ("tiny-512", "tiny-288"):
        s = synth.spec(name)
        p = str(d / f"{name}.gguf")
        synth.write_gguf(p, s)
        out[name] = (s, p)
    return out


def run(path, mode, budget, prompt, steps):
    with rf.Model(path, mode=mode, budget=budget) as m:
        ctx = m.context(96, n_batch=8)
        lg = ctx.eval(prompt)
        logits = [lg]
        for _ in range(steps):
            lg = ctx.eval([int(np.argmax(lg))])
            logits.append(lg)
        w = m.weights()
        reads = m.lib.fox_weights_reads(w)
        ev = m.lib.fox_weights_evictions(w)
        ctx.close()
        g = m.context(96, n_batch=8)
        g.eval(prompt)
        ids = g.decode_greedy(int(np.argmax(logits[0])), steps)
        g.close()
    return logits, ids, reads, ev


@pytest.mark.parametrize("name", ["tiny-512", "tiny-288"])
def test_streamed_equals_resident(models, name):
    s, p = models[name]
    layer, outside = split_bytes(s)
    prompt = synth.prompt_ids(16, s.n_vocab)
    print(f"case stream {name}: layer {layer} B, outside {outside} B", flush=True)
    want, want_ids, _, _ = run(p, rf.WEIGHTS_DEVICE, 0, prompt, 6)
    got, ids, reads, ev = run(p, rf.WEIGHTS_STREAM, outside + 2 * layer, prompt, 6)
    for k, (g, w) in enumerate(zip(got, want)):
        assert np.array_equal(bits(g), bits(w)), f"step {k}: streamed logits differ"
    assert list(ids) == list(want_ids)
    n_tensors = len(synth.tensor_list(s))
    assert ev > 0, "the budget should have forced layer slots to be reloaded"
    assert reads > n_tensors, "evicted layers are read again from the file"
    # a budget of three slots, and no budget (every layer keeps a slot)
    got3, _, _, _ = run(p, rf.WEIGHTS_STREAM, outside + 3 * layer, prompt, 2)
    got0, _, reads0, ev0 = run(p, rf.WEIGHTS_STREAM, 0, prompt, 2)
    for a, b, w in zip(got3, got0, want):
        assert np.array_equal(bits(a), bits(w)) and np.array_equal(bits(b), bits(w))
    assert ev0 == 0 and reads0 == n_tensors


@pytest.mark.parametrize("name", ["4b", "8b"])
def test_streamed_equals_resident_at_benchmark_dims(tmp_path, name):
    """Three layers of the benchmark models at their own dimensions: a 4B
    TQ1_0 layer (21 MB) and an 8B Q4_K/Q6_K layer (123 MB) are read by
    several reader threads over byte ranges that cross tensor boundaries,
    and the 8B layers are repacked from the staging buffer as Q4_K and Q6_K
    blocks.  Logits and greedy ids equal the resident backend's, with a
    budget of two layer slots that forces evictions."""
    s = synth.spec(name, n_layer=3, n_ctx=128)
    p = str(tmp_path / f"{name}.gguf")
    print(f"case stream {name}: writing the 3-layer GGUF", flush=True)
    synth.write_gguf(p, s)
    layer, outside = split_bytes(s)
    prompt = synth.prompt_ids(16, s.n_vocab)
    print(f"case stream {name}: layer {layer} B, outside {outside} B", flush=True)
    want, want_ids, _, _ = run(p, rf.WEIGHTS_DEVICE, 0, prompt, 4)
    got, ids, reads, ev = run(p, rf.WEIGHTS_STREAM, outside + 2 * layer, prompt, 4)
    for k, (g, w) in enumerate(zip(got, want)):
        assert np.array_equal(bits(g), bits(w)), f"{name} step {k}: streamed logits differ"
    assert list(ids) == list(want_ids)
    assert ev > 0 and reads > len(synth.tensor_list(s))


def test_stream_budget_and_leases(models):
    s, p = models["tiny-512"]
    layer, outside = split_bytes(s)
    with pytest.raises(rf.FoxError) as e:
        rf.Model(p, mode=rf.WEIGHTS_STREAM, budget=outside + 2 * layer - 1)
    assert e.value.status == 3                     # FOX_ERR_NOMEM: below two slots
    L = rf.host_lib()
    w = C.c_void_p()
    assert L.fox_weights_open(p.encode(), rf.WEIGHTS_STREAM, outside + 2 * layer,
                              C.byref(w)) == 0
    assert L.fox_weights_get_mode(w) == rf.WEIGHTS_STREAM
    q0 = L.fox_weights_tensor_find(w, b"blk.0.attn_q.weight")
    q3 = L.fox_weights_tensor_find(w, b"blk.3.attn_q.weight")
    k3 = L.fox_weights_tensor_find(w, b"blk.3.attn_k.weight")
    emb = L.fox_weights_tensor_find(w, b"token_embd.weight")
    lease = [rf.Lease() for _ in range(9)]
    assert L.fox_weights_acquire(w, q0, C.byref(lease[0])) == 0 and lease[0].data
    assert lease[0].bytes == synth.row_bytes(synth.TQ1_0, s.n_embd) * s.n_head * s.head_dim
    assert L.fox_weights_acquire(w, q3, C.byref(lease[1])) == 0
    # both slots are held by leases: a third layer has nowhere to go
    l5 = L.fox_weights_tensor_find(w, b"blk.5.ffn_up.weight")
    assert L.fox_weights_acquire(w, l5, C.byref(lease[2])) == 3
    assert L.fox_weights_acquire(w, k3, C.byref(lease[2])) == 0   # same slot as q3
    for k in range(3, 8):
        assert L.fox_weights_acquire(w, emb, C.byref(lease[k])) == 0
    assert L.fox_weights_acquire(w, emb, C.byref(lease[8])) == 7  # ninth live lease
    for k in range(8):
        L.fox_weights_release(w, C.byref(lease[k]))
        assert not lease[k].data
    assert L.fox_weights_live_leases(w) == 0
    # asynchronous prefetch of a layer, then its wait
    assert L.fox_weights_prefetch_async(w, l5) == 0
    assert L.fox_weights_prefetch_wait(w, l5) == 0
    assert L.fox_weights_prefetch_async(w, emb) == 5              # resident: nothing to start
    assert L.fox_weights_evictions(w) > 0
    L.fox_weights_close(w)
