"""End-to-end decode on the GPU through the RustFox host API (libfox.so).

Checked against the reference compiled from its own sources (oracle/_ref)
when it is present, else against the oracle (whose forward pass equals the
reference's bit for bit, tests/test_oracle.py).  With exact attention (the
default) logits must be bit-identical to the oracle's (the 1e-3 relative L2
bound is met with zero error); split (flash-decoding) attention is checked
only against gross error.  Greedy token sequences
must be identical over 64 steps; batched == stepped and decode_greedy ==
eval + argmax exactly on the device.
"""
import os
import struct

import numpy as np
import pytest

import rustfox_amd as rf
from rustfox_amd import synth

pytestmark = pytest.mark.gpu

REL_L2 = 1e-3
# Split attention reorders the attention sums (within 1e-5 of the reference
# order per call, tests/test_gpu_attention.py); a last-bit difference can
# flip an int8 activation rounding downstream, and through six random
# ternary layers that moves logits by 1e-3 to 2e-2.  It is not
# parity-certified: the bound here only catches a broken path (which is off
# by ~1), and greedy ids are not required to match.
SPLIT_REL_L2 = 1e-1


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def oracle_run(oracle, spec, tensors, path, prompt, steps, n_ctx, kv=None):
    """Prompt logits and greedy ids from the CPU oracle."""
    from oracle_libs import Ref, ref_available
    if ref_available() and kv is None:
        r = Ref()
        m = r.open_model(path)
        ctx = m.context(n_ctx, n_batch=32, n_threads=0)
        first = ctx.eval(prompt)
        ids, lg = [], first
        for _ in range(steps):
            t = int(np.argmax(lg))
            ids.append(t)
            lg = ctx.eval(np.array([t], np.uint32))
        ctx.close()
        m.close()
        return first, np.array(ids, np.uint32)
    om = oracle.model(spec, tensors)
    ctx = om.context(n_ctx, n_threads=8)
    if kv is not None:
        for l, (k, v) in enumerate(kv):
            ctx.set_kv(l, 0, k, v)
        ctx.set_pos(kv[0][0].shape[0])
    first = ctx.eval(prompt)
    ids, lg = [], first
    for _ in range(steps):
        t = int(np.argmax(lg))
        ids.append(t)
        lg = ctx.eval(np.array([t], np.uint32))
    ctx.close()
    return first, np.array(ids, np.uint32)


@pytest.fixture(scope="module")
def tiny_models(tmp_path_factory):
    d = tmp_path_factory.mktemp("models")
    out = {}
    for name in ("tiny-512", "tiny-288"):
        s = synth.spec(name)
        t = {}
        p = str(d / f"{name}.gguf")
        synth.write_gguf(p, s, tensors=t)
        out[name] = (s, t, p)
    return out


@pytest.mark.parametrize("mode", ["exact", "split"])
@pytest.mark.parametrize("name", ["tiny-512", "tiny-288"])
def test_tiny_model_greedy_64(tiny_models, oracle, name, mode):
    """Config 0 variants: 16 seeded prompt ids, then 64 greedy steps
    (repeat penalty 1.0).  tiny-288 keeps d_model 288 with F16 where K is
    not a multiple of 256 and TQ1_0 for ffn_down; tiny-512 is all TQ1_0."""
    s, t, p = tiny_models[name]
    print(f"case greedy64 {name} {mode}", flush=True)
    prompt = synth.prompt_ids(16, s.n_vocab)
    want_first, want_ids = oracle_run(oracle, s, t, p, prompt, 64, 96)
    with rf.Model(p) as m:
        ctx = m.context(96)
        ctx.set_attention(mode == "exact")
        first = ctx.eval(prompt)
        err = rel_l2(first, want_first)
        if mode == "exact":
            assert np.array_equal(first.view(np.uint32), want_first.view(np.uint32)), \
                f"exact mode: prompt logits differ (rel L2 {err:.2e})"
        else:
            assert err < SPLIT_REL_L2, f"split mode: prompt logits rel L2 {err:.2e}"
            ctx.close()
            return
        ids = ctx.decode_greedy(int(np.argmax(first)), 63)
        got = np.concatenate([[np.argmax(first)], ids]).astype(np.uint32)
        ctx.close()
    if not np.array_equal(got, want_ids):
        k = int(np.flatnonzero(got != want_ids)[0])
        pytest.fail(f"{mode}: greedy ids diverge at step {k}: {got[k]} vs {want_ids[k]}")


def test_batched_equals_stepped(tiny_models):
    """tests/test_forward.c:258-272 on the device: a 5-token batch gives
    bit-identical logits to five single-token evals."""
    s, t, p = tiny_models["tiny-512"]
    prompt = np.array([1, 4, 9, 2, 7], np.uint32)
    with rf.Model(p) as m:
        ctx = m.context(64, n_batch=8)
        batched = ctx.eval(prompt)
        assert ctx.position == 5
        ctx.reset()
        for tok in prompt:
            stepped = ctx.eval([tok])
        ctx.close()
    assert np.array_equal(batched.view(np.uint32), stepped.view(np.uint32))


def test_eval_all_equals_stepped(tiny_models):
    """fox_eval_all over 7 tokens in chunks of 3 (3, 3, 1): row i is
    bit-identical to the logits of a single-token eval after tokens 0..i
    (each position's norm and head product are independent of the batch)."""
    s, t, p = tiny_models["tiny-512"]
    prompt = np.array([3, 1, 4, 1, 5, 9, 2], np.uint32)
    with rf.Model(p) as m:
        ctx = m.context(64, n_batch=3)
        rows = ctx.eval_all(prompt)
        assert ctx.position == 7 and rows.shape == (7, m.info.n_vocab)
        ctx.reset()
        stepped = np.stack([ctx.eval([tok]) for tok in prompt])
        ctx.close()
    assert np.array_equal(rows.view(np.uint32), stepped.view(np.uint32))


def test_decode_greedy_equals_eval_argmax(tiny_models):
    """The captured-graph greedy loop is the same computation as eval +
    first argmax on the host (src/sample.c:147-153)."""
    s, t, p = tiny_models["tiny-288"]
    prompt = synth.prompt_ids(8, s.n_vocab, seed=3)
    with rf.Model(p) as m:
        a = m.context(64)
        lg = a.eval(prompt)
        want = []
        for _ in range(20):
            tok = int(np.argmax(lg))
            want.append(tok)
            lg = a.eval([tok])
        b = m.context(64)
        lg = b.eval(prompt)
        got = b.decode_greedy(int(np.argmax(lg)), 19)
        assert b.position == 8 + 19
        a.close()
        b.close()
    assert [want[0]] + list(got) == want


@pytest.mark.parametrize("mode", ["exact", "split"])
def test_prefilled_cache_decode(tmp_path, oracle, mode):
    """A pre-filled cache (f16 N(0,1) values, as in the 4B benchmark) then
    decode steps: logits equal to the oracle's (exact attention) or within
    tolerance (split attention) at every step."""
    s = synth.spec("tiny-512", n_layer=2, n_vocab=2000, n_head=8, n_head_kv=2)
    t = {}
    p = str(tmp_path / "kv.gguf")
    synth.write_gguf(p, s, tensors=t)
    n_pre, kvd = 300, s.n_head_kv * s.head_dim
    rng = np.random.default_rng(5)
    kv = [(rng.standard_normal((n_pre, kvd)).astype(np.float16).astype(np.float32),
           rng.standard_normal((n_pre, kvd)).astype(np.float16).astype(np.float32))
          for _ in range(s.n_layer)]
    om = oracle.model(s, t)
    octx = om.context(320, n_threads=8)
    for l, (k, v) in enumerate(kv):
        octx.set_kv(l, 0, k, v)
    octx.set_pos(n_pre)
    with rf.Model(p) as m:
        ctx = m.context(320)
        ctx.set_attention(mode == "exact")
        for l, (k, v) in enumerate(kv):
            ctx.set_kv(l, 0, k, v)
        ctx.set_position(n_pre)
        tok = 17
        for step in range(6):
            want = octx.eval(np.array([tok], np.uint32))
            got = ctx.eval([tok])
            err = rel_l2(got, want)
            if mode == "exact":
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
                    f"step {step}: exact logits differ (rel L2 {err:.2e})"
            else:
                assert err < SPLIT_REL_L2, f"step {step}: rel L2 {err:.2e}"
            tok = int(np.argmax(want))
        ctx.close()
    octx.close()


def _write_reference_forward_fixture(path):
    """The 2-layer all-F32 llama of tests/test_forward.c:91-186 (d 8, 2 heads,
    1 kv head, ff 16, vocab 16, context 64), values
    ((t*31 + i*17 + 7) mod 23 - 11) * 0.03 for tensor t, element i."""
    names = [("token_embd.weight", 8, 16), ("output_norm.weight", 8, 0),
             ("output.weight", 8, 16)]
    for l in range(2):
        names += [(f"blk.{l}.attn_norm.weight", 8, 0), (f"blk.{l}.attn_q.weight", 8, 8),
                  (f"blk.{l}.attn_k.weight", 8, 4), (f"blk.{l}.attn_v.weight", 8, 4),
                  (f"blk.{l}.attn_output.weight", 8, 8), (f"blk.{l}.ffn_norm.weight", 8, 0),
                  (f"blk.{l}.ffn_gate.weight", 8, 16), (f"blk.{l}.ffn_up.weight", 8, 16),
                  (f"blk.{l}.ffn_down.weight", 16, 8)]

    def kv_u32(k, v):
        return struct.pack("<Q", len(k)) + k.encode() + struct.pack("<II", 4, v)

    def kv_f32(k, v):
        return struct.pack("<Q", len(k)) + k.encode() + struct.pack("<If", 6, v)

    meta = [kv_u32("general.alignment", 32),
            struct.pack("<Q", 20) + b"general.architecture" + struct.pack("<IQ", 8, 5) + b"llama",
            kv_u32("llama.block_count", 2), kv_u32("llama.embedding_length", 8),
            kv_u32("llama.attention.head_count", 2), kv_u32("llama.attention.head_count_kv", 1),
            kv_u32("llama.feed_forward_length", 16), kv_u32("llama.context_length", 64),
            kv_f32("llama.attention.layer_norm_rms_epsilon", 1e-5),
            kv_f32("llama.rope.freq_base", 10000.0)]
    infos, datas, off = [], [], 0
    for ti, (n, a, b) in enumerate(names):
        count = a * (b or 1)
        off = (off + 31) // 32 * 32
        dims = [a] if b == 0 else [a, b]
        infos.append(struct.pack("<Q", len(n)) + n.encode() + struct.pack("<I", len(dims))
                     + b"".join(struct.pack("<Q", x) for x in dims) + struct.pack("<IQ", 0, off))
        i = np.arange(count, dtype=np.uint64)
        vals = (((ti * 31 + i * 17 + 7) % 23).astype(np.int64) - 11).astype(np.float32) * np.float32(0.03)
        datas.append((off, vals.astype(np.float32).tobytes()))
        off += count * 4
    head = b"GGUF" + struct.pack("<IQQ", 3, len(names), len(meta)) + b"".join(meta) + b"".join(infos)
    head += b"\0" * ((-len(head)) % 32)
    with open(path, "wb") as f:
        f.write(head)
        pos = 0
        for o, d in datas:
            f.write(b"\0" * (o - pos))
            f.write(d)
            pos = o + len(d)


def test_reference_forward_fixture(tmp_path):
    """tests/test_forward.c:198-272 on the device: metadata, finiteness,
    distinct logits, batched == stepped; logits within tolerance of the
    reference when oracle/_ref is present."""
    p = str(tmp_path / "rustfox-forward.gguf")
    _write_reference_forward_fixture(p)
    prompt = np.array([1, 4, 9, 2, 7], np.uint32)
    with rf.Model(p) as m:
        i = m.info
        assert (i.n_layer, i.n_embd, i.n_head, i.n_head_kv, i.n_ff) == (2, 8, 2, 1, 16)
        assert i.head_dim == 4 and i.n_vocab == 16 and i.tied_output == 0
        ctx = m.context(32, n_batch=8)
        batched = ctx.eval(prompt)
        assert np.all(np.isfinite(batched)) and len(set(batched.tolist())) > 1
        ctx.reset()
        for tok in prompt:
            stepped = ctx.eval([tok])
        assert np.array_equal(batched.view(np.uint32), stepped.view(np.uint32))
        ctx.close()
    from oracle_libs import Ref, ref_available
    if ref_available():
        r = Ref()
        rm = r.open_model(p)
        rc = rm.context(32, n_batch=8, n_threads=2)
        want = rc.eval(prompt)
        assert np.array_equal(batched.view(np.uint32), want.view(np.uint32))


def test_model_and_weights_contract(tiny_models, tmp_path):
    s, t, p = tiny_models["tiny-288"]
    with pytest.raises(rf.FoxError) as e:
        rf.Model(str(tmp_path / "missing.gguf"))
    assert e.value.status == 2                       # FOX_ERR_IO
    with rf.Model(p, mode=rf.WEIGHTS_RESIDENT) as m:
        with pytest.raises(rf.FoxError) as e:
            m.context(32)
        assert e.value.status == 5                   # compute needs DEVICE
    L = rf.host_lib()
    import ctypes as C
    w = C.c_void_p()
    assert L.fox_weights_open(p.encode(), rf.WEIGHTS_DEVICE, 0, C.byref(w)) == 0
    n = L.fox_weights_tensor_count(w)
    leases = [rf.Lease() for _ in range(9)]
    for k in range(8):
        assert L.fox_weights_acquire(w, k, C.byref(leases[k])) == 0
        assert leases[k].data
    assert L.fox_weights_acquire(w, 8, C.byref(leases[8])) == 7   # 9th live lease
    assert L.fox_weights_live_leases(w) == 8
    for k in range(8):
        L.fox_weights_release(w, C.byref(leases[k]))
        assert not leases[k].data
    for k in range(n):
        assert L.fox_weights_prefetch(w, k) == 0
    assert L.fox_weights_reads(w) == n               # one read per tensor
    assert L.fox_weights_resident_bytes(w) == synth.gguf_bytes(s)
    assert L.fox_weights_prefetch_async(w, 0) == 5
    L.fox_weights_close(w)
