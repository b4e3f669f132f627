"""The C ABI on the CPU: both libraries load, export every function that
include/fox_gpu.h and include/fox_host.h declare, refuse to run without a GPU
(no CPU fallback), and the host side keeps RustFox's file and lease contracts
(tests/test_gguf.c, tests/test_weights.c) in the host-memory mode.
"""
import ctypes as C
import os
import re
import struct
import subprocess

import numpy as np
import pytest

import rustfox_amd as rf
from rustfox_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fox_\w+)\s*\(", text)))


def exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


@pytest.mark.parametrize("header,lib", [("fox_gpu.h", rf.GPU_LIB), ("fox_host.h", rf.HOST_LIB)])
def test_every_declared_symbol_is_exported(header, lib):
    missing = [s for s in declared(header) if s not in exported(lib)]
    assert not missing, f"{os.path.basename(lib)} lacks {missing}"


def test_host_library_exports_only_the_api():
    api = set(declared("fox_host.h"))
    extra = [s for s in exported(rf.HOST_LIB) if s.startswith("fox_") and s not in api]
    assert not extra, f"internal symbols leak from libfox.so: {extra}"


def test_no_gpu_means_an_error_not_a_fallback():
    if os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK):
        pytest.skip("a GPU is visible here")
    L = rf.gpu_lib()
    ctx = C.c_void_p()
    st = L.fox_gpu_init(0, C.byref(ctx))
    assert st != 0 and not ctx.value
    assert b"device" in L.fox_gpu_last_error()


def test_ggml_tables():
    L = rf.host_lib()
    assert L.fox_row_bytes(34, 512) == 108 and L.fox_row_bytes(35, 512) == 132
    assert L.fox_row_bytes(12, 512) == 288 and L.fox_row_bytes(14, 256) == 210
    assert L.fox_row_bytes(34, 255) == 0
    for t in (0, 1, 12, 14, 34, 35):
        assert L.fox_gemv_supports(t)
    for t in (2, 8, 10, 13):      # types without a device kernel
        assert not L.fox_gemv_supports(t)


def _tiny(tmp_path, **over):
    s = synth.spec("tiny-288", n_layer=1, n_vocab=64, **over)
    p = str(tmp_path / "m.gguf")
    t = {}
    synth.write_gguf(p, s, tensors=t)
    return s, t, p


def test_gguf_rejections(tmp_path):
    """Truncation, bad magic and a bad version are refused with
    FOX_ERR_FORMAT / FOX_ERR_UNSUPPORTED (src/gguf.c:384-403)."""
    s, t, p = _tiny(tmp_path)
    data = open(p, "rb").read()
    bad = str(tmp_path / "bad.gguf")
    for blob, want in [(data[: len(data) // 2], 4), (b"GGUX" + data[4:], 4),
                       (data[:4] + struct.pack("<I", 9) + data[8:], 5)]:
        open(bad, "wb").write(blob)
        with pytest.raises(rf.FoxError) as e:
            rf.Model(bad, mode=rf.WEIGHTS_RESIDENT)
        assert e.value.status == want
    with pytest.raises(rf.FoxError) as e:
        rf.Model(str(tmp_path / "missing.gguf"), mode=rf.WEIGHTS_RESIDENT)
    assert e.value.status == 2


def test_model_metadata_and_defaults(tmp_path):
    s, t, p = _tiny(tmp_path)
    with rf.Model(p, mode=rf.WEIGHTS_RESIDENT) as m:
        i = m.info
        assert (i.n_layer, i.n_embd, i.n_head, i.n_head_kv, i.head_dim, i.n_ff, i.n_vocab) == \
            (1, 288, 6, 6, 48, 768, 64)
        assert i.arch == b"llama" and i.tied_output == 0
        assert i.weight_bytes == synth.gguf_bytes(s)
        with pytest.raises(rf.FoxError) as e:     # compute is on the GPU only
            m.context(16)
        assert e.value.status == 5


def test_resident_lease_contract(tmp_path):
    """tests/test_weights.c: bytes equal the file, one read per tensor, at most
    8 live leases, release clears the lease, no prefetch thread."""
    s, t, p = _tiny(tmp_path)
    L = rf.host_lib()
    w = C.c_void_p()
    assert L.fox_weights_open(p.encode(), rf.WEIGHTS_RESIDENT, 0, C.byref(w)) == 0
    n = L.fox_weights_tensor_count(w)
    names = [name for name, _, _, _ in synth.tensor_list(s)]
    leases = [rf.Lease() for _ in range(9)]
    for k in range(8):
        idx = L.fox_weights_tensor_find(w, names[k].encode())
        assert L.fox_weights_acquire(w, idx, C.byref(leases[k])) == 0
        got = np.ctypeslib.as_array(C.cast(leases[k].data, C.POINTER(C.c_uint8)),
                                    shape=(leases[k].bytes,))
        assert np.array_equal(got, t[names[k]])
    assert L.fox_weights_acquire(w, 8, C.byref(leases[8])) == 7
    for k in range(8):
        L.fox_weights_release(w, C.byref(leases[k]))
        assert not leases[k].data and leases[k].bytes == 0
    for k in range(n):
        assert L.fox_weights_prefetch(w, k) == 0
        assert L.fox_weights_prefetch(w, k) == 0
    assert L.fox_weights_reads(w) == n
    assert L.fox_weights_resident_bytes(w) == synth.gguf_bytes(s)
    assert L.fox_weights_prefetch_async(w, 0) == 5 and L.fox_weights_prefetch_wait(w, 0) == 5
    assert L.fox_weights_prefetch(w, n) == 6
    L.fox_weights_close(w)


def test_budget_too_small(tmp_path):
    s, t, p = _tiny(tmp_path)
    L = rf.host_lib()
    w = C.c_void_p()
    assert L.fox_weights_open(p.encode(), rf.WEIGHTS_RESIDENT, 1000, C.byref(w)) == 0
    lease = rf.Lease()
    assert L.fox_weights_acquire(w, 0, C.byref(lease)) == 3      # FOX_ERR_NOMEM
    L.fox_weights_close(w)


def ref_greedy(logits, history, window, penalty):
    """src/sample.c:95-107, 135-153 restated: the penalty once per entry of
    the last `window` accepted ids, then the first maximum."""
    w = logits.astype(np.float32).copy()
    if penalty > 1.0:
        for t in history[-window:]:
            if t < w.size:
                w[t] = w[t] / np.float32(penalty) if w[t] > 0 else w[t] * np.float32(penalty)
    best = 0
    for i in range(1, w.size):
        if w[i] > w[best]:
            best = i
    return best


def test_sampler_semantics():
    """Greedy picks: the first maximum after the repeat penalty, applied once
    per occurrence in the window; stochastic sampling is refused."""
    logits = np.array([0.5, 2.0, 2.0, -1.0, 1.9], np.float32)
    g = rf.Sampler(5, temperature=0.0, repeat_penalty=1.0)
    assert g.pick(logits) == 1
    p = rf.Sampler(5, temperature=0.0, repeat_penalty=1.1)
    p.accept(1)
    p.accept(2)
    assert p.pick(logits) == 4        # 2.0 / 1.1 < 1.9
    s = rf.Sampler(5, temperature=0.8, top_k=3, seed=12345)
    with pytest.raises(rf.FoxError) as e:
        s.pick(logits)
    assert e.value.status == 5
    with pytest.raises(rf.FoxError):
        rf.Sampler(0, temperature=0.0)


@pytest.mark.parametrize("window,penalty", [(64, 1.1), (3, 1.3), (0, 1.5), (1, 0.9), (7, 2.0)])
def test_sampler_matches_the_reference_rule(window, penalty):
    """Random logits (with ties, zeros, negatives and a NaN) and random
    accepted ids, some repeated, some outside the vocabulary: every pick
    equals the reference rule, including the window of one id that
    repeat_last_n = 0 gives."""
    rng = np.random.default_rng([window, int(penalty * 10)])
    V = 50
    s = rf.Sampler(V, temperature=0.0, repeat_penalty=penalty, repeat_last_n=window)
    ref = None
    from oracle_libs import ref_available
    if ref_available():
        # the reference itself, compiled from its sources (oracle/_ref)
        from oracle_libs import REF_SO
        R = C.CDLL(REF_SO)
        R.fox_sampler_config_default.argtypes = [C.POINTER(rf.SamplerConfig)]
        R.fox_sampler_create.argtypes = [C.POINTER(rf.SamplerConfig), C.c_size_t]
        R.fox_sampler_create.restype = C.c_void_p
        R.fox_sampler_accept.argtypes = [C.c_void_p, C.c_uint32]
        R.fox_sampler_pick.argtypes = [C.c_void_p, C.c_void_p, C.POINTER(C.c_uint32)]
        R.fox_sampler_destroy.argtypes = [C.c_void_p]
        cfg = rf.SamplerConfig()
        R.fox_sampler_config_default(C.byref(cfg))
        cfg.temperature, cfg.repeat_penalty, cfg.repeat_last_n = 0.0, penalty, window
        ref = R.fox_sampler_create(C.byref(cfg), V)
    hist = []
    for step in range(300):
        lg = rng.integers(-4, 5, V).astype(np.float32) * np.float32(0.25)
        if step % 17 == 0:
            lg[rng.integers(0, V)] = np.nan
        want = ref_greedy(lg, hist, window or 1, penalty)
        got = s.pick(lg)
        assert got == want, step
        if ref:
            r = C.c_uint32()
            assert R.fox_sampler_pick(ref, lg.ctypes.data_as(C.c_void_p), C.byref(r)) == 0
            assert r.value == got, step
        t = int(rng.integers(0, V + 3)) if step % 5 else int(hist[-1]) if hist else 0
        s.accept(t)
        hist.append(t)
        if ref:
            R.fox_sampler_accept(ref, t)
    if ref:
        R.fox_sampler_destroy(ref)


def test_operator_entries_check_arguments_then_need_the_gpu():
    """The reference's operator entries (include/fox/fox.h:322-368) validate
    their arguments as tests/test_gemv.c:132-139 expects before touching a
    device, and without a GPU fail with a status and a message instead of
    computing on the CPU."""
    L = rf.host_lib()
    vp, sz = C.c_void_p, C.c_size_t
    L.fox_gemv_tq2_i8.argtypes = [vp, vp, C.c_float, vp, sz, sz, vp]
    L.fox_gemv_tq2_f32.argtypes = [vp, vp, vp, sz, sz, vp]
    L.fox_dequant_row.argtypes = [C.c_int, vp, sz, vp]
    q = np.zeros(512, np.int8)
    w = np.zeros(2 * 66 * 4, np.uint8)
    out = np.zeros(4, np.float32)
    P = lambda a: a.ctypes.data_as(vp)
    assert L.fox_gemv_tq2_i8(None, P(q), 1.0, P(w), 4, 255, P(out)) == 1
    assert L.fox_gemv_tq2_i8(None, None, 1.0, P(w), 4, 512, P(out)) == 1
    assert L.fox_gemv_tq2_i8(None, P(q), 1.0, None, 4, 512, P(out)) == 1
    assert L.fox_gemv_tq2_i8(None, P(q), 1.0, P(w), 0, 512, P(out)) == 1
    assert L.fox_dequant_row(34, P(w), 256, P(out)) == 5
    if os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK):
        return
    x = np.zeros(512, np.float32)
    st = L.fox_gemv_tq2_f32(None, P(x), P(w), 4, 512, P(out))
    assert st != 0 and L.fox_last_error()


@pytest.mark.parametrize("victim,cols,rows", [("blk.0.attn_k.weight", None, 64),
                                              ("blk.0.attn_output.weight", 256, None),
                                              ("blk.0.ffn_down.weight", None, 32),
                                              ("output.weight", 256, None),
                                              ("blk.0.ffn_norm.weight", 256, None)])
def test_model_open_rejects_mismatched_shapes(tmp_path, monkeypatch, victim, cols, rows):
    """A GGUF whose tensor shapes disagree with its metadata is refused with
    FOX_ERR_FORMAT at open (host mode: no device involved) instead of
    reaching kernels that size their reads and writes by the tensor."""
    s = synth.spec("tiny-512", n_layer=1, n_vocab=64)
    real = synth.tensor_list

    def bent(spec):
        out = []
        for name, ne0, ne1, gt in real(spec):
            if name == victim:
                ne0 = ne0 + cols if cols else ne0
                ne1 = ne1 + rows if rows else ne1
            out.append((name, ne0, ne1, gt))
        return out
    monkeypatch.setattr(synth, "tensor_list", bent)
    p = str(tmp_path / "bent.gguf")
    synth.write_gguf(p, s)
    monkeypatch.setattr(synth, "tensor_list", real)
    L = rf.host_lib()
    m = C.c_void_p()
    st = L.fox_model_open(p.encode(), rf.WEIGHTS_RESIDENT, 0, C.byref(m))
    assert st == 4, (st, L.fox_last_error())
    assert victim.encode() in L.fox_last_error()
    good = str(tmp_path / "good.gguf")
    synth.write_gguf(good, s)
    assert L.fox_model_open(good.encode(), rf.WEIGHTS_RESIDENT, 0, C.byref(m)) == 0
    L.fox_model_close(m)
