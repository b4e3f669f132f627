"""GPU parity of the quantised GEMVs against the oracle (bit-exact).

Per-block integer sums, int8 activations and GEMV outputs must equal the
oracle's (the reference's arithmetic, src/gemv.c, src/ternary.c,
src/kernels.c, without FMA contraction) bit for bit.
"""
import numpy as np
import pytest

import rustfox_amd as rf
from rustfox_amd import synth

pytestmark = pytest.mark.gpu

TYPES = {"TQ1_0": 34, "TQ2_0": 35, "Q4_K": 12, "Q6_K": 14, "F16": 1, "F32": 0}


def weights(rng, gtype, N, K, raw_bytes=True):
    """Weights of N rows x K columns.  Block types use arbitrary bytes (every
    byte value a decoder can meet) with a valid f16 scale, as the reference's
    own tests do (tests/test_ternary.c:138-144)."""
    if gtype == 34:
        w = rng.integers(0, 256, size=(N * K // 256, 54), dtype=np.uint8) if raw_bytes \
            else synth.tq1_random(rng, N * K // 256)
        w[:, 52:54] = rng.uniform(0.01, 0.05, size=w.shape[0]).astype(np.float16).view(
            np.uint8).reshape(-1, 2)
        return w.reshape(-1)
    if gtype == 35:
        w = rng.integers(0, 256, size=(N * K // 256, 66), dtype=np.uint8)
        w[:, 64:66] = rng.uniform(0.01, 0.05, size=w.shape[0]).astype(np.float16).view(
            np.uint8).reshape(-1, 2)
        return w.reshape(-1)
    if gtype == 12:
        return synth.q4k_quantize(rng.standard_normal((N, K)).astype(np.float32) * 0.02).reshape(-1)
    if gtype == 14:
        return synth.q6k_quantize(rng.standard_normal((N, K)).astype(np.float32) * 0.02).reshape(-1)
    if gtype == 1:
        return (rng.standard_normal((N, K)) * 0.02).astype(np.float16).view(np.uint8).reshape(-1)
    return (rng.standard_normal((N, K)) * 0.02).astype(np.float32).view(np.uint8).reshape(-1)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def oracle_gemv(oracle, gtype, x, w, N, K):
    return np.stack([oracle.gemv(gtype, x[t], w, N, K) for t in range(x.shape[0])])


CASES = [
    # (type, N, K, M)
    ("TQ1_0", 16, 256, 1), ("TQ1_0", 37, 512, 1), ("TQ1_0", 100, 2560, 3),
    ("TQ1_0", 4096, 4096, 1), ("TQ1_0", 1024, 9728, 8), ("TQ1_0", 333, 768, 5),
    ("TQ2_0", 37, 512, 1), ("TQ2_0", 4096, 4096, 1), ("TQ2_0", 130, 1280, 8),
    ("TQ2_0", 200, 4096, 7), ("TQ1_0", 48, 1024, 2), ("TQ2_0", 40, 5376, 6),
    ("Q4_K", 33, 768, 1), ("Q4_K", 512, 4096, 2), ("Q4_K", 64, 2048, 8),
    ("Q6_K", 29, 512, 1), ("Q6_K", 300, 4096, 3), ("Q6_K", 48, 1024, 8),
    ("F16", 50, 288, 1), ("F16", 1000, 2560, 2), ("F16", 7, 8, 1), ("F16", 257, 1000, 8),
    ("F32", 9, 64, 1), ("F32", 300, 288, 4),
    ("TQ1_0", 64, 2048, 6), ("TQ2_0", 96, 512, 7),      # input groups of four, then two or three
    ("TQ1_0", 4096, 4096, 8), ("TQ2_0", 4096, 4096, 8),  # the 4096 x 4096 microbench, 8 stacked x
]


@pytest.mark.parametrize("tname,N,K,M", CASES)
def test_gemv_bit_exact(gpu, oracle, tname, N, K, M):
    print(f"case gemv {tname} N={N} K={K} M={M}", flush=True)
    gtype = TYPES[tname]
    rng = np.random.default_rng([N, K, M, gtype])
    w = weights(rng, gtype, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    want = oracle_gemv(oracle, gtype, x, w, N, K)
    t = gpu.tensor(gtype, K, N, w)
    dx = gpu.array(x)
    out = gpu.empty((M, N), np.float32)
    gpu.gemv(t, dx, M, out)
    got = out.numpy()
    mism = np.flatnonzero(bits(got) != bits(want))
    assert mism.size == 0, (f"{mism.size} of {got.size} outputs differ; first "
                            f"{mism[:5]} got {got.reshape(-1)[mism[:5]]} "
                            f"want {want.reshape(-1)[mism[:5]]}")


@pytest.mark.parametrize("tname,N,K,M", [c for c in CASES if c[0] in ("TQ1_0", "TQ2_0", "Q4_K", "Q6_K")])
def test_block_sums_exact(gpu, oracle, tname, N, K, M):
    print(f"case block_sums {tname} N={N} K={K} M={M}", flush=True)
    gtype = TYPES[tname]
    rng = np.random.default_rng([N, K, M, gtype, 1])
    w = weights(rng, gtype, N, K)
    q = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    per = {34: 1, 35: 1, 12: 8, 14: 4}[gtype]
    want = np.stack([oracle.block_sums(gtype, q[t], w, N, K).reshape(N, K // 256, per)
                     for t in range(M)])
    t = gpu.tensor(gtype, K, N, w)
    sums = gpu.empty((M, N, K // 256, per), np.int32)
    gpu.block_sums(t, gpu.array(q), M, sums)
    got = sums.numpy()
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} sums differ"


def test_tq1_closed_forms(gpu):
    """tests/test_ternary.c:100-136: byte 255 / qh 253 decode to all +1 and
    byte 0 to all -1, so with all-one activations and d = 1 a block sums to
    +256 / -256."""
    blk_p = np.zeros(54, np.uint8)
    blk_p[:48] = 255
    blk_p[48:52] = 253
    blk_p[52:54] = [0x00, 0x3C]
    blk_m = np.zeros(54, np.uint8)
    blk_m[52:54] = [0x00, 0x3C]
    w = np.concatenate([np.tile(blk_p, 3), np.tile(blk_m, 3)])
    t = gpu.tensor(34, 768, 2, w)
    q = gpu.array(np.ones((1, 768), np.int8))
    sums = gpu.empty((1, 2, 3, 1), np.int32)
    gpu.block_sums(t, q, 1, sums)
    assert np.array_equal(sums.numpy().reshape(2, 3), [[256] * 3, [-256] * 3])


def tq1_trits(w):
    """Trits (0..2, before the reference's - 1) of TQ1_0 blocks in element
    order: src/ternary.c:59-63 on the bytes and levels of 73-93."""
    b = w.reshape(-1, 54).astype(np.int64)
    cols = []
    for l in range(5):
        cols.append(b[:, 0:32] * 3 ** l)
    for l in range(5):
        cols.append(b[:, 32:48] * 3 ** l)
    for l in range(4):
        cols.append(b[:, 48:52] * 3 ** l)
    return ((np.concatenate(cols, axis=1) & 255) * 3) >> 8


def test_tq1_noncanonical_download(gpu):
    """TQ1_0 is held as 2-bit codes of its trits.  Bytes that are not the
    canonical encoding of their trits (every byte decodes) come back as the
    canonical byte, ceil(q * 256 / 243), of the same trits; scales exactly."""
    rng = np.random.default_rng(11)
    N, K = 24, 768
    w = weights(rng, 34, N, K)
    back = gpu.tensor(34, K, N, w).download()
    assert np.array_equal(tq1_trits(back), tq1_trits(w))
    t = tq1_trits(w)
    q = np.zeros((t.shape[0], 52), np.int64)
    for l in range(5):
        q[:, 0:32] = 3 * q[:, 0:32] + t[:, 32 * l: 32 * l + 32]
        q[:, 32:48] = 3 * q[:, 32:48] + t[:, 160 + 16 * l: 176 + 16 * l]
    for l in range(4):
        q[:, 48:52] = 3 * q[:, 48:52] + t[:, 240 + 4 * l: 244 + 4 * l]
    q[:, 48:52] *= 3
    b = back.reshape(-1, 54)
    assert np.array_equal(b[:, :52], synth.tq1_pack_value(q))
    assert np.array_equal(b[:, 52:], w.reshape(-1, 54)[:, 52:])
    assert (b[:, :52] != w.reshape(-1, 54)[:, :52]).any()   # some bytes were not canonical


@pytest.mark.parametrize("K,M,mode", [(512, 1, 0), (4096, 3, 0), (288, 1, 0), (9728, 8, 0),
                                      (4096, 2, 1), (768, 8, 1)])
def test_quantize_exact(gpu, oracle, K, M, mode):
    print(f"case quantize K={K} M={M} mode={mode}", flush=True)
    rng = np.random.default_rng([K, M, mode])
    x = (rng.standard_normal((M, K)) * rng.uniform(0.01, 100)).astype(np.float32)
    x[0, : min(K, 16)] = 0.0
    if M > 1:
        x[1] = 0.0  # an all-zero token gets q = 0 and scale 0 (tests/test_gemv.c:81-84)
    nsc = M if mode == 0 else M * (K // 256)
    dq, ds = gpu.empty((M, K), np.int8), gpu.empty(nsc, np.float32)
    gpu.quantize(mode, gpu.array(x), K, M, K, dq, ds)
    q, s = dq.numpy(), ds.numpy()
    for t in range(M):
        if mode == 0:
            wq, ws = oracle.quantize(x[t])
            assert np.array_equal(q[t], wq)
            assert bits(s[t]) == bits(np.float32(ws))
        else:
            wq, ws = oracle.quantize_k(x[t])
            assert np.array_equal(q[t], wq)
            assert np.array_equal(bits(s.reshape(M, -1)[t]), bits(ws))


def nonfinite_rows(rng, K):
    """Activation rows the fast quantiser must hand to its exact path: a NaN
    (amax skips it, its q is the x86 conversion of NaN: -127), +inf and -inf
    (amax = inf, inv = 0), a subnormal amax (inv = inf) and an amax just
    above 2^-120 (the fast path's limit)."""
    rows = []
    for kind in ("nan", "inf", "-inf", "tiny", "edge"):
        x = rng.standard_normal(K).astype(np.float32)
        if kind == "nan":
            x[rng.integers(0, K, 3)] = np.nan
        elif kind == "inf":
            x[K // 3] = np.inf
        elif kind == "-inf":
            x[K // 2] = -np.inf
        elif kind == "tiny":
            x = (x * np.float32(1e-40)).astype(np.float32)
        else:
            x = (x / np.abs(x).max() * np.float32(2.0 ** -120)).astype(np.float32)
        rows.append(x)
    return np.stack(rows)


@pytest.mark.parametrize("mode", [0, 1])
def test_quantize_nonfinite_follows_the_reference(gpu, oracle, mode):
    """src/gemv.c:20-38 on NaN, inf and tiny inputs as the reference's x86 build
    runs it: (int) of NaN or of an out-of-range value is INT_MIN, clamped to
    -127."""
    rng = np.random.default_rng(11 + mode)
    K = 512
    x = nonfinite_rows(rng, K)
    M = x.shape[0]
    nsc = M if mode == 0 else M * (K // 256)
    dq, ds = gpu.empty((M, K), np.int8), gpu.empty(nsc, np.float32)
    gpu.quantize(mode, gpu.array(x), K, M, K, dq, ds)
    q, s = dq.numpy(), ds.numpy()
    for t in range(M):
        wq, ws = oracle.quantize(x[t]) if mode == 0 else oracle.quantize_k(x[t])
        assert np.array_equal(q[t], wq), t
        got_s = s[t:t + 1] if mode == 0 else s.reshape(M, -1)[t]
        assert np.array_equal(bits(got_s), bits(np.atleast_1d(np.float32(ws)) if mode == 0
                                                 else ws)), t


def same_or_both_nan(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a)
    return np.array_equal(nan, np.isnan(b)) and np.array_equal(bits(a[~nan]), bits(b[~nan]))


@pytest.mark.parametrize("tname", ["TQ1_0", "TQ2_0", "Q4_K", "Q6_K"])
def test_fused_gemv_nonfinite_follows_the_reference(gpu, oracle, tname):
    """The fused GEMV's in-workgroup quantiser on the same rows (NaN outputs
    compared as NaN).  The K-quants quantise per 256-element block
    (src/kernels.c:722-754), so their rows add an all-zero block beside a
    normal one and a block of NaNs only (amax 0: zeros, scale 0)."""
    gtype = TYPES[tname]
    rng = np.random.default_rng(21 + gtype)
    K, N = 512, 48
    w = weights(rng, gtype, N, K)
    x = nonfinite_rows(rng, K)
    if gtype in (12, 14):
        z = rng.standard_normal((2, K)).astype(np.float32)
        z[0, :256] = 0.0
        z[1, 256:] = np.nan
        x = np.concatenate([x, z])
    M = x.shape[0]
    t = gpu.tensor(gtype, K, N, w)
    for r in range(M):
        out = gpu.empty((1, N), np.float32)
        gpu.gemv(t, gpu.array(x[r:r + 1]), 1, out)
        assert same_or_both_nan(out.numpy()[0], oracle.gemv(gtype, x[r], w, N, K)), r


@pytest.mark.parametrize("tname", ["TQ1_0", "TQ2_0", "Q4_K", "Q6_K"])
def test_i8_entry_equals_float_entry(gpu, oracle, tname):
    """f32 entry == pre-quantised entry exactly (tests/test_gemv.c:145-152)."""
    gtype = TYPES[tname]
    N, K, M = 70, 1024, 2
    rng = np.random.default_rng([7, gtype])
    w = weights(rng, gtype, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    t = gpu.tensor(gtype, K, N, w)
    mode = 1 if gtype in (12, 14) else 0
    dq = gpu.empty((M, K), np.int8)
    ds = gpu.empty(M * (K // 256) if mode else M, np.float32)
    dx = gpu.array(x)
    gpu.quantize(mode, dx, K, M, K, dq, ds)
    a, b = gpu.empty((M, N), np.float32), gpu.empty((M, N), np.float32)
    gpu.gemv(t, dx, M, a)
    gpu.gemv_i8(t, dq, ds, M, b)
    assert np.array_equal(bits(a.numpy()), bits(b.numpy()))
    want = oracle_gemv(oracle, gtype, x, w, N, K)
    assert np.array_equal(bits(a.numpy()), bits(want))


def test_gemv_multi_and_accumulate(gpu, oracle):
    """q/k/v in one call share the quantised input; ACCUMULATE adds into out
    exactly as fox_add would (src/ops.c:50-54)."""
    rng = np.random.default_rng(11)
    K = 2560
    shapes = [4096, 1024, 1024]
    ws = [weights(rng, 34, n, K) for n in shapes]
    x = rng.standard_normal((2, K)).astype(np.float32)
    ts = [gpu.tensor(34, K, n, w) for n, w in zip(shapes, ws)]
    outs = [gpu.empty((2, n), np.float32) for n in shapes]
    gpu.gemv_multi(ts, gpu.array(x), 2, outs)
    for n, w, o in zip(shapes, ws, outs):
        assert np.array_equal(bits(o.numpy()), bits(oracle_gemv(oracle, 34, x, w, n, K)))
    base = rng.standard_normal((2, 4096)).astype(np.float32)
    acc = gpu.array(base)
    gpu.gemv(ts[0], gpu.array(x), 2, acc, flags=rf.GEMV_ACCUMULATE)
    want = base + oracle_gemv(oracle, 34, x, ws[0], 4096, K)
    assert np.array_equal(bits(acc.numpy()), bits(want))


@pytest.mark.parametrize("tname,N,K", [("TQ1_0", 37, 512), ("TQ2_0", 20, 256),
                                       ("Q4_K", 17, 512), ("Q6_K", 33, 256), ("F16", 5, 288)])
def test_tensor_bytes_round_trip(gpu, tname, N, K):
    """The device backend holds the GGUF bytes exactly: repack then unpack
    gives them back (the resident == streamed byte check of
    tests/test_weights.c:142-175, for HBM)."""
    gtype = TYPES[tname]
    rng = np.random.default_rng(3)
    if tname == "TQ1_0":
        # TQ1_0 is held as 2-bit codes: the bytes come back exactly when they
        # are the canonical encoding of their trits, as the reference's
        # quantiser writes them
        w = synth.tq1_random(rng, N * K // 256).reshape(-1)
    else:
        w = rng.integers(0, 256, size=N * synth.row_bytes(gtype, K), dtype=np.uint8)
    t = gpu.tensor(gtype, K, N, w)
    assert np.array_equal(t.download(), w)
    info = t.info()
    assert info["gguf_bytes"] == w.nbytes
    assert info["device_bytes"] >= w.nbytes


def test_errors_follow_the_reference(gpu):
    """Ragged K, bad sizes and unknown types fail with the reference's
    status codes (src/gemv.c:80-85, src/kernels.c:852-857)."""
    with pytest.raises(rf.FoxError) as e:
        gpu.tensor(34, 255, 4, np.zeros(54 * 4, np.uint8))
    assert e.value.status == 1
    with pytest.raises(rf.FoxError) as e:
        gpu.tensor(10, 256, 1, np.zeros(84, np.uint8))   # Q2_K: no kernel
    assert e.value.status == 5
    t = gpu.tensor(34, 256, 16, np.zeros(54 * 16, np.uint8))
    x = gpu.array(np.zeros((9, 256), np.float32))
    out = gpu.empty((9, 16), np.float32)
    with pytest.raises(rf.FoxError) as e:
        gpu.gemv(t, x, 9, out)                           # more than 8 tokens
    assert e.value.status == 1
