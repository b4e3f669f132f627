"""One-launch decode-layer stages (fox_gpu_gemv_rmsnorm, fox_gpu_qkv_rope,
fox_gpu_gate_up_silu) against the oracle's separate steps: RMSNorm
(src/ops.c:7-22), the quantised GEMV (src/gemv.c), RoPE (src/ops.c:56-73),
the cache store (src/forward.c:346-362) and SwiGLU (src/ops.c:41-48).
Outputs must be bit-identical."""
import numpy as np
import pytest

import rustfox_amd as rf
from test_gpu_gemv import weights, bits, nonfinite_rows, same_or_both_nan

pytestmark = pytest.mark.gpu

EPS = 1e-5


def ref_norm_gemv(oracle, gtype, x, nw, W, N, K):
    return np.stack([oracle.gemv(gtype, oracle.rmsnorm(x[t], nw, EPS), W, N, K)
                     for t in range(x.shape[0])])


@pytest.mark.parametrize("tname,gtype", [("TQ1_0", 34), ("TQ2_0", 35)])
@pytest.mark.parametrize("K,M,accumulate", [(2560, 1, False), (4096, 1, True), (768, 3, False),
                                            (512, 8, True), (9728, 8, False), (4096, 2, True),
                                            (1536, 6, False), (1024, 7, True), (2560, 5, False)])
def test_gemv_rmsnorm_bit_exact(gpu, oracle, tname, gtype, K, M, accumulate):
    rng = np.random.default_rng(K * 10 + M)
    Ns = [48, 37]
    Ws = [weights(rng, gtype, N, K) for N in Ns]
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    ts = [gpu.tensor(gtype, K, N, w) for N, w in zip(Ns, Ws)]
    init = [rng.standard_normal((M, N)).astype(np.float32) for N in Ns]
    outs = [gpu.array(i if accumulate else np.zeros_like(i)) for i in init]
    gpu.gemv_rmsnorm(ts, gpu.array(x), M, gpu.array(nw), EPS, outs,
                     rf.GEMV_ACCUMULATE if accumulate else 0)
    gpu.sync()
    for N, W, o, i in zip(Ns, Ws, outs, init):
        want = ref_norm_gemv(oracle, gtype, x, nw, W, N, K)
        if accumulate:
            want = i + want
        assert np.array_equal(bits(o.numpy()), bits(want)), tname


@pytest.mark.parametrize("gtype", [34, 35])
@pytest.mark.parametrize("M,pos", [(1, 5), (3, 36), (2, 39), (5, 20), (7, 36), (8, 30)])
def test_qkv_rope_bit_exact(gpu, oracle, gtype, M, pos):
    """q, k, v projections of rmsnorm(x), RoPE at pos + t, k and v rows into
    the caches; a token at or past n_ctx is neither rotated nor stored."""
    K, n_head, n_kv, hd, n_ctx = 768, 4, 2, 64, 40
    rng = np.random.default_rng(100 + M + pos + gtype)
    Wq, Wk, Wv = (weights(rng, gtype, n, K) for n in (n_head * hd, n_kv * hd, n_kv * hd))
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    cos_t, sin_t = oracle.rope_tables(n_ctx, hd, 10000.0)
    kvd = n_kv * hd
    q_out = gpu.empty(M * n_head * hd, np.float32)
    kc = gpu.array(np.zeros(n_ctx * kvd, np.float32))
    vc = gpu.array(np.zeros((n_ctx + 3) // 4 * 4 * kvd, np.float32))
    gpu.qkv_rope(gpu.tensor(gtype, K, n_head * hd, Wq), gpu.tensor(gtype, K, kvd, Wk),
                 gpu.tensor(gtype, K, kvd, Wv), gpu.array(x), M, gpu.array(nw), EPS, q_out,
                 gpu.array(cos_t), gpu.array(sin_t), gpu.array(np.array([pos], np.uint32)),
                 n_ctx, kc, vc, hd)
    gpu.sync()
    got_q = q_out.numpy().reshape(M, -1)
    got_k = kc.numpy().reshape(n_ctx, kvd)
    vq = vc.numpy().reshape(-1, kvd, 4)
    got_v = np.stack([vq[p // 4, :, p % 4] for p in range(n_ctx)])
    want_k = np.zeros((n_ctx, kvd), np.float32)
    want_v = np.zeros((n_ctx, kvd), np.float32)
    half = hd // 2
    for t in range(M):
        xb = oracle.rmsnorm(x[t], nw, EPS)
        q = oracle.gemv(gtype, xb, Wq, n_head * hd, K)
        k = oracle.gemv(gtype, xb, Wk, kvd, K)
        v = oracle.gemv(gtype, xb, Wv, kvd, K)
        p = pos + t
        if p < n_ctx:
            cr, sr = cos_t[p * half:(p + 1) * half], sin_t[p * half:(p + 1) * half]
            q = oracle.rope(q, n_head, hd, cr, sr)
            want_k[p] = oracle.rope(k, n_kv, hd, cr, sr)
            want_v[p] = v
        assert np.array_equal(bits(got_q[t]), bits(q)), f"q of token {t}"
    assert np.array_equal(bits(got_k), bits(want_k))
    assert np.array_equal(bits(got_v), bits(want_v))


@pytest.mark.parametrize("gtype", [34, 35])
@pytest.mark.parametrize("K,ff,M", [(2560, 700, 1), (768, 1040, 2), (512, 96, 8), (768, 200, 5),
                                     (2048, 64, 7), (4096, 130, 6)])
def test_gate_up_silu_bit_exact(gpu, oracle, gtype, K, ff, M):
    rng = np.random.default_rng(K + ff + M + gtype)
    Wg, Wu = weights(rng, gtype, ff, K), weights(rng, gtype, ff, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    h = gpu.empty(M * ff, np.float32)
    gpu.gate_up_silu(gpu.tensor(gtype, K, ff, Wg), gpu.tensor(gtype, K, ff, Wu), gpu.array(x), M,
                     gpu.array(nw), EPS, h)
    gpu.sync()
    got = h.numpy().reshape(M, ff)
    for t in range(M):
        xb = oracle.rmsnorm(x[t], nw, EPS)
        want = oracle.silu_mul(oracle.gemv(gtype, xb, Wg, ff, K), oracle.gemv(gtype, xb, Wu, ff, K))
        assert np.array_equal(bits(got[t]), bits(want)), f"token {t}"


@pytest.mark.parametrize("gtype", [34, 35])
def test_gemv_rmsnorm_nonfinite_follows_the_reference(gpu, oracle, gtype):
    """RMSNorm then quantisation on rows with NaN, inf and tiny values, and
    on a normal row scaled by norm weights that hold a NaN and an inf: the
    exact path of the in-workgroup quantiser (NaN outputs compared as NaN)."""
    rng = np.random.default_rng(31 + gtype)
    K, N = 512, 40
    W = weights(rng, gtype, N, K)
    t = gpu.tensor(gtype, K, N, W)
    rows = list(nonfinite_rows(rng, K))
    nws = [rng.uniform(0.5, 1.5, K).astype(np.float32) for _ in rows]
    x = rng.standard_normal(K).astype(np.float32)
    for bad in (np.nan, np.inf):
        nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
        nw[7] = bad
        rows.append(x)
        nws.append(nw)
    for r, (xr, nw) in enumerate(zip(rows, nws)):
        out = gpu.array(np.zeros((1, N), np.float32))
        gpu.gemv_rmsnorm([t], gpu.array(xr[None, :]), 1, gpu.array(nw), EPS, [out], 0)
        want = oracle.gemv(gtype, oracle.rmsnorm(xr, nw, EPS), W, N, K)
        assert same_or_both_nan(out.numpy()[0], want), r


def test_unsupported_cases_say_so(gpu):
    """K-quants for more than one token, and activations too wide for one
    workgroup's LDS (16384 x 8 tokens: B operand and terms above 160 KB), are
    refused with FOX_GPU_ERR_UNSUPPORTED (the host then runs the separate
    steps)."""
    rng = np.random.default_rng(3)
    q4 = gpu.tensor(12, 512, 16, weights(rng, 12, 16, 512))
    x = gpu.array(rng.standard_normal((2, 512)).astype(np.float32))
    nw = gpu.array(np.ones(512, np.float32))
    out = gpu.empty(32, np.float32)
    with pytest.raises(rf.FoxError) as e:
        gpu.gemv_rmsnorm([q4], x, 2, nw, EPS, [out])
    assert e.value.status == 5
    K = 16384
    t = gpu.tensor(34, K, 16, weights(rng, 34, 16, K))
    xw = gpu.array(rng.standard_normal((8, K)).astype(np.float32))
    with pytest.raises(rf.FoxError) as e:
        gpu.gemv_rmsnorm([t], xw, 8, gpu.array(np.ones(K, np.float32)), EPS,
                         [gpu.empty(8 * 16, np.float32)])
    assert e.value.status == 5


def test_mixed_types_take_the_separate_steps(gpu):
    """Gate and up of different types, and q and k of different types other
    than the two K-quants, are refused by the one-launch stages with
    FOX_GPU_ERR_UNSUPPORTED, the status on which the host runs the separate
    steps; so is a Q4_K_M-style q/k/v (Q4_K q and k, Q6_K v) for more than
    one token.  Mismatched widths remain FOX_GPU_ERR_ARG."""
    rng = np.random.default_rng(4)
    K, hd, n_ctx = 512, 64, 8
    q4 = [gpu.tensor(12, K, 128, weights(rng, 12, 128, K)) for _ in range(2)]
    q6 = gpu.tensor(14, K, 128, weights(rng, 14, 128, K))
    x = gpu.array(rng.standard_normal(K).astype(np.float32))
    x2 = gpu.array(rng.standard_normal((2, K)).astype(np.float32))
    nw = gpu.array(np.ones(K, np.float32))
    cs = gpu.array(np.ones(n_ctx * hd // 2, np.float32))
    pos = gpu.array(np.zeros(1, np.uint32))
    kc = gpu.empty(n_ctx * 128, np.float32)
    vc = gpu.empty(n_ctx * 128, np.float32)
    tq = gpu.tensor(35, K, 128, weights(rng, 35, 128, K))
    with pytest.raises(rf.FoxError) as e:
        gpu.qkv_rope(tq, q4[0], q4[1], x, 1, nw, EPS, gpu.empty(128, np.float32), cs, cs, pos,
                     n_ctx, kc, vc, hd)
    assert e.value.status == 5
    with pytest.raises(rf.FoxError) as e:
        gpu.qkv_rope(q4[0], q4[1], q6, x2, 2, nw, EPS, gpu.empty(256, np.float32), cs, cs, pos,
                     n_ctx, kc, vc, hd)
    assert e.value.status == 5
    with pytest.raises(rf.FoxError) as e:
        gpu.gate_up_silu(q4[0], q6, x, 1, nw, EPS, gpu.empty(128, np.float32))
    assert e.value.status == 5
    wide = gpu.tensor(34, 2 * K, 128, weights(rng, 34, 128, 2 * K))
    narrow = gpu.tensor(34, K, 128, weights(rng, 34, 128, K))
    with pytest.raises(rf.FoxError) as e:
        gpu.gate_up_silu(narrow, wide, x, 1, nw, EPS, gpu.empty(128, np.float32))
    assert e.value.status == 1


@pytest.mark.parametrize("tname,gtype", [("Q4_K", 12), ("Q6_K", 14)])
@pytest.mark.parametrize("K", [768, 4096])
def test_kquant_one_token_stages_bit_exact(gpu, oracle, tname, gtype, K):
    """The K-quants' one-token stages: RMSNorm, per-block quantisation
    (src/kernels.c:722-754) and the int8 dots (src/kernels.c:571-661) in one
    launch, with the residual add, with RoPE and the cache store, and with
    SwiGLU; bit-identical to the oracle's separate steps."""
    rng = np.random.default_rng([K, gtype, 61])
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    x = rng.standard_normal((1, K)).astype(np.float32)
    xb = oracle.rmsnorm(x[0], nw, EPS)
    # gemv_rmsnorm over two matrices, the first accumulating
    Ns = [80, 45]
    Ws = [weights(rng, gtype, N, K) for N in Ns]
    base = [rng.standard_normal((1, N)).astype(np.float32) for N in Ns]
    outs = [gpu.array(b) for b in base]
    gpu.gemv_rmsnorm([gpu.tensor(gtype, K, N, w) for N, w in zip(Ns, Ws)], gpu.array(x), 1,
                     gpu.array(nw), EPS, outs, rf.GEMV_ACCUMULATE)
    for N, W, o, b in zip(Ns, Ws, outs, base):
        want = b[0] + oracle.gemv(gtype, xb, W, N, K)
        assert np.array_equal(bits(o.numpy()[0]), bits(want)), f"{tname} rmsnorm {N}"
    # q, k, v with RoPE
    n_head, n_kv, hd, n_ctx, pos = 4, 2, 64, 16, 9
    kvd = n_kv * hd
    Wq, Wk, Wv = (weights(rng, gtype, n, K) for n in (n_head * hd, kvd, kvd))
    cos_t, sin_t = oracle.rope_tables(n_ctx, hd, 10000.0)
    q_out = gpu.empty(n_head * hd, np.float32)
    kc = gpu.array(np.zeros(n_ctx * kvd, np.float32))
    vc = gpu.array(np.zeros(n_ctx * kvd, np.float32))
    gpu.qkv_rope(gpu.tensor(gtype, K, n_head * hd, Wq), gpu.tensor(gtype, K, kvd, Wk),
                 gpu.tensor(gtype, K, kvd, Wv), gpu.array(x), 1, gpu.array(nw), EPS, q_out,
                 gpu.array(cos_t), gpu.array(sin_t), gpu.array(np.array([pos], np.uint32)),
                 n_ctx, kc, vc, hd)
    half = hd // 2
    cr, sr = cos_t[pos * half:(pos + 1) * half], sin_t[pos * half:(pos + 1) * half]
    want_q = oracle.rope(oracle.gemv(gtype, xb, Wq, n_head * hd, K), n_head, hd, cr, sr)
    want_k = oracle.rope(oracle.gemv(gtype, xb, Wk, kvd, K), n_kv, hd, cr, sr)
    want_v = oracle.gemv(gtype, xb, Wv, kvd, K)
    vq = vc.numpy().reshape(-1, kvd, 4)
    assert np.array_equal(bits(q_out.numpy()), bits(want_q)), f"{tname} q"
    assert np.array_equal(bits(kc.numpy().reshape(n_ctx, kvd)[pos]), bits(want_k)), f"{tname} k"
    assert np.array_equal(bits(vq[pos // 4, :, pos % 4]), bits(want_v)), f"{tname} v"
    # gate / up with SwiGLU
    ff = 300
    Wg, Wu = weights(rng, gtype, ff, K), weights(rng, gtype, ff, K)
    h = gpu.empty(ff, np.float32)
    gpu.gate_up_silu(gpu.tensor(gtype, K, ff, Wg), gpu.tensor(gtype, K, ff, Wu), gpu.array(x), 1,
                     gpu.array(nw), EPS, h)
    want = oracle.silu_mul(oracle.gemv(gtype, xb, Wg, ff, K), oracle.gemv(gtype, xb, Wu, ff, K))
    assert np.array_equal(bits(h.numpy()), bits(want)), f"{tname} gate/up"


@pytest.mark.parametrize("gtype", [12, 14])
def test_kquant_rmsnorm_nonfinite_follows_the_reference(gpu, oracle, gtype):
    """RMSNorm then per-block quantisation on rows with NaN, inf and tiny
    values (NaN outputs compared as NaN)."""
    rng = np.random.default_rng(41 + gtype)
    K, N = 512, 40
    W = weights(rng, gtype, N, K)
    t = gpu.tensor(gtype, K, N, W)
    for r, xr in enumerate(nonfinite_rows(rng, K)):
        nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
        out = gpu.array(np.zeros((1, N), np.float32))
        gpu.gemv_rmsnorm([t], gpu.array(xr[None, :]), 1, gpu.array(nw), EPS, [out], 0)
        want = oracle.gemv(gtype, oracle.rmsnorm(xr, nw, EPS), W, N, K)
        assert same_or_both_nan(out.numpy()[0], want), r


@pytest.mark.parametrize("K,pos", [(768, 3), (4096, 13)])
@pytest.mark.parametrize("types", [(12, 12, 14), (12, 14, 12), (14, 14, 12), (14, 12, 14)],
                         ids=lambda t: "-".join({12: "q4", 14: "q6"}[x] for x in t))
def test_q4_k_m_qkv_rope_bit_exact(gpu, oracle, K, pos, types):
    """A Q4_K_M-style q/k/v for one token (and the other mixes of the two
    K-quants): one launch, each segment in its own format, q and k with
    RoPE, v into the cache, all from rmsnorm(x)."""
    n_head, n_kv, hd, n_ctx = 4, 2, 64, 16
    kvd = n_kv * hd
    tq_, tk_, tv_ = types
    rng = np.random.default_rng([K, pos, 62] + list(types))
    Wq, Wk = weights(rng, tq_, n_head * hd, K), weights(rng, tk_, kvd, K)
    Wv = weights(rng, tv_, kvd, K)
    x = rng.standard_normal((1, K)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    cos_t, sin_t = oracle.rope_tables(n_ctx, hd, 10000.0)
    q_out = gpu.empty(n_head * hd, np.float32)
    kc = gpu.array(np.zeros(n_ctx * kvd, np.float32))
    vc = gpu.array(np.zeros(n_ctx * kvd, np.float32))
    gpu.qkv_rope(gpu.tensor(tq_, K, n_head * hd, Wq), gpu.tensor(tk_, K, kvd, Wk),
                 gpu.tensor(tv_, K, kvd, Wv), gpu.array(x), 1, gpu.array(nw), EPS, q_out,
                 gpu.array(cos_t), gpu.array(sin_t), gpu.array(np.array([pos], np.uint32)),
                 n_ctx, kc, vc, hd)
    xb = oracle.rmsnorm(x[0], nw, EPS)
    half = hd // 2
    cr, sr = cos_t[pos * half:(pos + 1) * half], sin_t[pos * half:(pos + 1) * half]
    want_q = oracle.rope(oracle.gemv(tq_, xb, Wq, n_head * hd, K), n_head, hd, cr, sr)
    want_k = oracle.rope(oracle.gemv(tk_, xb, Wk, kvd, K), n_kv, hd, cr, sr)
    want_v = oracle.gemv(tv_, xb, Wv, kvd, K)
    vq = vc.numpy().reshape(-1, kvd, 4)
    got_k = kc.numpy().reshape(n_ctx, kvd)
    assert np.array_equal(bits(q_out.numpy()), bits(want_q))
    assert np.array_equal(bits(got_k[pos]), bits(want_k))
    assert np.array_equal(bits(vq[pos // 4, :, pos % 4]), bits(want_v))
    others = [p for p in range(n_ctx) if p != pos]
    assert not got_k[others].any()
