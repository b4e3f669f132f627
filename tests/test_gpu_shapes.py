"""GPU parity at the benchmark workloads' own shapes (bit-exact).

The fused ternary GEMV runs one persistent grid of at most two workgroups
per compute unit; a launch with more 16-row tiles than that makes every
workgroup walk several tiles in turn (double-buffered block terms, a weight
cursor that crosses tiles, the next tile's epilogue operands loaded during
the current tile's combine).  The 14336 x 4096 GEMV (896 tiles) and the
4B-class gate/up pair (608 tile pairs) do so at the default grid; every
case here also runs with the grid capped (fox_gpu_set_max_workgroups) to
1, 3 and 7 workgroups, so that each workgroup walks hundreds of tiles.
Results must not depend on the grid: every output row is combined by one
workgroup in block order (src/gemv.c:54-97).

Shapes: the single-op microbenchmark (TQ1_0/TQ2_0 14336 x 4096, M = 1 and
8), the 4B-class layer (q/k/v 2560 -> 4096/1024/1024 with RoPE at position
2048+, gate/up 2560 -> 9728, ffn_down 9728 -> 2560 and attn_output 4096 ->
2560 with the residual add), the 8B-class layer's Q4_K/Q6_K matrices
(14336 x 4096, 4096 x 14336) and the 27B-class layer's TQ1_0 ffn_down
(21504 -> 5376: the fused path for one token and for 8, where one
workgroup per compute unit has up to 160 KB of LDS; K = 24576 is past the
fused kernel's input registers and takes the unfused path) and its 8-token
pass at d_model 5376.
"""
import numpy as np
import pytest

import rustfox_amd as rf
from test_gpu_gemv import weights, bits

pytestmark = pytest.mark.gpu

EPS = 1e-5
THREADS = 8
CAPS = [0, 1, 3, 7]


def ogemv(oracle, gtype, x, w, N, K):
    return np.stack([oracle.gemv(gtype, x[t], w, N, K, n_threads=THREADS)
                     for t in range(x.shape[0])])


def first_diff(got, want):
    d = np.flatnonzero(bits(got).reshape(-1) != bits(want).reshape(-1))
    if d.size == 0:
        return ""
    return (f"{d.size} of {got.size} differ; first {d[:4]}: got {got.reshape(-1)[d[:4]]} "
            f"want {want.reshape(-1)[d[:4]]}")


@pytest.fixture
def capped(gpu):
    """Restores the default grid after a test that caps it."""
    yield gpu
    gpu.set_max_workgroups(0)


_cache = {}


def case_data(oracle, gtype, N, K, M, seed):
    key = (gtype, N, K, M, seed)
    if key not in _cache:
        rng = np.random.default_rng([N, K, M, gtype, seed])
        w = weights(rng, gtype, N, K)
        x = rng.standard_normal((M, K)).astype(np.float32)
        _cache.clear()
        _cache[key] = (w, x, ogemv(oracle, gtype, x, w, N, K))
    return _cache[key]


@pytest.mark.parametrize("cap", CAPS)
@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("tname,gtype", [("TQ1_0", 34), ("TQ2_0", 35)])
def test_microbench_shape_bit_exact(capped, oracle, tname, gtype, M, cap):
    """14336 x 4096, the roofline case: 896 tiles."""
    N, K = 14336, 4096
    print(f"case gemv {tname} {N}x{K} M={M} cap={cap}", flush=True)
    w, x, want = case_data(oracle, gtype, N, K, M, 1)
    capped.set_max_workgroups(cap)
    t = capped.tensor(gtype, K, N, w)
    dx = capped.array(x)
    out = capped.empty((M, N), np.float32)
    capped.gemv(t, dx, M, out)
    got = out.numpy()
    assert not first_diff(got, want), first_diff(got, want)
    if cap == 0:
        # a second launch over the same input gives the same bits
        out2 = capped.empty((M, N), np.float32)
        capped.gemv(t, dx, M, out2)
        assert np.array_equal(bits(out2.numpy()), bits(got))


@pytest.mark.parametrize("cap", CAPS)
@pytest.mark.parametrize("M", [1, 8])
def test_4b_gate_up_silu_bit_exact(capped, oracle, M, cap):
    """4B-class ffn_gate/ffn_up 2560 -> 9728 with the norm, the quantiser and
    SwiGLU in one launch: 608 tile pairs."""
    K, ff = 2560, 9728
    print(f"case gate_up 4b M={M} cap={cap}", flush=True)
    rng = np.random.default_rng([K, ff, M, 5])
    Wg, Wu = weights(rng, 34, ff, K), weights(rng, 34, ff, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    capped.set_max_workgroups(cap)
    h = capped.empty(M * ff, np.float32)
    capped.gate_up_silu(capped.tensor(34, K, ff, Wg), capped.tensor(34, K, ff, Wu),
                        capped.array(x), M, capped.array(nw), EPS, h)
    got = h.numpy().reshape(M, ff)
    for t in range(M):
        xb = oracle.rmsnorm(x[t], nw, EPS)
        want = oracle.silu_mul(oracle.gemv(34, xb, Wg, ff, K, n_threads=THREADS),
                               oracle.gemv(34, xb, Wu, ff, K, n_threads=THREADS))
        assert not first_diff(got[t], want), f"token {t}: {first_diff(got[t], want)}"


@pytest.mark.parametrize("cap", [0, 5])
@pytest.mark.parametrize("M,pos", [(1, 2048), (8, 2044), (3, 2174)])
def test_4b_qkv_rope_bit_exact(capped, oracle, M, pos, cap):
    """4B-class q/k/v (2560 -> 4096, 1024, 1024; 32/8 heads of 128, RoPE base
    1e6) at positions past 2048 of a 2176-row cache: 384 tiles.  The last
    case runs two tokens past the cache end (neither rotated nor stored)."""
    K, n_head, n_kv, hd, n_ctx = 2560, 32, 8, 128, 2176
    print(f"case qkv_rope 4b M={M} pos={pos} cap={cap}", flush=True)
    rng = np.random.default_rng([K, M, pos, 9])
    Wq, Wk, Wv = (weights(rng, 34, n, K) for n in (n_head * hd, n_kv * hd, n_kv * hd))
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    cos_t, sin_t = oracle.rope_tables(n_ctx, hd, 1e6)
    kvd = n_kv * hd
    capped.set_max_workgroups(cap)
    q_out = capped.empty(M * n_head * hd, np.float32)
    kc = capped.array(np.zeros(n_ctx * kvd, np.float32))
    vc = capped.array(np.zeros((n_ctx + 3) // 4 * 4 * kvd, np.float32))
    capped.qkv_rope(capped.tensor(34, K, n_head * hd, Wq), capped.tensor(34, K, kvd, Wk),
                    capped.tensor(34, K, kvd, Wv), capped.array(x), M, capped.array(nw), EPS,
                    q_out, capped.array(cos_t), capped.array(sin_t),
                    capped.array(np.array([pos], np.uint32)), n_ctx, kc, vc, hd)
    got_q = q_out.numpy().reshape(M, -1)
    got_k = kc.numpy().reshape(n_ctx, kvd)
    vq = vc.numpy().reshape(-1, kvd, 4)
    half = hd // 2
    for t in range(M):
        xb = oracle.rmsnorm(x[t], nw, EPS)
        q = oracle.gemv(34, xb, Wq, n_head * hd, K, n_threads=THREADS)
        k = oracle.gemv(34, xb, Wk, kvd, K, n_threads=THREADS)
        v = oracle.gemv(34, xb, Wv, kvd, K, n_threads=THREADS)
        p = pos + t
        if p < n_ctx:
            cr, sr = cos_t[p * half:(p + 1) * half], sin_t[p * half:(p + 1) * half]
            q = oracle.rope(q, n_head, hd, cr, sr)
            assert not first_diff(got_k[p], oracle.rope(k, n_kv, hd, cr, sr)), f"k of token {t}"
            assert not first_diff(vq[p // 4, :, p % 4], v), f"v of token {t}"
        assert not first_diff(got_q[t], q), f"q of token {t}"
    # rows the pass does not reach stay untouched
    untouched = [p for p in range(n_ctx) if not pos <= p < pos + M]
    assert not got_k[untouched].any()


@pytest.mark.parametrize("cap", [0, 3])
@pytest.mark.parametrize("name,N,K,M", [("ffn_down 4b", 2560, 9728, 1),
                                        ("attn_output 4b", 2560, 4096, 1),
                                        ("attn_output 4b", 2560, 4096, 8),
                                        ("ffn_down 27b", 5376, 21504, 1),
                                        ("ffn_down 27b", 5376, 21504, 8),
                                        ("K past the fused limit", 1024, 24576, 8)])
def test_residual_projections_bit_exact(capped, oracle, name, N, K, M, cap):
    """out += W x (the residual add fused into the GEMV, src/forward.c:374-377,
    393-396).  K = 24576 is more than the fused kernel's input registers hold
    (22528) and takes the unfused path (quantiser kernel over block slices,
    then the block kernel)."""
    print(f"case {name} N={N} K={K} M={M} cap={cap}", flush=True)
    rng = np.random.default_rng([N, K, M, 13])
    w = weights(rng, 34, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    base = rng.standard_normal((M, N)).astype(np.float32)
    capped.set_max_workgroups(cap)
    acc = capped.array(base)
    capped.gemv(capped.tensor(34, K, N, w), capped.array(x), M, acc, flags=rf.GEMV_ACCUMULATE)
    want = base + ogemv(oracle, 34, x, w, N, K)
    got = acc.numpy()
    assert not first_diff(got, want), first_diff(got, want)


@pytest.mark.parametrize("M", [1, 8])
def test_27b_qkv_and_gate_up_8_tokens(capped, oracle, M):
    """27B-class d_model 5376 (21 blocks): q/k/v 5376 -> 4096, 2048, 2048 and
    gate/up 5376 -> 21504 (1344 tile pairs) for the 8-token verify pass."""
    K, n_head, n_kv, hd, ff = 5376, 32, 16, 128, 21504
    print(f"case 27b layer M={M}", flush=True)
    rng = np.random.default_rng([K, M, 27])
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    Wg, Wu = weights(rng, 34, ff, K), weights(rng, 34, ff, K)
    h = capped.empty(M * ff, np.float32)
    capped.gate_up_silu(capped.tensor(34, K, ff, Wg), capped.tensor(34, K, ff, Wu),
                        capped.array(x), M, capped.array(nw), EPS, h)
    got = h.numpy().reshape(M, ff)
    Ws = [weights(rng, 34, n, K) for n in (n_head * hd, n_kv * hd, n_kv * hd)]
    ts = [capped.tensor(34, K, n, w) for n, w in zip((n_head * hd, n_kv * hd, n_kv * hd), Ws)]
    outs = [capped.empty((M, n), np.float32) for n in (n_head * hd, n_kv * hd, n_kv * hd)]
    capped.gemv_rmsnorm(ts, capped.array(x), M, capped.array(nw), EPS, outs, 0)
    for t in range(M):
        xb = oracle.rmsnorm(x[t], nw, EPS)
        want = oracle.silu_mul(oracle.gemv(34, xb, Wg, ff, K, n_threads=THREADS),
                               oracle.gemv(34, xb, Wu, ff, K, n_threads=THREADS))
        assert not first_diff(got[t], want), f"gate/up token {t}: {first_diff(got[t], want)}"
        for n, w, o in zip((n_head * hd, n_kv * hd, n_kv * hd), Ws, outs):
            want = oracle.gemv(34, xb, w, n, K, n_threads=THREADS)
            assert not first_diff(o.numpy()[t], want), f"q/k/v rows {n} token {t}"


@pytest.mark.parametrize("M,cap", [(1, 0), (1, 3), (8, 0)])
@pytest.mark.parametrize("tname,gtype,N,K", [("Q4_K", 12, 14336, 4096), ("Q6_K", 14, 4096, 14336),
                                             ("Q4_K", 12, 4096, 4096), ("Q6_K", 14, 1024, 4096)])
def test_8b_kquant_shapes_bit_exact(capped, oracle, tname, gtype, N, K, M, cap):
    """8B-class Q4_K_M-style matrices: ffn_gate/up (Q4_K 4096 -> 14336),
    ffn_down (Q6_K 14336 -> 4096), attn_q/o (Q4_K 4096 x 4096), attn_v (Q6_K
    4096 -> 1024), weights from the repository's quantiser
    (src/kernels.c:571-661 int8 dots, per-256 activation scales).  One token
    takes the fused kernel (also with its grid capped to 3 workgroups, each
    then walking hundreds of tiles), 8 tokens the unfused path."""
    print(f"case gemv 8b {tname} {N}x{K} M={M} cap={cap}", flush=True)
    w, x, want = case_data(oracle, gtype, N, K, M, 8)
    capped.set_max_workgroups(cap)
    out = capped.empty((M, N), np.float32)
    capped.gemv(capped.tensor(gtype, K, N, w), capped.array(x), M, out)
    got = out.numpy()
    assert not first_diff(got, want), first_diff(got, want)


@pytest.mark.parametrize("cap", [0, 5])
@pytest.mark.parametrize("v_type", [14, 12])
def test_8b_qkv_rope_kquant_mix_bit_exact(capped, oracle, v_type, cap):
    """8B-class q/k/v (4096 -> 4096, 1024, 1024; 32/8 heads of 128) for one
    token at position 4096 of a 4200-row cache: Q4_K q and k with a Q6_K v
    in one launch whose segments keep their own formats (the Q4_K_M mix),
    and all three Q4_K.  With the grid capped each workgroup walks tiles of
    both formats in turn."""
    K, n_head, n_kv, hd, n_ctx, pos = 4096, 32, 8, 128, 4200, 4096
    print(f"case qkv_rope 8b v_type={v_type} cap={cap}", flush=True)
    rng = np.random.default_rng([K, v_type, 17])
    Wq, Wk = weights(rng, 12, n_head * hd, K), weights(rng, 12, n_kv * hd, K)
    Wv = weights(rng, v_type, n_kv * hd, K)
    x = rng.standard_normal((1, K)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    cos_t, sin_t = oracle.rope_tables(n_ctx, hd, 5e5)
    kvd = n_kv * hd
    capped.set_max_workgroups(cap)
    q_out = capped.empty(n_head * hd, np.float32)
    kc = capped.array(np.zeros(n_ctx * kvd, np.float32))
    vc = capped.array(np.zeros((n_ctx + 3) // 4 * 4 * kvd, np.float32))
    capped.qkv_rope(capped.tensor(12, K, n_head * hd, Wq), capped.tensor(12, K, kvd, Wk),
                    capped.tensor(v_type, K, kvd, Wv), capped.array(x), 1, capped.array(nw), EPS,
                    q_out, capped.array(cos_t), capped.array(sin_t),
                    capped.array(np.array([pos], np.uint32)), n_ctx, kc, vc, hd)
    xb = oracle.rmsnorm(x[0], nw, EPS)
    half = hd // 2
    cr, sr = cos_t[pos * half:(pos + 1) * half], sin_t[pos * half:(pos + 1) * half]
    q = oracle.rope(oracle.gemv(12, xb, Wq, n_head * hd, K, n_threads=THREADS), n_head, hd, cr, sr)
    k = oracle.rope(oracle.gemv(12, xb, Wk, kvd, K, n_threads=THREADS), n_kv, hd, cr, sr)
    v = oracle.gemv(v_type, xb, Wv, kvd, K, n_threads=THREADS)
    assert not first_diff(q_out.numpy(), q), "q: " + first_diff(q_out.numpy(), q)
    got_k = kc.numpy().reshape(n_ctx, kvd)
    assert not first_diff(got_k[pos], k), "k: " + first_diff(got_k[pos], k)
    vq = vc.numpy().reshape(-1, kvd, 4)
    assert not first_diff(vq[pos // 4, :, pos % 4], v), "v: " + first_diff(vq[pos // 4, :, pos % 4], v)
    untouched = [p for p in range(n_ctx) if p != pos]
    assert not got_k[untouched].any()


@pytest.mark.parametrize("cap", [0, 5])
def test_8b_gate_up_silu_bit_exact(capped, oracle, cap):
    """8B-class ffn_gate/ffn_up (Q4_K 4096 -> 14336, 896 tile pairs) with
    RMSNorm and SwiGLU in one launch for one token."""
    K, ff = 4096, 14336
    print(f"case 8b gate/up cap={cap}", flush=True)
    rng = np.random.default_rng([K, ff, 88])
    x = rng.standard_normal((1, K)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    Wg, Wu = weights(rng, 12, ff, K), weights(rng, 12, ff, K)
    capped.set_max_workgroups(cap)
    h = capped.empty(ff, np.float32)
    capped.gate_up_silu(capped.tensor(12, K, ff, Wg), capped.tensor(12, K, ff, Wu),
                        capped.array(x), 1, capped.array(nw), EPS, h)
    xb = oracle.rmsnorm(x[0], nw, EPS)
    want = oracle.silu_mul(oracle.gemv(12, xb, Wg, ff, K, n_threads=THREADS),
                           oracle.gemv(12, xb, Wu, ff, K, n_threads=THREADS))
    got = h.numpy()
    assert not first_diff(got, want), first_diff(got, want)
