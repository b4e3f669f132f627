"""Attention on the GPU against the reference's order of operations
(src/forward.c:222-257, src/ops.c:24-39) restated with float32 numpy steps
(each numpy float32 operation rounds once, no contraction) and the oracle's
softmax (glibc expf).  Exact mode must be bit-identical; split mode within
float rounding.  Caches are written through fox_gpu_kv_write, so the
interleaved V layout is exercised as the decode path uses it."""
import numpy as np
import pytest

import rustfox_amd as rf

pytestmark = pytest.mark.gpu


def reference_attention(oracle, q, K, V, n_head, n_kv, hd, pos, M, n_ctx):
    """q [M][n_head*hd]; K, V [n_ctx][n_kv*hd] row-major."""
    gqa = n_head // n_kv
    out = np.zeros((M, n_head * hd), np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    for t in range(M):
        upto = min(pos + t + 1, n_ctx)
        for h in range(n_head):
            kvh = h // gqa
            qh = q[t, h * hd:(h + 1) * hd]
            Kh = K[:upto, kvh * hd:(kvh + 1) * hd]
            a = np.zeros(upto, np.float32)
            for d in range(hd):                    # fox_dot_f32 in d order
                a = a + qh[d] * Kh[:, d]
            att = oracle.softmax(a * scale)
            Vh = V[:upto, kvh * hd:(kvh + 1) * hd]
            acc = np.zeros(hd, np.float32)
            for j in range(upto):                  # dst[d] += a * vj[d], j order
                acc = acc + att[j] * Vh[j]
            out[t, h * hd:(h + 1) * hd] = acc
    return out


def run_gpu(gpu, q, K, V, n_head, n_kv, hd, pos, M, n_ctx, mode, before=None):
    kvd = n_kv * hd
    kc = gpu.empty(n_ctx * kvd, np.float32)
    vc = gpu.empty((n_ctx + 3) // 4 * 4 * kvd, np.float32)
    dk = gpu.array(K.astype(np.float32))
    dv = gpu.array(V.astype(np.float32))
    gpu.kv_write(kc, vc, kvd, n_ctx, 0, dk, dv, n_ctx)
    dq = gpu.array(q)
    dpos = gpu.array(np.array([pos], np.uint32))
    out = gpu.empty(M * n_head * hd, np.float32)
    if before:
        before()
    gpu.attention(out, dq, kc, vc, n_head, n_kv, hd, M, dpos, n_ctx, mode)
    gpu.sync()
    return out.numpy().reshape(M, n_head * hd)


CASES = [  # n_head, n_kv, hd, n_ctx, pos, M
    (32, 8, 128, 700, 650, 1),     # 4B/8B head shape, long chain with a ragged tail
    (32, 16, 128, 300, 299, 1),    # 27B head shape, last row of the cache
    (8, 8, 64, 130, 100, 4),       # no GQA, 4 tokens at consecutive positions
    (6, 6, 48, 77, 70, 1),         # tiny-288 heads
    (4, 1, 128, 64, 0, 1),         # a single visible row
    (16, 2, 128, 257, 200, 8),     # 8 tokens (verify batch), gqa 8
    (12, 4, 64, 100, 99, 1),       # gqa 3: softmax and values in launches of their own
    (8, 2, 64, 6000, 5990, 2),     # weights leave room for few product stages (4)
    (8, 2, 64, 9000, 8990, 2),     # two tokens: softmax and values in launches of their own
    # one token, scores in the same launch: several rounds of score tiles per
    # workgroup, partial chunks, workgroups without tiles
    (8, 8, 128, 1200, 1150, 1),    # gqa 1: two slices, 9 tiles each (3 rounds)
    (4, 1, 64, 3000, 2999, 1),     # gqa 4, hd 64: 12 tiles per slice
    (16, 2, 256, 500, 499, 1),     # gqa 8, hd 256: 32 slices for 8 tiles, two tiles a round
    (6, 6, 48, 400, 399, 1),       # hd 48: the second chunk partly filled
    (32, 8, 128, 2200, 2048, 1),   # 4B/8B heads past 2048 rows: 33 score tiles a kv head
    (32, 8, 128, 4200, 4150, 1),   # 66 tiles a kv head
    (32, 16, 128, 700, 699, 1),    # 27B heads, 16 kv heads, near the last row
    (8, 2, 128, 200, 127, 5),      # 5 tokens: a score tile first reached by the second token
    (16, 4, 64, 300, 250, 7),      # 7 tokens: four to a score workgroup, then three
    # several tokens: a softmax workgroup per (head, token), then value
    # workgroups of four tokens whose chains end at different positions
    (32, 8, 128, 2200, 2048, 8),   # 4B/8B heads, 8 tokens
    (32, 16, 128, 1100, 1000, 8),  # 27B heads, 8 tokens, gqa 2
    (32, 8, 128, 300, 295, 5),     # 5 tokens up to the cache end (the last group of one)
    (12, 4, 64, 500, 450, 3),      # gqa 3 (heads padded to 4), 3 tokens
    (12, 2, 64, 300, 280, 6),      # gqa 6 (heads padded to 8), 6 tokens
    (8, 8, 64, 1000, 190, 8),      # tokens ending on both sides of a value block (192 positions)
    (6, 6, 40, 120, 100, 2),       # hd 40: the last 16 columns of a head partly past its end
    (4, 2, 4, 32, 20, 3),          # hd 4 (the tiny fixture's heads): 8 columns per group
    (6, 6, 40, 120, 100, 1),       # one token, hd 40: a head's last column group partly past its end
    (4, 2, 4, 32, 20, 1),          # one token, hd 4
    (12, 4, 64, 3000, 2500, 1),    # one token, gqa 3 past several exp blocks
    # one token on either side of the largest context that takes 768-position
    # value blocks (16,000 weights beside their product buffers)
    (8, 2, 128, 16000, 15999, 1),  # 768-position value blocks, 21 of them, the last ragged
    (8, 2, 128, 16032, 16031, 1),  # 384-position value blocks
    # one token past the fused kernel's LDS: the two-launch path
    (16, 2, 128, 16400, 16399, 1), # gqa 8, 257 score tiles
    (8, 8, 64, 20000, 19990, 1),   # gqa 1, 20000 positions
    (4, 1, 64, 32768, 32767, 1),   # the longest context exact mode takes
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "h%d_kv%d_d%d_ctx%d_p%d_m%d" % c)
def test_attention_exact_is_bit_identical(gpu, oracle, case):
    n_head, n_kv, hd, n_ctx, pos, M = case
    rng = np.random.default_rng(sum(case))
    q = (rng.standard_normal((M, n_head * hd)) * 0.3).astype(np.float32)
    K = rng.standard_normal((n_ctx, n_kv * hd)).astype(np.float32)
    V = rng.standard_normal((n_ctx, n_kv * hd)).astype(np.float32)
    got = run_gpu(gpu, q, K, V, n_head, n_kv, hd, pos, M, n_ctx, rf.ATTN_EXACT)
    want = reference_attention(oracle, q, K, V, n_head, n_kv, hd, pos, M, n_ctx)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"max abs diff {np.abs(got - want).max()}"


# head_dim 256 (the largest taken) in split mode: two load rounds per workgroup,
# two column-quad passes in the merge
SPLIT_CASES = CASES + [(16, 2, 256, 700, 650, 2)]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=lambda c: "h%d_kv%d_d%d_ctx%d_p%d_m%d" % c)
def test_attention_split_within_rounding(gpu, oracle, case):
    n_head, n_kv, hd, n_ctx, pos, M = case
    rng = np.random.default_rng(7 + sum(case))
    q = (rng.standard_normal((M, n_head * hd)) * 0.3).astype(np.float32)
    K = rng.standard_normal((n_ctx, n_kv * hd)).astype(np.float32)
    V = rng.standard_normal((n_ctx, n_kv * hd)).astype(np.float32)
    got = run_gpu(gpu, q, K, V, n_head, n_kv, hd, pos, M, n_ctx, rf.ATTN_SPLIT)
    want = reference_attention(oracle, q, K, V, n_head, n_kv, hd, pos, M, n_ctx)
    err = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert err < 1e-5, err


@pytest.mark.parametrize("case", [(4, 2, 64, 40, 39, 1), (32, 8, 128, 300, 290, 8)],
                         ids=["one_token", "several_tokens"])
def test_nan_first_score_follows_the_reference(gpu, oracle, case):
    """src/ops.c:26-30: a NaN score at position 0 stays the maximum, so every
    weight of that head is NaN and the sum is not normalised; a NaN later in
    the row is skipped by the maximum.  Other heads are unaffected.  The
    second case runs the softmax in a launch of its own."""
    n_head, n_kv, hd, n_ctx, pos, M = case
    rng = np.random.default_rng(5)
    q = (rng.standard_normal((M, n_head * hd)) * 0.3).astype(np.float32)
    K = rng.standard_normal((n_ctx, n_kv * hd)).astype(np.float32)
    V = rng.standard_normal((n_ctx, n_kv * hd)).astype(np.float32)
    K[0, 0] = np.nan            # kv head 0: its query heads get a NaN first score
    got = run_gpu(gpu, q, K, V, n_head, n_kv, hd, pos, M, n_ctx, rf.ATTN_EXACT)
    want = reference_attention(oracle, q, K, V, n_head, n_kv, hd, pos, M, n_ctx)
    nh0 = (n_head // n_kv) * hd
    assert np.isnan(want[:, :nh0]).all() and np.isnan(got[:, :nh0]).all()
    assert np.array_equal(got[:, nh0:].view(np.uint32), want[:, nh0:].view(np.uint32))


def test_exact_mode_rejects_contexts_beyond_its_limit(gpu):
    """Exact mode keeps one head's weights in LDS: a longer cache is refused
    before anything is launched."""
    n_head, n_kv, hd, n_ctx = 4, 1, 64, 32772
    kc = gpu.empty(n_ctx * n_kv * hd, np.float32)
    vc = gpu.empty(n_ctx * n_kv * hd, np.float32)
    dq = gpu.empty(n_head * hd, np.float32)
    dpos = gpu.array(np.array([0], np.uint32))
    out = gpu.empty(n_head * hd, np.float32)
    with pytest.raises(rf.FoxError):
        gpu.attention(out, dq, kc, vc, n_head, n_kv, hd, 1, dpos, n_ctx, rf.ATTN_EXACT)


@pytest.mark.parametrize("hd, n_ctx", [(128, 65536 + 64), (64, 32768 + 32)],
                         ids=["hd128_65600", "hd64_32800"])
def test_split_mode_rejects_contexts_beyond_its_limit(gpu, hd, n_ctx):
    """The merge holds 1024 splits (64 positions each at head_dim 128, 32
    otherwise): a longer cache is refused before anything is launched."""
    n_head, n_kv = 4, 1
    kc = gpu.empty(n_ctx * n_kv * hd, np.float32)
    vc = gpu.empty((n_ctx + 3) // 4 * 4 * n_kv * hd, np.float32)
    dq = gpu.empty(n_head * hd, np.float32)
    dpos = gpu.array(np.array([0], np.uint32))
    out = gpu.empty(n_head * hd, np.float32)
    with pytest.raises(rf.FoxError):
        gpu.attention(out, dq, kc, vc, n_head, n_kv, hd, 1, dpos, n_ctx, rf.ATTN_SPLIT)


def _in_order(acc, e):
    """acc + e_0 + e_1 + ..., one float32 add at a time (src/ops.c:31-33)."""
    s = np.float32(acc)
    with np.errstate(all="ignore"):
        for x in e:
            s = np.float32(s + x)
    return s


def _sum_inputs():
    rng = np.random.default_rng(31)
    cases = []
    for n in (1, 3, 255, 256, 257, 2061, 8192):
        for sig in (0.5, 2.0, 8.0):
            s = rng.normal(0, sig, n)
            cases.append((f"softmax n={n} sigma={sig}", 0.0,
                          np.exp(s - s.max()).astype(np.float32)))
    n = 2000
    k, m = rng.integers(1, 8, n), rng.integers(8, 22, n)
    cases.append(("exact ties of small multiples of powers of two", 0.0,
                  np.ldexp(k.astype(np.float32), -m).astype(np.float32)))
    cases.append(("ties at a sum past 2^24", 2.0 ** 24, rng.integers(0, 8, n).astype(np.float32)))
    cases.append(("ties of halves past 2^23", 2.0 ** 23,
                  (rng.integers(0, 8, n) * 0.5).astype(np.float32)))
    # e/u = k 2^(23-m) against a sum near 1: for m = 24..26 most elements
    # are ties, several to a lane, whose rounding follows the running parity
    for bits in (1, 6, 12):
        k, m = rng.integers(1, 2 ** bits, 3000), rng.integers(18, 27, 3000)
        cases.append((f"dense ties at the sum's own scale, {bits}-bit multiples", 1.0,
                      np.ldexp(k.astype(np.float32), -m).astype(np.float32)))
    s = rng.normal(0, 6.0, 3000)
    cases.append(("a peaked softmax after a sum of 1", 1.0, np.exp(s - s.max()).astype(np.float32)))
    cases.append(("thirty decades", 0.0, (10.0 ** rng.uniform(-30, 0, n)).astype(np.float32)))
    z = rng.uniform(0, 1, n).astype(np.float32)
    z[rng.random(n) < 0.3] = 0.0
    z[rng.random(n) < 0.1] = np.float32(1e-40)
    cases.append(("zeros and subnormals", 0.0, z))
    cases.append(("a subnormal start", 1e-40, rng.uniform(0, 1e-38, n).astype(np.float32)))
    cases.append(("negative elements", 0.25, rng.uniform(-1, 1, 600).astype(np.float32)))
    x = rng.uniform(0, 1, 600).astype(np.float32)
    x[300] = np.nan
    cases.append(("a NaN element", 0.0, x))
    x = rng.uniform(0, 1, 600).astype(np.float32)
    x[200] = np.inf
    cases.append(("an infinite element", 0.0, x))
    cases.append(("no elements", 0.5, np.zeros(0, np.float32)))
    return cases


@pytest.mark.parametrize("name,acc,e", _sum_inputs(), ids=lambda v: v if isinstance(v, str) else "")
def test_softmax_sum_in_order_is_the_chain(gpu, name, acc, e):
    """The attention kernels' softmax sum, formed a wave at a time from
    integer sums over runs that stay in one binade, equals the one add at a
    time chain bit for bit, on inputs that hit its events: binade
    crossings, exact ties (whose rounding depends on the sum so far), zeros,
    subnormals, negative, infinite and NaN elements."""
    print(f"case sum_in_order {name} n={e.size}", flush=True)
    de = gpu.array(e if e.size else np.zeros(1, np.float32))
    out = gpu.array(np.full(4, np.nan, np.float32))
    gpu.sum_probe(de, int(e.size), float(acc), out)
    gpu.sync()
    res, want = out.numpy(), _in_order(acc, e)
    for got, what in ((res[0], "whole-wave sum"), (res[2], "chain")):
        assert (np.isnan(got) and np.isnan(want)) or got.view(np.uint32) == want.view(np.uint32), \
            f"{name}, {what}: got {got!r} want {want!r}"
    print(f"  clocks: whole-wave {res[1]:.0f}, chain {res[3]:.0f}", flush=True)
