"""Device ops beside the GEMVs and attention, against the oracle."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _argmax_cases():
    rng = np.random.default_rng(11)
    big = rng.standard_normal(151936).astype(np.float32)
    tie = big.copy()
    tie[[777, 9000, 150000]] = 50.0                    # first of equal maxima wins
    nan0 = big.copy()
    nan0[0] = np.nan                                   # a NaN at index 0 stays
    nans = big.copy()
    nans[rng.integers(1, big.size, 500)] = np.nan      # NaN elsewhere never wins
    neg = np.full(5000, -np.inf, np.float32)           # nothing beats x[0]
    first = big.copy()
    first[0] = 100.0
    small = rng.standard_normal(7).astype(np.float32)
    return dict(big=big, tie=tie, nan0=nan0, nans=nans, neg=neg, first=first, small=small)


@pytest.mark.parametrize("name", list(_argmax_cases()))
def test_argmax_follows_the_reference(gpu, oracle, name):
    """src/sample.c:147-153 through the multi-workgroup reduction; the
    device position advances and the history records the choice."""
    x = _argmax_cases()[name]
    idx = gpu.empty(1, np.uint32)
    pos = gpu.array(np.array([3], np.uint32))
    hist = gpu.array(np.zeros(8, np.uint32))
    dx = gpu.array(x)
    for _ in range(2):
        gpu.argmax(dx, x.size, idx)
    gpu.argmax(dx, x.size, idx, pos, 1, hist)
    gpu.sync()
    want = oracle.argmax(x)
    assert int(idx.numpy()[0]) == want
    assert int(pos.numpy()[0]) == 4 and int(hist.numpy()[3]) == want


def test_argmax_sees_this_launchs_partials(gpu, oracle):
    """Back-to-back argmax launches whose maxima sit in different partial
    ranges: every result must come from its own input.  (A single launch
    whose last workgroup merged the other workgroups' partials read a
    partial of the previous launch now and then and returned the runner-up
    range's maximum.)  Two inputs alternate: A has a large value in one
    range and its maximum in another range, B the reverse, so that any
    partial carried over from the other input changes the answer."""
    rng = np.random.default_rng(5)
    n = 151936
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    a[77700], a[95832] = 9.0, 8.5                      # A: max at 77700, runner-up 95832
    b[77700], b[95832] = 8.0, 8.75                     # B: max at 95832, 77700 below it
    want = [oracle.argmax(a), oracle.argmax(b)]
    assert want == [77700, 95832]
    da, db = gpu.array(a), gpu.array(b)
    steps = 64
    idx = gpu.empty(1, np.uint32)
    pos = gpu.array(np.array([0], np.uint32))
    hist = gpu.array(np.zeros(steps, np.uint32))
    for s in range(steps):
        gpu.argmax(da if s % 2 == 0 else db, n, idx, pos, 1, hist)
    gpu.sync()
    got = hist.numpy()
    assert [int(v) for v in got] == [want[s % 2] for s in range(steps)]
    assert int(pos.numpy()[0]) == steps


# sizes that reach every register-held variant of the kernel (256 R >= n for
# R = 2 .. 16) and the strided loop past 4096
_RMS_N = [1, 7, 288, 512, 1000, 1536, 2048, 2560, 3072, 4096, 4097, 9728]


@pytest.mark.parametrize("n", _RMS_N)
def test_rmsnorm_bit_exact(gpu, oracle, n):
    """src/ops.c:7-22 (double sum of squares in index order, two float
    roundings): three rows at a padded stride, with and without weights."""
    rng = np.random.default_rng(n)
    M, stride = 3, n + 5
    x = np.zeros((M, stride), np.float32)
    x[:, :n] = rng.standard_normal((M, n)).astype(np.float32) * np.float32(3.0)
    x[1, :n] *= np.float32(1e-3)                       # a small-norm row
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    dx, dw = gpu.array(x), gpu.array(w)
    for weighted in (True, False):
        dout = gpu.array(np.full((M, stride), 7.0, np.float32))
        gpu.rmsnorm(dout, dx, dw if weighted else None, n, M, EPS, stride, stride)
        gpu.sync()
        got = dout.numpy()
        for t in range(M):
            want = oracle.rmsnorm(x[t, :n], w if weighted else np.ones(n, np.float32), EPS)
            assert np.array_equal(got[t, :n].view(np.uint32), want.view(np.uint32)), (t, weighted)
            assert np.all(got[t, n:] == 7.0)           # nothing past n is written
