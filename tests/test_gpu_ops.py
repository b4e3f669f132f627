"""Device ops beside the GEMVs and attention, against the oracle."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


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
    for _ in range(2):                                 # the counter resets itself
        gpu.argmax(dx, x.size, idx)
    gpu.argmax(dx, x.size, idx, pos, 1, hist)
    gpu.sync()
    want = oracle.argmax(x)
    assert int(idx.numpy()[0]) == want
    assert int(pos.numpy()[0]) == 4 and int(hist.numpy()[3]) == want
