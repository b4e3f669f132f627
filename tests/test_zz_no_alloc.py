"""fox_gpu_gemv_noalloc (the entry point that allocates nothing) against
fox_gpu_gemv, through the C ABI: bit-identical outputs on two calls in a
row, the second with a smaller input, for weights whose GEMV uses the
scratch (Q4_K, Q6_K; TQ1_0 with 8 tokens of 21504 values or 2 of 24576,
more than the fused path holds; fused TQ1_0 from three tokens on, whose
input is quantised once per launch into the scratch) and for one that needs
none (fused TQ1_0, one token).  The no-alloc calls run first, on a fresh
context, and must leave
its workspace exactly as it was; fox_gpu_gemv runs afterwards on the same
context for the expected outputs."""
import numpy as np
import pytest

import rustfox_amd as rf
from test_gpu_gemv import weights, bits

pytestmark = pytest.mark.gpu


def noalloc(gpu, t, x, M, out, flags=0):
    st = gpu.lib.fox_gpu_gemv_noalloc(gpu.ctx, t.h, x.ptr, t.ne0, M, out.ptr, t.ne1, flags)
    if st:
        raise rf.FoxError(st, gpu.lib.fox_gpu_last_error().decode())


@pytest.mark.parametrize("tname,gtype,first,second", [
    ("Q4_K", 12, (4096, 14336, 8), (1024, 2048, 3)),
    ("Q6_K", 14, (14336, 4096, 8), (512, 1024, 1)),
    ("TQ1_0", 34, (21504, 5376, 8), (24576, 300, 2)),
    ("TQ1_0", 34, (4096, 14336, 8), (2560, 640, 3)),
    ("TQ1_0", 34, (2560, 4096, 1), (512, 64, 1)),
])
def test_noalloc_equals_gemv(tname, gtype, first, second):
    rng = np.random.default_rng([gtype, first[0], 3])
    with rf.Gpu(0) as g:
        ws0 = g.workspace_bytes()
        cases = []
        for K, N, M in (first, second):
            print(f"case noalloc {tname} K={K} N={N} M={M}", flush=True)
            w = weights(rng, gtype, N, K)
            t = g.tensor(gtype, K, N, w)
            x = g.array(rng.standard_normal((M, K)).astype(np.float32))
            base = rng.standard_normal((M, N)).astype(np.float32)
            b = g.array(base)
            noalloc(g, t, x, M, b, rf.GEMV_ACCUMULATE)
            assert g.workspace_bytes() == ws0, "the no-alloc call grew the workspace"
            cases.append((t, x, M, base, b))
        for t, x, M, base, b in cases:
            a = g.array(base)
            g.gemv(t, x, M, a, flags=rf.GEMV_ACCUMULATE)
            assert np.array_equal(bits(a.numpy()), bits(b.numpy())), (t.ne0, t.ne1, M)
            for arr in (a, b, x, t):
                arr.free()
