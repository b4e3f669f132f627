"""The reference's operator entry points (include/fox/fox.h:322-368) exported
by libfox.so with their own signatures, on host buffers, computed on the
GPU, called through ctypes as a C caller of the reference would call them.

test_reference_gemv_test_replayed runs every check of the reference's own
tests/test_gemv.c:51-152 (quantiser known answers; the 37 x 512 TQ2_0 GEMV
with xorshift32 seed 0xC0FFEE and d = 1.0; serial == pooled == per-row
dot; argument errors; f32 entry == i8 entry) and then compares the GEMV
with the oracle bit for bit.  The others check fox_gemv for every device
type, the TQ1_0 known answers of tests/test_ternary.c:100-136 through
fox_tq1_dot_i8 and fox_dequant_row against the oracle (every f16 bit
pattern, Q4_K and Q6_K blocks).
"""
import ctypes as C

import numpy as np
import pytest

import rustfox_amd as rf
from test_gpu_gemv import weights, bits

pytestmark = pytest.mark.gpu

vp, sz = C.c_void_p, C.c_size_t
f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
PFN = C.CFUNCTYPE(None, vp, C.c_int, sz, sz)


@pytest.fixture(scope="module")
def L():
    L = rf.host_lib()
    L.fox_threadpool_create.argtypes = [C.c_int]
    L.fox_threadpool_create.restype = vp
    L.fox_threadpool_destroy.argtypes = [vp]
    L.fox_threadpool_destroy.restype = None
    L.fox_threadpool_size.argtypes = [vp]
    L.fox_parallel_for.argtypes = [vp, sz, PFN, vp]
    L.fox_quantize_activations_i8.argtypes = [f32p, sz, i8p, C.POINTER(C.c_float)]
    for n in ("fox_gemv_tq1_i8", "fox_gemv_tq2_i8"):
        getattr(L, n).argtypes = [vp, vp, C.c_float, vp, sz, sz, vp]
    for n in ("fox_gemv_tq1_f32", "fox_gemv_tq2_f32"):
        getattr(L, n).argtypes = [vp, f32p, u8p, sz, sz, f32p]
    for n in ("fox_tq1_dot_i8", "fox_tq2_dot_i8", "fox_tq1_dot_i8_scalar",
              "fox_tq2_dot_i8_scalar"):
        getattr(L, n).argtypes = [i8p, u8p, sz, C.POINTER(C.c_float)]
    L.fox_gemv.argtypes = [vp, C.c_int, f32p, u8p, sz, sz, f32p]
    L.fox_dequant_row.argtypes = [C.c_int, u8p, sz, f32p]
    return L


def xorshift32(state):
    x = state[0]
    x ^= (x << 13) & 0xFFFFFFFF
    x ^= x >> 17
    x ^= (x << 5) & 0xFFFFFFFF
    state[0] = x
    return x


def ptr(a):
    return a.ctypes.data_as(vp) if a is not None else None


def test_reference_gemv_test_replayed(L, oracle):
    ROWS, COLS = 37, 512
    row_bytes = COLS // 256 * 66
    tp = L.fox_threadpool_create(4)
    assert tp
    assert L.fox_threadpool_size(tp) >= 1
    assert L.fox_threadpool_size(None) == 1

    def coverage_is_exact(pool, n):
        hits = np.zeros(max(n, 1), np.int32)

        def mark(ctx, worker, begin, end):
            hits[begin:end] += 1
        assert L.fox_parallel_for(pool, n, PFN(mark), None) == 0
        return bool(np.all(hits[:n] == 1))
    for n in (1000, 1, 3, 4097):
        assert coverage_is_exact(tp, n)
    assert coverage_is_exact(None, 500)
    assert L.fox_parallel_for(tp, 0, PFN(lambda *a: None), None) == 0
    assert L.fox_parallel_for(tp, 10, C.cast(None, PFN), None) == 1

    q = np.empty(COLS, np.int8)
    scale = C.c_float(-1.0)
    x = np.zeros(COLS, np.float32)
    assert L.fox_quantize_activations_i8(x, COLS, q, C.byref(scale)) == 0
    assert scale.value == 0.0 and q[0] == 0 and q[-1] == 0
    x = (np.arange(COLS, dtype=np.float32) - np.float32(200.0)).astype(np.float32)
    assert L.fox_quantize_activations_i8(x, COLS, q, C.byref(scale)) == 0
    assert scale.value > 0.0
    assert q.min() >= -127 and q.max() <= 127 and q[-1] == 127
    wq, ws = oracle.quantize(x)
    assert np.array_equal(q, wq) and bits(np.float32(scale.value)) == bits(np.float32(ws))

    seed = [0xC0FFEE]
    w = np.array([xorshift32(seed) & 0xFF for _ in range(ROWS * row_bytes)], np.uint8)
    blk = w.reshape(ROWS, COLS // 256, 66)
    blk[:, :, 64] = 0x00
    blk[:, :, 65] = 0x3C
    x = np.array([np.float32((xorshift32(seed) & 0xFF) - 128) * np.float32(0.01)
                  for _ in range(COLS)], np.float32)
    assert L.fox_quantize_activations_i8(x, COLS, q, C.byref(scale)) == 0
    s = scale.value
    serial = np.empty(ROWS, np.float32)
    parallel = np.empty(ROWS, np.float32)
    assert L.fox_gemv_tq2_i8(None, ptr(q), s, ptr(w), ROWS, COLS, ptr(serial)) == 0
    assert L.fox_gemv_tq2_i8(tp, ptr(q), s, ptr(w), ROWS, COLS, ptr(parallel)) == 0
    assert np.array_equal(bits(serial), bits(parallel))
    direct = np.empty(ROWS, np.float32)
    for r in range(ROWS):
        acc = C.c_float(0.0)
        assert L.fox_tq2_dot_i8(q, w[r * row_bytes:(r + 1) * row_bytes].copy(), COLS,
                                C.byref(acc)) == 0
        direct[r] = np.float32(acc.value) * np.float32(s)
    assert np.array_equal(bits(direct), bits(serial))
    assert L.fox_gemv_tq2_i8(tp, ptr(q), s, ptr(w), ROWS, 255, ptr(serial)) == 1
    assert L.fox_gemv_tq2_i8(tp, None, s, ptr(w), ROWS, COLS, ptr(serial)) == 1
    assert L.fox_gemv_tq2_i8(tp, ptr(q), s, None, ROWS, COLS, ptr(serial)) == 1
    assert L.fox_gemv_tq2_i8(tp, ptr(q), s, ptr(w), 0, COLS, ptr(serial)) == 1
    parallel[:] = 0
    assert L.fox_gemv_tq2_f32(tp, x, w, ROWS, COLS, parallel) == 0
    assert np.array_equal(bits(parallel), bits(direct))
    want = oracle.gemv_tq_i8(35, q, np.float32(s), w, ROWS, COLS)
    assert np.array_equal(bits(direct), bits(want))
    L.fox_threadpool_destroy(tp)
    L.fox_threadpool_destroy(None)


@pytest.mark.parametrize("tname,gtype,N,K", [("TQ1_0", 34, 100, 2560), ("TQ2_0", 35, 64, 1024),
                                             ("Q4_K", 12, 48, 4096), ("Q6_K", 14, 40, 2048),
                                             ("F16", 1, 50, 288), ("F32", 0, 9, 64)])
def test_fox_gemv_every_type(L, oracle, tname, gtype, N, K):
    rng = np.random.default_rng([N, K, gtype, 77])
    w = weights(rng, gtype, N, K)
    x = rng.standard_normal(K).astype(np.float32)
    out = np.empty(N, np.float32)
    assert L.fox_gemv(None, gtype, x, w, N, K, out) == 0, L.fox_last_error()
    assert np.array_equal(bits(out), bits(oracle.gemv(gtype, x, w, N, K)))
    if gtype in (34, 35):
        f = L.fox_gemv_tq1_f32 if gtype == 34 else L.fox_gemv_tq2_f32
        out2 = np.empty(N, np.float32)
        assert f(None, x, w, N, K, out2) == 0
        assert np.array_equal(bits(out2), bits(out))
        qq, sc = oracle.quantize(x)
        g = L.fox_gemv_tq1_i8 if gtype == 34 else L.fox_gemv_tq2_i8
        out3 = np.empty(N, np.float32)
        assert g(None, ptr(qq), sc, ptr(w), N, K, ptr(out3)) == 0
        assert np.array_equal(bits(out3), bits(out))


def test_unsupported_type_is_named(L):
    x = np.zeros(256, np.float32)
    out = np.zeros(4, np.float32)
    assert L.fox_gemv(None, 10, x, np.zeros(84 * 4, np.uint8), 4, 256, out) == 5   # Q2_K
    assert b"Q2_K" in L.fox_last_error() or b"type" in L.fox_last_error()


def test_tq1_dot_known_answers(L):
    """tests/test_ternary.c:100-136: bytes 255 (qs) / 253 (qh) decode to all
    +1 and byte 0 to all -1; with all-one activations and d = 1 the dot of
    two blocks is +512 / -512."""
    plus = np.zeros(54, np.uint8)
    plus[:48] = 255
    plus[48:52] = 253
    plus[52:54] = [0x00, 0x3C]
    minus = np.zeros(54, np.uint8)
    minus[52:54] = [0x00, 0x3C]
    ones = np.ones(512, np.int8)
    for blk, want in ((plus, 512.0), (minus, -512.0)):
        for f in (L.fox_tq1_dot_i8, L.fox_tq1_dot_i8_scalar):
            out = C.c_float(0.0)
            assert f(ones, np.tile(blk, 2), 512, C.byref(out)) == 0
            assert out.value == want
    out = C.c_float(0.0)
    assert L.fox_tq1_dot_i8(ones, np.tile(plus, 2), 300, C.byref(out)) == 1   # ragged n
    assert L.fox_tq2_dot_i8(ones, np.zeros(66, np.uint8), 0, C.byref(out)) == 1


@pytest.mark.parametrize("tname,gtype,n", [("F16", 1, 65536), ("F32", 0, 1000),
                                           ("Q4_K", 12, 4096), ("Q6_K", 14, 4096),
                                           ("Q8_0", 8, 4096), ("Q4_0", 2, 4096),
                                           ("Q5_K", 13, 4096)])
def test_dequant_row_equals_the_oracle(L, oracle, tname, gtype, n):
    rng = np.random.default_rng([n, gtype])
    if gtype == 1:
        row = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.uint8)   # every f16
    elif gtype == 0:
        row = rng.standard_normal(n).astype(np.float32).view(np.uint8)
    elif gtype in (8, 2, 13):
        bb, offs, be = {8: (34, [0], 32), 2: (18, [0], 32), 13: (176, [0, 2], 256)}[gtype]
        blk = rng.integers(0, 256, (n // be, bb), dtype=np.uint8)
        for o in offs:
            blk[:, o:o + 2] = rng.uniform(-0.1, 0.1, n // be).astype(np.float16).view(
                np.uint8).reshape(-1, 2)
        row = blk.reshape(-1)
    else:
        row = weights(rng, gtype, 1, n)
    out = np.empty(n, np.float32)
    assert L.fox_dequant_row(gtype, row, n, out) == 0, L.fox_last_error()
    want = oracle.dequant(gtype, row, n)
    assert np.array_equal(bits(out), bits(want)), tname
    assert L.fox_dequant_row(34, np.zeros(54, np.uint8), 256, out) == 5   # no TQ decoder
    assert L.fox_dequant_row(gtype if gtype > 1 else 12, row, 100, out) == 1   # ragged
