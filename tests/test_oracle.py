"""Pin the oracle (oracle/fox_oracle.c) before trusting it to judge the GPU path.

Each function is checked by something that would catch a plausible mistake
(a dropped term, a wrong index, a transposed operand):
  * known answers of the reference's own tests (tests/test_ternary.c,
    tests/test_gemv.c, tests/test_kernels.c);
  * textbook decoders written here from the format description, not from
    the reference's arithmetic (base-3 digits instead of the fixed-point
    trick, element-by-element nibble unpacking);
  * the committed golden fixtures (tests/golden/, written by the reference);
  * the reference compiled from its own sources (oracle/_ref), bit for bit
    on seeded inputs, where it was built.
"""
import hashlib
import os
import tempfile

import numpy as np
import pytest

from rustfox_amd import synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------- textbook

def tq1_trits(block: np.ndarray) -> np.ndarray:
    """TQ1_0 block -> 256 weights in {-1,0,1}: each byte holds the base-3
    digits (most significant first) of V = floor(b * 243 / 256)."""
    out = np.empty(256, np.int32)

    def digits(b, n):
        v = (int(b) * 243) // 256
        ds = []
        for _ in range(5):
            ds.append(v % 3)
            v //= 3
        return ds[::-1][:n]            # level 0 is the most significant digit

    for m in range(32):
        for l, d in enumerate(digits(block[m], 5)):
            out[l * 32 + m] = d - 1
    for m in range(16):
        for l, d in enumerate(digits(block[32 + m], 5)):
            out[160 + l * 16 + m] = d - 1
    for m in range(4):
        for l, d in enumerate(digits(block[48 + m], 4)):
            out[240 + l * 4 + m] = d - 1
    return out


def tq2_trits(block):
    out = np.empty(256, np.int32)
    for i in range(256):
        half, rest = divmod(i, 128)
        level, m = divmod(rest, 32)
        out[i] = ((int(block[half * 32 + m]) >> (2 * level)) & 3) - 1
    return out


def f16(b, o):
    return np.frombuffer(bytes(b[o:o + 2]), np.float16)[0].astype(np.float32)


def q4k_values(blk):
    """(nibble, sub-block) per element from the block layout description."""
    sc_raw = blk[4:16].astype(np.int32)
    sc, mn = np.zeros(8, np.int32), np.zeros(8, np.int32)
    for j in range(8):
        if j < 4:
            sc[j], mn[j] = sc_raw[j] & 63, sc_raw[j + 4] & 63
        else:
            sc[j] = (sc_raw[j + 4] & 15) | ((sc_raw[j - 4] >> 6) << 4)
            mn[j] = (sc_raw[j + 4] >> 4) | ((sc_raw[j] >> 6) << 4)
    nib = np.empty(256, np.int32)
    for i in range(256):
        p, r = divmod(i, 64)
        byte = int(blk[16 + 32 * p + (r % 32)])
        nib[i] = (byte >> 4) if r >= 32 else (byte & 15)
    return nib, sc, mn


def q6k_values(blk):
    q = np.empty(256, np.int32)
    scale_idx = np.empty(256, np.int32)
    for i in range(256):
        h, r = divmod(i, 128)
        grp, l = divmod(r, 32)
        lo_byte = int(blk[64 * h + l + (32 if grp in (1, 3) else 0)])
        lo = (lo_byte >> 4) if grp >= 2 else (lo_byte & 15)
        hi = (int(blk[128 + 32 * h + l]) >> (2 * grp)) & 3
        q[i] = (lo | (hi << 4)) - 32
        scale_idx[i] = 8 * h + l // 16 + 2 * grp
    return q, scale_idx


# ------------------------------------------------------------- known answers

def test_tq1_closed_forms(oracle):
    """tests/test_ternary.c:112-136"""
    blk = np.zeros(54, np.uint8)
    blk[:48], blk[48:52], blk[52:54] = 255, 253, [0x00, 0x3C]
    ones = np.ones(256, np.int8)
    assert oracle.lib.or_tq1_block_sum(ones, blk) == 256
    blk[:52] = 0
    assert oracle.lib.or_tq1_block_sum(ones, blk) == -256


def test_tq1_textbook_all_bytes(oracle):
    """Every byte value at every level, through one-hot activations."""
    rng = np.random.default_rng(0)
    for trial in range(24):
        blk = rng.integers(0, 256, 54, dtype=np.uint8)
        want = tq1_trits(blk)
        for e in range(256):
            q = np.zeros(256, np.int8)
            q[e] = 1
            assert oracle.lib.or_tq1_block_sum(q, blk) == want[e], (trial, e)


def test_tq1_tq2_random_sums_vs_textbook(oracle):
    rng = np.random.default_rng(1)
    for _ in range(200):
        q = rng.integers(-127, 128, 256, dtype=np.int8)
        b1 = rng.integers(0, 256, 54, dtype=np.uint8)
        b2 = rng.integers(0, 256, 66, dtype=np.uint8)
        assert oracle.lib.or_tq1_block_sum(q, b1) == int(tq1_trits(b1) @ q.astype(np.int32))
        assert oracle.lib.or_tq2_block_sum(q, b2) == int(tq2_trits(b2) @ q.astype(np.int32))


def test_tq1_encoder_round_trip():
    """synth's encoder (ceil(V * 256/243)) decodes back to the same trits,
    for every 5-trit and 4-trit value."""
    rng = np.random.default_rng(2)
    t = rng.integers(-1, 2, size=(64, 256))
    t[0, :160] = np.repeat(np.arange(32) % 3 - 1, 5)
    blocks = synth.tq1_encode(t, np.full(64, 0.03))
    for i in range(64):
        assert np.array_equal(tq1_trits(blocks[i]), t[i])
    for v in range(243):
        b = synth.tq1_pack_value(np.array([v]))[0]
        assert (int(b) * 243) // 256 == v


def test_q4k_q6k_sums_vs_textbook(oracle):
    rng = np.random.default_rng(3)
    for _ in range(40):
        q = rng.integers(-127, 128, 256, dtype=np.int8)
        blk4 = rng.integers(0, 256, 144, dtype=np.uint8)
        nib, _, _ = q4k_values(blk4)
        d = np.zeros(8, np.int32)
        s = np.zeros(8, np.int32)
        oracle.lib.or_q4k_block_sums(q, blk4, d.ctypes.data, s.ctypes.data)
        qi = q.astype(np.int32)
        for j in range(8):
            assert d[j] == int(nib[32 * j:32 * j + 32] @ qi[32 * j:32 * j + 32])
            assert s[j] == int(qi[32 * j:32 * j + 32].sum())
        blk6 = rng.integers(0, 256, 210, dtype=np.uint8)
        q6, sidx = q6k_values(blk6)
        sc = blk6[192:208].view(np.int8).astype(np.int32)
        g = np.zeros(4, np.int32)
        oracle.lib.or_q6k_block_sums(q, blk6, g.ctypes.data)
        for h in range(2):
            for sub in range(2):
                want = 0
                for grp in range(4):
                    idx = [128 * h + 32 * grp + 16 * sub + l for l in range(16)]
                    want += int(sc[sidx[idx[0]]]) * int(q6[idx] @ qi[idx])
                assert g[2 * h + sub] == want


def test_dequant_vs_textbook(oracle):
    """One-hot layout probes of tests/test_kernels.c:157-184, here against
    the element-by-element decoders above."""
    rng = np.random.default_rng(4)
    blk4 = rng.integers(0, 256, 144, dtype=np.uint8)
    blk4[0:2] = [0x00, 0x3C]
    blk4[2:4] = [0x00, 0x38]
    nib, sc, mn = q4k_values(blk4)
    want4 = np.array([np.float32(np.float32(1.0) * np.float32(sc[i // 32])) * np.float32(nib[i])
                      - np.float32(np.float32(0.5) * np.float32(mn[i // 32]))
                      for i in range(256)], np.float32)
    assert np.array_equal(bits(oracle.dequant(12, blk4, 256)), bits(want4))
    blk6 = rng.integers(0, 256, 210, dtype=np.uint8)
    blk6[208:210] = [0x00, 0x3C]
    q6, sidx = q6k_values(blk6)
    sc6 = blk6[192:208].view(np.int8)
    want6 = np.array([np.float32(sc6[sidx[i]]) * np.float32(q6[i]) for i in range(256)],
                     np.float32)
    assert np.array_equal(bits(oracle.dequant(14, blk6, 256)), bits(want6))


def _rand_blocks(rng, nblk, bb, half_offsets):
    """nblk random blocks of bb bytes with finite f16 scales at the offsets."""
    b = rng.integers(0, 256, (nblk, bb), dtype=np.uint8)
    for o in half_offsets:
        b[:, o:o + 2] = rng.uniform(-0.1, 0.1, nblk).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return b


def _k4_scale_min(s12, j):
    """6-bit scale and min j of a K-quant 12-byte scale table (textbook:
    j < 4 the low six bits of bytes j and j + 4; otherwise four bits from
    byte j + 4 and the top two bits of bytes j - 4 and j)."""
    s12 = [int(x) for x in s12]
    if j < 4:
        return s12[j] & 63, s12[j + 4] & 63
    return (s12[j + 4] & 15) | ((s12[j - 4] >> 6) << 4), (s12[j + 4] >> 4) | ((s12[j] >> 6) << 4)


def test_dequant_small_block_types_vs_textbook(oracle):
    """Q8_0, Q4_0 (src/kernels.c:896-920) and Q5_K (src/kernels.c:286-306)
    rows against element-wise decoders written from the block layouts, in
    float32 with the reference's operation order."""
    rng = np.random.default_rng(896)
    f32 = np.float32
    b8 = _rand_blocks(rng, 6, 34, [0])
    want = np.concatenate([b[2:].view(np.int8).astype(f32) * b[:2].view(np.float16).astype(f32)
                           for b in b8])
    assert np.array_equal(bits(oracle.dequant(8, b8.reshape(-1), 192)), bits(want))
    b4 = _rand_blocks(rng, 6, 18, [0])
    want = []
    for b in b4:
        d = b[:2].view(np.float16).astype(f32)[0]
        nib = np.concatenate([b[2:] & 15, b[2:] >> 4]).astype(np.int32) - 8
        want.append(nib.astype(f32) * d)
    assert np.array_equal(bits(oracle.dequant(2, b4.reshape(-1), 192)), bits(np.concatenate(want)))
    b5 = _rand_blocks(rng, 3, 176, [0, 2])
    want = []
    for b in b5:
        d, dmin = b[:4].view(np.float16).astype(f32)
        qh, qs = b[16:48].astype(np.int32), b[48:176].astype(np.int32)
        for grp in range(8):
            sc, mn = _k4_scale_min(b[4:16], grp)
            lo = qs[32 * (grp % 4):32 * (grp % 4) + 32]
            v = (lo & 15 if grp < 4 else lo >> 4) | (((qh >> grp) & 1) << 4)
            want.append((d * f32(sc)) * v.astype(f32) - dmin * f32(mn))
    assert np.array_equal(bits(oracle.dequant(13, b5.reshape(-1), 768)), bits(np.concatenate(want)))


def test_dequant_vs_reference(oracle, ref):
    """Every row type the reference decodes, bit for bit against it."""
    rng = np.random.default_rng(874)
    cases = {8: (34, [0], 32), 2: (18, [0], 32), 13: (176, [0, 2], 256),
             12: (144, [0, 2], 256), 14: (210, [208], 256)}
    for gtype, (bb, offs, be) in cases.items():
        row = _rand_blocks(rng, 8, bb, offs).reshape(-1)
        n = 8 * be
        assert np.array_equal(bits(oracle.dequant(gtype, row, n)), bits(ref.dequant(gtype, row, n)))


def test_f16_conversions(oracle):
    """tests/test_kernels.c:199-208 known answers; every f16 bit pattern
    widens exactly (numpy's IEEE conversion)."""
    L = oracle.lib
    assert L.or_f16_to_f32(0x3C00) == 1.0 and L.or_f16_to_f32(0xBC00) == -1.0
    assert L.or_f16_to_f32(0x4000) == 2.0 and L.or_f16_to_f32(0x3800) == 0.5
    assert L.or_f16_to_f32(0x0001) > 0.0
    assert L.or_f32_to_f16(1.0) == 0x3C00 and L.or_f32_to_f16(-2.0) == 0xC000
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([L.or_f16_to_f32(int(v)) for v in h], np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(bits(got[finite]), bits(want[finite]))
    assert np.all(np.isnan(got[np.isnan(want)]))


def test_quantizer_known_answers(oracle):
    """tests/test_gemv.c:81-94: zero vector -> zero, ramp -> in range with
    the largest magnitude at +127; and q = round-half-away(x * 127/amax)."""
    q, s = oracle.quantize(np.zeros(512, np.float32))
    assert s == 0.0 and not q.any()
    x = np.arange(512, dtype=np.float32) - 200.0
    q, s = oracle.quantize(x)
    assert s > 0 and q[-1] == 127 and q.min() >= -127
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float32)
    q, s = oracle.quantize(x)
    amax = np.abs(x).max()
    inv = np.float32(127.0) / amax
    v = (x * inv).astype(np.float64)
    ref = np.where(v < 0, np.ceil(v - 0.5), np.floor(v + 0.5))
    away = np.abs(np.abs(v) % 1.0 - 0.5) > 1e-6   # skip exact .5 boundaries
    assert np.array_equal(q[away].astype(np.int64), np.clip(ref[away], -127, 127).astype(np.int64))
    assert np.float32(s) == np.float32(amax / np.float32(127.0))


# --------------------------------------------------------- golden fixtures

@pytest.mark.parametrize("name", ["tq1_0", "tq2_0", "q4_k", "q6_k", "f16"])
def test_gemv_golden(oracle, name):
    z = np.load(os.path.join(GOLD, f"gemv_{name}.npz"))
    N, K, gtype = int(z["rows"]), int(z["cols"]), int(z["gtype"])
    for t in range(z["x"].shape[0]):
        got = oracle.gemv(gtype, z["x"][t], z["w"], N, K)
        assert np.array_equal(bits(got), bits(z["out"][t]))
        if "q" in z.files:
            q, s = oracle.quantize(z["x"][t])
            assert np.array_equal(q, z["q"][t]) and np.float32(s) == z["scale"][t]


def test_quantize_golden(oracle):
    z = np.load(os.path.join(GOLD, "quantize.npz"))
    for i in range(3):
        q, s = oracle.quantize(z[f"x{i}"])
        assert np.array_equal(q, z[f"q{i}"]) and np.float32(s) == z[f"s{i}"]


def test_decode_golden(oracle):
    z = np.load(os.path.join(GOLD, "decode_tiny.npz"))
    spec = synth.spec("tiny-512", n_layer=2, n_vocab=2000)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tiny.gguf")
        tensors = {}
        synth.write_gguf(path, spec, tensors=tensors)
        if hashlib.sha256(open(path, "rb").read()).hexdigest() != str(z["sha256"]):
            pytest.skip("this numpy draws a different synthetic model than the fixture's")
    ctx = oracle.model(spec, tensors).context(64)
    logits = ctx.eval(z["prompt"])
    assert np.array_equal(bits(logits), bits(z["logits"]))
    ids, lg = [], logits
    for _ in range(len(z["ids"])):
        ids.append(int(np.argmax(lg)))
        lg = ctx.eval(np.array([ids[-1]], np.uint32))
    assert ids == [int(i) for i in z["ids"]]


# -------------------------------------------------------- against oracle/_ref

@pytest.mark.parametrize("gtype,N,K", [(34, 130, 2560), (35, 77, 1024), (12, 40, 1024),
                                       (14, 40, 1024), (1, 64, 2560), (0, 20, 288)])
def test_gemv_vs_reference(oracle, ref, gtype, N, K):
    rng = np.random.default_rng([gtype, N, K])
    if gtype in (34, 35):
        bb = 54 if gtype == 34 else 66
        w = rng.integers(0, 256, size=(N * K // 256, bb), dtype=np.uint8)
        w[:, bb - 2:] = rng.uniform(0.01, 0.05, w.shape[0]).astype(np.float16).view(
            np.uint8).reshape(-1, 2)
    elif gtype == 12:
        w = synth.q4k_quantize(rng.standard_normal((N, K)).astype(np.float32))
    elif gtype == 14:
        w = synth.q6k_quantize(rng.standard_normal((N, K)).astype(np.float32))
    elif gtype == 1:
        w = rng.standard_normal((N, K)).astype(np.float16)
    else:
        w = rng.standard_normal((N, K)).astype(np.float32)
    w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
    for _ in range(3):
        x = (rng.standard_normal(K) * rng.uniform(0.1, 50)).astype(np.float32)
        assert np.array_equal(bits(oracle.gemv(gtype, x, w, N, K)),
                              bits(ref.gemv(gtype, x, w, N, K, n_threads=1)))
    # threaded == serial (tests/test_gemv.c:116-125)
    assert np.array_equal(bits(ref.gemv(gtype, x, w, N, K, n_threads=4)),
                          bits(oracle.gemv(gtype, x, w, N, K, n_threads=3)))


# Grouped-query attention and a query width other than d_model, as the
# 4B, 8B and 27B configurations have them (src/forward.c:82-83 sets the
# group, :238 maps query head h to kv head h / gqa; head_dim comes from
# attention.key_length, src/model.c:188-237): four query heads per kv head
# with head_dim 128 over d_model 512 (q width 1024), the 4B/8B head layout
# 32/8 x 128 (q width 4096, attn_output K = 4096), the 27B group of two
# (32/16 x 64), and the 8B Q4_K/Q6_K mix with 8/2 x 128.
_FWD = {
    "tiny-288": ("tiny-288", {}),
    "tiny-512": ("tiny-512", {}),
    "gqa4-8x2x128": ("tiny-512", dict(n_head=8, n_head_kv=2, head_dim=128)),
    "gqa4-32x8x128": ("tiny-512", dict(n_head=32, n_head_kv=8, head_dim=128)),
    "gqa2-32x16x64": ("tiny-512", dict(n_head=32, n_head_kv=16, head_dim=64)),
    "kquant-gqa4-8x2x128": ("tiny-512", dict(n_head=8, n_head_kv=2, head_dim=128,
                                             linear_type=synth.Q4_K,
                                             types={"attn_v": synth.Q6_K,
                                                    "ffn_down": synth.Q6_K},
                                             output_type=synth.Q6_K)),
}


@pytest.mark.parametrize("case", list(_FWD))
def test_forward_vs_reference(oracle, ref, case):
    name, over = _FWD[case]
    spec = synth.spec(name, n_layer=2, n_vocab=3000, **over)
    if case != name:
        assert spec.n_head * spec.head_dim != spec.n_embd or spec.n_head != spec.n_head_kv
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "m.gguf")
        tensors = {}
        synth.write_gguf(path, spec, tensors=tensors)
        rm = ref.open_model(path)
        rc = rm.context(48, n_batch=32, n_threads=1)
        oc = oracle.model(spec, tensors).context(48)
        prompt = synth.prompt_ids(12, spec.n_vocab)
        a, b = oc.eval(prompt), rc.eval(prompt)
        assert np.array_equal(bits(a), bits(b))
        for _ in range(6):
            t = np.array([np.argmax(a)], np.uint32)
            a, b = oc.eval(t), rc.eval(t)
            assert np.array_equal(bits(a), bits(b))
        rc.close()
        rm.close()
