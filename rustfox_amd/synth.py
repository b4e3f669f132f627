"""Seeded synthetic models for the decode path: block encoders, a K-quant
quantiser and a GGUF v3 writer.

RustFox ships no weight quantiser and no quantised-GGUF writer (its only
writers emit F32 test fixtures, tests/test_forward.c:129-186), so the
synthetic models of the benchmark configurations are produced here.

Block layouts follow the reference decoders:
  TQ1_0  54 B / 256: qs[48] @0, qh[4] @48, f16 d @52   (src/ternary.c:17-21, 73-93)
  TQ2_0  66 B / 256: qs[64] @0, f16 d @64              (src/ternary.c:17-21, 177-188)
  Q4_K  144 B / 256: f16 d, f16 dmin, scales[12], qs[128] (src/kernels.c:246-283)
  Q6_K  210 B / 256: ql[128], qh[64], int8 sc[16], f16 d (src/kernels.c:217-244)
GGUF metadata keys are the llama.* keys read by src/model.c:188-237.

Random streams: numpy's PCG64 (numpy.random.default_rng) seeded with
(seed, tensor index), so every tensor is reproducible on its own.
"""
from __future__ import annotations

import dataclasses
import os
import struct

import numpy as np

F32, F16, Q4_K, Q6_K, TQ1_0, TQ2_0 = 0, 1, 12, 14, 34, 35
BLOCK_BYTES = {F32: 4, F16: 2, Q4_K: 144, Q6_K: 210, TQ1_0: 54, TQ2_0: 66}
BLOCK_ELEMS = {F32: 1, F16: 1, Q4_K: 256, Q6_K: 256, TQ1_0: 256, TQ2_0: 256}
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_K: "Q4_K", Q6_K: "Q6_K",
              TQ1_0: "TQ1_0", TQ2_0: "TQ2_0"}


def row_bytes(gtype: int, n_cols: int) -> int:
    be, bb = BLOCK_ELEMS[gtype], BLOCK_BYTES[gtype]
    if n_cols % be:
        raise ValueError(f"{n_cols} columns is not a whole number of "
                         f"{TYPE_NAMES[gtype]} blocks")
    return n_cols // be * bb


# ------------------------------------------------------------------ TQ1_0

_POW3_DESC = np.array([81, 27, 9, 3, 1], dtype=np.int32)


def tq1_pack_value(v: np.ndarray) -> np.ndarray:
    """Base-3 value V in [0, 243) -> byte ceil(V * 256 / 243), the fixed-point
    form the reference decodes with ((uint8)(b*3^l) * 3) >> 8."""
    return ((v.astype(np.int32) * 256 + 242) // 243).astype(np.uint8)


def tq1_encode(trits: np.ndarray, d: np.ndarray) -> np.ndarray:
    """trits: int array (..., 256) in {-1, 0, 1}; d: f16-representable scales
    (...,).  Returns uint8 (..., 54)."""
    t = (np.asarray(trits, dtype=np.int32) + 1)
    lead = t.shape[:-1]
    t = t.reshape(-1, 256)
    n = t.shape[0]
    out = np.empty((n, 54), dtype=np.uint8)
    # qs[m], m < 32: elements m + 32 l, level 0 most significant
    a = t[:, :160].reshape(n, 5, 32)
    out[:, 0:32] = tq1_pack_value(np.einsum("nlm,l->nm", a, _POW3_DESC))
    b = t[:, 160:240].reshape(n, 5, 16)
    out[:, 32:48] = tq1_pack_value(np.einsum("nlm,l->nm", b, _POW3_DESC))
    c = t[:, 240:256].reshape(n, 4, 4)
    v4 = np.einsum("nlm,l->nm", c, _POW3_DESC[1:])
    out[:, 48:52] = tq1_pack_value(v4 * 3)
    out[:, 52:54] = np.asarray(d, dtype=np.float16).reshape(n).view(np.uint8).reshape(n, 2)
    return out.reshape(*lead, 54)


def tq1_random(rng: np.random.Generator, n_blocks: int,
               dlo: float = 0.01, dhi: float = 0.05) -> np.ndarray:
    """n_blocks TQ1_0 blocks with i.i.d. uniform trits and d ~ U(dlo, dhi)
    rounded to f16.  Drawing the 5-trit value V uniformly on [0, 243) is the
    same distribution as drawing its five trits uniformly."""
    out = np.empty((n_blocks, 54), dtype=np.uint8)
    out[:, :48] = tq1_pack_value(rng.integers(0, 243, size=(n_blocks, 48), dtype=np.int32))
    out[:, 48:52] = tq1_pack_value(rng.integers(0, 81, size=(n_blocks, 4), dtype=np.int32) * 3)
    d = rng.uniform(dlo, dhi, size=n_blocks).astype(np.float16)
    out[:, 52:54] = d.view(np.uint8).reshape(n_blocks, 2)
    return out


# ------------------------------------------------------------------ TQ2_0

def tq2_encode(trits: np.ndarray, d: np.ndarray) -> np.ndarray:
    """trits (..., 256) in {-1, 0, 1} (code = trit + 1; codes are 2 bits)."""
    t = (np.asarray(trits, dtype=np.int32) + 1).reshape(-1, 256)
    n = t.shape[0]
    out = np.zeros((n, 66), dtype=np.uint8)
    g = t.reshape(n, 2, 4, 32)  # half, level, m
    packed = (g[:, :, 0] | (g[:, :, 1] << 2) | (g[:, :, 2] << 4) | (g[:, :, 3] << 6))
    out[:, :64] = packed.reshape(n, 64).astype(np.uint8)
    out[:, 64:66] = np.asarray(d, dtype=np.float16).reshape(n).view(np.uint8).reshape(n, 2)
    return out.reshape(*np.asarray(trits).shape[:-1], 66)


def tq2_random(rng: np.random.Generator, n_blocks: int,
               dlo: float = 0.01, dhi: float = 0.05) -> np.ndarray:
    """Ternary TQ2_0 blocks: codes uniform on {0, 1, 2}."""
    codes = rng.integers(0, 3, size=(n_blocks, 2, 4, 32), dtype=np.int32)
    out = np.empty((n_blocks, 66), dtype=np.uint8)
    out[:, :64] = (codes[:, :, 0] | (codes[:, :, 1] << 2) | (codes[:, :, 2] << 4)
                   | (codes[:, :, 3] << 6)).reshape(n_blocks, 64).astype(np.uint8)
    d = rng.uniform(dlo, dhi, size=n_blocks).astype(np.float16)
    out[:, 64:66] = d.view(np.uint8).reshape(n_blocks, 2)
    return out


# ------------------------------------------------------------------- Q4_K

def _f16(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def q4k_quantize(w: np.ndarray) -> np.ndarray:
    """Affine 4-bit quantiser: per 32-element sub-block a scale and a min,
    each a 6-bit multiple of the block's f16 d / dmin.  w: (..., 256*k)."""
    x = np.asarray(w, dtype=np.float32).reshape(-1, 8, 32)
    n = x.shape[0]
    lo = np.minimum(x.min(axis=2), 0.0)
    hi = x.max(axis=2)
    sub_scale = (hi - lo) / 15.0
    sub_min = -lo
    d = _f16(sub_scale.max(axis=1) / 63.0)
    dmin = _f16(sub_min.max(axis=1) / 63.0)
    df, mf = d.astype(np.float32), dmin.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(df[:, None] > 0, np.rint(sub_scale / df[:, None]), 0)
        mn = np.where(mf[:, None] > 0, np.rint(sub_min / mf[:, None]), 0)
    sc = np.clip(sc, 0, 63).astype(np.int32)
    mn = np.clip(mn, 0, 63).astype(np.int32)
    step = df[:, None] * sc
    off = mf[:, None] * mn
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(step[:, :, None] > 0,
                     np.rint((x + off[:, :, None]) / step[:, :, None]), 0)
    q = np.clip(q, 0, 15).astype(np.uint8)

    out = np.zeros((n, 144), dtype=np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    out[:, 2:4] = dmin.view(np.uint8).reshape(n, 2)
    s = np.zeros((n, 12), dtype=np.int32)
    s[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    s[:, 4:8] = (mn[:, 0:4] & 63) | ((mn[:, 4:8] >> 4) << 6)
    s[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    out[:, 4:16] = s.astype(np.uint8)
    qq = q.reshape(n, 4, 2, 32)
    out[:, 16:144] = (qq[:, :, 0] | (qq[:, :, 1] << 4)).reshape(n, 128)
    return out.reshape(*np.asarray(w).shape[:-1], -1)


# ------------------------------------------------------------------- Q6_K

def q6k_quantize(w: np.ndarray) -> np.ndarray:
    """Symmetric 6-bit quantiser: per 16-element group an int8 scale of the
    block's f16 d, values in [-32, 31].  w: (..., 256*k)."""
    x = np.asarray(w, dtype=np.float32).reshape(-1, 16, 16)
    n = x.shape[0]
    amax = np.abs(x).max(axis=2)
    sub = amax / 31.0
    d = _f16(sub.max(axis=1) / 127.0)
    df = d.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(df[:, None] > 0, np.rint(sub / df[:, None]), 0)
    sc = np.clip(sc, -128, 127).astype(np.int32)
    step = df[:, None] * sc
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(step[:, :, None] > 0, np.rint(x / step[:, :, None]), 0)
    q = (np.clip(q, -32, 31) + 32).astype(np.int32).reshape(n, 2, 4, 32)  # half, grp, l

    out = np.zeros((n, 210), dtype=np.uint8)
    for h in range(2):
        g = q[:, h]
        ql = np.zeros((n, 64), dtype=np.int32)
        ql[:, 0:32] = (g[:, 0] & 15) | ((g[:, 2] & 15) << 4)
        ql[:, 32:64] = (g[:, 1] & 15) | ((g[:, 3] & 15) << 4)
        qh = ((g[:, 0] >> 4) | ((g[:, 1] >> 4) << 2) | ((g[:, 2] >> 4) << 4)
              | ((g[:, 3] >> 4) << 6))
        out[:, 64 * h:64 * h + 64] = ql.astype(np.uint8)
        out[:, 128 + 32 * h:128 + 32 * h + 32] = qh.astype(np.uint8)
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    out[:, 208:210] = d.view(np.uint8).reshape(n, 2)
    return out.reshape(*np.asarray(w).shape[:-1], -1)


# ------------------------------------------------------------ model specs

@dataclasses.dataclass
class ModelSpec:
    name: str
    n_layer: int
    n_embd: int
    n_head: int
    n_head_kv: int
    head_dim: int
    n_ff: int
    n_vocab: int
    rope_base: float = 10000.0
    rms_eps: float = 1e-5
    n_ctx: int = 2048
    # ggml type per role; "auto" picks TQ1_0 where K % 256 == 0, else F16
    linear_type: object = TQ1_0
    types: dict = dataclasses.field(default_factory=dict)
    embd_type: int = F16
    output_type: int = F16
    seed: int = 1

    def type_of(self, role: str, k: int) -> int:
        t = self.types.get(role, self.linear_type)
        if t == "auto":
            return TQ1_0 if k % 256 == 0 else F16
        return t


def spec(name: str, **over) -> ModelSpec:
    """Named configurations (the architectures of the benchmark workloads)."""
    base = {
        # 6 x d288 (6 heads x 48) ff768: TQ1_0 only where K % 256 == 0
        "tiny-288": dict(n_layer=6, n_embd=288, n_head=6, n_head_kv=6, head_dim=48,
                         n_ff=768, n_vocab=32000, linear_type="auto", n_ctx=128),
        # 6 x d512 (8 heads x 64) ff768: every linear weight TQ1_0
        "tiny-512": dict(n_layer=6, n_embd=512, n_head=8, n_head_kv=8, head_dim=64,
                         n_ff=768, n_vocab=32000, n_ctx=128),
        # 36 x d2560, 32/8 heads x 128, ff 9728, vocab 151936
        "4b": dict(n_layer=36, n_embd=2560, n_head=32, n_head_kv=8, head_dim=128,
                   n_ff=9728, n_vocab=151936, rope_base=1e6, n_ctx=2176),
        # 32 x d4096, 32/8 x 128, ff 14336, vocab 128256, Q4_K_M-style mix
        "8b": dict(n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128,
                   n_ff=14336, n_vocab=128256, rope_base=500000.0, n_ctx=4224,
                   linear_type=Q4_K, types={"attn_v": Q6_K, "ffn_down": Q6_K},
                   output_type=Q6_K),
        # 62 x d5376, 32/16 x 128, ff 21504, vocab 262144
        "27b": dict(n_layer=62, n_embd=5376, n_head=32, n_head_kv=16, head_dim=128,
                    n_ff=21504, n_vocab=262144, rope_base=1e6, n_ctx=8320),
    }[name]
    base.update(over)
    return ModelSpec(name=name, **base)


def tensor_list(s: ModelSpec):
    """(name, ne0=K, ne1=N or 0, ggml type) in file order."""
    d, q, kv = s.n_embd, s.n_head * s.head_dim, s.n_head_kv * s.head_dim
    out = [("token_embd.weight", d, s.n_vocab, s.embd_type),
           ("output_norm.weight", d, 0, F32),
           ("output.weight", d, s.n_vocab, s.output_type)]
    for l in range(s.n_layer):
        p = f"blk.{l}."
        out += [
            (p + "attn_norm.weight", d, 0, F32),
            (p + "attn_q.weight", d, q, s.type_of("attn_q", d)),
            (p + "attn_k.weight", d, kv, s.type_of("attn_k", d)),
            (p + "attn_v.weight", d, kv, s.type_of("attn_v", d)),
            (p + "attn_output.weight", q, d, s.type_of("attn_output", q)),
            (p + "ffn_norm.weight", d, 0, F32),
            (p + "ffn_gate.weight", d, s.n_ff, s.type_of("ffn_gate", d)),
            (p + "ffn_up.weight", d, s.n_ff, s.type_of("ffn_up", d)),
            (p + "ffn_down.weight", s.n_ff, d, s.type_of("ffn_down", s.n_ff)),
        ]
    return out


# Tensors above this many elements are generated in row ranges, each range
# from its own stream (seed, tensor index, first row), so that ranges can be
# produced in parallel processes; smaller tensors come from one stream
# (seed, tensor index).
CHUNK_ELEMS = 1 << 25


def _chunk_rows(ne0: int) -> int:
    return max(1, (1 << 22) // ne0)


def tensor_chunks(ne0: int, ne1: int):
    """Row ranges [(r0, r1)] a tensor is generated in (one range when small)."""
    rows = max(ne1, 1)
    if rows * ne0 <= CHUNK_ELEMS:
        return [(0, rows)]
    step = _chunk_rows(ne0)
    return [(r0, min(rows, r0 + step)) for r0 in range(0, rows, step)]


def _gen_rows(rng, name, ne0, nrows, gtype):
    if name.endswith("norm.weight"):
        return np.ones(ne0 * nrows, dtype=np.float32).view(np.uint8)
    if gtype == F16:
        w = rng.standard_normal((nrows, ne0), dtype=np.float32) * np.float32(0.02)
        return w.astype(np.float16).view(np.uint8).reshape(-1)
    if gtype == F32:
        w = rng.standard_normal((nrows, ne0), dtype=np.float32) * np.float32(0.02)
        return w.view(np.uint8).reshape(-1)
    if gtype == TQ1_0:
        return tq1_random(rng, nrows * ne0 // 256).reshape(-1)
    if gtype == TQ2_0:
        return tq2_random(rng, nrows * ne0 // 256).reshape(-1)
    if gtype in (Q4_K, Q6_K):
        rb = row_bytes(gtype, ne0)
        out = np.empty(nrows * rb, dtype=np.uint8)
        step = _chunk_rows(ne0)
        for r0 in range(0, nrows, step):
            r1 = min(nrows, r0 + step)
            w = rng.standard_normal((r1 - r0, ne0), dtype=np.float32) * np.float32(0.02)
            enc = q4k_quantize(w) if gtype == Q4_K else q6k_quantize(w)
            out[r0 * rb:r1 * rb] = enc.reshape(-1)
        return out
    raise ValueError(f"no generator for type {gtype}")


def make_chunk(s: ModelSpec, index: int, name: str, ne0: int, ne1: int, gtype: int,
               r0: int, r1: int) -> np.ndarray:
    """Bytes of rows [r0, r1) of one tensor (a range of tensor_chunks)."""
    if (r0, r1) == (0, max(ne1, 1)) and max(ne1, 1) * ne0 <= CHUNK_ELEMS:
        rng = np.random.default_rng([s.seed, index])
    else:
        rng = np.random.default_rng([s.seed, index, r0])
    return _gen_rows(rng, name, ne0, r1 - r0, gtype)


def make_tensor(s: ModelSpec, index: int, name: str, ne0: int, ne1: int,
                gtype: int) -> np.ndarray:
    """Bytes of one tensor.  Norms are 1.0; f16 matrices ~ N(0, 0.02);
    ternary matrices uniform trits with d ~ U(0.01, 0.05); K-quants quantise
    N(0, 0.02) weights with the quantisers above."""
    parts = [make_chunk(s, index, name, ne0, ne1, gtype, r0, r1)
             for r0, r1 in tensor_chunks(ne0, ne1)]
    return parts[0] if len(parts) == 1 else np.concatenate(parts)


def _chunk_job(args):
    return make_chunk(*args)


def _workers() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


# ------------------------------------------------------------------- GGUF

_GGUF_U32, _GGUF_F32, _GGUF_STR = 4, 6, 8


def _kv_u32(key, v):
    k = key.encode()
    return struct.pack("<Q", len(k)) + k + struct.pack("<II", _GGUF_U32, v)


def _kv_f32(key, v):
    k = key.encode()
    return struct.pack("<Q", len(k)) + k + struct.pack("<If", _GGUF_F32, v)


def _kv_str(key, v):
    k, b = key.encode(), v.encode()
    return struct.pack("<Q", len(k)) + k + struct.pack("<IQ", _GGUF_STR, len(b)) + b


def gguf_header(s: ModelSpec, alignment: int = 32):
    """(header bytes including the padding to the data section, tensor
    offsets from the data section's start) of the file write_gguf writes."""
    tl = tensor_list(s)
    meta = [
        _kv_u32("general.alignment", alignment),
        _kv_str("general.architecture", "llama"),
        _kv_str("general.name", f"synthetic-{s.name}"),
        _kv_u32("llama.block_count", s.n_layer),
        _kv_u32("llama.embedding_length", s.n_embd),
        _kv_u32("llama.attention.head_count", s.n_head),
        _kv_u32("llama.attention.head_count_kv", s.n_head_kv),
        _kv_u32("llama.attention.key_length", s.head_dim),
        _kv_u32("llama.feed_forward_length", s.n_ff),
        _kv_u32("llama.context_length", s.n_ctx),
        _kv_f32("llama.attention.layer_norm_rms_epsilon", s.rms_eps),
        _kv_f32("llama.rope.freq_base", s.rope_base),
    ]
    infos, offsets, off = [], [], 0
    for name, ne0, ne1, gt in tl:
        nbytes = (max(ne1, 1) * row_bytes(gt, ne0))
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        nm = name.encode()
        dims = [ne0] if ne1 == 0 else [ne0, ne1]
        infos.append(struct.pack("<Q", len(nm)) + nm + struct.pack("<I", len(dims))
                     + b"".join(struct.pack("<Q", x) for x in dims)
                     + struct.pack("<IQ", gt, off))
        off += nbytes
    head = (b"GGUF" + struct.pack("<IQQ", 3, len(tl), len(meta)) + b"".join(meta)
            + b"".join(infos))
    return head + b"\0" * ((-len(head)) % alignment), offsets


def map_tensors(path: str, s: ModelSpec, alignment: int = 32) -> dict:
    """{name: read-only uint8 array} over a file write_gguf wrote, memory
    mapped (no copy)."""
    head, offsets = gguf_header(s, alignment)
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    out = {}
    for (name, ne0, ne1, gt), o in zip(tensor_list(s), offsets):
        a = len(head) + o
        out[name] = mm[a:a + max(ne1, 1) * row_bytes(gt, ne0)]
    return out


def write_gguf(path: str, s: ModelSpec, alignment: int = 32, tensors=None) -> dict:
    """Write the model as a GGUF v3 file; returns {name: bytes ndarray} only
    when tensors == {} is passed in to collect them.  Row ranges of large
    tensors are generated by a pool of worker processes (the bytes do not
    depend on the number of workers)."""
    tl = tensor_list(s)
    head, offsets = gguf_header(s, alignment)
    jobs = [(i, r0, r1) for i, (name, ne0, ne1, gt) in enumerate(tl)
            for r0, r1 in tensor_chunks(ne0, ne1)]
    nw = _workers() if sum(max(t[2], 1) * t[1] for t in tl) > 4 * CHUNK_ELEMS else 1
    pool = None
    if nw > 1:
        import concurrent.futures as cf
        import multiprocessing as mp
        pool = cf.ProcessPoolExecutor(nw, mp_context=mp.get_context("fork"))
    try:
        def results():
            if pool is None:
                for i, r0, r1 in jobs:
                    yield i, make_chunk(s, i, *tl[i], r0, r1)
                return
            window = []
            for i, r0, r1 in jobs:
                window.append((i, pool.submit(_chunk_job, (s, i, *tl[i], r0, r1))))
                if len(window) >= 2 * nw:
                    j, f = window.pop(0)
                    yield j, f.result()
            for j, f in window:
                yield j, f.result()

        with open(path, "wb") as f:
            f.write(head)
            pos = 0
            parts = {}
            for i, data in results():
                o = offsets[i]
                if pos < o:
                    f.write(b"\0" * (o - pos))
                    pos = o
                f.write(data.tobytes())
                pos += data.nbytes
                if tensors is not None:
                    parts.setdefault(i, []).append(data)
            if tensors is not None:
                for i, ps in parts.items():
                    tensors[tl[i][0]] = ps[0] if len(ps) == 1 else np.concatenate(ps)
    finally:
        if pool is not None:
            pool.shutdown()
    return tensors


def gguf_bytes(s: ModelSpec) -> int:
    return sum(max(ne1, 1) * row_bytes(gt, ne0) for _, ne0, ne1, gt in tensor_list(s))


def prompt_ids(n: int, n_vocab: int, seed: int = 7) -> np.ndarray:
    return np.random.default_rng([seed, 0xF0C5]).integers(0, n_vocab, size=n,
                                                          dtype=np.uint32)


def path_in(dirname: str, s: ModelSpec) -> str:
    return os.path.join(dirname, f"synthetic-{s.name}-s{s.seed}.gguf")
