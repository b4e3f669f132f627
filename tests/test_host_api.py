"""The reference's host entry points beside the decode path, on the CPU:
IEEE half conversions (include/fox/fox.h:357-358) and the GGUF reader
(fox.h:204-262) with fox_weights_model (fox.h:390), checked against their
known answers, against numpy, and against RustFox itself (oracle/_ref) on
the same inputs."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

import rustfox_amd as rf
from rustfox_amd import synth
from oracle_libs import REF_SO, ref_available


def _bind(path):
    L = C.CDLL(path)
    L.fox_f16_to_f32.restype = C.c_float
    L.fox_f16_to_f32.argtypes = [C.c_uint16]
    L.fox_f32_to_f16.restype = C.c_uint16
    L.fox_f32_to_f16.argtypes = [C.c_float]
    vp, sz = C.c_void_p, C.c_size_t
    L.fox_gguf_open.argtypes = [C.c_char_p, C.POINTER(vp)]
    L.fox_gguf_close.argtypes = [vp]
    L.fox_gguf_close.restype = None
    for n in ("fox_gguf_metadata_count", "fox_gguf_tensor_count"):
        getattr(L, n).argtypes = [vp]
        getattr(L, n).restype = sz
    L.fox_gguf_version.argtypes = [vp]
    L.fox_gguf_version.restype = C.c_uint32
    for n in ("fox_gguf_find", "fox_gguf_tensor_find"):
        getattr(L, n).argtypes = [vp, C.c_char_p]
        getattr(L, n).restype = sz
    for n in ("fox_gguf_metadata_type", "fox_gguf_metadata_array_type"):
        getattr(L, n).argtypes = [vp, sz]
        getattr(L, n).restype = C.c_int
    L.fox_gguf_metadata_array_count.argtypes = [vp, sz]
    L.fox_gguf_metadata_array_count.restype = sz
    L.fox_gguf_read_tensor.argtypes = [vp, sz, vp, sz]
    return L


def _host():
    return _bind(rf.HOST_LIB)


def _f16_all():
    return np.arange(65536, dtype=np.uint32).astype(np.uint16)


# ----------------------------------------------------------------- halves

def test_f16_known_answers():
    """tests/test_kernels.c:199-208 of the reference."""
    L = _host()
    assert L.fox_f16_to_f32(0x3C00) == 1.0 and L.fox_f16_to_f32(0x0000) == 0.0
    assert L.fox_f16_to_f32(0xBC00) == -1.0 and L.fox_f16_to_f32(0x4000) == 2.0
    assert L.fox_f16_to_f32(0x3800) == 0.5 and L.fox_f16_to_f32(0x0001) > 0.0
    assert L.fox_f32_to_f16(1.0) == 0x3C00 and L.fox_f32_to_f16(-2.0) == 0xC000
    assert L.fox_f16_to_f32(L.fox_f32_to_f16(0.25)) == 0.25


def _f16_to_f32_all(L):
    f = L.fox_f16_to_f32
    out = np.empty(65536, np.float32)
    for h in range(65536):
        out[h] = f(h)
    return out


def test_f16_to_f32_exhaustive():
    """Every half against numpy's exact widening, NaN payloads included.
    (A float returned through ctypes becomes a Python double, which sets
    the quiet bit of a signalling NaN, so NaNs are compared with it set.)"""
    got = _f16_to_f32_all(_host()).view(np.uint32)
    want = _f16_all().view(np.float16).astype(np.float32).view(np.uint32)
    nan = np.isnan(want.view(np.float32))
    want = np.where(nan, want | np.uint32(0x00400000), want)
    assert np.array_equal(got, want)


def _f32_probe():
    """Every half's value and the midpoints to its neighbours, one ulp either
    side of each, random bit patterns, the overflow and underflow edges."""
    with np.errstate(all="ignore"):
        return _f32_probe_()


def _f32_probe_():
    h = _f16_all()
    v = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(v)
    vv = v[fin].astype(np.float64)
    nxt = np.nextafter(h[fin].view(np.float16), np.float16(np.inf)).astype(np.float64)
    mid = ((vv + nxt) / 2).astype(np.float32)
    bits = [v.view(np.uint32), mid.view(np.uint32)]
    bits += [mid.view(np.uint32) + 1, mid.view(np.uint32) - 1]
    rng = np.random.default_rng(357)
    bits.append(rng.integers(0, 2**32, 400000, dtype=np.uint64).astype(np.uint32))
    edges = np.array([65504, 65519.99, 65520, 65536, 2.0**-24, 2.0**-25, 2.0**-26,
                      3 * 2.0**-26, 2.0**-14, 1e-40, 3.4e38, np.inf, -np.inf, np.nan],
                     np.float32)
    bits.append(edges.view(np.uint32))
    bits.append(np.array([0x7F800001, 0xFFC00000, 0x7FFFFFFF, 0x80000000, 0x00000001],
                         np.uint32))
    allb = np.concatenate(bits)
    return np.concatenate([allb, allb ^ np.uint32(0x80000000)]).view(np.float32)


def _f32_to_f16_many(L, xs):
    f = L.fox_f32_to_f16
    return np.fromiter((f(float(x)) for x in xs), np.uint16, count=len(xs))


def test_f32_to_f16_closed_form():
    """Normal results round to nearest even (numpy's conversion); NaN is
    0x7E00 with its sign; subnormal results round half up."""
    L = _host()
    xs = _f32_probe()
    got = _f32_to_f16_many(L, xs)
    np.seterr(all="ignore")
    a = np.abs(xs.astype(np.float64))
    normal = np.isfinite(xs) & (a >= 2.0**-14 * (1 - 2.0**-12))
    want = xs[normal].astype(np.float16).view(np.uint16)
    assert np.array_equal(got[normal], want)
    nan = np.isnan(xs)
    assert np.all((got[nan] & 0x7FFF) == 0x7E00)
    assert np.array_equal(got[nan] >> 15, (xs[nan].view(np.uint32) >> 31).astype(np.uint16))
    sub = np.isfinite(xs) & ~normal
    k = np.floor(a[sub] * 2.0**24 + 0.5)          # half up in units of 2^-24
    sign = (xs[sub].view(np.uint32) >> 16).astype(np.uint16) & 0x8000
    assert np.array_equal(got[sub], (k.astype(np.uint16) | sign))


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref was not built")
def test_f16_conversions_equal_the_reference():
    ours, ref = _host(), _bind(REF_SO)
    assert np.array_equal(_f16_to_f32_all(ours).view(np.uint32),
                          _f16_to_f32_all(ref).view(np.uint32))
    xs = _f32_probe()
    assert np.array_equal(_f32_to_f16_many(ours, xs), _f32_to_f16_many(ref, xs))


# ------------------------------------------------------------------- gguf

def _kv(key, t, payload):
    k = key.encode()
    return struct.pack("<Q", len(k)) + k + struct.pack("<I", t) + payload


def _s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _gguf_with_metadata(path):
    """A GGUF v3 file holding every metadata value type, arrays of strings,
    i32, f32 and u8, and three tensors."""
    meta = [
        _kv("general.architecture", 8, _s("llama")),
        _kv("u8", 0, struct.pack("<B", 200)), _kv("i8", 1, struct.pack("<b", -5)),
        _kv("u16", 2, struct.pack("<H", 60000)), _kv("i16", 3, struct.pack("<h", -300)),
        _kv("u32", 4, struct.pack("<I", 4000000000)), _kv("i32", 5, struct.pack("<i", -7)),
        _kv("f32", 6, struct.pack("<f", 1e-5)), _kv("yes", 7, struct.pack("<B", 1)),
        _kv("no", 7, struct.pack("<B", 0)),
        _kv("u64", 10, struct.pack("<Q", 2**40 + 3)), _kv("i64", 11, struct.pack("<q", -2**35)),
        _kv("f64", 12, struct.pack("<d", 0.1)),
        _kv("tok.strings", 9, struct.pack("<IQ", 8, 4) + b"".join(_s(w) for w in
                                                                   ["<s>", "fox", "", "é"])),
        _kv("tok.ids", 9, struct.pack("<IQ", 5, 3) + struct.pack("<3i", -1, 0, 77)),
        _kv("tok.scores", 9, struct.pack("<IQ", 6, 2) + struct.pack("<2f", 0.5, -2.25)),
        _kv("tok.bytes", 9, struct.pack("<IQ", 0, 3) + bytes([1, 2, 255])),
        _kv("general.alignment", 4, struct.pack("<I", 64)),
    ]
    tens = [("a", [256, 2], 34, 0), ("b", [7], 0, 128), ("c", [32, 3], 1, 192)]
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tens), len(meta)) + b"".join(meta)
    for name, ne, t, off in tens:
        head += _s(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne)
        head += struct.pack("<IQ", t, off)
    data_off = (len(head) + 63) // 64 * 64
    blob = bytearray(head + b"\0" * (data_off - len(head)))
    data = bytearray(512)
    data[0:108] = bytes(range(108))
    data[128:156] = np.arange(7, dtype=np.float32).tobytes()
    data[192:384] = np.arange(96, dtype=np.float16).tobytes()
    blob += data
    open(path, "wb").write(bytes(blob))


def _survey(L, path):
    """Everything the accessors report about the file, as plain values."""
    g = C.c_void_p()
    st = L.fox_gguf_open(path.encode(), C.byref(g))
    assert st == 0 and g.value
    out = {"version": L.fox_gguf_version(g), "meta": L.fox_gguf_metadata_count(g),
           "tensors": L.fox_gguf_tensor_count(g)}
    keys = ["general.architecture", "u8", "i8", "u16", "i16", "u32", "i32", "f32", "yes", "no",
            "u64", "i64", "f64", "tok.strings", "tok.ids", "tok.scores", "tok.bytes",
            "general.alignment", "absent"]
    for k in keys:
        i = L.fox_gguf_find(g, k.encode())
        row = [i, L.fox_gguf_metadata_type(g, i), L.fox_gguf_metadata_array_count(g, i),
               L.fox_gguf_metadata_array_type(g, i)]
        u32, u64, f32, b, s = C.c_uint32(), C.c_uint64(), C.c_float(), C.c_int(), C.c_char_p()
        row.append((L.fox_gguf_get_u32(C.c_void_p(g.value), C.c_size_t(i), C.byref(u32)), u32.value))
        row.append((L.fox_gguf_get_uint(C.c_void_p(g.value), C.c_size_t(i), C.byref(u64)), u64.value))
        row.append((L.fox_gguf_get_f32(C.c_void_p(g.value), C.c_size_t(i), C.byref(f32)), f32.value))
        row.append((L.fox_gguf_get_bool(C.c_void_p(g.value), C.c_size_t(i), C.byref(b)), b.value))
        row.append((L.fox_gguf_get_string(C.c_void_p(g.value), C.c_size_t(i), C.byref(s)), s.value))
        for el in range(5):
            s2, i32, f2 = C.c_char_p(), C.c_int32(), C.c_float()
            row.append((L.fox_gguf_get_array_string(C.c_void_p(g.value), C.c_size_t(i),
                                                    C.c_size_t(el), C.byref(s2)), s2.value))
            row.append((L.fox_gguf_get_array_i32(C.c_void_p(g.value), C.c_size_t(i),
                                                 C.c_size_t(el), C.byref(i32)), i32.value))
            row.append((L.fox_gguf_get_array_f32(C.c_void_p(g.value), C.c_size_t(i),
                                                 C.c_size_t(el), C.byref(f2)), f2.value))
        out[k] = row
    # null arguments
    out["null"] = (L.fox_gguf_get_u32(C.c_void_p(g.value), C.c_size_t(0), None),
                   L.fox_gguf_get_uint(None, C.c_size_t(0), C.byref(C.c_uint64())))

    class Tensor(C.Structure):
        _fields_ = [("name", C.c_char_p), ("n_dims", C.c_uint32), ("ne", C.c_uint64 * 4),
                    ("type", C.c_int), ("offset", C.c_uint64), ("size_bytes", C.c_uint64)]
    for name in ("a", "b", "c", "zz"):
        i = L.fox_gguf_tensor_find(g, name.encode())
        t = Tensor()
        st = L.fox_gguf_tensor_at(C.c_void_p(g.value), C.c_size_t(i), C.byref(t))
        row = [i, st]
        if st == 0:
            row += [t.name, t.n_dims, list(t.ne), t.type, t.offset, t.size_bytes]
            buf = (C.c_uint8 * int(t.size_bytes))()
            row.append(L.fox_gguf_read_tensor(g, i, C.cast(buf, C.c_void_p), t.size_bytes))
            row.append(bytes(buf))
            row.append(L.fox_gguf_read_tensor(g, i, C.cast(buf, C.c_void_p), t.size_bytes - 1))
        out["tensor " + name] = row
    L.fox_gguf_close(g)
    return out


def test_gguf_accessors(tmp_path):
    p = str(tmp_path / "meta.gguf")
    _gguf_with_metadata(p)
    got = _survey(_host(), p)
    assert got["version"] == 3 and got["meta"] == 18 and got["tensors"] == 3
    ok, fmt, nf, arg = 0, 4, 6, 1                     # fox_status values
    assert got["u32"][4] == (ok, 4000000000) and got["u8"][4][0] == fmt
    assert got["i8"][5] == (ok, 2**64 - 5) and got["u64"][5] == (ok, 2**40 + 3)
    assert got["yes"][7] == (ok, 1) and got["no"][7] == (ok, 0)
    assert got["general.architecture"][8] == (ok, b"llama")
    assert got["absent"][0] == 2**64 - 1 and got["absent"][4][0] == nf
    assert got["tok.strings"][2:4] == [4, 8]
    assert [got["tok.strings"][9 + 3 * e] for e in range(5)] == [
        (ok, b"<s>"), (ok, b"fox"), (ok, b""), (ok, "é".encode()), (nf, None)]
    assert [got["tok.ids"][10 + 3 * e][1] for e in range(3)] == [-1, 0, 77]
    assert got["tok.ids"][9][0] == fmt and got["tok.scores"][11] == (ok, 0.5)
    assert got["null"] == (arg, arg)
    a = got["tensor a"]
    assert a[2:8] == [b"a", 2, [256, 2, 0, 0], 34, 0, 108]
    assert a[8] == ok and a[9] == bytes(range(108)) and a[10] == arg
    assert got["tensor zz"][:2] == [2**64 - 1, nf]


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref was not built")
def test_gguf_accessors_equal_the_reference(tmp_path):
    """Every accessor's status and value on the same file, against RustFox's
    own reader; and on a synthetic model, plus fox_weights_model."""
    p = str(tmp_path / "meta.gguf")
    _gguf_with_metadata(p)
    assert _survey(_host(), p) == _survey(_bind(REF_SO), p)


def test_weights_model_exposes_the_file(tmp_path):
    """tests/test_weights.c:97-99: every tensor is visible through the
    weights handle."""
    s = synth.spec("tiny-288", n_layer=1, n_vocab=64)
    p = str(tmp_path / "m.gguf")
    synth.write_gguf(p, s)
    L = _host()
    L.fox_weights_open.argtypes = [C.c_char_p, C.c_int, C.c_uint64, C.POINTER(C.c_void_p)]
    L.fox_weights_model.argtypes = [C.c_void_p]
    L.fox_weights_model.restype = C.c_void_p
    L.fox_weights_close.argtypes = [C.c_void_p]
    w = C.c_void_p()
    assert L.fox_weights_open(p.encode(), 0, 0, C.byref(w)) == 0
    g = L.fox_weights_model(w)
    assert g and L.fox_gguf_tensor_count(g) == len(synth.tensor_list(s))
    assert L.fox_gguf_find(g, b"llama.block_count") != 2**64 - 1
    assert L.fox_weights_model(None) is None
    L.fox_weights_close(w)
