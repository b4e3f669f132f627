"""ctypes bindings of the two oracle libraries used by the tests.

  Oracle  -- oracle/liboracle.so, this repository's C restatement of the
             RustFox decode path (oracle/fox_oracle.c).
  Ref     -- oracle/_ref/libfoxref.so, the RustFox sources compiled as they
             lie (oracle/Makefile); present only where the sources were
             available when the tree was built.

Both are test infrastructure: the product under rustfox_amd/ never loads
them.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libfoxref.so")
REF_FAST_SO = os.path.join(ROOT, "oracle", "_ref", "libfoxref_fast.so")

P = C.c_void_p
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class OrTensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("type", C.c_int)]


class OrLayer(C.Structure):
    _fields_ = [(n, OrTensor) for n in ("attn_norm", "attn_q", "attn_k", "attn_v",
                                        "attn_out", "ffn_norm", "ffn_gate", "ffn_up",
                                        "ffn_down")]


class OrModel(C.Structure):
    _fields_ = [("n_layer", C.c_uint32), ("n_embd", C.c_uint32), ("n_head", C.c_uint32),
                ("n_head_kv", C.c_uint32), ("head_dim", C.c_uint32), ("n_ff", C.c_uint32),
                ("n_vocab", C.c_uint32), ("rms_eps", C.c_float), ("rope_base", C.c_float),
                ("token_embd", OrTensor), ("output_norm", OrTensor), ("output", OrTensor),
                ("layers", C.POINTER(OrLayer))]


class Oracle:
    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (make -C oracle oracle)")
        L = self.lib = C.CDLL(path)
        L.or_f16_to_f32.restype = C.c_float
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_f32_to_f16.restype = C.c_uint16
        L.or_f32_to_f16.argtypes = [C.c_float]
        L.or_quantize_act_i8.argtypes = [_f32p, C.c_size_t, _i8p, C.POINTER(C.c_float)]
        L.or_quantize_act_k.argtypes = [_f32p, C.c_size_t, _i8p, _f32p]
        L.or_tq1_block_sum.argtypes = [_i8p, _u8p]
        L.or_tq1_block_sum.restype = C.c_int32
        L.or_tq2_block_sum.argtypes = [_i8p, _u8p]
        L.or_tq2_block_sum.restype = C.c_int32
        L.or_q4k_block_sums.argtypes = [_i8p, _u8p, C.c_void_p, C.c_void_p]
        L.or_q4k_block_sums.restype = None
        L.or_q6k_block_sums.argtypes = [_i8p, _u8p, C.c_void_p]
        L.or_q6k_block_sums.restype = None
        L.or_block_sums.argtypes = [C.c_int, _i8p, _u8p, C.c_size_t, C.c_size_t, _i32p]
        L.or_gemv_tq_i8.argtypes = [C.c_int, _i8p, C.c_float, _u8p, C.c_size_t,
                                    C.c_size_t, _f32p]
        L.or_gemv_qk_i8.argtypes = [C.c_int, _i8p, _f32p, _u8p, C.c_size_t,
                                    C.c_size_t, _f32p]
        L.or_gemv.argtypes = [C.c_int, _f32p, _u8p, C.c_size_t, C.c_size_t, _f32p, C.c_int]
        L.or_dequant_row.argtypes = [C.c_int, _u8p, C.c_size_t, _f32p]
        L.or_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_size_t, C.c_float]
        L.or_softmax.argtypes = [_f32p, C.c_size_t]
        L.or_silu_mul.argtypes = [_f32p, _f32p, C.c_size_t]
        L.or_rope.argtypes = [_f32p, C.c_size_t, C.c_size_t, _f32p, _f32p]
        L.or_rope_tables.argtypes = [_f32p, _f32p, C.c_size_t, C.c_size_t, C.c_float]
        L.or_argmax.argtypes = [_f32p, C.c_size_t]
        L.or_argmax.restype = C.c_uint32
        L.or_context_create.argtypes = [C.POINTER(OrModel), C.c_uint32, C.c_uint32,
                                        C.c_int, C.POINTER(C.c_void_p)]
        L.or_context_destroy.argtypes = [C.c_void_p]
        L.or_context_reset.argtypes = [C.c_void_p]
        L.or_eval.argtypes = [C.c_void_p, _u32p, C.c_size_t, C.POINTER(C.POINTER(C.c_float))]
        L.or_context_set_kv.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32,
                                        _f32p, _f32p]
        L.or_context_set_pos.argtypes = [C.c_void_p, C.c_uint32]
        L.or_context_pos.argtypes = [C.c_void_p]
        L.or_context_pos.restype = C.c_uint32

    # -- kernels
    def quantize(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        q = np.empty(x.size, np.int8)
        s = C.c_float()
        assert self.lib.or_quantize_act_i8(x, x.size, q, C.byref(s)) == 0
        return q, s.value

    def quantize_k(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        q = np.empty(x.size, np.int8)
        s = np.empty(x.size // 256, np.float32)
        self.lib.or_quantize_act_k(x, x.size, q, s)
        return q, s

    def block_sums(self, gtype, q, w, rows, cols):
        per = {34: 1, 35: 1, 12: 8, 14: 4}[gtype]
        out = np.empty(rows * (cols // 256) * per, np.int32)
        assert self.lib.or_block_sums(gtype, np.ascontiguousarray(q, np.int8),
                                      np.ascontiguousarray(w, np.uint8), rows, cols, out) == 0
        return out.reshape(rows, cols // 256, per) if per > 1 else out.reshape(rows, cols // 256)

    def gemv(self, gtype, x, w, rows, cols, n_threads=1):
        out = np.empty(rows, np.float32)
        st = self.lib.or_gemv(gtype, np.ascontiguousarray(x, np.float32),
                              np.ascontiguousarray(w, np.uint8), rows, cols, out, n_threads)
        assert st == 0, st
        return out

    def gemv_tq_i8(self, gtype, q, scale, w, rows, cols):
        out = np.empty(rows, np.float32)
        assert self.lib.or_gemv_tq_i8(gtype, q, scale, np.ascontiguousarray(w, np.uint8),
                                      rows, cols, out) == 0
        return out

    def gemv_qk_i8(self, gtype, q, ascale, w, rows, cols):
        out = np.empty(rows, np.float32)
        assert self.lib.or_gemv_qk_i8(gtype, q, ascale, np.ascontiguousarray(w, np.uint8),
                                      rows, cols, out) == 0
        return out

    def rmsnorm(self, x, w, eps):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self.lib.or_rmsnorm(out, x, np.ascontiguousarray(w, np.float32), x.size, eps)
        return out

    def rope(self, vec, n_heads, head_dim, cos_row, sin_row):
        v = np.array(vec, dtype=np.float32)
        self.lib.or_rope(v, n_heads, head_dim, np.ascontiguousarray(cos_row, np.float32),
                         np.ascontiguousarray(sin_row, np.float32))
        return v

    def silu_mul(self, gate, up):
        g = np.array(gate, dtype=np.float32)
        self.lib.or_silu_mul(g, np.ascontiguousarray(up, np.float32), g.size)
        return g

    def argmax(self, x):
        return int(self.lib.or_argmax(np.ascontiguousarray(x, np.float32), len(x)))

    def softmax(self, x):
        x = np.array(x, dtype=np.float32)
        self.lib.or_softmax(x, x.size)
        return x

    def dequant(self, gtype, row, n):
        out = np.empty(n, np.float32)
        assert self.lib.or_dequant_row(gtype, np.ascontiguousarray(row, np.uint8), n, out) == 0
        return out

    def rope_tables(self, n_ctx, head_dim, base):
        c = np.empty(n_ctx * (head_dim // 2), np.float32)
        s = np.empty_like(c)
        self.lib.or_rope_tables(c, s, n_ctx, head_dim, base)
        return c, s

    # -- forward
    def model(self, spec, tensors):
        """Build an or_model over the byte arrays of a synthetic model."""
        from rustfox_amd import synth
        keep = []

        def T(name):
            arr = np.ascontiguousarray(tensors[name])
            keep.append(arr)
            gt = {n: t for n, _, _, t in synth.tensor_list(spec)}[name]
            return OrTensor(_ptr(arr), gt)

        layers = (OrLayer * spec.n_layer)()
        for l in range(spec.n_layer):
            p = f"blk.{l}."
            layers[l] = OrLayer(T(p + "attn_norm.weight"), T(p + "attn_q.weight"),
                                T(p + "attn_k.weight"), T(p + "attn_v.weight"),
                                T(p + "attn_output.weight"), T(p + "ffn_norm.weight"),
                                T(p + "ffn_gate.weight"), T(p + "ffn_up.weight"),
                                T(p + "ffn_down.weight"))
        m = OrModel(spec.n_layer, spec.n_embd, spec.n_head, spec.n_head_kv, spec.head_dim,
                    spec.n_ff, spec.n_vocab, spec.rms_eps, spec.rope_base,
                    T("token_embd.weight"), T("output_norm.weight"), T("output.weight"),
                    layers)
        return OracleModel(self, m, layers, keep)


class OracleModel:
    def __init__(self, o, m, layers, keep):
        self.o, self.m, self._layers, self._keep = o, m, layers, keep

    def context(self, n_ctx, n_batch=32, n_threads=1):
        ctx = C.c_void_p()
        assert self.o.lib.or_context_create(C.byref(self.m), n_ctx, n_batch, n_threads,
                                            C.byref(ctx)) == 0
        return OracleContext(self, ctx)


class OracleContext:
    def __init__(self, model, ctx):
        self.model, self.ctx, self.lib = model, ctx, model.o.lib

    def eval(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        lp = C.POINTER(C.c_float)()
        st = self.lib.or_eval(self.ctx, t, t.size, C.byref(lp))
        assert st == 0, st
        return np.ctypeslib.as_array(lp, shape=(self.model.m.n_vocab,)).copy()

    def set_kv(self, layer, p0, k, v):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        n = k.shape[0]
        assert self.lib.or_context_set_kv(self.ctx, layer, p0, n, k, v) == 0

    def set_pos(self, pos):
        assert self.lib.or_context_set_pos(self.ctx, pos) == 0

    def reset(self):
        self.lib.or_context_reset(self.ctx)

    def close(self):
        if self.ctx:
            self.lib.or_context_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        self.close()


# ------------------------------------------------------------------ ref

class ContextConfig(C.Structure):
    _fields_ = [("n_ctx", C.c_uint32), ("n_batch", C.c_uint32), ("n_threads", C.c_int)]


class ModelInfo(C.Structure):
    _fields_ = [("arch", C.c_char * 32), ("name", C.c_char * 128), ("n_layer", C.c_uint32),
                ("n_embd", C.c_uint32), ("n_head", C.c_uint32), ("n_head_kv", C.c_uint32),
                ("n_ff", C.c_uint32), ("head_dim", C.c_uint32), ("n_vocab", C.c_uint32),
                ("n_ctx_train", C.c_uint32), ("rms_eps", C.c_float),
                ("rope_freq_base", C.c_float), ("weight_bytes", C.c_uint64),
                ("tied_output", C.c_int)]


def ref_available(path: str = REF_SO) -> bool:
    return os.path.exists(path)


class Ref:
    """The reference, compiled from its own sources (oracle/_ref)."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (make -C oracle ref)")
        L = self.lib = C.CDLL(path)
        L.fox_last_error.restype = C.c_char_p
        L.fox_threadpool_create.restype = C.c_void_p
        L.fox_threadpool_create.argtypes = [C.c_int]
        L.fox_threadpool_destroy.argtypes = [C.c_void_p]
        L.fox_quantize_activations_i8.argtypes = [_f32p, C.c_size_t, _i8p,
                                                  C.POINTER(C.c_float)]
        L.fox_tq1_dot_i8.argtypes = [_i8p, _u8p, C.c_size_t, C.POINTER(C.c_float)]
        L.fox_tq2_dot_i8.argtypes = [_i8p, _u8p, C.c_size_t, C.POINTER(C.c_float)]
        L.fox_gemv.argtypes = [C.c_void_p, C.c_int, _f32p, _u8p, C.c_size_t, C.c_size_t,
                               _f32p]
        L.fox_gemv_tq1_i8.argtypes = [C.c_void_p, _i8p, C.c_float, _u8p, C.c_size_t,
                                      C.c_size_t, _f32p]
        L.fox_gemv_tq2_i8.argtypes = L.fox_gemv_tq1_i8.argtypes
        L.fox_dequant_row.argtypes = [C.c_int, _u8p, C.c_size_t, _f32p]
        L.fox_f16_to_f32.restype = C.c_float
        L.fox_f16_to_f32.argtypes = [C.c_uint16]
        L.fox_f32_to_f16.restype = C.c_uint16
        L.fox_f32_to_f16.argtypes = [C.c_float]
        L.fox_model_open.argtypes = [C.c_char_p, C.c_int, C.c_uint64, C.POINTER(C.c_void_p)]
        L.fox_model_close.argtypes = [C.c_void_p]
        L.fox_model_get_info.restype = C.POINTER(ModelInfo)
        L.fox_model_get_info.argtypes = [C.c_void_p]
        L.fox_context_config_default.argtypes = [C.POINTER(ContextConfig), C.c_void_p]
        L.fox_context_create.argtypes = [C.c_void_p, C.POINTER(ContextConfig),
                                         C.POINTER(C.c_void_p)]
        L.fox_context_destroy.argtypes = [C.c_void_p]
        L.fox_context_reset.argtypes = [C.c_void_p]
        L.fox_eval.argtypes = [C.c_void_p, _u32p, C.c_size_t, C.POINTER(C.POINTER(C.c_float))]
        L.fox_context_last_eval_seconds.restype = C.c_double
        L.fox_context_last_eval_seconds.argtypes = [C.c_void_p]

    def err(self):
        e = self.lib.fox_last_error()
        return e.decode() if e else ""

    def quantize(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        q = np.empty(x.size, np.int8)
        s = C.c_float()
        assert self.lib.fox_quantize_activations_i8(x, x.size, q, C.byref(s)) == 0
        return q, s.value

    def gemv(self, gtype, x, w, rows, cols, n_threads=0):
        out = np.empty(rows, np.float32)
        tp = self.lib.fox_threadpool_create(n_threads) if n_threads != 1 else None
        try:
            st = self.lib.fox_gemv(tp, gtype, np.ascontiguousarray(x, np.float32),
                                   np.ascontiguousarray(w, np.uint8), rows, cols, out)
        finally:
            if tp:
                self.lib.fox_threadpool_destroy(tp)
        assert st == 0, (st, self.err())
        return out

    def gemv_tq_i8(self, gtype, q, scale, w, rows, cols):
        out = np.empty(rows, np.float32)
        f = self.lib.fox_gemv_tq1_i8 if gtype == 34 else self.lib.fox_gemv_tq2_i8
        assert f(None, q, scale, np.ascontiguousarray(w, np.uint8), rows, cols, out) == 0
        return out

    def dequant(self, gtype, row, n):
        out = np.empty(n, np.float32)
        assert self.lib.fox_dequant_row(gtype, np.ascontiguousarray(row, np.uint8), n, out) == 0
        return out

    def open_model(self, path):
        m = C.c_void_p()
        st = self.lib.fox_model_open(path.encode(), 0, 0, C.byref(m))
        assert st == 0, (st, self.err())
        return RefModel(self, m)


class RefModel:
    def __init__(self, ref, m):
        self.ref, self.m, self.lib = ref, m, ref.lib
        self.info = self.lib.fox_model_get_info(m).contents

    def context(self, n_ctx, n_batch=32, n_threads=1):
        cfg = ContextConfig()
        self.lib.fox_context_config_default(C.byref(cfg), self.m)
        cfg.n_ctx, cfg.n_batch, cfg.n_threads = n_ctx, n_batch, n_threads
        ctx = C.c_void_p()
        st = self.lib.fox_context_create(self.m, C.byref(cfg), C.byref(ctx))
        assert st == 0, (st, self.ref.err())
        return RefContext(self, ctx)

    def close(self):
        if self.m:
            self.lib.fox_model_close(self.m)
            self.m = None


class RefContext:
    def __init__(self, model, ctx):
        self.model, self.ctx, self.lib = model, ctx, model.lib

    def eval(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        lp = C.POINTER(C.c_float)()
        st = self.lib.fox_eval(self.ctx, t, t.size, C.byref(lp))
        assert st == 0, (st, self.model.ref.err())
        return np.ctypeslib.as_array(lp, shape=(self.model.info.n_vocab,)).copy()

    def last_seconds(self):
        return self.lib.fox_context_last_eval_seconds(self.ctx)

    def reset(self):
        self.lib.fox_context_reset(self.ctx)

    def close(self):
        if self.ctx:
            self.lib.fox_context_destroy(self.ctx)
            self.ctx = None
