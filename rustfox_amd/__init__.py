"""rustfox_amd -- MI355X (gfx950) decode path for RustFox.

Python view of the two native libraries built by ``make -C rustfox_amd``:

  lib/librustfox_amd.so  the HIP kernels behind the C ABI of include/fox_gpu.h
  lib/libfox.so          the C host library that keeps RustFox's API
                         (fox_model_open, fox_eval, ...) over that ABI

There is no CPU fallback: if the native library is missing, loading fails
with an error that says how to build it.
"""
from __future__ import annotations

import ctypes as C
import os
import weakref

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GPU_LIB = os.path.join(HERE, "lib", "librustfox_amd.so")
HOST_LIB = os.path.join(HERE, "lib", "libfox.so")

F32, F16, Q4_K, Q6_K, TQ1_0, TQ2_0 = 0, 1, 12, 14, 34, 35
ACT_PER_VECTOR, ACT_PER_BLOCK = 0, 1
GEMV_ACCUMULATE = 1
ATTN_SPLIT, ATTN_EXACT = 0, 1
MAX_TOKENS = 8

STATUS = ["OK", "ERR_ARG", "ERR_IO", "ERR_NOMEM", "ERR_FORMAT", "ERR_UNSUPPORTED",
          "ERR_NOTFOUND", "ERR_INTERNAL"]


class FoxError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{STATUS[status] if 0 <= status < len(STATUS) else status}: {msg}")
        self.status = status


_gpu = None


PROBE_LIB = os.path.join(HERE, "lib", "librustfox_probe.so")
_probe = None


def probe_lib() -> C.CDLL:
    """bench.py's diagnostics (read ceiling, launch cost): a separate
    library, not part of the decode ABI."""
    global _probe
    if _probe is None:
        gpu_lib()
        L = C.CDLL(PROBE_LIB)
        vp, sz = C.c_void_p, C.c_size_t
        L.fox_gpu_read_probe.argtypes = [vp, vp, sz, C.c_int, C.c_int, vp]
        L.fox_gpu_empty_probe.argtypes = [vp, C.c_int, vp]
        L.fox_gpu_sum_probe.argtypes = [vp, vp, C.c_int, C.c_float, vp]
        _probe = L
    return _probe


def gpu_lib() -> C.CDLL:
    """Load librustfox_amd.so (raises if it has not been built)."""
    global _gpu
    if _gpu is not None:
        return _gpu
    if not os.path.exists(GPU_LIB):
        raise FileNotFoundError(f"{GPU_LIB} is missing: build it with `make -C rustfox_amd` "
                                "(or __graft_entry__.build()); there is no CPU fallback")
    L = C.CDLL(GPU_LIB)
    vp, sz, u32p = C.c_void_p, C.c_size_t, C.POINTER(C.c_uint32)
    sigs = {
        "fox_gpu_init": [C.c_int, C.POINTER(vp)],
        "fox_gpu_shutdown": [vp],
        "fox_gpu_device_info": [vp, C.c_char_p, sz, C.POINTER(C.c_int), C.POINTER(C.c_uint64)],
        "fox_gpu_set_max_workgroups": [vp, C.c_int],
        "fox_gpu_malloc": [vp, sz, C.POINTER(vp)],
        "fox_gpu_free": [vp, vp],
        "fox_gpu_memcpy_h2d": [vp, vp, vp, sz],
        "fox_gpu_memcpy_d2h": [vp, vp, vp, sz],
        "fox_gpu_memcpy_d2d": [vp, vp, vp, sz],
        "fox_gpu_memset": [vp, vp, C.c_int, sz],
        "fox_gpu_sync": [vp],
        "fox_gpu_tensor_upload": [vp, C.c_int, C.c_uint64, C.c_uint64, vp, C.c_uint64,
                                  C.POINTER(vp)],
        "fox_gpu_tensor_info": [vp, C.POINTER(C.c_int), C.POINTER(C.c_uint64),
                                C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                C.POINTER(C.c_uint64)],
        "fox_gpu_tensor_download": [vp, vp, vp, C.c_uint64],
        "fox_gpu_tensor_free": [vp, vp],
        "fox_gpu_quantize": [vp, C.c_int, vp, sz, sz, sz, vp, vp],
        "fox_gpu_gemv": [vp, vp, vp, sz, sz, vp, sz, C.c_uint],
        "fox_gpu_gemv_noalloc": [vp, vp, vp, sz, sz, vp, sz, C.c_uint],
        "fox_gpu_gemv_multi": [vp, sz, C.POINTER(vp), vp, sz, sz, C.POINTER(vp),
                               C.POINTER(sz), C.c_uint],
        "fox_gpu_gemv_i8": [vp, vp, vp, vp, sz, vp, sz],
        "fox_gpu_block_sums": [vp, vp, vp, sz, vp],
        "fox_gpu_act_prepare": [vp, C.c_int, vp, sz, sz, sz, C.POINTER(vp)],
        "fox_gpu_gemv_act": [vp, vp, vp, vp, sz, C.c_uint],
        "fox_gpu_act_free": [vp, vp],
        "fox_gpu_get_rows": [vp, vp, vp, sz, vp, sz, vp],
        "fox_gpu_rmsnorm": [vp, vp, sz, vp, sz, vp, sz, sz, C.c_float],
        "fox_gpu_rope_store": [vp, vp, sz, vp, sz, vp, sz, sz, sz, sz, sz, vp, vp, vp, sz,
                               vp, vp],
        "fox_gpu_attention": [vp, vp, sz, vp, sz, vp, vp, sz, sz, sz, sz, vp, sz, C.c_int],
        "fox_gpu_kv_write": [vp, vp, vp, sz, sz, sz, sz, vp, vp],
        "fox_gpu_gemv_rmsnorm": [vp, sz, C.POINTER(vp), vp, sz, sz, vp, C.c_float,
                                 C.POINTER(vp), C.POINTER(sz), C.c_uint],
        "fox_gpu_qkv_rope": [vp, vp, vp, vp, vp, sz, sz, vp, C.c_float, vp, sz, vp, vp, vp, sz,
                             vp, vp, sz],
        "fox_gpu_gate_up_silu": [vp, vp, vp, vp, sz, sz, vp, C.c_float, vp, sz],
        "fox_gpu_silu_mul": [vp, vp, vp, sz, sz, sz],
        "fox_gpu_add": [vp, vp, vp, sz, sz, sz],
        "fox_gpu_argmax": [vp, vp, sz, vp, vp, C.c_uint32, vp],
        "fox_gpu_graph_begin": [vp],
        "fox_gpu_graph_end": [vp, C.POINTER(vp)],
        "fox_gpu_graph_launch": [vp, vp],
        "fox_gpu_graph_free": [vp],
        "fox_gpu_event_create": [vp, C.POINTER(vp)],
        "fox_gpu_event_record": [vp, vp],
        "fox_gpu_event_elapsed": [vp, vp, C.POINTER(C.c_float)],
        "fox_gpu_event_destroy": [vp],
    }
    for name, args in sigs.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = None if name in ("fox_gpu_shutdown", "fox_gpu_tensor_free", "fox_gpu_act_free",
                                     "fox_gpu_graph_free", "fox_gpu_event_destroy") else C.c_int
    L.fox_gpu_last_error.restype = C.c_char_p
    L.fox_gpu_last_error.argtypes = []
    L.fox_gpu_workspace_bytes.restype = C.c_size_t
    L.fox_gpu_workspace_bytes.argtypes = [vp]
    _gpu = L
    return L


def _check(st: int):
    if st != 0:
        msg = gpu_lib().fox_gpu_last_error()
        raise FoxError(st, msg.decode() if msg else "")


class DeviceArray:
    """A device allocation with a numpy dtype and shape (no compute)."""

    def __init__(self, gpu: "Gpu", shape, dtype):
        self.gpu = gpu
        self.shape = tuple(shape) if isinstance(shape, (tuple, list)) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = C.c_void_p()
        _check(gpu.lib.fox_gpu_malloc(gpu.ctx, max(self.nbytes, 1), C.byref(p)))
        self.ptr = p.value

    def upload(self, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        _check(self.gpu.lib.fox_gpu_memcpy_h2d(self.gpu.ctx, self.ptr, a.ctypes.data, a.nbytes))
        return self

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        _check(self.gpu.lib.fox_gpu_memcpy_d2h(self.gpu.ctx, out.ctypes.data, self.ptr,
                                                self.nbytes))
        return out

    def fill(self, byte: int = 0) -> "DeviceArray":
        _check(self.gpu.lib.fox_gpu_memset(self.gpu.ctx, self.ptr, byte, self.nbytes))
        return self

    def at(self, offset_elems: int) -> int:
        return self.ptr + offset_elems * self.dtype.itemsize

    def free(self):
        if self.ptr:
            self.gpu.lib.fox_gpu_free(self.gpu.ctx, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and self.gpu.ctx:
                self.free()
        except Exception:
            pass


class Tensor:
    """A weight tensor resident in HBM (fox_gpu_tensor)."""

    def __init__(self, gpu: "Gpu", gtype: int, ne0: int, ne1: int, data: np.ndarray):
        self.gpu, self.type, self.ne0, self.ne1 = gpu, gtype, ne0, max(ne1, 1)
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        h = C.c_void_p()
        _check(gpu.lib.fox_gpu_tensor_upload(gpu.ctx, gtype, ne0, ne1, data.ctypes.data,
                                             data.nbytes, C.byref(h)))
        self.h = h.value
        self.gguf_bytes = data.nbytes

    def info(self):
        t, a, b, g, d = C.c_int(), C.c_uint64(), C.c_uint64(), C.c_uint64(), C.c_uint64()
        _check(self.gpu.lib.fox_gpu_tensor_info(self.h, C.byref(t), C.byref(a), C.byref(b),
                                                C.byref(g), C.byref(d)))
        return dict(type=t.value, ne0=a.value, ne1=b.value, gguf_bytes=g.value,
                    device_bytes=d.value)

    def download(self) -> np.ndarray:
        out = np.empty(self.gguf_bytes, np.uint8)
        _check(self.gpu.lib.fox_gpu_tensor_download(self.gpu.ctx, self.h, out.ctypes.data,
                                                    out.nbytes))
        return out

    def free(self):
        if self.h:
            self.gpu.lib.fox_gpu_tensor_free(self.gpu.ctx, self.h)
            self.h = None

    def __del__(self):
        try:
            if self.h and self.gpu.ctx:
                self.free()
        except Exception:
            pass


class Gpu:
    """One device context (one HIP stream) of librustfox_amd.so."""

    def __init__(self, device: int = 0):
        self.lib = gpu_lib()
        ctx = C.c_void_p()
        _check(self.lib.fox_gpu_init(device, C.byref(ctx)))
        self.ctx = ctx.value

    def close(self):
        if self.ctx:
            self.lib.fox_gpu_shutdown(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def set_max_workgroups(self, n: int):
        """Cap the fused GEMVs' persistent grid (0: two per compute unit)."""
        _check(self.lib.fox_gpu_set_max_workgroups(self.ctx, n))

    def workspace_bytes(self) -> int:
        """Device bytes the context's workspace holds now."""
        return int(self.lib.fox_gpu_workspace_bytes(self.ctx))

    def info(self):
        name = C.create_string_buffer(128)
        cu, hbm = C.c_int(), C.c_uint64()
        _check(self.lib.fox_gpu_device_info(self.ctx, name, 128, C.byref(cu), C.byref(hbm)))
        return dict(name=name.value.decode(), compute_units=cu.value, hbm_bytes=hbm.value)

    # -- memory
    def empty(self, shape, dtype) -> DeviceArray:
        return DeviceArray(self, shape, dtype)

    def array(self, a: np.ndarray) -> DeviceArray:
        a = np.ascontiguousarray(a)
        return DeviceArray(self, a.shape, a.dtype).upload(a)

    def tensor(self, gtype, ne0, ne1, data) -> Tensor:
        return Tensor(self, gtype, ne0, ne1, data)

    def sync(self):
        _check(self.lib.fox_gpu_sync(self.ctx))

    def copy(self, dst: DeviceArray, src: DeviceArray, nbytes: int):
        """Device-to-device copy on the context's stream (fox_gpu_memcpy_d2d)."""
        _check(self.lib.fox_gpu_memcpy_d2d(self.ctx, dst.ptr, src.ptr, nbytes))

    def read_probe(self, src: DeviceArray, nbytes: int, loads: int, grid: int, sink: DeviceArray):
        """Streaming read of nbytes with `loads` 16-byte loads in flight per
        thread (a diagnostic of the HBM read ceiling, from the bench-only
        librustfox_probe.so)."""
        _check(probe_lib().fox_gpu_read_probe(self.ctx, src.ptr, nbytes, loads, grid, sink.ptr))

    def empty_probe(self, grid: int, sink: DeviceArray):
        """One empty kernel of `grid` workgroups (librustfox_probe.so)."""
        _check(probe_lib().fox_gpu_empty_probe(self.ctx, grid, sink.ptr))

    def sum_probe(self, e: DeviceArray, n: int, acc: float, out: DeviceArray):
        """The attention kernels' whole-wave in-order softmax sum of n floats
        from acc into out[0] and the one-add-at-a-time chain's into out[2]
        (out[1], out[3]: their shader clocks; librustfox_probe.so, for its
        tests)."""
        _check(probe_lib().fox_gpu_sum_probe(self.ctx, e.ptr, n, acc, out.ptr))

    # -- compute (device arrays in, device arrays out)
    def quantize(self, mode, x: DeviceArray, K, M, x_stride, q: DeviceArray, scale: DeviceArray):
        _check(self.lib.fox_gpu_quantize(self.ctx, mode, x.ptr, K, M, x_stride, q.ptr, scale.ptr))

    def gemv(self, w: Tensor, x: DeviceArray, M, out: DeviceArray, x_stride=None,
             out_stride=None, flags=0):
        _check(self.lib.fox_gpu_gemv(self.ctx, w.h, x.ptr, x_stride or w.ne0, M, out.ptr,
                                     out_stride or w.ne1, flags))

    def gemv_multi(self, ws, x: DeviceArray, M, outs, x_stride=None, out_strides=None, flags=0):
        n = len(ws)
        hs = (C.c_void_p * n)(*[w.h for w in ws])
        os_ = (C.c_void_p * n)(*[o.ptr for o in outs])
        st = (C.c_size_t * n)(*(out_strides or [w.ne1 for w in ws]))
        _check(self.lib.fox_gpu_gemv_multi(self.ctx, n, hs, x.ptr, x_stride or ws[0].ne0, M,
                                           os_, st, flags))

    def gemv_i8(self, w: Tensor, q: DeviceArray, scale: DeviceArray, M, out: DeviceArray,
                out_stride=None):
        _check(self.lib.fox_gpu_gemv_i8(self.ctx, w.h, q.ptr, scale.ptr, M, out.ptr,
                                        out_stride or w.ne1))

    def act_prepare(self, gtype, x: DeviceArray, K, M, x_stride=None):
        a = C.c_void_p()
        _check(self.lib.fox_gpu_act_prepare(self.ctx, gtype, x.ptr, K, M, x_stride or K,
                                            C.byref(a)))
        return a.value

    def gemv_act(self, w: Tensor, act, out: DeviceArray, out_stride=None, flags=0):
        _check(self.lib.fox_gpu_gemv_act(self.ctx, w.h, act, out.ptr, out_stride or w.ne1, flags))

    def act_free(self, act):
        self.lib.fox_gpu_act_free(self.ctx, act)

    def block_sums(self, w: Tensor, q: DeviceArray, M, sums: DeviceArray):
        _check(self.lib.fox_gpu_block_sums(self.ctx, w.h, q.ptr, M, sums.ptr))

    def gemv_rmsnorm(self, ws, x: DeviceArray, M, norm: DeviceArray, eps, outs, flags=0):
        n = len(ws)
        wa = (C.c_void_p * n)(*[w.h for w in ws])
        oa = (C.c_void_p * n)(*[o.ptr for o in outs])
        sa = (C.c_size_t * n)(*[w.info()["ne1"] for w in ws])
        K = ws[0].info()["ne0"]
        _check(self.lib.fox_gpu_gemv_rmsnorm(self.ctx, n, wa, x.ptr, K, M, norm.ptr, eps, oa, sa,
                                             flags))

    def qkv_rope(self, wq, wk, wv, x: DeviceArray, M, norm: DeviceArray, eps, q_out: DeviceArray,
                 cos_t: DeviceArray, sin_t: DeviceArray, pos: DeviceArray, n_ctx, kc: DeviceArray,
                 vc: DeviceArray, head_dim):
        K, nq = wq.info()["ne0"], wq.info()["ne1"]
        _check(self.lib.fox_gpu_qkv_rope(self.ctx, wq.h, wk.h, wv.h, x.ptr, K, M, norm.ptr, eps,
                                         q_out.ptr, nq, cos_t.ptr, sin_t.ptr, pos.ptr, n_ctx,
                                         kc.ptr, vc.ptr, head_dim))

    def gate_up_silu(self, wg, wu, x: DeviceArray, M, norm: DeviceArray, eps, h: DeviceArray):
        K, ff = wg.info()["ne0"], wg.info()["ne1"]
        _check(self.lib.fox_gpu_gate_up_silu(self.ctx, wg.h, wu.h, x.ptr, K, M, norm.ptr, eps,
                                             h.ptr, ff))

    def rmsnorm(self, out: DeviceArray, x: DeviceArray, w: DeviceArray, n, M, eps,
                out_stride=None, x_stride=None):
        _check(self.lib.fox_gpu_rmsnorm(self.ctx, out.ptr, out_stride or n, x.ptr, x_stride or n,
                                        w.ptr if w else None, n, M, eps))

    def argmax(self, logits: DeviceArray, n, idx: DeviceArray, pos: DeviceArray = None,
               advance=0, history: DeviceArray = None):
        _check(self.lib.fox_gpu_argmax(self.ctx, logits.ptr, n, idx.ptr, pos.ptr if pos else None,
                                       advance, history.ptr if history else None))

    def kv_write(self, kc: DeviceArray, vc: DeviceArray, kv_dim, n_ctx, p0, k: DeviceArray,
                 v: DeviceArray, n):
        _check(self.lib.fox_gpu_kv_write(self.ctx, kc.ptr, vc.ptr, kv_dim, n_ctx, p0, n, k.ptr,
                                         v.ptr))

    def attention(self, out: DeviceArray, q: DeviceArray, kc: DeviceArray, vc: DeviceArray,
                  n_head, n_head_kv, head_dim, M, pos: DeviceArray, n_ctx, mode,
                  q_stride=None, out_stride=None):
        w = n_head * head_dim
        _check(self.lib.fox_gpu_attention(self.ctx, out.ptr, out_stride or w, q.ptr,
                                          q_stride or w, kc.ptr, vc.ptr, n_head, n_head_kv,
                                          head_dim, M, pos.ptr, n_ctx, mode))

    def event(self):
        e = C.c_void_p()
        _check(self.lib.fox_gpu_event_create(self.ctx, C.byref(e)))
        return e.value

    def record(self, e):
        _check(self.lib.fox_gpu_event_record(self.ctx, e))

    def elapsed_ms(self, a, b) -> float:
        ms = C.c_float()
        _check(self.lib.fox_gpu_event_elapsed(a, b, C.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ----------------------------------------------------------------- host API

WEIGHTS_RESIDENT, WEIGHTS_STREAM, WEIGHTS_DEVICE = 0, 1, 2
_host = None


class ModelInfo(C.Structure):
    """fox_model_info (include/fox_host.h)."""
    _fields_ = [("arch", C.c_char * 32), ("name", C.c_char * 128), ("n_layer", C.c_uint32),
                ("n_embd", C.c_uint32), ("n_head", C.c_uint32), ("n_head_kv", C.c_uint32),
                ("n_ff", C.c_uint32), ("head_dim", C.c_uint32), ("n_vocab", C.c_uint32),
                ("n_ctx_train", C.c_uint32), ("rms_eps", C.c_float),
                ("rope_freq_base", C.c_float), ("weight_bytes", C.c_uint64),
                ("tied_output", C.c_int)]


class ContextConfig(C.Structure):
    _fields_ = [("n_ctx", C.c_uint32), ("n_batch", C.c_uint32), ("n_threads", C.c_int)]


class SamplerConfig(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float),
                ("repeat_penalty", C.c_float), ("repeat_last_n", C.c_uint32),
                ("seed", C.c_uint64)]


class Lease(C.Structure):
    _fields_ = [("data", C.c_void_p), ("bytes", C.c_uint64), ("tensor_index", C.c_size_t),
                ("slot", C.c_void_p)]


def host_lib() -> C.CDLL:
    """Load libfox.so (the RustFox host API over the GPU path)."""
    global _host
    if _host is not None:
        return _host
    if not os.path.exists(HOST_LIB):
        raise FileNotFoundError(f"{HOST_LIB} is missing: build it with `make -C rustfox_amd`")
    L = C.CDLL(HOST_LIB)
    vp, sz, u32 = C.c_void_p, C.c_size_t, C.c_uint32
    u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
    f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
    sigs = {
        "fox_model_open": ([C.c_char_p, C.c_int, C.c_uint64, C.POINTER(vp)], C.c_int),
        "fox_model_close": ([vp], None),
        "fox_model_get_info": ([vp], C.POINTER(ModelInfo)),
        "fox_model_weights": ([vp], vp),
        "fox_context_config_default": ([C.POINTER(ContextConfig), vp], None),
        "fox_context_create": ([vp, C.POINTER(ContextConfig), C.POINTER(vp)], C.c_int),
        "fox_context_destroy": ([vp], None),
        "fox_context_reset": ([vp], None),
        "fox_eval": ([vp, u32p, sz, C.POINTER(C.POINTER(C.c_float))], C.c_int),
        "fox_eval_all": ([vp, u32p, sz, C.POINTER(C.c_float)], C.c_int),
        "fox_decode_greedy": ([vp, u32, sz, u32p], C.c_int),
        "fox_context_position": ([vp], u32),
        "fox_context_last_eval_seconds": ([vp], C.c_double),
        "fox_context_weight_reads": ([vp], C.c_uint64),
        "fox_context_set_kv": ([vp, u32, u32, u32, f32p, f32p], C.c_int),
        "fox_context_set_position": ([vp, u32], C.c_int),
        "fox_context_set_attention": ([vp, C.c_int], C.c_int),
        "fox_weights_open": ([C.c_char_p, C.c_int, C.c_uint64, C.POINTER(vp)], C.c_int),
        "fox_weights_close": ([vp], None),
        "fox_weights_get_mode": ([vp], C.c_int),
        "fox_weights_tensor_count": ([vp], sz),
        "fox_weights_tensor_find": ([vp, C.c_char_p], sz),
        "fox_weights_acquire": ([vp, sz, C.POINTER(Lease)], C.c_int),
        "fox_weights_release": ([vp, C.POINTER(Lease)], None),
        "fox_weights_prefetch": ([vp, sz], C.c_int),
        "fox_weights_prefetch_async": ([vp, sz], C.c_int),
        "fox_weights_prefetch_wait": ([vp, sz], C.c_int),
        "fox_weights_live_leases": ([vp], sz),
        "fox_weights_resident_bytes": ([vp], C.c_uint64),
        "fox_weights_reads": ([vp], C.c_uint64),
        "fox_weights_evictions": ([vp], C.c_uint64),
        "fox_sampler_config_default": ([C.POINTER(SamplerConfig)], None),
        "fox_sampler_create": ([C.POINTER(SamplerConfig), sz], vp),
        "fox_sampler_destroy": ([vp], None),
        "fox_sampler_accept": ([vp, u32], None),
        "fox_sampler_pick": ([vp, f32p, C.POINTER(u32)], C.c_int),
        "fox_gemv_supports": ([C.c_int], C.c_int),
        "fox_row_bytes": ([C.c_int, sz], sz),
        "fox_last_error": ([], C.c_char_p),
        "fox_version": ([], C.c_char_p),
    }
    for name, (args, res) in sigs.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _host = L
    return L


def _hcheck(st: int):
    if st != 0:
        msg = host_lib().fox_last_error()
        raise FoxError(st, msg.decode() if msg else "")


class Model:
    """fox_model_open(path, mode): the RustFox model API on the GPU build."""

    def __init__(self, path: str, mode: int = WEIGHTS_DEVICE, budget: int = 0):
        self.lib = host_lib()
        m = C.c_void_p()
        _hcheck(self.lib.fox_model_open(path.encode(), mode, budget, C.byref(m)))
        self.m = m.value
        self.info = self.lib.fox_model_get_info(self.m).contents
        self._contexts = weakref.WeakSet()

    def context(self, n_ctx: int = 0, n_batch: int = 32) -> "Context":
        c = Context(self, n_ctx, n_batch)
        self._contexts.add(c)
        return c

    def weights(self):
        return self.lib.fox_model_weights(self.m)

    def close(self):
        """Destroys the model's live contexts first: a context uses the
        model's device and weights (fox_context_destroy after fox_model_close
        would touch freed memory)."""
        for c in list(self._contexts):
            c.close()
        if self.m:
            self.lib.fox_model_close(self.m)
            self.m = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Context:
    def __init__(self, model: Model, n_ctx: int = 0, n_batch: int = 32):
        self.model, self.lib = model, model.lib
        cfg = ContextConfig()
        self.lib.fox_context_config_default(C.byref(cfg), model.m)
        if n_ctx:
            cfg.n_ctx = n_ctx
        cfg.n_batch = n_batch
        ctx = C.c_void_p()
        _hcheck(self.lib.fox_context_create(model.m, C.byref(cfg), C.byref(ctx)))
        self.ctx = ctx.value

    def eval(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(np.atleast_1d(tokens), dtype=np.uint32)
        lp = C.POINTER(C.c_float)()
        _hcheck(self.lib.fox_eval(self.ctx, t, t.size, C.byref(lp)))
        return np.ctypeslib.as_array(lp, shape=(self.model.info.n_vocab,)).copy()

    def eval_all(self, tokens) -> np.ndarray:
        """Logits of every position, one row per token."""
        t = np.ascontiguousarray(np.atleast_1d(tokens), dtype=np.uint32)
        out = np.empty((t.size, self.model.info.n_vocab), np.float32)
        _hcheck(self.lib.fox_eval_all(self.ctx, t, t.size,
                                      out.ctypes.data_as(C.POINTER(C.c_float))))
        return out

    def decode_greedy(self, token: int, n_steps: int) -> np.ndarray:
        out = np.zeros(n_steps, np.uint32)
        _hcheck(self.lib.fox_decode_greedy(self.ctx, int(token), n_steps, out))
        return out

    def set_kv(self, layer, p0, k, v):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        _hcheck(self.lib.fox_context_set_kv(self.ctx, layer, p0, k.shape[0], k, v))

    def set_position(self, pos):
        _hcheck(self.lib.fox_context_set_position(self.ctx, pos))

    def set_attention(self, exact: bool):
        _hcheck(self.lib.fox_context_set_attention(self.ctx, 1 if exact else 0))

    @property
    def position(self) -> int:
        return self.lib.fox_context_position(self.ctx)

    @property
    def last_seconds(self) -> float:
        return self.lib.fox_context_last_eval_seconds(self.ctx)

    def reset(self):
        self.lib.fox_context_reset(self.ctx)

    def close(self):
        if self.ctx:
            self.lib.fox_context_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Sampler:
    def __init__(self, n_vocab: int, temperature=None, **kw):
        self.lib = host_lib()
        cfg = SamplerConfig()
        self.lib.fox_sampler_config_default(C.byref(cfg))
        if temperature is not None:
            cfg.temperature = temperature
        for k, v in kw.items():
            setattr(cfg, k, v)
        self.s = self.lib.fox_sampler_create(C.byref(cfg), n_vocab)
        if not self.s:
            raise FoxError(1, host_lib().fox_last_error().decode())

    def accept(self, tok):
        self.lib.fox_sampler_accept(self.s, int(tok))

    def pick(self, logits) -> int:
        out = C.c_uint32()
        _hcheck(self.lib.fox_sampler_pick(self.s, np.ascontiguousarray(logits, np.float32),
                                          C.byref(out)))
        return out.value

    def __del__(self):
        try:
            if self.s:
                self.lib.fox_sampler_destroy(self.s)
                self.s = None
        except Exception:
            pass
