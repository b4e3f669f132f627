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

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GPU_LIB = os.path.join(HERE, "lib", "librustfox_amd.so")
HOST_LIB = os.path.join(HERE, "lib", "libfox.so")

F32, F16, Q4_K, Q6_K, TQ1_0, TQ2_0 = 0, 1, 12, 14, 34, 35
ACT_PER_VECTOR, ACT_PER_BLOCK = 0, 1
GEMV_ACCUMULATE = 1
MAX_TOKENS = 8

STATUS = ["OK", "ERR_ARG", "ERR_IO", "ERR_NOMEM", "ERR_FORMAT", "ERR_UNSUPPORTED",
          "ERR_NOTFOUND", "ERR_INTERNAL"]


class FoxError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{STATUS[status] if 0 <= status < len(STATUS) else status}: {msg}")
        self.status = status


_gpu = None


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
        "fox_gpu_gemv_multi": [vp, sz, C.POINTER(vp), vp, sz, sz, C.POINTER(vp),
                               C.POINTER(sz), C.c_uint],
        "fox_gpu_gemv_i8": [vp, vp, vp, vp, sz, vp, sz],
        "fox_gpu_block_sums": [vp, vp, vp, sz, vp],
        "fox_gpu_get_rows": [vp, vp, vp, sz, vp, sz, vp],
        "fox_gpu_rmsnorm": [vp, vp, sz, vp, sz, vp, sz, sz, C.c_float],
        "fox_gpu_rope_store": [vp, vp, sz, vp, sz, vp, sz, sz, sz, sz, sz, vp, vp, vp, sz,
                               vp, vp],
        "fox_gpu_attention": [vp, vp, sz, vp, sz, vp, vp, sz, sz, sz, sz, vp, sz],
        "fox_gpu_silu_mul": [vp, vp, vp, sz, sz, sz],
        "fox_gpu_add": [vp, vp, vp, sz, sz, sz],
        "fox_gpu_argmax": [vp, vp, sz, vp, vp, C.c_uint32],
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
        f.restype = None if name in ("fox_gpu_shutdown", "fox_gpu_tensor_free",
                                     "fox_gpu_graph_free", "fox_gpu_event_destroy") else C.c_int
    L.fox_gpu_last_error.restype = C.c_char_p
    L.fox_gpu_last_error.argtypes = []
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

    def block_sums(self, w: Tensor, q: DeviceArray, M, sums: DeviceArray):
        _check(self.lib.fox_gpu_block_sums(self.ctx, w.h, q.ptr, M, sums.ptr))

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
