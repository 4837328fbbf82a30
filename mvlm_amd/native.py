"""ctypes binding of libmvlm_hip.so (the C ABI declared in include/mvlm_hip.h).

The Python side only moves buffers and calls the C ABI; every computation runs
in the HIP library.  If the library has not been built, importing the binding
raises instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, byref, c_char_p, c_double, c_float, c_int, c_int64, c_size_t, c_uint64, c_void_p

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("MVLM_LIB_PATH") or os.path.join(PKG, "lib", "libmvlm_hip.so")

F32, F16, Q4_0, Q8_0, BF16 = 0, 1, 2, 8, 30
LAYOUT_NK, LAYOUT_KN = 0, 1
DTYPE_SIZE = {F32: 4, F16: 2, BF16: 2}
DTYPE_NAMES = {F32: "f32", F16: "f16", BF16: "bf16", Q8_0: "q8_0", Q4_0: "q4_0"}

OK = 0
ERR_INVALID_ARG, ERR_NO_DEVICE, ERR_OUT_OF_MEMORY, ERR_HIP, ERR_UNSUPPORTED, ERR_BUFFER_TOO_SMALL = -1, -2, -3, -4, -5, -6
ERR_NOT_FOUND, ERR_FORMAT = -7, -8


class MvlmError(RuntimeError):
    def __init__(self, code: int, fn: str, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.code = code


class DeviceInfo(ctypes.Structure):
    _fields_ = [("device_name", ctypes.c_char * 256), ("arch_name", ctypes.c_char * 64),
                ("ordinal", c_int), ("compute_units", c_int), ("max_clock_mhz", c_int),
                ("memory_clock_mhz", c_int), ("memory_bus_width_bits", c_int), ("wavefront_size", c_int),
                ("global_mem_size", c_uint64), ("local_mem_size", c_uint64), ("l2_cache_size", c_uint64),
                ("peak_hbm_gbs", c_double), ("peak_fp16_tflops", c_double),
                ("box_peak_hbm_gbs", c_double), ("box_peak_fp16_tflops", c_double)]


class GgufInfo(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint32), ("tensor_count", c_uint64), ("metadata_kv_count", c_uint64),
                ("alignment", c_uint64), ("data_offset", c_uint64), ("file_size", c_uint64)]


class GgufTensor(ctypes.Structure):
    _fields_ = [("name", c_void_p), ("name_len", c_uint64), ("n_dims", ctypes.c_uint32),
                ("dims", c_uint64 * 4), ("type", ctypes.c_uint32), ("offset", c_uint64), ("bytes", c_uint64)]


ACT_NONE, ACT_GELU_TANH, ACT_SILU = 0, 1, 2


class Epilogue(ctypes.Structure):
    _fields_ = [("bias", c_void_p), ("activation", c_int), ("mul", c_void_p), ("residual", c_void_p)]


def _epilogue(bias=None, act=ACT_NONE, mul=None, residual=None):
    return Epilogue(bias.handle if bias is not None else None, act,
                    mul.handle if mul is not None else None, residual.handle if residual is not None else None)


class GemvDesc(ctypes.Structure):
    _fields_ = [("x", c_void_p), ("x_dtype", c_int), ("W", c_void_p), ("y", c_void_p), ("y_dtype", c_int)]


MAX_GROUP = 8

_P = c_void_p
_PP = POINTER(c_void_p)
_SIGNATURES = {
    "mvlm_last_error": (c_char_p, []),
    "mvlm_abi_version": (c_int, []),
    "mvlm_device_count": (c_int, [POINTER(c_int)]),
    "mvlm_device_create": (c_int, [c_int, _PP]),
    "mvlm_device_destroy": (c_int, [_P]),
    "mvlm_device_get_info": (c_int, [_P, POINTER(DeviceInfo)]),
    "mvlm_device_synchronize": (c_int, [_P]),
    "mvlm_buffer_alloc": (c_int, [_P, c_size_t, _PP]),
    "mvlm_buffer_view": (c_int, [_P, c_size_t, c_size_t, _PP]),
    "mvlm_buffer_free": (c_int, [_P]),
    "mvlm_buffer_size": (c_size_t, [_P]),
    "mvlm_buffer_upload": (c_int, [_P, c_size_t, c_void_p, c_size_t]),
    "mvlm_buffer_download": (c_int, [_P, c_size_t, c_void_p, c_size_t]),
    "mvlm_buffer_fill_zero": (c_int, [_P]),
    "mvlm_pool_init": (c_int, [_P, c_size_t, _PP]),
    "mvlm_pool_current": (c_void_p, [_P]),
    "mvlm_pool_next": (c_void_p, [_P]),
    "mvlm_pool_swap": (c_int, [_P]),
    "mvlm_pool_destroy": (c_int, [_P]),
    "mvlm_weight_pack": (c_int, [_P, c_void_p, c_int, c_int, c_int, c_int, _PP]),
    "mvlm_weight_pack_device": (c_int, [_P, _P, c_int, c_int, c_int, c_int, _PP]),
    "mvlm_weight_free": (c_int, [_P]),
    "mvlm_weight_dtype": (c_int, [_P]),
    "mvlm_weight_shape": (c_int, [_P, POINTER(c_int), POINTER(c_int)]),
    "mvlm_weight_bytes": (c_size_t, [_P]),
    "mvlm_weight_dequant": (c_int, [_P, _P, _P, _PP]),
    "mvlm_gemm_naive": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, _PP]),
    "mvlm_gemm_tiled": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, _PP]),
    "mvlm_gemv_exact": (c_int, [_P, _P, _P, _P, c_int, c_int, _PP]),
    "mvlm_gemm_packed": (c_int, [_P, _P, c_int, _P, _P, c_int, c_int, c_int, c_int, _PP]),
    "mvlm_gemv": (c_int, [_P, _P, c_int, _P, _P, c_int, c_int, c_int, _PP]),
    "mvlm_gemv_grouped": (c_int, [_P, c_int, POINTER(GemvDesc), _PP]),
    "mvlm_gemm_packed_ex": (c_int, [_P, _P, c_int, _P, _P, c_int, c_int, c_int, c_int, POINTER(Epilogue), _PP]),
    "mvlm_gemv_ex": (c_int, [_P, _P, c_int, _P, _P, c_int, c_int, c_int, POINTER(Epilogue), _PP]),
    "mvlm_gemm_packed_ex_noalloc": (c_int, [_P, _P, c_int, _P, _P, c_int, c_int, c_int, c_int, POINTER(Epilogue)]),
    "mvlm_probe_grid_barrier": (c_int, [_P, c_int, c_int, c_int, POINTER(c_double)]),
    "mvlm_probe_load_latency": (c_int, [_P, c_int, c_int, POINTER(c_double)]),
    "mvlm_plan_add_gemv_ex": (c_int, [_P, _P, c_int, _P, _P, c_int, POINTER(Epilogue)]),
    "mvlm_plan_add_gemm_packed_ex": (c_int, [_P, _P, c_int, _P, _P, c_int, c_int, POINTER(Epilogue)]),
    "mvlm_plan_add_gemv_grouped": (c_int, [_P, c_int, POINTER(GemvDesc)]),
    "mvlm_gemm_quant_grouped": (c_int, [_P, c_int, c_int, POINTER(GemvDesc), _PP]),
    "mvlm_gemv_grouped_ex": (c_int, [_P, c_int, POINTER(GemvDesc), POINTER(Epilogue), _PP]),
    "mvlm_gemm_quant_grouped_ex": (c_int, [_P, c_int, c_int, POINTER(GemvDesc), POINTER(Epilogue), _PP]),
    "mvlm_plan_add_gemv_grouped_ex": (c_int, [_P, c_int, POINTER(GemvDesc), POINTER(Epilogue)]),
    "mvlm_plan_add_gemm_quant_grouped_ex": (c_int, [_P, c_int, c_int, POINTER(GemvDesc), POINTER(Epilogue)]),
    "mvlm_plan_add_gemm_quant_grouped": (c_int, [_P, c_int, c_int, POINTER(GemvDesc)]),
    "mvlm_gemv_q8_0": (c_int, [_P, _P, _P, _P, c_int, c_int, _PP]),
    "mvlm_gemv_q4_0": (c_int, [_P, _P, _P, _P, c_int, c_int, _PP]),
    "mvlm_gemm_q8_0": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, _PP]),
    "mvlm_gemm_q4_0": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, _PP]),
    "mvlm_gemm_batched": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, c_int,
                                  c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, _PP]),
    "mvlm_attention": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, _PP]),
    "mvlm_attention_prefill": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, _PP]),
    "mvlm_attention_decode": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, _PP]),
    "mvlm_plan_add_attention": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_float]),
    "mvlm_argmax": (c_int, [_P, _P, c_int, c_int, c_int, c_int64, _P, _PP]),
    "mvlm_plan_add_argmax": (c_int, [_P, _P, c_int, c_int, c_int, c_int64, _P]),
    "mvlm_fill_normal": (c_int, [_P, _P, c_int, c_size_t, c_uint64, c_double]),
    "mvlm_weight_random": (c_int, [_P, c_int, c_int, c_int, c_uint64, c_double, _PP]),
    "mvlm_event_wait": (c_int, [_P]),
    "mvlm_event_elapsed_ms": (c_int, [_P, POINTER(c_float)]),
    "mvlm_event_release": (c_int, [_P]),
    "mvlm_plan_create": (c_int, [_P, _PP]),
    "mvlm_plan_destroy": (c_int, [_P]),
    "mvlm_plan_size": (c_int, [_P]),
    "mvlm_plan_add_gemv": (c_int, [_P, _P, c_int, _P, _P, c_int, c_int]),
    "mvlm_plan_add_gemm_packed": (c_int, [_P, _P, c_int, _P, _P, c_int, c_int]),
    "mvlm_plan_add_gemm_batched": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, c_int,
                                           c_int64, c_int64, c_int64, c_int64, c_int64, c_int64]),
    "mvlm_plan_use_graph": (c_int, [_P, c_int]),
    "mvlm_plan_run": (c_int, [_P, c_int, _PP]),
    "mvlm_plan_profile": (c_int, [_P, POINTER(c_float), c_int]),
    "mvlm_plan_set_fusion": (c_int, [_P, c_int]),
    "mvlm_attention_decode_step": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_float, _PP]),
    "mvlm_plan_add_attention_decode_step": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, c_float]),
    "mvlm_plan_fused": (c_int, [_P]),
    "mvlm_plan_check": (c_int, [_P]),
    "mvlm_marker_record": (c_int, [_P, _PP]),
    "mvlm_marker_elapsed_ms": (c_int, [_P, _P, POINTER(c_float)]),
    "mvlm_gguf_open": (c_int, [c_char_p, _PP]),
    "mvlm_gguf_close": (c_int, [_P]),
    "mvlm_gguf_get_info": (c_int, [_P, POINTER(GgufInfo)]),
    "mvlm_gguf_tensor_info": (c_int, [_P, c_uint64, POINTER(GgufTensor)]),
    "mvlm_gguf_find_tensor": (c_int, [_P, c_char_p, POINTER(c_uint64)]),
    "mvlm_gguf_tensor_data": (c_int, [_P, c_uint64, _PP]),
    "mvlm_gguf_get_u32": (c_int, [_P, c_char_p, POINTER(ctypes.c_uint32)]),
    "mvlm_gguf_get_string": (c_int, [_P, c_char_p, _PP, POINTER(c_uint64)]),
    "mvlm_gguf_get_array": (c_int, [_P, c_char_p, POINTER(ctypes.c_uint32), POINTER(c_uint64), _PP]),
    "mvlm_gguf_get_array_string": (c_int, [_P, c_char_p, c_uint64, _PP, POINTER(c_uint64)]),
    "mvlm_ggml_type_size": (c_int, [ctypes.c_uint32, POINTER(c_uint64), POINTER(ctypes.c_uint32)]),
    "mvlm_weight_from_gguf": (c_int, [_P, _P, c_uint64, _PP]),
}

_lib = None


def lib():
    """Load the HIP library; raise if it is missing (no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run `python -m mvlm_amd.build` "
                              "(or __graft_entry__.build()) first")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return (lib().mvlm_last_error() or b"").decode()


def check(status: int, fn: str) -> None:
    if status != OK:
        raise MvlmError(status, fn, last_error())


def _call(name, *args):
    check(getattr(lib(), name)(*args), name)


def device_count() -> int:
    n = c_int(0)
    _call("mvlm_device_count", byref(n))
    return n.value


class Event:
    def __init__(self, handle):
        self.handle = handle

    def elapsed_ms(self) -> float:
        ms = c_float(0.0)
        _call("mvlm_event_elapsed_ms", self.handle, byref(ms))
        return ms.value

    def wait(self) -> None:
        _call("mvlm_event_wait", self.handle)

    def release(self) -> None:
        if self.handle:
            _call("mvlm_event_release", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class Buffer:
    def __init__(self, dev: "Device", handle, nbytes: int, parent: "Buffer | None" = None):
        self.dev, self.handle, self.nbytes, self.parent = dev, handle, nbytes, parent

    def upload(self, arr: np.ndarray, offset: int = 0) -> "Buffer":
        a = np.ascontiguousarray(arr)
        _call("mvlm_buffer_upload", self.handle, offset, a.ctypes.data, a.nbytes)
        return self

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype)
        _call("mvlm_buffer_download", self.handle, offset, out.ctypes.data, out.nbytes)
        return out

    def zero(self) -> "Buffer":
        _call("mvlm_buffer_fill_zero", self.handle)
        return self

    def view(self, offset: int, nbytes: int) -> "Buffer":
        h = c_void_p()
        _call("mvlm_buffer_view", self.handle, offset, nbytes, byref(h))
        return Buffer(self.dev, h, nbytes, parent=self)

    def free(self) -> None:
        if self.handle:
            _call("mvlm_buffer_free", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weight:
    def __init__(self, dev: "Device", handle):
        self.dev, self.handle = dev, handle

    @property
    def dtype(self) -> int:
        return lib().mvlm_weight_dtype(self.handle)

    @property
    def shape(self):
        n, k = c_int(), c_int()
        _call("mvlm_weight_shape", self.handle, byref(n), byref(k))
        return n.value, k.value

    @property
    def nbytes(self) -> int:
        return lib().mvlm_weight_bytes(self.handle)

    def dequant(self) -> np.ndarray:
        n, k = self.shape
        out = self.dev.alloc(n * k * 4)
        _call("mvlm_weight_dequant", self.dev.handle, self.handle, out.handle, None)
        self.dev.sync()
        return out.download(np.float32).reshape(n, k)

    def dequant_rows(self, rows, scratch: "Buffer") -> np.ndarray:
        """fp32 values of the given rows: the whole weight is dequantized on the
        device into `scratch` (at least N*K*4 bytes), only those rows come back."""
        n, k = self.shape
        _call("mvlm_weight_dequant", self.dev.handle, self.handle, scratch.handle, None)
        self.dev.sync()
        return np.stack([scratch.download(np.float32, k, int(r) * k * 4) for r in rows])

    def free(self) -> None:
        if self.handle:
            _call("mvlm_weight_free", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Gguf:
    """A memory-mapped GGUF file (include/mvlm_gguf.h); parsing runs in the C
    library, tensors and strings are read through the mapping."""

    _NP = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32, 6: np.float32,
           7: np.uint8, 10: np.uint64, 11: np.int64, 12: np.float64}

    def __init__(self, path: str):
        h = c_void_p()
        _call("mvlm_gguf_open", os.fsencode(path), byref(h))
        self.handle = h

    def info(self) -> GgufInfo:
        out = GgufInfo()
        _call("mvlm_gguf_get_info", self.handle, byref(out))
        return out

    def tensor(self, index: int) -> dict:
        t = GgufTensor()
        _call("mvlm_gguf_tensor_info", self.handle, index, byref(t))
        return {"name": ctypes.string_at(t.name, t.name_len).decode(), "n_dims": t.n_dims,
                "dims": list(t.dims), "type": t.type, "offset": t.offset, "bytes": t.bytes}

    def find(self, name: str) -> int:
        i = c_uint64()
        _call("mvlm_gguf_find_tensor", self.handle, name.encode(), byref(i))
        return i.value

    def data(self, index: int) -> bytes:
        p = c_void_p()
        _call("mvlm_gguf_tensor_data", self.handle, index, byref(p))
        return ctypes.string_at(p, self.tensor(index)["bytes"])

    def get_u32(self, key: str) -> int:
        v = ctypes.c_uint32()
        _call("mvlm_gguf_get_u32", self.handle, key.encode(), byref(v))
        return v.value

    def get_string(self, key: str) -> str:
        p, n = c_void_p(), c_uint64()
        _call("mvlm_gguf_get_string", self.handle, key.encode(), byref(p), byref(n))
        return ctypes.string_at(p, n.value).decode()

    def get_array(self, key: str):
        et, n, p = ctypes.c_uint32(), c_uint64(), c_void_p()
        _call("mvlm_gguf_get_array", self.handle, key.encode(), byref(et), byref(n), byref(p))
        if et.value == 8:
            out = []
            for i in range(n.value):
                s, ln = c_void_p(), c_uint64()
                _call("mvlm_gguf_get_array_string", self.handle, key.encode(), i, byref(s), byref(ln))
                out.append(ctypes.string_at(s, ln.value).decode())
            return out
        dt = np.dtype(self._NP[et.value])
        return np.frombuffer(ctypes.string_at(p, n.value * dt.itemsize), dtype=dt).copy()

    def close(self) -> None:
        if self.handle:
            _call("mvlm_gguf_close", self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def ggml_type_size(t: int):
    b, e = c_uint64(), ctypes.c_uint32()
    _call("mvlm_ggml_type_size", t, byref(b), byref(e))
    return b.value, e.value


def _ev(want: bool):
    return (c_void_p(), True) if want else (None, False)


def _descs(entries):
    arr = (GemvDesc * max(1, len(entries)))()
    for i, (x, xd, W, y, yd) in enumerate(entries):
        arr[i] = GemvDesc(x.handle, xd, W.handle, y.handle, yd)
    return arr


def _epilogues(epilogues, n):
    """per-entry epilogues: a list of dicts (keys bias, act, mul, residual) or None"""
    arr = (Epilogue * max(1, n))()
    keep = []
    for i, e in enumerate(epilogues):
        if e:
            arr[i] = _epilogue(e.get("bias"), e.get("act", ACT_NONE), e.get("mul"), e.get("residual"))
            keep += [v for k, v in e.items() if k != "act" and v is not None]
    return arr, keep


class Plan:
    """A recorded launch sequence run from native code (eagerly or as a HIP graph).
    Keeps references to the buffers and weights it names so they outlive it."""

    def __init__(self, dev: "Device"):
        self.dev = dev
        h = c_void_p()
        _call("mvlm_plan_create", dev.handle, byref(h))
        self.handle = h
        self._keep = []

    def __len__(self):
        return lib().mvlm_plan_size(self.handle)

    def add_gemv(self, x, x_dtype, W, y, y_dtype, M=1):
        _call("mvlm_plan_add_gemv", self.handle, x.handle, x_dtype, W.handle, y.handle, y_dtype, M)
        self._keep += [x, W, y]
        return self

    def add_gemv_grouped(self, entries, epilogues=None):
        """entries: [(x, x_dtype, W, y, y_dtype), ...] served by one launch;
        epilogues: optional per-entry dicts (bias, act, mul, residual)."""
        arr = _descs(entries)
        if epilogues is None:
            _call("mvlm_plan_add_gemv_grouped", self.handle, len(entries), arr)
        else:
            eps, keep = _epilogues(epilogues, len(entries))
            _call("mvlm_plan_add_gemv_grouped_ex", self.handle, len(entries), arr, eps)
            self._keep += keep
        for x, _, W, y, _ in entries:
            self._keep += [x, W, y]
        return self

    def add_gemm_quant_grouped(self, M, entries, epilogues=None):
        """entries: [(X, F32, W, Y, F32), ...] of M-row products over Q8_0 / Q4_0 weights, one launch."""
        arr = _descs(entries)
        if epilogues is None:
            _call("mvlm_plan_add_gemm_quant_grouped", self.handle, M, len(entries), arr)
        else:
            eps, keep = _epilogues(epilogues, len(entries))
            _call("mvlm_plan_add_gemm_quant_grouped_ex", self.handle, M, len(entries), arr, eps)
            self._keep += keep
        for x, _, W, y, _ in entries:
            self._keep += [x, W, y]
        return self

    def add_gemv_ex(self, x, x_dtype, W, y, y_dtype, bias=None, act=ACT_NONE, mul=None, residual=None):
        ep = _epilogue(bias, act, mul, residual)
        _call("mvlm_plan_add_gemv_ex", self.handle, x.handle, x_dtype, W.handle, y.handle, y_dtype, byref(ep))
        self._keep += [x, W, y] + [b for b in (bias, mul, residual) if b is not None]
        return self

    def add_gemm_packed_ex(self, A, a_dtype, W, C, c_dtype, M, bias=None, act=ACT_NONE, mul=None, residual=None):
        ep = _epilogue(bias, act, mul, residual)
        _call("mvlm_plan_add_gemm_packed_ex", self.handle, A.handle, a_dtype, W.handle, C.handle, c_dtype, M,
              byref(ep))
        self._keep += [A, W, C] + [b for b in (bias, mul, residual) if b is not None]
        return self

    def add_gemm_packed(self, A, a_dtype, W, C, c_dtype, M):
        _call("mvlm_plan_add_gemm_packed", self.handle, A.handle, a_dtype, W.handle, C.handle, c_dtype, M)
        self._keep += [A, W, C]
        return self

    def add_gemm_batched(self, A, B, C, batch, M, N, K, lda, ldb, ldc, sA, sB, sC):
        _call("mvlm_plan_add_gemm_batched", self.handle, A.handle, B.handle, C.handle, batch, M, N, K,
              lda, ldb, ldc, sA, sB, sC)
        self._keep += [A, B, C]
        return self

    def add_attention(self, Q, K, V, O, o_dtype, seq_q, seq_kv, num_heads, head_dim, causal=False, scale=0.0):
        _call("mvlm_plan_add_attention", self.handle, Q.handle, K.handle, V.handle, O.handle, o_dtype, seq_q,
              seq_kv, num_heads, head_dim, 1 if causal else 0, scale)
        self._keep += [Q, K, V, O]
        return self

    def add_attention_decode_step(self, qkv, K_cache, V_cache, O, cached, num_heads, head_dim, scale=0.0):
        _call("mvlm_plan_add_attention_decode_step", self.handle, qkv.handle, K_cache.handle, V_cache.handle,
              O.handle, cached, num_heads, head_dim, scale)
        self._keep += [qkv, K_cache, V_cache, O]
        return self

    def add_argmax(self, x, dtype, rows, n, ld, out_index):
        _call("mvlm_plan_add_argmax", self.handle, x.handle, dtype, rows, n, ld, out_index.handle)
        self._keep += [x, out_index]
        return self

    def use_graph(self, enable=True):
        _call("mvlm_plan_use_graph", self.handle, 1 if enable else 0)
        return self

    def run(self, repeats=1, event=False):
        ev, want = _ev(event)
        _call("mvlm_plan_run", self.handle, repeats, byref(ev) if want else None)
        return Event(ev) if want else None

    def set_fusion(self, enable=True):
        """Plan fusion on (default) or off: a decode attention entry runs inside
        the grouped GEMV launch after it that reads its output."""
        _call("mvlm_plan_set_fusion", self.handle, 1 if enable else 0)
        return self

    def fused(self) -> int:
        """Number of attention entries carried by the launch after them."""
        n = lib().mvlm_plan_fused(self.handle)
        if n < 0:
            raise MvlmError(n, "mvlm_plan_fused", last_error())
        return n

    def check(self):
        """Synchronizes; raises MvlmError if a fused launch gave up waiting."""
        _call("mvlm_plan_check", self.handle)
        return self

    def profile(self) -> np.ndarray:
        n = len(self)
        out = (c_float * n)()
        _call("mvlm_plan_profile", self.handle, out, n)
        return np.frombuffer(out, np.float32).copy()

    def destroy(self):
        if self.handle:
            _call("mvlm_plan_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Device:
    """One HIP device with its in-order stream (the DeviceInfo of the reference)."""

    def __init__(self, ordinal: int = 0):
        h = c_void_p()
        _call("mvlm_device_create", ordinal, byref(h))
        self.handle = h

    def info(self) -> DeviceInfo:
        inf = DeviceInfo()
        _call("mvlm_device_get_info", self.handle, byref(inf))
        return inf

    def sync(self) -> None:
        _call("mvlm_device_synchronize", self.handle)

    def close(self) -> None:
        if self.handle:
            _call("mvlm_device_destroy", self.handle)
            self.handle = None

    # -- memory -------------------------------------------------------------
    def alloc(self, nbytes: int) -> Buffer:
        h = c_void_p()
        _call("mvlm_buffer_alloc", self.handle, nbytes, byref(h))
        return Buffer(self, h, nbytes)

    def upload(self, arr: np.ndarray, pad_bytes: int = 0) -> Buffer:
        a = np.ascontiguousarray(arr)
        b = self.alloc(max(a.nbytes + pad_bytes, 1))
        if a.nbytes:
            b.upload(a)
        return b

    def pack(self, src: np.ndarray, dtype: int, N: int, K: int, layout: int = LAYOUT_NK) -> Weight:
        a = np.ascontiguousarray(src)
        h = c_void_p()
        _call("mvlm_weight_pack", self.handle, a.ctypes.data, dtype, layout, N, K, byref(h))
        return Weight(self, h)

    def pack_device(self, src: Buffer, dtype: int, N: int, K: int, layout: int = LAYOUT_NK) -> Weight:
        h = c_void_p()
        _call("mvlm_weight_pack_device", self.handle, src.handle, dtype, layout, N, K, byref(h))
        return Weight(self, h)

    def weight_from_gguf(self, g: "Gguf", index: int) -> Weight:
        h = c_void_p()
        _call("mvlm_weight_from_gguf", self.handle, g.handle, index, byref(h))
        return Weight(self, h)

    def random_weight(self, dtype: int, N: int, K: int, seed: int, wstd: float = 0.02) -> Weight:
        h = c_void_p()
        _call("mvlm_weight_random", self.handle, dtype, N, K, seed, wstd, byref(h))
        return Weight(self, h)

    def fill_normal(self, buf: Buffer, dtype: int, count: int, seed: int, std: float = 1.0) -> Buffer:
        _call("mvlm_fill_normal", self.handle, buf.handle, dtype, count, seed, std)
        return buf

    def marker(self) -> Event:
        h = c_void_p()
        _call("mvlm_marker_record", self.handle, byref(h))
        return Event(h)

    # -- launches (event=True returns an Event timing the launch) -------------
    def _launch(self, name, args, event):
        ev, want = _ev(event)
        _call(name, self.handle, *args, byref(ev) if want else None)
        return Event(ev) if want else None

    def gemm_naive(self, A, B, C, M, N, K, event=False):
        return self._launch("mvlm_gemm_naive", (A.handle, B.handle, C.handle, M, N, K), event)

    def gemm_tiled(self, A, B, C, M, N, K, event=False):
        return self._launch("mvlm_gemm_tiled", (A.handle, B.handle, C.handle, M, N, K), event)

    def gemv_exact(self, x, W, y, N, K, event=False):
        return self._launch("mvlm_gemv_exact", (x.handle, W.handle, y.handle, N, K), event)

    def gemm_packed(self, A, a_dtype, W, C, c_dtype, M, N, K, event=False):
        return self._launch("mvlm_gemm_packed", (A.handle, a_dtype, W.handle, C.handle, c_dtype, M, N, K), event)

    def gemm_packed_ex(self, A, a_dtype, W, C, c_dtype, M, N, K, bias=None, act=ACT_NONE, mul=None, residual=None,
                       event=False):
        ep = _epilogue(bias, act, mul, residual)
        return self._launch("mvlm_gemm_packed_ex", (A.handle, a_dtype, W.handle, C.handle, c_dtype, M, N, K,
                                                     byref(ep)), event)

    def gemm_packed_ex_noalloc(self, A, a_dtype, W, C, c_dtype, M, N, K, bias=None, act=ACT_NONE, mul=None,
                               residual=None):
        """mvlm_gemm_packed_ex with its workspace in the library's fixed per-GPU array (no allocation)."""
        ep = _epilogue(bias, act, mul, residual)
        _call("mvlm_gemm_packed_ex_noalloc", self.handle, A.handle, a_dtype, W.handle, C.handle, c_dtype, M, N, K,
              byref(ep))

    def probe_grid_barrier(self, variant, rounds=200, background=False):
        """microseconds per software grid barrier round (mvlm_probe_grid_barrier)"""
        us = c_double()
        _call("mvlm_probe_grid_barrier", self.handle, variant, rounds, 1 if background else 0, byref(us))
        return us.value

    def probe_load_latency(self, variant: int, after: int) -> list:
        """[min, median, p90, max] microseconds of a wave's first load (mvlm_probe_load_latency)"""
        us = (c_double * 4)()
        _call("mvlm_probe_load_latency", self.handle, variant, after, us)
        return list(us)

    def gemv_ex(self, x, x_dtype, W, y, y_dtype, N, K, bias=None, act=ACT_NONE, mul=None, residual=None,
                event=False):
        ep = _epilogue(bias, act, mul, residual)
        return self._launch("mvlm_gemv_ex", (x.handle, x_dtype, W.handle, y.handle, y_dtype, N, K, byref(ep)), event)

    def gemv(self, x, x_dtype, W, y, y_dtype, N, K, event=False):
        return self._launch("mvlm_gemv", (x.handle, x_dtype, W.handle, y.handle, y_dtype, N, K), event)

    def gemv_grouped(self, entries, event=False, epilogues=None):
        """entries: [(x, x_dtype, W, y, y_dtype), ...], one launch for all;
        epilogues: optional per-entry dicts (bias, act, mul, residual)."""
        if epilogues is None:
            return self._launch("mvlm_gemv_grouped", (len(entries), _descs(entries)), event)
        eps, _ = _epilogues(epilogues, len(entries))
        return self._launch("mvlm_gemv_grouped_ex", (len(entries), _descs(entries), eps), event)

    def gemm_quant_grouped(self, M, entries, event=False, epilogues=None):
        """entries: [(X, F32, W, Y, F32), ...]: Y = X W^T for each, M rows, one launch."""
        if epilogues is None:
            return self._launch("mvlm_gemm_quant_grouped", (M, len(entries), _descs(entries)), event)
        eps, _ = _epilogues(epilogues, len(entries))
        return self._launch("mvlm_gemm_quant_grouped_ex", (M, len(entries), _descs(entries), eps), event)

    def gemv_q8_0(self, x, W, y, N, K, event=False):
        return self._launch("mvlm_gemv_q8_0", (x.handle, W.handle, y.handle, N, K), event)

    def gemv_q4_0(self, x, W, y, N, K, event=False):
        return self._launch("mvlm_gemv_q4_0", (x.handle, W.handle, y.handle, N, K), event)

    def gemm_q8_0(self, X, W, Y, M, N, K, event=False):
        return self._launch("mvlm_gemm_q8_0", (X.handle, W.handle, Y.handle, M, N, K), event)

    def gemm_q4_0(self, X, W, Y, M, N, K, event=False):
        return self._launch("mvlm_gemm_q4_0", (X.handle, W.handle, Y.handle, M, N, K), event)

    def gemm_batched(self, A, B, C, batch, M, N, K, lda, ldb, ldc, sA, sB, sC, event=False):
        return self._launch("mvlm_gemm_batched", (A.handle, B.handle, C.handle, batch, M, N, K,
                                                  lda, ldb, ldc, sA, sB, sC), event)

    def attention(self, Q, K, V, O, o_dtype, seq_q, seq_kv, num_heads, head_dim, causal=False, scale=0.0,
                  event=False):
        """O = softmax(scale Q K^T + mask) V per head; [seq][heads][head_dim] fp16 in, F16/F32 out."""
        return self._launch("mvlm_attention", (Q.handle, K.handle, V.handle, O.handle, o_dtype, seq_q, seq_kv,
                                               num_heads, head_dim, 1 if causal else 0, scale), event)

    def attention_prefill(self, Q, K, V, O, seq_len, num_heads, head_dim, event=False):
        return self._launch("mvlm_attention_prefill", (Q.handle, K.handle, V.handle, O.handle, seq_len, num_heads,
                                                       head_dim), event)

    def attention_decode(self, Q, K_cache, V_cache, O, cache_len, num_heads, head_dim, event=False):
        return self._launch("mvlm_attention_decode", (Q.handle, K_cache.handle, V_cache.handle, O.handle, cache_len,
                                                      num_heads, head_dim), event)

    def attention_decode_step(self, qkv, K_cache, V_cache, O, cached, num_heads, head_dim, scale=0.0, event=False):
        """Append the new key/value of qkv (fp32 q | k | v) to row `cached` of the fp16 caches, then attend."""
        return self._launch("mvlm_attention_decode_step", (qkv.handle, K_cache.handle, V_cache.handle, O.handle,
                                                           cached, num_heads, head_dim, scale), event)

    def argmax(self, x, dtype, rows, n, ld, out_index, event=False):
        """out_index[r] (int32 on the device) = first index of the largest key of row r."""
        return self._launch("mvlm_argmax", (x.handle, dtype, rows, n, ld, out_index.handle), event)

    def gemm_quant(self, X, W, Y, M, N, K, event=False):
        """Dispatch by the weight's dtype (Q8_0 or Q4_0)."""
        fn = self.gemm_q8_0 if W.dtype == Q8_0 else self.gemm_q4_0
        return fn(X, W, Y, M, N, K, event=event)
