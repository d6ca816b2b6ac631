"""ctypes binding of the C-ABI in ``include/tt_attn.h`` (``libtt_hip.so``).

This is the reference-side binding a Python caller would use to reach the
attention kernels without pybind11: plain pointers and sizes, an int status
per call, and ``tt_last_error()`` turned into an exception.  Device memory is
owned by :class:`DeviceBuffer` (``tt_malloc`` / ``tt_free``).

Loading fails loudly (``OSError``/``RuntimeError``) when the library has not
been built; nothing here falls back to a CPU path.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
HEADER = os.path.join(os.path.dirname(HERE), "include", "tt_attn.h")
# TT_LIB_PATH selects another build of the library (e.g. a tuning variant).
LIB_PATH = os.environ.get("TT_LIB_PATH") or os.path.join(HERE, "libtt_hip.so")

TT_OK, TT_ERR_ARG, TT_ERR_HIP, TT_ERR_UNSUPPORTED, TT_ERR_NOMEM = range(5)
TT_F32, TT_F64, TT_I32, TT_BF16 = range(4)

_p = C.c_void_p
_i64 = C.c_int64
_SIGS = {
    "tt_last_error": (C.c_char_p, []),
    "tt_version": (C.c_char_p, []),
    "tt_device_count": (C.c_int, [C.POINTER(C.c_int)]),
    "tt_init": (C.c_int, [C.c_int]),
    "tt_stream": (_p, []),
    "tt_stream_create": (C.c_int, [C.POINTER(_p)]),
    "tt_stream_sync": (C.c_int, [_p]),
    "tt_stream_destroy": (C.c_int, [_p]),
    "tt_malloc": (C.c_int, [C.POINTER(_p), C.c_size_t]),
    "tt_free": (C.c_int, [_p]),
    "tt_empty_cache": (C.c_int, []),
    "tt_mem_stats": (C.c_int, [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "tt_memcpy_h2d": (C.c_int, [_p, _p, C.c_size_t]),
    "tt_memcpy_d2h": (C.c_int, [_p, _p, C.c_size_t]),
    "tt_memcpy_d2d": (C.c_int, [_p, _p, C.c_size_t]),
    "tt_upload_bf16_from_f32": (C.c_int, [_p, _p, C.c_size_t]),
    "tt_download_bf16_to_f32": (C.c_int, [_p, _p, C.c_size_t]),
    "tt_host_malloc": (C.c_int, [C.POINTER(_p), C.c_size_t]),
    "tt_host_free": (C.c_int, [_p]),
    "tt_memset": (C.c_int, [_p, C.c_int, C.c_size_t]),
    "tt_sync": (C.c_int, []),
    "tt_event_create": (C.c_int, [C.POINTER(_p)]),
    "tt_event_record": (C.c_int, [_p, _p]),
    "tt_event_elapsed_ms": (C.c_int, [C.POINTER(C.c_float), _p, _p]),
    "tt_event_destroy": (C.c_int, [_p]),
    "tt_set_launch_events": (C.c_int, [C.POINTER(_p), C.c_int]),
    "tt_launch_events_recorded": (C.c_int, [C.POINTER(C.c_int)]),
    "tt_read_probe": (C.c_int, [_p, _i64, _p, _p]),
    "tt_elementwise": (C.c_int, [C.c_int, C.c_int, _p, _p, _p, _i64, C.c_double, C.c_double, C.c_uint64, _p]),
    "tt_fill_normal": (C.c_int, [C.c_int, _p, _i64, C.c_uint64, C.c_float, _p]),
    "tt_im2col": (C.c_int, [C.c_int, _p, _p, _i64] + [C.c_int] * 10 + [_p]),
    "tt_cross_entropy_f32": (C.c_int, [_p, _p, _p, _i64, _i64, _p]),
    "tt_maxpool_f32": (C.c_int, [_p, _p, _p, _i64] + [C.c_int] * 8 + [_p]),
    "tt_maxpool_backward_f32": (C.c_int, [_p, _p, _p, _i64] + [C.c_int] * 8 + [_p]),
    "tt_cross_entropy_backward_f32": (C.c_int, [_p, _p, _p, _i64, _i64, _p]),
    "tt_col2im": (C.c_int, [C.c_int, _p, _p, _i64] + [C.c_int] * 10 + [_p]),
    "tt_attn_fwd_f32": (C.c_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, C.c_float, C.c_int, _p]),
    "tt_attn_fwd_bf16": (C.c_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, C.c_float, C.c_int, _p]),
    "tt_attn_bwd_f32": (C.c_int, [_p] * 9 + [_i64] * 5 + [C.c_float, C.c_int, _p]),
    "tt_attn_bwd_bf16": (C.c_int, [_p] * 9 + [_i64] * 5 + [C.c_float, C.c_int, _p]),
    "tt_attn_bwd_bf16_noalloc": (C.c_int, [_p] * 9 + [_i64] * 5 + [C.c_float, C.c_int, _p]),
    "tt_attn_decode_bf16": (C.c_int, [_p] * 5 + [_i64] * 4 + [C.c_float, _p]),
    "tt_attn_decode_f32": (C.c_int, [_p] * 5 + [_i64] * 4 + [C.c_float, _p]),
    "tt_softmax_rows_f32": (C.c_int, [_p, _p, _i64, _i64, _p]),
    "tt_gemm_f32": (C.c_int, [C.c_int, C.c_int, _i64, _i64, _i64, C.c_float, _p, _p, C.c_float, _p, _p]),
    "tt_gemm_bf16": (C.c_int, [C.c_int, C.c_int, _i64, _i64, _i64, C.c_float, _p, _p, C.c_float, _p, _p]),
}


class TTError(RuntimeError):
    def __init__(self, code: int, what: str, msg: str):
        super().__init__(f"{what} failed ({code}): {msg}")
        self.code = code


def header_functions(path: str = HEADER) -> list:
    """Names of every function the C header declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tt_\w+)\s*\(", text)))


class Lib:
    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise OSError(f"{path} is not built; run pku-aiprogramming_amd/build.py")
        self.path = path
        self.lib = C.CDLL(path)
        for name, (res, args) in _SIGS.items():
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args

    def last_error(self) -> str:
        return self.lib.tt_last_error().decode()

    def check(self, rc: int, what: str):
        if rc != TT_OK:
            raise TTError(rc, what, self.last_error())

    def call(self, name: str, *args):
        rc = getattr(self.lib, name)(*args)
        self.check(rc, name)

    def device_count(self) -> int:
        n = C.c_int(0)
        self.lib.tt_device_count(C.byref(n))
        return n.value

    def sync(self):
        self.call("tt_sync")


_LIB: Optional[Lib] = None


def lib() -> Lib:
    global _LIB
    if _LIB is None:
        _LIB = Lib()
    return _LIB


# ----------------------------------------------------------------- buffers

def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (NaN stays NaN)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


class DeviceBuffer:
    """A tt_malloc'd device block holding a tensor of ``shape`` and ``dtype``
    ("f32", "bf16" or "i32"), freed with tt_free when collected."""

    ITEM = {"f32": 4, "bf16": 2, "i32": 4, "f64": 8}

    def __init__(self, shape: Sequence[int], dtype: str = "f32"):
        self.L = lib()
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.ITEM[dtype]
        p = C.c_void_p()
        self.L.check(self.L.lib.tt_malloc(C.byref(p), max(self.nbytes, 1)), "tt_malloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a: np.ndarray, dtype: str = "f32") -> "DeviceBuffer":
        b = cls(a.shape, dtype)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray):
        """Copy a host array in.  A bf16 buffer takes float values (rounded
        to nearest even by tt_upload_bf16_from_f32) or uint16 bit patterns."""
        if self.dtype == "bf16" and a.dtype != np.uint16:
            host = np.ascontiguousarray(a, dtype=np.float32)
            assert 2 * host.size == self.nbytes, (host.shape, self.shape)
            self.L.call("tt_upload_bf16_from_f32", self.ptr, host.ctypes.data, host.size)
            return
        if self.dtype == "bf16":
            host = np.ascontiguousarray(a)
        elif self.dtype == "f32":
            host = np.ascontiguousarray(a, dtype=np.float32)
        elif self.dtype == "i32":
            host = np.ascontiguousarray(a, dtype=np.int32)
        else:
            host = np.ascontiguousarray(a, dtype=np.float64)
        assert host.nbytes == self.nbytes, (host.shape, self.shape)
        self.L.call("tt_memcpy_h2d", self.ptr, host.ctypes.data, self.nbytes)

    def download(self) -> np.ndarray:
        """Copy back; bf16 is returned as float32 values (tt_download_bf16_to_f32)."""
        if self.dtype == "bf16":
            out = np.empty(self.shape, np.float32)
            self.L.call("tt_download_bf16_to_f32", out.ctypes.data, self.ptr, out.size)
            return out
        raw = np.empty(self.shape, {"f32": np.float32, "i32": np.int32, "f64": np.float64}[self.dtype])
        self.L.call("tt_memcpy_d2h", raw.ctypes.data, self.ptr, self.nbytes)
        return raw

    def download_bytes(self) -> np.ndarray:
        """The stored bytes as is (bf16 as uint16 bit patterns)."""
        raw = np.empty(self.shape, {"f32": np.float32, "i32": np.int32, "f64": np.float64, "bf16": np.uint16}[self.dtype])
        self.L.call("tt_memcpy_d2h", raw.ctypes.data, self.ptr, self.nbytes)
        return raw

    def fill_normal(self, seed: int, scale: float = 1.0):
        code = TT_BF16 if self.dtype == "bf16" else TT_F32
        n = self.nbytes // self.ITEM[self.dtype]
        self.L.call("tt_fill_normal", code, self.ptr, n, seed, scale, None)

    def zero(self):
        self.L.call("tt_memset", self.ptr, 0, self.nbytes)

    def free(self):
        if getattr(self, "ptr", None):
            self.L.lib.tt_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ----------------------------------------------------------------- attention

def attn_fwd(q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer, o: DeviceBuffer, lse: Optional[DeviceBuffer],
             scale: float, causal: bool, stream=None):
    B, H, Lq, d = q.shape
    Lk = k.shape[2]
    name = "tt_attn_fwd_bf16" if q.dtype == "bf16" else "tt_attn_fwd_f32"
    lib().call(name, q.ptr, k.ptr, v.ptr, o.ptr, lse.ptr if lse else None, B, H, Lq, Lk, d, scale, int(causal), stream)


def attn_bwd(q, k, v, o, lse, do, dq, dk, dv, scale: float, causal: bool, stream=None):
    B, H, Lq, d = q.shape
    Lk = k.shape[2]
    name = "tt_attn_bwd_bf16" if q.dtype == "bf16" else "tt_attn_bwd_f32"
    lib().call(name, q.ptr, k.ptr, v.ptr, o.ptr, lse.ptr, do.ptr, dq.ptr, dk.ptr, dv.ptr, B, H, Lq, Lk, d, scale,
               int(causal), stream)


def attn_decode(q, k, v, o, lse, scale: float, stream=None):
    B, H, _, d = q.shape
    Lkv = k.shape[2]
    name = "tt_attn_decode_bf16" if q.dtype == "bf16" else "tt_attn_decode_f32"
    lib().call(name, q.ptr, k.ptr, v.ptr, o.ptr, lse.ptr if lse else None, B, H, Lkv, d, scale, stream)


# ------------------------------------------------------------------ GEMM

def gemm(transa: bool, transb: bool, m: int, n: int, k: int, alpha: float, A: DeviceBuffer, B: DeviceBuffer,
         beta: float, C: DeviceBuffer, stream=None):
    """C = alpha op(A) op(B) + beta C (row-major, the cudaGemm contract)."""
    if not (A.dtype == B.dtype == C.dtype):
        raise ValueError("gemm: A, B and C must share one dtype")
    name = "tt_gemm_bf16" if C.dtype == "bf16" else "tt_gemm_f32"
    lib().call(name, int(transa), int(transb), m, n, k, alpha, A.ptr, B.ptr, beta, C.ptr, stream)


# ------------------------------------------------------------------ softmax

def softmax_rows(x: DeviceBuffer, y: DeviceBuffer, stream=None):
    """Row softmax over the last axis of x (fp32) into y (may be x)."""
    if x.dtype != "f32" or y.dtype != "f32":
        raise ValueError("softmax_rows: fp32 buffers only")
    cols = x.shape[-1] if len(x.shape) else 1
    rows = (int(np.prod(x.shape[:-1])) if len(x.shape) > 1 else 1) if cols else 0
    lib().call("tt_softmax_rows_f32", x.ptr, y.ptr, rows, cols, stream)


class Stream:
    """A caller stream (tt_stream_create; default priority).  ``handle`` is
    what the launchers take as their stream argument."""

    def __init__(self):
        self.L = lib()
        s = C.c_void_p()
        self.L.call("tt_stream_create", C.byref(s))
        self.handle = s.value

    def sync(self):
        self.L.call("tt_stream_sync", self.handle)

    def destroy(self):
        if self.handle:
            self.L.call("tt_stream_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Event:
    """One hipEvent; ``elapsed(a, b)`` reads the time between two of them."""

    def __init__(self):
        self.L = lib()
        e = C.c_void_p()
        self.L.call("tt_event_create", C.byref(e))
        self.ptr = e.value

    def record(self, stream=None):
        self.L.call("tt_event_record", self.ptr, stream)

    @staticmethod
    def elapsed(a: "Event", b: "Event") -> float:
        ms = C.c_float(0)
        lib().call("tt_event_elapsed_ms", C.byref(ms), a.ptr, b.ptr)
        return ms.value

    def __del__(self):
        try:
            self.L.lib.tt_event_destroy(self.ptr)
        except Exception:
            pass


def set_launch_events(events: Sequence[Event]):
    """Record events[i] after the library's i-th next kernel launch
    (instrumentation for per-kernel timing); [] disables it."""
    arr = (C.c_void_p * max(1, len(events)))(*[e.ptr for e in events])
    lib().call("tt_set_launch_events", arr, len(events))


def launch_events_recorded() -> int:
    """How many events set by set_launch_events have been recorded so far."""
    n = C.c_int(0)
    lib().call("tt_launch_events_recorded", C.byref(n))
    return n.value


class Timer:
    """hipEvent pair on the library stream (or ``stream``)."""

    def __init__(self, stream=None):
        self.L = lib()
        self.stream = stream
        a, b = C.c_void_p(), C.c_void_p()
        self.L.call("tt_event_create", C.byref(a))
        self.L.call("tt_event_create", C.byref(b))
        self.a, self.b = a.value, b.value

    def start(self):
        self.L.call("tt_event_record", self.a, self.stream)

    def stop(self) -> float:
        self.L.call("tt_event_record", self.b, self.stream)
        ms = C.c_float(0)
        self.L.call("tt_event_elapsed_ms", C.byref(ms), self.a, self.b)
        return ms.value

    def __del__(self):
        try:
            self.L.lib.tt_event_destroy(self.a)
            self.L.lib.tt_event_destroy(self.b)
        except Exception:
            pass
