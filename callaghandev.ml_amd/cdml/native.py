"""ctypes binding of the C ABI in include/cdml.h (libcdml_hip.so).

This is the Python twin of the P/Invoke declarations a C# manager would use:
plain pointers and sizes, status codes turned into exceptions.  Device
memory, streams and events are owned by the caller through the objects
below.  Loading fails loudly when the library has not been built; there is
no fallback implementation.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "_build", "libcdml_hip.so")
HEADER = os.path.join(ROOT, "include", "cdml.h")

OK, E_INVALID, E_NODEVICE, E_HIP, E_CAUSAL = 0, -1, -2, -3, -4
ACT = {"none": 0, "sigmoid": 1, "tanh": 2, "relu": 3, "leakyrelu": 4, "swish": 5}


class CdmlError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"cdml error {code}: {msg}")
        self.code = code


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 128), ("arch", C.c_char * 64), ("compute_units", C.c_int),
                ("max_clock_mhz", C.c_int), ("memory_clock_mhz", C.c_int),
                ("memory_bus_bits", C.c_int), ("total_memory", C.c_size_t),
                ("lds_per_workgroup", C.c_size_t)]


_vp, _i, _f, _sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t
SIGNATURES = {
    "cdml_device_count": [C.POINTER(_i)],
    "cdml_init": [_i],
    "cdml_device_info_get": [_i, C.POINTER(DeviceInfo)],
    "cdml_last_error": [],
    "cdml_version": [],
    "cdml_stream_create": [C.POINTER(_vp)],
    "cdml_stream_destroy": [_vp],
    "cdml_stream_synchronize": [_vp],
    "cdml_graph_capture_begin": [_vp],
    "cdml_graph_capture_end": [_vp, C.POINTER(_vp)],
    "cdml_graph_launch": [_vp, _vp],
    "cdml_graph_destroy": [_vp],
    "cdml_tiny_layer_check": [_vp, _i],
    "cdml_tiny_decode": [_vp, _vp, _i, _i, _i, _vp],
    "cdml_stream_wait_event": [_vp, _vp],
    "cdml_event_create": [C.POINTER(_vp)],
    "cdml_event_create_sync_only": [C.POINTER(_vp)],
    "cdml_event_destroy": [_vp],
    "cdml_event_record": [_vp, _vp],
    "cdml_event_synchronize": [_vp],
    "cdml_event_elapsed_ms": [_vp, _vp, C.POINTER(_f)],
    "cdml_malloc": [C.POINTER(_vp), _sz],
    "cdml_free": [_vp],
    "cdml_host_alloc_pinned": [C.POINTER(_vp), _sz],
    "cdml_host_free_pinned": [_vp],
    "cdml_memcpy_h2d_async": [_vp, _vp, _sz, _vp],
    "cdml_memcpy_d2h_async": [_vp, _vp, _sz, _vp],
    "cdml_memcpy_d2d_async": [_vp, _vp, _sz, _vp],
    "cdml_zero_f32_async": [_vp, _sz, _vp],
    "cdml_fill_i32_async": [_vp, _sz, _i, _vp],
    "cdml_memcpy2d_d2d_async": [_vp, _sz, _vp, _sz, _sz, _sz, _vp],
    "cdml_argmax_rows": [_vp, _i, _i, _i, _vp, _i, _vp],
    "cdml_project_qkv": [_vp] * 10 + [_i, _i, _i, _vp],
    "cdml_linear": [_vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "cdml_rope": [_vp, _i, _i, _i, _i, _i, _f, _i, _i, _i, _vp, _vp],
    "cdml_linear_backward_workspace_size": [_i, _i, _i, C.POINTER(_sz)],
    "cdml_linear_backward": [_vp, _i, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp],
    "cdml_backprop_qkv_workspace_size": [_i, _i, _i, C.POINTER(_sz)],
    "cdml_backprop_qkv": [_vp] * 14 + [_i, _i, _i, _vp, _sz, _vp],
    "cdml_sdpa_bwd_workspace_size": [_i, _i, _i, _i, _i, C.POINTER(_sz)],
    "cdml_sdpa_bwd_saved_workspace_size": [_i, _i, _i, _i, _i, _i, C.POINTER(_sz)],
    "cdml_sdpa_bwd_stored_ds_workspace_size": [_i, _i, _i, _i, _i, _i, C.POINTER(_sz)],
    "cdml_sdpa_bwd": [_vp, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _i,
                      _i, _i, _i, _i, _i, _f, _i, _vp, _vp, _sz, _vp],
    "cdml_sdpa_fwd_lse": [_vp, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _i, _f, _i, _vp, _vp],
    "cdml_sdpa_bwd_saved": [_vp, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _vp, _i, _vp, _i, _vp, _i, _vp, _i,
                            _i, _i, _i, _i, _i, _f, _i, _vp, _vp, _sz, _vp],
    "cdml_sdpa_bwd_saved_rope": [_vp, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _vp, _i, _vp, _i, _vp, _i, _vp, _i,
                                 _i, _i, _i, _i, _i, _f, _i, _vp, _vp, _i, _vp, _sz, _vp],
    "cdml_rope_table": [_vp, _i, _i, _f, _vp],
    "cdml_rope_qk_table": [_vp, _vp, _i, _i, _i, _i, _vp, _i, _i, _i, _i, _vp],
    "cdml_project_qkv_rope": [_vp] * 10 + [_i, _i, _i, _i, _vp, _i, _i, _i, _vp],
    "cdml_sdpa_fwd": [_vp, _i, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _f, _i, _vp, _vp],
    "cdml_mha_layer_fwd_workspace_size": [_i, _i, _i, _i, C.POINTER(_sz)],
    "cdml_mha_layer_fwd": [_vp] * 10 + [_i, _i, _i, _i, _f, _i, _vp, _vp, _vp, _sz, _vp],
    "cdml_decode_attn_workspace_size": [_i, _i, _i, _i, C.POINTER(_sz)],
    "cdml_decode_attn": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp, _sz, _vp],
    "cdml_decode_attn_noalloc": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp],
    "cdml_kv_cache_append": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp],
    "cdml_residual_layernorm": [_vp, _vp, _vp, _vp, _vp, _i, _i, _f, _vp],
    "cdml_embed_tokens": [_vp, _i, _vp, _i, _i, _vp, _vp, _vp],
    "cdml_matmul": [_vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _vp],
    "cdml_linear_preact": [_vp, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "cdml_linear_backward_act": [_vp, _i, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _i, _i,
                                 _vp, _sz, _vp],
    "cdml_residual_layernorm_fwd": [_vp] * 9 + [_i, _i, _f, _vp],
    "cdml_layernorm_backward_workspace_size": [_i, _i, C.POINTER(_sz)],
    "cdml_layernorm_backward": [_vp] * 10 + [_i, _i, _f, _i, _vp, _sz, _vp],
    "cdml_cross_entropy_workspace_size": [_i, C.POINTER(_sz)],
    "cdml_cross_entropy": [_vp, _i, _vp, _i, _i, _i, _f, _f, _vp, _vp, _i, _vp, _sz, _vp],
    "cdml_mse_loss": [_vp, _i, _vp, _i, _i, _i, _i, _f, _f, _vp, _vp, _i, _vp, _sz, _vp],
    "cdml_add_inplace": [_vp, _vp, _sz, _vp],
    "cdml_update_f32": [_vp, _vp, _f, _sz, _vp],
    "cdml_scale_f32": [_vp, _f, _sz, _vp],
    "cdml_sum_squares_workspace_size": [C.POINTER(_sz)],
    "cdml_sum_squares": [_vp, _sz, _vp, _vp, _sz, _vp],
    "cdml_embedding_grad": [_vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _i, _vp],
    "cdml_grad_norm_workspace_size": [_i, C.POINTER(_sz)],
    "cdml_grad_norm": [_vp, _i, _f, _i, _f, _vp, _vp, _sz, _vp],
    "cdml_sgd_update": [_vp, _i, _f, _f, _vp, _i, _vp],
}


class Param(C.Structure):
    """cdml_param: one parameter tensor of cdml_grad_norm / cdml_sgd_update."""
    _fields_ = [("weight", C.c_void_p), ("grad", C.c_void_p), ("count", C.c_longlong),
                ("group", C.c_int), ("reserved", C.c_int)]

_lib = None


def header_functions() -> list[str]:
    """Names of every function declared in include/cdml.h."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(cdml_\w+)\s*\(", text, re.M)))


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise CdmlError(E_INVALID, f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = C.c_char_p if name in ("cdml_last_error", "cdml_version") else _i
        _lib = L
    return _lib


def check(rc: int):
    if rc != OK:
        raise CdmlError(rc, lib().cdml_last_error().decode(errors="replace"))


def device_count() -> int:
    n = C.c_int(0)
    check(lib().cdml_device_count(C.byref(n)))
    return n.value


def init(device: int = 0):
    check(lib().cdml_init(device))


def device_info(device: int = 0) -> dict:
    info = DeviceInfo()
    check(lib().cdml_device_info_get(device, C.byref(info)))
    return {"name": info.name.decode(), "arch": info.arch.decode(),
            "compute_units": info.compute_units, "max_clock_mhz": info.max_clock_mhz,
            "memory_clock_mhz": info.memory_clock_mhz, "memory_bus_bits": info.memory_bus_bits,
            "total_memory": info.total_memory, "lds_per_workgroup": info.lds_per_workgroup}


class Stream:
    def __init__(self):
        h = C.c_void_p()
        check(lib().cdml_stream_create(C.byref(h)))
        self.handle = h.value

    def synchronize(self):
        check(lib().cdml_stream_synchronize(self.handle))

    def close(self):
        if self.handle:
            check(lib().cdml_stream_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        h = C.c_void_p()
        check(lib().cdml_event_create(C.byref(h)))
        self.handle = h.value

    def record(self, stream: Stream | None):
        check(lib().cdml_event_record(self.handle, stream.handle if stream else None))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0)
        check(lib().cdml_event_elapsed_ms(self.handle, end.handle, C.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                lib().cdml_event_destroy(self.handle)
        except Exception:
            pass


class DeviceBuffer:
    """A caller-owned device allocation."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        check(lib().cdml_malloc(C.byref(p), int(nbytes)))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray, stream: Stream | None = None) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(max(a.nbytes, 4))
        buf.upload(a, stream)
        return buf

    def upload(self, a: np.ndarray, stream: Stream | None = None):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().cdml_memcpy_h2d_async(self.ptr, a.ctypes.data, a.nbytes, stream.handle if stream else None))
        if stream:
            stream.synchronize()
        else:
            check(lib().cdml_stream_synchronize(None))

    def download(self, shape, dtype=np.float32, stream: Stream | None = None) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(lib().cdml_memcpy_d2h_async(out.ctypes.data, self.ptr, out.nbytes, stream.handle if stream else None))
        if stream:
            stream.synchronize()
        else:
            check(lib().cdml_stream_synchronize(None))
        return out

    def free(self):
        if self.ptr:
            check(lib().cdml_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sptr(stream: Stream | None):
    return stream.handle if stream else None
