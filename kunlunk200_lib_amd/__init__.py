"""Python host interface to the KunlunK200 matmul path on MI355X (gfx950).

This mirrors the reference's C++ surface (reference include/kunlun/k200.h:10-105,
345-350) over the library's C ABI (include/kunlun/k200_c.h): same names, same
argument meaning, same fail-fast behaviour (invalid arguments abort the
process, as the reference's require() does). Device memory is owned through
`Buffer`; numpy arrays move in and out with `Buffer.upload` / `Buffer.download`.

The compiled library is `kunlunk200_lib_amd/lib/libkunlunk200.so.0`, built by
`__graft_entry__.build()` (make -C kunlunk200_lib_amd/csrc). Loading fails
loudly when it is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import dataclasses
import enum
import os
import threading
from contextlib import contextmanager

import numpy as np

from .formats import q4_0_row_bytes, quantize_q4_0, weight_bytes  # noqa: F401

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(PACKAGE_DIR, "lib", "libkunlunk200.so.0")

_lib = None
_lib_lock = threading.Lock()

_c_size = ctypes.c_size_t
_c_void_p = ctypes.c_void_p
_c_int = ctypes.c_int

# (name, restype, argtypes) for every function of include/kunlun/k200_c.h.
C_FUNCTIONS = [
    ("kunlun_lock", None, []),
    ("kunlun_unlock", None, []),
    ("kunlun_check", None, [_c_int]),
    ("kunlun_require", None, [_c_int]),
    ("kunlun_diagnostic_tensor", None, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
    ("kunlun_device_count", _c_int, [ctypes.POINTER(_c_int)]),
    ("kunlun_select", None, [_c_int]),
    ("kunlun_wait", _c_int, []),
    ("kunlun_copy", _c_int, [_c_void_p, _c_void_p, _c_size, _c_int]),
    ("kunlun_peer", None, [_c_int, _c_void_p, _c_int, _c_void_p, _c_size]),
    ("kunlun_allocate", _c_void_p, [_c_int, _c_size]),
    ("kunlun_release", None, [_c_int, _c_void_p, _c_size]),
    ("kunlun_allocated_bytes", _c_size, [_c_int]),
    ("kunlun_kernel_create", _c_void_p, []),
    ("kunlun_kernel_destroy", None, [_c_void_p]),
    ("kunlun_aligned", _c_size, [_c_size]),
    ("kunlun_packed_i8_size", _c_size, [_c_int, _c_int]),
    ("kunlun_packed_i8_scales", _c_void_p, [_c_void_p, _c_int, _c_int]),
    ("kunlun_packed_i8_maxima", _c_void_p, [_c_void_p, _c_int, _c_int]),
    ("kunlun_upload_i8_rows", None, [_c_int, _c_void_p, _c_int, _c_int, _c_int, _c_int, _c_void_p]),
    ("kunlun_matmul", None, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
                             _c_int, _c_void_p, _c_void_p, _c_int]),
    ("kunlun_statistics", None, [ctypes.POINTER(_c_size)]),
    ("kunlun_version", ctypes.c_char_p, []),
    ("kunlun_matmul_count", _c_size, [_c_int]),
    ("kunlun_stream", _c_void_p, [_c_int]),
    ("kunlun_kernel_route", ctypes.c_char_p, [_c_void_p]),
    ("kunlun_set_tuning", _c_int, [ctypes.c_char_p, ctypes.c_char_p]),
    ("kunlun_matmul_noalloc", _c_int, [_c_int, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int, _c_int,
                                       _c_void_p, ctypes.POINTER(ctypes.c_char_p)]),
    ("kunlun_get_tuning", _c_int, [ctypes.c_char_p]),
    ("kunlun_elementwise", None, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
                                  _c_int, ctypes.c_float]),
    ("kunlun_swiglu_reason", ctypes.c_char_p, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    ("kunlun_swiglu", _c_int, [_c_void_p, _c_int, _c_void_p, _c_size, _c_void_p, _c_size, _c_void_p, _c_size,
                               _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    ("kunlun_matmul_swiglu", None, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int,
                                    _c_int, _c_int]),
    ("kunlun_native_q4_layout_supported", _c_int, [_c_int, _c_int]),
    ("kunlun_native_q4_size", _c_size, [_c_int, _c_int]),
    ("kunlun_pack_native_q4", _c_int, [_c_void_p, _c_size, _c_void_p, _c_int, _c_int]),
    ("kunlun_upload_native_q4", None, [_c_int, _c_void_p, _c_void_p, _c_int, _c_int]),
    ("kunlun_native_q4_reason", ctypes.c_char_p, [_c_int, _c_int, _c_int, _c_int]),
    ("kunlun_native_q4_workspace_create", _c_void_p, []),
    ("kunlun_native_q4_workspace_destroy", None, [_c_void_p]),
    ("kunlun_native_q4_statistics", None, [_c_void_p, ctypes.POINTER(_c_size)]),
    ("kunlun_native_q4_matmul", _c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
                                         _c_int]),
    ("kunlun_common_q4_supported", _c_int, [_c_int, _c_int]),
    ("kunlun_common_q4_size", _c_size, [_c_int, _c_int]),
    ("kunlun_common_q4_weight_create", _c_void_p, [_c_int, _c_int, _c_int, _c_void_p, _c_size]),
    ("kunlun_common_q4_weight_destroy", None, [_c_void_p]),
    ("kunlun_common_q4_weight_info", None, [_c_void_p, _c_void_p]),
    ("kunlun_common_q4_weight_data", _c_void_p, [_c_void_p]),
    ("kunlun_common_q4_weight_upload", None, [_c_void_p, _c_void_p, _c_size]),
    ("kunlun_common_q4_weight_statistics", None, [_c_void_p, ctypes.POINTER(_c_size), ctypes.POINTER(ctypes.c_double)]),
    ("kunlun_common_q4_workspace_create", _c_void_p, []),
    ("kunlun_common_q4_workspace_destroy", None, [_c_void_p]),
    ("kunlun_common_q4_workspace_statistics", None, [_c_void_p, ctypes.POINTER(_c_size)]),
    ("kunlun_common_q4_activation_statistics", None, [_c_void_p, ctypes.POINTER(ctypes.c_uint64)]),
    ("kunlun_common_q4_mac_statistics", None, [_c_void_p, ctypes.POINTER(_c_size)]),
    ("kunlun_common_q4_quantization", None, [_c_void_p, ctypes.POINTER(_c_void_p), ctypes.POINTER(_c_void_p),
                                             ctypes.POINTER(_c_int)]),
    ("kunlun_common_q4_matmul", None, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int]),
    ("kunlun_common_q4_lease_create", _c_void_p, []),
    ("kunlun_common_q4_lease_destroy", None, [_c_void_p]),
    ("kunlun_common_q4_lease_reset", None, [_c_void_p]),
    ("kunlun_common_q4_lease_matches", _c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_int, ctypes.c_uint64]),
    ("kunlun_common_q4_lease_chunks", _c_size, [_c_void_p]),
    ("kunlun_common_q4_lease_chunk", None, [_c_void_p, _c_size, ctypes.POINTER(_c_void_p), ctypes.POINTER(_c_void_p),
                                            ctypes.POINTER(_c_int), ctypes.POINTER(_c_size)]),
    ("kunlun_common_q4_prepare", _c_int, [_c_void_p, _c_int, _c_void_p, _c_int, _c_int, _c_int, ctypes.c_uint64,
                                          _c_void_p]),
    ("kunlun_common_q4_matmul_shared", _c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p,
                                                ctypes.c_uint64]),
    ("kunlun_common_q4_matmul_pair", _c_int, [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                              _c_void_p, ctypes.c_uint64]),
    ("kunlun_common_q4_pair_statistics", None, [_c_void_p, ctypes.POINTER(_c_size)]),
    ("kunlun_common_q4_pair_last_status", _c_int, [_c_void_p]),
]


def load(path: str | None = None) -> ctypes.CDLL:
    """Load the HIP library (once) and declare every C entry point."""
    global _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        path = path or LIBRARY_PATH
        if not os.path.exists(path):
            raise RuntimeError(
                f"KunlunK200 HIP library not built: {path} is missing "
                "(run __graft_entry__.build() or make -C kunlunk200_lib_amd/csrc)")
        lib = ctypes.CDLL(path)
        for name, restype, argtypes in C_FUNCTIONS:
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


class WeightType(enum.IntEnum):
    """reference include/kunlun/k200.h:40"""
    f32 = 0
    f16 = 1
    q4_0 = 2
    rowwise_i8 = 3
    q6_k = 4


class CopyKind(enum.IntEnum):
    """reference include/kunlun/k200.h:18"""
    host_to_device = 0
    device_to_host = 1
    device_to_device = 2


def _ptr(value) -> int | None:
    if value is None:
        return None
    if isinstance(value, Buffer):
        return value.data
    if isinstance(value, np.ndarray):
        return value.ctypes.data
    return int(value)


@contextmanager
def runtime_mutex():
    """Hold the process-wide recursive runtime lock (reference k200.h:10)."""
    lib = load()
    lib.kunlun_lock()
    try:
        yield
    finally:
        lib.kunlun_unlock()


def check(status: int) -> None:
    load().kunlun_check(int(status))


def require(condition: bool) -> None:
    load().kunlun_require(1 if condition else 0)


def device_count() -> int:
    count = _c_int(0)
    check(load().kunlun_device_count(ctypes.byref(count)))
    return count.value


def select(device: int) -> None:
    load().kunlun_select(int(device))


def wait() -> int:
    return load().kunlun_wait()


def copy(dst, src, nbytes: int, kind: CopyKind) -> int:
    return load().kunlun_copy(_ptr(dst), _ptr(src), int(nbytes), int(kind))


def peer(dst_device: int, dst, src_device: int, src, nbytes: int) -> None:
    load().kunlun_peer(int(dst_device), _ptr(dst), int(src_device), _ptr(src), int(nbytes))


def allocate(device: int, nbytes: int) -> int | None:
    return load().kunlun_allocate(int(device), int(nbytes))


def release(device: int, ptr, nbytes: int) -> None:
    load().kunlun_release(int(device), _ptr(ptr), int(nbytes))


def allocated_bytes(device: int) -> int:
    return load().kunlun_allocated_bytes(int(device))


def aligned(nbytes: int) -> int:
    return load().kunlun_aligned(int(nbytes))


def packed_i8_size(k: int, rows: int) -> int:
    return load().kunlun_packed_i8_size(int(k), int(rows))


def packed_i8_scales(weights, k: int, rows: int) -> int:
    return load().kunlun_packed_i8_scales(_ptr(weights), int(k), int(rows))


def packed_i8_maxima(weights, k: int, rows: int) -> int:
    return load().kunlun_packed_i8_maxima(_ptr(weights), int(k), int(rows))


def upload_i8_rows(device: int, weights, k: int, rows: int, first_row: int, count: int,
                   values: np.ndarray) -> None:
    """Quantize F32 host rows [count, k] and upload them (reference k200.h:95-96)."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    if values.size < count * k:
        raise ValueError("upload_i8_rows: input holds fewer than count*k values")
    load().kunlun_upload_i8_rows(int(device), _ptr(weights), int(k), int(rows), int(first_row), int(count),
                                 values.ctypes.data)


class Buffer:
    """RAII device allocation (reference k200.h:25-37)."""

    def __init__(self, device: int, nbytes: int):
        self.device = int(device)
        self.size = int(nbytes)
        ptr = allocate(self.device, self.size)
        require(ptr is not None and ptr != 0)
        self.data = int(ptr)

    def close(self) -> None:
        if self.data:
            release(self.device, self.data, self.size)
            self.data = 0

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def upload(self, array: np.ndarray, offset: int = 0) -> None:
        array = np.ascontiguousarray(array)
        if offset < 0 or offset + array.nbytes > self.size:
            raise ValueError("Buffer.upload: out of range")
        with runtime_mutex():
            select(self.device)
            check(copy(self.data + offset, array, array.nbytes, CopyKind.host_to_device))
            check(wait())

    def download(self, shape, dtype, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if offset < 0 or offset + out.nbytes > self.size:
            raise ValueError("Buffer.download: out of range")
        with runtime_mutex():
            select(self.device)
            check(copy(out, self.data + offset, out.nbytes, CopyKind.device_to_host))
            check(wait())
        return out


class Kernel:
    """Per-call state owner bound to one device (reference k200.h:62-88)."""

    def __init__(self):
        self.handle = load().kunlun_kernel_create()
        require(bool(self.handle))

    def close(self) -> None:
        if self.handle:
            load().kunlun_kernel_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def route(self) -> str | None:
        name = load().kunlun_kernel_route(self.handle)
        return name.decode() if name else None


def matmul(kernel: Kernel, device: int, y, w, x, k: int, n: int, batch: int, type: WeightType,
           scales=None, maxima=None, tile: int = 16) -> None:
    """Submit Y[batch,n] = X[batch,k] . W[n,k]^T (reference k200.h:103-105).

    All pointers are device memory; select(device) + check(wait()) completes it.
    """
    load().kunlun_matmul(kernel.handle, int(device), _ptr(y), _ptr(w), _ptr(x), int(k), int(n), int(batch),
                         int(type), _ptr(scales), _ptr(maxima), int(tile))


class ElementwiseOp(enum.IntEnum):
    """reference k200.h:41"""
    add = 0
    multiply = 1
    silu = 2
    rms_norm = 3
    scale = 4


def elementwise(kernel: Kernel, device: int, y, a, b, count: int, width: int, b_count: int, op: ElementwiseOp,
                parameter: float = 0.0) -> None:
    """F32 elementwise op, completed before returning (reference k200.h:106-107)."""
    load().kunlun_elementwise(kernel.handle, int(device), _ptr(y), _ptr(a), _ptr(b), int(count), int(width),
                              int(b_count), int(op), float(parameter))


class InputType(enum.IntEnum):
    """Element type of SwiGLU inputs and outputs (reference k200.h:132)."""
    f32 = 0
    f16 = 1


@dataclasses.dataclass
class SwiGLULayout:
    """reference k200.h:185-190; strides are bytes between rows."""
    width: int
    rows: int
    gate_stride: int
    up_stride: int
    output_stride: int
    type: InputType = InputType.f32

    def _args(self):
        return (int(self.width), int(self.rows), int(self.gate_stride), int(self.up_stride),
                int(self.output_stride), int(self.type))


def swiglu_reason(layout: SwiGLULayout) -> str:
    """"" when supported, else the first rule broken (reference k200.h:192)."""
    return load().kunlun_swiglu_reason(*layout._args()).decode()


def swiglu(kernel: Kernel, device: int, y, y_bytes: int, gate, gate_bytes: int, up, up_bytes: int,
           layout: SwiGLULayout) -> bool:
    """y = SiLU(gate) * up, completed before returning; False when the layout or the
    pointer contract is not met (reference k200.h:197-199)."""
    return bool(load().kunlun_swiglu(kernel.handle, int(device), _ptr(y), int(y_bytes), _ptr(gate),
                                     int(gate_bytes), _ptr(up), int(up_bytes), *layout._args()))


def matmul_swiglu(kernel: Kernel, device: int, y, w_gate, w_up, x, k: int, n: int, batch: int,
                  type: WeightType) -> None:
    """Submit Y[batch,n] = SiLU(X W_gate^T) * (X W_up^T) (no reference counterpart:
    the reference runs two matmul calls and swiglu)."""
    load().kunlun_matmul_swiglu(kernel.handle, int(device), _ptr(y), _ptr(w_gate), _ptr(w_up), _ptr(x), int(k),
                                int(n), int(batch), int(type))


def native_q4_layout_supported(k: int, n: int) -> bool:
    """reference k200.h:128"""
    return bool(load().kunlun_native_q4_layout_supported(int(k), int(n)))


def native_q4_size(k: int, n: int) -> int:
    """Bytes of the native Q4 layout, 0 when unsupported (reference k200.h:129)."""
    return load().kunlun_native_q4_size(int(k), int(n))


def pack_native_q4(destination, nbytes: int, q4, k: int, n: int) -> bool:
    """Host repack of Q4_0 rows into the native layout (reference k200.h:130).
    destination and q4 are host arrays or addresses."""
    return bool(load().kunlun_pack_native_q4(_ptr(destination), int(nbytes), _ptr(q4), int(k), int(n)))


def pack_native_q4_array(q4: np.ndarray, k: int, n: int) -> np.ndarray:
    """pack_native_q4 into a new uint8 array of native_q4_size(k, n) bytes."""
    q4 = np.ascontiguousarray(q4, dtype=np.uint8)
    if q4.size < n * (k // 32) * 18:
        raise ValueError("pack_native_q4_array: fewer than n rows of Q4_0 blocks")
    out = np.empty(native_q4_size(k, n), np.uint8)
    require(out.size > 0 and pack_native_q4(out, out.size, q4, k, n))
    return out


def upload_native_q4(device: int, weights, q4: np.ndarray, k: int, n: int) -> None:
    """Pack on the host and copy to device memory; completes before returning (reference k200.h:131)."""
    q4 = np.ascontiguousarray(q4, dtype=np.uint8)
    if q4.size < n * (k // 32) * 18:
        raise ValueError("upload_native_q4: fewer than n rows of Q4_0 blocks")
    load().kunlun_upload_native_q4(int(device), _ptr(weights), q4.ctypes.data, int(k), int(n))


def native_q4_reason(k: int, n: int, batch: int, type: InputType = InputType.f32) -> str:
    """"" when the reference takes its accelerated route (reference k200.h:203)."""
    return load().kunlun_native_q4_reason(int(k), int(n), int(batch), int(type)).decode()


class NativeQ4Workspace:
    """Per-call state owner for native_q4_matmul, bound to one device (reference k200.h:208-219)."""

    def __init__(self):
        self.handle = load().kunlun_native_q4_workspace_create()
        require(bool(self.handle))

    def close(self) -> None:
        if self.handle:
            load().kunlun_native_q4_workspace_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def statistics(self) -> dict:
        out = (_c_size * 4)()
        load().kunlun_native_q4_statistics(self.handle, out)
        return {"accelerated": out[0], "fallback": out[1], "hbm_workspace_bytes": out[2],
                "l3_workspace_bytes": out[3]}


def native_q4_matmul(workspace: NativeQ4Workspace, device: int, y, weights, x, k: int, n: int, batch: int = 1,
                     type: InputType = InputType.f32) -> bool:
    """Y[batch,n] = X W^T over the native layout, completed before returning;
    True where the reference takes its accelerated route (reference k200.h:223-224)."""
    return bool(load().kunlun_native_q4_matmul(workspace.handle, int(device), _ptr(y), _ptr(weights), _ptr(x),
                                               int(k), int(n), int(batch), int(type)))


def common_q4_supported(k: int, n: int) -> bool:
    """reference k200.h:232"""
    return bool(load().kunlun_common_q4_supported(int(k), int(n)))


def common_q4_size(k: int, n: int) -> int:
    """Payload bytes of the common Q4 ABI v1 layout, 0 when unsupported (reference k200.h:233)."""
    return load().kunlun_common_q4_size(int(k), int(n))


class _CommonQ4InfoC(ctypes.Structure):
    _fields_ = [("abi_version", ctypes.c_uint32), ("quant_type", ctypes.c_uint32), ("layout", ctypes.c_uint32),
                ("scale_order", ctypes.c_uint32), ("k", _c_int), ("n", _c_int), ("kp", _c_int), ("np", _c_int),
                ("device", _c_int), ("scale_offset", _c_size), ("payload_bytes", _c_size)]


class CommonQ4PairStatus(enum.IntEnum):
    """reference k200.h:285"""
    NotAttempted = 0
    Success = 1
    Disabled = 2
    InvalidInput = 3
    Configuration = 4
    WeightAbi = 5
    Lease = 6
    Alias = 7
    Workspace = 8


class _Handle:
    _destroy = ""

    def close(self) -> None:
        if getattr(self, "handle", None):
            getattr(load(), self._destroy)(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class CommonQ4Weight(_Handle):
    """Common Q4 ABI v1 weight on one device (reference k200.h:249-268)."""
    _destroy = "kunlun_common_q4_weight_destroy"

    def __init__(self, device: int, k: int, n: int, storage=None, nbytes: int = 0):
        self.handle = load().kunlun_common_q4_weight_create(int(device), int(k), int(n), _ptr(storage), int(nbytes))
        require(bool(self.handle))

    def info(self) -> dict:
        out = _CommonQ4InfoC()
        load().kunlun_common_q4_weight_info(self.handle, ctypes.byref(out))
        return {name: getattr(out, name) for name, _ in out._fields_}

    def data(self) -> int:
        return load().kunlun_common_q4_weight_data(self.handle)

    def upload(self, q4: np.ndarray) -> None:
        q4 = np.ascontiguousarray(q4, dtype=np.uint8)
        load().kunlun_common_q4_weight_upload(self.handle, q4.ctypes.data, q4.nbytes)

    def statistics(self) -> dict:
        counts, ms = (_c_size * 2)(), (ctypes.c_double * 2)()
        load().kunlun_common_q4_weight_statistics(self.handle, counts, ms)
        return {"uploads": counts[0], "upload_bytes": counts[1], "pack_ms": ms[0], "upload_ms": ms[1]}


class CommonQ4Workspace(_Handle):
    """Per-device state of the common Q4 calls (reference k200.h:286-303)."""
    _destroy = "kunlun_common_q4_workspace_destroy"

    def __init__(self):
        self.handle = load().kunlun_common_q4_workspace_create()
        require(bool(self.handle))

    def statistics(self) -> dict:
        out = (_c_size * 13)()
        load().kunlun_common_q4_workspace_statistics(self.handle, out)
        return {"paths": list(out[0:8]), "calls": out[8], "chunks": out[9], "hbm_workspace_bytes": out[10],
                "l3_workspace_bytes": out[11], "slice_bytes": out[12]}

    def activation_statistics(self) -> dict:
        out = (ctypes.c_uint64 * 10)()
        load().kunlun_common_q4_activation_statistics(self.handle, out)
        names = ("prepare_calls", "quantized_chunks", "quant_kernel_launches", "prepared_matmuls", "prepared_chunks",
                 "invalidations", "rejected_calls", "hbm_activation_bytes", "quantization_ns", "preparation_ns")
        return dict(zip(names, list(out)))

    def mac_statistics(self) -> dict:
        out = (_c_size * 4)()
        load().kunlun_common_q4_mac_statistics(self.handle, out)
        return dict(zip(("baseline_sd_calls", "stream_sd_calls", "shape_fallbacks", "resident_l1d_bytes"), list(out)))

    def quantization(self) -> dict:
        values, scales, ints = _c_void_p(), _c_void_p(), (_c_int * 3)()
        load().kunlun_common_q4_quantization(self.handle, ctypes.byref(values), ctypes.byref(scales), ints)
        return {"values": values.value or 0, "scales": scales.value or 0, "rows": ints[0], "kp": ints[1],
                "components": ints[2]}


class CommonQ4ActivationLease(_Handle):
    """Quantized activation snapshot (reference k200.h:306-322)."""
    _destroy = "kunlun_common_q4_lease_destroy"

    def __init__(self):
        self.handle = load().kunlun_common_q4_lease_create()
        require(bool(self.handle))

    def reset(self) -> None:
        load().kunlun_common_q4_lease_reset(self.handle)

    def matches(self, device: int, k: int, rows: int, type: InputType, generation: int) -> bool:
        return bool(load().kunlun_common_q4_lease_matches(self.handle, int(device), int(k), int(rows), int(type),
                                                          int(generation)))

    def chunks(self) -> int:
        return load().kunlun_common_q4_lease_chunks(self.handle)

    def chunk(self, index: int) -> dict:
        values, scales, ints, nbytes = _c_void_p(), _c_void_p(), (_c_int * 5)(), (_c_size * 2)()
        load().kunlun_common_q4_lease_chunk(self.handle, int(index), ctypes.byref(values), ctypes.byref(scales),
                                            ints, nbytes)
        return {"values": values.value or 0, "scales": scales.value or 0, "first": ints[0], "rows": ints[1],
                "padded_rows": ints[2], "kp": ints[3], "components": ints[4], "values_bytes": nbytes[0],
                "scales_bytes": nbytes[1]}


def common_q4_matmul(workspace: CommonQ4Workspace, device: int, y, weight: CommonQ4Weight, x, m: int,
                     type: InputType = InputType.f32) -> None:
    """Y[m,n] = X W^T, completed before returning (reference k200.h:300-302)."""
    load().kunlun_common_q4_matmul(workspace.handle, int(device), _ptr(y), weight.handle, _ptr(x), int(m), int(type))


def common_q4_prepare(workspace: CommonQ4Workspace, device: int, x, k: int, rows: int, type: InputType,
                      generation: int, lease: CommonQ4ActivationLease) -> bool:
    """reference k200.h:327-328"""
    return bool(load().kunlun_common_q4_prepare(workspace.handle, int(device), _ptr(x), int(k), int(rows), int(type),
                                                int(generation), lease.handle))


def common_q4_matmul_shared(workspace: CommonQ4Workspace, device: int, y, weight: CommonQ4Weight,
                            lease: CommonQ4ActivationLease, generation: int) -> bool:
    """reference k200.h:331-332"""
    return bool(load().kunlun_common_q4_matmul_shared(workspace.handle, int(device), _ptr(y), weight.handle,
                                                      lease.handle, int(generation)))


def common_q4_matmul_pair(workspace: CommonQ4Workspace, device: int, y0, y1, w0: CommonQ4Weight,
                          w1: CommonQ4Weight, lease: CommonQ4ActivationLease, generation: int) -> bool:
    """reference k200.h:381"""
    return bool(load().kunlun_common_q4_matmul_pair(workspace.handle, int(device), _ptr(y0), _ptr(y1), w0.handle,
                                                    w1.handle, lease.handle, int(generation)))


def common_q4_pair_statistics(workspace: CommonQ4Workspace) -> dict:
    out = (_c_size * 3)()
    load().kunlun_common_q4_pair_statistics(workspace.handle, out)
    return {"calls": out[0], "declined": out[1], "l3_partial_bytes": out[2]}


def common_q4_pair_last_status(workspace: CommonQ4Workspace) -> CommonQ4PairStatus:
    return CommonQ4PairStatus(load().kunlun_common_q4_pair_last_status(workspace.handle))


def statistics() -> dict:
    out = (_c_size * 4)()
    load().kunlun_statistics(out)
    return {"matmuls": [out[0], out[1]], "peer_copies": out[2], "peer_bytes": out[3]}


def version() -> str:
    return load().kunlun_version().decode()


def matmul_count(device: int) -> int:
    return load().kunlun_matmul_count(int(device))


NOALLOC_SCRATCH_BYTES = 16 << 20
NOALLOC_INVALID, NOALLOC_TOO_LARGE = -1, -2


def matmul_noalloc(device: int, y, w, x, k: int, n: int, batch: int, type: WeightType, stream=None):
    """kunlun_matmul_noalloc: matmul for F32/F16/Q4_0 without device allocation (no reference
    counterpart). Submits on `stream` (None: the null stream); returns (status, route)."""
    route = ctypes.c_char_p()
    rc = load().kunlun_matmul_noalloc(int(device), _ptr(y), _ptr(w), _ptr(x), int(k), int(n), int(batch),
                                      int(type), _ptr(stream), ctypes.byref(route))
    return rc, (route.value.decode() if route.value else None)


def set_tuning(name: str, value) -> None:
    """Sets a route/tile knob (named by its environment variable) from text in the
    variable's syntax; None restores the value the library read from the environment."""
    raw = None if value is None else str(value).encode()
    if load().kunlun_set_tuning(name.encode(), raw) != 0:
        raise ValueError(f"set_tuning: unknown knob or malformed value: {name}={value!r}")


def get_tuning(name: str) -> int:
    """Current value of a knob (-1: unset, the built-in choice)."""
    v = load().kunlun_get_tuning(name.encode())
    if v == -2:
        raise ValueError(f"get_tuning: unknown knob {name}")
    return v


class tuning:
    """Context manager: knobs set for the duration of a block, then restored."""

    def __init__(self, **knobs):
        self.knobs = knobs

    def __enter__(self):
        for name, value in self.knobs.items():
            set_tuning(name, value)
        return self

    def __exit__(self, *exc):
        for name in self.knobs:
            set_tuning(name, None)
        return False


def stream(device: int) -> int:
    """The HIP stream (as an integer handle) the library submits to on `device`."""
    return load().kunlun_stream(int(device))
