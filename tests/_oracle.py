"""ctypes access to the CPU oracle (oracle/liboracle.so) and to the reference's
own CPU oracle header compiled into oracle/_ref/libkref.so. Test
infrastructure: only tests, smoke() and bench.py's cpu_baseline leg use it."""
from __future__ import annotations

import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
KREF_PATH = os.path.join(ROOT, "oracle", "_ref", "libkref.so")

P = ctypes.c_void_p
I = ctypes.c_int
Z = ctypes.c_size_t


def _p(a: np.ndarray):
    return a.ctypes.data


class Oracle:
    F32, F16, Q4_0, I8 = 0, 1, 2, 3

    def __init__(self, path: str = ORACLE_PATH):
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run __graft_entry__.build() (make -C oracle)")
        lib = ctypes.CDLL(path)
        sig = {
            "orc_xorshift32": (ctypes.c_uint32, [P]),
            "orc_half_to_float": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_float_to_half": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_bench_half": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_round_clamp": (I, [ctypes.c_float, I]),
            "orc_q4_decode": (None, [P, I, I, P]),
            "orc_f16_decode": (None, [P, Z, P]),
            "orc_f16_encode": (None, [P, Z, P]),
            "orc_q4_quantize": (None, [P, I, I, P]),
            "orc_bench_weights": (None, [I, I, P, P, P]),
            "orc_bench_input": (None, [I, I, P]),
            "orc_fused_bench_weights": (None, [I, I, P, P]),
            "orc_fixture_q4": (None, [I, I, P]),
            "orc_fixture_input": (None, [I, I, I, P]),
            "orc_gold": (None, [P, P, I, I, I, I, P]),
            "orc_matvec_f32": (None, [P, I, P, I, I, I, P]),
            "orc_i8_rows": (None, [P, I, I, P, P]),
            "orc_i8_activation": (I, [P, Z, P, P, P, P]),
            "orc_i8_dots": (None, [P, I, P, I, I, P]),
            "orc_i8_combine": (None, [P, P, P, ctypes.c_float, ctypes.c_float, I, I, P]),
            "orc_swiglu_value": (ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
            "orc_swiglu": (None, [P, P, P, I, I, I, I, I, I]),
            "orc_elementwise": (None, [P, P, P, I, I, I, I, ctypes.c_float]),
            "orc_native_q4_size": (ctypes.c_size_t, [I, I]),
            "orc_pack_native_q4": (None, [P, I, I, P]),
            "orc_native_q4_decode": (None, [P, I, I, P]),
            "orc_common_q4_size": (ctypes.c_size_t, [I, I]),
            "orc_common_q4_pack": (None, [P, I, I, P]),
            "orc_common_q4_decode": (None, [P, I, I, P]),
            "orc_common_quant_pair": (I, [P, I, P, P]),
            "orc_common_quant_rows": (None, [P, I, I, I, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        self.lib = lib

    # scalar helpers
    def half_to_float(self, h: int) -> float:
        return self.lib.orc_half_to_float(h)

    def float_to_half(self, v: float) -> int:
        return self.lib.orc_float_to_half(v)

    def round_clamp(self, v: float, limit: int = 127) -> int:
        return self.lib.orc_round_clamp(v, limit)

    # arrays
    def q4_decode(self, q4: np.ndarray, k: int, n: int) -> np.ndarray:
        q4 = np.ascontiguousarray(q4, dtype=np.uint8)
        w = np.empty((n, k), np.float32)
        self.lib.orc_q4_decode(_p(q4), k, n, _p(w))
        return w

    def f16_decode(self, h: np.ndarray) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        w = np.empty(h.shape, np.float32)
        self.lib.orc_f16_decode(_p(h), h.size, _p(w))
        return w

    def f16_encode(self, w: np.ndarray) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.float32)
        h = np.empty(w.shape, np.uint16)
        self.lib.orc_f16_encode(_p(w), w.size, _p(h))
        return h

    def q4_quantize(self, w: np.ndarray) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.float32)
        n, k = w.shape
        q4 = np.empty((n, k // 32 * 18), np.uint8)
        self.lib.orc_q4_quantize(_p(w), k, n, _p(q4))
        return q4

    def bench_weights(self, k: int, n: int):
        w = np.empty((n, k), np.float32)
        wh = np.empty((n, k), np.uint16)
        q4 = np.empty((n, k // 32 * 18), np.uint8)
        self.lib.orc_bench_weights(k, n, _p(w), _p(wh), _p(q4))
        return w, wh, q4

    def bench_input(self, k: int, batch: int) -> np.ndarray:
        x = np.empty((batch, k), np.float32)
        self.lib.orc_bench_input(k, batch, _p(x))
        return x

    def fused_bench_weights(self, k: int, n: int):
        w = np.empty((n, k), np.float32)
        q4 = np.empty((n, k // 32 * 18), np.uint8)
        self.lib.orc_fused_bench_weights(k, n, _p(w), _p(q4))
        return w, q4

    def fixture_q4(self, k: int, n: int) -> np.ndarray:
        q4 = np.empty((n, k // 32 * 18), np.uint8)
        self.lib.orc_fixture_q4(k, n, _p(q4))
        return q4

    def fixture_input(self, k: int, batch: int, pattern: int) -> np.ndarray:
        x = np.empty((batch, k), np.float32)
        self.lib.orc_fixture_input(k, batch, pattern, _p(x))
        return x

    def gold(self, w: np.ndarray, x: np.ndarray, threads: int = 8) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        n, k = w.shape
        batch = x.shape[0]
        y = np.empty((batch, n), np.float64)
        self.lib.orc_gold(_p(w), _p(x), k, n, batch, threads, _p(y))
        return y

    def matvec_f32(self, w_bytes: np.ndarray, type_: int, x: np.ndarray, k: int, n: int) -> np.ndarray:
        w_bytes = np.ascontiguousarray(w_bytes)
        x = np.ascontiguousarray(x, dtype=np.float32)
        batch = x.shape[0]
        y = np.empty((batch, n), np.float32)
        self.lib.orc_matvec_f32(_p(w_bytes), type_, _p(x), k, n, batch, _p(y))
        return y

    def i8_rows(self, w: np.ndarray):
        w = np.ascontiguousarray(w, dtype=np.float32)
        rows, k = w.shape
        codes = np.empty((rows, k), np.int8)
        scales = np.empty(rows, np.float32)
        self.lib.orc_i8_rows(_p(w), k, rows, _p(codes), _p(scales))
        return codes, scales

    def i8_activation(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        q0 = np.empty(x.shape, np.int8)
        q1 = np.empty(x.shape, np.int8)
        m0 = ctypes.c_float(0)
        m1 = ctypes.c_float(0)
        rc = self.lib.orc_i8_activation(_p(x), x.size, _p(q0), _p(q1), ctypes.byref(m0), ctypes.byref(m1))
        if rc != 0:
            return None
        return q0, q1, np.float32(m0.value), np.float32(m1.value)

    def i8_dots(self, a: np.ndarray, w: np.ndarray) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=np.int8)
        w = np.ascontiguousarray(w, dtype=np.int8)
        rows, k = a.shape
        n = w.shape[0]
        out = np.empty((rows, n), np.int64)
        self.lib.orc_i8_dots(_p(a), rows, _p(w), n, k, _p(out))
        return out

    def i8_combine(self, primary, residual, scales, max0, max1) -> np.ndarray:
        primary = np.ascontiguousarray(primary, dtype=np.int64)
        residual = np.ascontiguousarray(residual, dtype=np.int64)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        batch, n = primary.shape
        y = np.empty((batch, n), np.float32)
        self.lib.orc_i8_combine(_p(primary), _p(residual), _p(scales), float(max0), float(max1), n, batch, _p(y))
        return y

    def swiglu_value(self, g: float, u: float) -> float:
        return self.lib.orc_swiglu_value(g, u)

    def swiglu_bytes(self, gate: np.ndarray, up: np.ndarray, y: np.ndarray, width: int, rows: int,
                     gate_stride: int, up_stride: int, output_stride: int, bytes_: int,
                     gate_offset: int = 0, up_offset: int = 0, output_offset: int = 0) -> None:
        """orc_swiglu on byte buffers (uint8 arrays), in place into y; offsets in bytes."""
        for a in (gate, up, y):
            assert a.dtype == np.uint8 and a.flags.c_contiguous
        base = lambda a, off: ctypes.c_void_p(a.ctypes.data + off)  # noqa: E731
        self.lib.orc_swiglu(base(gate, gate_offset), base(up, up_offset), base(y, output_offset), width, rows,
                            gate_stride, up_stride, output_stride, bytes_)

    def swiglu(self, g: np.ndarray, u: np.ndarray) -> np.ndarray:
        """Dense [rows, width] F32 (or float16) SwiGLU; output dtype follows the input."""
        g = np.ascontiguousarray(g)
        u = np.ascontiguousarray(u, dtype=g.dtype)
        bytes_ = g.dtype.itemsize
        assert bytes_ in (2, 4)
        rows, width = g.shape
        y = np.empty_like(g)
        gb, ub, yb = (a.view(np.uint8).reshape(-1) for a in (g, u, y))
        self.swiglu_bytes(gb, ub, yb, width, rows, width * bytes_, width * bytes_, width * bytes_, bytes_)
        return y

    def elementwise(self, a: np.ndarray, b: np.ndarray, width: int, op: int, parameter: float = 0.0,
                    out: np.ndarray | None = None) -> np.ndarray:
        """orc_elementwise over F32 a (n values) and b (n or width values);
        out may be a itself (aliasing)."""
        a = np.ascontiguousarray(a, dtype=np.float32).ravel()
        b = np.ascontiguousarray(b, dtype=np.float32).ravel()
        y = np.empty_like(a) if out is None else out
        assert y.dtype == np.float32 and y.flags.c_contiguous and y.size == a.size
        self.lib.orc_elementwise(_p(y), _p(a), _p(b), a.size, int(width), b.size, int(op), float(parameter))
        return y

    def native_q4_size(self, k: int, n: int) -> int:
        return self.lib.orc_native_q4_size(k, n)

    def pack_native_q4(self, q4: np.ndarray, k: int, n: int) -> np.ndarray:
        q4 = np.ascontiguousarray(q4, dtype=np.uint8)
        assert q4.size >= n * (k // 32) * 18
        out = np.empty(self.native_q4_size(k, n), np.uint8)
        self.lib.orc_pack_native_q4(_p(q4), k, n, _p(out))
        return out

    def native_q4_decode(self, native: np.ndarray, k: int, n: int) -> np.ndarray:
        native = np.ascontiguousarray(native, dtype=np.uint8)
        assert native.size >= self.native_q4_size(k, n)
        w = np.empty((n, k), np.float32)
        self.lib.orc_native_q4_decode(_p(native), k, n, _p(w))
        return w

    @staticmethod
    def common_dims(k: int, n: int):
        kp = -(-k // (512 if k < 512 else 256)) * (512 if k < 512 else 256)
        np_ = -(-n // 256) * 256
        return kp, np_

    def common_q4_size(self, k: int, n: int) -> int:
        return self.lib.orc_common_q4_size(k, n)

    def common_q4_pack(self, q4: np.ndarray, k: int, n: int) -> np.ndarray:
        q4 = np.ascontiguousarray(q4, dtype=np.uint8)
        assert q4.size == n * (-(-k // 32)) * 18
        out = np.empty(self.common_q4_size(k, n), np.uint8)
        self.lib.orc_common_q4_pack(_p(q4), k, n, _p(out))
        return out

    def common_q4_decode(self, packed: np.ndarray, k: int, n: int) -> np.ndarray:
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        w = np.empty((n, k), np.float32)
        self.lib.orc_common_q4_decode(_p(packed), k, n, _p(w))
        return w

    def common_quant_pair(self, x: np.ndarray, k: int):
        """(values [4kp+1024] int8, params [16] f32) or None for non-finite x."""
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        kp, _ = self.common_dims(k, 1)
        values = np.empty(4 * kp + 1024, np.int8)
        params = np.empty(16, np.float32)
        if self.lib.orc_common_quant_pair(_p(x), k, _p(values), _p(params)) != 0:
            return None
        return values, params

    def common_quant_rows(self, x: np.ndarray, k: int, rows: int, defined: int):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        kp, _ = self.common_dims(k, 1)
        values = np.empty(defined * kp, np.int8)
        params = np.empty(defined * 16, np.float32)
        self.lib.orc_common_quant_rows(_p(x), k, rows, defined, _p(values), _p(params))
        return values, params

    def rowwise_i8_matmul(self, w: np.ndarray, x: np.ndarray) -> np.ndarray:
        """Whole reference rowwise_i8 path: weight upload quantization, two-pass
        activation quantization, exact dots, combine."""
        codes, scales = self.i8_rows(w)
        q0, q1, m0, m1 = self.i8_activation(x)
        return self.i8_combine(self.i8_dots(q0, codes), self.i8_dots(q1, codes), scales, m0, m1)


class ReferenceOracle:
    """The reference's bench/native-q4-reference.h, compiled (test infrastructure)."""

    @classmethod
    def load(cls, path: str = KREF_PATH):
        if not os.path.exists(path):
            return None
        return cls(path)

    def __init__(self, path: str):
        lib = ctypes.CDLL(path)
        lib.kref_weights.argtypes = [I, I, P, P, P]
        lib.kref_input.argtypes = [I, I, I, P]
        lib.kref_reference.argtypes = [P, P, I, I, I, P]
        lib.kref_activation.argtypes = [P, I, I, I, I, P, P]
        for fn in (lib.kref_weights, lib.kref_input, lib.kref_reference, lib.kref_activation):
            fn.restype = I
        lib.kref_prepare.argtypes = [P, P, I, I, I]
        lib.kref_prepare.restype = ctypes.c_void_p
        lib.kref_run.argtypes = [ctypes.c_void_p, P]
        lib.kref_run.restype = I
        lib.kref_release.argtypes = [ctypes.c_void_p]
        lib.kref_release.restype = None
        self.lib = lib

    def weights(self, k: int, n: int):
        q4 = np.empty((n, k // 32 * 18), np.uint8)
        dec = np.empty((n, k), np.float32)
        rs = np.empty(n, np.float32)
        self.lib.kref_weights(k, n, _p(q4), _p(dec), _p(rs))
        return q4, dec, rs

    def input(self, k: int, batch: int, pattern: int) -> np.ndarray:
        x = np.empty((batch, k), np.float32)
        self.lib.kref_input(k, batch, pattern, _p(x))
        return x

    def reference(self, w: np.ndarray, x: np.ndarray) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        n, k = w.shape
        batch = x.shape[0]
        y = np.empty((batch, n), np.float64)
        self.lib.kref_reference(_p(w), _p(x), k, n, batch, _p(y))
        return y

    def prepared(self, w: np.ndarray, x: np.ndarray) -> "PreparedReference":
        """reference() on vectors built once, timed alone per call as the reference's
        bench/native-q4-bench.cpp:22-25 times it."""
        return PreparedReference(self.lib, w, x)

    def activation(self, x: np.ndarray, bits: int = 8, components: int = 2):
        x = np.ascontiguousarray(x, dtype=np.float32)
        batch, k = x.shape
        linear = np.empty((components,) + x.shape, np.int8)
        scales = np.empty(components, np.float32)
        self.lib.kref_activation(_p(x), k, batch, bits, components, _p(linear), _p(scales))
        return linear, scales


class PreparedReference:
    """A kref_prepare handle: run() calls the reference's reference() on the stored vectors."""

    def __init__(self, lib, w: np.ndarray, x: np.ndarray):
        w = np.ascontiguousarray(w, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        self.lib = lib
        self.n, self.k = w.shape
        self.batch = x.shape[0]
        self.handle = lib.kref_prepare(_p(w), _p(x), self.k, self.n, self.batch)
        self.y = np.empty((self.batch, self.n), np.float64)

    def run(self) -> np.ndarray:
        self.lib.kref_run(self.handle, _p(self.y))
        return self.y

    def close(self) -> None:
        if self.handle:
            self.lib.kref_release(self.handle)
            self.handle = None
