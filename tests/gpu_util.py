"""Helpers for GPU tests: run one matmul through the C ABI with numpy inputs."""
from __future__ import annotations

import numpy as np

import kunlunk200_lib_amd as kl

GUARD = np.float32(-1234567.0)


def weight_payload(type_: int, w: np.ndarray, oracle) -> tuple[np.ndarray, np.ndarray]:
    """(bytes to upload, exact decoded F32 weights) for F32/F16/Q4_0 from F32 w."""
    if type_ == kl.WeightType.f32:
        return w.astype(np.float32).view(np.uint8).reshape(w.shape[0], -1), w.astype(np.float32)
    if type_ == kl.WeightType.f16:
        h = w.astype(np.float16)
        return h.view(np.uint8).reshape(w.shape[0], -1), h.astype(np.float32)
    q4 = kl.quantize_q4_0(w)
    return q4, oracle.q4_decode(q4, w.shape[1], w.shape[0])


def run_matmul(type_: int, w_bytes, x: np.ndarray, k: int, n: int, batch: int, *, kernel=None,
               w_offset: int = 0, x_offset: int = 0, w_f32=None, guard: int = 64, device: int = 0):
    """Upload, submit, wait, download. Returns (y [batch, n], route, guard_ok).

    w_bytes: raw weight bytes for F32/F16/Q4_0; for rowwise_i8 pass w_f32
    (host F32 rows quantized by upload_i8_rows)."""
    kernel = kernel or kl.Kernel()
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(batch, k)
    if type_ == kl.WeightType.rowwise_i8:
        wsize = kl.packed_i8_size(k, n)
    else:
        w_bytes = np.ascontiguousarray(w_bytes).view(np.uint8).ravel()
        wsize = w_bytes.nbytes
    wbuf = kl.Buffer(device, wsize + w_offset)
    xbuf = kl.Buffer(device, x.nbytes + x_offset)
    ybuf = kl.Buffer(device, (batch * n + guard) * 4)
    try:
        if type_ == kl.WeightType.rowwise_i8:
            kl.upload_i8_rows(device, wbuf.data + w_offset, k, n, 0, n, w_f32)
            scales = kl.packed_i8_scales(wbuf.data + w_offset, k, n)
            maxima = kl.packed_i8_maxima(wbuf.data + w_offset, k, n)
        else:
            wbuf.upload(w_bytes, offset=w_offset)
            scales = maxima = None
        xbuf.upload(x, offset=x_offset)
        ybuf.upload(np.full(batch * n + guard, GUARD, np.float32))
        with kl.runtime_mutex():
            kl.matmul(kernel, device, ybuf.data, wbuf.data + w_offset, xbuf.data + x_offset, k, n, batch, type_,
                      scales, maxima)
            kl.select(device)
            kl.check(kl.wait())
        out = ybuf.download(batch * n + guard, np.float32)
        x_after = xbuf.download(x.size, np.float32, offset=x_offset)
        assert np.array_equal(x_after.view(np.uint32), x.ravel().view(np.uint32)), "activations modified"
        if type_ != kl.WeightType.rowwise_i8:
            w_after = wbuf.download(wsize, np.uint8, offset=w_offset)
            assert np.array_equal(w_after, w_bytes), "weights modified"
        guard_ok = bool(np.all(out[batch * n:].view(np.uint32) == np.full(guard, GUARD).view(np.uint32)))
        return out[:batch * n].reshape(batch, n), kernel.route, guard_ok
    finally:
        wbuf.close()
        xbuf.close()
        ybuf.close()


def check_f32_accumulate(y: np.ndarray, gold: np.ndarray, w_dec: np.ndarray, x: np.ndarray, *,
                         ns_tol: float = 1e-4, ref_tol: float = 1e-3) -> dict:
    """north_star: |err| <= 1e-4 * ||x_b|| * ||w_r||; reference: |err| <= 1e-3 * (1 + |gold|)
    (reference bench/library-bench.cpp:125-126)."""
    err = np.abs(y.astype(np.float64) - gold)
    xn = np.linalg.norm(x.astype(np.float64), axis=1)[:, None]
    wn = np.linalg.norm(w_dec.astype(np.float64), axis=1)[None, :]
    ns_bound = ns_tol * xn * wn
    ref_bound = ref_tol * (1 + np.abs(gold))
    energy = float(np.sum(gold * gold))
    return {
        "finite": bool(np.all(np.isfinite(y))),
        "north_star": bool(np.all(err <= ns_bound)),
        "reference": bool(np.all(err <= ref_bound)),
        "max_abs": float(err.max()) if err.size else 0.0,
        "max_ns_ratio": float(np.max(err / np.maximum(ns_bound, 1e-300))) if err.size else 0.0,
        "nmse": float(np.sum(err * err) / max(energy, 1e-30)),
    }
