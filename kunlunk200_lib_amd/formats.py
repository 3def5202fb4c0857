"""Host-side weight formats of the matmul path.

Q4_0 (reference README.md:48, include/kunlun/k200.h:99): per 32 values one
18-byte block, a little-endian F16 scale d followed by 16 bytes; byte j holds
value j in its low nibble and value j+16 in its high nibble; value =
(nibble - 8) * d. Rows are K/32 consecutive blocks.

`quantize_q4_0` produces such blocks from F32 weights with ggml's reference
closed form (the one BASELINE's configs name): per block, the signed value of
largest magnitude m (first occurrence), d = m / -8, id = 1/d (0 if d == 0),
F16 scale by round-to-nearest-even, nibble = min(15, trunc(x*id + 8.5)).
"""
from __future__ import annotations

import numpy as np

F32, F16, Q4_0, ROWWISE_I8 = 0, 1, 2, 3


def q4_0_row_bytes(k: int) -> int:
    if k % 32:
        raise ValueError("Q4_0 rows need K % 32 == 0")
    return k // 32 * 18


def weight_bytes(type_: int, k: int, n: int) -> int:
    """Bytes of a row-major [n, k] weight matrix in format `type_` (not rowwise_i8)."""
    if type_ == F32:
        return 4 * k * n
    if type_ == F16:
        return 2 * k * n
    if type_ == Q4_0:
        return q4_0_row_bytes(k) * n
    raise ValueError("weight_bytes: rowwise_i8 uses packed_i8_size")


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """F32 [n, k] -> uint8 [n, k/32*18] Q4_0 blocks (vectorised numpy)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    blocks = w.reshape(n, k // 32, 32)
    idx = np.argmax(np.abs(blocks), axis=2)                       # first maximal |x|
    m = np.take_along_axis(blocks, idx[..., None], axis=2)[..., 0]
    m = np.where(np.abs(m) > 0, m, np.float32(0.0)).astype(np.float32)  # all-zero block: +0 as in C
    with np.errstate(divide="ignore", invalid="ignore"):
        d = (m / np.float32(-8.0)).astype(np.float32)
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    scaled = (blocks * inv[..., None]).astype(np.float32) + np.float32(8.5)
    q = np.minimum(np.trunc(scaled).astype(np.int32), 15).astype(np.uint8)
    out = np.empty((n, k // 32, 18), dtype=np.uint8)
    out[..., 0:2] = d.astype(np.float16).view(np.uint8).reshape(n, k // 32, 2)
    out[..., 2:] = q[..., :16] | (q[..., 16:] << 4)
    return out.reshape(n, k // 32 * 18)


def dequantize_q4_0(q4: np.ndarray, k: int) -> np.ndarray:
    """uint8 [n, k/32*18] Q4_0 blocks -> exact F32 [n, k] values."""
    q4 = np.ascontiguousarray(q4, dtype=np.uint8)
    n = q4.shape[0]
    blocks = q4.reshape(n, k // 32, 18)
    d = blocks[..., 0:2].copy().view(np.float16).astype(np.float32)        # [n, nb, 1]
    lo = (blocks[..., 2:] & 15).astype(np.float32) - 8.0
    hi = (blocks[..., 2:] >> 4).astype(np.float32) - 8.0
    values = np.concatenate([lo, hi], axis=2) * d
    return values.reshape(n, k).astype(np.float32)
