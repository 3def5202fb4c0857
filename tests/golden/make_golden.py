"""Writes tests/golden/native_q4_reference.npz from the reference's own CPU
oracle header (bench/native-q4-reference.h), compiled from the reference
checkout into oracle/_ref/libkref.so by oracle/Makefile.

Vectors (all produced by the reference's code, not by this repository's):
  q4, decoded, row_scales   seeded Q4_0 weights K=256, N=8 (Weights)
  x{p}                      activation pattern p = 0..4, batch 2 (input)
  y{p}                      FP64 reference of decoded . x{p} (reference)
  act{p}, act_scales{p}     two-component per-tensor INT8 codes/scales of x{p}
  row_codes, row_scales8    one-component INT8 codes/scales of each weight row
Run: python tests/golden/make_golden.py  (after make -C oracle)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import _oracle  # noqa: E402

K, N, BATCH = 256, 8, 2


def main():
    ref = _oracle.ReferenceOracle.load()
    if ref is None:
        raise SystemExit("oracle/_ref/libkref.so missing: build it with make -C oracle (needs the reference checkout)")
    q4, decoded, row_scales = ref.weights(K, N)
    out = {"k": np.int32(K), "n": np.int32(N), "batch": np.int32(BATCH),
           "q4": q4, "decoded": decoded, "row_scales": row_scales}
    for p in range(5):
        x = ref.input(K, BATCH, p)
        out[f"x{p}"] = x
        out[f"y{p}"] = ref.reference(decoded, x)
        linear, scales = ref.activation(x, bits=8, components=2)
        out[f"act{p}"] = linear
        out[f"act_scales{p}"] = scales
    row_codes = np.empty((N, K), np.int8)
    row_scales8 = np.empty(N, np.float32)
    for r in range(N):
        linear, scales = ref.activation(decoded[r:r + 1], bits=8, components=1)
        row_codes[r] = linear[0, 0]
        row_scales8[r] = scales[0]
    out["row_codes"] = row_codes
    out["row_scales8"] = row_scales8
    path = os.path.join(HERE, "native_q4_reference.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
