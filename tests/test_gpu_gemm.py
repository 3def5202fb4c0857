"""GPU parity of the fp16-MFMA prefill GEMM (Q4_0 and F16 weights, batch >= 64).

Bound (fp16 MFMA, f32 accumulate): |y - gold| <= 2e-3 * ||x_b|| * ||w_r|| per
element and ||Y - G||_F <= 2e-3 * ||G||_F, gold = FP64 dot of the exactly
decoded weights (reference bench/library-bench.cpp:121-122).
"""
import numpy as np
import pytest

import kunlunk200_lib_amd as kl
from gpu_util import run_matmul, weight_payload

pytestmark = pytest.mark.gpu


def gaussian(shape, sigma, seed):
    return (np.random.default_rng(seed).standard_normal(shape) * sigma).astype(np.float32)


def check_gemm(y, gold, w_dec, x, tol=2e-3):
    err = np.abs(y.astype(np.float64) - gold)
    bound = tol * np.linalg.norm(x.astype(np.float64), axis=1)[:, None] * \
        np.linalg.norm(w_dec.astype(np.float64), axis=1)[None, :]
    rel = np.linalg.norm(y.astype(np.float64) - gold) / max(np.linalg.norm(gold), 1e-30)
    return bool(np.all(np.isfinite(y))), bool(np.all(err <= bound + 1e-30)), float(rel)


# K up to 1024, 4096, 6144 and 16384: the activation prepass's 1, 2, 4 and 8
# groups of 8 values per thread
SHAPES = [(4096, 4096, 512), (4096, 11008, 512), (256, 65, 64), (96, 17, 70), (512, 300, 130),
          (16384, 64, 64), (1024, 129, 200), (384, 200, 96), (6144, 80, 66)]


@pytest.mark.parametrize("type_", [kl.WeightType.q4_0, kl.WeightType.f16], ids=["q4_0", "f16"])
@pytest.mark.parametrize("k,n,batch", SHAPES)
def test_gemm_gaussian(gpu, oracle, type_, k, n, batch):
    if type_ == kl.WeightType.f16 and k * n > 4096 * 4096:
        pytest.skip("f16 GEMM covered at smaller shapes")
    seed = k * 31 + n * 7 + batch
    w = gaussian((n, k), 0.02, seed)
    x = gaussian((batch, k), 1.0, seed + 1)
    payload, dec = weight_payload(type_, w, oracle)
    y, route, guard_ok = run_matmul(type_, payload, x, k, n, batch)
    gold = oracle.gold(dec, x, threads=16)
    finite, ok, rel = check_gemm(y, gold, dec, x)
    print(f"  gemm {int(type_)} k={k} n={n} b={batch} route={route} rel={rel:.3g}", flush=True)
    assert route.endswith("gemm_mfma")
    assert guard_ok and finite and ok and rel <= 2e-3


def test_gemm_extreme_rows(gpu, oracle):
    # per-row power-of-two scaling keeps huge and tiny rows inside fp16 range
    k, n, batch = 512, 96, 64
    w = gaussian((n, k), 0.02, 5)
    x = gaussian((batch, k), 1.0, 6)
    x[3] *= 1e6
    x[7] *= 1e-30
    x[9] = 0.0
    payload, dec = weight_payload(kl.WeightType.q4_0, w, oracle)
    y, _, _ = run_matmul(kl.WeightType.q4_0, payload, x, k, n, batch)
    gold = oracle.gold(dec, x)
    finite, ok, _ = check_gemm(y, gold, dec, x)
    assert finite and ok
    assert np.all(y[9] == 0)


def test_gemm_matches_gemv_within_fp16(gpu, oracle, knobs):
    # the same call below and above the GEMM batch threshold
    k, n, batch = 1024, 200, 64
    w = gaussian((n, k), 0.02, 8)
    x = gaussian((batch, k), 1.0, 9)
    payload, dec = weight_payload(kl.WeightType.q4_0, w, oracle)
    y_gemm, r1, _ = run_matmul(kl.WeightType.q4_0, payload, x, k, n, batch)
    knobs("KUNLUN_GEMM_MIN_BATCH", "100000")
    y_gemv, r2, _ = run_matmul(kl.WeightType.q4_0, payload, x, k, n, batch)
    assert r1 == "q4_gemm_mfma" and r2 != r1
    gold = oracle.gold(dec, x)
    _, ok, _ = check_gemm(y_gemm, gold, dec, x)
    assert ok
    assert np.max(np.abs(y_gemv - gold)) < np.max(np.abs(y_gemm - gold)) + 1e-6


# Q4_0 with K % 256 == 0 and 16-byte aligned weights runs the LDS-copy kernel
# (other shapes the register-staged one); KUNLUN_GEMM_TILE forces each of its
# tile shapes (BM x WN, 4*WN weight rows).
TILES = ["128x48", "128x32", "64x64", "64x32"]
TILE_SHAPES = [(512, 700, 200), (256, 64, 64), (768, 1000, 129)]   # partial M/N tiles; 2..6 K stages


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("k,n,batch", TILE_SHAPES)
def test_gemm_tile_variants(gpu, oracle, knobs, tile, k, n, batch):
    knobs("KUNLUN_GEMM_TILE", tile)
    seed = k + n + batch
    w = gaussian((n, k), 0.02, seed)
    x = gaussian((batch, k), 1.0, seed + 1)
    payload, dec = weight_payload(kl.WeightType.q4_0, w, oracle)
    y, route, guard_ok = run_matmul(kl.WeightType.q4_0, payload, x, k, n, batch)
    gold = oracle.gold(dec, x, threads=16)
    finite, ok, rel = check_gemm(y, gold, dec, x)
    print(f"  tile {tile} k={k} n={n} b={batch} rel={rel:.3g}", flush=True)
    assert route == "q4_gemm_mfma"
    assert guard_ok and finite and ok and rel <= 2e-3


@pytest.mark.parametrize("w_offset", [2, 1, 8])
def test_gemm_misaligned_weights(gpu, oracle, w_offset):
    # weights off a 16-byte boundary take the register-staged kernel; same bound
    k, n, batch = 512, 130, 96
    w = gaussian((n, k), 0.02, 40 + w_offset)
    x = gaussian((batch, k), 1.0, 41)
    payload, dec = weight_payload(kl.WeightType.q4_0, w, oracle)
    y, route, guard_ok = run_matmul(kl.WeightType.q4_0, payload, x, k, n, batch, w_offset=w_offset)
    gold = oracle.gold(dec, x)
    finite, ok, rel = check_gemm(y, gold, dec, x)
    assert route == "q4_gemm_mfma"
    assert guard_ok and finite and ok and rel <= 2e-3


def test_gemm_tiles_agree_exactly(gpu, oracle, knobs):
    # every tile shape sums each output in the same order: identical bits
    k, n, batch = 512, 384, 128
    w = gaussian((n, k), 0.02, 50)
    x = gaussian((batch, k), 1.0, 51)
    payload, _ = weight_payload(kl.WeightType.q4_0, w, oracle)
    outs = []
    for tile in TILES:
        knobs("KUNLUN_GEMM_TILE", tile)
        outs.append(run_matmul(kl.WeightType.q4_0, payload, x, k, n, batch)[0])
    for y in outs[1:]:
        assert np.array_equal(y.view(np.uint32), outs[0].view(np.uint32))
