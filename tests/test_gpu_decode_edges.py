"""GPU parity of the weight decoders on special values, on every route.

The reference decodes F16 weights and Q4_0 block scales exactly, subnormals,
infinities and NaN included (reference kernels/kunlun-matvec.xpu:4-18,
kernels/q4-device.h:3-12).

* F16: every finite F16 bit pattern (63,488 of them, both zeros and all
  subnormals) is one weight row of K = 32 with the value in column r % 32 and
  zeros elsewhere. With activations +-2^j every product and every sum is exact
  in F32, so Y must equal value * x bit for bit (+0 and -0 compare equal) on
  each F16 route: f16_gemv (batch 1), f16_mfma_gemv (batch 2..16: the
  streamed fp16-MFMA kernel with activations split into hi and lo fp16 parts
  at batch <= 8 and K <= 4096, the K-split F32-MFMA kernel beyond) and the
  fp16-MFMA GEMM (batch >= 64). Rows holding +Inf, -Inf, NaN, and +Inf with
  -Inf give +Inf, -Inf, NaN, NaN.
* F16 small batch, split activations: a non-finite activation poisons its
  column as in F32 arithmetic, and activations spanning 2^-60 .. 2^60 inside
  one 512-value chunk keep the north-star bound.
* Q4_0: rows whose block scales are F16 subnormals (all blocks, or every other
  block beside normal scales), with random nibbles and Gaussian activations,
  on every Q4_0 route: q4_gemv_dot8 (batch 1 and 2), the streamed
  q4_stream_gemv (K = 4096,
  batch 5..8), the block-diagonal q4_bdiag_gemv, the
  streamed and the register-staged q4_mfma_gemv (under KUNLUN_Q4_BDIAG=0),
  the LDS GEMM and the register-staged GEMM, native_q4_matmul and common_q4_matmul (M = 1 and M > 1). Each route meets
  its own bound against FP64 gold of the exactly decoded weights: the
  north-star 1e-4 * ||x_b|| * ||w_r|| for the F32-accumulate GEMVs,
  2e-3 * ||x_b|| * ||w_r|| for the fp16-MFMA GEMM, and the common route's
  bound against its represented (quantized) activations.
"""
import numpy as np
import pytest

import kunlunk200_lib_amd as kl
from gpu_util import check_f32_accumulate, run_matmul

pytestmark = pytest.mark.gpu

# batch 8 (K <= 4096): the streamed fp16-MFMA GEMV with split activations;
# batch 16: the K-split F32-MFMA GEMV
F16_ROUTES = [(1, "f16_gemv"), (8, "f16_mfma_gemv"), (16, "f16_mfma_gemv"), (64, "f16_gemm_mfma")]
F16_ROUTE_IDS = ["f16_gemv", "f16_mfma_gemv_stream", "f16_mfma_gemv_ksplit", "f16_gemm_mfma"]


def all_finite_f16():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (bits & 0x7C00) != 0x7C00
    return bits[finite]


def one_hot_rows(values_f16: np.ndarray, k: int = 32) -> np.ndarray:
    n = values_f16.size
    w = np.zeros((n, k), np.float16)
    w[np.arange(n), np.arange(n) % k] = values_f16
    return w


def power_of_two_activations(batch, k=32):
    j = np.arange(batch)
    col = ((-1.0) ** j) * np.exp2((j % 7) - 3.0)
    return np.repeat(col[:, None], k, axis=1).astype(np.float32)


@pytest.mark.parametrize("batch,route", F16_ROUTES, ids=F16_ROUTE_IDS)
def test_f16_every_finite_pattern_exact(gpu, batch, route):
    values = all_finite_f16().view(np.float16)
    w = one_hot_rows(values)
    k, n = w.shape[1], w.shape[0]
    x = power_of_two_activations(batch, k)
    y, got_route, guard_ok = run_matmul(kl.WeightType.f16, w.view(np.uint8), x, k, n, batch)
    assert got_route == route
    assert guard_ok
    want = values.astype(np.float32)[None, :] * x[:, :1]
    bad = np.argwhere(y != want)
    assert bad.size == 0, (f"{bad.shape[0]} mismatches, first (b, r) {bad[:3].tolist()}: "
                           f"f16 bits {[hex(int(values.view(np.uint16)[r])) for _, r in bad[:3]]} "
                           f"got {[float(y[b, r]) for b, r in bad[:3]]}")
    sub = (values.view(np.uint16) & 0x7C00) == 0
    print(f"  f16 {route}: {values.size} patterns ({int(sub.sum())} zero/subnormal) exact", flush=True)


@pytest.mark.parametrize("batch,route", F16_ROUTES, ids=F16_ROUTE_IDS)
def test_f16_nonfinite_rows(gpu, batch, route):
    k = 64
    inf, nan = np.float16(np.inf), np.float16(np.nan)
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((8, k)) * 0.02).astype(np.float16)
    w[0, 5] = inf
    w[1, 40] = -inf
    w[2, 17] = nan
    w[3, 3], w[3, 60] = inf, -inf
    w[4, :] = 0
    w[4, 9] = inf                    # a lone +Inf among zeros
    x = np.abs(rng.standard_normal((batch, k))).astype(np.float32) + 0.5   # no zero activation meets an Inf
    y, got_route, guard_ok = run_matmul(kl.WeightType.f16, w.view(np.uint8), x, k, 8, batch)
    assert got_route == route and guard_ok
    assert np.all(y[:, 0] == np.inf) and np.all(y[:, 1] == -np.inf) and np.all(y[:, 4] == np.inf)
    assert np.all(np.isnan(y[:, 2])) and np.all(np.isnan(y[:, 3]))
    assert np.all(np.isfinite(y[:, 5:]))


@pytest.mark.parametrize("stream", [True, False], ids=["stream", "ksplit"])
def test_f16_small_batch_nonfinite_activation(gpu, knobs, stream):
    # one non-finite activation: its column is the F32 result (Inf / NaN),
    # the other columns stay finite and within the bound
    if not stream:
        knobs("KUNLUN_DENSE_STREAM", "0")
    k, n, batch = 1024, 48, 6
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    w[:, 700] = np.abs(w[:, 700]) + np.float16(0.01)       # the Inf meets positive weights only
    x = rng.standard_normal((batch, k)).astype(np.float32)
    x[1, 700] = np.inf
    x[3, 9] = np.nan
    x[4, 1000] = -np.inf
    y, route, guard_ok = run_matmul(kl.WeightType.f16, w.view(np.uint8), x, k, n, batch)
    assert route == "f16_mfma_gemv" and guard_ok
    assert np.all(y[1] == np.inf) and np.all(np.isnan(y[3]))
    want4 = np.where(w[:, 1000] > 0, -np.inf, np.where(w[:, 1000] < 0, np.inf, np.nan))
    assert np.array_equal(np.isnan(y[4]), np.isnan(want4)) and np.all(y[4][~np.isnan(want4)] == want4[~np.isnan(want4)])
    ok = [0, 2, 5]
    dec = w.astype(np.float32)
    gold = (x[ok].astype(np.float64) @ dec.astype(np.float64).T)
    res = check_f32_accumulate(y[ok], gold, dec, x[ok])
    assert res["finite"] and res["north_star"] and res["reference"], res


@pytest.mark.parametrize("stream", [True, False], ids=["stream", "ksplit"])
def test_f16_small_batch_wide_activation_range(gpu, knobs, stream):
    # activations from 2^-60 to 2^60 inside one chunk, largest finite F16
    # weights and subnormal ones: the hi/lo split keeps the F32-accumulate bound
    if not stream:
        knobs("KUNLUN_DENSE_STREAM", "0")
    k, n, batch = 4096, 96, 8
    rng = np.random.default_rng(6)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    w[:, ::97] = np.float16(65504.0)
    w[:, 5::97] = np.float16(2.0 ** -24)
    mag = np.exp2(rng.integers(-60, 61, size=(batch, k))).astype(np.float32)
    x = (rng.standard_normal((batch, k)) * mag).astype(np.float32)
    x[7] = rng.standard_normal(k).astype(np.float32) * np.float32(3e38 / 65504 / 64)   # near the F32 range
    y, route, guard_ok = run_matmul(kl.WeightType.f16, w.view(np.uint8), x, k, n, batch)
    assert route == "f16_mfma_gemv" and guard_ok
    dec = w.astype(np.float32)
    gold = x.astype(np.float64) @ dec.astype(np.float64).T
    res = check_f32_accumulate(y, gold, dec, x)
    # terms of 2^60 and more cancel in places, so only the norm bound holds
    # for every F32-accumulate order; the relative bound is not asserted
    assert res["finite"] and res["north_star"], res


# --- Q4_0 with F16-subnormal block scales ----------------------------------------

def q4_subnormal(k, n, seed, mixed, tiny=False, low_normal=False):
    """Q4_0 rows with subnormal scales (|d| < 2^-14) in every block, or in
    every other block beside normal scales near 0.0075 when `mixed`. `tiny`
    draws every scale from the far end instead: subnormals m * 2^-24 with
    m = 1..15 (then (q - 8) / 8 * d is itself a fraction of the smallest
    F16 subnormal), or with `low_normal` normals below 2^-11 (exponent
    fields 1..3), where (q - 8) / 8 * d falls below the F16 normal range."""
    rng = np.random.default_rng(seed)
    blocks = k // 32
    q4 = np.empty((n, blocks, 18), np.uint8)
    sub = rng.integers(1, 1024, size=(n, blocks), dtype=np.uint16) | \
        (rng.integers(0, 2, size=(n, blocks), dtype=np.uint16) << 15)
    # the smallest magnitudes too: exact powers 2^-24 .. 2^-15
    sub[:, ::7] = (np.uint16(1) << rng.integers(0, 10, size=sub[:, ::7].shape, dtype=np.uint16))
    if tiny:
        sign = rng.integers(0, 2, size=(n, blocks), dtype=np.uint16) << 15
        small = rng.integers(1, 16, size=(n, blocks), dtype=np.uint16)
        low = (rng.integers(1, 4, size=(n, blocks), dtype=np.uint16) << 10) | \
            rng.integers(0, 1024, size=(n, blocks), dtype=np.uint16)
        sub = (low if low_normal else small) | sign
    if mixed:
        normal = (rng.standard_normal((n, blocks)) * 0.0075).astype(np.float16).view(np.uint16)
        sub[:, 1::2] = normal[:, 1::2]
    q4[..., 0:2] = sub.view(np.uint8).reshape(n, blocks, 2)
    q4[..., 2:] = rng.integers(0, 256, size=(n, blocks, 16), dtype=np.uint8)
    return q4.reshape(n, blocks * 18)


def gemm_bound_ok(y, gold, dec, x, tol):
    err = np.abs(y.astype(np.float64) - gold)
    bound = tol * np.linalg.norm(x.astype(np.float64), axis=1)[:, None] * \
        np.linalg.norm(dec.astype(np.float64), axis=1)[None, :]
    return bool(np.all(err <= bound + 1e-300)), float(np.max(err / np.maximum(bound, 1e-300)))


# (k, batch, w_offset, route, tolerance): the route a default matmul takes
Q4_ROUTES = [
    (4096, 1, 0, "q4_gemv_dot8", 1e-4),
    (1088, 1, 0, "q4_gemv_dot8", 1e-4),        # K % 128 != 0
    (4096, 2, 0, "q4_gemv_dot8", 1e-4),
    (4096, 8, 0, "q4_stream_gemv", 1e-4),      # streamed MFMA GEMV (K = 4096, batch 5..8)
    (4096, 6, 0, "q4_stream_gemv", 1e-4),
    (4096, 8, 0, "q4_bdiag_gemv", 1e-4),       # block-diagonal MFMA GEMV (KUNLUN_Q4_STREAM_MIN=9)
    (1088, 8, 0, "q4_bdiag_gemv", 1e-4),
    (4096, 8, 0, "q4_mfma_gemv", 1e-4),        # streamed (KUNLUN_Q4_BDIAG=0; K % 256 == 0, 16-byte aligned)
    (1088, 8, 0, "q4_mfma_gemv", 1e-4),        # register-staged (KUNLUN_Q4_BDIAG=0; K % 256 != 0)
    (4096, 64, 0, "q4_gemm_mfma", 2e-3),       # LDS GEMM
    (1088, 64, 0, "q4_gemm_mfma", 2e-3),       # register-staged GEMM (K % 256 != 0)
    (4096, 128, 4, "q4_gemm_mfma", 2e-3),      # register-staged GEMM (weights off 16 bytes)
]


@pytest.mark.parametrize("scales", ["all_subnormal", "mixed", "tiny", "tiny_mixed", "low_normal"])
@pytest.mark.parametrize("k,batch,w_offset,route,tol", Q4_ROUTES,
                         ids=[f"{r}-k{k}-b{b}-o{o}" for k, b, o, r, _ in Q4_ROUTES])
def test_q4_subnormal_scales(gpu, oracle, knobs, k, batch, w_offset, route, tol, scales):
    if route == "q4_mfma_gemv":
        knobs("KUNLUN_Q4_BDIAG", "0")
    if route != "q4_stream_gemv":
        knobs("KUNLUN_Q4_STREAM_MIN", "9")
    n = 160
    mixed = scales.endswith("mixed")
    tiny = scales.startswith("tiny") or scales == "low_normal"
    q4 = q4_subnormal(k, n, k + batch + int(mixed) + 2 * len(scales), mixed, tiny=tiny,
                      low_normal=scales == "low_normal")
    dec = oracle.q4_decode(q4, k, n)
    x = np.random.default_rng(k * batch).standard_normal((batch, k)).astype(np.float32)
    y, got_route, guard_ok = run_matmul(kl.WeightType.q4_0, q4, x, k, n, batch, w_offset=w_offset)
    assert got_route == route and guard_ok
    gold = oracle.gold(dec, x, threads=16)
    assert np.all(np.isfinite(y))
    ok, ratio = gemm_bound_ok(y, gold, dec, x, tol)
    print(f"  q4 subnormal scales {route} k={k} b={batch} {scales}: max err / bound = {ratio:.3g}",
          flush=True)
    assert ok, f"{route}: error {ratio:.3g} x the bound {tol} * ||x|| * ||w||"
    if tol == 1e-4:
        res = check_f32_accumulate(y, gold, dec, x)
        assert res["reference"], res


@pytest.mark.parametrize("tile", ["128x48", "128x32", "64x64", "64x32"])
def test_q4_subnormal_scales_gemm_tiles(gpu, oracle, knobs, tile):
    # the subnormal-scale correction of every LDS GEMM tile (partial M and N tiles)
    knobs("KUNLUN_GEMM_TILE", tile)
    k, n, batch = 512, 200, 160
    q4 = q4_subnormal(k, n, 91, True, tiny=True)
    dec = oracle.q4_decode(q4, k, n)
    x = np.random.default_rng(92).standard_normal((batch, k)).astype(np.float32)
    y, got_route, guard_ok = run_matmul(kl.WeightType.q4_0, q4, x, k, n, batch)
    assert got_route == "q4_gemm_mfma" and guard_ok
    gold = oracle.gold(dec, x, threads=16)
    assert np.all(np.isfinite(y))
    ok, ratio = gemm_bound_ok(y, gold, dec, x, 2e-3)
    print(f"  q4 subnormal scales tile {tile}: max err / bound = {ratio:.3g}", flush=True)
    assert ok, f"tile {tile}: error {ratio:.3g} x the bound"


def q4_sparse_subnormal(k, n, seed):
    """Q4_0 rows in three kinds: ordinary rows (normal scales near 0.0075),
    rows whose only non-zero blocks are a few with subnormal scales (about 3%
    of the blocks, three in four of them m * 2^-24 with m < 16; the others
    hold q = 8 everywhere, so their values are 0),
    and ordinary rows with the same sprinkling of subnormal blocks. Rows of the
    second kind have outputs made of the subnormal blocks alone, so a missing
    or misplaced correction breaks the bound there."""
    rng = np.random.default_rng(seed)
    blocks = k // 32
    q4 = np.empty((n, blocks, 18), np.uint8)
    scale = (rng.standard_normal((n, blocks)) * 0.0075).astype(np.float16).view(np.uint16)
    q4[..., 2:] = rng.integers(0, 256, size=(n, blocks, 16), dtype=np.uint8)
    kind = np.arange(n) % 3
    sparse = rng.random((n, blocks)) < 0.03
    sparse[kind == 0] = False
    zero = (kind == 1)[:, None] & ~sparse
    q4[zero, 2:] = 0x88
    # magnitudes m * 2^-24 with m = 1..15 (the decode keeps almost nothing of
    # them: without the correction the zero-block rows miss the bound by about
    # 4.5x) and m = 1..1023
    m = np.where(rng.random((n, blocks)) < 0.75, rng.integers(1, 16, size=(n, blocks)),
                 rng.integers(1, 1024, size=(n, blocks))).astype(np.uint16)
    sub = m | (rng.integers(0, 2, size=(n, blocks), dtype=np.uint16) << 15)
    scale[sparse] = sub[sparse]
    q4[..., 0:2] = scale.view(np.uint8).reshape(n, blocks, 2)
    return q4.reshape(n, blocks * 18)


@pytest.mark.parametrize("tile", ["128x48", "128x32", "64x64", "64x32"])
def test_q4_sparse_subnormal_scales_gemm_tiles(gpu, oracle, knobs, tile):
    # a few subnormal-scale blocks per row (the correction walks many work
    # items, most with no marked block), partial M and N tiles
    knobs("KUNLUN_GEMM_TILE", tile)
    k, n, batch = 4096, 700, 200
    q4 = q4_sparse_subnormal(k, n, 97)
    dec = oracle.q4_decode(q4, k, n)
    x = np.random.default_rng(98).standard_normal((batch, k)).astype(np.float32)
    y, got_route, guard_ok = run_matmul(kl.WeightType.q4_0, q4, x, k, n, batch)
    assert got_route == "q4_gemm_mfma" and guard_ok
    gold = oracle.gold(dec, x, threads=16)
    assert np.all(np.isfinite(y))
    ok, ratio = gemm_bound_ok(y, gold, dec, x, 2e-3)
    print(f"  q4 sparse subnormal scales tile {tile}: max err / bound = {ratio:.3g}", flush=True)
    assert ok, f"tile {tile}: error {ratio:.3g} x the bound"


@pytest.mark.parametrize("mixed", [False, True], ids=["all_subnormal", "mixed"])
def test_native_q4_subnormal_scales(gpu, oracle, mixed):
    from test_gpu_native_q4 import NativeCase, check
    k, n = 4096, 256
    q4 = q4_subnormal(k, n, 77 + int(mixed), mixed)
    case = NativeCase(oracle, k, n, q4=q4)
    ws = kl.NativeQ4Workspace()
    for batch in (1, 3):
        x = np.random.default_rng(batch).standard_normal((batch, k)).astype(np.float32)
        y, _ = case.run(ws, x, batch)
        check(oracle, case, y, x)


@pytest.mark.parametrize("m", [1, 16])
def test_common_q4_subnormal_scales(gpu, oracle, m):
    import test_gpu_common_q4 as common
    k, n = 4096, 512
    q4 = q4_subnormal(k, n, 91 + m, True)
    case = common.Case.__new__(common.Case)
    case.k, case.n, case.raw = k, n, q4
    case.w = oracle.q4_decode(q4, k, n)
    case.weight = kl.CommonQ4Weight(0, k, n)
    case.weight.upload(q4)
    ws = kl.CommonQ4Workspace()
    x = oracle.fixture_input(k, m, 3)
    y = case.run(ws, x, m)
    kp, _ = oracle.common_dims(k, n)
    if m == 1:
        values, params = oracle.common_quant_pair(x, k)
        qa = common.represented_pair(values, params, k, kp)
    else:
        values, params = oracle.common_quant_rows(x, k, m, 32)
        qa = values.reshape(32, kp)[:m, :k].astype(np.float32) * params.reshape(32, 16)[:m, :1]
    common.check_against(oracle, y, case.w, qa, f"subnormal m={m}")
