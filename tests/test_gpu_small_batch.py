"""GPU parity of the single-pass small-batch Q4_0 GEMVs (batch 2..16, fp16
MFMA with hi/lo activations): the streamed kernel (q4_stream_gemv, K = 4096
and batch <= 8, from batch 5 by default, from 2 under KUNLUN_Q4_STREAM_MIN=2),
the block-diagonal kernel (q4_bdiag_gemv, where the activation fragments of
all of K fit in LDS) and the LDS-staged kernels (q4_mfma_gemv, everywhere else
and under KUNLUN_Q4_BDIAG=0), on
BASELINE configs[2] shapes, K chunk tails, N tails, extreme and zero
activation rows, against the FP64 gold of the exactly decoded weights
(reference bench/library-bench.cpp:121-122) with the f32-accumulate bound
|err| <= 1e-4 * ||x_b|| * ||w_r||.
"""
import numpy as np
import pytest

# The MFMA GEMVs take batch 3..16 by default (the register-staged one from
# 5); tests reach the smaller batches through KUNLUN_Q4_MFMA_MIN.

import kunlunk200_lib_amd as kl
from gpu_util import check_f32_accumulate, run_matmul

pytestmark = pytest.mark.gpu

KERNELS = ["bdiag", "lds", "stream"]


def gaussian(shape, sigma, seed):
    return (np.random.default_rng(seed).standard_normal(shape) * sigma).astype(np.float32)


def bdiag_fits(k, batch):
    """Whether q4_bdiag_gemv takes (k, batch) (K % 64 == 0 assumed): for some
    T in 1, 2, 4, 8, 16 tiles per workgroup (16 / T K-parts per tile, none of
    them padding only), the per-wave steps (4 block pairs each) stay within 4
    (1 from column group 3), 4480 LDS bytes per step and column group plus
    4 KiB per group fit 160 KiB, and at most 4 activation items per thread."""
    q = (batch + 3) // 4
    need = (k + 255) // 256
    for t in (1, 2, 4, 8, 16):
        parts = 16 // t
        spw = (need + parts - 1) // parts
        steps = parts * spw
        lds = steps * q * 4480 + 4096 * q
        items = (4 * q * steps * 32 + 1023) // 1024
        if spw <= (1 if q > 2 else 4) and lds <= 160 * 1024 and items <= 4 and (parts <= need or t == 16):
            return True
    return False


def expected_route(kernel, k, batch, w_offset=0):
    if kernel == "stream" and k == 4096 and batch <= 8 and w_offset % 16 == 0:
        return "q4_stream_gemv"
    return "q4_bdiag_gemv" if kernel != "lds" and bdiag_fits(k, batch) else "q4_mfma_gemv"


@pytest.fixture(autouse=True)
def mfma_from_batch_two(gpu, knobs):
    knobs("KUNLUN_Q4_MFMA_MIN", "2")


@pytest.fixture(params=KERNELS)
def kernel(request, knobs):
    knobs("KUNLUN_Q4_BDIAG", "0" if request.param == "lds" else "1")
    knobs("KUNLUN_Q4_STREAM_MIN", "2" if request.param == "stream" else "9")
    return request.param


def q4_case(oracle, k, n, batch, seed, x=None):
    w = gaussian((n, k), 0.02, seed)
    if x is None:
        x = gaussian((batch, k), 1.0, seed + 1)
    q4 = kl.quantize_q4_0(w)
    dec = oracle.q4_decode(q4, k, n)
    y, route, guard_ok = run_matmul(kl.WeightType.q4_0, q4, x, k, n, batch)
    gold = oracle.gold(dec, x, threads=16)
    res = check_f32_accumulate(y, gold, dec, x)
    print(f"  q4 k={k} n={n} b={batch} route={route} {res}", flush=True)
    return y, route, guard_ok, res


@pytest.mark.parametrize("batch", [2, 4, 8, 16])
def test_config2_shapes(gpu, oracle, kernel, batch):
    y, route, guard_ok, res = q4_case(oracle, 4096, 14336, batch, 100 + batch)
    assert route == expected_route(kernel, 4096, batch)
    assert guard_ok and res["finite"] and res["north_star"] and res["reference"]


# LDS-staged kernels: 16-block stages for K % 512 == 0 (1024, 2048, 4096,
# 16384), 8-block stages for K % 256 == 0 only (11008), register-staged for the
# rest; block-diagonal kernel: partial last steps (4160, 576) and the tile and
# K-part splits of 1, 2 and 4 tiles per workgroup
@pytest.mark.parametrize("k,n,batch", [(64, 1, 2), (64, 17, 16), (4160, 33, 3), (11008, 4096, 4), (16384, 70, 16),
                                       (1024, 16, 5), (2048, 1000, 9), (4096, 4096, 15), (576, 130, 12),
                                       (8192, 300, 4), (2048, 5000, 16), (4096, 4200, 7),
                                       (4096, 1, 6), (4096, 33, 8)])   # streamed kernel: one row, one partial tile
def test_tails(gpu, oracle, kernel, k, n, batch):
    y, route, guard_ok, res = q4_case(oracle, k, n, batch, k + n + batch)
    assert route == expected_route(kernel, k, batch)
    assert guard_ok and res["finite"] and res["north_star"] and res["reference"]


def test_weights_off_16_bytes(gpu, oracle, kernel):
    # K % 256 == 0 streams through LDS when the weights are 16-byte aligned;
    # 4-byte aligned weights take the chunked kernel (the block-diagonal one
    # takes both): same bound either way
    k, n, batch = 2048, 300, 7
    w = gaussian((n, k), 0.02, 91)
    x = gaussian((batch, k), 1.0, 92)
    q4 = kl.quantize_q4_0(w)
    dec = oracle.q4_decode(q4, k, n)
    gold = oracle.gold(dec, x)
    for w_offset in (0, 4):
        y, route, guard_ok = run_matmul(kl.WeightType.q4_0, q4, x, k, n, batch, w_offset=w_offset)
        res = check_f32_accumulate(y, gold, dec, x)
        assert route == expected_route(kernel, k, batch, w_offset)
        assert guard_ok and res["finite"] and res["north_star"] and res["reference"]


def test_default_batch_routing(gpu, oracle, kernel):
    # defaults: the block-diagonal kernel from batch 3 where it fits;
    # otherwise (and under KUNLUN_Q4_BDIAG=0) the streamed kernel (K % 256 ==
    # 0, 16-byte aligned weights) from batch 3, the register-staged one from
    # batch 5, batch-1 passes below
    kl.set_tuning("KUNLUN_Q4_MFMA_MIN", None)
    if kernel == "stream":
        # streamed from batch 5 at K = 4096 (16-byte aligned weights), else as before
        kl.set_tuning("KUNLUN_Q4_STREAM_MIN", None)
        cases = [(4096, 5, 0, "q4_stream_gemv"), (4096, 8, 0, "q4_stream_gemv"), (4096, 4, 0, "q4_bdiag_gemv"),
                 (4096, 8, 4, "q4_bdiag_gemv"), (512, 8, 0, "q4_bdiag_gemv"), (4096, 9, 0, "q4_mfma_gemv")]
    elif kernel == "bdiag":
        cases = [(512, 3, 0, "q4_bdiag_gemv"), (512, 2, 0, "q4_gemv_dot8"), (576, 3, 0, "q4_bdiag_gemv"),
                 (576, 5, 0, "q4_bdiag_gemv"), (512, 4, 4, "q4_bdiag_gemv"), (4096, 16, 0, "q4_mfma_gemv")]
    else:
        cases = [(512, 3, 0, "q4_mfma_gemv"), (512, 2, 0, "q4_gemv_dot8"), (576, 3, 0, "q4_gemv_dot8"),
                 (576, 5, 0, "q4_mfma_gemv"), (512, 4, 4, "q4_gemv_dot8")]
    for k, batch, w_offset, want in cases:
        w = gaussian((70, k), 0.02, k + batch)
        x = gaussian((batch, k), 1.0, k + batch + 1)
        q4 = kl.quantize_q4_0(w)
        dec = oracle.q4_decode(q4, k, 70)
        y, route, guard_ok = run_matmul(kl.WeightType.q4_0, q4, x, k, 70, batch, w_offset=w_offset)
        res = check_f32_accumulate(y, oracle.gold(dec, x), dec, x)
        print(f"  k={k} b={batch} w_offset={w_offset} route={route}", flush=True)
        assert route == want, (k, batch, w_offset, route)
        assert guard_ok and res["finite"] and res["north_star"] and res["reference"]


def test_extreme_rows(gpu, oracle, kernel):
    k, n, batch = 4096, 300, 6
    x = gaussian((batch, k), 1.0, 77)
    x[1] *= 1e6
    x[2] *= 1e-30
    x[3] = 0.0
    x[4, ::7] *= 1000.0           # a row with a wide dynamic range
    y, route, guard_ok, res = q4_case(oracle, k, n, batch, 78, x=x)
    assert route == expected_route(kernel, k, batch)
    assert guard_ok and res["finite"] and res["north_star"]
    assert np.all(y[3] == 0.0)


def test_stream_nonfinite_activation_poisons_column(gpu, oracle, knobs):
    # an Inf or NaN in a batch column makes that column NaN in every row (the
    # batch-1 GEMV's rule); the other columns keep the bound
    knobs("KUNLUN_Q4_STREAM_MIN", "2")
    k, n, batch = 4096, 100, 6
    x = gaussian((batch, k), 1.0, 31)
    x[2, 5] = np.inf
    x[4, 3000] = np.nan
    x[5, 4095] = -np.inf
    w = gaussian((n, k), 0.02, 32)
    q4 = kl.quantize_q4_0(w)
    dec = oracle.q4_decode(q4, k, n)
    y, route, guard_ok = run_matmul(kl.WeightType.q4_0, q4, x, k, n, batch)
    assert route == "q4_stream_gemv" and guard_ok
    assert np.all(np.isnan(y[[2, 4, 5]]))
    ok = [0, 1, 3]
    res = check_f32_accumulate(y[ok], oracle.gold(dec, x[ok]), dec, x[ok])
    assert res["finite"] and res["north_star"] and res["reference"], res


def test_matches_batch_one_kernel(gpu, oracle, knobs, kernel):
    # the same call with the MFMA GEMV disabled (pairs of dot8 columns)
    k, n, batch = 4096, 1000, 8
    w = gaussian((n, k), 0.02, 5)
    x = gaussian((batch, k), 1.0, 6)
    q4 = kl.quantize_q4_0(w)
    y_mfma, r1, _ = run_matmul(kl.WeightType.q4_0, q4, x, k, n, batch)
    knobs("KUNLUN_Q4_MFMA_MIN", "17")
    knobs("KUNLUN_Q4_STREAM_MIN", "9")
    y_dot8, r2, _ = run_matmul(kl.WeightType.q4_0, q4, x, k, n, batch)
    assert r1 == expected_route(kernel, k, batch) and r2 == "q4_gemv_dot8"
    dec = oracle.q4_decode(q4, k, n)
    xn = np.linalg.norm(x.astype(np.float64), axis=1)[:, None]
    wn = np.linalg.norm(dec.astype(np.float64), axis=1)[None, :]
    assert np.all(np.abs(y_mfma.astype(np.float64) - y_dot8) <= 2e-4 * xn * wn)


# ---------------------------------------------------------------------------
# F16 / F32 weights, batch 2..16: the fp32-MFMA single-pass GEMV

def dense_case(oracle, type_, k, n, batch, seed):
    from gpu_util import weight_payload
    w = gaussian((n, k), 0.02, seed)
    x = gaussian((batch, k), 1.0, seed + 1)
    payload, dec = weight_payload(type_, w, oracle)
    y, route, guard_ok = run_matmul(type_, payload, x, k, n, batch)
    gold = oracle.gold(dec, x, threads=16)
    res = check_f32_accumulate(y, gold, dec, x)
    print(f"  {int(type_)} k={k} n={n} b={batch} route={route} {res}", flush=True)
    return y, route, guard_ok, res, payload, x


@pytest.mark.parametrize("type_", [kl.WeightType.f16, kl.WeightType.f32], ids=["f16", "f32"])
@pytest.mark.parametrize("k,n,batch", [(4096, 4096, 8), (4096, 4096, 2), (4096, 1000, 16), (32, 17, 3),
                                       (16384, 40, 5), (11008, 300, 12), (96, 1, 16),
                                       (4096, 1, 8), (4064, 17, 5), (544, 4100, 7)])   # F16 streamed: one row,
                                                                                    # a partial last chunk, N tail
def test_dense_mfma(gpu, oracle, type_, k, n, batch):
    _, route, guard_ok, res, _, _ = dense_case(oracle, type_, k, n, batch, k + 5 * n + batch)
    assert route == ("f16_mfma_gemv" if type_ == kl.WeightType.f16 else "f32_mfma_gemv")
    assert guard_ok and res["finite"] and res["north_star"] and res["reference"]


def test_dense_mfma_matches_vector_kernel(gpu, oracle, knobs):
    for type_ in (kl.WeightType.f16, kl.WeightType.f32):
        y1, r1, _, _, payload, x = dense_case(oracle, type_, 2048, 700, 8, 41)
        knobs("KUNLUN_DENSE_MFMA_MIN", "17")
        y2, r2, _ = run_matmul(type_, payload, x, 2048, 700, 8)
        kl.set_tuning("KUNLUN_DENSE_MFMA_MIN", None)
        assert r1.endswith("mfma_gemv") and not r2.endswith("mfma_gemv")
        # both accumulate exact products in F32, in different orders
        scale = np.abs(y2).max()
        assert np.max(np.abs(y1 - y2)) <= 1e-5 * scale
