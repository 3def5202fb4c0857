"""GPU parity of kunlun::matmul through the C ABI against the CPU oracle.

F32 / F16 / Q4_0 (F32 accumulate): every output within the north-star bound
|y - gold| <= 1e-4 * ||x_b|| * ||w_r|| and the reference bench's tolerance
|y - gold| <= 1e-3 * (1 + |gold|) (reference bench/library-bench.cpp:125-126),
gold = FP64 dot of the exactly decoded weights (library-bench.cpp:121-122).

rowwise_i8: bit-exact against the oracle's restatement of the reference path
(weight quantization k200.cpp:107-116, two-pass activation quantization
k200.cpp:212-225, exact integer dots, combine kunlun-combine.xpu:19); bitwise
equality of the F32 output pins codes, maxima and int32 sums at once. Against
unquantized FP64: the reference tolerance 2e-2 * (1 + |gold|) on the library
bench's data, and the algorithm's quantization-error bound on Gaussian data.
"""
import os
import signal
import subprocess
import sys

import numpy as np
import pytest

import kunlunk200_lib_amd as kl
from gpu_util import check_f32_accumulate, run_matmul, weight_payload

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DENSE = [kl.WeightType.f32, kl.WeightType.f16, kl.WeightType.q4_0]
TYPE_NAME = {0: "f32", 1: "f16", 2: "q4_0", 3: "i8"}


def gaussian(shape, sigma, seed):
    return (np.random.default_rng(seed).standard_normal(shape) * sigma).astype(np.float32)


def _dense_case(oracle, type_, w, x, k, n, batch, **kw):
    payload, dec = weight_payload(type_, w, oracle)
    y, route, guard_ok = run_matmul(type_, payload, x, k, n, batch, **kw)
    gold = oracle.gold(dec, x)
    res = check_f32_accumulate(y, gold, dec, x)
    print(f"  {TYPE_NAME[type_]} k={k} n={n} b={batch} route={route} max_abs={res['max_abs']:.3g} "
          f"ns_ratio={res['max_ns_ratio']:.3g} nmse={res['nmse']:.3g}", flush=True)
    assert guard_ok, "wrote past the output"
    assert res["finite"] and res["north_star"] and res["reference"], res
    return y, route


# --- the reference's own deterministic bench data --------------------------

@pytest.mark.parametrize("type_", DENSE, ids=lambda t: TYPE_NAME[t])
@pytest.mark.parametrize("k,n,batch", [(256, 65, 4), (4096, 4096, 1), (512, 33, 32)])
def test_library_bench_dense(gpu, oracle, type_, k, n, batch):
    w, wh, q4 = oracle.bench_weights(k, n)
    x = oracle.bench_input(k, batch)
    payload = {0: w.view(np.uint8), 1: wh.view(np.uint8), 2: q4}[int(type_)]
    y, route, guard_ok = run_matmul(type_, payload, x, k, n, batch)
    gold = oracle.gold(w, x)
    res = check_f32_accumulate(y, gold, w, x)
    print(f"  library-bench {TYPE_NAME[type_]} {k}/{n}/{batch} route={route} {res}", flush=True)
    assert guard_ok and res["finite"] and res["reference"] and res["north_star"]


@pytest.mark.parametrize("k,n,batch", [(256, 65, 4), (4096, 4096, 1), (256, 65, 32)])
def test_library_bench_i8(gpu, oracle, k, n, batch):
    w, _, _ = oracle.bench_weights(k, n)
    x = oracle.bench_input(k, batch)
    y, route, guard_ok = run_matmul(kl.WeightType.rowwise_i8, None, x, k, n, batch, w_f32=w)
    expect = oracle.rowwise_i8_matmul(w, x)
    gold = oracle.gold(w, x)
    print(f"  library-bench i8 {k}/{n}/{batch} route={route} max_abs_vs_fp64="
          f"{np.max(np.abs(y - gold)):.3g}", flush=True)
    assert guard_ok
    assert np.array_equal(y.view(np.uint32), expect.view(np.uint32)), "rowwise_i8 not bit-exact"
    assert np.all(np.abs(y - gold) <= 0.02 * (1 + np.abs(gold)))


def test_fused_bench_periodic_rows(gpu, oracle):
    # reference bench/fused-bench.cpp: gold of row r equals row r % 16
    k, n, batch = 4096, 4096, 1
    w, q4 = oracle.fused_bench_weights(k, n)
    x = oracle.bench_input(k, batch)
    gold16 = oracle.gold(w[:16], x)
    y, _, _ = run_matmul(kl.WeightType.q4_0, q4, x, k, n, batch)
    ref = gold16[:, np.arange(n) % 16]
    assert np.all(np.abs(y - ref) <= 0.001 * (1 + np.abs(ref)))


# --- seeded Gaussian weights, BASELINE shapes and edge shapes --------------

SHAPES = [
    (32, 1, 1), (64, 7, 1), (96, 17, 3), (256, 65, 4), (512, 300, 2), (4096, 4096, 1),
    (4096, 11008, 1), (11008, 4096, 1), (4096, 12288, 1), (4096, 1024, 8), (4096, 512, 16),
    (4096, 64, 5), (16384, 96, 1), (16384, 40, 3), (14336, 256, 2),
    (512, 130, 17), (1024, 70, 22),   # F32/F16 above 16 columns: passes of 4 columns (and a last single one)
]


@pytest.mark.parametrize("type_", DENSE, ids=lambda t: TYPE_NAME[t])
@pytest.mark.parametrize("k,n,batch", SHAPES)
def test_gaussian_dense(gpu, oracle, type_, k, n, batch):
    seed = k * 1_000_003 + n * 101 + batch
    w = gaussian((n, k), 0.02, seed)
    x = gaussian((batch, k), 1.0, seed + 1)
    _dense_case(oracle, type_, w, x, k, n, batch)


@pytest.mark.parametrize("pattern", range(5))
@pytest.mark.parametrize("batch", [1, 2, 4])
def test_native_q4_fixture_patterns(gpu, oracle, pattern, batch):
    # seeded weights and the five activation patterns of bench/native-q4-reference.h
    k, n = 512, 160
    q4 = oracle.fixture_q4(k, n)
    dec = oracle.q4_decode(q4, k, n)
    x = oracle.fixture_input(k, batch, pattern)
    y, route, guard_ok = run_matmul(kl.WeightType.q4_0, q4, x, k, n, batch)
    gold = oracle.gold(dec, x)
    res = check_f32_accumulate(y, gold, dec, x)
    assert guard_ok and res["finite"] and res["north_star"] and res["reference"], res
    if pattern == 2:
        assert np.all(y == 0)


# --- routing, alignment fallbacks, stability --------------------------------

def test_q4_misaligned_weights_use_general_kernel(gpu, oracle):
    k, n, batch = 4096, 300, 2
    w = gaussian((n, k), 0.02, 11)
    x = gaussian((batch, k), 1.0, 12)
    _, route = _dense_case(oracle, kl.WeightType.q4_0, w, x, k, n, batch, w_offset=2)
    assert route == "gemv_general"
    _, route = _dense_case(oracle, kl.WeightType.q4_0, w, x, k, n, batch, w_offset=0)
    assert route in ("q4_gemv_dot8", "q4_bdiag_gemv", "q4_mfma_gemv")


# batches between the small-batch kernels (<= 16) and the GEMM (>= 64): chunks
# of 16 columns, each on the small-batch route a 16-column call takes
@pytest.mark.parametrize("type_", DENSE, ids=lambda t: TYPE_NAME[t])
@pytest.mark.parametrize("k,n,batch", [(4096, 300, 33), (512, 130, 17), (1088, 65, 48)])
def test_mid_batch_chunks(gpu, oracle, type_, k, n, batch):
    seed = k + n + batch + int(type_)
    w = gaussian((n, k), 0.02, seed)
    x = gaussian((batch, k), 1.0, seed + 1)
    _, route = _dense_case(oracle, type_, w, x, k, n, batch)
    assert route in ("q4_stream_gemv", "q4_bdiag_gemv", "q4_mfma_gemv", "f16_mfma_gemv", "f32_mfma_gemv")


def test_unaligned_activation_uses_general_kernel(gpu, oracle):
    k, n, batch = 1024, 129, 1
    w = gaussian((n, k), 0.02, 13)
    x = gaussian((batch, k), 1.0, 14)
    for type_ in DENSE:
        _, route = _dense_case(oracle, type_, w, x, k, n, batch, x_offset=4)
        assert route == "gemv_general"


def test_odd_block_count_uses_general_kernel(gpu, oracle):
    k, n, batch = 32 * 33, 70, 2
    w = gaussian((n, k), 0.02, 15)
    x = gaussian((batch, k), 1.0, 16)
    _, route = _dense_case(oracle, kl.WeightType.q4_0, w, x, k, n, batch)
    assert route == "gemv_general"


def test_repeat_is_bitwise_stable(gpu, oracle):
    k, n, batch = 4096, 2048, 1
    w = gaussian((n, k), 0.02, 17)
    x = gaussian((batch, k), 1.0, 18)
    kernel = kl.Kernel()
    payload, _ = weight_payload(kl.WeightType.q4_0, w, oracle)
    y1, _, _ = run_matmul(kl.WeightType.q4_0, payload, x, k, n, batch, kernel=kernel)
    y2, _, _ = run_matmul(kl.WeightType.q4_0, payload, x, k, n, batch, kernel=kernel)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


def test_statistics_count_submissions(gpu, oracle):
    before = kl.statistics()["matmuls"][0]
    k, n = 64, 8
    w = gaussian((n, k), 0.02, 19)
    x = gaussian((1, k), 1.0, 20)
    run_matmul(kl.WeightType.f32, w.view(np.uint8), x, k, n, 1)
    assert kl.statistics()["matmuls"][0] == before + 1
    assert kl.matmul_count(0) == before + 1


# --- rowwise_i8 --------------------------------------------------------------

# batch <= 64: K-split kernel with 1, 2, 4 or 8 row tiles of 16 code rows
# (batch 1-8, 9-16, 17-32, 33-64); above: the LDS-staged GEMM when K % 128 == 0
# (partial M and N tiles: 100, 130, 97 batch rows, N 300, 130), else the
# register-tiled one (96, 70)
I8_SHAPES = [(64, 3, 1), (1024, 512, 4), (4096, 4096, 1), (96, 17, 9), (4096, 1024, 32), (4096, 4096, 32),
             (4096, 4096, 512),
             (16384, 64, 2), (2048, 300, 8), (1024, 256, 100), (2048, 96, 17), (256, 70, 40), (512, 200, 64),
             (512, 300, 130), (2048, 130, 97), (96, 40, 70)]


@pytest.mark.parametrize("k,n,batch", I8_SHAPES)
def test_rowwise_i8_bit_exact(gpu, oracle, k, n, batch):
    seed = k * 7 + n * 3 + batch
    w = gaussian((n, k), 0.02, seed)
    x = gaussian((batch, k), 1.0, seed + 1)
    y, route, guard_ok = run_matmul(kl.WeightType.rowwise_i8, None, x, k, n, batch, w_f32=w)
    expect = oracle.rowwise_i8_matmul(w, x)
    gold = oracle.gold(w, x)
    print(f"  i8 k={k} n={n} b={batch} route={route} max_abs_vs_fp64={np.max(np.abs(y - gold)):.3g}", flush=True)
    assert guard_ok
    assert np.array_equal(y.view(np.uint32), expect.view(np.uint32)), "rowwise_i8 not bit-exact"
    # On Gaussian data the reference algorithm itself (per-row INT8 weights) can
    # exceed the library bench's 2e-2*(1+|gold|); bound its error instead:
    # |dw| <= max|w_r|/254 per weight, |dx| <= max|r|/254 per activation.
    assert np.all(np.abs(y - gold) <= i8_error_bound(w, x))


@pytest.mark.parametrize("k,n,batch", [(1024, 96, 3), (2048, 64, 40), (4096, 32, 20)])
def test_rowwise_i8_activation_4_byte_aligned(gpu, oracle, k, n, batch):
    # X only float-aligned: the quantizer's 16-byte loads run at 4-byte alignment
    # (single-workgroup quantizer up to 16384 values by default, three passes above)
    w = gaussian((n, k), 0.02, k + n)
    x = gaussian((batch, k), 1.0, k + n + 1)
    y, route, guard_ok = run_matmul(kl.WeightType.rowwise_i8, None, x, k, n, batch, w_f32=w, x_offset=4)
    assert guard_ok
    assert np.array_equal(y.view(np.uint32), oracle.rowwise_i8_matmul(w, x).view(np.uint32))


def i8_error_bound(w, x):
    amax_w = np.abs(w).max(axis=1).astype(np.float64)[None, :]
    x64 = x.astype(np.float64)
    max0 = max(np.abs(x64).max(), 1e-30)
    max1 = max0 / 254.0                      # |residual| <= half a primary step
    l1x = np.abs(x64).sum(axis=1)[:, None]
    k = x.shape[1]
    return 1.01 * (amax_w / 254.0 * (l1x + k * max1 / 254.0) + amax_w * (1 + 1 / 254.0) * k * max1 / 254.0) + 1e-6


@pytest.mark.parametrize("pattern", range(5))
def test_rowwise_i8_fixture_patterns(gpu, oracle, pattern):
    k, n, batch = 512, 96, 3
    dec = oracle.q4_decode(oracle.fixture_q4(k, n), k, n)
    x = oracle.fixture_input(k, batch, pattern)
    y, _, _ = run_matmul(kl.WeightType.rowwise_i8, None, x, k, n, batch, w_f32=dec)
    expect = oracle.rowwise_i8_matmul(dec, x)
    assert np.array_equal(y.view(np.uint32), expect.view(np.uint32))


@pytest.mark.parametrize("limit,k,n,batch", [(None, 1024, 64, 16), (None, 1024, 64, 17), ("65536", 4096, 48, 16),
                                              ("65536", 2048, 96, 17), ("65536", 16384, 64, 2)])
def test_rowwise_i8_single_workgroup_quantizer_limit(gpu, oracle, knobs, limit, k, n, batch):
    # batch*k = 16384 (the default limit) and 17408 either side of it; with the
    # limit raised to its maximum, the single-workgroup quantizer up to 65536 values
    if limit is not None:
        knobs("KUNLUN_I8_FUSED_QUANT_LIMIT", limit)
    w = gaussian((n, k), 0.02, k + batch)
    x = gaussian((batch, k), 1.0, k + batch + 1)
    x[batch - 1, k - 1] = -11.0
    y, _, guard_ok = run_matmul(kl.WeightType.rowwise_i8, None, x, k, n, batch, w_f32=w)
    assert guard_ok
    assert np.array_equal(y.view(np.uint32), oracle.rowwise_i8_matmul(w, x).view(np.uint32))


def test_rowwise_i8_large_activation_path(gpu, oracle):
    # batch*k above the single-workgroup quantizer limit: three-pass quantizer
    k, n, batch = 4096, 128, 24
    w = gaussian((n, k), 0.02, 23)
    x = gaussian((batch, k), 1.0, 24)
    x[5, 7] = 37.0   # a single outlier sets max0
    y, _, _ = run_matmul(kl.WeightType.rowwise_i8, None, x, k, n, batch, w_f32=w)
    expect = oracle.rowwise_i8_matmul(w, x)
    assert np.array_equal(y.view(np.uint32), expect.view(np.uint32))


@pytest.mark.parametrize("k,n,batch", [(4096, 64, 300), (4096, 48, 600), (16384, 32, 300), (2080, 40, 1009)])
def test_rowwise_i8_quantizer_pass_shapes(gpu, oracle, k, n, batch):
    # the three passes at 2 and 4 float4 groups per thread (X above 1M and 2M
    # values), their grid-stride loop (above 4M values) and a grid whose last
    # workgroup is partial (2080 * 1009 values); the outliers that set max0
    # sit in the last group and in the middle
    w = gaussian((n, k), 0.02, k + n + batch)
    x = gaussian((batch, k), 1.0, k + n + batch + 1)
    x[batch - 1, k - 1] = -23.5
    x[batch // 2, 5] = 19.0
    y, _, guard_ok = run_matmul(kl.WeightType.rowwise_i8, None, x, k, n, batch, w_f32=w)
    assert guard_ok
    assert np.array_equal(y.view(np.uint32), oracle.rowwise_i8_matmul(w, x).view(np.uint32))


@pytest.mark.parametrize("k,batch", [(64, 1), (4096, 20)])
def test_rowwise_i8_nonfinite_activation_aborts_at_wait(gpu, k, batch):
    # reference src/k200.cpp:213 aborts on a non-finite activation; here the
    # device flags it and wait() aborts with the same diagnostic (batch 1: the
    # fused GEMV's quantizer; 4096 x 20: the three-pass quantizer).
    code = (
        "import numpy as np, sys\n"
        f"sys.path.insert(0, {os.path.join(ROOT, 'tests')!r})\n"
        "import kunlunk200_lib_amd as kl\n"
        "from gpu_util import run_matmul\n"
        f"w = np.ones((8, {k}), np.float32); x = np.ones(({batch}, {k}), np.float32); x[{batch} - 1, 3] = np.inf\n"
        f"run_matmul(kl.WeightType.rowwise_i8, None, x, {k}, 8, {batch}, w_f32=w)\n"
        "print('NOT REJECTED')\n"
    )
    env = dict(os.environ, PYTHONPATH=ROOT)
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=300)
    assert "NOT REJECTED" not in proc.stdout
    assert proc.returncode == -signal.SIGABRT, proc.stderr[-2000:]
    assert "non-finite" in proc.stderr


# --- BASELINE configs on the route a default matmul takes ---------------------

@pytest.mark.parametrize("k,n,batch,route", [
    (4096, 32000, 1, "q4_gemv_dot8"),      # configs[1]: LM head
    (4096, 14336, 2, "q4_gemv_dot8"),      # configs[2]: batch 2 (two columns per pass)
    (4096, 14336, 4, "q4_bdiag_gemv"),     # activation fragments of all of K fit in LDS
    (4096, 14336, 8, "q4_stream_gemv"),    # batch 5..8 at K = 4096: rows streamed through per-wave LDS
    (4096, 14336, 16, "q4_mfma_gemv"),     # they do not: the LDS-staged kernel
])
def test_q4_baseline_configs_default_route(gpu, oracle, k, n, batch, route):
    seed = k * 3 + n + batch
    w = gaussian((n, k), 0.02, seed)
    x = gaussian((batch, k), 1.0, seed + 1)
    _, got = _dense_case(oracle, kl.WeightType.q4_0, w, x, k, n, batch)
    assert got == route


def two_fc_rowwise_i8(oracle, w, x):
    """The reference's batch > 8 rowwise_i8 order (src/k200.cpp:233-239): two
    int8 FCs with input maxima max0 and max1 and weight maxima 127, each
    y_c = sum_k (q_x * m_c / 127) * (q_w * 127 / 127), added, then multiplied
    by the row scales. The FC's own accumulation order is closed (XDNN); it is
    taken here as the exact dot times m_c / 127 in FP64, rounded to F32."""
    codes, scales = oracle.i8_rows(w)
    q0, q1, m0, m1 = oracle.i8_activation(x)
    fc0 = (oracle.i8_dots(q0, codes).astype(np.float64) * (np.float64(m0) / 127.0)).astype(np.float32)
    fc1 = (oracle.i8_dots(q1, codes).astype(np.float64) * (np.float64(m1) / 127.0)).astype(np.float32)
    return ((fc0 + fc1) * scales[None, :]).astype(np.float32)


@pytest.mark.parametrize("k,n,batch", [(4096, 512, 9), (4096, 4096, 16), (1024, 512, 32)])
def test_rowwise_i8_matches_two_fc_order(gpu, oracle, k, n, batch):
    # reference bench/fused-bench.cpp:29-51: fused and two-FC results agree to
    # NMSE <= 1e-8 (:48); batch > 8 is where the reference takes the two-FC order
    w, _ = oracle.fused_bench_weights(k, n)
    x = oracle.bench_input(k, batch)
    y, _, guard_ok = run_matmul(kl.WeightType.rowwise_i8, None, x, k, n, batch, w_f32=w)
    legacy = two_fc_rowwise_i8(oracle, w, x)
    e = y.astype(np.float64) - legacy
    nmse = float((e * e).sum() / max(float((legacy.astype(np.float64) ** 2).sum()), 1e-30))
    print(f"  i8 vs two-FC k={k} n={n} b={batch}: nmse={nmse:.3g}", flush=True)
    assert guard_ok and np.all(np.isfinite(y)) and nmse <= 1e-8
