"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against something other than its own formula:
the reference's own CPU oracle header compiled from the reference checkout
(golden vectors in tests/golden/, and the live oracle/_ref build when present),
numpy's float16 conversions, brute force and closed forms of the reference's
deterministic bench data.
"""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "native_q4_reference.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


# --- against the reference's own CPU oracle (golden vectors) ---------------

def test_fixture_q4_bytes_match_reference(oracle, golden):
    k, n = int(golden["k"]), int(golden["n"])
    assert np.array_equal(oracle.fixture_q4(k, n), golden["q4"])


def test_q4_decode_matches_reference_decoded(oracle, golden):
    k, n = int(golden["k"]), int(golden["n"])
    dec = oracle.q4_decode(golden["q4"], k, n)
    assert np.array_equal(dec.view(np.uint32), golden["decoded"].view(np.uint32))


@pytest.mark.parametrize("pattern", range(5))
def test_fixture_inputs_match_reference(oracle, golden, pattern):
    k, batch = int(golden["k"]), int(golden["batch"])
    x = oracle.fixture_input(k, batch, pattern)
    assert np.array_equal(x.view(np.uint32), golden[f"x{pattern}"].view(np.uint32))


@pytest.mark.parametrize("pattern", range(5))
def test_gold_matches_reference_fp64(oracle, golden, pattern):
    # The reference sums with an OpenMP simd reduction (another order), so the
    # FP64 results agree to rounding of the sum, far below any test tolerance.
    w, x = golden["decoded"], golden[f"x{pattern}"]
    y = oracle.gold(w, x)
    bound = 1e-13 * (np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T) + 1e-300
    assert np.all(np.abs(y - golden[f"y{pattern}"]) <= bound)


@pytest.mark.parametrize("pattern", range(5))
def test_i8_activation_matches_reference(oracle, golden, pattern):
    x = golden[f"x{pattern}"]
    q0, q1, m0, m1 = oracle.i8_activation(x)
    act, scales = golden[f"act{pattern}"], golden[f"act_scales{pattern}"]
    assert np.array_equal(q0, act[0]) and np.array_equal(q1, act[1])
    assert np.float32(m0 / np.float32(127)) == scales[0]
    assert np.float32(m1 / np.float32(127)) == scales[1]


def test_i8_rows_match_reference_one_component(oracle, golden):
    codes, scales = oracle.i8_rows(golden["decoded"])
    assert np.array_equal(codes, golden["row_codes"])
    assert np.array_equal(scales, golden["row_scales8"])
    assert np.array_equal(scales, golden["row_scales"])


def test_reference_build_agrees_live(oracle, kref):
    # Wider shapes than the committed fixture, straight from oracle/_ref.
    for k, n in ((512, 37), (1024, 64), (96, 5)):
        q4, dec, _ = kref.weights(k, n)
        assert np.array_equal(oracle.fixture_q4(k, n), q4)
        assert np.array_equal(oracle.q4_decode(q4, k, n).view(np.uint32), dec.view(np.uint32))
        for pattern in range(5):
            x = kref.input(k, 3, pattern)
            assert np.array_equal(oracle.fixture_input(k, 3, pattern).view(np.uint32), x.view(np.uint32))
            act, sc = kref.activation(x)
            q0, q1, m0, m1 = oracle.i8_activation(x)
            assert np.array_equal(q0, act[0]) and np.array_equal(q1, act[1])


# --- F16 conversions against numpy ---------------------------------------

def test_half_to_float_all_bit_patterns(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = oracle.f16_decode(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_float_to_half_round_trip_and_rne(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    values = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(values)
    assert np.array_equal(oracle.f16_encode(values[finite]), bits[finite])
    # midpoints between neighbouring finite halves exercise ties-to-even
    pos = np.sort(values[finite & (values >= 0)])
    mids = ((pos[:-1].astype(np.float64) + pos[1:].astype(np.float64)) / 2).astype(np.float32)
    for sample in (mids, -mids):
        assert np.array_equal(oracle.f16_encode(sample), sample.astype(np.float16).view(np.uint16))
    rng = np.random.default_rng(7)
    raw = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    raw = raw[np.isfinite(raw)]
    with np.errstate(over="ignore"):
        assert np.array_equal(oracle.f16_encode(raw), raw.astype(np.float16).view(np.uint16))


# --- rounding rule against brute force -----------------------------------

def _nearest_away(v: float, limit: int) -> int:
    best = None
    for q in range(-limit, limit + 1):
        d = abs(np.float64(v) - q)
        if best is None or d < best[0] - 1e-12 or (abs(d - best[0]) <= 1e-12 and abs(q) > abs(best[1])):
            best = (d, q)
    return best[1]


def test_round_clamp_brute_force(oracle):
    values = [0.0, -0.0, 0.49, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5, 126.49, 127.0, -127.0,
              127.4, 300.0, -300.0, 1e-30, -1e-30, 63.5, -63.5]
    for v in values:
        assert oracle.round_clamp(np.float32(v), 127) == _nearest_away(np.float32(v), 127), v


# --- closed forms of the reference's deterministic benches ----------------

@pytest.mark.parametrize("k,n", [(256, 65), (4096, 3), (96, 17)])
def test_bench_weights_q4_and_f16_encode_the_same_values(oracle, k, n):
    w, wh, q4 = oracle.bench_weights(k, n)
    r = np.arange(n)[:, None]
    j = np.arange(k)[None, :]
    assert np.array_equal(w, (((r + j) % 16 - 8) * 0.0625).astype(np.float32))
    assert np.array_equal(oracle.q4_decode(q4, k, n), w)
    assert np.array_equal(oracle.f16_decode(wh), w)


def test_fused_bench_rows_repeat_every_16(oracle):
    k, n = 256, 48
    w, q4 = oracle.fused_bench_weights(k, n)
    assert np.array_equal(oracle.q4_decode(q4, k, n), w)
    x = oracle.bench_input(k, 2)
    y = oracle.gold(w, x)
    for r in range(n):
        assert np.array_equal(y[:, r], y[:, r % 16])


def test_bench_input_is_sine(oracle):
    x = oracle.bench_input(64, 3).ravel()
    expect = np.sin(np.arange(x.size, dtype=np.float32) * np.float32(0.017)).astype(np.float32)
    assert np.max(np.abs(x - expect)) <= 2e-7


# --- FP64 gold, F32 order, integer dots, combine ----------------------------

def test_gold_against_numpy_float64(oracle):
    rng = np.random.default_rng(1)
    w = rng.standard_normal((37, 96)).astype(np.float32)
    x = rng.standard_normal((3, 96)).astype(np.float32)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.allclose(oracle.gold(w, x), ref, rtol=1e-13, atol=1e-13)


def test_matvec_f32_order_within_f32_error(oracle):
    rng = np.random.default_rng(2)
    k, n = 512, 40
    w = rng.standard_normal((n, k)).astype(np.float32)
    x = rng.standard_normal((2, k)).astype(np.float32)
    gold = oracle.gold(w, x)
    for type_, wb in ((0, w), (1, w.astype(np.float16)), (2, oracle.q4_quantize(w))):
        dec = w if type_ == 0 else (wb.astype(np.float32) if type_ == 1 else oracle.q4_decode(wb, k, n))
        ref = oracle.gold(dec, x)
        got = oracle.matvec_f32(np.asarray(wb), type_, x, k, n)
        bound = 2 * k * 2.0**-24 * (np.abs(x.astype(np.float64)) @ np.abs(dec.astype(np.float64)).T)
        assert np.all(np.abs(got - ref) <= bound + 1e-30)
    assert gold.shape == (2, n)


def test_i8_dots_against_numpy(oracle):
    rng = np.random.default_rng(3)
    a = rng.integers(-127, 128, size=(5, 160)).astype(np.int8)
    w = rng.integers(-127, 128, size=(9, 160)).astype(np.int8)
    assert np.array_equal(oracle.i8_dots(a, w), a.astype(np.int64) @ w.astype(np.int64).T)
    big = np.full((1, 16384), 127, np.int8)
    assert oracle.i8_dots(big, -big)[0, 0] == -16384 * 127 * 127


def test_i8_combine_known_answers(oracle):
    # s0 = 127/127 = 1, s1 = 254/127 = 2: (10*1 + 4*2) * 0.25 = 4.5; swapping the
    # components or scales would give 6.0.
    y = oracle.i8_combine(np.array([[10]]), np.array([[4]]), np.array([0.25], np.float32), 127.0, 254.0)
    assert y[0, 0] == np.float32(4.5)
    y = oracle.i8_combine(np.array([[10, -3]]), np.array([[4, 5]]), np.array([0.25, 2.0], np.float32),
                          63.5, 127.0)
    assert y[0, 0] == np.float32(2.25) and y[0, 1] == np.float32(7.0)


def test_i8_activation_rejects_nonfinite(oracle):
    x = np.ones((1, 64), np.float32)
    x[0, 5] = np.inf
    assert oracle.i8_activation(x) is None
    x[0, 5] = np.nan
    assert oracle.i8_activation(x) is None


def test_i8_activation_zero_tensor(oracle):
    q0, q1, m0, m1 = oracle.i8_activation(np.zeros((2, 64), np.float32))
    assert m0 == 1.0 and m1 == 1.0 and not q0.any() and not q1.any()


# --- Q4_0 quantizer: properties only (ggml absent: parity unpinned) --------

def test_q4_quantize_properties(oracle):
    rng = np.random.default_rng(4)
    k, n = 256, 64
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[3, 32:64] = 0.0
    q4 = oracle.q4_quantize(w)
    blocks = q4.reshape(n, k // 32, 18)
    d = blocks[..., :2].copy().view(np.float16).astype(np.float32)[..., 0]
    dec = oracle.q4_decode(q4, k, n).reshape(n, k // 32, 32)
    wb = w.reshape(n, k // 32, 32)
    nib = np.concatenate([blocks[..., 2:] & 15, blocks[..., 2:] >> 4], axis=2)
    # the signed extreme maps to nibble 0 and decodes to -8*d (d = max/-8)
    idx = np.argmax(np.abs(wb), axis=2)
    nonzero = d != 0
    assert np.all(np.take_along_axis(nib, idx[..., None], 2)[..., 0][nonzero] == 0)
    assert np.all(np.sign(d) == -np.sign(np.take_along_axis(wb, idx[..., None], 2)[..., 0]))
    # every element within half a step of its value (plus F16 scale rounding)
    err = np.abs(dec - wb)
    tol = np.abs(d)[..., None] * (0.5 + 8 * 2.0**-11) + 1e-12
    clamp = nib == 15
    assert np.all(err[~clamp] <= tol[..., 0:1].repeat(32, 2)[~clamp])
    # the all-zero block: zero scale, every nibble 8
    assert d[3, 1] == 0 and np.all(nib[3, 1] == 8)


# ---------------------------------------------------------------------------
# SwiGLU (reference kernels/kunlun-swiglu.xpu:27-39): the non-finite cases
# worked by hand from the rule, and finite values against the FP64 closed form.

INF, NAN = float("inf"), float("nan")


def _classify(v):
    if np.isnan(v):
        return "nan"
    if np.isinf(v):
        return "+inf" if v > 0 else "-inf"
    return "finite"


@pytest.mark.parametrize("g,u,expected", [
    (0.0, INF, "nan"),        # SiLU(0) = 0, 0 * Inf
    (-0.0, -INF, "nan"),
    (1.0, INF, "+inf"),
    (-1.0, INF, "-inf"),      # SiLU(-1) < 0
    (-1.0, -INF, "+inf"),
    (-200.0, INF, "nan"),     # SiLU(-200) underflows to -0
    (INF, 0.0, "nan"),
    (INF, 2.0, "+inf"),
    (INF, -2.0, "-inf"),
    (-INF, 0.0, "nan"),       # g = -Inf is always NaN
    (-INF, 5.0, "nan"),
    (1.0, NAN, "nan"),
    (NAN, 1.0, "nan"),
    (NAN, INF, "nan"),
])
def test_swiglu_nonfinite_rule(oracle, g, u, expected):
    assert _classify(oracle.swiglu_value(g, u)) == expected


def test_swiglu_finite_closed_form(oracle):
    rng = np.random.default_rng(3)
    g = np.concatenate([rng.standard_normal(4000) * 8, np.linspace(-100, 100, 1001), [0.0, -0.0, 1e-8, -1e-8]])
    u = rng.standard_normal(g.size) * 4
    got = np.array([oracle.swiglu_value(float(a), float(b)) for a, b in zip(g.astype(np.float32),
                                                                          u.astype(np.float32))])
    g64, u64 = g.astype(np.float32).astype(np.float64), u.astype(np.float32).astype(np.float64)
    ref = g64 * u64 / (1.0 + np.exp(-g64))
    # e^-g overflows F32 below g = -88.72: the F32 formula then gives g / Inf = -0
    # exactly, times u (a signed zero), where FP64 still has a subnormal result
    overflow = -g64 > np.log(np.finfo(np.float32).max)
    assert np.all(got[overflow] == 0.0)
    # elsewhere expf, the division and the product round once each: a few ulp of F32
    tol = 4 * np.finfo(np.float32).eps * np.abs(ref) + 1e-44
    assert np.all(np.abs(got - ref)[~overflow] <= tol[~overflow])
    # sign and zero structure
    assert oracle.swiglu_value(0.0, 3.0) == 0.0
    assert oracle.swiglu_value(2.0, 0.0) == 0.0


def test_swiglu_rows_strides_f16_and_alias(oracle):
    rng = np.random.default_rng(4)
    width, rows = 37, 5
    for bytes_, dt in ((4, np.float32), (2, np.float16)):
        stride = width * bytes_ + 3 * bytes_          # gap between rows
        gate = np.zeros(rows * stride, np.uint8)
        up = np.zeros(rows * stride, np.uint8)
        gv = (rng.standard_normal((rows, width)) * 3).astype(dt)
        uv = (rng.standard_normal((rows, width)) * 3).astype(dt)
        for r in range(rows):
            gate[r * stride:r * stride + width * bytes_] = gv[r].view(np.uint8)
            up[r * stride:r * stride + width * bytes_] = uv[r].view(np.uint8)
        y = np.full(rows * stride, 0xA5, np.uint8)
        oracle.swiglu_bytes(gate, up, y, width, rows, stride, stride, stride, bytes_)
        for r in range(rows):
            row = y[r * stride:(r + 1) * stride]
            out = row[:width * bytes_].view(dt)
            expect = np.array([oracle.swiglu_value(float(a), float(b)) for a, b in zip(gv[r], uv[r])],
                              np.float32).astype(dt)   # one final rounding (numpy float16 is RNE)
            assert np.array_equal(out.view(np.uint8), expect.view(np.uint8))
            assert np.all(row[width * bytes_:] == 0xA5)  # the gap is not written
        # output aliasing gate element for element gives the same values
        alias = gate.copy()
        oracle.swiglu_bytes(alias, up, alias, width, rows, stride, stride, stride, bytes_)
        for r in range(rows):
            assert np.array_equal(alias[r * stride:r * stride + width * bytes_],
                                  y[r * stride:r * stride + width * bytes_])


# ---------------------------------------------------------------------------
# Elementwise (reference kernels/kunlun-elementwise.xpu, src/k200.cpp:280-323)

def _library_bench_data(k: int, batch: int):
    """Inputs of the reference bench/library-bench.cpp:51-53."""
    count = k * batch
    a = np.sin(np.arange(count, dtype=np.float32) * np.float32(0.021)).astype(np.float32)
    b = np.cos(np.arange(k, dtype=np.float32) * np.float32(0.04)).astype(np.float32)
    return a, b


def _library_bench_gold(a, b, k, batch, op, parameter):
    """The reference's gold (bench/library-bench.cpp:62-67): FP64 row sums."""
    rows = a.reshape(batch, k).astype(np.float64)
    if op == 0:
        return (rows + b).ravel()
    if op == 1:
        return (rows * b).ravel()
    if op == 2:
        return (rows / (1 + np.exp(-rows))).ravel()
    if op == 4:
        return (rows * parameter).ravel()
    sums = (rows * rows).sum(axis=1, keepdims=True)
    return (rows / np.sqrt(sums / k + parameter)).ravel()


@pytest.mark.parametrize("op", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("k,batch", [(256, 4), (4096, 1), (32, 32)])
def test_elementwise_library_bench_gold(oracle, op, k, batch):
    a, b = _library_bench_data(k, batch)
    parameter = 0.75 if op == 4 else 1e-5
    y = oracle.elementwise(a, b, k, op, parameter)
    assert np.all(np.isfinite(y))
    assert np.max(np.abs(y - _library_bench_gold(a, b, k, batch, op, parameter))) < 1e-4


def test_elementwise_add_multiply_scale_exact(oracle):
    rng = np.random.default_rng(5)
    width, rows = 96, 7
    a = rng.standard_normal(width * rows).astype(np.float32) * 100
    full = rng.standard_normal(width * rows).astype(np.float32)
    row = rng.standard_normal(width).astype(np.float32)
    assert np.array_equal(oracle.elementwise(a, full, width, 0), a + full)
    assert np.array_equal(oracle.elementwise(a, row, width, 0), a + np.tile(row, rows))
    assert np.array_equal(oracle.elementwise(a, row, width, 1), a * np.tile(row, rows))
    assert np.array_equal(oracle.elementwise(a, full, width, 1), a * full)
    assert np.array_equal(oracle.elementwise(a, row, width, 4, -0.375), a * np.float32(-0.375))


def test_elementwise_silu_closed_form(oracle):
    v = np.concatenate([np.linspace(-80, 80, 4001), [0.0, -0.0, 1e-30, -1e-30, 87.0, -87.0]]).astype(np.float32)
    y = oracle.elementwise(v, v, v.size, 2)
    exact = v.astype(np.float64) / (1 + np.exp(-v.astype(np.float64)))
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(y - exact) <= 4 * ulp)
    assert y[v.size - 6] == 0.0
    # a << 0: expf(-a) overflows to inf and a / inf is -0
    assert oracle.elementwise(np.float32([-100.0]), np.float32([0]), 1, 2)[0] == 0.0


def test_elementwise_rms_norm_closed_form_and_alias(oracle):
    rng = np.random.default_rng(11)
    width, rows = 1000, 5
    a = (rng.standard_normal(width * rows) * rng.uniform(0.01, 50, width * rows)).astype(np.float32)
    eps = 1e-5
    y = oracle.elementwise(a, a, width, 3, eps)
    r = a.reshape(rows, width).astype(np.float64)
    exact = r / np.sqrt((r * r).mean(axis=1, keepdims=True) + eps)
    assert np.max(np.abs(y.reshape(rows, width) - exact) / np.max(np.abs(exact))) < 1e-6
    # constant row c: y = c / sqrt(c^2 + eps) -> sign(c) for eps << c^2
    const = np.full(64, -3.0, np.float32)
    yc = oracle.elementwise(const, const, 64, 3, 1e-30)
    assert np.all(np.abs(yc + 1) <= 2 ** -22)
    # output aliasing the input gives the same values
    alias = a.copy()
    oracle.elementwise(alias, alias, width, 3, eps, out=alias)
    assert np.array_equal(alias, y)
    # a dropped eps would fail: a zero row stays zero only with eps > 0
    z = oracle.elementwise(np.zeros(32, np.float32), np.zeros(1, np.float32), 32, 3, 1e-5)
    assert np.array_equal(z, np.zeros(32, np.float32))
