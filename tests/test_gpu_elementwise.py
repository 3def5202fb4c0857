"""GPU parity of kunlun::elementwise, the library bench's pipeline and memory
operations (reference bench/library-bench.cpp:23-38, 51-78, 104-127).

elementwise against the oracle's orc_elementwise on identical F32 inputs:
add, multiply and scale bit-exact (one rounded F32 operation each); silu
within 4 F32 ulp of the oracle (the device and host expf may differ by an
ulp); rms_norm within the summation error bounds of both (the workgroup sums
squares in another order than the oracle's loop), each also checked against
the FP64 closed form. Every case
also meets the reference bench's own gate: max |y - gold| < 1e-4 against its
FP64 gold. Aliasing (y == a, y == b with b of count or of width values) and
the reference's rms_norm alias case are covered, and bytes past the output are
checked untouched.
"""
import numpy as np
import pytest

import kunlunk200_lib_amd as kl
from gpu_util import check_f32_accumulate

pytestmark = pytest.mark.gpu

GUARD = 64
GUARD_VALUE = np.float32(-7777.0)
OPS = {"add": 0, "multiply": 1, "silu": 2, "rms": 3, "scale": 4}


def library_bench_data(k: int, batch: int):
    """Inputs of reference bench/library-bench.cpp:51-53."""
    a = np.sin(np.arange(k * batch, dtype=np.float32) * np.float32(0.021)).astype(np.float32)
    b = np.cos(np.arange(k, dtype=np.float32) * np.float32(0.04)).astype(np.float32)
    return a, b


def library_bench_gold(a, b, k, batch, op, parameter):
    """Reference bench/library-bench.cpp:62-67 in FP64."""
    rows = a.reshape(batch, k).astype(np.float64)
    if op == 0:
        return (rows + b[:k]).ravel()
    if op == 1:
        return (rows * b[:k]).ravel()
    if op == 2:
        return (rows / (1 + np.exp(-rows))).ravel()
    if op == 4:
        return (rows * parameter).ravel()
    return (rows / np.sqrt((rows * rows).sum(axis=1, keepdims=True) / k + parameter)).ravel()


def run_elementwise(a, b, width, op, parameter=0.0, alias=None, kernel=None):
    """Upload a and b, run elementwise, return (y, route). alias: None (own
    output), "a" (y = a) or "b" (y = b)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    kernel = kernel or kl.Kernel()
    guard = np.full(GUARD, GUARD_VALUE, np.float32)
    # as the output, b spans all count elements; its first b.size are the input
    b_span = np.concatenate([b, np.full(a.size - b.size, GUARD_VALUE, np.float32)]) if alias == "b" else b
    abuf = kl.Buffer(0, (a.size + GUARD) * 4)
    bbuf = kl.Buffer(0, (b_span.size + GUARD) * 4)
    ybuf = kl.Buffer(0, (a.size + GUARD) * 4)
    abuf.upload(np.concatenate([a, guard]))
    bbuf.upload(np.concatenate([b_span, guard]))
    ybuf.upload(np.full(a.size + GUARD, GUARD_VALUE, np.float32))
    out = {None: ybuf, "a": abuf, "b": bbuf}[alias]
    with kl.runtime_mutex():
        kl.elementwise(kernel, 0, out.data, abuf.data, bbuf.data, a.size, width, b.size, op, parameter)
    y = out.download(a.size + GUARD, np.float32)
    assert np.array_equal(y[a.size:].view(np.uint32), guard.view(np.uint32)), "wrote past the output"
    if alias != "a":
        assert np.array_equal(abuf.download(a.size, np.float32).view(np.uint32), a.view(np.uint32))
    if alias != "b":
        assert np.array_equal(bbuf.download(b.size, np.float32).view(np.uint32), b.view(np.uint32))
    return y[:a.size], kernel.route


def check_against_oracle(y, expected, op, width, a=None, eps=0.0):
    if op in (0, 1, 4):
        assert np.array_equal(y.view(np.uint32), expected.view(np.uint32))
    elif op == 2:
        finite = np.isfinite(expected)
        assert np.array_equal(np.isnan(y), np.isnan(expected))
        assert np.array_equal(y[~finite & ~np.isnan(expected)], expected[~finite & ~np.isnan(expected)])
        ulp = np.spacing(np.abs(expected[finite]))
        assert np.all(np.abs(y[finite] - expected[finite]) <= 4 * ulp)
    else:
        rms_bounds(y, expected, a, width, eps)


def rms_bounds(y, expected, a, width, eps):
    """rms_norm: y = a * s with s = 1 / sqrt(sum(a^2) / width + eps). The
    oracle sums squares left to right in F32 (relative error <= width * u,
    u = 2^-24, so s within (width / 2 + 3) * u); the kernel sums 256 strided
    partials of width / 256 terms and a tree of 256 (s within
    (width / 512 + 12) * u). Each is checked against the FP64 closed form,
    and the two against each other by the sum of both bounds."""
    u = 2.0 ** -24
    r = a.reshape(-1, width).astype(np.float64)
    exact = (r / np.sqrt((r * r).sum(axis=1, keepdims=True) / width + eps)).ravel()
    gpu_rel = (width / 512 + 12 + 1) * u
    oracle_rel = (width / 2 + 3 + 1) * u
    assert np.all(np.abs(y - exact) <= gpu_rel * np.abs(exact) + 1e-37)
    assert np.all(np.abs(expected - exact) <= oracle_rel * np.abs(exact) + 1e-37)
    assert np.all(np.abs(y.astype(np.float64) - expected) <= (gpu_rel + oracle_rel) * np.abs(exact) + 1e-37)


@pytest.mark.parametrize("name", list(OPS))
@pytest.mark.parametrize("k,batch", [(256, 4), (4096, 1), (32, 32), (16384, 8), (11008, 16)])
def test_library_bench_elementwise(gpu, oracle, name, k, batch):
    op = OPS[name]
    a, b = library_bench_data(k, batch)
    parameter = 0.75 if name == "scale" else 1e-5
    alias = "a" if name == "rms" else None          # the reference bench's rms alias case
    y, route = run_elementwise(a, b, k, op, parameter, alias=alias)
    print(f"  {name} k={k} batch={batch} route={route}", flush=True)
    assert route == f"elementwise_{'rms_norm' if name == 'rms' else name}"
    assert np.all(np.isfinite(y))
    assert np.max(np.abs(y - library_bench_gold(a, b, k, batch, op, parameter))) < 1e-4
    check_against_oracle(y, oracle.elementwise(a, b, k, op, parameter), op, k, a, parameter)


@pytest.mark.parametrize("op", [0, 1])
@pytest.mark.parametrize("full", [False, True], ids=["row_b", "full_b"])
@pytest.mark.parametrize("alias", [None, "a", "b"])
def test_add_multiply_broadcast_and_alias(gpu, oracle, op, full, alias):
    rng = np.random.default_rng(op * 10 + full)
    width, rows = 1000, 37
    a = (rng.standard_normal(width * rows) * 30).astype(np.float32)
    b = rng.standard_normal(width * rows if full else width).astype(np.float32)
    y, _ = run_elementwise(a, b, width, op, alias=alias)
    check_against_oracle(y, oracle.elementwise(a, b, width, op), op, width)


@pytest.mark.parametrize("width,rows", [(1, 1), (7, 3), (64, 1), (257, 5), (16384, 3), (4096, 512)])
@pytest.mark.parametrize("op", [2, 3, 4])
def test_ragged_shapes(gpu, oracle, op, width, rows):
    rng = np.random.default_rng(width + rows)
    a = (rng.standard_normal(width * rows) * rng.uniform(0.01, 20, width * rows)).astype(np.float32)
    b = np.zeros(width, np.float32)
    parameter = {2: 0.0, 3: 1e-6, 4: -1.5}[op]
    y, _ = run_elementwise(a, b, width, op, parameter)
    check_against_oracle(y, oracle.elementwise(a, b, width, op, parameter), op, width, a, parameter)


def test_silu_special_values(gpu, oracle):
    a = np.float32([0.0, -0.0, np.inf, -np.inf, np.nan, 88.0, -88.0, -100.0, 1e-38, -1e-38, 3.0e38, -3.0e38])
    y, _ = run_elementwise(a, np.zeros(a.size, np.float32), a.size, 2)
    check_against_oracle(y, oracle.elementwise(a, np.zeros(a.size, np.float32), a.size, 2), 2, a.size)


def test_rms_norm_zero_and_constant_rows(gpu, oracle):
    width = 512
    a = np.concatenate([np.zeros(width), np.full(width, -3.0), np.full(width, 1e-20)]).astype(np.float32)
    b = np.zeros(width, np.float32)
    y, _ = run_elementwise(a, b, width, 3, 1e-5)
    check_against_oracle(y, oracle.elementwise(a, b, width, 3, 1e-5), 3, width, a, 1e-5)
    assert np.array_equal(y[:width], np.zeros(width, np.float32))


def test_kernel_binds_to_first_device(gpu):
    kernel = kl.Kernel()
    a = np.ones(64, np.float32)
    run_elementwise(a, a, 64, 4, 2.0, kernel=kernel)
    y, _ = run_elementwise(a, a, 64, 4, 3.0, kernel=kernel)      # same device again: accepted
    assert np.all(y == 3.0)


def test_pipeline_matmul_then_silu_in_place(gpu, oracle):
    """library-bench `pipeline` (bench/library-bench.cpp:104-127): matmul,
    wait, then silu over y in place; gold = SiLU(FP64 dot), tolerance
    1e-3 * (1 + |gold|) (0.02 for rowwise_i8 is not exercised here)."""
    for type_, k, n, batch in ((kl.WeightType.q4_0, 256, 65, 4), (kl.WeightType.f16, 4096, 4096, 1),
                               (kl.WeightType.f32, 512, 33, 32), (kl.WeightType.q4_0, 4096, 11008, 1)):
        w, wh, q4 = oracle.bench_weights(k, n)
        x = oracle.bench_input(k, batch)
        payload = {0: w.view(np.uint8), 1: wh.view(np.uint8), 2: q4}[int(type_)].ravel()
        wbuf, xbuf, ybuf = kl.Buffer(0, payload.nbytes), kl.Buffer(0, x.nbytes), kl.Buffer(0, batch * n * 4)
        wbuf.upload(payload)
        xbuf.upload(x)
        kernel = kl.Kernel()
        with kl.runtime_mutex():
            for _ in range(2):          # run() twice, as the bench does, on fresh y each time
                kl.matmul(kernel, 0, ybuf.data, wbuf.data, xbuf.data, k, n, batch, type_)
                kl.select(0)
                kl.check(kl.wait())
                kl.elementwise(kernel, 0, ybuf.data, ybuf.data, ybuf.data, n * batch, n, n * batch,
                               kl.ElementwiseOp.silu)
        y = ybuf.download((batch, n), np.float32)
        gold = oracle.gold(w, x)
        # the matmul alone meets its own bound; the pipeline meets the bench's
        ref = gold / (1 + np.exp(-gold))
        diff = np.abs(y.astype(np.float64) - ref)
        print(f"  pipeline type={int(type_)} {k}/{n}/{batch} max_abs={diff.max():.3g}", flush=True)
        assert np.all(np.isfinite(y)) and np.all(diff <= 1e-3 * (1 + np.abs(ref)))
        # and equals silu of the matmul's own output, as the oracle computes it
        yb = kl.Buffer(0, batch * n * 4)
        with kl.runtime_mutex():
            kl.matmul(kernel, 0, yb.data, wbuf.data, xbuf.data, k, n, batch, type_)
            kl.select(0)
            kl.check(kl.wait())
        plain = yb.download(batch * n, np.float32)
        res = check_f32_accumulate(plain.reshape(batch, n), gold, w, x)
        assert res["north_star"] and res["reference"], res
        check_against_oracle(y.ravel(), oracle.elementwise(plain, plain, n, 2), 2, n)


def test_memory_round_trip(gpu):
    """library-bench `memory` (bench/library-bench.cpp:23-38): H2D, D2D, peer
    copy, D2H, and peer back. One GPU here: the peer copies go device 0 to
    device 0 through the same entry point."""
    nbytes = 4 << 20
    src = ((np.arange(nbytes, dtype=np.uint64) * 131 + 7) & 255).astype(np.uint8)
    before = kl.statistics()
    a, b, remote = kl.Buffer(0, nbytes), kl.Buffer(0, nbytes), kl.Buffer(0, nbytes)
    with kl.runtime_mutex():
        kl.select(0)
        kl.check(kl.copy(a.data, src.ctypes.data, nbytes, kl.CopyKind.host_to_device))
        kl.check(kl.wait())
        kl.select(0)
        kl.check(kl.copy(b.data, a.data, nbytes, kl.CopyKind.device_to_device))
        kl.peer(0, remote.data, 0, b.data, nbytes)
        result = np.zeros(nbytes, np.uint8)
        kl.select(0)
        kl.check(kl.copy(result.ctypes.data, remote.data, nbytes, kl.CopyKind.device_to_host))
        kl.check(kl.wait())
        assert np.array_equal(result, src)
        zeros = np.zeros(nbytes, np.uint8)
        kl.check(kl.copy(a.data, zeros.ctypes.data, nbytes, kl.CopyKind.host_to_device))
        kl.check(kl.wait())
        kl.peer(0, a.data, 0, remote.data, nbytes)
        result[:] = 0
        kl.select(0)
        kl.check(kl.copy(result.ctypes.data, a.data, nbytes, kl.CopyKind.device_to_host))
        kl.check(kl.wait())
    assert np.array_equal(result, src)
    after = kl.statistics()
    assert after["peer_copies"] - before["peer_copies"] == 2
    assert after["peer_bytes"] - before["peer_bytes"] == 2 * nbytes
