"""GPU parity of native_q4_matmul and upload_native_q4 (reference
src/k200.cpp:546-617, src/q4-layout.cpp:38-45; tests
bench/native-q4-state-bench.cpp, native-q4-mixed-bench.cpp,
native-q4-bench.cpp).

Gold is the FP64 dot of the exactly decoded weights (reference
bench/native-q4-reference.h:98-108). Every output meets the north-star bound
|y - gold| <= 1e-4 * ||x_b|| * ||w_r||, and NMSE < 1e-10: the reference's gate
for its exact route (native-q4-state-bench.cpp:24), stricter than its 1e-5
gate for the accelerated one (native-q4-bench.cpp:76) - every route here is
exact up to the activations' 23-bit block fixed point. The returned flag and
the workspace counters follow the reference's routing rule (reason empty and
y, x 64-byte aligned). Inputs stay unchanged and bytes past Y untouched.
"""
import numpy as np
import pytest

import kunlunk200_lib_amd as kl

pytestmark = pytest.mark.gpu

GUARD = 64
GUARD_VALUE = np.float32(-4321.0)


def nmse(gold: np.ndarray, y: np.ndarray) -> float:
    """reference bench/native-q4-reference.h:109-115"""
    e = y.astype(np.float64) - gold
    return float((e * e).sum() / max(float((gold * gold).sum()), 1e-30))


def north_star_ok(y, gold, w, x) -> bool:
    bound = 1e-4 * np.linalg.norm(x.astype(np.float64), axis=1)[:, None] * \
        np.linalg.norm(w.astype(np.float64), axis=1)[None, :]
    return bool(np.all(np.abs(y.astype(np.float64) - gold) <= bound + 1e-30))


class NativeCase:
    """Packed weights resident on device 0 (uploaded by upload_native_q4)."""

    def __init__(self, oracle, k, n, q4=None):
        self.k, self.n = k, n
        self.q4 = oracle.fixture_q4(k, n) if q4 is None else q4
        self.w = oracle.q4_decode(self.q4, k, n)
        self.size = kl.native_q4_size(k, n)
        self.wbuf = kl.Buffer(0, self.size)
        kl.upload_native_q4(0, self.wbuf.data, self.q4, k, n)
        self.packed = oracle.pack_native_q4(self.q4, k, n)

    def run(self, ws, x, batch, f16=False, x_offset=0, y_offset=0):
        """Returns (y [batch, n], flag). x is F32 [batch, k] (rounded to F16 first when f16)."""
        k, n = self.k, self.n
        xh = x.astype(np.float16) if f16 else x.astype(np.float32)
        xbuf = kl.Buffer(0, xh.nbytes + x_offset + 64)
        ybuf = kl.Buffer(0, batch * n * 4 + y_offset + GUARD * 4)
        xbuf.upload(xh, offset=x_offset)
        ybuf.upload(np.full(batch * n + GUARD, GUARD_VALUE, np.float32), offset=y_offset)
        before = kl.matmul_count(0)
        with kl.runtime_mutex():
            flag = kl.native_q4_matmul(ws, 0, ybuf.data + y_offset, self.wbuf.data, xbuf.data + x_offset, k, n, batch,
                                       kl.InputType.f16 if f16 else kl.InputType.f32)
        assert kl.matmul_count(0) == before + 1
        out = ybuf.download(batch * n + GUARD, np.float32, offset=y_offset)
        assert np.array_equal(out[batch * n:].view(np.uint32), np.full(GUARD, GUARD_VALUE).view(np.uint32)), \
            "wrote past Y"
        assert np.array_equal(xbuf.download(xh.size, xh.dtype, offset=x_offset).view(np.uint8), xh.view(np.uint8).ravel())
        return out[:batch * n].reshape(batch, n), flag

    def weights_unchanged(self) -> bool:
        return bool(np.array_equal(self.wbuf.download(self.size, np.uint8), self.packed))


def check(oracle, case, y, x):
    gold = oracle.gold(case.w, x)
    e = nmse(gold, y)
    assert np.all(np.isfinite(y))
    assert north_star_ok(y, gold, case.w, x), "north-star bound"
    assert e < 1e-10, e
    return e


def test_upload_matches_oracle_pack(gpu, oracle):
    for k, n in ((4096, 512), (96, 384), (64, 65)):
        case = NativeCase(oracle, k, n)
        assert case.weights_unchanged()


@pytest.mark.parametrize("index", range(6))
def test_state_bench_sequence(gpu, oracle, index):
    """reference bench/native-q4-state-bench.cpp:10-36: per shape, aligned
    call (accelerated), y + 4 and x + 4 (exact route), F16 x + 2 (exact)."""
    widths = [4096, 96, 544, 32, 4096, 96]
    k, n = widths[index], 384 if index % 2 else 512
    first, second = kl.NativeQ4Workspace(), kl.NativeQ4Workspace()
    ws = first if index % 3 else second
    case = NativeCase(oracle, k, n)
    x = oracle.fixture_input(k, 1, 3)
    y, flag = case.run(ws, x, 1)
    assert flag
    check(oracle, case, y, x)
    y, flag = case.run(ws, x, 1, y_offset=4)
    assert not flag
    check(oracle, case, y, x)
    y, flag = case.run(ws, x, 1, x_offset=4)
    assert not flag
    check(oracle, case, y, x)
    xh = x.astype(np.float16).astype(np.float32)
    y, flag = case.run(ws, x, 1, f16=True, x_offset=2)
    assert not flag
    check(oracle, case, y, xh)
    s = ws.statistics()
    assert (s["accelerated"], s["fallback"]) == (1, 3)
    assert s["hbm_workspace_bytes"] == 0 and s["l3_workspace_bytes"] == 0
    assert case.weights_unchanged()


@pytest.mark.parametrize("k,n", [(4096, 4096), (4096, 11008), (11008, 4096)])
@pytest.mark.parametrize("pattern", [0, 1, 3, 4])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
def test_baseline_shapes(gpu, oracle, k, n, pattern, f16):
    """The reference's published native shapes (docs/native-q4.md:62-71)."""
    case = NativeCase(oracle, k, n)
    ws = kl.NativeQ4Workspace()
    x = oracle.fixture_input(k, 1, pattern)
    y, flag = case.run(ws, x, 1, f16=f16)
    assert flag == (kl.native_q4_reason(k, n, 1) == "")
    e = check(oracle, case, y, x.astype(np.float16).astype(np.float32) if f16 else x)
    print(f"  native k={k} n={n} pattern={pattern} f16={f16} nmse={e:.3g}", flush=True)


def test_zero_input_gives_zero(gpu, oracle):
    case = NativeCase(oracle, 544, 384)
    y, _ = case.run(kl.NativeQ4Workspace(), oracle.fixture_input(544, 1, 2), 1)
    assert np.array_equal(y, np.zeros_like(y))


@pytest.mark.parametrize("k,n,batch", [(256, 65, 4), (32, 1, 1), (64, 33, 2), (4096, 512, 5), (544, 384, 8),
                                       (16384, 128, 3), (1024, 4096, 16), (160, 97, 7)])
def test_batches_and_tails(gpu, oracle, k, n, batch):
    """Batches (the reference's exact route) and N tails: columns run in
    launches of up to four."""
    case = NativeCase(oracle, k, n)
    ws = kl.NativeQ4Workspace()
    x = oracle.fixture_input(k, batch, 0)
    y, flag = case.run(ws, x, batch)
    assert flag == (batch == 1 and n % 128 == 0)
    check(oracle, case, y, x)


def test_repeat_is_bitwise_stable(gpu, oracle):
    case = NativeCase(oracle, 4096, 11008)
    ws = kl.NativeQ4Workspace()
    x = oracle.fixture_input(4096, 1, 1)
    y0, _ = case.run(ws, x, 1)
    for _ in range(3):
        y1, _ = case.run(ws, x, 1)
        assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))


def test_same_values_as_row_major_q4_matmul(gpu, oracle):
    """The native layout and the 18-byte Q4_0 rows of the same matrix give
    results within F32 summation-order differences of each other."""
    k, n = 4096, 4096
    case = NativeCase(oracle, k, n)
    x = oracle.fixture_input(k, 1, 0)
    y_native, _ = case.run(kl.NativeQ4Workspace(), x, 1)
    from gpu_util import run_matmul
    y_q4, route, guard_ok = run_matmul(kl.WeightType.q4_0, case.q4, x, k, n, 1)
    assert guard_ok
    scale = np.abs(case.w).astype(np.float64) @ np.abs(x[0]).astype(np.float64)
    assert np.all(np.abs(y_native[0].astype(np.float64) - y_q4[0]) <= 1e-5 * scale + 1e-30), route


def test_mixed_with_rowwise_i8(gpu, oracle):
    """reference bench/native-q4-mixed-bench.cpp: native calls interleaved with
    rowwise_i8 matmuls on one device keep their results."""
    from gpu_util import run_matmul
    for n in (5504, 11008):
        k = 4096
        case = NativeCase(oracle, k, n)
        ws = kl.NativeQ4Workspace()
        x = oracle.fixture_input(k, 1, 3)
        gold = oracle.gold(case.w, x)
        for step in range(4):
            if step % 2:
                y, _, guard_ok = run_matmul(kl.WeightType.rowwise_i8, None, x, k, n, 1, w_f32=case.w)
                assert guard_ok and nmse(gold, y) < 1e-2
            else:
                y, flag = case.run(ws, x, 1)
                assert flag
                check(oracle, case, y, x)


def test_nonfinite_input_poisons_its_column(gpu, oracle):
    k, n, batch = 256, 128, 2
    case = NativeCase(oracle, k, n)
    x = oracle.fixture_input(k, batch, 0)
    x[1, 77] = np.inf
    y, _ = case.run(kl.NativeQ4Workspace(), x, batch)
    assert np.all(np.isnan(y[1]))
    check(oracle, case, y[:1], x[:1])


def test_workspace_binds_to_its_device(gpu, oracle):
    case = NativeCase(oracle, 64, 128)
    ws = kl.NativeQ4Workspace()
    x = oracle.fixture_input(64, 1, 0)
    case.run(ws, x, 1)
    y, flag = case.run(ws, x, 1)
    assert flag
    check(oracle, case, y, x)
