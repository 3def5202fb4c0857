"""GPU parity of the common Q4 ABI v1 (reference src/q4-common.inc,
src/q4-activation.inc, src/q4-pair.inc; tests bench/common-q4-bench.cpp,
common-q4-state-bench.cpp, common-q4-contract.cpp, gate-up-pair-api.cpp).

* upload: the device bytes equal the oracle's pack of the same Q4_0 rows.
* quantized activations: the workspace view (values, scales) equals the
  oracle's bit for bit (M = 1 two-component codes and parameters; M > 1 the
  last chunk's row codes and scales).
* outputs: against the FP64 product of the decoded weights with the
  represented activations (code * scale), the reference bench's gate
  implementation NMSE <= 1e-10 (common-q4-bench.cpp:65), and every element
  within 1e-5 * sum_j |w_cj qa_j| (F32 summation of exact block sums); the
  exact route (Np * Kp > 2^27) against the FP64 product with X itself.
* state: repeated calls of mixed M on one workspace give bitwise the results
  of fresh workspaces, with no new device memory after the first round.
* leases, the gate/up pair and the argument rules as the reference's tests.
"""
import os
import signal
import subprocess
import sys

import numpy as np
import pytest

import kunlunk200_lib_amd as kl

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
POISON = np.float32(-1234567.0)
F32, F16 = kl.InputType.f32, kl.InputType.f16


def raw_q4(oracle, k, n):
    """The reference bench's xorshift weights for ceil(k/32) blocks per row."""
    blocks = -(-k // 32)
    return oracle.fixture_q4(blocks * 32, n)


class Case:
    def __init__(self, oracle, k, n, storage=None):
        self.k, self.n = k, n
        self.raw = raw_q4(oracle, k, n)
        self.w = oracle.q4_decode(self.raw, -(-k // 32) * 32, n)[:, :k]
        self.weight = kl.CommonQ4Weight(0, k, n) if storage is None else kl.CommonQ4Weight(0, k, n, storage,
                                                                                         storage.size)
        self.weight.upload(self.raw)

    def run(self, ws, x, m, type_=F32):
        """common_q4_matmul into a poisoned buffer; returns Y [m, n]."""
        xin = x.astype(np.float16) if type_ == F16 else x.astype(np.float32)
        xb = kl.Buffer(0, xin.nbytes)
        xb.upload(xin)
        yb = kl.Buffer(0, (m * self.n + 128) * 4)
        yb.upload(np.full(m * self.n + 128, POISON, np.float32))
        with kl.runtime_mutex():
            kl.common_q4_matmul(ws, 0, yb.data + 256, self.weight, xb.data, m, type_)
        out = yb.download(m * self.n + 128, np.float32)
        assert np.all(out[:64] == POISON) and np.all(out[64 + m * self.n:] == POISON), "wrote outside Y"
        return out[64:64 + m * self.n].reshape(m, self.n)


def check_against(oracle, y, w, qa, label=""):
    """NMSE against the FP64 product with the represented activations, and an
    elementwise bound of F32 summation."""
    gold = oracle.gold(w, qa)
    e = y.astype(np.float64) - gold
    nmse = float((e * e).sum() / max(float((gold * gold).sum()), 1e-30))
    scale = np.abs(qa).astype(np.float64) @ np.abs(w).astype(np.float64).T
    assert np.all(np.isfinite(y))
    assert nmse <= 1e-10, (label, nmse)
    assert np.all(np.abs(e) <= 1e-5 * scale + 1e-30), label
    return nmse


def represented_pair(values, params, k, kp):
    j = np.arange(k)
    i = (j // 32) * 64 + j % 32
    return (values[i].astype(np.float32) * params[0] + values[2 * kp + i].astype(np.float32) * params[1])[None, :]


def view_bytes(ws, nbytes, dtype, which):
    q = ws.quantization()
    assert q[which]
    b = np.empty(nbytes // np.dtype(dtype).itemsize, dtype)
    with kl.runtime_mutex():
        kl.select(0)
        kl.check(kl.copy(b.ctypes.data, q[which], nbytes, kl.CopyKind.device_to_host))
        kl.check(kl.wait())
    return b


def test_upload_bytes_info_and_borrowed_storage(gpu, oracle):
    for k, n in ((4096, 300), (33, 33), (544, 513)):
        case = Case(oracle, k, n)
        info = case.weight.info()
        kp, np_ = oracle.common_dims(k, n)
        assert (info["abi_version"], info["quant_type"], info["layout"], info["scale_order"]) == (1, 2, 1, 1)
        assert (info["k"], info["n"], info["kp"], info["np"], info["device"]) == (k, n, kp, np_, 0)
        assert info["scale_offset"] == np_ * kp // 2 and info["payload_bytes"] == kl.common_q4_size(k, n)
        got = np.empty(info["payload_bytes"], np.uint8)
        with kl.runtime_mutex():
            kl.select(0)
            kl.check(kl.copy(got.ctypes.data, case.weight.data(), got.size, kl.CopyKind.device_to_host))
            kl.check(kl.wait())
        assert np.array_equal(got, oracle.common_q4_pack(case.raw, k, n))
        st = case.weight.statistics()
        assert st["uploads"] == 1 and st["upload_bytes"] == info["payload_bytes"]
    storage = kl.Buffer(0, kl.common_q4_size(512, 512) + 256)
    borrowed = Case(oracle, 512, 512, storage=storage)
    assert borrowed.weight.data() == storage.data


@pytest.mark.parametrize("k,n", [(4096, 11008), (4096, 4096), (11008, 4096), (544, 513), (33, 33), (16383, 65)])
@pytest.mark.parametrize("pattern", [0, 1, 3, 4])
def test_gemv_two_component(gpu, oracle, k, n, pattern):
    case = Case(oracle, k, n)
    ws = kl.CommonQ4Workspace()
    x = oracle.fixture_input(k, 1, pattern)
    y = case.run(ws, x, 1)
    kp, _ = oracle.common_dims(k, n)
    values, params = oracle.common_quant_pair(x, k)
    assert np.array_equal(view_bytes(ws, 4 * kp + 1024, np.int8, "values"), values)
    assert np.array_equal(view_bytes(ws, 64, np.float32, "scales").view(np.uint32), params.view(np.uint32))
    q = ws.quantization()
    assert (q["rows"], q["kp"], q["components"]) == (1, kp, 2)
    nmse = check_against(oracle, y, case.w, represented_pair(values, params, k, kp), f"{k}x{n} p{pattern}")
    s = ws.statistics()
    assert s["paths"][0] == 1 and s["calls"] == 1 and s["chunks"] == 1 and s["l3_workspace_bytes"] == 0
    print(f"  common gemv k={k} n={n} pattern={pattern} impl_nmse={nmse:.3g}", flush=True)


def test_gemv_f16_input(gpu, oracle):
    k, n = 4096, 512
    case = Case(oracle, k, n)
    ws = kl.CommonQ4Workspace()
    x = oracle.fixture_input(k, 1, 0)
    y = case.run(ws, x, 1, F16)
    xh = x.astype(np.float16).astype(np.float32)
    values, params = oracle.common_quant_pair(xh, k)
    assert np.array_equal(view_bytes(ws, 4 * k + 1024, np.int8, "values"), values)
    check_against(oracle, y, case.w, represented_pair(values, params, k, k))


def test_exact_route_for_large_layouts(gpu, oracle):
    """Np * Kp > 2^27: the reference's exact route (components 0, paths[7])."""
    k, n = 16384, 8448
    case = Case(oracle, k, n)
    ws = kl.CommonQ4Workspace()
    x = oracle.fixture_input(k, 1, 1)
    y = case.run(ws, x, 1)
    assert ws.quantization()["components"] == 0 and ws.statistics()["paths"][7] == 1
    check_against(oracle, y, case.w, x)


@pytest.mark.parametrize("m", [2, 8, 9, 32, 33, 64, 128, 129, 256])
@pytest.mark.parametrize("k,n", [(4096, 512), (544, 513), (11008, 256)])
def test_gemm_row_a8(gpu, oracle, k, n, m):
    case = Case(oracle, k, n)
    ws = kl.CommonQ4Workspace()
    x = oracle.fixture_input(k, m, 3)
    y = case.run(ws, x, m)
    kp, _ = oracle.common_dims(k, n)
    qa = np.empty((m, k), np.float32)
    for first in range(0, m, 128):
        rows = min(128, m - first)
        padded = 8 if rows <= 8 else 32 if rows <= 32 else 64 if rows <= 64 else 128
        values, params = oracle.common_quant_rows(x[first:first + rows], k, rows, padded)
        codes = values.reshape(padded, kp)[:rows, :k]
        qa[first:first + rows] = codes.astype(np.float32) * params.reshape(padded, 16)[:rows, :1]
    # the view holds the last chunk
    q = ws.quantization()
    assert q["components"] == 1 and q["rows"] == rows and q["kp"] == kp
    defined = -(-padded // 32) * 32
    vals = view_bytes(ws, defined * kp, np.int8, "values")
    sc = view_bytes(ws, defined * 64, np.float32, "scales")
    ref_values, ref_params = oracle.common_quant_rows(x[first:first + rows], k, rows, defined)
    assert np.array_equal(vals, ref_values) and np.array_equal(sc.view(np.uint32), ref_params.view(np.uint32))
    check_against(oracle, y, case.w, qa, f"m={m}")
    paths = ws.statistics()["paths"]
    assert sum(paths[1:7]) == -(-m // 128) and paths[0] == 0


def test_state_bench_mixed_m(gpu, oracle):
    """reference bench/common-q4-state-bench.cpp: one weight, mixed M on one
    workspace, bitwise equal to fresh workspaces, stable device memory."""
    k, n = 544, 513
    case = Case(oracle, k, n)
    ms = [1, 8, 32, 64, 128, 129, 256]
    for f16 in (False, True):
        type_ = F16 if f16 else F32
        x = oracle.fixture_input(k, 256, 0)
        gold = {m: case.run(kl.CommonQ4Workspace(), x[:m], m, type_) for m in ms}
        ws = kl.CommonQ4Workspace()
        plateau = None
        for rnd in range(3):
            for m in ms + [1]:
                y = case.run(ws, x[:m], m, type_)
                assert np.array_equal(y.view(np.uint32), gold[m].view(np.uint32))
            if rnd == 0:
                plateau = kl.allocated_bytes(0)
            else:
                assert kl.allocated_bytes(0) == plateau
        assert ws.statistics()["calls"] == 3 * (len(ms) + 1)
        assert case.weight.statistics()["uploads"] == 1


def test_lease_prepare_and_shared(gpu, oracle):
    k, n = 4096, 512
    case = Case(oracle, k, n)
    other = Case(oracle, k, 1024)
    for m in (1, 40, 200):
        ws = kl.CommonQ4Workspace()
        lease = kl.CommonQ4ActivationLease()
        x = oracle.fixture_input(k, m, 1)
        xb = kl.Buffer(0, x.nbytes)
        xb.upload(x)
        direct = case.run(kl.CommonQ4Workspace(), x, m)
        with kl.runtime_mutex():
            assert not kl.common_q4_prepare(ws, 0, xb.data, k, m, F32, 0, lease)          # generation 0
            assert not kl.common_q4_prepare(ws, 0, xb.data + 2, k, m, F32, 5, lease)      # misaligned
            assert kl.common_q4_prepare(ws, 0, xb.data, k, m, F32, 7, lease)
            assert lease.matches(0, k, m, F32, 7) and not lease.matches(0, k, m, F32, 8)
            assert lease.chunks() == -(-m // 128)
            c0 = lease.chunk(0)
            assert c0["first"] == 0 and c0["components"] == (2 if m == 1 else 1) and c0["kp"] == k
            for weight, dims, expect in ((case, (m, n), direct), (other, (m, 1024), None)):
                yb = kl.Buffer(0, dims[0] * dims[1] * 4)
                assert kl.common_q4_matmul_shared(ws, 0, yb.data, weight.weight, lease, 7)
                got = yb.download(dims[0] * dims[1], np.float32).reshape(dims)
                if expect is not None:
                    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))
            yb = kl.Buffer(0, m * n * 4)
            assert not kl.common_q4_matmul_shared(ws, 0, yb.data, case.weight, lease, 8)   # wrong generation
            assert not kl.common_q4_matmul_shared(ws, 0, xb.data, case.weight, lease, 7)   # Y overlaps X
        ast = ws.activation_statistics()
        assert ast["prepare_calls"] == 1 and ast["prepared_matmuls"] == 2 and ast["rejected_calls"] == 4
        # an ordinary call retires the lease
        case.run(ws, x[:1], 1)
        assert not lease.matches(0, k, m, F32, 7) and lease.chunks() == 0
        with kl.runtime_mutex():
            assert not kl.common_q4_matmul_shared(ws, 0, yb.data, case.weight, lease, 7)
        assert ws.activation_statistics()["invalidations"] >= 1


def test_gate_up_pair(gpu, oracle):
    """reference src/q4-pair.inc:9-80 (bench/gate-up-pair-api.cpp): one F32
    M = 1 lease, two weights, results bitwise equal to the shared calls."""
    k, n = 4096, 11008
    gate, up = Case(oracle, k, n), Case(oracle, k, n)
    up.weight.upload(oracle.fixture_q4(k, n)[::-1].copy())           # a different matrix
    ws = kl.CommonQ4Workspace()
    lease = kl.CommonQ4ActivationLease()
    x = oracle.fixture_input(k, 1, 0)
    xb = kl.Buffer(0, x.nbytes)
    xb.upload(x)
    y0, y1, ya, yb_ = (kl.Buffer(0, n * 4) for _ in range(4))
    with kl.runtime_mutex():
        assert kl.common_q4_prepare(ws, 0, xb.data, k, 1, F32, 3, lease)
        assert kl.common_q4_matmul_pair(ws, 0, y0.data, y1.data, gate.weight, up.weight, lease, 3)
        assert kl.common_q4_pair_last_status(ws) == kl.CommonQ4PairStatus.Success
        assert kl.common_q4_matmul_shared(ws, 0, ya.data, gate.weight, lease, 3)
        assert kl.common_q4_matmul_shared(ws, 0, yb_.data, up.weight, lease, 3)
        assert not kl.common_q4_matmul_pair(ws, 0, y0.data + 4, y1.data, gate.weight, up.weight, lease, 3)
        assert kl.common_q4_pair_last_status(ws) == kl.CommonQ4PairStatus.Alias
        assert not kl.common_q4_matmul_pair(ws, 0, y0.data, y1.data, gate.weight, up.weight, lease, 4)
        assert kl.common_q4_pair_last_status(ws) == kl.CommonQ4PairStatus.Lease
    for a, b in ((y0, ya), (y1, yb_)):
        assert np.array_equal(a.download(n, np.uint32), b.download(n, np.uint32))
    ps = kl.common_q4_pair_statistics(ws)
    assert ps["calls"] == 1 and ps["declined"] == 2
    small = Case(oracle, 512, 512)
    with kl.runtime_mutex():
        assert not kl.common_q4_matmul_pair(ws, 0, y0.data, y1.data, small.weight, small.weight, lease, 3)
    assert kl.common_q4_pair_last_status(ws) == kl.CommonQ4PairStatus.InvalidInput
    values, params = oracle.common_quant_pair(x, k)
    check_against(oracle, y0.download(n, np.float32)[None, :], gate.w, represented_pair(values, params, k, k))


# reference bench/common-q4-contract.cpp: each case aborts before any launch.
CONTRACT = ["device", "borrow-alignment", "borrow-capacity", "unready", "old-native-borrow", "m-zero", "type",
            "input-alignment", "output-alignment", "overlap"]


@pytest.mark.parametrize("case", CONTRACT)
def test_contract_aborts(gpu, case):
    code = f"""
import numpy as np, kunlunk200_lib_amd as kl
test = {case!r}
k = n = 512
if test == "device":
    kl.CommonQ4Weight(kl.device_count(), k, n)
x, y = kl.Buffer(0, k * 4 + 256), kl.Buffer(0, n * 4 + 256)
storage = kl.Buffer(0, kl.common_q4_size(k, n) + 256)
if test == "borrow-alignment":
    kl.CommonQ4Weight(0, k, n, storage.data + 4, storage.size - 4)
if test == "borrow-capacity":
    kl.CommonQ4Weight(0, k, n, storage.data, kl.common_q4_size(k, n) - 1)
raw = np.full((k * n // 32, 18), 0x12, np.uint8)
raw[:, 0] = 0
raw[:, 1] = 0x3c
if test == "old-native-borrow":
    kl.upload_native_q4(0, storage.data, raw, k, n)
weight = kl.CommonQ4Weight(0, k, n, storage.data, storage.size)
if test not in ("unready", "old-native-borrow"):
    weight.upload(raw)
work = kl.CommonQ4Workspace()
m = 0 if test == "m-zero" else 1
type_ = 99 if test == "type" else 0
inp = x.data + 1 if test == "input-alignment" else x.data
out = y.data + 2 if test == "output-alignment" else x.data if test == "overlap" else y.data
print("EXPECTED_CONTRACT_REJECTION", test, flush=True)
kl.common_q4_matmul(work, 0, out, weight, inp, m, type_)
print("NOT REJECTED", flush=True)
"""
    env = dict(os.environ, PYTHONPATH=ROOT)
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert "NOT REJECTED" not in proc.stdout
    assert proc.returncode == -signal.SIGABRT, (proc.returncode, proc.stderr[-400:])
    assert "invalid argument" in proc.stderr
