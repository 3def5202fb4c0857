"""kunlun_matmul_noalloc (no reference counterpart: the entry point for callers
that cannot allocate device memory) against kunlun_matmul, the entry point it
is a variant of. Both take the same routes and kernels, the no-alloc one with
its scratch in a fixed per-GPU device array, so Y must be bit-identical. Each
case makes two calls in a row, the second with a smaller input (the array
keeps the first call's contents), and checks both. Calls past the array's
size and unsupported types return their status without launching."""
import numpy as np
import pytest

import kunlunk200_lib_amd as kl
from gpu_util import GUARD, run_matmul, weight_payload

pytestmark = pytest.mark.gpu

Q4, F16, F32 = kl.WeightType.q4_0, kl.WeightType.f16, kl.WeightType.f32

# (type, route, first (k, n, batch), second, smaller (k, n, batch))
CASES = [
    (Q4, "q4_gemm_mfma", (4096, 1024, 128), (2048, 520, 64)),     # LDS GEMM, scratch: fp16 X + row scales
    (Q4, "q4_gemm_mfma", (1088, 384, 96), (544, 130, 64)),        # register-staged GEMM (K % 256 != 0)
    (F16, "f16_gemm_mfma", (1024, 256, 96), (512, 130, 64)),      # F16 GEMM
    (Q4, "q4_stream_gemv", (4096, 2048, 8), (4096, 300, 5)),      # streamed MFMA GEMV (K = 4096), no scratch
    (Q4, "q4_bdiag_gemv", (1024, 2048, 8), (1024, 300, 4)),       # block-diagonal MFMA GEMV, no scratch
    (Q4, "q4_mfma_gemv", (4096, 2048, 16), (4096, 300, 12)),      # LDS-staged MFMA GEMV, scratch: X fragments
    (Q4, "q4_mfma_gemv", (4096, 520, 40), (4096, 300, 33)),       # chunks of 16 columns, the array reused in order
    (Q4, "q4_gemv_dot8", (4096, 1024, 1), (1024, 129, 1)),        # no scratch
    (F32, "f32_mfma_gemv", (1024, 256, 8), (512, 65, 2)),         # no scratch
]


def noalloc_run(type_, payload, x, k, n, batch):
    """One kunlun_matmul_noalloc call on the library's stream; (y, route, guard_ok)."""
    x = np.ascontiguousarray(x, np.float32).reshape(batch, k)
    w_bytes = np.ascontiguousarray(payload).view(np.uint8).ravel()
    guard = 64
    with kl.Buffer(0, w_bytes.nbytes) as wb, kl.Buffer(0, x.nbytes) as xb, \
            kl.Buffer(0, (batch * n + guard) * 4) as yb:
        wb.upload(w_bytes)
        xb.upload(x)
        yb.upload(np.full(batch * n + guard, GUARD, np.float32))
        with kl.runtime_mutex():
            kl.select(0)
            rc, route = kl.matmul_noalloc(0, yb.data, wb.data, xb.data, k, n, batch, type_, kl.stream(0))
            assert rc == 0, f"kunlun_matmul_noalloc returned {rc}"
            kl.check(kl.wait())
        out = yb.download(batch * n + guard, np.float32)
    guard_ok = bool(np.all(out[batch * n:].view(np.uint32) == np.full(guard, GUARD).view(np.uint32)))
    return out[:batch * n].reshape(batch, n), route, guard_ok


@pytest.mark.parametrize("type_,route,first,second", CASES, ids=[f"{c[1]}-k{c[2][0]}" for c in CASES])
def test_noalloc_matches_matmul(gpu, oracle, type_, route, first, second):
    for i, (k, n, batch) in enumerate((first, second)):
        rng = np.random.default_rng(k + n + batch + i)
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        x = rng.standard_normal((batch, k)).astype(np.float32)
        payload, _ = weight_payload(type_, w, oracle)
        y_ref, r_ref, g_ref = run_matmul(type_, payload, x, k, n, batch)
        y, r, g = noalloc_run(type_, payload, x, k, n, batch)
        print(f"  noalloc {r} k={k} n={n} b={batch} (call {i + 1})", flush=True)
        assert r == r_ref == route
        assert g and g_ref, "wrote past the output"
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), \
            f"call {i + 1}: max |diff| {np.max(np.abs(y - y_ref)):.3g}"


def test_noalloc_rejects_beyond_scratch(gpu):
    # the GEMM's fp16 activations alone (2 * batch * K bytes) exceed the array
    k, n, batch = 4096, 32, 4096
    assert 2 * batch * k > kl.NOALLOC_SCRATCH_BYTES
    q4 = np.zeros((n, k // 32 * 18), np.uint8)
    with kl.Buffer(0, q4.nbytes) as wb, kl.Buffer(0, batch * k * 4) as xb, kl.Buffer(0, batch * n * 4) as yb:
        wb.upload(q4)
        yb.upload(np.full(batch * n, GUARD, np.float32))
        with kl.runtime_mutex():
            kl.select(0)
            rc, route = kl.matmul_noalloc(0, yb.data, wb.data, xb.data, k, n, batch, Q4, kl.stream(0))
            kl.check(kl.wait())
        assert rc == kl.NOALLOC_TOO_LARGE and route is None
        assert np.all(yb.download(batch * n, np.float32).view(np.uint32) == np.uint32(GUARD.view(np.uint32)))
        # rowwise INT8 and unknown types are not taken; K % 32 != 0 is rejected as kunlun_matmul does
        with kl.runtime_mutex():
            assert kl.matmul_noalloc(0, yb.data, wb.data, xb.data, k, n, 1, kl.WeightType.rowwise_i8)[0] == \
                kl.NOALLOC_INVALID
            assert kl.matmul_noalloc(0, yb.data, wb.data, xb.data, k + 16, n, 1, Q4)[0] == kl.NOALLOC_INVALID


# Two host threads whose first no-alloc calls overlap, each on its own HIP
# stream, in a fresh process (so the per-device set-up and every launcher's
# one-time LDS opt-in happen under the race), on the routes that use no
# scratch (calls overlapping on one GPU may share only those). Each thread's
# results must equal the same calls made one at a time.
_TWO_THREADS = r"""
import ctypes, sys, threading
import numpy as np
sys.path.insert(0, sys.argv[1])
import kunlunk200_lib_amd as kl
hip = ctypes.CDLL("libamdhip64.so")
hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
Q4, F32 = kl.WeightType.q4_0, kl.WeightType.f32
# scratch-free routes: batch-1 dot8, block-diagonal, F32 MFMA, streamed Q4_0, F32 MFMA (small)
CASES = [(Q4, 4096, 3000, 1), (Q4, 1024, 2048, 4), (F32, 1024, 256, 8), (Q4, 4096, 1000, 8), (F32, 512, 65, 2)]
rng = np.random.default_rng(7)
jobs = []
for type_, k, n, batch in CASES:
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    payload = kl.quantize_q4_0(w) if type_ == Q4 else w
    x = rng.standard_normal((batch, k)).astype(np.float32)
    wb, xb = kl.Buffer(0, payload.nbytes), kl.Buffer(0, x.nbytes)
    wb.upload(payload)
    xb.upload(x)
    jobs.append((type_, k, n, batch, wb, xb))
outs = [[kl.Buffer(0, batch * n * 4) for (_, k, n, batch, _, _) in jobs] for _ in range(3)]
kl.select(0)
streams = []
for _ in range(2):
    s = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(s)) == 0
    streams.append(s)
status = [[None] * len(jobs) for _ in range(3)]
start = threading.Barrier(2)

def worker(t):
    kl.select(0)
    order = range(len(jobs)) if t == 0 else reversed(range(len(jobs)))
    start.wait()
    for i in order:
        type_, k, n, batch, wb, xb = jobs[i]
        status[t][i] = kl.matmul_noalloc(0, outs[t][i].data, wb.data, xb.data, k, n, batch, type_, streams[t].value)
    assert hip.hipStreamSynchronize(streams[t]) == 0

threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
for t in threads:
    t.start()
for t in threads:
    t.join()
# the same calls one at a time on the library's stream
for i, (type_, k, n, batch, wb, xb) in enumerate(jobs):
    status[2][i] = kl.matmul_noalloc(0, outs[2][i].data, wb.data, xb.data, k, n, batch, type_, kl.stream(0))
    kl.check(kl.wait())
    ys = [outs[t][i].download(batch * n, np.float32) for t in range(3)]
    assert status[0][i] == status[1][i] == status[2][i] and status[2][i][0] == 0, [status[t][i] for t in range(3)]
    for t in range(2):
        assert np.array_equal(ys[t].view(np.uint32), ys[2].view(np.uint32)), (status[2][i], "thread", t)
    print("two-thread noalloc", status[2][i][1], k, n, batch, "equal", flush=True)
for s in streams:
    hip.hipStreamDestroy(s)
print("TWO_THREADS_OK", flush=True)
"""


def test_noalloc_two_threads_first_calls(gpu):
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    proc = subprocess.run([sys.executable, "-c", _TWO_THREADS, root], capture_output=True, text=True, timeout=100)
    print(proc.stdout, flush=True)
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-3000:]
    assert "TWO_THREADS_OK" in proc.stdout
