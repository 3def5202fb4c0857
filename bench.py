#!/usr/bin/env python3
"""Q4_0 GEMV bandwidth benchmark of the KunlunK200 matmul path on one MI355X.

Workload (the metric's own shape, the gate GEMV of BASELINE.json configs[1]):
one step = one kunlun::matmul() of Q4_0 K4096 x N11008 at batch 1, weights
from N(0, 0.02) quantized with the ggml closed form, F32 activations N(0, 1).
Distinct device copies of the matrix (>= 640 MB in all) rotate so the 256 MB
Infinity Cache cannot hold the weights. value = algorithmic bytes of a step /
step time, bytes per GEMV = n*(k/32)*18 + 4*b*k + 4*b*n. Timing uses HIP events
recorded on the library's own stream around K steps (after 200 ms of untimed
steps and W warm-up steps).

Beside it, on the same rotating copies:
  layer_set     the whole decode layer set of configs[1] (K4096->N12288 QKV,
                K4096->N11008 x2 gate/up, K11008->N4096 down, K4096->N32000
                LM head), five matmul() calls per step, and each shape alone
                in per_shape, with configs[0] (K4096 x N4096) beside them.
  read_ceiling  read-only streaming kernels (libkunlunk200_stream.so) reading
                25.4 MB, 73.9 MB and 268 MB once per launch over rotating
                buffers of >= 640 MB: the measured HBM read ceiling at the
                GEMVs' sizes. roofline reports the GEMV's fraction of the spec
                peak and of this ceiling.
  cpu_baseline  the reference's CPU path on the K4096 x N11008 GEMV (decoded
                F32 weights, FP64 sums) at 1 thread (the oracle's restatement of
                bench/library-bench.cpp:121-122), 6 threads (the reference's own
                bench/native-q4-reference.h:98-108, compiled under oracle/_ref)
                and nproc threads (the restatement), each repeated for about
                --cpu-seconds, with the host CPU model.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import kunlunk200_lib_amd as kl  # noqa: E402

METRIC = "Q4_0 GEMV GB/s (% HBM peak) K4096×N11008 batch1; GEMM TFLOP/s at batch512"
HBM_PEAK_GBPS = 8000.0
LAYER = [("qkv", 4096, 12288), ("gate", 4096, 11008), ("up", 4096, 11008), ("down", 11008, 4096),
         ("lm_head", 4096, 32000)]
CONFIG0 = ("cfg0", 4096, 4096)          # configs[0]: k200-bench matmul q4_0 0 4096 4096 1
SHAPES = LAYER + [CONFIG0]
DOMINANT = ("gate", 4096, 11008)
COPIES = 3
ROTATE_BYTES = 640 * 1000 * 1000     # > 2x the 256 MB Infinity Cache
SPREAD_LOOPS, SPREAD_LAUNCHES = 10, 30  # per-shape spread: loops of launches (median, min, max)
SETTLE_MS = 200                         # untimed layer-set steps before the warm-up steps


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def q4_bytes(k: int, n: int, b: int = 1) -> int:
    return n * (k // 32) * 18 + 4 * b * k + 4 * b * n


class HipEvents:
    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self):
        ev = ctypes.c_void_p()
        assert self.lib.hipEventCreate(ctypes.byref(ev)) == 0
        return ev

    def record(self, ev, stream):
        assert self.lib.hipEventRecord(ev, ctypes.c_void_p(stream)) == 0

    def elapsed_ms(self, start, stop) -> float:
        assert self.lib.hipEventSynchronize(stop) == 0
        ms = ctypes.c_float()
        assert self.lib.hipEventElapsedTime(ctypes.byref(ms), start, stop) == 0
        return float(ms.value)


def upload_q4_matrix(buf: kl.Buffer, k: int, n: int, seed: int) -> None:
    rng = np.random.Generator(np.random.PCG64(seed))
    row_bytes = k // 32 * 18
    chunk = 2048
    for r0 in range(0, n, chunk):
        rows = min(chunk, n - r0)
        w = (rng.standard_normal((rows, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
        buf.upload(kl.quantize_q4_0(w), offset=r0 * row_bytes)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_threads() -> int:
    """CPUs this process may run on (the box's share, not the machine's count)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline(seconds: float) -> dict | None:
    """The reference CPU path on the dominant GEMV at 1, 6 and nproc threads; the 6-thread
    figure (the reference's own setting) is the headline `value`."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import _oracle
    _, k, n = DOMINANT
    rng = np.random.Generator(np.random.PCG64(99))
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    orc = _oracle.Oracle()
    dec = orc.q4_decode(kl.quantize_q4_0(w), k, n)
    x = rng.standard_normal((1, k), dtype=np.float32)
    ref = _oracle.ReferenceOracle.load()
    nproc = host_threads()

    def timed_calls(run) -> tuple:
        run()
        reps, start = 0, time.perf_counter()
        while True:
            run()
            reps += 1
            elapsed = time.perf_counter() - start
            if elapsed >= seconds or reps >= 10000:
                return reps, elapsed

    runs = [(1, "port", "oracle orc_gold: FP64 restatement of bench/library-bench.cpp:121-122, 1 thread",
             lambda: orc.gold(dec, x, threads=1))]
    prepared = None
    if ref is not None:
        # the vectors are built once, and each timed call is reference() alone, as
        # the reference's bench/native-q4-bench.cpp:22-25 times it
        prepared = ref.prepared(dec, x)
        runs.append((6, "reference", "kref_run: the reference's bench/native-q4-reference.h:98-108 "
                     "compiled as is (FP64, 6 OpenMP threads) on vectors built once", prepared.run))
    else:
        runs.append((6, "port", "oracle orc_gold, 6 threads (oracle/_ref not built)",
                     lambda: orc.gold(dec, x, threads=6)))
    runs.append((nproc, "port", f"oracle orc_gold, {nproc} threads (this process's CPUs)",
                 lambda: orc.gold(dec, x, threads=nproc)))
    by_threads = []
    for threads, kind, what, run in runs:
        reps, elapsed = timed_calls(run)
        per_call = elapsed / reps
        by_threads.append({"threads": threads, "kind": kind, "what": what,
                           "gbps": round(q4_bytes(k, n) / per_call / 1e9, 4),
                           "ms_per_call": round(per_call * 1e3, 3), "calls": reps,
                           "seconds": round(elapsed, 2)})
        log(f"cpu baseline {threads} thread(s): {per_call * 1e3:.3f} ms/call")
    if prepared is not None:
        prepared.close()
    head = by_threads[1]
    return {"value": head["gbps"], "unit": "GB/s", "cores": head["threads"], "kind": head["kind"],
            "sample": f"{head['what']}; K{k}xN{n} batch 1, decoded Q4_0 weights, {head['calls']} calls in "
                      f"{head['seconds']} s ({head['ms_per_call']} ms/call); 1/6/nproc-thread runs in by_threads",
            "cpu_model": cpu_model(), "host_cpus": nproc, "by_threads": by_threads}


COPY_BYTES = 512 << 20
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "q4_gemv_dot8_k4096_n11008_traffic.md")


def copy_leg(events, stream, device: int, reps: int = 10) -> dict:
    """A plain device-to-device copy of COPY_BYTES: its FETCH_SIZE and WRITE_SIZE per dispatch
    calibrate the counters (the copy reads and writes exactly COPY_BYTES). Each copy completes
    before the next is submitted, so `us` includes the host round trip."""
    src, dst = kl.Buffer(device, COPY_BYTES), kl.Buffer(device, COPY_BYTES)
    with kl.runtime_mutex():
        kl.select(device)
        start, stop = events.create(), events.create()
        events.record(start, stream)
        for _ in range(reps):
            kl.check(kl.copy(dst.data, src.data, COPY_BYTES, kl.CopyKind.device_to_device))
        events.record(stop, stream)
        ms = events.elapsed_ms(start, stop) / reps
        kl.check(kl.wait())
    src.close()
    dst.close()
    return {"bytes": COPY_BYTES, "reps": reps, "us": round(ms * 1e3, 2)}


# the read leg at the size of every per-shape GEMV (down K11008 x N4096 has the
# gate's bytes), of the small-batch Q4_0 weights (configs[2], K4096 x N14336
# at batch 8) and of 256 MiB
READ_SIZES = (("gate_gemv", q4_bytes(4096, 11008)), ("qkv_gemv", q4_bytes(4096, 12288)),
              ("lm_head_gemv", q4_bytes(4096, 32000)), ("cfg0_gemv", q4_bytes(4096, 4096)),
              ("small_batch_q4", q4_bytes(4096, 14336, 8)), ("256mib", 256 << 20))
READ_OF_SHAPE = {"qkv": "qkv_gemv", "gate": "gate_gemv", "up": "gate_gemv", "down": "gate_gemv",
                 "lm_head": "lm_head_gemv", "cfg0": "cfg0_gemv"}
READ_WAVES = (2048, 4096, 8192)          # 8, 16 and 32 waves per CU
READ_VARIANTS = ((0, "grid_stride"), (1, "all_issued"), (2, "all_issued_nt"))


def read_ceiling_leg(events, stream, device: int, reps: int, sizes=None, variants=None, waves_list=None) -> dict:
    """Measured HBM read ceiling: kk_stream_read (kunlunk200_lib_amd/csrc/stream_read.hip) reads
    each size once per launch from a buffer slot that rotates over >= ROTATE_BYTES, for every
    variant and grid size that fits (at most 64 KiB per wave); `best` is the fastest. `sizes`,
    `variants` and `waves_list` restrict the runs (names, variant numbers, wave counts)."""
    lib = ctypes.CDLL(os.path.join(ROOT, "kunlunk200_lib_amd", "lib", "libkunlunk200_stream.so"))
    lib.kk_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_void_p, ctypes.c_void_p]
    lib.kk_stream_read.restype = ctypes.c_int
    out_word = kl.Buffer(device, 256)
    out = {}
    for name, size in READ_SIZES:
        if sizes and name not in sizes:
            continue
        size = size // 16 * 16
        slot = (size + 255) & ~255
        slots = max(2, -(-ROTATE_BYTES // slot))
        buf = kl.Buffer(device, slot * slots)
        buf.upload(np.zeros(1, np.uint32))
        runs = []
        for variant, vname in READ_VARIANTS:
            for waves in READ_WAVES:
                if variant > 0 and -(-size // waves) > 64 * 1024:
                    continue
                if (variants and variant not in variants) or (waves_list and waves not in waves_list):
                    continue

                def one(i, variant=variant, waves=waves):
                    rc = lib.kk_stream_read(ctypes.c_void_p(buf.data + (i % slots) * slot), size, variant, waves,
                                            ctypes.c_void_p(out_word.data), ctypes.c_void_p(stream))
                    if rc != 0:
                        raise RuntimeError(f"kk_stream_read({name}, variant {variant}, waves {waves}) -> {rc}")
                with kl.runtime_mutex():
                    kl.select(device)
                    for i in range(slots + 2):
                        one(i)
                    kl.check(kl.wait())
                    start, stop = events.create(), events.create()
                    events.record(start, stream)
                    for i in range(reps):
                        one(i)
                    events.record(stop, stream)
                    us = events.elapsed_ms(start, stop) / reps * 1e3
                    kl.check(kl.wait())
                runs.append({"variant": vname, "waves": waves, "us": round(us, 3),
                             "gbps": round(size / (us * 1e-6) / 1e9, 1)})
        buf.close()
        best = min(runs, key=lambda r: r["us"])
        out[name] = {"bytes": size, "rotating_slots": slots, "best": best, "runs": runs}
        log(f"read ceiling {name}: {best['us']} us, {best['gbps']} GB/s ({best['variant']}, {best['waves']} waves)")
    out_word.close()
    return out


def measured_traffic() -> int | None:
    """HBM bytes per launch of the dominant GEMV from the committed counter summary
    (line 'traffic_bytes_per_launch: N'), or None when it is absent."""
    try:
        with open(TRAFFIC_PROFILE, encoding="utf-8") as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except (OSError, ValueError):
        return None
    return None


GEMM_SHAPES = [("k4096_n4096", 4096, 4096), ("k4096_n11008", 4096, 11008)]
PAIR_N = 11008
MFMA_F16_PEAK_TFLOPS = 2500.0


def rotating_copies(device: int, first: kl.Buffer, nbytes: int, total: int = ROTATE_BYTES) -> list:
    """`first` and device copies of it, at least `total` bytes in all (at least 2 buffers), so a
    loop over them reads its weights from HBM rather than from the 256 MB Infinity Cache."""
    bufs = [first]
    for _ in range(max(2, -(-total // nbytes)) - 1):
        b = kl.Buffer(device, nbytes)
        with kl.runtime_mutex():
            kl.select(device)
            kl.check(kl.copy(b.data, first.data, nbytes, kl.CopyKind.device_to_device))
            kl.check(kl.wait())
        bufs.append(b)
    return bufs


def gemm_leg(kernel, events, stream, device: int, reps: int) -> dict:
    """Q4_0 prefill GEMM at batch 512: TFLOP/s = 2*b*k*n / time; the
    gate/up pair with SiLU * up counts 2 * 2*b*k*n per call. Weights rotate over >= 640 MB of
    device copies (the gate/up pair: pairs of copies), so each call reads them from HBM."""
    batch = 512
    out = {}
    rng = np.random.Generator(np.random.PCG64(11))

    def timed_calls(call) -> float:
        with kl.runtime_mutex():
            for i in range(3):
                call(i)
            kl.select(device)
            kl.check(kl.wait())
            start, stop = events.create(), events.create()
            events.record(start, stream)
            for i in range(reps):
                call(i)
            events.record(stop, stream)
            ms = events.elapsed_ms(start, stop) / reps
            kl.check(kl.wait())
        return ms

    for tag, k, n in GEMM_SHAPES:
        nbytes = n * (k // 32) * 18
        first = kl.Buffer(device, nbytes)
        upload_q4_matrix(first, k, n, seed=2000 + n)
        wbufs = rotating_copies(device, first, nbytes)
        xbuf = kl.Buffer(device, 4 * batch * k)
        xbuf.upload(rng.standard_normal((batch, k), dtype=np.float32))
        ybuf = kl.Buffer(device, 4 * batch * n)
        ms = timed_calls(lambda i: kl.matmul(kernel, device, ybuf.data, wbufs[i % len(wbufs)].data, xbuf.data,
                                             k, n, batch, kl.WeightType.q4_0))
        tflops = 2.0 * batch * k * n / (ms * 1e-3) / 1e12
        out[tag] = {"us": round(ms * 1e3, 2), "tflops": round(tflops, 1),
                    "mfma_f16_frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4), "route": kernel.route,
                    "rotating_copies": len(wbufs)}
        if n == PAIR_N:
            # gate/up pair sharing X, then SiLU(gate) * up, one call
            ufirst = kl.Buffer(device, nbytes)
            upload_q4_matrix(ufirst, k, n, seed=3000 + n)
            half = ROTATE_BYTES // 2
            gates = wbufs[:max(2, -(-half // nbytes))]
            ups = rotating_copies(device, ufirst, nbytes, half)
            pairs = list(zip(gates, ups))
            ms = timed_calls(lambda i: kl.matmul_swiglu(kernel, device, ybuf.data, pairs[i % len(pairs)][0].data,
                                                        pairs[i % len(pairs)][1].data, xbuf.data, k, n, batch,
                                                        kl.WeightType.q4_0))
            tflops = 4.0 * batch * k * n / (ms * 1e-3) / 1e12
            out[f"pair_swiglu_{tag}"] = {"us": round(ms * 1e3, 2), "tflops": round(tflops, 1),
                                         "mfma_f16_frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                                         "route": kernel.route, "rotating_copies": len(pairs)}
            for b in ups:
                b.close()
        for b in wbufs + [xbuf, ybuf]:
            b.close()
    return out


SMALL_BATCH_Q4 = (4096, 14336, (2, 4, 8, 16))
DECODE_PAIR_BATCHES = (1, 4, 8, 16, 32)                # matmul_swiglu at decode batch sizes
SMALL_DENSE = (4096, 4096, (1, 8))                   # F16 / F32 part of configs[2]
DECODE_PAIR = (4096, 11008)                          # gate/up pair of the decode layer (matmul_swiglu, batch 1)


def small_batch_leg(kernel, events, stream, device: int, reps: int) -> dict:
    """Q4_0 K4096 x N14336 at batch 2..16 and F16/F32 4096^2 at
    batch 1 and 8, each over rotating weight copies (>= 640 MB) so weights stream
    from HBM. GB/s = algorithmic bytes (weights + 4bk + 4bn) / launch time. Also
    the decode gate/up pair (matmul_swiglu, Q4_0 K4096 x 2 x N11008, batch 1, 4, 8 and 16)."""
    out = {}
    rng = np.random.Generator(np.random.PCG64(21))

    def run(tag, type_, k, n, batch, nbytes, fill):
        first = kl.Buffer(device, nbytes)
        fill(first)
        bufs = [first]
        for _ in range(max(2, -(-ROTATE_BYTES // nbytes)) - 1):
            b = kl.Buffer(device, nbytes)
            with kl.runtime_mutex():
                kl.select(device)
                kl.check(kl.copy(b.data, first.data, nbytes, kl.CopyKind.device_to_device))
                kl.check(kl.wait())
            bufs.append(b)
        xb = kl.Buffer(device, 4 * batch * k)
        xb.upload(rng.standard_normal((batch, k), dtype=np.float32))
        yb = kl.Buffer(device, 4 * batch * n)
        with kl.runtime_mutex():
            for i in range(5):
                kl.matmul(kernel, device, yb.data, bufs[i % len(bufs)].data, xb.data, k, n, batch, type_)
            kl.select(device)
            kl.check(kl.wait())
            start, stop = events.create(), events.create()
            events.record(start, stream)
            for i in range(reps):
                kl.matmul(kernel, device, yb.data, bufs[i % len(bufs)].data, xb.data, k, n, batch, type_)
            events.record(stop, stream)
            ms = events.elapsed_ms(start, stop) / reps
            kl.check(kl.wait())
        total = nbytes + 4 * batch * k + 4 * batch * n
        out[tag] = {"us": round(ms * 1e3, 3), "gbps": round(total / (ms * 1e-3) / 1e9, 1),
                    "hbm_frac": round(total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "route": kernel.route}
        for b in bufs + [xb, yb]:
            b.close()

    k, n, batches = SMALL_BATCH_Q4
    for batch in batches:
        run(f"q4_k{k}_n{n}_b{batch}", kl.WeightType.q4_0, k, n, batch, n * (k // 32) * 18,
            lambda b: upload_q4_matrix(b, k, n, seed=4000 + n))
    # decode gate/up pair with the SwiGLU epilogue: both matrices rotate
    k, n = DECODE_PAIR
    nbytes = n * (k // 32) * 18
    first_g, first_u = kl.Buffer(device, nbytes), kl.Buffer(device, nbytes)
    upload_q4_matrix(first_g, k, n, seed=5000)
    upload_q4_matrix(first_u, k, n, seed=5001)
    pairs = [(first_g, first_u)]
    for _ in range(max(2, -(-ROTATE_BYTES // (2 * nbytes))) - 1):
        g, u = kl.Buffer(device, nbytes), kl.Buffer(device, nbytes)
        with kl.runtime_mutex():
            kl.select(device)
            kl.check(kl.copy(g.data, first_g.data, nbytes, kl.CopyKind.device_to_device))
            kl.check(kl.copy(u.data, first_u.data, nbytes, kl.CopyKind.device_to_device))
            kl.check(kl.wait())
        pairs.append((g, u))
    for batch in DECODE_PAIR_BATCHES:
        xb = kl.Buffer(device, 4 * batch * k)
        xb.upload(rng.standard_normal((batch, k), dtype=np.float32))
        yb = kl.Buffer(device, 4 * batch * n)
        with kl.runtime_mutex():
            for i in range(5):
                g, u = pairs[i % len(pairs)]
                kl.matmul_swiglu(kernel, device, yb.data, g.data, u.data, xb.data, k, n, batch, kl.WeightType.q4_0)
            kl.select(device)
            kl.check(kl.wait())
            start, stop = events.create(), events.create()
            events.record(start, stream)
            for i in range(reps):
                g, u = pairs[i % len(pairs)]
                kl.matmul_swiglu(kernel, device, yb.data, g.data, u.data, xb.data, k, n, batch, kl.WeightType.q4_0)
            events.record(stop, stream)
            ms = events.elapsed_ms(start, stop) / reps
            kl.check(kl.wait())
        total = 2 * nbytes + 4 * batch * k + 4 * batch * n
        out[f"q4_pair_swiglu_k{k}_n{n}_b{batch}"] = {
            "us": round(ms * 1e3, 3), "gbps": round(total / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "route": kernel.route}
        xb.close()
        yb.close()
    for g, u in pairs:
        g.close()
        u.close()

    k, n, batches = SMALL_DENSE
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    for type_, name, arr in ((kl.WeightType.f16, "f16", w.astype(np.float16)), (kl.WeightType.f32, "f32", w)):
        for batch in batches:
            run(f"{name}_k{k}_n{n}_b{batch}", type_, k, n, batch, arr.nbytes, lambda b, arr=arr: b.upload(arr))
    return out


I8_CASES = ((1024, 512, 4), (4096, 4096, 1), (4096, 4096, 32), (4096, 4096, 512))
INT8_PEAK_TOPS = 5000.0


def i8_leg(kernel, events, stream, device: int, reps: int) -> dict:
    """rowwise_i8 weights (upload_i8_rows packing) at K1024 x N512
    batch 4 and K4096 x N4096 batch 1, 32, 512, over rotating copies of the packed
    weights. A call includes the on-GPU two-pass activation quantization. GB/s =
    (nk + 4n + 4bk + 4bn) / time; TOPS = 2bkn / time (int8 MFMA)."""
    out = {}
    rng = np.random.Generator(np.random.PCG64(31))
    for k, n, batch in I8_CASES:
        w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
        size = kl.packed_i8_size(k, n)
        first = kl.Buffer(device, size)
        kl.upload_i8_rows(device, first.data, k, n, 0, n, w)
        bufs = [first]
        for _ in range(max(2, -(-ROTATE_BYTES // size)) - 1):
            b = kl.Buffer(device, size)
            with kl.runtime_mutex():
                kl.select(device)
                kl.check(kl.copy(b.data, first.data, size, kl.CopyKind.device_to_device))
                kl.check(kl.wait())
            bufs.append(b)
        xb = kl.Buffer(device, 4 * batch * k)
        xb.upload(rng.standard_normal((batch, k), dtype=np.float32))
        yb = kl.Buffer(device, 4 * batch * n)

        def call(i):
            b = bufs[i % len(bufs)]
            kl.matmul(kernel, device, yb.data, b.data, xb.data, k, n, batch, kl.WeightType.rowwise_i8,
                      kl.packed_i8_scales(b.data, k, n), kl.packed_i8_maxima(b.data, k, n))
        with kl.runtime_mutex():
            for i in range(5):
                call(i)
            kl.select(device)
            kl.check(kl.wait())
            start, stop = events.create(), events.create()
            events.record(start, stream)
            for i in range(reps):
                call(i)
            events.record(stop, stream)
            ms = events.elapsed_ms(start, stop) / reps
            kl.check(kl.wait())
        nbytes = n * k + 4 * n + 4 * batch * k + 4 * batch * n
        tops = 2.0 * batch * k * n / (ms * 1e-3) / 1e12
        out[f"i8_k{k}_n{n}_b{batch}"] = {"us": round(ms * 1e3, 3), "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                         "tops": round(tops, 2), "int8_frac": round(tops / INT8_PEAK_TOPS, 4),
                                         "route": kernel.route}
        for b in bufs + [xb, yb]:
            b.close()
    return out


NATIVE_SHAPES = ((4096, 4096), (4096, 11008), (11008, 4096))   # reference docs/native-q4.md:62-71
NATIVE_REFERENCE_MS = {(4096, 4096): 0.338455, (4096, 11008): 0.712449, (11008, 4096): 0.843438}


def native_leg(events, stream, device: int, reps: int) -> dict:
    """native_q4_matmul at the reference's published shapes, batch 1, F32 X, over
    rotating weight copies. Each call completes before returning (as the
    reference's does), so `us` is the time per call including its
    synchronization; GB/s = layout bytes + 4k + 4n over that time."""
    out = {}
    rng = np.random.Generator(np.random.PCG64(33))
    ws = kl.NativeQ4Workspace()
    for k, n in NATIVE_SHAPES:
        nbytes = kl.native_q4_size(k, n)
        q4 = kl.quantize_q4_0(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
        first = kl.Buffer(device, nbytes)
        kl.upload_native_q4(device, first.data, q4, k, n)
        bufs = [first]
        for _ in range(max(2, -(-ROTATE_BYTES // nbytes)) - 1):
            b = kl.Buffer(device, nbytes)
            with kl.runtime_mutex():
                kl.select(device)
                kl.check(kl.copy(b.data, first.data, nbytes, kl.CopyKind.device_to_device))
                kl.check(kl.wait())
            bufs.append(b)
        xb = kl.Buffer(device, 4 * k)
        xb.upload(rng.standard_normal(k, dtype=np.float32))
        yb = kl.Buffer(device, 4 * n)
        with kl.runtime_mutex():
            for i in range(5):
                kl.native_q4_matmul(ws, device, yb.data, bufs[i % len(bufs)].data, xb.data, k, n)
            start, stop = events.create(), events.create()
            events.record(start, stream)
            t0 = time.perf_counter()
            for i in range(reps):
                kl.native_q4_matmul(ws, device, yb.data, bufs[i % len(bufs)].data, xb.data, k, n)
            wall_us = (time.perf_counter() - t0) * 1e6 / reps
            events.record(stop, stream)
            kl.select(device)
            kl.check(kl.wait())
            ms = events.elapsed_ms(start, stop) / reps
        total = nbytes + 4 * k + 4 * n
        out[f"k{k}_n{n}"] = {"us": round(ms * 1e3, 3), "host_wall_us": round(wall_us, 3),
                             "gbps": round(total / (ms * 1e-3) / 1e9, 1),
                             "hbm_frac": round(total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                             "reference_k200_ms": NATIVE_REFERENCE_MS[(k, n)]}
        for b in bufs + [xb, yb]:
            b.close()
    return out


COMMON_SHAPES = ((4096, 11008, 1), (4096, 4096, 1), (11008, 4096, 1), (4096, 11008, 128), (4096, 4096, 128))


def common_leg(events, stream, device: int, reps: int) -> dict:
    """common_q4_matmul (common Q4 ABI v1) at the reference's main shapes, M = 1
    (two-component A8 GEMV) and M = 128 (Row A8 GEMM), F32 X, over rotating
    weight copies. Calls complete before returning; `us` is per call. GB/s =
    layout bytes + 4mk + 4mn over that time; TOP/s = 2mkn / time for M > 1."""
    out = {}
    rng = np.random.Generator(np.random.PCG64(44))
    ws = kl.CommonQ4Workspace()
    for k, n, m in COMMON_SHAPES:
        q4 = kl.quantize_q4_0(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
        nbytes = kl.common_q4_size(k, n)
        weights = []
        for _ in range(max(2, -(-ROTATE_BYTES // nbytes))):
            w = kl.CommonQ4Weight(device, k, n)
            w.upload(q4)                         # a handle is usable once uploaded
            weights.append(w)
        xb = kl.Buffer(device, 4 * m * k)
        xb.upload(rng.standard_normal((m, k), dtype=np.float32))
        yb = kl.Buffer(device, 4 * m * n)
        with kl.runtime_mutex():
            for i in range(3):
                kl.common_q4_matmul(ws, device, yb.data, weights[i % len(weights)], xb.data, m)
            start, stop = events.create(), events.create()
            events.record(start, stream)
            t0 = time.perf_counter()
            for i in range(reps):
                kl.common_q4_matmul(ws, device, yb.data, weights[i % len(weights)], xb.data, m)
            wall_us = (time.perf_counter() - t0) * 1e6 / reps
            events.record(stop, stream)
            kl.select(device)
            kl.check(kl.wait())
            ms = events.elapsed_ms(start, stop) / reps
        total = nbytes + 4 * m * k + 4 * m * n
        entry = {"us": round(ms * 1e3, 3), "host_wall_us": round(wall_us, 3),
                 "gbps": round(total / (ms * 1e-3) / 1e9, 1)}
        if m > 1:
            entry["tops"] = round(2.0 * m * k * n / (ms * 1e-3) / 1e12, 1)
        out[f"k{k}_n{n}_m{m}"] = entry
        for w in weights:
            w.close()
        xb.close()
        yb.close()
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--kernel-reps", type=int, default=300, help="launches of the dominant GEMV for roofline")
    ap.add_argument("--cpu-seconds", type=float, default=5.0, help="seconds per CPU-baseline thread count")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--gemm-reps", type=int, default=50, help="timed batch-512 GEMM calls per shape (0: skip)")
    ap.add_argument("--small-reps", type=int, default=100, help="timed calls per small-batch config (0: skip)")
    ap.add_argument("--native-reps", type=int, default=100, help="timed native_q4_matmul calls per shape (0: skip)")
    ap.add_argument("--common-reps", type=int, default=50, help="timed common_q4_matmul calls per shape (0: skip)")
    ap.add_argument("--i8-reps", type=int, default=50, help="timed rowwise_i8 matmul calls per case (0: skip)")
    ap.add_argument("--read-reps", type=int, default=200, help="timed launches per read-ceiling run (0: skip)")
    ap.add_argument("--tune", action="append", default=[], metavar="NAME=V1,V2",
                    help="profiling aid with --only SHAPE: time the GEMV once per value of this tuning knob "
                         "(repeatable: every combination)")
    ap.add_argument("--read-sizes", default="", help="profiling aid: comma list of read-leg size names to run")
    ap.add_argument("--read-variants", default="", help="profiling aid: comma list of read-leg variants (0, 1, 2)")
    ap.add_argument("--read-waves", default="", help="profiling aid: comma list of read-leg wave counts")
    ap.add_argument("--only", choices=[name for name, _, _ in SHAPES] + ["gemm", "copy", "small", "native", "common",
                                                                          "i8", "read"],
                    help="profiling aid: time only this GEMV's launch loop, one leg, or (copy) a "
                         f"{COPY_BYTES >> 20} MiB device-to-device copy that calibrates the traffic counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported (this build has no "
              "multi-GPU path)", file=sys.stderr)
        return 2

    kl.load()
    device = 0
    events = HipEvents()
    stream = kl.stream(device)
    kernel = kl.Kernel()

    if args.only == "gemm":
        print(json.dumps({"gemm_b512": gemm_leg(kernel, events, stream, device, args.gemm_reps)}), flush=True)
        return 0
    if args.only == "small":
        print(json.dumps({"small_batch": small_batch_leg(kernel, events, stream, device, args.small_reps)}),
              flush=True)
        return 0
    if args.only == "i8":
        print(json.dumps({"rowwise_i8": i8_leg(kernel, events, stream, device, args.i8_reps)}), flush=True)
        return 0
    if args.only == "common":
        print(json.dumps({"common_q4": common_leg(events, stream, device, args.common_reps)}), flush=True)
        return 0
    if args.only == "native":
        print(json.dumps({"native_q4": native_leg(events, stream, device, args.native_reps)}), flush=True)
        return 0
    read_filter = {"sizes": [v for v in args.read_sizes.split(",") if v] or None,
                   "variants": [int(v) for v in args.read_variants.split(",") if v] or None,
                   "waves_list": [int(v) for v in args.read_waves.split(",") if v] or None}
    if args.only == "read":
        print(json.dumps({"read_ceiling": read_ceiling_leg(events, stream, device, args.read_reps, **read_filter)}),
              flush=True)
        return 0
    if args.only == "copy":
        print(json.dumps({"copy": copy_leg(events, stream, device)}), flush=True)
        return 0

    log("generating and uploading weights")
    # copies[name][c]: distinct device copies of each matrix, at least
    # ROTATE_BYTES per shape, so every launch reads its weights from HBM.
    copies = {}
    for i, (name, k, n) in enumerate(SHAPES):
        if args.only and name != args.only:
            continue
        nbytes = n * (k // 32) * 18
        first = kl.Buffer(device, nbytes)
        upload_q4_matrix(first, k, n, seed=1000 + i)
        bufs = [first]
        for _ in range(max(COPIES, -(-ROTATE_BYTES // nbytes)) - 1):
            buf = kl.Buffer(device, nbytes)
            with kl.runtime_mutex():
                kl.select(device)
                kl.check(kl.copy(buf.data, first.data, nbytes, kl.CopyKind.device_to_device))
                kl.check(kl.wait())
            bufs.append(buf)
        copies[name] = bufs
    rng = np.random.Generator(np.random.PCG64(7))
    xs, ys = {}, {}
    for name, k, n in SHAPES:
        xb = kl.Buffer(device, 4 * k)
        xb.upload(rng.standard_normal(k, dtype=np.float32))
        xs[name] = xb
        ys[name] = kl.Buffer(device, 4 * n)

    def weights(name: str, i: int) -> int:
        bufs = copies[name]
        return bufs[i % len(bufs)].data

    def step(i: int) -> None:
        for name, k, n in LAYER:
            kl.matmul(kernel, device, ys[name].data, weights(name, i), xs[name].data, k, n, 1, kl.WeightType.q4_0)

    host_us = {}

    def timed(fn, count: int, warmup: int, tag: str = "") -> float:
        with kl.runtime_mutex():
            for i in range(warmup):
                fn(i)
            kl.select(device)
            kl.check(kl.wait())
            start, stop = events.create(), events.create()
            events.record(start, stream)
            t0 = time.perf_counter()
            for i in range(count):
                fn(i)
            host_us[tag] = (time.perf_counter() - t0) * 1e6 / count
            events.record(stop, stream)
            ms = events.elapsed_ms(start, stop)
            kl.check(kl.wait())
        return ms

    if args.only:
        name, k, n = next(item for item in SHAPES if item[0] == args.only)

        def only(i):
            kl.matmul(kernel, device, ys[name].data, weights(name, i), xs[name].data, k, n, 1, kl.WeightType.q4_0)
        # --tune NAME=V1,V2 (repeatable): one timed loop per combination of knob values
        knobs = [(t.split("=", 1)[0], t.split("=", 1)[1].split(",")) for t in args.tune]
        combos = [[]]
        for knob, values in knobs:
            combos = [c + [(knob, v)] for c in combos for v in values]
        for combo in combos:
            for knob, value in combo:
                kl.set_tuning(knob, value)
            ms = timed(only, args.kernel_reps, args.warmup, "only") / args.kernel_reps
            print(json.dumps({"only": name, "k": k, "n": n, "tuning": dict(combo), "us_per_launch": round(ms * 1e3, 3),
                              "host_us_per_call": round(host_us["only"], 3),
                              "gbps": round(q4_bytes(k, n) / (ms * 1e-3) / 1e9, 1), "route": kernel.route}),
                  flush=True)
        return 0

    dname, dk, dn = DOMINANT

    def gate_step(i: int) -> None:
        kl.matmul(kernel, device, ys[dname].data, weights(dname, i), xs[dname].data, dk, dn, 1, kl.WeightType.q4_0)

    # settle: untimed layer-set steps for SETTLE_MS of wall time before the
    # warm-up steps, so the timed region does not start while the GPU is still
    # ramping up from idle
    log(f"settling for {SETTLE_MS} ms")
    settle_steps = 0
    with kl.runtime_mutex():
        kl.select(device)
        t_settle = time.perf_counter()
        while (time.perf_counter() - t_settle) * 1e3 < SETTLE_MS:
            for i in range(50):
                step(settle_steps + i)
            settle_steps += 50
            kl.check(kl.wait())
    log("timing the K4096xN11008 GEMV steps")
    wall0 = time.perf_counter()
    step_ms = timed(gate_step, args.steps, args.warmup, "step") / args.steps
    wall_ms = (time.perf_counter() - wall0) * 1e3
    step_bytes = q4_bytes(dk, dn)
    value = step_bytes / (step_ms * 1e-3) / 1e9
    gate_route = kernel.route

    log("timing the layer set")
    layer_ms = timed(step, args.steps, args.warmup) / args.steps
    layer_bytes = sum(q4_bytes(k, n) for _, k, n in LAYER)

    # Spread: SPREAD_LOOPS more event-timed loops of SPREAD_LAUNCHES launches
    # each (an event per launch would make the loop host-bound and time the
    # submission instead); median, min and max of the loops' per-launch means.
    def loop_means(fn) -> list:
        return [timed(fn, SPREAD_LAUNCHES, 2) / SPREAD_LAUNCHES * 1e3 for _ in range(SPREAD_LOOPS)]

    per_shape = {}
    for name, k, n in SHAPES:
        def one(i, name=name, k=k, n=n):
            kl.matmul(kernel, device, ys[name].data, weights(name, i), xs[name].data, k, n, 1, kl.WeightType.q4_0)
        ms = timed(one, args.kernel_reps, 5) / args.kernel_reps
        gbps = q4_bytes(k, n) / (ms * 1e-3) / 1e9
        spread = loop_means(one)
        per_shape[f"{name}_k{k}_n{n}"] = {"us": round(ms * 1e3, 3), "gbps": round(gbps, 1),
                                           "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4), "route": kernel.route,
                                           "rotating_copies": len(copies[name]),
                                           "loop_mean_us": {"loops": SPREAD_LOOPS, "launches": SPREAD_LAUNCHES,
                                                            "median": round(float(np.median(spread)), 3),
                                                            "min": round(min(spread), 3),
                                                            "max": round(max(spread), 3)}}
    dom = per_shape[f"{dname}_k{dk}_n{dn}"]
    achieved = dom["gbps"]

    gemm = gemm_leg(kernel, events, stream, device, args.gemm_reps) if args.gemm_reps > 0 else None
    small = small_batch_leg(kernel, events, stream, device, args.small_reps) if args.small_reps > 0 else None
    native = native_leg(events, stream, device, args.native_reps) if args.native_reps > 0 else None
    common = common_leg(events, stream, device, args.common_reps) if args.common_reps > 0 else None
    i8 = i8_leg(kernel, events, stream, device, args.i8_reps) if args.i8_reps > 0 else None
    read = read_ceiling_leg(events, stream, device, args.read_reps, **read_filter) if args.read_reps > 0 else None
    read_gbps = read["gate_gemv"]["best"]["gbps"] if read and "gate_gemv" in read else None
    if read:
        # each GEMV against the read leg at its own size: read time / GEMV time
        for name, k, n in SHAPES:
            leg = read.get(READ_OF_SHAPE[name])
            if leg:
                entry = per_shape[f"{name}_k{k}_n{n}"]
                entry["read_leg_us"] = leg["best"]["us"]
                entry["frac_of_read_leg"] = round(leg["best"]["us"] / entry["us"], 4)
        if small:
            leg = read.get("small_batch_q4")
            for tag, entry in small.items():
                if leg and tag.startswith("q4_k4096_n14336_"):
                    entry["read_leg_us"] = leg["best"]["us"]
                    entry["frac_of_read_leg"] = round(leg["best"]["us"] / entry["us"], 4)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: Q4_0 from seeded N(0,0.02) (ggml closed form), X ~ N(0,1) f32",
        "config": {
            "workload": "q4_0-gemv-k4096-n11008-b1 (the metric's shape; the gate GEMV of BASELINE configs[1])",
            "k": dk,
            "n": dn,
            "batch": 1,
            "bytes_per_step": step_bytes,
            "hbm_frac": round(value / HBM_PEAK_GBPS, 4),
            "rotating_copies": len(copies[dname]),
            "route": gate_route,
            "wall_ms_timed_region": round(wall_ms, 3),
            "settle": {"ms": SETTLE_MS, "untimed_layer_set_steps": settle_steps},
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"q4 GEMV K{dk}xN{dn} b1 ({dom['route']})",
            "achieved": achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(),
            "traffic_source": os.path.relpath(TRAFFIC_PROFILE, ROOT) if measured_traffic() else None,
            "bytes_per_launch": q4_bytes(dk, dn),
            "avg_launch_us": dom["us"],
            "read_ceiling_gbps": read_gbps,
            "frac_of_read_ceiling": round(achieved / read_gbps, 4) if read_gbps else None,
        },
        "cpu_baseline": cpu,
        "layer_set": {
            "shapes_k_n": [[k, n] for _, k, n in LAYER],
            "ms_per_step": round(layer_ms, 6),
            "bytes_per_step": layer_bytes,
            "gbps": round(layer_bytes / (layer_ms * 1e-3) / 1e9, 1),
            "weight_set_mb": round(sum(n * (k // 32) * 18 for _, k, n in LAYER) / 1e6, 1),
        },
        "per_shape": per_shape,
        "read_ceiling": read,
        "gemm_b512": gemm,
        "small_batch": small,
        "native_q4": native,
        "common_q4": common,
        "rowwise_i8": i8,
    }
    print(json.dumps(result), flush=True)
    for bufs in copies.values():
        for buf in bufs:
            buf.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
