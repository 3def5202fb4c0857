"""Common Q4 ABI v1 on the CPU: the oracle's layout and activation
quantization (reference src/q4-common-pack.h, docs/q4-common-ABI.json,
bench/common-q4-layout.cpp, bench/common-q4-bench.cpp:38-47,
kernels/kunlun-common-{max,main,residual}-exact.xpu) and the library's pure
functions and argument rules.

Pins: decode(pack(q4)) equals the Q4_0 decode bit for bit on random blocks
and on every FP16 scale pattern (the reference layout test's all-FP16 case);
every (column, K pair) lands on its own byte (no two share one: the packed
count of a marker nibble equals the number of pairs); the published ABI sizes;
the column-block addresses the GPU kernels use read back the source nibbles;
M = 1 codes equal orc_i8_activation's on the zero-padded input; M > 1 codes
follow the reference bench's CPU row rule.
"""
import os
import signal
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DIMS = [(33, 33), (512, 512), (11008, 129), (16383, 65), (4096, 300), (544, 513)]


def _raw(k, n, seed):
    """Random Q4_0 rows (ceil(k/32) blocks) with finite FP16 scales."""
    rng = np.random.default_rng(seed)
    blocks = -(-k // 32)
    raw = rng.integers(0, 256, (n, blocks, 18), dtype=np.uint8)
    scales = (rng.standard_normal((n, blocks)) * 0.01).astype(np.float16)
    raw[:, :, 0:2] = scales.view(np.uint8).reshape(n, blocks, 2)
    return raw.reshape(n, blocks * 18)


@pytest.mark.parametrize("k,n", DIMS)
def test_pack_round_trip(oracle, k, n):
    raw = _raw(k, n, k + n)
    packed = oracle.common_q4_pack(raw, k, n)
    kp, np_ = oracle.common_dims(k, n)
    assert packed.size == np_ * kp * 9 // 16                      # 4.5 padded bits per weight
    blocks = -(-k // 32)
    full = oracle.q4_decode(raw, blocks * 32, n)[:, :k]           # the last block may be partial
    assert np.array_equal(oracle.common_q4_decode(packed, k, n).view(np.uint32), full.view(np.uint32))


def test_pack_every_fp16_scale(oracle):
    """reference bench/common-q4-layout.cpp:17-19: all 65536 scale bit patterns."""
    k, n = 16384, 128
    raw = np.full((n * (k // 32), 18), 0x88, np.uint8)
    bits = np.arange(65536, dtype=np.uint32)
    raw[:, 0] = bits & 255
    raw[:, 1] = bits >> 8
    packed = oracle.common_q4_pack(raw.reshape(n, -1), k, n)
    kp, np_ = oracle.common_dims(k, n)
    scales = packed[np_ * kp // 2:].view(np.uint16).reshape(kp // 32, np_)   # [block][column]
    expect = bits.reshape(n, k // 32).T.astype(np.uint16)
    assert np.array_equal(scales[:, :n], expect)
    assert not packed[:np_ * kp // 2].any()                     # q = 8 -> signed 0


@pytest.mark.parametrize("k,n", [(33, 33), (544, 513), (4096, 300)])
def test_pack_is_injective(oracle, k, n):
    """Every nibble 0xf (q - 8 = 7 -> byte 0x77): a map sending two pairs to one
    byte would leave fewer 0x77 bytes than pairs."""
    blocks = -(-k // 32)
    raw = np.full((n, blocks, 18), 0xff, np.uint8)
    raw[:, :, 0:2] = 0x11
    packed = oracle.common_q4_pack(raw.reshape(n, -1), k, n)
    kp, np_ = oracle.common_dims(k, n)
    weights = packed[:np_ * kp // 2]
    assert int((weights == 0x77).sum()) == n * blocks * 16
    assert int((weights != 0).sum()) == n * blocks * 16


def test_published_sizes(oracle, kl):
    # docs/q4-common-ABI.json: payload Np*Kp*9/16, scale offset Np*Kp/2
    assert oracle.common_q4_size(4096, 11008) == 11008 * 4096 * 9 // 16
    assert oracle.common_q4_size(33, 33) == 256 * 512 * 9 // 16
    assert oracle.common_q4_size(0, 5) == 0 and oracle.common_q4_size(5, 32001) == 0
    for k, n in DIMS + [(4096, 4096), (11008, 4096), (16384, 32000)]:
        assert kl.common_q4_size(k, n) == oracle.common_q4_size(k, n)
    assert not kl.common_q4_supported(0, 1) and not kl.common_q4_supported(16385, 1)
    assert not kl.common_q4_supported(1, 32001) and kl.common_q4_supported(16384, 32000)


@pytest.mark.parametrize("k,n", [(512, 512), (4096, 300), (33, 40)])
def test_column_block_addresses(oracle, k, n):
    """The kernels read column c's block b as 16 contiguous bytes at
    ((c/32)(Kp/32) + b) 512 + (c%16) 32 + ((c%32)/16) 16, pair p at byte p."""
    raw = _raw(k, n, 7)
    packed = oracle.common_q4_pack(raw, k, n)
    kp, _ = oracle.common_dims(k, n)
    blocks = -(-k // 32)
    rng = np.random.default_rng(1)
    for c in sorted(set(rng.integers(0, n, 12).tolist()) | {0, 15, 16, 31, n - 1}):
        for b in sorted(set(rng.integers(0, blocks, 4).tolist()) | {0, blocks - 1}):
            at = ((c // 32) * (kp // 32) + b) * 512 + (c % 16) * 32 + ((c % 32) // 16) * 16
            src = raw[c, b * 18:(b + 1) * 18]
            for p in range(16):
                lo = (int(src[2 + (2 * p) % 16]) >> (0 if 2 * p < 16 else 4)) & 15
                hi = (int(src[2 + (2 * p + 1) % 16]) >> (0 if 2 * p + 1 < 16 else 4)) & 15
                assert packed[at + p] == ((lo ^ 8) | ((hi ^ 8) << 4))


@pytest.mark.parametrize("k", [33, 512, 4096, 11008, 16383])
@pytest.mark.parametrize("pattern", [0, 1, 3, 4])
def test_quant_pair_matches_two_pass_rule(oracle, k, pattern):
    x = oracle.fixture_input(k, 1, pattern).ravel()
    values, params = oracle.common_quant_pair(x, k)
    kp, _ = oracle.common_dims(k, 1)
    padded = np.zeros(kp, np.float32)
    padded[:k] = x
    q0, q1, m0, m1 = oracle.i8_activation(padded)
    j = np.arange(kp)
    i = (j // 32) * 64 + j % 32                                  # reference bench/common-q4-bench.cpp:40
    assert np.array_equal(values[i], q0) and np.array_equal(values[2 * kp + i], q1)
    gaps = np.ones(values.size, bool)
    gaps[i] = False
    gaps[2 * kp + i] = False
    assert not values[gaps].any()
    assert params[0] == np.float32(m0 / np.float32(127)) and params[1] == np.float32(m1 / np.float32(127))
    assert params[2] == m0 and params[3] == m1 and not params[4:].any()
    # the represented value is within the second component's half step of x
    # (plus the rounding of the residual x - q0 s0 and of 127/max1)
    qa = q0.astype(np.float64) * params[0] + q1.astype(np.float64) * params[1]
    assert np.all(np.abs(qa[:k] - x) <= params[1] * 0.5 * (1 + 1e-4) + np.spacing(np.abs(x)))


def test_quant_pair_zero_input_uses_unit_maximum(oracle):
    values, params = oracle.common_quant_pair(np.zeros(100, np.float32), 100)
    assert not values.any() and params[2] == 1.0 and params[3] == 1.0


@pytest.mark.parametrize("k,rows,defined", [(512, 3, 32), (4096, 32, 32), (544, 70, 96)])
def test_quant_rows_bench_rule(oracle, k, rows, defined):
    x = oracle.fixture_input(k, rows, 1)
    values, params = oracle.common_quant_rows(x, k, rows, defined)
    kp, _ = oracle.common_dims(k, 1)
    values = values.reshape(defined, kp)
    params = params.reshape(defined, 16)
    for r in range(rows):
        mx = np.float32(np.abs(x[r]).max()) or np.float32(1)
        inv, s = np.float32(127) / mx, mx / np.float32(127)
        v = (x[r] * inv).astype(np.float32)
        q = np.clip(np.trunc(v + np.where(v >= 0, np.float32(0.5), np.float32(-0.5))), -127, 127).astype(np.int8)
        assert np.array_equal(values[r, :k], q) and not values[r, k:].any()
        assert np.all(params[r] == s)
        assert np.all(np.abs(q * s - x[r]) <= s * 0.5 * (1 + 1e-6))
    assert not values[rows:].any() and np.all(params[rows:] == np.float32(1) / np.float32(127))


def test_weight_constructor_rejects_dimensions():
    """reference bench/common-q4-contract.cpp:8 ("dimensions"): aborts before any device use."""
    code = "import kunlunk200_lib_amd as kl\nkl.CommonQ4Weight(0, 0, 512)\nprint('NOT REJECTED')\n"
    env = dict(os.environ, PYTHONPATH=ROOT, HIP_VISIBLE_DEVICES="")
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert proc.returncode == -signal.SIGABRT and "NOT REJECTED" not in proc.stdout
    assert "device=-1" in proc.stderr


def test_pair_status_values(kl):
    assert [int(s) for s in kl.CommonQ4PairStatus] == list(range(9))
