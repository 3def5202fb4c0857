"""Native Q4 layout and API on the CPU (reference src/q4-layout.cpp:7-45,
src/k200.cpp:546-617, bench/native-q4-bench.cpp:38-53,
bench/native-q4-state-bench.cpp:6-8).

The oracle's layout restatement is pinned by the reference bench's own
inverse-mapping check (every nibble and FP16 scale recovered from the packed
bytes), by decode(pack(q4)) == Q4_0 decode bit for bit, and by the
reference's published size for K = N = 4096. The library's host packer must
then equal the oracle byte for byte. native_q4_matmul's argument rules must
abort before any device is selected.
"""
import os
import signal
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SHAPES = [(4096, 512), (96, 384), (544, 512), (32, 384), (64, 65), (32, 1), (160, 33), (1024, 128)]


def _q4_nibble(block: np.ndarray, e: int) -> int:
    """Element e of an 18-byte Q4_0 block as q - 8 (reference native-q4-reference.h:17)."""
    return int((block[2 + e % 16] >> (0 if e < 16 else 4)) & 15) - 8


def _signed4(v: int) -> int:
    v &= 15
    return v - 16 if v >= 8 else v


@pytest.mark.parametrize("k,n", SHAPES)
def test_oracle_pack_inverse_mapping(oracle, k, n):
    """The reference bench's check (native-q4-bench.cpp:44-52), element by element."""
    q4 = oracle.fixture_q4(k, n)
    packed = oracle.pack_native_q4(q4, k, n)
    rows = (n + 31) // 32 * 32
    payload = (rows * k // 2 + 255) // 256 * 256
    blocks = k // 32
    rng = np.random.default_rng(k + n)
    for r in sorted(set(rng.integers(0, n, 24).tolist()) | {0, n - 1}):
        for b in sorted(set(rng.integers(0, blocks, 6).tolist()) | {0, blocks - 1}):
            tb = (r // 32) * blocks + b
            p = q4[r, b * 18:(b + 1) * 18]
            assert bytes(packed[payload + (tb * 32 + r % 32) * 2:][:2]) == bytes(p[:2])
            for j in range(32):
                v = int(packed[tb * 512 + (j // 2) * 32 + r % 32])
                assert _signed4(v >> (j % 2 * 4)) == _q4_nibble(p, j)


@pytest.mark.parametrize("k,n", SHAPES)
def test_oracle_decode_of_pack_is_q4_decode(oracle, k, n):
    q4 = oracle.fixture_q4(k, n)
    w_native = oracle.native_q4_decode(oracle.pack_native_q4(q4, k, n), k, n)
    w_q4 = oracle.q4_decode(q4, k, n)
    assert np.array_equal(w_native.view(np.uint32), w_q4.view(np.uint32))


def test_oracle_size_closed_form(oracle):
    # reference docs/native-q4.md:73: "weights 9,437,184 B" for 4096 x 4096
    assert oracle.native_q4_size(4096, 4096) == 9437184
    for k, n in SHAPES:
        rows = (n + 31) // 32 * 32
        up = lambda v: (v + 255) // 256 * 256  # noqa: E731
        assert oracle.native_q4_size(k, n) == up(rows * k // 2) + up(rows * (k // 32) * 2)


def test_oracle_padding_rows_are_zero(oracle):
    k, n = 64, 33
    packed = oracle.pack_native_q4(oracle.fixture_q4(k, n), k, n)
    blocks = k // 32
    for b in range(blocks):
        tile_block = 1 * blocks + b                      # second tile holds row 32 only
        chunk = packed[tile_block * 512:(tile_block + 1) * 512].reshape(16, 32)
        assert not chunk[:, 1:].any()


def test_layout_supported_and_size(kl, oracle):
    # reference bench/native-q4-state-bench.cpp:6-8
    assert not kl.native_q4_layout_supported(31, 256)
    assert not kl.native_q4_layout_supported(17408, 256)
    assert not kl.native_q4_layout_supported(4096, 0)
    assert kl.native_q4_layout_supported(4096, 90000000 // 4096)
    assert not kl.native_q4_layout_supported(4096, 90000000 // 4096 + 1)
    assert kl.native_q4_layout_supported(16384, 1) and not kl.native_q4_layout_supported(0, 1)
    assert kl.native_q4_size(31, 256) == 0
    for k, n in SHAPES + [(4096, 4096), (4096, 11008), (11008, 4096)]:
        assert kl.native_q4_size(k, n) == oracle.native_q4_size(k, n)


@pytest.mark.parametrize("k,n", SHAPES)
def test_library_pack_equals_oracle(kl, oracle, k, n):
    q4 = oracle.fixture_q4(k, n)
    assert np.array_equal(kl.pack_native_q4_array(q4, k, n), oracle.pack_native_q4(q4, k, n))


def test_library_pack_random_bytes(kl, oracle):
    k, n = 256, 70
    q4 = np.random.default_rng(3).integers(0, 256, (n, k // 32 * 18), dtype=np.uint8)
    assert np.array_equal(kl.pack_native_q4_array(q4, k, n), oracle.pack_native_q4(q4, k, n))


def test_pack_rejections(kl):
    k, n = 64, 40
    need = kl.native_q4_size(k, n)
    q4 = np.zeros(n * (k // 32) * 18, np.uint8)
    out = np.full(need + 64, 0xAB, np.uint8)
    assert not kl.pack_native_q4(out, need - 1, q4, k, n)         # short destination
    assert not kl.pack_native_q4(None, need, q4, k, n)
    assert not kl.pack_native_q4(out, need, None, k, n)
    assert not kl.pack_native_q4(out, need, q4, 31, n)             # unsupported shape
    assert np.all(out == 0xAB), "a rejected pack wrote"
    # overlapping source and destination
    both = np.zeros(need + q4.size, np.uint8)
    assert not kl.pack_native_q4(both, need, both[need // 2:], k, n)
    assert kl.pack_native_q4(both, need, both[need:], k, n)       # adjacent ranges are fine
    # the whole destination is written: stale bytes become zero padding
    assert kl.pack_native_q4(out, need, q4, k, n)
    assert np.all(out[need:] == 0xAB)


def test_native_q4_reason_strings(kl):
    f32, f16 = kl.InputType.f32, kl.InputType.f16
    assert kl.native_q4_reason(4096, 4096, 1, f32) == ""
    assert kl.native_q4_reason(4096, 4096, 1, f16) == ""
    assert kl.native_q4_reason(31, 4096, 1) == "K/N/layout capacity"
    assert kl.native_q4_reason(4096, 4096, 1, 7) == "input type"
    assert kl.native_q4_reason(4096, 4096, 2) == "batch != 1"
    assert kl.native_q4_reason(4096, 4160, 1) == "rows not divisible by 128 (N64 requires 256)"
    # "partial capacity" (n * (k/32) * 4 > 16 MiB) needs n * k > 2^27, beyond
    # the layout's n * k <= 9e7: every supported shape passes that rule
    assert kl.native_q4_reason(16384, 90000000 // 16384 // 128 * 128, 1) == ""
    assert kl.native_q4_reason(4096, 384, 1) == ""


# native_q4_matmul argument rules (reference src/k200.cpp:557-566): each call
# aborts before a device is selected; pointers are fake and never dereferenced.
NQ_BAD_CALLS = {
    "device_negative": "device=-1",
    "k_not_multiple_of_32": "k=48",
    "k_above_16384": "k=16416",
    "n_zero": "n=0",
    "type_2": "type=2",
    "batch_zero": "batch=0",
    "n_batch_overflow": "n=20000, batch=30000",
    "null_y": "y=0",
    "null_w": "w=0",
    "null_x": "x=0",
    "misaligned_y": "y=0x40000002",
    "weights_not_256_aligned": "w=0x20000040",
    "misaligned_f32_x": "x=0x10000002",
    "misaligned_f16_x": "x=0x10000001, type=1",
    "y_overlaps_w": "y=0x20000100",
    "x_overlaps_w": "x=0x20001000",
    "y_overlaps_x": "y=0x10000000",
}


@pytest.mark.parametrize("case", sorted(NQ_BAD_CALLS))
def test_native_q4_matmul_contract_aborts(case):
    args = dict(device="0", y="0x40000000", w="0x20000000", x="0x10000000", k="256", n="128", batch="1",
                type="0")
    for part in NQ_BAD_CALLS[case].split(", "):
        key, value = part.split("=", 1)
        args[key.strip()] = value
    code = (
        "import kunlunk200_lib_amd as kl\n"
        "ws = kl.NativeQ4Workspace()\n"
        f"kl.native_q4_matmul(ws, {args['device']}, {args['y']}, {args['w']}, {args['x']}, {args['k']}, "
        f"{args['n']}, {args['batch']}, {args['type']})\n"
        "print('NOT REJECTED')\n"
    )
    env = dict(os.environ, PYTHONPATH=ROOT, HIP_VISIBLE_DEVICES="")
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert "NOT REJECTED" not in proc.stdout
    assert proc.returncode == -signal.SIGABRT, proc.stderr
    assert "invalid argument" in proc.stderr
    assert "device=-1" in proc.stderr, "rejected only after selecting a device"


def test_native_q4_valid_call_passes_validation():
    """The base arguments of the contract cases are valid: without a device
    they fail only when the device is selected (diagnostic device 0)."""
    code = (
        "import kunlunk200_lib_amd as kl\n"
        "ws = kl.NativeQ4Workspace()\n"
        "kl.native_q4_matmul(ws, 0, 0x40000000, 0x20000000, 0x10000000, 256, 128, 1, 0)\n"
    )
    env = dict(os.environ, PYTHONPATH=ROOT, HIP_VISIBLE_DEVICES="")
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert proc.returncode == -signal.SIGABRT and "device=0" in proc.stderr, proc.stderr
