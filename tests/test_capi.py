"""CPU checks of the C-ABI library: it loads, exports every symbol the public
headers declare, host-only functions compute the reference's layout
arithmetic, and invalid matmul arguments abort before any device work
(reference src/k200.cpp:271-277; contract style of bench/common-q4-contract.cpp)."""
import ctypes
import os
import re
import signal
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
C_HEADER = os.path.join(ROOT, "include", "kunlun", "k200_c.h")
CXX_HEADER = os.path.join(ROOT, "include", "kunlun", "k200.h")


def _c_names():
    text = open(C_HEADER).read()
    return sorted(set(re.findall(r"\b(kunlun_[a-z0-9_]+)\s*\(", text)))


def _dynamic_symbols(path):
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", path], capture_output=True, text=True, check=True)
    return out.stdout


def test_every_c_symbol_is_exported(kl):
    names = _c_names()
    assert len(names) >= 25
    lib = ctypes.CDLL(kl.LIBRARY_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing
    declared = {name for name, _, _ in kl.C_FUNCTIONS}
    assert declared == set(names), "Python bindings and k200_c.h disagree"


def test_every_cxx_function_is_exported(kl):
    text = open(CXX_HEADER).read()
    body = text[text.index("namespace kunlun {"):]
    names = set(re.findall(r"^\s*[\w:&<>\s\*]+?\b([a-z_][a-z0-9_]*)\s*\(", body, re.M))
    names -= {"if", "return", "sizeof", "data", "size"}
    symbols = _dynamic_symbols(kl.LIBRARY_PATH)
    # free functions as kunlun::name(, member functions as kunlun::Class::name(
    missing = [n for n in sorted(names) if not re.search(rf"kunlun::(\w+::)?{n}\(", symbols)]
    assert not missing
    for cls in ("NativeQ4Workspace", "CommonQ4Weight", "CommonQ4Workspace", "CommonQ4ActivationLease"):
        assert f"kunlun::{cls}::~{cls}()" in symbols
    for special in ("kunlun::Buffer::Buffer(int, unsigned long)", "kunlun::Buffer::~Buffer()",
                    "kunlun::Kernel::Kernel()", "kunlun::Kernel::~Kernel()"):
        assert special in symbols
    assert "kk_dense_matmul" not in symbols, "internal launchers must stay hidden"


def test_soname(kl):
    out = subprocess.run(["readelf", "-d", kl.LIBRARY_PATH], capture_output=True, text=True, check=True).stdout
    assert "libkunlunk200.so.0" in out


def test_layout_arithmetic(kl):
    # reference src/k200.cpp:98-101
    assert kl.aligned(0) == 0 and kl.aligned(1) == 256 and kl.aligned(256) == 256 and kl.aligned(257) == 512
    assert kl.packed_i8_size(4096, 4096) == 16777216 + 16384 + 256
    assert kl.packed_i8_size(1024, 512) == 524288 + 2048 + 256
    assert kl.packed_i8_size(33 * 32, 7) == 7424 + 256 + 256
    base = 1 << 20
    assert kl.packed_i8_scales(base, 1024, 512) == base + 524288
    assert kl.packed_i8_maxima(base, 1024, 512) == base + 524288 + 2048
    assert kl.packed_i8_scales(base, 100 * 32, 3) == base + 9728


def test_version_and_statistics(kl):
    assert kl.version().startswith("0.7.12")
    s = kl.statistics()
    assert s["matmuls"] == [0, 0] and s["peer_copies"] == 0 and s["peer_bytes"] == 0


def test_weight_type_values(kl):
    assert [int(t) for t in kl.WeightType] == [0, 1, 2, 3, 4]
    assert [int(t) for t in kl.CopyKind] == [0, 1, 2]


def test_runtime_mutex_is_recursive(kl):
    with kl.runtime_mutex():
        with kl.runtime_mutex():
            assert kl.aligned(5) == 256


# Each call aborts in argument validation, before selecting a device. Pointers
# are fake non-null addresses that are never dereferenced.
BAD_CALLS = {
    "k_not_multiple_of_32": "k=33",
    "k_zero": "k=0",
    "k_above_16384": "k=16416",
    "n_zero": "n=0",
    "batch_zero": "batch=0",
    "n_batch_overflow": "n=1 << 20, batch=1 << 10",
    "null_y": "y=0",
    "null_w": "w=0",
    "null_x": "x=0",
    "tile_8": "tile=8",
    "type_q6_k": "type=kl.WeightType.q6_k",
    "type_5": "type=5",
    "i8_without_scales": "type=kl.WeightType.rowwise_i8, scales=None, maxima=4096",
    "i8_without_maxima": "type=kl.WeightType.rowwise_i8, scales=4096, maxima=None",
    "misaligned_x": "x=4096 + 2",
    "misaligned_y": "y=8192 + 1",
}


@pytest.mark.parametrize("case", sorted(BAD_CALLS))
def test_matmul_contract_aborts(case):
    args = dict(y="8192", w="12288", x="4096", k="256", n="65", batch="4", type="kl.WeightType.q4_0",
                scales="None", maxima="None", tile="16")
    for part in BAD_CALLS[case].split(", "):
        key, value = part.split("=", 1)
        args[key.strip()] = value
    code = (
        "import kunlunk200_lib_amd as kl\n"
        "kern = kl.Kernel()\n"
        f"kl.matmul(kern, 0, {args['y']}, {args['w']}, {args['x']}, {args['k']}, {args['n']}, {args['batch']}, "
        f"{args['type']}, scales={args['scales']}, maxima={args['maxima']}, tile={args['tile']})\n"
        "print('NOT REJECTED')\n"
    )
    env = dict(os.environ, PYTHONPATH=ROOT, HIP_VISIBLE_DEVICES="")
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert "NOT REJECTED" not in proc.stdout
    assert proc.returncode == -signal.SIGABRT, proc.stderr
    assert "invalid argument" in proc.stderr
    assert "device=-1" in proc.stderr, "rejected only after selecting a device"


def test_upload_i8_rows_contract_aborts():
    code = (
        "import numpy as np, kunlunk200_lib_amd as kl\n"
        "kl.upload_i8_rows(0, 4096, 64, 4, 3, 2, np.zeros((2, 64), np.float32))\n"
        "print('NOT REJECTED')\n"
    )
    env = dict(os.environ, PYTHONPATH=ROOT, HIP_VISIBLE_DEVICES="")
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert proc.returncode == -signal.SIGABRT and "NOT REJECTED" not in proc.stdout


# ---------------------------------------------------------------------------
# SwiGLU layout and pointer contract (reference src/k200.cpp:324-350;
# contract cases of reference bench/swiglu-contract.cpp). Every case is
# rejected before any device work, so these run without a GPU.

def test_swiglu_reason_rules(kl):
    L = kl.SwiGLULayout
    f32, f16 = kl.InputType.f32, kl.InputType.f16
    assert kl.swiglu_reason(L(256, 2, 1024, 1024, 1024, f32)) == ""
    assert kl.swiglu_reason(L(256, 2, 512, 512, 512, f16)) == ""
    assert kl.swiglu_reason(L(256, 2, 1024, 1024, 1024, 99)) == "type"
    for width, rows in ((0, 1), (1, 0), (65537, 1), (-3, 2), (256, 2 ** 31 // 256 // 4 + 1)):
        assert kl.swiglu_reason(L(width, rows, 2 ** 20, 2 ** 20, 2 ** 20, f32)) == "shape"
    assert kl.swiglu_reason(L(65536, 1, 262144, 262144, 262144, f32)) == ""
    assert kl.swiglu_reason(L(256, 2, 1023, 1024, 1024, f32)) == "stride"      # shorter than a row
    assert kl.swiglu_reason(L(256, 2, 1024, 1026, 1024, f32)) == "stride"      # not a multiple of 4
    assert kl.swiglu_reason(L(256, 2, 1024, 1024, 514, f16)) == ""             # f16: multiple of 2 is enough
    assert kl.swiglu_reason(L(256, 2, 1024, 1024, 513, f16)) == "stride"
    # rows - 1 strides plus one row must stay within INT_MAX bytes
    assert kl.swiglu_reason(L(256, 2 ** 16, 2 ** 15 + 1024, 1024, 1024, f32)) == "byte extent"


SWIGLU_CONTRACT = list(range(11))


@pytest.mark.parametrize("case", SWIGLU_CONTRACT)
def test_swiglu_contract_rejects_before_device(kl, case):
    count = ctypes.c_int(0)
    if kl.load().kunlun_device_count(ctypes.byref(count)) == 0 and count.value > 0:
        pytest.skip("contract cases pass fabricated pointers: they run on a host without a GPU")
    base = kl.SwiGLULayout(256, 2, 1024, 1024, 1024, kl.InputType.f32)
    layout = kl.SwiGLULayout(**vars(base))
    device, y, g, u = 0, 0x100000, 0x200000, 0x300000
    yb = gb = ub = 2048
    if case == 0:
        layout.width = 0
    elif case == 1:
        layout.rows = 0
    elif case == 2:
        layout.width = 65537
    elif case == 3:
        layout.gate_stride = 1023
    elif case == 4:
        layout.rows = 2 ** 31 - 1
    elif case == 5:
        layout.type = 99
    elif case == 6:
        yb = 1024                       # output span beyond its size
    elif case == 7:
        g = None
    elif case == 8:
        y = 0x100001                    # misaligned output
    elif case == 9:
        y = g + 4                       # partial overlap with gate
    elif case == 10:
        device = -1
    kernel = kl.Kernel()
    before = kl.allocated_bytes(0)
    assert kl.swiglu(kernel, device, y, yb, g, gb, u, ub, layout) is False
    assert kl.allocated_bytes(0) == before
    assert kernel.route is None


# ---------------------------------------------------------------------------
# elementwise argument rules (reference src/k200.cpp:283-286). Each call aborts
# before selecting a device; pointers are fake and never dereferenced.
EW_BAD_CALLS = {
    "null_y": "y=0",
    "null_a": "a=0",
    "null_b": "b=0",
    "count_zero": "count=0, width=1, b_count=1",
    "count_above_int_max_over_4": "count=(2 ** 31 - 1) // 4 + 1, width=1, b_count=1",
    "width_zero": "width=0",
    "width_above_16384": "count=16385 * 2, width=16385, b_count=16385",
    "count_not_multiple_of_width": "count=1000, width=256, b_count=256",
    "op_5": "op=5",
    "op_negative": "op=-1",
    "b_count_other": "b_count=100",
    "rms_eps_zero": "op=3, parameter=0.0",
    "rms_eps_negative": "op=3, parameter=-1e-5",
    "rms_eps_nan": "op=3, parameter=float('nan')",
    "rms_eps_inf": "op=3, parameter=float('inf')",
    "misaligned_y": "y=8192 + 2",
}


@pytest.mark.parametrize("case", sorted(EW_BAD_CALLS))
def test_elementwise_contract_aborts(case):
    args = dict(y="8192", a="4096", b="12288", count="1024", width="256", b_count="256", op="0",
                parameter="1e-5")
    for part in EW_BAD_CALLS[case].split(", "):
        key, value = part.split("=", 1)
        args[key.strip()] = value
    code = (
        "import kunlunk200_lib_amd as kl\n"
        "kern = kl.Kernel()\n"
        f"kl.elementwise(kern, 0, {args['y']}, {args['a']}, {args['b']}, {args['count']}, {args['width']}, "
        f"{args['b_count']}, {args['op']}, {args['parameter']})\n"
        "print('NOT REJECTED')\n"
    )
    env = dict(os.environ, PYTHONPATH=ROOT, HIP_VISIBLE_DEVICES="")
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=120)
    assert "NOT REJECTED" not in proc.stdout
    assert proc.returncode == -signal.SIGABRT, proc.stderr
    assert "invalid argument" in proc.stderr
    assert "device=-1" in proc.stderr, "rejected only after selecting a device"


def test_elementwise_op_values(kl):
    assert [int(o) for o in kl.ElementwiseOp] == [0, 1, 2, 3, 4]
