"""The drop-in boundary as a C++ user of the reference meets it: a program
that includes only <kunlun/k200.h>, finds the library with
find_package(KunlunK200 0.1 CONFIG) and links KunlunK200::kunlunk200 (the
reference's consumer pattern, reference examples/library/CMakeLists.txt:1-5,
and its package, reference CMakeLists.txt:175-184), then runs the reference
library-bench call sequence (reference bench/library-bench.cpp:102-129) for
F32, F16, Q4_0 and rowwise INT8 on the GPU (tests/consumer/library_consumer.cpp).

CPU: the package configures, the program builds and links libkunlunk200.so.0
by its soname. GPU: the program built by __graft_entry__.build() runs and
every case passes its bounds."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import __graft_entry__ as entry  # noqa: E402


def test_consumer_builds_against_cmake_package(kl, tmp_path):
    exe = entry.build_consumer(str(tmp_path / "consumer"))
    assert os.path.exists(exe)
    needed = subprocess.run(["readelf", "-d", exe], capture_output=True, text=True, check=True).stdout
    assert "Shared library: [libkunlunk200.so.0]" in needed
    assert "amdhip64" not in needed, "the consumer needs no HIP library of its own"


def test_package_version_rules(tmp_path):
    # find_package(KunlunK200 0.1) is accepted (the reference consumer's request);
    # a newer or another major version is not
    for request, ok in (("0.1", True), ("0.7.12", True), ("0.8", False), ("1.0", False)):
        src = tmp_path / f"v{request}"
        src.mkdir()
        (src / "CMakeLists.txt").write_text(
            "cmake_minimum_required(VERSION 3.22)\nproject(v LANGUAGES NONE)\n"
            f"find_package(KunlunK200 {request} CONFIG REQUIRED)\n")
        proc = subprocess.run(["cmake", "-S", str(src), "-B", str(src / "b"),
                               f"-DKunlunK200_DIR={os.path.join(ROOT, 'kunlunk200_lib_amd', 'cmake')}"],
                              capture_output=True, text=True)
        assert (proc.returncode == 0) == ok, (request, proc.stderr[-800:])


@pytest.mark.gpu
def test_consumer_library_bench_sequence(gpu):
    exe = entry.CONSUMER_BIN
    assert os.path.exists(exe), "build the consumer first (__graft_entry__.build())"
    proc = subprocess.run([exe], capture_output=True, text=True, timeout=110)
    print(proc.stdout, flush=True)
    assert proc.returncode == 0, proc.stdout[-3000:] + proc.stderr[-2000:]
    lines = [line for line in proc.stdout.splitlines() if line.startswith("matmul")]
    assert len(lines) == 10 and all(line.endswith("PASS") for line in lines)
    assert "ALL PASS" in proc.stdout
