"""The product's host-side Q4_0 quantizer (kunlunk200_lib_amd.formats, which
generates every test and bench weight) against the oracle's C restatement of
the same closed form (oracle/oracle.c orc_q4_quantize): identical bytes.

Both follow the ggml Q4_0 closed form BASELINE's configs state (per block: the
signed value of largest magnitude m, first occurrence; d = m / -8; id = 1/d or
0; F16(d) round-to-nearest-even; nibble = min(15, trunc(x*id + 8.5))). The
cases cover the branches a restatement can get wrong: ties in |x| (first
occurrence wins), negative and positive extremes, all-zero blocks (d = +0),
blocks whose scale rounds to an F16 subnormal, to zero, or overflows F16, and
values that land exactly on a nibble boundary.
"""
import numpy as np
import pytest

from kunlunk200_lib_amd import formats


def _cases():
    rng = np.random.default_rng(7)
    yield "gaussian", (rng.standard_normal((64, 4096)) * 0.02).astype(np.float32)
    yield "unit", rng.standard_normal((16, 1024)).astype(np.float32)
    z = np.zeros((3, 64), np.float32)
    z[1, 40] = -0.0
    yield "zeros", z
    t = np.tile(np.linspace(-1, 1, 32, dtype=np.float32), (4, 2))
    t[0, 5] = 1.0          # ties |x| = 1 with the -1 at index 0, which comes first: d = -1/-8 > 0
    t[1, :] = np.float32(0.5)
    t[2, 0::2] = np.float32(-0.75)
    t[2, 1::2] = np.float32(0.75)
    yield "ties", t
    b = np.arange(-8, 8, dtype=np.float32)
    yield "grid", np.tile(np.concatenate([b, b[::-1]]) * np.float32(0.125), (2, 2))
    tiny = (rng.standard_normal((8, 256)) * 1e-6).astype(np.float32)      # d in F16 subnormals
    tiny[0] *= np.float32(1e-3)                                            # d rounds to F16 zero
    yield "subnormal_scales", tiny
    huge = (rng.standard_normal((4, 128)) * 1e5).astype(np.float32)        # |d| above F16 max -> inf
    yield "huge", huge
    mixed = (rng.standard_normal((8, 512)) * np.logspace(-8, 3, 512, dtype=np.float32)).astype(np.float32)
    yield "mixed_magnitudes", mixed


@pytest.mark.parametrize("name,w", list(_cases()), ids=[c[0] for c in _cases()])
def test_quantize_q4_0_matches_oracle_bytes(oracle, name, w):
    with np.errstate(over="ignore", invalid="ignore"):
        got = formats.quantize_q4_0(w)
    want = oracle.q4_quantize(w)
    assert got.shape == want.shape == (w.shape[0], w.shape[1] // 32 * 18)
    diff = np.argwhere(got != want)
    assert diff.size == 0, f"{name}: first differing byte at {diff[:4].tolist()}"


def test_dequantize_q4_0_matches_oracle_decode(oracle):
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((32, 2048)) * 0.02).astype(np.float32)
    q4 = formats.quantize_q4_0(w)
    got = formats.dequantize_q4_0(q4, 2048)
    want = oracle.q4_decode(q4, 2048, 32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
