"""Self-check of the f32 square root the per-point kernels use for pair radii: it must equal the
correctly rounded sqrtf bit for bit over every float the kernels can pass it (0 and the integers
up to 2^46, the squared lattice distances) and beyond, on the device itself."""
import ctypes as C
import struct

import pytest

pytestmark = pytest.mark.gpu


def _bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


@pytest.mark.parametrize("lo,hi", [(0.0, 0.0), (1.0, 2.0 ** 64), (1e-30, 1.0)])
def test_lattice_sqrt_is_correctly_rounded(gpu, lo, hi):
    from graphgp_hip import _native as nat
    b0, b1 = _bits(lo), _bits(hi)
    bad = C.c_uint64(0)
    nat.call("ggp_selftest_sqrt_f32", b0, b1 - b0 + 1, C.byref(bad))
    assert bad.value == 0


@pytest.mark.parametrize("lo,hi", [(2.0 ** -20, 2.0 ** 0), (2.0 ** 0, 2.0 ** 20)])
def test_cholesky_division_matches_ieee_f32(gpu, lo, hi):
    """The per-point Cholesky and mean_vec divide by one reciprocal per column plus a one-fma
    remainder correction; over every f32 divisor in [lo, hi) (the range of L[j][j] for tables of
    moderate variance) with zero and 3 random numerators over 2^-100 .. 2^100 each, it must equal
    the IEEE division bit for bit."""
    from graphgp_hip import _native as nat
    b0, b1 = _bits(lo), _bits(hi)
    bad = C.c_uint64(0)
    nat.call("ggp_selftest_div", 0, b0, b1 - b0, 4, 20261202, C.byref(bad))
    assert bad.value == 0


def test_cholesky_division_matches_ieee_f64(gpu):
    """The same division in f64: 2^26 random divisors over 2^-60 .. 2^60, each with zero and 7
    random numerators over 2^-900 .. 2^900."""
    from graphgp_hip import _native as nat
    bad = C.c_uint64(0)
    nat.call("ggp_selftest_div", 1, 0, 1 << 26, 8, 7, C.byref(bad))
    assert bad.value == 0


@pytest.mark.parametrize("part", range(4))
def test_pivot_sqrt_is_correctly_rounded_everywhere(gpu, part):
    """The dense factor's f32 pivots go through the range-reduced square root; over every float
    bit pattern (a quarter per case: positive and negative, zero, subnormal, infinite, NaN) it
    must equal sqrtf bit for bit (NaN for NaN)."""
    from graphgp_hip import _native as nat
    bad = C.c_uint64(0)
    nat.call("ggp_selftest_sqrt_f32", part << 30, 1 << 30, C.byref(bad))
    assert bad.value == 0


@pytest.mark.parametrize("lo,hi", [(2.0 ** -126, 2.0 ** 0), (2.0 ** 0, 2.0 ** 126)])
def test_reciprocal_matches_ieee_f32(gpu, lo, hi):
    """The kernels' f32 reciprocal (v_rcp_f32 and one Newton step) against 1/d for every divisor
    bit pattern of the normal range (no numerators: the reciprocal alone)."""
    from graphgp_hip import _native as nat
    b0, b1 = _bits(lo), _bits(hi)
    bad = C.c_uint64(0)
    nat.call("ggp_selftest_div", 0, b0, b1 - b0, 0, 1, C.byref(bad))
    assert bad.value == 0


@pytest.mark.parametrize("x", [0.0, -0.0, float("inf"), float("-inf"), float("nan")])
def test_reciprocal_special_values_f32(gpu, x):
    from graphgp_hip import _native as nat
    bad = C.c_uint64(0)
    nat.call("ggp_selftest_div", 0, _bits(x), 1, 0, 1, C.byref(bad))
    assert bad.value == 0
