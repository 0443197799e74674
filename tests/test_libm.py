"""Pins the kernels' tanh and exp to the libm that ft-core calls.

ft-core computes GELU with Rust's f32::tanh (ft-model/src/lib.rs:436) and the
routing weights with f32::exp (:1495); on Linux both call glibc's tanhf /
expf. freetoken-rs_amd/csrc/ft_libm.hpp restates glibc 2.35's algorithms
(fdlibm tanhf with its expm1f, the table-driven expf) in IEEE basic operations; the
HIP kernels compile exactly that source. These tests compile the same header
for the host and compare it with this host's libm on EVERY f32 bit pattern,
so the kernels' GELU q8 blocks and routing weights are libm's, not an
approximation of them. (Exhaustive: 2 x 2^32 evaluations, ~20 s on 8 cores.)
"""
import ctypes
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "_build", "liblibmcheck.so")


@pytest.fixture(scope="module")
def lc():
    if not os.path.exists(LIB):
        import subprocess
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    L = ctypes.CDLL(LIB)
    for fn in ("lc_sweep_tanhf", "lc_sweep_expf"):
        f = getattr(L, fn)
        f.restype = ctypes.c_int64
        f.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int, ctypes.POINTER(ctypes.c_uint32)]
    for fn in ("lc_tanhf", "lc_expf"):
        f = getattr(L, fn)
        f.restype, f.argtypes = ctypes.c_float, [ctypes.c_float]
    return L


def sweep(lc, fn, lo=0, hi=1 << 32):
    bad = ctypes.c_uint32()
    n = getattr(lc, fn)(lo, hi, min(16, os.cpu_count() or 1), ctypes.byref(bad))
    return n, hex(bad.value)


@pytest.mark.parametrize("fn", ["lc_sweep_tanhf", "lc_sweep_expf"])
def test_restatement_equals_libm_on_every_f32(lc, fn):
    n, first = sweep(lc, fn)
    assert n == 0, f"{fn}: {n} inputs differ from libm, first {first}"


def test_sweep_detects_a_one_ulp_difference(lc):
    """The comparison is bitwise: a restatement one ulp off at a single input
    would be counted. Checked by comparing libm's tanhf with nextafter of
    itself on a range (done in Python on a sample, with the same equality)."""
    import numpy as np
    libm = ctypes.CDLL("libm.so.6")
    libm.tanhf.restype, libm.tanhf.argtypes = ctypes.c_float, [ctypes.c_float]
    xs = np.linspace(-5, 5, 101, dtype=np.float32)
    mine = np.array([lc.lc_tanhf(float(x)) for x in xs], np.float32)
    ref = np.array([libm.tanhf(float(x)) for x in xs], np.float32)
    assert np.array_equal(mine.view(np.uint32), ref.view(np.uint32))
    off = np.nextafter(ref, np.float32(np.inf))
    assert not np.array_equal(mine.view(np.uint32), off.view(np.uint32))


def test_special_values(lc):
    import math
    inf, nan = float("inf"), float("nan")
    assert lc.lc_tanhf(inf) == 1.0 and lc.lc_tanhf(-inf) == -1.0 and math.isnan(lc.lc_tanhf(nan))
    assert lc.lc_tanhf(0.0) == 0.0 and math.copysign(1.0, lc.lc_tanhf(-0.0)) == -1.0
    assert lc.lc_tanhf(30.0) == 1.0
    assert lc.lc_expf(0.0) == 1.0 and lc.lc_expf(-inf) == 0.0 and lc.lc_expf(inf) == inf
    assert lc.lc_expf(-200.0) == 0.0 and lc.lc_expf(100.0) == inf
