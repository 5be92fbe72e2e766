"""The restated float math against the host libm, exhaustively (every 32-bit float).

tsa_math.h claims that its expf and exp2f return exactly glibc's result for all 2^32 inputs and that its
log2f core is within one ulp of glibc's log2f on every float of [1, 2] (so that the 2-bit correction table
can express the difference).  tests/math_check.cpp checks all three with the host compiler; the C ABI's
tsa_host_math (the library's host copy of the device functions, with the correction table) must then equal
libm's log2f on every float of [1, 2] and libm's expf / exp2f on a dense sample.
"""
import ctypes
import os
import subprocess

import numpy as np

from treesa_gpu_amd import capi

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_restated_expf_exp2f_log2_core_exhaustive(tmp_path):
    exe = str(tmp_path / "math_check")
    subprocess.run(["g++", "-O2", "-fopenmp", "-ffp-contract=off", "-I", os.path.join(ROOT, "treesa_gpu_amd", "csrc"),
                    os.path.join(HERE, "math_check.cpp"), "-o", exe], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    bad_e, bad_2, far, fixed, bad_lse = map(int, r.stdout.split())
    assert (bad_e, bad_2, far, bad_lse) == (0, 0, 0, 0), r.stdout
    assert 0 < fixed < (1 << 23) // 20  # the correction table is sparse: about 1 % of [1, 2)


def test_metropolis_threshold_exhaustive(tmp_path):
    """Pre-order sweeps with their random numbers drawn ahead test x >= T(u) instead of u < expf(x): the same
    decision for every x when the restated expf is non-decreasing over all 2^32 floats and T(u) is the least float
    whose expf exceeds u, for every uniform u = k * 2^-24 the kernels draw (tests/threshold_check.cpp)."""
    exe = str(tmp_path / "threshold_check")
    subprocess.run(["g++", "-O2", "-fopenmp", "-ffp-contract=off", "-I", os.path.join(ROOT, "treesa_gpu_amd", "csrc"),
                    os.path.join(HERE, "threshold_check.cpp"), "-o", exe], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    drops, bad, nans = map(int, r.stdout.split())
    assert (drops, bad, nans) == (0, 0, 0), r.stdout


def test_library_host_math_equals_libm():
    lib = capi.load()
    libm = ctypes.CDLL("libm.so.6")
    for fn in ("log2f", "expf", "exp2f"):
        getattr(libm, fn).argtypes = [ctypes.c_float]
        getattr(libm, fn).restype = ctypes.c_float
    # log2f on every float of [1, 2] (2^23 + 1 values), vectorised through numpy's float32 log2 would not be
    # libm's; compare the library against libm through a small C loop instead
    src = r'''
#include <math.h>
#include <stdint.h>
#include <string.h>
extern float tsa_host_math(int which, float x);
long long run(void) {
  long long bad = 0;
  for (uint32_t k = 0; k <= (1u << 23); k++) {
    uint32_t u = 0x3f800000u + k; float y; memcpy(&y, &u, 4);
    float a = log2f(y), b = tsa_host_math(2, y);
    if (memcmp(&a, &b, 4) != 0) bad++;
  }
  uint32_t s = 0x9e3779b9u;
  for (int i = 0; i < (1 << 22); i++) {
    s = s * 1664525u + 1013904223u; float x; memcpy(&x, &s, 4);
    float a = expf(x), b = tsa_host_math(0, x), c = exp2f(x), d = tsa_host_math(1, x);
    if (memcmp(&a, &b, 4) != 0 && !(a != a && b != b)) bad++;
    if (memcmp(&c, &d, 4) != 0 && !(c != c && d != d)) bad++;
  }
  return bad;
}
'''
    import tempfile
    with tempfile.TemporaryDirectory() as td:
        c = os.path.join(td, "m.c")
        so = os.path.join(td, "m.so")
        with open(c, "w") as f:
            f.write(src)
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-shared", "-fPIC", c, "-o", so,
                        "-L", os.path.dirname(capi.LIB_PATH), "-ltreesa_hip", "-lm",
                        "-Wl,-rpath," + os.path.dirname(capi.LIB_PATH)], check=True)
        m = ctypes.CDLL(so)
        m.run.restype = ctypes.c_longlong
        assert m.run() == 0


def test_lse_table_matches_reference_definition():
    import oracle as orc
    t = orc.lse_table()
    assert t[0] == 1.0 and t[63] == 0.0 and t[53] == 0.0
    assert float(t[1]) == float.fromhex("0x1.2b8034p-1") and float(t[2]) == float.fromhex("0x1.49a784p-2")


def test_log2_core_table_matches_its_generator():
    # the constants of the log2 core in tsa_math.h are exactly what gen_log2_table.py prints; the generator
    # itself is pinned by the identities it must satisfy: inv_j * c_j rounds to 1, t_j is -log2(inv_j)
    # to double precision, and A_k are the series coefficients of log2(1 + z)
    import importlib.util
    import math
    import re
    import struct
    from fractions import Fraction
    spec = importlib.util.spec_from_file_location("gen_log2_table",
                                                  os.path.join(ROOT, "treesa_gpu_amd", "csrc", "gen_log2_table.py"))
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    hdr = open(os.path.join(ROOT, "treesa_gpu_amd", "csrc", "tsa_math.h")).read()
    body = hdr[hdr.index("#define TSA_LOG2_TAB"):]
    body = body[:body.index("}")]
    words = [int(x, 16) for x in re.findall(r"0x([0-9a-f]{16})ull", body)]
    rows = gen.table()
    assert words == [w for r in rows for w in r]
    for k, a in enumerate(gen.coeffs(), 1):
        m = re.search(rf"#define TSA_LOG2_A{k} (\S+)", hdr)
        assert m and float.fromhex(m.group(1)) == a
        assert abs(a - (-1) ** (k + 1) / (k * math.log(2))) <= 2e-16 * abs(a)
    d = lambda b: struct.unpack("<d", struct.pack("<Q", b))[0]
    for j, (bi, bt) in enumerate(rows):
        inv, t = d(bi), d(bt)
        c = Fraction(128 + j, 128)
        assert abs(Fraction(inv) * c - 1) <= Fraction(1, 2 ** 53)
        assert abs(t + math.log2(inv)) <= 4e-16 * max(t, 1e-300) + 1e-300
