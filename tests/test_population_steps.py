"""The level loop's population arithmetic on the host, against the oracle and against the textbook.

* Systematic resampling (population annealing, csrc/treesa_gpu.cu:1836-1855) and truncation selection
  (1857-1869): the binary's host code (lib/libtreesa_host.so, tsh_systematic / tsh_truncation) equals the
  oracle's on random energies with ties, infinities and every weight regime; the oracle's systematic step
  equals an independent numpy statement (cumulative normalized weights, the j-th point j + u taken by the
  first chain whose cumulative weight exceeds it) and has the textbook's properties; truncation on distinct
  energies equals a sort-based statement.
* The selection score and population energy (1737-1753): the binary's host formulas equal the oracle's on
  every mode and flag.
* The device's selection score (tsa_select.h, restated double exp2 / log2 so that kernels select without the
  host) against the reference's formula with the host libm: exp2 within 1 ulp and log2 within 4 ulp over the
  arguments the score passes, scores within 1 ulp, and on 20000 random populations the same best chain and no
  distinct glibc scores within 8 ulp of the best (tests/select_check.cpp).
"""
import ctypes
import json
import os
import subprocess

import numpy as np
import pytest

import oracle as orc
from treesa_gpu_amd import capi

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def host_lib():
    lib = ctypes.CDLL(capi.HOST_LIB_PATH)
    P, I, D, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_double, ctypes.c_float
    lib.tsh_systematic.argtypes = [P, I, D, D, P]
    lib.tsh_truncation.argtypes = [P, I, D, P]
    lib.tsh_score.argtypes = [P, D, D, F, I, I, I]
    lib.tsh_score.restype = D
    return lib


def product_systematic(lib, E, db, u):
    E = np.ascontiguousarray(E, np.float64)
    out = np.zeros(len(E), np.int32)
    lib.tsh_systematic(E.ctypes.data, len(E), db, u, out.ctypes.data)
    return out


def product_truncation(lib, E, frac):
    E = np.ascontiguousarray(E, np.float64)
    out = np.zeros(len(E), np.int32)
    lib.tsh_truncation(E.ctypes.data, len(E), frac, out.ctypes.data)
    return out


def energies(rng, n, kind):
    if kind == "distinct":
        return rng.normal(40.0, 5.0, n)
    if kind == "ties":
        return np.round(rng.normal(40.0, 2.0, n))
    if kind == "inf":
        E = rng.normal(40.0, 5.0, n)
        E[rng.random(n) < 0.1] = np.inf
        E[0] = 35.0
        return E
    return np.full(n, 33.25)  # all equal


def numpy_systematic(E, db, u):
    nc = len(E)
    with np.errstate(invalid="ignore"):
        w = np.exp(-db * (E - E.min()))
    cum = np.cumsum(w / w.sum() * nc)  # sequential sums, as the reference accumulates them
    hit = cum[None, :] > (np.arange(nc) + u)[:, None]  # NaN weights (0 * inf) never exceed a point
    return np.where(hit.any(axis=1), hit.argmax(axis=1), nc - 1).astype(np.int32)


@pytest.mark.parametrize("n", [1, 2, 7, 64, 128, 1000])
@pytest.mark.parametrize("kind", ["distinct", "ties", "inf", "equal"])
def test_systematic_resampling(n, kind):
    lib = host_lib()
    rng = np.random.default_rng(n * 7 + len(kind))
    for db in (0.0, 0.05, 0.5, 3.0, 50.0, 1e4):
        for _ in range(5):
            E = energies(rng, n, kind)
            u = float(rng.random())
            want = orc.systematic(E, db, u)
            assert np.array_equal(product_systematic(lib, E, db, u), want)
            assert np.array_equal(numpy_systematic(E, db, u), want), (n, kind, db)
            # properties: ancestors in order; every chain with zero weight dies; copies of chain c number
            # floor or ceil of its expected count n w_c / sum w (up to rounding of the cumulative sums)
            assert np.all(np.diff(want) >= 0) and want.min() >= 0 and want.max() < n
            with np.errstate(invalid="ignore"):
                w = np.exp(-db * (E - E.min()))
            if np.isfinite(w).all():
                expect = w / w.sum() * n
                got = np.bincount(want, minlength=n)
                assert np.all(got[w == 0] == 0)
                assert np.all(np.abs(got - expect) < 1.0 + 1e-9)


@pytest.mark.parametrize("n", [1, 4, 64, 128, 1000])
@pytest.mark.parametrize("kind", ["distinct", "ties", "inf", "equal"])
def test_truncation_selection(n, kind):
    lib = host_lib()
    rng = np.random.default_rng(n + 11 * len(kind))
    for frac in (0.0, 0.1, 0.25, 0.5):
        E = energies(rng, n, kind)
        want = orc.truncation(E, frac)
        assert np.array_equal(product_truncation(lib, E, frac), want)
        k = int(frac * n)
        if kind == "distinct":
            order = np.argsort(E)
            ref = np.arange(n, dtype=np.int32)
            ref[order[n - k:][::-1]] = order[:k]
            assert np.array_equal(want, ref)
        # every replaced chain copies one of the k best, and the k best survive
        assert np.sum(want != np.arange(n)) == min(k, n)


def test_scores_equal_oracle():
    lib = host_lib()
    rng = np.random.default_rng(5)
    for mode in (0, 1, 2):
        for slicing in (0, 1):
            for select_sc in (0, 1):
                for _ in range(300):
                    lc = float(np.float32(rng.uniform(-5, 80)))
                    sc, ns = int(rng.integers(5, 60)), int(rng.integers(0, 20))
                    sct, w = float(rng.integers(10, 50)), float(rng.choice([0.0, 1.0, 4.0, 0.5]))
                    flags = (ctypes.c_int * 3)(mode, slicing, select_sc)
                    for which in (0, 1):
                        got = lib.tsh_score(flags, sct, w, lc, sc, ns, which)
                        want = orc.score(mode, lc, sc, ns, slicing=bool(slicing), select_sc=bool(select_sc),
                                         sc_target=sct, sc_weight=w, energy=bool(which))
                        assert got == want or (np.isnan(got) and np.isnan(want)), (mode, slicing, select_sc, which)


def test_device_score_against_glibc_formula(tmp_path):
    exe = str(tmp_path / "select_check")
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-I", os.path.join(ROOT, "treesa_gpu_amd", "csrc"),
                    os.path.join(HERE, "select_check.cpp"), "-o", exe], check=True)
    r = json.loads(subprocess.run([exe], capture_output=True, text=True, timeout=300, check=True).stdout)
    assert r["exp2_max_ulp"] <= 1 and r["log2_max_ulp"] <= 4 and r["score_max_ulp"] <= 1, r
    assert r["best_chain_differs"] == 0 and r["glibc_near_ties_within_8ulp"] == 0, r
