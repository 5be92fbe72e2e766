"""ctypes binding of the CPU oracle (oracle/liboracle.so) -- the checker of every parity test.

The oracle restates the reference's CPU port (csrc/cpu_ref.h) with its own vector-label data structures;
see oracle/tsa_oracle.cpp.  Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use it.
"""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "liboracle.so")
REF_BIN = os.path.join(ROOT, "oracle", "_ref", "ref_harness")

_lib = None


class OParams(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int32), ("sc_target", ctypes.c_float), ("sc_weight", ctypes.c_float),
                ("key0", ctypes.c_uint32), ("key1", ctypes.c_uint32), ("slicing", ctypes.c_int32),
                ("slice_moves", ctypes.c_int32), ("slice_every", ctypes.c_int32), ("max_slices", ctypes.c_int32),
                ("par_follow", ctypes.c_int32), ("par_band", ctypes.c_int32),
                ("lpeak", ctypes.c_float), ("lbw", ctypes.c_float), ("llaunch", ctypes.c_float),
                ("m0", ctypes.c_int32), ("n0", ctypes.c_int32), ("k0", ctypes.c_int32),
                ("v2_l3launch", ctypes.c_float), ("v2_lperm2", ctypes.c_float), ("v2_lcc_bit", ctypes.c_float),
                ("v2_lcc_cell", ctypes.c_float), ("v2_ltc_bit", ctypes.c_float), ("v2_ltc_pad", ctypes.c_float),
                ("v2_ltc_out", ctypes.c_float), ("v2_lsmall_cell", ctypes.c_float), ("v2_small_rank", ctypes.c_int32),
                ("leaf_sc", ctypes.c_int32)]


class OAnnealIn(ctypes.Structure):
    _fields_ = [("nlev", ctypes.c_int32), ("order", ctypes.c_int32), ("scheme", ctypes.c_int32),
                ("eval_every", ctypes.c_int32), ("select_sc", ctypes.c_int32), ("pad", ctypes.c_int32),
                ("trunc_frac", ctypes.c_double), ("sc_target", ctypes.c_double), ("sc_weight", ctypes.c_double),
                ("seed", ctypes.c_uint64), ("betas", ctypes.c_void_p), ("lmode", ctypes.c_void_p),
                ("lniters", ctypes.c_void_p), ("gm", ctypes.c_void_p), ("hm", ctypes.c_void_p),
                ("near_tol", ctypes.c_double), ("near_cap", ctypes.c_int32), ("pad2", ctypes.c_int32),
                ("near_out", ctypes.c_void_p), ("near_count", ctypes.c_void_p)]


# one level of oracle_anneal (struct OLevel)
LEVEL_DTYPE = np.dtype([("evaluated", "<i4"), ("best", "<i4"), ("sc", "<i4"), ("ns", "<i4"), ("families", "<i4"),
                        ("mode", "<i4"), ("resampled", "<i4"), ("lc", "<f4"), ("score", "<f8"), ("meanE", "<f8"),
                        ("meanNs", "<f8"), ("sel_margin", "<f8"), ("pop_margin", "<f8"), ("metropolis_near", "<i4"),
                        ("pad", "<i4")])

SCHEMES = {"indep": 0, "pa": 1, "trunc": 2}

DEFAULT_GM = (11.9e15, 1.6e13, 6, 6, 8, 4e-6)
DEFAULT_H100 = (4e-6, 1.23e13, 5.44e-14, 7.68e-15, 6.37e-14, 2.02e-16, 1.77e-13, 14, 1e-12)


def build():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB):
        build()
    lib = ctypes.CDLL(LIB)
    P, I, U32, U64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float
    lib.oracle_new.argtypes = [I, I, P, P, I, P]
    lib.oracle_new.restype = P
    lib.oracle_free.argtypes = [P]
    lib.oracle_splitmix64.argtypes = [U64]
    lib.oracle_splitmix64.restype = U64
    lib.oracle_philox.argtypes = [P, U32, U32, P]
    lib.oracle_par_pri.argtypes = [U32, U32, U32, U32]
    lib.oracle_par_pri.restype = U32
    lib.oracle_lse_table.argtypes = [P]
    lib.oracle_random_tree.argtypes = [I, U64, P]
    lib.oracle_labels.argtypes = [P, P, I, P]
    lib.oracle_random_slices.argtypes = [I, U64, I, I, I, P]
    lib.oracle_sweeps.argtypes = [P, ctypes.POINTER(OParams), I, I, I, I, P, I, I, I, F, U32, I, P]
    lib.oracle_energy.argtypes = [P, ctypes.POINTER(OParams), I, I, I, I, P, I, P, P, P]
    lib.oracle_slice_propose.argtypes = [P, ctypes.POINTER(OParams), I, I, I, I, P, P, P, P]
    lib.oracle_host_energy.argtypes = [P, P, P, I, I, I, I, P, I, P]
    lib.oracle_anneal.argtypes = [P, ctypes.POINTER(OParams), I, I, I, I, P, I, ctypes.POINTER(OAnnealIn), P, P, P,
                                  P, P]
    lib.oracle_repair.argtypes = [P, I, I, I, I, P, ctypes.c_double]
    lib.oracle_systematic.argtypes = [P, I, ctypes.c_double, ctypes.c_double, P]
    lib.oracle_truncation.argtypes = [P, I, ctypes.c_double, P]
    lib.oracle_score.argtypes = [I, I, I, ctypes.c_double, ctypes.c_double, F, I, I, I]
    lib.oracle_score.restype = ctypes.c_double
    lib.oracle_pa_uniforms.argtypes = [U64, I, P]
    lib.oracle_fnv64.argtypes = [P, ctypes.c_size_t]
    lib.oracle_fnv64.restype = U64
    lib.oracle_set_variant.argtypes = [I, U32]
    _lib = lib
    return lib


def params_from_config(cfg, leaf_sc, nlab):
    """OParams with the same values as a treesa_gpu_amd.capi.Config."""
    p = OParams()
    for name, _ in OParams._fields_:
        if name == "leaf_sc":
            continue
        setattr(p, name, getattr(cfg, name))
    if p.max_slices <= 0:
        p.max_slices = nlab
    if not p.slicing:
        p.slice_moves = 0
    p.leaf_sc = leaf_sc
    return p


class Oracle:
    def __init__(self, m, nlab, ixs, iy=()):
        self.lib = load()
        offs = np.zeros(m + 1, np.int32)
        for i, ix in enumerate(ixs):
            offs[i + 1] = offs[i] + len(ix)
        labs = np.array([l for ix in ixs for l in ix] or [0], np.int32)
        iya = np.array(list(iy) or [0], np.int32)
        self.h = self.lib.oracle_new(m, nlab, offs.ctypes.data, labs.ctypes.data, len(iy), iya.ctypes.data)
        self.m, self.nlab = m, nlab

    def labels(self, ch, W):
        ch = np.ascontiguousarray(ch, np.uint32)
        lab = np.zeros((self.m - 1, W), np.uint64)
        if self.lib.oracle_labels(self.h, ch.ctypes.data, W, lab.ctypes.data) != 0:
            return None
        return lab

    def sweeps(self, params, lay, pop, order, beta, sweep0, nsweeps, c0=0):
        """In-place sweeps of a (n, chain_words) population whose row k is chain c0 + k; returns stats."""
        assert pop.dtype == np.uint64 and pop.flags.c_contiguous
        st = np.zeros(6, np.int64)
        self.lib.oracle_sweeps(self.h, ctypes.byref(params), lay.W, lay.ch_off, lay.s_off, lay.chain_words,
                               pop.ctypes.data, c0, pop.shape[0], order, beta, sweep0, nsweeps, st.ctypes.data)
        return [int(x) for x in st]

    def energy(self, params, lay, pop):
        n = pop.shape[0]
        lc = np.zeros(n, np.float32)
        sc = np.zeros(n, np.int32)
        ns = np.zeros(n, np.int32)
        pop = np.ascontiguousarray(pop, np.uint64)
        self.lib.oracle_energy(self.h, ctypes.byref(params), lay.W, lay.ch_off, lay.s_off, lay.chain_words,
                               pop.ctypes.data, n, lc.ctypes.data, sc.ctypes.data, ns.ctypes.data)
        return lc, sc, ns

    def slice_propose(self, params, lay, rec, r1):
        """The chain evaluation of one record and the slice proposal words r1 make from it: dict(type, ladd, lrem,
        sc_int, ncand, ns, sc, lcost); type 0 add, 1 remove, 2 swap, -1 no move."""
        rec = np.ascontiguousarray(rec, np.uint64)
        w = np.array(r1, np.uint32)
        out = np.zeros(7, np.int32)
        lc = np.zeros(1, np.float32)
        self.lib.oracle_slice_propose(self.h, ctypes.byref(params), lay.W, lay.ch_off, lay.s_off, lay.chain_words,
                                      rec.ctypes.data, w.ctypes.data, out.ctypes.data, lc.ctypes.data)
        keys = ("type", "ladd", "lrem", "sc_int", "ncand", "ns", "sc")
        return dict(zip(keys, (int(x) for x in out)), lcost=float(lc[0]))

    def host_energy(self, lay, rec, slicing, gm, h100):
        rec = np.ascontiguousarray(rec, np.uint64)
        g = np.array(gm, np.float64)
        h = np.array(h100, np.float64)
        out = np.zeros(5, np.float64)
        self.lib.oracle_host_energy(self.h, g.ctypes.data, h.ctypes.data, lay.W, lay.ch_off, lay.s_off,
                                    lay.chain_words, rec.ctypes.data, 1 if slicing else 0, out.ctypes.data)
        return float(out[0]), int(out[1]), float(out[2]), float(out[3]), int(out[4])

    def anneal(self, params, lay, pop, betas, lmode, lniters, order, scheme="indep", eval_every=1, select_sc=False,
               trunc_frac=0.25, sc_target=20.0, sc_weight=1.0, seed=1, gm=DEFAULT_GM, h100=DEFAULT_H100,
               near_tol=0.0, near_cap=0):
        """The reference's level loop over a (nc, chain_words) population, in place (oracle_anneal).  Returns
        a dict: levels (LEVEL_DTYPE per level), anc (nlev x nc), best_rec, best_chain, nresample, staged,
        total_sweeps, h1 (the stage-1 incumbent's host energy when staged)."""
        assert pop.dtype == np.uint64 and pop.flags.c_contiguous
        nlev, nc = len(betas), pop.shape[0]
        b = np.array(betas, np.float32)
        lm = np.array(lmode, np.int32)
        ln = np.array(lniters, np.int32)
        g = np.array(gm, np.float64)
        hm = np.array(h100, np.float64)
        near = np.zeros((max(1, near_cap), 6), np.float64)
        nnear = np.zeros(1, np.int32)
        a = OAnnealIn(nlev, order, SCHEMES[scheme], eval_every, 1 if select_sc else 0, 0, trunc_frac, sc_target,
                      sc_weight, seed, b.ctypes.data, lm.ctypes.data, ln.ctypes.data, g.ctypes.data, hm.ctypes.data,
                      near_tol, near_cap, 0, near.ctypes.data, nnear.ctypes.data)
        levels = np.zeros(nlev, LEVEL_DTYPE)
        anc = np.zeros((nlev, nc), np.int32)
        best = np.zeros(lay.chain_words, np.uint64)
        iout = np.zeros(4, np.int32)
        h1 = np.zeros(5, np.float64)
        self.lib.oracle_anneal(self.h, ctypes.byref(params), lay.W, lay.ch_off, lay.s_off, lay.chain_words,
                               pop.ctypes.data, nc, ctypes.byref(a), levels.ctypes.data, anc.ctypes.data,
                               best.ctypes.data, iout.ctypes.data, h1.ctypes.data)
        return {"levels": levels, "anc": anc, "best_rec": best, "best_chain": int(iout[0]), "nresample": int(iout[1]),
                "staged": bool(iout[2]), "total_sweeps": int(iout[3]), "h1": h1, "near": near[:int(nnear[0])]}

    def repair(self, lay, rec, sc_target):
        """Final greedy slice repair of rec's tree, S updated in place; returns the labels added."""
        assert rec.dtype == np.uint64 and rec.flags.c_contiguous
        return self.lib.oracle_repair(self.h, lay.W, lay.ch_off, lay.s_off, lay.chain_words, rec.ctypes.data,
                                      float(sc_target))

    def __del__(self):
        try:
            self.lib.oracle_free(self.h)
        except Exception:
            pass


def philox(ctr, k0, k1):
    lib = load()
    c = np.array(ctr, np.uint32)
    out = np.zeros(4, np.uint32)
    lib.oracle_philox(c.ctypes.data, k0, k1, out.ctypes.data)
    return [int(x) for x in out]


def random_tree(m, seed):
    out = np.zeros(m - 1, np.uint32)
    load().oracle_random_tree(m, seed, out.ctypes.data)
    return out


def lse_table():
    out = np.zeros(64, np.float32)
    load().oracle_lse_table(out.ctypes.data)
    return out


def read_instance_py(path):
    """Plain-Python reader of the instance format (m nlab / k l.. / ny y..), independent of the host layer."""
    with open(path) as f:
        tok = f.read().split()
    it = iter(tok)
    m, nlab = int(next(it)), int(next(it))
    ixs = []
    for _ in range(m):
        k = int(next(it))
        ixs.append(sorted(int(next(it)) for _ in range(k)))
    iy = []
    try:
        ny = int(next(it))
        iy = [int(next(it)) for _ in range(ny)]
    except StopIteration:
        pass
    return m, nlab, ixs, iy


def read_trees_py(path, m):
    with open(path) as f:
        vals = [int(x) for x in f.read().split()]
    per = 2 * (m - 1)
    assert len(vals) % per == 0
    out = []
    for k in range(len(vals) // per):
        v = vals[k * per:(k + 1) * per]
        out.append(np.array([v[2 * i] | (v[2 * i + 1] << 16) for i in range(m - 1)], np.uint32))
    return np.array(out, np.uint32)


def systematic(E, db, u):
    E = np.ascontiguousarray(E, np.float64)
    out = np.zeros(len(E), np.int32)
    load().oracle_systematic(E.ctypes.data, len(E), float(db), float(u), out.ctypes.data)
    return out


def truncation(E, frac):
    E = np.ascontiguousarray(E, np.float64)
    out = np.zeros(len(E), np.int32)
    load().oracle_truncation(E.ctypes.data, len(E), float(frac), out.ctypes.data)
    return out


def score(mode, lc, sc, ns, slicing=False, select_sc=False, sc_target=20.0, sc_weight=1.0, energy=False):
    return load().oracle_score(mode, 1 if slicing else 0, 1 if select_sc else 0, float(sc_target), float(sc_weight),
                               float(lc), int(sc), int(ns), 1 if energy else 0)


def pa_uniforms(seed, n):
    out = np.zeros(n, np.float64)
    load().oracle_pa_uniforms(seed, n, out.ctypes.data)
    return out


def set_variant(v, noise_seed=0):
    """Rounding variant of the oracle's float lse (0: the reference's arithmetic; see oracle_set_variant)."""
    load().oracle_set_variant(int(v), int(noise_seed))


def fnv64_bytes(a):
    """FNV-1a of an array's bytes, as the reference harness hashes a chain's label sets (hex string)."""
    a = np.ascontiguousarray(a)
    return "%016x" % load().oracle_fnv64(a.ctypes.data, a.nbytes)
