"""ctypes binding of libtreesa_hip's host layer (lib/libtreesa_host.so): instance / tree / betas files,
topology labels, Julia random trees, the initial population and the double-precision energy.

These are the same C++ functions bin/treesa_gpu uses (treesa_gpu_amd/host/tsa_host.cpp); the reference's
host code they follow is csrc/treesa_gpu.cu:1027-1274, 1300-1328, 1585-1630.

Start trees (treesa_gpu_amd/host/tsa_starts.cpp) under the reference's Python signatures, which take ixs (one
label list per tensor, any hashable labels) and iy (open labels) and return what treesa_gpu/spectral.py returns;
trees are children words (internal node m+i: left | right << 16, root 2m-2):

* path_tree(order): contract the tensors left to right: node m+0 = (order[0], order[1]), node m+i =
  (m+i-1, order[i+1]) (treesa_gpu/spectral.py:129-134 as a nested dict; path_tree_dict gives that form).
* path_cost(order, ixs, iy): exact (tc, sc) of that path tree in O(sum of tensor sizes)
  (treesa_gpu/spectral.py:95-126).
* laplacian_vectors(ixs, k, seed): eigenvectors 1..k of the tensor graph's Laplacian and their eigenvalues
  (treesa_gpu/spectral.py:22-92).
* spectral_orders(ixs, iy, k, nangles, nrandom, seed): the k best distinct spectral orderings as
  (tc, sc, order), best first (treesa_gpu/spectral.py:136-199); spectral_search does the same candidate
  search over eigenvectors and random directions the caller gives.
* greedy_tree(ixs, iy, nrepeat, seed): the greedy contraction tree, in place of omeco's GreedyMethod
  (treesa_gpu/driver.py:117-122).
"""
import ctypes
import os

import numpy as np

from . import capi

_lib = None


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(capi.HOST_LIB_PATH):
        raise FileNotFoundError(f"{capi.HOST_LIB_PATH} is missing: build it with `make -C treesa_gpu_amd`")
    lib = ctypes.CDLL(capi.HOST_LIB_PATH)
    P, I, U64, D = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_double
    C = ctypes.c_char_p
    lib.tsh_instance_load.argtypes = [C, ctypes.c_char_p, I]
    lib.tsh_instance_load.restype = P
    lib.tsh_instance_make.argtypes = [I, I, P, P, I, P, ctypes.c_char_p, I]
    lib.tsh_instance_make.restype = P
    lib.tsh_instance_free.argtypes = [P]
    lib.tsh_instance_info.argtypes = [P, P, P, P]
    lib.tsh_instance_leaf.argtypes = [P, I, P]
    lib.tsh_read_trees.argtypes = [C, I, P, I, ctypes.c_char_p, I]
    lib.tsh_parse_betas.argtypes = [C, P, I, ctypes.c_char_p, I]
    lib.tsh_splitmix64.argtypes = [U64]
    lib.tsh_splitmix64.restype = U64
    lib.tsh_random_tree.argtypes = [I, U64, P]
    lib.tsh_labels.argtypes = [P, I, P, P]
    lib.tsh_build_population.argtypes = [P, I, I, I, I, P, I, I, U64, P, I, P, ctypes.c_char_p, I]
    lib.tsh_host_energy.argtypes = [P, I, P, P, P, P, P, P]
    lib.tsh_greedy_repair.argtypes = [P, I, P, P, D]
    lib.tsh_path_cost.argtypes = [P, P, I, P]
    lib.tsh_spectral_orders.argtypes = [P, I, I, I, U64, P, P, P]
    lib.tsh_spectral_search.argtypes = [P, P, I, P, I, I, I, P, P, P]
    lib.tsh_laplacian_vectors.argtypes = [P, I, U64, P, P]
    lib.tsh_greedy_tree.argtypes = [P, I, U64, P, P]
    _lib = lib
    return lib


class HostError(RuntimeError):
    pass


class Instance:
    """A tensor network read from the reference's instance format (or built from ixs / iy)."""

    def __init__(self, path=None, m=None, nlab=None, ixs=None, iy=()):
        self.lib = load()
        err = ctypes.create_string_buffer(512)
        if path is not None:
            h = self.lib.tsh_instance_load(path.encode(), err, 512)
        else:
            offs = np.zeros(m + 1, np.int32)
            for i, ix in enumerate(ixs):
                offs[i + 1] = offs[i] + len(ix)
            labs = np.array([l for ix in ixs for l in ix] or [0], np.int32)
            iya = np.array(list(iy) or [0], np.int32)
            h = self.lib.tsh_instance_make(m, nlab, offs.ctypes.data, labs.ctypes.data, len(iy), iya.ctypes.data, err,
                                           512)
        if not h:
            raise HostError(err.value.decode())
        self.h = h
        m_, n_, s_ = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        self.lib.tsh_instance_info(h, ctypes.byref(m_), ctypes.byref(n_), ctypes.byref(s_))
        self.m, self.nlab, self.leaf_sc = m_.value, n_.value, s_.value
        self.nint = self.m - 1

    def leaf(self, W):
        out = np.zeros((self.m, W), np.uint64)
        self.lib.tsh_instance_leaf(self.h, W, out.ctypes.data)
        return out

    def read_trees(self, path, maxk=64):
        out = np.zeros((maxk, self.nint), np.uint32)
        err = ctypes.create_string_buffer(512)
        k = self.lib.tsh_read_trees(path.encode(), self.m, out.ctypes.data, maxk, err, 512)
        if k < 0:
            raise HostError(err.value.decode())
        return out[:min(k, maxk)].copy()

    def labels(self, ch, W):
        ch = np.ascontiguousarray(ch, np.uint32)
        lab = np.zeros((self.nint, W), np.uint64)
        if self.lib.tsh_labels(self.h, W, ch.ctypes.data, lab.ctypes.data) != 0:
            return None
        return lab

    def population(self, lay, trees, nchains, seed=1, S0=None, random_slices=0):
        """Initial population in the C ABI record format (nchains x chain_words)."""
        trees = np.ascontiguousarray(trees if trees is not None and len(trees) else np.zeros((0, self.nint)),
                                     np.uint32)
        pop = np.zeros((nchains, lay.chain_words), np.uint64)
        s0 = None if S0 is None else np.ascontiguousarray(S0, np.uint64)
        err = ctypes.create_string_buffer(512)
        rc = self.lib.tsh_build_population(self.h, lay.W, lay.ch_off, lay.s_off, lay.chain_words, trees.ctypes.data,
                                           len(trees), nchains, seed, None if s0 is None else s0.ctypes.data,
                                           random_slices, pop.ctypes.data, err, 512)
        if rc != 0:
            raise HostError(err.value.decode())
        return pop

    def host_energy(self, lay, rec, slicing=False, gm=capi.DEFAULT_GM, h100=capi.DEFAULT_H100):
        """(tc, sc, gpu_time, h100_time, |S|) of one chain record, in double."""
        rec = np.ascontiguousarray(rec, np.uint64)
        g = np.array(gm, np.float64)
        h = np.array(h100, np.float64)
        out = np.zeros(5, np.float64)
        ch = rec[lay.ch_off:].view(np.uint32)
        S = rec[lay.s_off:lay.s_off + lay.W]
        self.lib.tsh_host_energy(self.h, lay.W, g.ctypes.data, h.ctypes.data, rec.ctypes.data, ch.ctypes.data,
                                 S.ctypes.data if slicing else None, out.ctypes.data)
        return float(out[0]), int(out[1]), float(out[2]), float(out[3]), int(out[4])

    def greedy_repair(self, lab, S, sc_target):
        """Final slice repair (csrc/treesa_gpu.cu:1248-1274) of a tree given by its internal label sets lab
        (nint x W words): while the largest tensor outside S (leaves included) exceeds sc_target, add the label
        that occurs in most of the largest tensors (lowest id on ties).  S (W words) is updated in place;
        returns the number of labels added."""
        lab = np.ascontiguousarray(lab, np.uint64)
        assert S.dtype == np.uint64 and S.flags.c_contiguous
        return self.lib.tsh_greedy_repair(self.h, S.shape[-1], lab.ctypes.data, S.ctypes.data, float(sc_target))

    def path_cost(self, order):
        """(tc, sc) of the path tree contracting the tensors in `order` left to right."""
        o = np.ascontiguousarray(order, np.int32)
        out = np.zeros(2, np.float64)
        if self.lib.tsh_path_cost(self.h, o.ctypes.data, len(o), out.ctypes.data) != 0:
            raise HostError("path_cost: the order must list every tensor")
        return float(out[0]), int(out[1])

    def laplacian_vectors(self, k, seed=1):
        """Eigenvectors 1..k of the tensor graph's Laplacian (m x k) and their eigenvalues."""
        vecs = np.zeros((self.m, k), np.float64)
        vals = np.zeros(k, np.float64)
        kk = self.lib.tsh_laplacian_vectors(self.h, k, seed, vecs.ctypes.data, vals.ctypes.data)
        return vecs[:, :kk].copy(), vals[:kk].copy()

    def spectral_orders(self, k=4, nangles=64, nrandom=64, seed=1):
        """The k best spectral orderings as a list of (tc, sc, order), best first."""
        orders = np.zeros((k, self.m), np.int32)
        tc = np.zeros(k, np.float64)
        sc = np.zeros(k, np.int32)
        n = self.lib.tsh_spectral_orders(self.h, k, nangles, nrandom, seed, orders.ctypes.data, tc.ctypes.data,
                                         sc.ctypes.data)
        return [(float(tc[i]), int(sc[i]), orders[i].copy()) for i in range(n)]

    def spectral_search(self, V, dirs, k=8, nangles=24):
        """spectral_orders' candidate search over given eigenvectors V (m x d) and directions dirs (r x d)."""
        V = np.ascontiguousarray(V, np.float64)
        d = V.shape[1]
        dirs = np.ascontiguousarray(np.reshape(dirs, (-1, d)), np.float64)
        orders = np.zeros((k, self.m), np.int32)
        tc = np.zeros(k, np.float64)
        sc = np.zeros(k, np.int32)
        n = self.lib.tsh_spectral_search(self.h, V.ctypes.data, d, dirs.ctypes.data, len(dirs), k, nangles,
                                         orders.ctypes.data, tc.ctypes.data, sc.ctypes.data)
        return [(float(tc[i]), int(sc[i]), orders[i].copy()) for i in range(n)]

    def greedy_tree(self, nrepeat=1, seed=1):
        """(children words, tc) of the greedy contraction tree, best of nrepeat runs."""
        out = np.zeros(self.m - 1, np.uint32)
        tc = ctypes.c_double()
        self.lib.tsh_greedy_tree(self.h, nrepeat, seed, out.ctypes.data, ctypes.byref(tc))
        return out, tc.value

    def close(self):
        if self.h:
            self.lib.tsh_instance_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def parse_betas(spec):
    lib = load()
    n = 1 << 16
    out = np.zeros(n, np.float32)
    err = ctypes.create_string_buffer(512)
    k = lib.tsh_parse_betas(spec.encode(), out.ctypes.data, n, err, 512)
    if k < 0:
        raise HostError(err.value.decode())
    return out[:k].copy()


def path_tree(order):
    """Children words of the path tree over `order`: node m = (order[0], order[1]), node m+i = (m+i-1, order[i+1])."""
    o = np.asarray(order, np.uint32)
    m = len(o)
    left = np.concatenate([o[:1], np.arange(m, 2 * m - 2, dtype=np.uint32)])
    return left | (o[1:] << np.uint32(16))


def random_tree(m, seed):
    out = np.zeros(m - 1, np.uint32)
    load().tsh_random_tree(m, seed, out.ctypes.data)
    return out


def splitmix64(x):
    return int(load().tsh_splitmix64(x))


# start trees under the reference's Python signatures (see the module docstring)
def _instance(ixs, iy=()):
    ids = {}
    for ix in ixs:
        for l in ix:
            ids.setdefault(l, len(ids))
    for l in iy:
        ids.setdefault(l, len(ids))
    return Instance(m=len(ixs), nlab=max(1, len(ids)), ixs=[[ids[l] for l in ix] for ix in ixs],
                    iy=[ids[l] for l in iy])


def path_tree_dict(order):
    """The path tree as the reference's nested dict ({"args": [l, r]} / {"tensor_index": i})."""
    t = {"tensor_index": int(order[0])}
    for i in order[1:]:
        t = {"args": [t, {"tensor_index": int(i)}]}
    return t


def path_cost(order, ixs, iy=()):
    return _instance(ixs, iy).path_cost(order)


def laplacian_vectors(ixs, k=3, seed=0):
    return _instance(ixs).laplacian_vectors(k, seed)


def spectral_orders(ixs, iy=(), k=8, nangles=24, nrandom=24, seed=0):
    n = len(ixs)
    if n < 3:
        return [(0.0, max((len(ix) for ix in ixs), default=0), list(range(n)))]
    return [(t, s, [int(x) for x in o]) for t, s, o in _instance(ixs, iy).spectral_orders(k, nangles, nrandom, seed)]


def spectral_search(ixs, iy, V, dirs, k=8, nangles=24):
    """spectral_orders' candidate search over the eigenvectors V (n x d) and random unit directions dirs
    (r x d) given by the caller."""
    return [(t, s, [int(x) for x in o]) for t, s, o in _instance(ixs, iy).spectral_search(V, dirs, k, nangles)]


def greedy_tree(ixs, iy=(), nrepeat=10, seed=0):
    return _instance(ixs, iy).greedy_tree(nrepeat, seed)[0]


def write_trees(path, trees):
    with open(path, "w") as f:
        for t in trees:
            for w in t:
                f.write(f"{int(w) & 0xFFFF} {int(w) >> 16}\n")
