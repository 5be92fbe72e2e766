"""Start trees for the annealer, computed by the native host library (lib/libtreesa_host.so,
treesa_gpu_amd/host/tsa_starts.cpp).  Trees are children words (internal node m+i: left | right << 16, root
2m-2).  The functions take the reference's arguments -- ixs (one label list per tensor, any hashable labels)
and iy (open labels) -- and return what its treesa_gpu/spectral.py returns:

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
import numpy as np

from . import host


def _instance(ixs, iy=()):
    ids = {}
    for ix in ixs:
        for l in ix:
            ids.setdefault(l, len(ids))
    for l in iy:
        ids.setdefault(l, len(ids))
    return host.Instance(m=len(ixs), nlab=max(1, len(ids)), ixs=[[ids[l] for l in ix] for ix in ixs],
                         iy=[ids[l] for l in iy])


def path_tree(order):
    return host.path_tree(order)


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
