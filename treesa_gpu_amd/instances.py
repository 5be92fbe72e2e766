"""Benchmark instances of the reference, generated the same way.

* random_ksat / sat(n): random k-SAT clause networks, one tensor per clause over its variables, scalar output.
  Same random calls as the reference's generator (bench/instances.py:10-16, 41-43; Python's random.Random(seed),
  sample k distinct variables, one sign draw per variable), so sat(40), sat(60), sat(100) equal the reference's
  committed tests/data instances after the driver's first-appearance label map (treesa_gpu/driver.py:60-77).
* sq(L): the L x L open-boundary lattice graph network, one tensor per site, one label per edge, edges numbered
  site by site (x major), vertical before horizontal (bench/large_compare.py:25-35).
* reg3(n, seed): a random 3-regular graph from a seeded configuration model (pair up 3n stubs uniformly, restart
  when a self-loop or multi-edge appears), one tensor per vertex over its three edge labels, edges numbered in
  pairing order.  (The reference draws its large 3-regular graphs with networkx, bench/large_compare.py:38-44;
  no such instance is committed, so this generator is this build's own and the instance is not the reference's.)
"""
import random

import numpy as np


def random_ksat(n, m, k, seed=0):
    rng = random.Random(seed)
    clauses = []
    for _ in range(m):
        vs = rng.sample(range(1, n + 1), k)
        clauses.append([v if rng.random() < 0.5 else -v for v in vs])
    return clauses


def sat(n, seed=1, alpha=4.26, k=3):
    """(ixs, iy) of random k-SAT with n variables and round(alpha n) clauses, labels = variables - 1."""
    clauses = random_ksat(n, round(alpha * n), k, seed)
    return [[abs(l) - 1 for l in c] for c in clauses], []


def sq(L):
    lab = {}
    ixs = [[] for _ in range(L * L)]
    for x in range(L):
        for y in range(L):
            v = x * L + y
            for u in ((x + 1) * L + y if x + 1 < L else None, x * L + y + 1 if y + 1 < L else None):
                if u is not None:
                    e = len(lab)
                    lab[(v, u)] = e
                    ixs[v].append(e)
                    ixs[u].append(e)
    return ixs, []


def reg3(n, seed=1):
    rng = np.random.default_rng(seed)
    while True:
        stubs = np.repeat(np.arange(n), 3)
        rng.shuffle(stubs)
        pairs = stubs.reshape(-1, 2)
        a, b = np.minimum(pairs[:, 0], pairs[:, 1]), np.maximum(pairs[:, 0], pairs[:, 1])
        if np.any(a == b):
            continue
        key = a.astype(np.int64) * n + b
        if len(np.unique(key)) != len(key):
            continue
        break
    ixs = [[] for _ in range(n)]
    for e, (u, v) in enumerate(zip(a.tolist(), b.tolist())):
        ixs[u].append(e)
        ixs[v].append(e)
    return ixs, []


def label_map(ixs, iy):
    """Labels renumbered 0..L-1 in order of first appearance (treesa_gpu/driver.py:60-67)."""
    mp = {}
    for ix in list(ixs) + [iy]:
        for l in ix:
            if l not in mp:
                mp[l] = len(mp)
    return mp


def instance_text(ixs, iy):
    """The instance file the driver writes (treesa_gpu/driver.py:70-77)."""
    mp = label_map(ixs, iy)
    lines = [f"{len(ixs)} {len(mp)}"]
    for ix in ixs:
        lines.append(" ".join([str(len(ix))] + [str(mp[l]) for l in ix]))
    lines.append(" ".join([str(len(iy))] + [str(mp[l]) for l in iy]))
    return "\n".join(lines) + "\n"
