"""Start trees for the annealer, as children words (internal node m+i: left | right << 16, root 2m-2).

* path_tree(order): contract the tensors left to right: node m+0 = (order[0], order[1]), node m+i =
  (m+i-1, order[i+1]) -- the reference's row-major "sweep" tree for lattices (bench/large_compare.py:59-63
  through the post-order numbering of treesa_gpu/driver.py:80-95).
* path_cost(order): exact (tc, sc) of that path tree in O(sum of tensor sizes): step i contracts the prefix's
  surviving labels with tensor i, and for dimension-2 indices its cost is the size of the union of the two
  label sets (B + M + N + K = |x u y| because every label of x u y is either kept or shared).
* greedy_tree: repeatedly contract the pair of tensors that share a label and give the smallest result,
  outer products of the two smallest tensors when nothing is shared -- the loss of OMEinsumContractionOrders'
  GreedyMethod with alpha = 0 -- best of nrepeat runs with seeded random tie-breaking (the reference takes its
  greedy trees from omeco, treesa_gpu/driver.py:117-122; its committed greedy trees are the fixtures used
  wherever they exist).
* spectral_orders: linear orderings from the low Laplacian eigenvectors of the tensor graph (one vertex per
  tensor, one edge weight per shared label), candidates along directions in the span of eigenvectors 1-3,
  each scored exactly with path_cost; the k best distinct ones (the idea of treesa_gpu/spectral.py:1-15, this
  build's own candidate set and weighting).
"""
import heapq
import math

import numpy as np


def path_tree(order):
    order = [int(x) for x in order]
    m = len(order)
    ch = np.zeros(m - 1, np.uint32)
    for i in range(m - 1):
        left = order[0] if i == 0 else m + i - 1
        ch[i] = left | (order[i + 1] << 16)
    return ch


def path_cost(order, ixs, iy=()):
    m = len(order)
    pos = np.empty(m, np.int64)
    pos[np.asarray(order)] = np.arange(m)
    first, last = {}, {}
    for t, ix in enumerate(ixs):
        p = int(pos[t])
        for l in ix:
            first[l] = min(first.get(l, p), p)
            last[l] = max(last.get(l, p), p)
    for l in iy:
        if l in last:
            last[l] = m  # open labels never die
    alive = np.zeros(m + 1, np.int64)  # alive[i]: labels with first <= i < last
    newc = np.zeros(m, np.int64)
    for l in first:
        f, la = first[l], last[l]
        newc[f] += 1
        if la > f:
            alive[f] += 1
            alive[la] -= 1
    alive = np.cumsum(alive)
    cost = []
    for i in range(1, m):
        if i == 1:
            cost.append(len(set(ixs[order[0]]) | set(ixs[order[1]])))
        else:
            cost.append(int(alive[i - 1] + newc[i]))
    outs = [int(alive[i]) for i in range(1, m)]
    sc = max(outs + [len(ix) for ix in ixs])
    cm = max(cost)
    tc = cm + math.log2(sum(2.0 ** (c - cm) for c in cost))
    return tc, sc


def greedy_tree(ixs, iy=(), nrepeat=10, seed=0):
    """Best (lowest tc) of nrepeat greedy runs; run 0 breaks ties by discovery order, the others at random."""
    rng = np.random.default_rng(seed)
    best = None
    for r in range(nrepeat):
        ch, tc = _greedy_once(ixs, iy, rng if r > 0 else None)
        if best is None or tc < best[1]:
            best = (ch, tc)
    return best[0]


def _greedy_once(ixs, iy, rng):
    m = len(ixs)
    sets = {t: frozenset(ix) for t, ix in enumerate(ixs)}
    cnt = {}
    for ix in ixs:
        for l in ix:
            cnt[l] = cnt.get(l, 0) + 1
    open_ = set(iy)
    holders = {}
    for t, s in sets.items():
        for l in s:
            holders.setdefault(l, set()).add(t)

    def result(a, b):
        sa, sb = sets[a], sets[b]
        out = set()
        for l in sa | sb:
            inside = (l in sa) + (l in sb)
            # occurrences outside a and b: total minus the ones a and b hold (each tensor holds a label once)
            if l in open_ or cnt[l] - inside > 0:
                out.add(l)
        return frozenset(out)

    heap = []
    tick = 0

    def push(a, b):
        nonlocal tick
        if a > b:
            a, b = b, a
        heapq.heappush(heap, (len(result(a, b)), rng.random() if rng is not None else 0.0, tick, a, b))
        tick += 1

    for l in sorted(holders):
        hs = sorted(holders[l])
        for i in range(len(hs)):
            for j in range(i + 1, len(hs)):
                push(hs[i], hs[j])
    alive = set(range(m))
    ch = []
    costs = []
    nxt = m
    while len(alive) > 1:
        pair = None
        while heap:
            _, _, _, a, b = heapq.heappop(heap)
            if a in alive and b in alive:
                pair = (a, b)
                break
        if pair is None:  # disconnected: outer product of the two smallest
            a, b = sorted(alive, key=lambda t: (len(sets[t]), t))[:2]
            pair = (a, b)
        a, b = pair
        out = result(a, b)
        costs.append(len(sets[a] | sets[b]))
        for l in sets[a] | sets[b]:
            cnt[l] -= (l in sets[a]) + (l in sets[b])
            holders[l].discard(a)
            holders[l].discard(b)
        for l in out:
            cnt[l] += 1
            holders[l].add(nxt)
        sets[nxt] = out
        alive -= {a, b}
        alive.add(nxt)
        ch.append(a | (b << 16))
        nbrs = set()
        for l in out:
            nbrs |= holders[l]
        nbrs.discard(nxt)
        for t in sorted(nbrs):
            push(t, nxt)
        nxt += 1
    cm = max(costs)
    return np.array(ch, np.uint32), cm + math.log2(sum(2.0 ** (c - cm) for c in costs))


def spectral_orders(ixs, iy=(), k=4, nangles=32, nrandom=16, seed=0):
    """The k best distinct orderings: list of (tc, sc, order), best first."""
    n = len(ixs)
    holders = {}
    for t, ix in enumerate(ixs):
        for l in ix:
            holders.setdefault(l, []).append(t)
    A = np.zeros((n, n))
    for ts in holders.values():
        for i in range(len(ts)):
            for j in range(i + 1, len(ts)):
                A[ts[i], ts[j]] += 1.0
                A[ts[j], ts[i]] += 1.0
    Lap = np.diag(A.sum(axis=1)) - A
    _, V = np.linalg.eigh(Lap)
    V = V[:, 1:4]
    rng = np.random.default_rng(seed)
    dirs = [np.array([math.cos(math.pi * a / nangles), math.sin(math.pi * a / nangles), 0.0]) for a in range(nangles)]
    for _ in range(nrandom):
        v = rng.standard_normal(3)
        dirs.append(v / np.linalg.norm(v))
    seen, cands = set(), []
    for d in dirs:
        o = np.argsort(V @ d, kind="stable")
        for oo in (o, o[::-1]):
            key = oo.tobytes()
            if key in seen:
                continue
            seen.add(key)
            tc, sc = path_cost(oo, ixs, iy)
            cands.append((tc, sc, [int(x) for x in oo]))
    cands.sort(key=lambda c: (c[0], c[1]))
    return cands[:k]


def write_trees(path, trees):
    with open(path, "w") as f:
        for t in trees:
            for w in t:
                f.write(f"{int(w) & 0xFFFF} {int(w) >> 16}\n")
