"""The slice move's proposal rule and chain energy, brute-forced on small networks (m <= 8 tensors).

For random instances, random trees and random slice sets, an independent enumeration -- every internal node's
label set computed from its subtree (labels of the subtree's leaves that also occur outside it or are open),
its size outside S, the nodes of maximal size in node-id order, S's labels in id order -- predicts what the
slice move of csrc/treesa_gpu.cu:445-502 proposes for a word r1: the move type (add when |S| = 0; remove or
swap at max_slices; else add / remove / swap by r1.x's top bits), the node r1.y picks among the largest ones,
the label r1.z picks among its unsliced labels and the label r1.w picks among the sliced ones.  The oracle's
proposal (the one the sweep kernels are checked against, bit for bit, by the GPU parity tests) must equal it.
The same enumeration gives E = |S| + log2 sum_v 2^cost(v) in double (tc costs |z| + |x & y & ~z| outside S)
and the oracle's 32-lane float fold must lie within the fold's rounding bound of it.
"""
import math
import random

import numpy as np
import pytest

import oracle as orc
from treesa_gpu_amd import capi


def random_instance(rng, m):
    nlab = rng.randint(m, 3 * m)
    ixs = [sorted(rng.sample(range(nlab), rng.randint(1, min(5, nlab)))) for _ in range(m)]
    used = sorted({l for ix in ixs for l in ix})
    remap = {l: i for i, l in enumerate(used)}
    ixs = [[remap[l] for l in ix] for ix in ixs]
    nlab = len(used)
    iy = sorted(rng.sample(range(nlab), rng.randint(0, min(2, nlab))))
    return nlab, ixs, iy


def random_tree(rng, m):
    """Internal nodes m .. 2m-2 in creation order, children words l | r << 16."""
    live = list(range(m))
    ch = []
    for k in range(m - 1):
        a, b = rng.sample(live, 2)
        live.remove(a)
        live.remove(b)
        ch.append(a | (b << 16))
        live.append(m + k)
    return np.array(ch, np.uint32)


def brute(m, nlab, ixs, iy, ch, S, r1, max_slices):
    kids = {m + k: (int(w) & 0xFFFF, int(w) >> 16) for k, w in enumerate(ch)}
    leaves = {}

    def under(v):
        if v < m:
            return {v}
        if v not in leaves:
            a, b = kids[v]
            leaves[v] = under(a) | under(b)
        return leaves[v]

    def labels(v):
        inside = set().union(*(set(ixs[i]) for i in under(v)))
        outside = set().union(*(set(ixs[i]) for i in range(m) if i not in under(v)), set())
        return {l for l in inside if l in outside or l in iy}

    lab = {v: labels(v) for v in range(2 * m - 1)}
    Z = {v: len(lab[v] - S) for v in range(m, 2 * m - 1)}
    sc_int = max(Z.values())
    cands = [v for v in range(m, 2 * m - 1) if Z[v] == sc_int]
    ns = len(S)
    a, b, c, d = r1
    if ns == 0:
        typ = 0
    elif ns >= max_slices:
        typ = 1 if a >> 31 else 2
    else:
        typ = 0 if a < 0x80000000 else (1 if a < 0xC0000000 else 2)
    ladd = lrem = -1
    if typ != 1 and cands and sc_int > 0:
        node = cands[b % len(cands)]
        ladd = sorted(lab[node] - S)[c % sc_int]
    if typ != 0:
        lrem = sorted(S)[d % ns]
    if typ == 2 and ladd < 0:
        typ = 1
    if typ == 0 and ladd < 0:
        typ = -1
    # tc costs of every contraction outside S, and E's log2-sum in double
    costs = []
    for v in range(m, 2 * m - 1):
        x, y = kids[v]
        z = lab[v] - S
        k = len((lab[x] & lab[y]) - lab[v] - S)
        costs.append(len(z) + k)
    mx = max(costs)
    lsum = mx + math.log2(sum(2.0 ** (q - mx) for q in costs))
    return dict(type=typ, ladd=ladd, lrem=lrem, sc_int=sc_int, ncand=len(cands), ns=ns), lsum


@pytest.mark.parametrize("m", [3, 4, 5, 6, 7, 8])
def test_slice_proposal_and_energy_by_enumeration(m):
    rng = random.Random(1000 + m)
    checked = moves = 0
    for trial in range(60):
        nlab, ixs, iy = random_instance(rng, m)
        O = orc.Oracle(m, nlab, ixs, iy)
        lay = capi.layout(m, nlab)
        cfg = capi.make_config(mode="tc", sc_target=1000.0, seed=1, slicing=True, slice_moves=1)
        P = orc.params_from_config(cfg, max(len(x) for x in ixs), nlab)
        if trial % 3 == 0:
            P.max_slices = rng.randint(1, max(1, nlab // 2))
        for _ in range(4):
            ch = random_tree(rng, m)
            lab = O.labels(ch, lay.W)
            assert lab is not None
            S = set(rng.sample(range(nlab), rng.randint(0, min(P.max_slices, nlab))))
            rec = np.zeros(lay.chain_words, np.uint64)
            rec[:lay.nint * lay.W] = lab.reshape(-1)
            rec[lay.ch_off:].view(np.uint32)[:m - 1] = ch
            for l in S:
                rec[lay.s_off + (l >> 6)] |= np.uint64(1) << np.uint64(l & 63)
            for _ in range(6):
                r1 = [rng.getrandbits(32) for _ in range(4)]
                got = O.slice_propose(P, lay, rec, r1)
                want, lsum = brute(m, nlab, ixs, iy, ch, S, r1, P.max_slices)
                assert {k: got[k] for k in want} == want, (m, trial, r1, got, want)
                # the float fold of m-1 costs (at most log2(2m) in magnitude above the largest) against double
                tol = 4 * m * 2.0 ** (math.frexp(max(abs(lsum), 1.0))[1] - 24)
                assert abs(got["lcost"] - lsum) <= tol, (got["lcost"], lsum)
                checked += 1
                moves += got["type"] >= 0
    assert checked == 60 * 4 * 6 and moves > checked // 2
