"""The final greedy slice repair, pinned by enumeration on small networks (m <= 9 tensors).

The rule (csrc/treesa_gpu.cu:1248-1274): while the largest tensor of the tree outside S -- the m input tensors
and the m-1 contraction results -- has more than sc_target labels (and at least one), add to S the label that
occurs in the most tensors of that largest size, the lowest label id on ties.

An independent statement computes every tensor's label set from first principles (a leaf: its own labels; an
internal node: the labels of its subtree's leaves that also occur outside the subtree or are open), then runs
that loop with Python sets.  The oracle's restatement (oracle_repair, the checker of the binary's n_repair and
sliced set) and the host layer's word-wise repair (greedy_repair, what bin/treesa_gpu runs) must both add the
same labels in the same number.  The trials cover repairs of one to many labels, leaves that are the largest
tensor, ties between labels, fractional targets, a target of zero and a negative one (every label is cut);
planted mistakes in the enumeration (leaves left out, ties to the highest id, counts over every tensor instead
of the largest, the stop test with < instead of <=, the zero-size stop dropped) each disagree with the oracle
on some trial.
"""
import random

import numpy as np
import pytest

import oracle as orc
from treesa_gpu_amd import capi
from treesa_gpu_amd import host


def random_instance(rng, m):
    nlab = rng.randint(m, 3 * m)
    ixs = [sorted(rng.sample(range(nlab), rng.randint(1, min(6, nlab)))) for _ in range(m)]
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


def tensor_sets(m, ixs, iy, ch):
    """Label set of every tensor 0 .. 2m-2 of the tree, from its subtree's leaves."""
    kids = {m + k: (int(w) & 0xFFFF, int(w) >> 16) for k, w in enumerate(ch)}
    under = {v: {v} for v in range(m)}
    for v in range(m, 2 * m - 1):
        a, b = kids[v]
        under[v] = under[a] | under[b]
    sets = {v: set(ixs[v]) for v in range(m)}
    for v in range(m, 2 * m - 1):
        inside = set().union(*(set(ixs[i]) for i in under[v]))
        outside = set().union(set(), *(set(ixs[i]) for i in range(m) if i not in under[v]))
        sets[v] = {l for l in inside if l in outside or l in iy}
    return sets


def enumerate_repair(sets, S, sc_target, mistake=None):
    """The labels the repair adds, in order, and whether a leaf was ever the only largest tensor."""
    S = set(S)
    added = []
    leaf_top = False
    tensors = sorted(sets)
    while True:
        size = {v: len(sets[v] - S) for v in tensors}
        pool = [v for v in tensors if mistake != "no_leaves" or v >= len(tensors) // 2 + 1]
        top = max(size[v] for v in pool)
        stop = top < sc_target if mistake == "lt" else top <= sc_target
        if (top == 0 and mistake != "no_zero_stop") or stop:
            return added, leaf_top
        if top == 0:
            return added + ["loop"], leaf_top
        largest = [v for v in pool if size[v] == top]
        if all(v < len(tensors) // 2 + 1 for v in largest):
            leaf_top = True
        hits = {}
        for v in (pool if mistake == "all_tensors" else largest):
            for l in sets[v] - S:
                hits[l] = hits.get(l, 0) + 1
        best = max(hits.values())
        ties = [l for l in hits if hits[l] == best]
        pick = max(ties) if mistake == "high_tie" else min(ties)
        S.add(pick)
        added.append(pick)


def bits(labels, W):
    out = np.zeros(W, np.uint64)
    for l in labels:
        out[l >> 6] |= np.uint64(1) << np.uint64(l & 63)
    return out


def labels_of(words, nlab):
    return {l for l in range(nlab) if (int(words[l >> 6]) >> (l & 63)) & 1}


MISTAKES = ("no_leaves", "high_tie", "all_tensors", "lt", "no_zero_stop")


def trials(seed, count):
    rng = random.Random(seed)
    for t in range(count):
        m = rng.randint(3, 9)
        nlab, ixs, iy = random_instance(rng, m)
        ch = random_tree(rng, m)
        S = set(rng.sample(range(nlab), rng.randint(0, nlab // 3)))
        kind = t % 5
        if kind == 0:
            sct = 0.0
        elif kind == 4:
            sct = -1.0
        elif kind == 1:
            sct = rng.randint(0, 3) + 0.5
        else:
            sct = float(rng.randint(0, 4))
        yield m, nlab, ixs, iy, ch, S, sct


def run_both(m, nlab, ixs, iy, ch, S, sct):
    """(labels the oracle adds, its count), (labels the host layer adds, its count)."""
    O = orc.Oracle(m, nlab, ixs, iy)
    lay = capi.layout(m, nlab)
    rec = np.zeros(lay.chain_words, np.uint64)
    lab = O.labels(ch, lay.W)
    assert lab is not None
    rec[:lay.nint * lay.W] = lab.reshape(-1)
    rec[lay.ch_off:].view(np.uint32)[:m - 1] = ch
    rec[lay.s_off:lay.s_off + lay.W] = bits(S, lay.W)
    k_or = O.repair(lay, rec, sct)
    got_or = labels_of(rec[lay.s_off:lay.s_off + lay.W], nlab)

    inst = host.Instance(m=m, nlab=nlab, ixs=ixs, iy=iy)
    hl = inst.labels(ch, lay.W)
    assert hl is not None and np.array_equal(hl, lab)
    Sh = bits(S, lay.W)
    k_h = inst.greedy_repair(hl, Sh, sct)
    got_h = labels_of(Sh, nlab)
    inst.close()
    return (got_or, k_or), (got_h, k_h)


def test_repair_matches_enumeration():
    n = many = leafy = ties = 0
    for m, nlab, ixs, iy, ch, S, sct in trials(2024, 600):
        sets = tensor_sets(m, ixs, iy, ch)
        want, leaf_top = enumerate_repair(sets, S, sct)
        (got_or, k_or), (got_h, k_h) = run_both(m, nlab, ixs, iy, ch, S, sct)
        assert k_or == len(want) and got_or == S | set(want), (m, ixs, iy, list(ch), S, sct, want, k_or, got_or)
        assert k_h == len(want) and got_h == S | set(want), (m, ixs, iy, list(ch), S, sct, want, k_h, got_h)
        # ties: some step where the chosen label shares the top count with a higher id
        Sx = set(S)
        for l in want:
            size = {v: len(sets[v] - Sx) for v in sets}
            top = max(size.values())
            hits = {}
            for v in sets:
                if size[v] == top:
                    for q in sets[v] - Sx:
                        hits[q] = hits.get(q, 0) + 1
            if sum(1 for q in hits if hits[q] == hits[l]) > 1:
                ties += 1
                break
            Sx.add(l)
        n += 1
        many += len(want) >= 3
        leafy += leaf_top
    # the trials exercise what the rule distinguishes
    print(f"{n} trials: {many} add 3 or more labels, {leafy} have a leaf as the only largest tensor, {ties} tie")
    assert n == 600 and many >= 100 and leafy >= 20 and ties >= 100, (n, many, leafy, ties)


@pytest.mark.parametrize("mistake", MISTAKES)
def test_planted_mistakes_are_caught(mistake):
    """Each planted mistake in the enumeration disagrees with the oracle on at least one trial."""
    caught = 0
    for m, nlab, ixs, iy, ch, S, sct in trials(77, 300):
        sets = tensor_sets(m, ixs, iy, ch)
        bad, _ = enumerate_repair(sets, S, sct, mistake=mistake)
        (got_or, k_or), _ = run_both(m, nlab, ixs, iy, ch, S, sct)
        if k_or != len(bad) or got_or != S | {x for x in bad if x != "loop"}:
            caught += 1
    assert caught > 0, mistake


def test_repair_of_an_all_sliced_tree_is_empty():
    """Every label already in S: the largest size is 0 and nothing is added whatever the target."""
    rng = random.Random(5)
    nlab, ixs, iy = random_instance(rng, 6)
    ch = random_tree(rng, 6)
    (got_or, k_or), (got_h, k_h) = run_both(6, nlab, ixs, iy, ch, set(range(nlab)), -1.0)
    assert k_or == 0 and k_h == 0 and got_or == got_h == set(range(nlab))
