"""CPU tests of the tree and result formats (treesa_gpu_amd/formats.py).

* Known answers: the complexity of the reference's committed omeco greedy trees equals the values its own
  test printed (tests/test_python_results.txt:1,15,29,43 -- "trees == omeco complexity (GreedyMethod: ...)").
* dict <-> children conversion round-trips (tests/test_python.py:44-47), also on path trees of 4096 tensors;
  recompute_outputs is idempotent on converted trees.
* Closed forms: tc and sc of a path tree equal the prefix-cut formula (starts.path_cost), the model times of
  a tree equal the host layer's double computation (host_energy), with and without sliced labels, and
  result_tree reads a result the way the driver does (tests/test_python.py:86-87 for runner_json).
"""
import json
import os
import re

import numpy as np
import pytest

import common
from treesa_gpu_amd import capi, host
from treesa_gpu_amd import formats as F
from treesa_gpu_amd import host as S

PAT = re.compile(r"ok   (\w+): trees == omeco complexity \(GreedyMethod: ([\d.]+)/(\d+)\)")


def greedy_known():
    out = []
    with open(os.path.join(common.HERE, "golden", "test_python_results_par.txt")) as f:
        for line in f:
            m = PAT.match(line)
            if m:
                out.append((m.group(1), float(m.group(2)), int(m.group(3))))
    return out


def pairs(ch):
    return [(int(w) & 0xFFFF, int(w) >> 16) for w in ch]


@pytest.mark.parametrize("name,tc,sc", greedy_known())
def test_complexity_of_omeco_trees_matches_reference_output(name, tc, sc):
    m, nlab, ixs, iy = common.load_instance(name)
    inst = host.Instance(common.inst_path(name))
    ch = pairs(inst.read_trees(common.tree_file(name, "greedy"))[0])
    d = F.children_to_dict(ch, m, ixs, iy)
    t, s = F.complexity(d, ixs)
    assert round(t, 3) == tc and s == sc
    assert F.dict_to_children(d, m) == ch
    assert F.recompute_outputs(d, ixs, iy) == d
    assert sorted(F.leaf_ids(d)) == list(range(m))


@pytest.mark.parametrize("name", ["sat40", "reg3_100", "lat10", "sq64"])
def test_round_trip_and_path_cost(name):
    m, nlab, ixs, iy = common.load_instance(name)
    rng = np.random.default_rng(11)
    for order in (np.arange(m), rng.permutation(m)):
        ch = pairs(S.path_tree(order))
        d = F.children_to_dict(ch, m, ixs, iy)  # m - 1 levels deep
        assert F.dict_to_children(d, m) == ch
        t, s = F.complexity(d, ixs)
        t2, s2 = S.path_cost(order, ixs, iy)
        assert abs(t - t2) < 1e-9 and s == s2
    d = S.path_tree_dict(list(range(m)))  # the reference's path dict: no "eins" until recomputed
    assert F.dict_to_children(d, m) == pairs(S.path_tree(list(range(m))))


def relabel(ch, m, rng):
    """The same tree with its internal nodes renumbered at random (root kept last), as the annealer's records
    hold them: a child may have a larger id than its parent."""
    perm = list(range(m, 2 * m - 2))
    rng.shuffle(perm)
    mp = {old: new for old, new in zip(range(m, 2 * m - 2), perm)}
    mp[2 * m - 2] = 2 * m - 2
    out = [None] * (m - 1)
    for i, (l, r) in enumerate(ch):
        out[mp[m + i] - m] = (mp.get(l, l), mp.get(r, r))
    return out


@pytest.mark.parametrize("name", ["sat40", "lat10"])
def test_children_in_any_order(name):
    m, nlab, ixs, iy = common.load_instance(name)
    rng = np.random.default_rng(3)
    ch = pairs(host.random_tree(m, 9))
    ch2 = relabel(ch, m, rng)
    assert any(max(l, r) > m + i for i, (l, r) in enumerate(ch2))
    d, d2 = F.children_to_dict(ch, m, ixs, iy), F.children_to_dict(ch2, m, ixs, iy)
    assert d == d2 and F.dict_to_children(d2, m) == F.dict_to_children(d, m)
    bad = list(ch2)
    bad[0] = (bad[1][0], bad[0][1])  # a subtree shared by two parents
    with pytest.raises(ValueError):
        F.children_to_dict(bad, m, ixs, iy)


def test_dict_to_children_rejects_bad_trees():
    with pytest.raises(ValueError):
        F.dict_to_children({"args": [{"tensor_index": 0}, {"tensor_index": 0}]}, 2)
    with pytest.raises(ValueError):
        F.dict_to_children({"args": [{"tensor_index": 0}, {"tensor_index": 1}]}, 3)


def test_small_trees():
    ixs, iy = [["a", "b"], ["b", "c"], ["c", "a"]], ["a"]
    d = F.children_to_dict([(0, 1), (3, 2)], 3, ixs, iy)
    assert d["eins"]["ixs"] == [["a", "c"], ["c", "a"]] and d["eins"]["iy"] == ["a"]
    assert d["args"][0]["eins"] == {"ixs": [["a", "b"], ["b", "c"]], "iy": ["a", "c"]}
    assert F.contractions(d, ixs) == [(0, 1, 1, 1), (1, 0, 0, 1)]
    tc, sc = F.complexity(d, ixs)
    assert abs(tc - np.log2(2 ** 3 + 2 ** 2)) < 1e-12 and sc == 2
    assert F.children_to_dict([], 1, [["x"]], []) == {"tensor_index": 0}


@pytest.mark.parametrize("name,nsl", [("sat60", 0), ("reg3_250", 6), ("grid24", 4)])
def test_model_times_equal_host_layer(name, nsl):
    m, nlab, ixs, iy = common.load_instance(name)
    inst = host.Instance(common.inst_path(name))
    lay = capi.layout(m, nlab)
    rng = np.random.default_rng(5)
    gm = dict(F.GPU_MODEL, m0=5, n0=7)  # asymmetric tiles: the children's order matters
    for seed in range(3):
        ch = host.random_tree(m, 100 + seed)
        rec = inst.population(lay, np.array([ch]), 1, seed=0, random_slices=nsl)[0]
        tc, sc, t1, t2, ns = inst.host_energy(lay, rec, slicing=nsl > 0,
                                              gm=tuple(gm[k] for k in F.GPU_KEYS))
        Sw = rec[lay.s_off:lay.s_off + lay.W]
        sliced = [l for l in range(nlab) if nsl and (int(Sw[l >> 6]) >> (l & 63)) & 1]
        assert len(sliced) == ns
        res = {"tree": [[a, b] for a, b in pairs(ch)], "sliced": sliced, "tc": tc}
        tree, info = F.result_tree(json.loads(json.dumps(res)), ixs, iy, gpu_model=gm)
        assert abs(info["tc_py"] - tc) < 1e-9 and info["sc_py"] == sc
        # the binary keeps the model constants as float log2 values (csrc/treesa_gpu.cu:1181-1203): relative
        # differences of about 1e-7; the reference's own test allows 1e-5 in log (tests/test_python.py:60-61)
        assert abs(np.log(info["gpu_time_py"]) - np.log(t1)) < 1e-5
        assert abs(np.log(info["h100_time_py"]) - np.log(t2)) < 1e-5
        assert info["tc_total_py"] == info["tc_py"] + ns
        rj = json.loads(json.dumps(F.runner_json(tree, info)))
        assert rj["tree"] == tree and rj["sliced"] == sliced
        sl = set(sliced)
        assert F.recompute_outputs(tree, [[l for l in ix if l not in sl] for ix in ixs], []) == tree


def test_write_instance_and_tree_file(tmp_path):
    m, nlab, ixs, iy = common.load_instance("sat40")
    p = str(tmp_path / "i.txt")
    mp = F.write_instance(p, ixs, iy)
    inst = host.Instance(p)
    ref = host.Instance(common.inst_path("sat40"))
    assert len(mp) == nlab and (inst.m, inst.nlab) == (ref.m, ref.nlab)
    assert np.array_equal(inst.leaf(1), ref.leaf(1))  # same label set per tensor (the order within may differ)
    ch = pairs(S.path_tree(np.arange(m)))
    d = F.children_to_dict(ch, m, ixs, iy)
    tp = str(tmp_path / "t.tree")
    F.write_tree_file(tp, [d, ch, S.path_tree(np.arange(m)[::-1])], m)
    got = inst.read_trees(tp)
    assert len(got) == 3 and pairs(got[0]) == ch and pairs(got[1]) == ch
