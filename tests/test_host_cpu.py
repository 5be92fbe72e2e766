"""CPU tests of the product's host side: the C ABI library loads and exports every declared entry point,
the host layer (libtreesa_host.so) agrees with the oracle, and the CLI rejects bad input with the
reference's messages and exit codes before touching a GPU."""
import os
import re
import subprocess

import numpy as np
import pytest

import common
import edge_instances
import oracle as orc
from treesa_gpu_amd import capi, formats, host

ROOT = common.HERE.rsplit(os.sep, 1)[0]


def declared_functions():
    names = []
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            with open(os.path.join(ROOT, "include", fn)) as f:
                txt = f.read()
            names += re.findall(r"^\s*(?:int|float|const char\*|void\s*\*?)\s*(tsa_\w+)\s*\(", txt, re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = capi.load()
    names = declared_functions()
    assert len(names) >= 20 and {"tsa_host_alloc", "tsa_host_free", "tsa_chunk_stats"} <= set(names)
    for n in names:
        assert hasattr(lib, n), n
    assert set(capi.EXPORTS) <= set(names)


def test_layout_is_pure_host():
    lay = capi.layout(426, 100)
    assert (lay.W, lay.runtime_width, lay.nint) == (2, 0, 425)
    assert lay.ch_off == 850 and lay.s_off == 850 + 213 and lay.chain_words % 2 == 0
    wide = capi.layout(4096, 8064)
    assert (wide.W, wide.runtime_width) == (126, 1)
    assert capi.layout(426, 100, wide=True).runtime_width == 1
    with pytest.raises(capi.TsaError, match="at least 3 tensors"):
        capi.layout(2, 10)
    with pytest.raises(capi.TsaError, match="16-bit"):
        capi.layout(40000, 10)


def test_philox_and_hash_known_answers():
    # Random123 Philox4x32-10 known-answer vectors
    assert orc.philox([0, 0, 0, 0], 0, 0) == [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]
    assert orc.philox([0xffffffff] * 4, 0xffffffff, 0xffffffff) == [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]
    assert orc.philox([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], 0xa4093822, 0x299f31d0) == \
        [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]
    assert host.splitmix64(0) == 0xe220a8397b1dcdaf == capi.splitmix64(0)
    assert host.splitmix64(1) == 0x910a2dec89025cc1 == orc.load().oracle_splitmix64(1)


@pytest.mark.parametrize("name", ["sat40", "sat100", "reg3_250", "lat14", "grid24"])
def test_host_layer_matches_oracle(name):
    inst = host.Instance(common.inst_path(name))
    m, nlab, ixs, iy = common.load_instance(name)
    O = orc.Oracle(m, nlab, ixs, iy)
    assert (inst.m, inst.nlab, inst.leaf_sc) == (m, nlab, max(len(x) for x in ixs))
    lay = capi.layout(m, nlab)
    trees = inst.read_trees(common.tree_file(name, "greedy"))
    assert np.array_equal(trees, orc.read_trees_py(common.tree_file(name, "greedy"), m))
    for ch in list(trees) + [host.random_tree(m, s) for s in (1, 2, 3)]:
        assert np.array_equal(inst.labels(ch, lay.W), O.labels(ch, lay.W))
    for s in (0, 1, 12345):
        assert np.array_equal(host.random_tree(m, s), orc.random_tree(m, s))
    # population: greedy tree replicated, random trees, random slice sets
    pop_h = inst.population(lay, trees, 7, seed=7, random_slices=5)
    pop_o = common.oracle_population(O, lay, m, 7, 7, trees, 5)
    assert np.array_equal(pop_h, pop_o)
    pop_h = inst.population(lay, None, 5, seed=3)
    pop_o = common.oracle_population(O, lay, m, 5, 3, None)
    assert np.array_equal(pop_h, pop_o)
    # host double energy (tc, sc, model times, |S|)
    for rec, sl in ((pop_h[0], False), (inst.population(lay, trees, 1, seed=7, random_slices=5)[0], True)):
        a = inst.host_energy(lay, rec, slicing=sl)
        b = O.host_energy(lay, rec, sl, capi.DEFAULT_GM, capi.DEFAULT_H100)
        assert a[1] == b[1] and a[4] == b[4]
        assert abs(a[0] - b[0]) < 1e-12 and abs(a[2] / b[2] - 1) < 1e-12 and abs(a[3] / b[3] - 1) < 1e-12


def test_betas_spec():
    assert list(host.parse_betas("0.2:0.7:7")) == common.CHECK_BETAS
    assert len(host.parse_betas("0.01:0.05:15")) == 300 and len(host.parse_betas("1:0.05:15")) == 281
    assert list(host.parse_betas("1,2.5, 3")) == [1.0, 2.5, 3.0]


def test_reader_errors(tmp_path):
    bad = tmp_path / "bad.txt"
    bad.write_text("3 4\n2 0 0\n1 1\n1 2\n0\n")
    with pytest.raises(host.HostError, match="repeated label"):
        host.Instance(str(bad))
    bad.write_text("3 2\n2 0 5\n1 1\n1 0\n0\n")
    with pytest.raises(host.HostError, match="label out of range"):
        host.Instance(str(bad))
    bad.write_text("x")
    with pytest.raises(host.HostError, match="bad header"):
        host.Instance(str(bad))
    inst = host.Instance(common.inst_path("sat40"))
    tr = tmp_path / "t.txt"
    tr.write_text("1 2\n3 4\n")
    with pytest.raises(host.HostError, match="truncated tree"):
        inst.read_trees(str(tr))
    tr.write_text("")
    with pytest.raises(host.HostError, match="no tree"):
        inst.read_trees(str(tr))


def cli(*args):
    return subprocess.run([capi.BIN_PATH] + list(args), capture_output=True, text=True, timeout=120)


def test_cli_errors_before_any_gpu_call(tmp_path):
    p = cli()
    assert p.returncode == 1 and "usage: treesa_gpu" in p.stderr
    p = cli("-i", "/nonexistent.txt")
    assert p.returncode == 1 and "cannot open" in p.stderr
    inst = common.inst_path("sat40")
    assert "--order par|preorder" in cli("-i", inst, "--order", "x").stderr
    assert "--par-band" in cli("-i", inst, "--par-band", "1").stderr
    assert "slice moves need" in cli("-i", inst, "--slicing", "--kernel", "seq").stderr
    assert cli("-i", inst, "--nchains", "abc").returncode == 1
    small = tmp_path / "two.txt"
    small.write_text("2 1\n1 0\n1 0\n0\n")
    assert "need at least 3 tensors" in cli("-i", str(small)).stderr
    bt = tmp_path / "t.txt"
    bt.write_text("1 2\n")
    p = cli("-i", inst, "--tree", str(bt))
    assert p.returncode == 1 and "truncated tree" in p.stderr
    bt.write_text("".join(f"{i} {i}\n" for i in range(169)))  # 169 lines but not a tree
    p = cli("-i", inst, "--tree", str(bt))
    assert p.returncode == 1 and "invalid initial tree" in p.stderr


@pytest.mark.parametrize("name", edge_instances.NAMES)
def test_host_layer_on_edge_instances(name):
    """Empty tensors, labels held by one tensor, open labels and every width boundary: the host layer's
    topology labels equal the oracle's, and its exact energy equals the Python formats' closed form."""
    m, nlab, ixs, iy = edge_instances.instance(name)
    O = orc.Oracle(m, nlab, ixs, iy)
    inst = host.Instance(m=m, nlab=nlab, ixs=ixs, iy=iy)
    lay = capi.layout(m, nlab)
    for seed in range(3):
        ch = host.random_tree(m, 100 + seed)
        assert np.array_equal(inst.labels(ch, lay.W), O.labels(ch, lay.W))
        rec = inst.population(lay, np.array([ch]), 1, seed=0)[0]
        tc, sc = inst.host_energy(lay, rec, slicing=False)[:2]
        d = formats.children_to_dict([(int(w) & 0xFFFF, int(w) >> 16) for w in ch], m, ixs, iy)
        t2, s2 = formats.complexity(d, ixs)
        assert abs(tc - t2) < 1e-9 and sc == s2


def test_layout_rejects_fewer_than_three_tensors_and_17_bit_node_ids():
    m, nlab, ixs, iy = edge_instances.instance("pair")
    with pytest.raises(capi.TsaError, match="at least 3 tensors"):
        capi.layout(m, nlab)
    assert capi.layout(32768, 3).nint == 32767  # node ids up to 65534
    with pytest.raises(capi.TsaError, match="16-bit"):
        capi.layout(32769, 3)
