"""CPU tests of the workload generators and start trees: the generators reproduce the reference's committed
instances byte for byte, the committed larger fixtures are what the generators make, and the closed-form path
cost equals the host layer's exact energy of the same tree."""
import os

import numpy as np
import pytest

import common
from treesa_gpu_amd import capi, host
from treesa_gpu_amd import instances as I
from treesa_gpu_amd import host as S


def fixture(name):
    with open(common.inst_path(name)) as f:
        return f.read()


@pytest.mark.parametrize("n", [40, 60, 100])
def test_sat_generator_matches_reference_fixture(n):
    assert I.instance_text(*I.sat(n)) == fixture(f"sat{n}")


def test_lattice_generator_matches_reference_fixture():
    assert I.instance_text(*I.sq(46)) == fixture("sq46")


def test_larger_fixtures_are_the_generated_instances():
    assert I.instance_text(*I.sat(70)) == fixture("sat70")
    assert I.instance_text(*I.sq(64)) == fixture("sq64")
    assert I.instance_text(*I.reg3(2000, seed=1)) == fixture("reg3_2000")


def test_reg3_is_simple_and_cubic():
    ixs, _ = I.reg3(300, seed=5)
    assert all(len(ix) == 3 for ix in ixs)
    holders = {}
    for t, ix in enumerate(ixs):
        for l in ix:
            holders.setdefault(l, []).append(t)
    assert all(len(h) == 2 and h[0] != h[1] for h in holders.values())
    pairs = {tuple(sorted(h)) for h in holders.values()}
    assert len(pairs) == len(holders)


def path_energy(name, order):
    inst = host.Instance(common.inst_path(name))
    lay = capi.layout(inst.m, inst.nlab)
    ch = S.path_tree(order)
    rec = inst.population(lay, np.array([ch]), 1, seed=0)[0]
    return inst.host_energy(lay, rec, slicing=False)


@pytest.mark.parametrize("name", ["sat40", "sq46", "lat14"])
def test_path_cost_equals_exact_energy(name):
    m, nlab, ixs, iy = common.load_instance(name)
    rng = np.random.default_rng(3)
    for order in (np.arange(m), rng.permutation(m), rng.permutation(m)):
        tc, sc = S.path_cost(order, ixs, iy)
        e = path_energy(name, order)
        assert abs(tc - e[0]) < 1e-9 and sc == e[1]


def test_greedy_and_spectral_starts_are_valid_and_good():
    m, nlab, ixs, iy = common.load_instance("sq46")
    inst = host.Instance(common.inst_path("sq46"))
    lay = capi.layout(m, nlab)
    g = S.greedy_tree(ixs, iy, nrepeat=3, seed=1)
    rec = inst.population(lay, np.array([g]), 1, seed=0)[0]  # population() validates the tree
    tc_g = inst.host_energy(lay, rec, slicing=False)[0]
    tc_r = path_energy("sq46", np.random.default_rng(0).permutation(m))[0]
    assert tc_g < tc_r
    so = S.spectral_orders(ixs, iy, k=2)
    assert len(so) == 2 and so[0][0] <= so[1][0]
    tc_row = S.path_cost(np.arange(m), ixs, iy)[0]
    assert so[0][0] <= tc_row + 0.01  # within 0.01 of the row sweep, the best order known for the lattice
