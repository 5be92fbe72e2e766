"""The five benchmark workloads at their full sizes, run exactly as bench.py times them, against the oracle (GPU).

bench.py runs the drop-in binary on each workload (its own level loop, after ten untimed warm-up levels and a
fresh upload of the start population).  Here the same runs also write their final population
(--dump-population, after the timed loop), and it must equal the oracle's chain by chain:

* c1 (256 chains x 100 pre-order levels from the greedy tree: the whole level loop in one launch, with helper
  waves): every record, and the oracle's level loop (csrc/treesa_gpu.cu:1788-1832) gives the same best tree and
  final tc to 1e-9;
* c2 (8192 chains x 200 par levels from the spectral trees: node costs folded and chains selected beside the
  next sweep, each level's sweep two launches on two streams): 128 chains, half from each end of the
  population, so that both launches are covered;
* c3 (2048 chains x 20 levels of 10 par sweeps with one slice move each, population annealing after every
  level): the oracle's whole level loop, every record, the best tree, its slice set and repair, tc to 1e-9;
* c4 (512 chains x 100 levels of 47-word sets, the dense wide kernel): 32 chains from both ends;
* c5 (72 chains x 20 levels of 126-word sets): every chain, for the chunk-summary kernel and for dense
  streaming (--no-sum).
"""
import os
import tempfile

import numpy as np
import pytest

import bench
import common
import oracle as orc
from treesa_gpu_amd import capi

pytestmark = pytest.mark.gpu

_oracle_cache = {}


def binary_final(cfgname, extra=()):
    C, inst, lay, trees, _, cfg, betas, order = bench.setup(cfgname, population=False)
    with tempfile.TemporaryDirectory() as td:
        dump = os.path.join(td, "pop.u64")
        print(f"[gpu] {cfgname} full size {' '.join(extra)}", flush=True)
        res = bench.run_binary(C, trees, betas, C["levels"], 10, None, list(extra), dump)
        pop = bench.load_population(dump, C["nchains"], lay)
    assert res["valid"] and res["labels_ok"] and res["total_sweeps"] == C["levels"] * C["niters"]
    return res, pop


def oracle_sample(cfgname, n):
    """The oracle's final records of n chain slots (both ends of the population), by independent sweeps."""
    key = (cfgname, n)
    if key in _oracle_cache:
        return _oracle_cache[key]
    C, inst, lay, trees, _, cfg, betas, order = bench.setup(cfgname, population=False)
    m, nlab, ixs, iy = common.load_instance(C["inst"])
    O = orc.Oracle(m, nlab, ixs, iy)
    P = orc.params_from_config(cfg, inst.leaf_sc, nlab)
    out = {}
    print(f"[oracle] {cfgname}: {n} chains", flush=True)
    for c0, k in bench.sample_slots(C["nchains"], n):
        sub = common.oracle_population(O, lay, m, k, 1, trees, first=c0)
        for lev, b in enumerate(betas):
            O.sweeps(P, lay, sub, order, b, lev * C["niters"], C["niters"], c0=c0)
        for j in range(k):
            out[c0 + j] = sub[j].copy()
    _oracle_cache[key] = out
    return out


def oracle_level_loop(cfgname):
    """The oracle's level loop over the whole population: final records, best record, n_repair, host tc."""
    C, inst, lay, trees, _, cfg, betas, order = bench.setup(cfgname, population=False)
    m, nlab, ixs, iy = common.load_instance(C["inst"])
    O = orc.Oracle(m, nlab, ixs, iy)
    ocfg = capi.make_config(mode="tc", sc_target=C["sc_target"], seed=1, slicing=C["slicing"], slice_moves=1)
    P = orc.params_from_config(ocfg, inst.leaf_sc, nlab)
    pop = common.oracle_population(O, lay, m, C["nchains"], 1, trees)
    nlev = len(betas)
    print(f"[oracle] {cfgname}: level loop, {C['nchains']} chains", flush=True)
    r = O.anneal(P, lay, pop, betas, [0] * nlev, [C["niters"]] * nlev, order, scheme=C["scheme"], eval_every=1,
                 sc_target=C["sc_target"], seed=1)
    best = r["best_rec"].copy()
    ch = np.ascontiguousarray(best[lay.ch_off:]).view(np.uint32)[:m - 1]
    best[:lay.nint * lay.W] = O.labels(ch, lay.W).reshape(-1)
    n_repair = O.repair(lay, best, C["sc_target"]) if C["slicing"] else 0
    tc, sc, _, _, ns = O.host_energy(lay, best, C["slicing"], orc.DEFAULT_GM, orc.DEFAULT_H100)
    return dict(pop=pop, best=best, tree=[[int(w & 0xFFFF), int(w >> 16)] for w in ch], n_repair=n_repair, tc=tc,
                sc=sc, ns=ns, best_chain=r["best_chain"], nresample=r["nresample"], lay=lay, nlab=nlab)


def assert_same_records(pop, want):
    bad = [c for c in sorted(want) if not np.array_equal(pop[c], want[c])]
    assert not bad, f"{len(bad)} of {len(want)} chains differ from the oracle (first {bad[:5]})"


@pytest.mark.parametrize("cfgname", ["c1", "c3"])
def test_level_loop_at_full_size(cfgname):
    res, pop = binary_final(cfgname)
    o = oracle_level_loop(cfgname)
    assert_same_records(pop, {c: o["pop"][c] for c in range(pop.shape[0])})
    assert res["tree"] == o["tree"] and res["best_chain"] == o["best_chain"]
    assert abs(res["tc_exact"] - o["tc"]) <= 1e-9 and res["sc"] == o["sc"]
    assert res["nresample"] == o["nresample"]
    if cfgname == "c1":
        assert res["hip_kernel"].endswith("anneal=level_loop") and "preorder_draw_waves=3" in res["hip_kernel"]
    else:
        lay = o["lay"]
        S = o["best"][lay.s_off:lay.s_off + lay.W]
        assert res["sliced"] == [l for l in range(o["nlab"]) if int(S[l >> 6]) >> (l & 63) & 1]
        assert res["n_repair"] == o["n_repair"] and res["nsliced"] == o["ns"]
        assert res["nresample"] == 19
    print(f"[ok] {cfgname}: {pop.shape[0]} chains equal the oracle, tc {res['tc_exact']!r}", flush=True)


@pytest.mark.parametrize("cfgname,n,extra", [("c2", 128, ()), ("c4", 32, ()), ("c5", 72, ()),
                                             ("c5", 72, ("--no-sum",))])
def test_sampled_chains_at_full_size(cfgname, n, extra):
    res, pop = binary_final(cfgname, extra)
    if cfgname == "c2":
        assert "fold=apart" in res["hip_kernel"] and "split_levels=" in res["hip_kernel"], res["hip_kernel"]
    if cfgname == "c5":
        assert (" sums=0 " in res["hip_kernel"]) == ("--no-sum" in extra), res["hip_kernel"]
    assert_same_records(pop, oracle_sample(cfgname, n))
    print(f"[ok] {cfgname} {' '.join(extra)}: {n} chains equal the oracle", flush=True)
