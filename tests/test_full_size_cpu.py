"""The oracle against the reference's own CPU port at the benchmark workloads' full sizes (CPU).

bench.py's CPU baseline runs the reference's csrc/cpu_ref.h (oracle/_ref/ref_harness, compiled in place from
the reference's sources) on a sample of each workload's chains over the whole schedule, and compares the
binary's final population with it chain by chain.  This test runs the same samples through the oracle (the
checker every GPU parity test uses) and requires the same answer from it: c1 (all 256 chains, 100 pre-order
sweeps from the greedy tree), c2 (64 of its 8192 chains, half from each end of the population, 200 par sweeps
from the three spectral trees), c4 (16 of 512 chains, 100 sweeps of 47-word sets) and c5 (24 of 72 chains, 20
sweeps of 126-word sets) -- children words and label sets of every chain, and the proposal and accept counts.
It also runs bench.py's own comparison (parity_of) on the oracle's population, so that the check the benchmark
line reports is the one tested here, and shows that comparison catches a chain whose tree differs.
"""
import os

import numpy as np
import pytest

import bench
import common
import oracle as orc

REF = os.path.join(bench.ROOT, "oracle", "_ref", "ref_harness")

pytestmark = pytest.mark.skipif(not os.path.exists(REF), reason="the reference's CPU port is not built here")


def oracle_final(cfgname, ranges):
    """The oracle's final records of the given chain slots (a full-size array; other rows stay zero) and its
    proposal / accept totals over them."""
    C, inst, lay, trees, _, cfg, betas, order = bench.setup(cfgname, population=False)
    m, nlab, ixs, iy = common.load_instance(C["inst"])
    O = orc.Oracle(m, nlab, ixs, iy)
    P = orc.params_from_config(cfg, inst.leaf_sc, nlab)
    out = np.zeros((C["nchains"], lay.chain_words), np.uint64)
    npr = nac = 0
    for c0, k in ranges:
        sub = common.oracle_population(O, lay, m, k, 1, trees, first=c0)
        for lev, b in enumerate(betas):
            st = O.sweeps(P, lay, sub, order, b, lev * C["niters"], C["niters"], c0=c0)
            npr += st[0]
            nac += st[1]
        out[c0:c0 + k] = sub
    return C, inst, lay, trees, betas, out, npr, nac


@pytest.mark.parametrize("cfgname,n", [("c1", None), ("c2", 64), ("c4", 16), ("c5", 24)])
def test_oracle_equals_reference_port_at_full_size(cfgname, n):
    C = bench.CONFIGS[cfgname]
    ranges = bench.sample_slots(C["nchains"], n or C["nchains"])
    C, inst, lay, trees, betas, pop, npr, nac = oracle_final(cfgname, ranges)
    threads = max(1, min(8, os.cpu_count() or 1))
    outs = [bench.ref_harness_run(C, trees, betas, c0, k, threads) for c0, k in ranges]
    chains = [ch for o in outs for ch in o["chains"]]
    assert sorted(ch["chain"] for ch in chains) == [c for c0, k in ranges for c in range(c0, c0 + k)]
    par = bench.parity_of(lay, inst.nlab, pop, ref_chains=chains)
    assert par["mismatches"] == 0 and par["chains"] == len(chains), par
    assert sum(ch["nprop"] for ch in chains) == npr and sum(ch["nacc"] for ch in chains) == nac
    print(f"{cfgname}: {len(chains)} chains x {len(betas) * C['niters']} sweeps equal, {npr} proposals")
    # the comparison catches one chain whose tree differs (two children swapped in its last internal node)
    c = chains[-1]["chain"]
    w = np.ascontiguousarray(pop[c, lay.ch_off:]).view(np.uint32)
    w[lay.nint - 1] = (w[lay.nint - 1] >> 16) | ((w[lay.nint - 1] & 0xFFFF) << 16)
    pop[c, lay.ch_off:] = w.view(np.uint64)[:lay.chain_words - lay.ch_off]
    bad = bench.parity_of(lay, inst.nlab, pop, ref_chains=chains)
    assert bad["mismatches"] == 1 and bad["first_mismatches"] == [c]
