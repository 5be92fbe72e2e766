"""The oracle against the reference's own CPU port.

tests/golden/ref_sweeps.json was written by tests/golden/make_golden.py from csrc/cpu_ref.h compiled in
place (oracle/_ref).  For every case the oracle, starting from the same chains, must reproduce each
chain's final children and label sets (FNV hashes) and its proposal / accept counts exactly.  When
oracle/_ref is present the full children lists are also compared directly.
"""
import json
import os
import subprocess

import numpy as np
import pytest

import common
import oracle as orc
from treesa_gpu_amd import capi


def run_oracle_case(case, nchains=4):
    m, nlab, ixs, iy = common.load_instance(case["inst"])
    O = orc.Oracle(m, nlab, ixs, iy)
    lay = capi.layout(m, nlab)
    rs, pf, pb = common.case_options(case)
    tf = common.tree_file(case["inst"], case["init"])
    trees = orc.read_trees_py(tf, m) if tf else None
    pop = common.oracle_population(O, lay, m, nchains, common.CHECK_SEED, trees, rs)
    cfg = capi.make_config(mode=case["mode"], sc_target=common.CHECK_SC_TARGET, seed=common.CHECK_SEED,
                           slicing=rs > 0, slice_moves=0, par_follow=pf, par_band=pb)
    P = orc.params_from_config(cfg, max(len(x) for x in ixs), nlab)
    order = capi.ORDER_PAR if case["order"] == "par" else capi.ORDER_PREORDER
    per_chain = []
    for c in range(nchains):
        row = np.ascontiguousarray(pop[c:c + 1])
        np_, na_ = 0, 0
        for lev, beta in enumerate(common.CHECK_BETAS):
            st = O.sweeps(P, lay, row, order, beta, lev * common.CHECK_NITERS, common.CHECK_NITERS, c0=c)
            np_ += st[0]
            na_ += st[1]
        pop[c] = row[0]
        per_chain.append((np_, na_))
    return lay, nlab, pop, per_chain


@pytest.mark.parametrize("case", common.golden_cases(), ids=common.case_id)
def test_oracle_matches_reference_cpu_port(case):
    lay, nlab, pop, per_chain = run_oracle_case(case)
    for c, want in enumerate(case["chains"]):
        chf, labf = common.record_hashes(pop[c], lay, nlab)
        assert per_chain[c] == (want["nprop"], want["nacc"]), f"chain {c} counts"
        assert chf == want["children_fnv"], f"chain {c} children"
        assert labf == want["labels_fnv"], f"chain {c} labels"


@pytest.mark.skipif(not os.path.exists(orc.REF_BIN), reason="oracle/_ref not built (reference sources absent)")
def test_oracle_children_equal_reference_lists():
    case = dict(inst="reg3_250", order="par", mode="h100", init="greedy", extra=["--par-follow"])
    lay, nlab, pop, _ = run_oracle_case(case)
    args = [orc.REF_BIN, "-i", common.inst_path("reg3_250"), "--tree", common.tree_file("reg3_250", "greedy"),
            "--chains", "4", "--niters", "4", "--betas", "0.2:0.7:7", "--sc-target", "24", "--seed", "7",
            "--order", "par", "--mode", "h100", "--par-follow"]
    ref = json.loads(subprocess.run(args, check=True, capture_output=True, text=True).stdout)
    for c, ch in enumerate(ref["chains"]):
        w = np.array(ch["children"], np.uint32).reshape(-1, 2)
        got = pop[c, lay.ch_off:].view(np.uint32)[:lay.nint]
        assert np.array_equal(got, w[:, 0] | (w[:, 1] << 16))
