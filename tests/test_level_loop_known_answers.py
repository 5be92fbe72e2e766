"""The oracle's level loop against the reference's logged end-to-end answers (tests/test_python.py output for both
sweep orders, tests/golden/test_python_results_{par,preorder}.txt), through the fixture
tests/golden/level_loop_answers.json (tests/golden/make_level_loop_answers.py).

* A fast subset of the cases is run again here and must give the fixture's answer, and the reference's printed
  one where the fixture says it reproduces (every scheme, start, selection rule and both orders among them).
* Every case the oracle does not reproduce is explained, by one of two recorded facts:
  - float sensitivity: under perturbations of the float functions within the bounds the reference's GPU
    documents (exp2f / log2f moved by one ulp, Metropolis's expf by up to two, at hash-chosen operands; or the
    energy fold's lse evaluated in double), the run's answer moves -- a device whose functions round differently
    from this host's libm cannot be expected to land on the same answer; several of these perturbed runs land
    exactly on the reference's printed answer (one is run again below);
  - the pre-order log's H100 model: that log prints, for the trees whose tc, sc and GPU-model time the oracle
    reproduces, H100-model times that differ from the H100 model both the par log and this build evaluate (the
    par log agrees on every run), so its h100-mode runs were made with another H100 model and cannot reproduce.
"""
import json
import os

import pytest

import level_loop_cases as K
import oracle as orc

CASES = {c["id"]: c for order in ("par", "preorder") for c in K.known_answer_cases(order)}
FIX = {c["id"]: c for c in K.load_fixture()["cases"]}

# a fast subset: indep, pa and select runs, greedy / random / spectral starts, both orders
FAST = ["par:7", "par:12", "par:40", "par:64", "par:69/free-sc", "preorder:5", "preorder:33"]


def test_fixture_covers_every_logged_run():
    assert set(FIX) == set(CASES)
    assert len(CASES) == 112
    for cid, c in FIX.items():
        assert c["reproduces"] == K.agrees_with_reference(CASES[cid], dict(c["oracle"])), cid


@pytest.mark.parametrize("cid", FAST)
def test_oracle_level_loop_reproduces(cid, tmp_path):
    c, fx = CASES[cid], FIX[cid]
    orc.set_variant(0)
    got = K.oracle_run(c, str(tmp_path))
    assert K.tree_hash(got["tree"]) == fx["oracle"]["tree_fnv"]
    assert round(got["tc"], 9) == fx["oracle"]["tc"] and got["sc"] == fx["oracle"]["sc"]
    assert got["best_chain"] == fx["oracle"]["best_chain"] and got["nresample"] == fx["oracle"]["nresample"]
    assert fx["reproduces"] and K.agrees_with_reference(c, got), (c["ref"], got["tc"])


def test_float_perturbation_lands_on_the_reference_answer(tmp_path):
    """lat10, population annealing, tc (test_python_results.txt line 49): the oracle ends at 20.2181, the
    reference printed 20.2198; with Metropolis's expf moved by at most two ulp at hash-chosen operands (seed 4)
    the decisions part at level 34 and the run ends exactly on the reference's answer."""
    c, fx = CASES["par:49"], FIX["par:49"]
    assert not fx["reproduces"]
    hit = [p for p in fx["perturbed"] if p["reproduces"]]
    assert hit and hit[0]["variant"] == 20 and hit[0]["noise_seed"] == 4
    orc.set_variant(20, 4)
    try:
        got = K.oracle_run(c, str(tmp_path))
    finally:
        orc.set_variant(0)
    assert K.agrees_with_reference(c, got), got["tc"]
    assert K.tree_hash(got["tree"]) == hit[0]["answer"]["tree_fnv"]


def uses_h100(c):
    return c["mode"] == "h100" or (c["stage2"] is not None and c["stage2"][0] == "h100")


def test_preorder_log_was_made_with_another_h100_model():
    """Runs both logs print and the oracle reproduces (tc, sc and the GPU-model time of the returned tree all
    equal): the par log's H100-model times equal this build's on every one, the pre-order log's differ on
    most."""
    counts = {}
    for order in ("par", "preorder"):
        same = differ = 0
        for cid, fx in FIX.items():
            c = CASES[cid]
            if c["order"] != order or fx["kind"] != "run" or not fx["reproduces"]:
                continue
            ref, o = c["ref"], fx["oracle"]
            assert abs(o["gpu_time"] - float(ref["gpu_time"])) <= 1e-4 * float(ref["gpu_time"]), cid
            if abs(o["h100_time"] - float(ref["h100_time"])) <= 1e-4 * float(ref["h100_time"]):
                same += 1
            else:
                differ += 1
        counts[order] = (same, differ)
    assert counts["par"][1] == 0 and counts["par"][0] >= 25, counts
    assert counts["preorder"][1] >= 15, counts


def test_every_unreproduced_answer_is_explained():
    unexplained, kinds = [], {"float": 0, "h100_log": 0}
    for cid, fx in FIX.items():
        if fx["reproduces"]:
            continue
        c = CASES[cid]
        moved = [p for p in fx["perturbed"] if p["answer_changes"]]
        if moved:
            kinds["float"] += 1
            assert all(p["first_level"] is not None for p in moved), cid
        elif c["order"] == "preorder" and uses_h100(c):
            kinds["h100_log"] += 1
        else:
            unexplained.append(cid)
    assert not unexplained, unexplained
    reproduced = sum(fx["reproduces"] for fx in FIX.values())
    assert reproduced >= 80, reproduced
    print(f"reproduced {reproduced} of {len(FIX)}; unreproduced: {kinds}")


def test_truncation_runs_part_where_the_cut_is_a_float_tie():
    """Truncation ranks every chain by its float energy at every level and copies the best quarter over the
    worst (csrc/treesa_gpu.cu:1857-1869).  In every truncation run the oracle does not reproduce:
    * the perturbation of the energy arithmetic alone (exp2f / log2f moved by one ulp, variant 1) first changes
      the run at a level whose ranking around the cut is a float tie -- a population margin of at most one float
      ulp at the run's energy scale, in fact exactly zero: which of the tied chains survives is decided by the
      energies' last bit;
    * every other perturbation (Metropolis's expf moved by up to two ulp, variant 20) first changes the run at
      such a tie or at or after a level whose sweeps hold a Metropolis decision within two ulp of expf.
    So a device whose exp2f / log2f / expf round differently from this host's libm parts from this answer at a
    tie of float energies or at a Metropolis decision on the edge, as these runs show."""
    import numpy as np
    rows = []
    for cid, fx in FIX.items():
        c = CASES[cid]
        if c["scheme"] != "trunc" or fx["reproduces"]:
            continue
        ulp = float(np.spacing(np.float32(fx["oracle"]["tc"])))
        near = fx.get("metropolis_near_levels") or []
        moved = [p for p in fx["perturbed"] if p["answer_changes"]]
        energy = [p for p in moved if p["variant"] == 1]
        assert energy and all(p["pop_margin"] <= ulp for p in energy), (cid, energy)
        for p in moved:
            assert p["pop_margin"] <= ulp or any(L <= p["first_level"] for L in near), (cid, p, near)
        rows.append((cid, energy[0]["first_level"], energy[0]["pop_margin"] / ulp, near[:3]))
    assert len(rows) == 11, rows
    for cid, first, m, near in rows:
        print(f"{cid}: energy rounding first parts at level {first} (cut margin {m:.2f} ulp); "
              f"Metropolis decisions within two ulp at levels {near}")
