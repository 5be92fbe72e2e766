"""The binary on every run of the reference's logged end-to-end test (tests/test_python.py, both sweep orders):
its final tree, tc, sc, |S|, repair count, best chain and resampling count equal the oracle's level loop on the
same case (tests/golden/level_loop_answers.json, written by tests/golden/make_level_loop_answers.py), and where
the oracle reproduces the reference's printed answer, so does the binary.  Where it does not, the fixture records
why (tests/test_level_loop_known_answers.py checks that every such case is explained)."""
import json
import math
import os
import subprocess

import pytest

import common
import level_loop_cases as K
from treesa_gpu_amd import capi, formats

pytestmark = pytest.mark.gpu

CASES = [c for order in ("par", "preorder") for c in K.known_answer_cases(order)]
FIXTURE = {c["id"]: c for c in K.load_fixture()["cases"]} if os.path.exists(K.FIXTURE) else {}


@pytest.mark.parametrize("case", CASES, ids=[c["id"] for c in CASES])
def test_binary_equals_oracle_on_known_answer(case, tmp_path):
    fx = FIXTURE.get(case["id"])
    assert fx is not None, f"{case['id']} missing from the fixture"
    out = str(tmp_path / "out.json")
    args = K.binary_args(case, capi.BIN_PATH, str(tmp_path), out)
    print(f"[gpu] known answer {case['id']} {case['inst']} {case['scheme']} {case['mode']} order={case['order']}",
          flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, r.stderr[-2000:]
    with open(out) as f:
        got = json.load(f)
    want = fx["oracle"]
    tree = [[int(a), int(b)] for a, b in got["tree"]]
    assert K.tree_hash(tree) == want["tree_fnv"], "final tree differs from the oracle's level loop"
    # the fixture holds the oracle's tc rounded to 9 decimals: equal values differ by at most 5e-10
    assert abs(got["tc_exact"] - want["tc"]) <= 1e-9, (got["tc_exact"], want["tc"])
    assert got["sc"] == want["sc"] and got.get("nsliced", 0) == want["ns"]
    assert got["n_repair"] == want["n_repair"] and got["best_chain"] == want["best_chain"]
    assert got["nresample"] == want["nresample"]
    assert sorted(got["sliced"]) == sorted(want["sliced"])
    if fx["reproduces"]:
        assert K.agrees_with_reference(case, dict(got, ns=got.get("nsliced", 0))), (case["ref"], got["tc"])
    assert got["valid"] and got["labels_ok"]
    if not case["slicing"]:
        # the driver's reading of the result (treesa_gpu/driver.py:313-328): the tree dict and its model times
        # recomputed in Python equal the binary's (1e-5 in log, the reference's own check, tests/test_python.py:
        # 60-61)
        m, nlab, ixs, iy = common.load_instance(case["inst"])
        tdict, info = formats.result_tree(got, ixs, iy)
        assert formats.recompute_outputs(tdict, ixs, iy) == tdict
        assert abs(info["tc_py"] - got["tc"]) < 1e-4 and info["sc_py"] == got["sc"]
        assert abs(math.log(got["gpu_time"]) - math.log(info["gpu_time_py"])) < 1e-5
        assert abs(math.log(got["h100_time"]) - math.log(info["h100_time_py"])) < 1e-5
