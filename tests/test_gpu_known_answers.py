"""End-to-end known answers of the reference, replayed through the drop-in binary.

tests/golden/test_python_results_{par,preorder}.txt are the reference's committed outputs of its Python
wrapper test (tests/test_python.py:49-65): treesa_gpu.optimize(ixs, iy, nchains=128, niters=4, sc_target=30,
seed=1, scheme, init, mode) with the default betas 0.01:0.05:15, on sat40 / sat60 / reg3_100 / lat10.  This
test builds the argv that driver.optimize builds (treesa_gpu/driver.py:222-296) and checks tc / sc of the
returned tree, then reads the result as the driver does (treesa_gpu_amd.formats.result_tree): the Python model
times equal the binary's (the reference's own check, tests/test_python.py:60-61) and, for the par order, the
values the reference printed.

Asserted: the independent-chain runs (scheme indep, tc mode, greedy and random starts, both orders).  Their
outcome depends only on the integer tc counts, the Metropolis expf (equal to glibc here) and the selection of
the best chain, so they pin random_tree, both sweep orders and the level loop.  The population runs (pa,
trunc) and the float energy modes also depend on the reference GPU's own log2f / exp2f inside its energy and
sweep kernels, which the reference documents as not bit-exact with its CPU port (docs/REPORT.md:1037-1041);
they are not asserted here (bit-exactness of those paths is pinned against the CPU port instead).
"""
import json
import math
import os
import re
import subprocess

import pytest

import common
from treesa_gpu_amd import capi, formats

pytestmark = pytest.mark.gpu

PAT = re.compile(r"ok   (\w+) (indep|pa|trunc)\s+(greedy|random) ([\w+]+)\s*: valid=True iy=True tc ([\d.]+)==.* "
                 r"sc (\d+)==\d+ time ([\d.e+-]+)==([\d.e+-]+) time2 ([\d.e+-]+)==([\d.e+-]+)")


def known(order):
    out = []
    with open(os.path.join(common.HERE, "golden", f"test_python_results_{order}.txt")) as f:
        for line in f:
            m = PAT.match(line)
            if m and m.group(2) == "indep" and m.group(4) == "tc":
                out.append((order, m.group(1), m.group(3), float(m.group(5)), int(m.group(6)),
                            tuple(m.group(i) for i in (7, 8, 9, 10))))
    return out


CASES = known("par") + known("preorder")


def julia_betas(a=0.01, step=0.05, b=15.0):
    n = int(math.floor((b - a) / step + 1e-9)) + 1
    return [a + i * step for i in range(n)]


def same_printed(x, printed):
    """x printed with %.4e gives the reference's printed value."""
    return f"{x:.4e}" == printed


@pytest.mark.parametrize("order,inst,init,tc,sc,times", CASES, ids=[f"{c[0]}-{c[1]}-{c[2]}" for c in CASES])
def test_driver_argv_reproduces_reference_results(order, inst, init, tc, sc, times, tmp_path):
    bf = tmp_path / "betas.txt"
    bf.write_text("\n".join(repr(float(b)) for b in julia_betas()) + "\n")
    out = str(tmp_path / "out.json")
    args = [capi.BIN_PATH, "-i", common.inst_path(inst)]
    if init == "greedy":
        args += ["--tree", common.tree_file(inst, "greedy")]
    args += ["--betas", "file:" + str(bf), "--nchains", "128", "--niters", "4", "--sc-target", "30.0", "--sc-weight",
             "1.0", "--mode", "tc", "--scheme", "indep", "--order", order, "--kernel", "auto", "--seed", "1",
             "--trunc-frac", "0.25", "--eval-every", "1", "--out", out,
             "--gm", "11900000000000000.0,16000000000000.0,6,6,8,4e-06",
             "--h100-model", "4e-06,12300000000000.0,5.44e-14,7.68e-15,6.37e-14,2.02e-16,1.77e-13,14,1e-12", "--quiet"]
    print("[cli]", inst, order, init, flush=True)
    p = subprocess.run(args, capture_output=True, text=True, timeout=600)
    assert p.returncode == 0, p.stderr[-2000:]
    with open(out) as f:
        r = json.load(f)
    assert r["valid"] and r["labels_ok"]
    assert abs(r["tc"] - tc) < 6e-5 and r["sc"] == sc, (r["tc"], r["sc"])
    # the driver's reading of the result (treesa_gpu/driver.py:313-328): the tree dict and its model times
    # recomputed in Python equal the reference's printed values and the binary's own (1e-5 in log,
    # tests/test_python.py:60-61)
    m, nlab, ixs, iy = common.load_instance(inst)
    tree, info = formats.result_tree(r, ixs, iy)
    assert formats.recompute_outputs(tree, ixs, iy) == tree
    assert abs(info["tc_py"] - r["tc"]) < 1e-4 and info["sc_py"] == r["sc"]
    printed = same_printed(info["gpu_time_py"], times[1]) and same_printed(info["h100_time_py"], times[3])
    print("[times]", order, inst, init, "printed" if printed else "differ",
          f"{info['gpu_time_py']:.4e} {info['h100_time_py']:.4e}", times, flush=True)
    # par: the returned tree is the reference's (its model times print identically).  Pre-order: the tc and
    # sc above are the reference's, but on sat40 / sat60 / lat10 the snapshot picked among trees of that
    # same tc is another one (its h100 time differs): the score that picks it is the float fold of the node
    # costs, which the reference's GPU computes with CUDA's log2f / exp2f and this build with the host libm's
    # (docs/REPORT.md:1037-1041), and pre-order sweeps of these runs reach several trees of equal tc
    if order == "par":
        assert printed, times
    assert abs(math.log(r["gpu_time"]) - math.log(info["gpu_time_py"])) < 1e-5
    assert abs(math.log(r["h100_time"]) - math.log(info["h100_time_py"])) < 1e-5
