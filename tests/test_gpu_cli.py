"""The drop-in binary (bin/treesa_gpu) end to end on the GPU.

* Device-side selection (scheme indep: energies, scores and the best-chain snapshot stay on the GPU) returns
  exactly what the host-side level loop returns (--host-select), for both orders.
* --check passes: valid trees, maintained labels equal the topology's, the energy kernel agrees with the host
  double computation, and the LDS and global kernel mappings are bit-identical
  (the reference's validation matrix parameters, tests/run_checks.sh:13).
* Every result is valid (exit code 0, valid, labels_ok) and its tc / sc equal the host double recomputation.
"""
import json
import os
import subprocess

import pytest

import common
from treesa_gpu_amd import capi, host

pytestmark = pytest.mark.gpu

CHECK_ARGS = ["--check", "--nchains", "48", "--niters", "4", "--betas", "0.2:0.7:7", "--sc-target", "24",
              "--ref-chains", "4", "--seed", "7"]


def run(args, tmp_path, name="out.json"):
    out = str(tmp_path / name)
    print("[cli]", " ".join(args), flush=True)
    p = subprocess.run([capi.BIN_PATH] + args + ["--out", out, "--quiet"], capture_output=True, text=True,
                       timeout=600)
    assert p.returncode == 0, p.stderr[-2000:]
    with open(out) as f:
        return json.load(f)


# sq46 runs the wide path: with chunk summaries (one workgroup per chain: the fold and selection of a level
# run on a second stream beside the next sweep), without (several workgroups per chain: no overlap), and
# without with one workgroup per chain and the selection on the sweep's stream (the sweep launch folds the
# energies itself)
@pytest.mark.parametrize("order", ["par", "preorder"])
@pytest.mark.parametrize("inst,extra", [("sat60", []), ("lat14", []), ("sq46", []), ("sq46", ["--no-sum"]),
                                        ("sq46", ["--no-sum", "--wide-wgs", "1", "--no-overlap"])])
def test_device_selection_equals_host_selection(inst, extra, order, tmp_path):
    args = ["-i", common.inst_path(inst), "--nchains", "96", "--niters", "2", "--betas", "0.01:0.05:15",
            "--sc-target", "30", "--order", order, "--seed", "3"] + extra
    a = run(args, tmp_path, "a.json")
    b = run(args + ["--host-select"], tmp_path, "b.json")
    for k in ("tc", "sc", "best_chain", "tree", "proposals", "accepts", "node_visits", "valid", "labels_ok"):
        assert a[k] == b[k], k
    assert a["valid"] and a["labels_ok"]
    ta = json.loads("[" + json.dumps(a["trace"])[1:-1] + "]")
    tb = json.loads("[" + json.dumps(b["trace"])[1:-1] + "]")
    assert [r[1:5] + r[6:] for r in ta] == [r[1:5] + r[6:] for r in tb]  # all columns but t and meanE
    assert max(abs(x[5] - y[5]) for x, y in zip(ta, tb)) < 1e-9


# The selection of each level runs on a second stream beside the next level's sweep, on a snapshot the sweep
# left: with 8192 chains of sat100 (more than twice what the device holds at once) node costs and children
# words, folded by the fold kernel there, the sweep itself split into two launches on two streams; with 256 chains (one wave per compute unit) energies folded by the
# sweep kernel and children words.  The result equals the same run with the selection on the sweep's stream
# and the host-side level loop.
@pytest.mark.parametrize("order", ["par", "preorder"])
@pytest.mark.parametrize("nchains", [8192, 256])
def test_overlapped_selection(nchains, order, tmp_path):
    args = ["-i", common.inst_path("sat100"), "--tree", common.tree_file("sat100", "greedy"), "--nchains",
            str(nchains), "--niters", "1", "--betas", "1:0.5:15", "--sc-target", "20", "--order", order, "--seed", "2"]
    a = run(args, tmp_path, "a.json")
    assert ("fold=apart" in a["hip_kernel"]) == (nchains == 8192), a["hip_kernel"]
    assert ("split_levels=" in a["hip_kernel"]) == (nchains == 8192), a["hip_kernel"]
    # with the fold apart each level's sweep is two launches on two streams; the kernel time is the union of
    # their intervals, so it stays within the loop's wall time
    assert 0.0 < a["kernel_s"] <= a["t_anneal"], (a["kernel_s"], a["t_anneal"])
    b = run(args + ["--no-overlap"], tmp_path, "b.json")
    c = run(args + ["--host-select"], tmp_path, "c.json")
    for k in ("tc", "sc", "best_chain", "tree", "proposals", "accepts", "node_visits", "valid", "labels_ok"):
        assert a[k] == b[k] == c[k], k
    assert a["valid"] and a["labels_ok"]
    ta, tb, tc = ([list(r) for r in x["trace"]] for x in (a, b, c))
    assert [r[1:] for r in ta] == [r[1:] for r in tb]  # device-side runs: every column but the time
    assert [r[1:5] + r[6:] for r in ta] == [r[1:5] + r[6:] for r in tc]
    assert max(abs(x[5] - y[5]) for x, y in zip(ta, tc)) < 1e-9


# The wide path with one workgroup per chain and more chains than compute units (MI355X: 256): the sweep launch
# folds the energies into the level's snapshot slot beside the tree, and the selection runs on a second stream
# beside the next sweep.  The result equals the same run with the selection after each sweep on its stream and
# the host-side level loop.
def test_wide_selection_beside_the_sweep(tmp_path):
    args = ["-i", common.inst_path("sq46"), "--nchains", "320", "--niters", "1", "--betas", "0.5:0.5:4",
            "--sc-target", "30", "--order", "par", "--seed", "4", "--no-sum", "--wide-wgs", "1"]
    a = run(args, tmp_path, "a.json")
    b = run(args + ["--no-overlap"], tmp_path, "b.json")
    c = run(args + ["--host-select"], tmp_path, "c.json")
    for k in ("tc", "sc", "best_chain", "tree", "proposals", "accepts", "node_visits", "valid", "labels_ok"):
        assert a[k] == b[k] == c[k], k
    assert a["valid"] and a["labels_ok"]
    ta, tb, tc = ([list(r) for r in x["trace"]] for x in (a, b, c))
    assert [r[1:] for r in ta] == [r[1:] for r in tb]
    assert [r[1:5] + r[6:] for r in ta] == [r[1:5] + r[6:] for r in tc]
    assert max(abs(x[5] - y[5]) for x, y in zip(ta, tc)) < 1e-9


# The wide path with chunk summaries and one workgroup per chain sweeps blocks of up to 8 levels per launch,
# each evaluated level leaving its node-cost snapshot for the fold and selection beside the next block: the
# same result as one level per launch and as the host-side level loop.
def test_wide_blocks_of_levels(tmp_path):
    args = ["-i", common.inst_path("sq46"), "--nchains", "72", "--niters", "1", "--betas", "0.5:0.5:6",
            "--sc-target", "30", "--order", "par", "--seed", "6", "--wide-wgs", "1"]
    a = run(args, tmp_path, "a.json")
    assert "anneal=level_blocks8" in a["hip_kernel"] and " sums=1 " in a["hip_kernel"], a["hip_kernel"]
    b = run(args + ["--level-blocks", "1"], tmp_path, "b.json")
    assert "anneal=level_blocks" not in b["hip_kernel"], b["hip_kernel"]
    c = run(args + ["--host-select"], tmp_path, "c.json")
    for k in ("tc", "sc", "best_chain", "tree", "proposals", "accepts", "node_visits", "valid", "labels_ok"):
        assert a[k] == b[k] == c[k], k
    ta, tb, tc = ([list(r) for r in x["trace"]] for x in (a, b, c))
    assert [r[1:] for r in ta] == [r[1:] for r in tb]
    assert [r[1:5] + r[6:] for r in ta] == [r[1:5] + r[6:] for r in tc]
    assert max(abs(x[5] - y[5]) for x, y in zip(ta, tc)) < 1e-9


@pytest.mark.parametrize("inst,extra", [("sat100", ["--kernel", "par"]), ("sat100", ["--order", "preorder"]),
                                        ("reg3_250", ["--mode", "h100"]), ("grid24", ["--mode", "gpu"]),
                                        ("sat60", ["--random-slices", "8"]), ("sq46", ["--kernel", "par"]),
                                        ("grid45", ["--kernel", "par", "--mode", "h100"]),
                                        ("grid28", ["--slicing", "--sc-target", "20", "--mode", "h100"])])
def test_check_mode_passes(inst, extra, tmp_path):
    args = [capi.BIN_PATH, "-i", common.inst_path(inst), "--tree", common.tree_file(inst, "greedy")] + CHECK_ARGS + extra
    print("[cli]", " ".join(args), flush=True)
    p = subprocess.run(args, capture_output=True, text=True, timeout=600)
    assert p.returncode == 0 and "CHECK PASSED" in p.stdout, p.stdout + p.stderr


@pytest.mark.parametrize("scheme", ["indep", "pa", "trunc"])
def test_result_is_valid_and_consistent(scheme, tmp_path):
    r = run(["-i", common.inst_path("sat40"), "--nchains", "64", "--niters", "2", "--betas", "0.1:0.5:10",
             "--scheme", scheme, "--slicing", "--sc-target", "24"], tmp_path)
    assert r["valid"] and r["labels_ok"]
    inst = host.Instance(common.inst_path("sat40"))
    lay = capi.layout(inst.m, inst.nlab)
    import numpy as np
    rec = np.zeros(lay.chain_words, np.uint64)
    ch = np.array([a | (b << 16) for a, b in r["tree"]], np.uint32)
    rec[lay.ch_off:].view(np.uint32)[:lay.nint] = ch
    rec[:lay.nint * lay.W] = inst.labels(ch, lay.W).reshape(-1)
    for l in r["sliced"]:
        rec[lay.s_off + (l >> 6)] |= np.uint64(1) << np.uint64(l & 63)
    tc, sc, _, _, ns = inst.host_energy(lay, rec, slicing=True)
    assert abs(tc - r["tc"]) < 1e-6 and sc == r["sc"] and ns == r["nsliced"] and sc <= 24


# --init spectral / greedy make the start trees natively; the run equals the same trees passed as a --tree file
@pytest.mark.parametrize("inst,init", [("sat60", "spectral"), ("lat14", "spectral"), ("reg3_250", "greedy")])
def test_native_start_trees_equal_tree_file(inst, init, tmp_path):
    from treesa_gpu_amd import host as S
    m, nlab, ixs, iy = common.load_instance(inst)
    if init == "spectral":
        so = S.spectral_orders(ixs, iy, k=3, seed=5)
        trees, tcs = [S.path_tree(o) for _, _, o in so], [t for t, _, _ in so]
        extra = ["--init", "spectral", "--spectral-k", "3"]
    else:
        g = S.greedy_tree(ixs, iy, nrepeat=4, seed=5)
        trees, tcs = [g], None
        extra = ["--init", "greedy", "--greedy-repeat", "4"]
    tf = str(tmp_path / "t.tree")
    S.write_trees(tf, trees)
    base = ["-i", common.inst_path(inst), "--nchains", "64", "--niters", "1", "--betas", "1:0.5:15",
            "--sc-target", "30", "--seed", "5"]
    a = run(base + extra, tmp_path, "a.json")
    b = run(base + ["--tree", tf], tmp_path, "b.json")
    for k in ("tc", "sc", "best_chain", "tree", "proposals", "accepts", "valid", "labels_ok"):
        assert a[k] == b[k], k
    assert a["valid"] and a["labels_ok"] and a["init"] == init
    if tcs is not None:
        assert a["init_tcs"] == [round(t, 4) for t in tcs]
