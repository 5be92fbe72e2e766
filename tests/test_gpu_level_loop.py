"""The binary's level loop against the oracle's, level by level (GPU).

bin/treesa_gpu runs a whole anneal on the device (sweeps, energies, selection, population steps on the host)
and writes one --level-log line per evaluated level.  tests/oracle.py's anneal() restates the reference's
run_anneal (csrc/treesa_gpu.cu:1756-1877) on the CPU from the same start population: sweeps, the energy fold,
the glibc selection score, population annealing's systematic resampling, truncation selection, the stage
switch of two-stage runs.  Every evaluated level must agree exactly: the best chain, its lc (float bits), sc
and |S|, the score and the mean energy (double bits), the family count and the ancestor list of the
population step; then the final tree, slice set, repair and host-energy tc / sc of the JSON result.

Cases: pa and trunc (tc mode), two-stage tc+gpu / tc+h100, the float modes with pa, select-sc, the tc-mode
penalty branch of the score with host-side selection, slicing with pa and the final repair, --max-slices,
--init-slices, --eval-every, the sat70 slicing workload with population annealing after every 10-sweep level
(2048 x 200 in the benchmark; here 64 chains over all 20 levels), and sat70 with a slice limit and a target the
anneal cannot reach, so that the final repair adds many labels.  The final tc (tc_exact, the JSON's
full-precision key) must equal the oracle's within 1e-9.
"""
import json
import math
import os
import subprocess

import numpy as np
import pytest

import common
import oracle as orc
from treesa_gpu_amd import capi, formats

pytestmark = pytest.mark.gpu


def julia_betas(a=0.01, step=0.05, b=15.0):
    n = int(math.floor((b - a) / step + 1e-9)) + 1
    return [a + i * step for i in range(n)]


def linear_betas(a, b, n):
    return [a + (b - a) * i / (n - 1) for i in range(n)]


def f32(xs):
    return [float(np.float32(x)) for x in xs]


class Case:
    def __init__(self, name, inst, init="greedy", nchains=64, niters=4, betas=None, scheme="pa", mode="tc",
                 stage2=None, sc_target=30.0, sc_weight=1.0, seed=1, slicing=False, max_slices=0, init_slices=None,
                 eval_every=1, select_sc=False, host_select=False, order="par", max_levels=None, min_repair=0):
        self.__dict__.update(locals())
        del self.__dict__["self"]
        self.betas = betas if betas is not None else julia_betas()
        if max_levels:
            self.betas = self.betas[:max_levels]


CASES = [
    Case("sat40-pa-greedy", "sat40", nchains=128),
    Case("sat40-trunc-random", "sat40", init="random", nchains=128, scheme="trunc"),
    Case("sat40-pa-tc+gpu", "sat40", nchains=64, stage2=("gpu", [1.0 + 0.1 * i for i in range(40)]),
         max_levels=120),
    Case("sat40-pa-tc+h100", "sat40", nchains=64, stage2=("h100", [1.0 + 0.1 * i for i in range(40)]),
         max_levels=120),
    Case("reg3_100-pa-h100", "reg3_100", nchains=64, mode="h100", max_levels=150),
    Case("lat10-trunc-preorder", "lat10", nchains=64, scheme="trunc", order="preorder", max_levels=150),
    Case("sat40-indep-host-penalty", "sat40", init="random", nchains=96, scheme="indep", sc_target=24.0,
         host_select=True, max_levels=150),
    Case("sat60-select-sc", "sat60", nchains=96, niters=3, scheme="indep", sc_target=14.0, sc_weight=4.0, seed=3,
         select_sc=True, max_levels=120),
    Case("sat60-slicing-pa", "sat60", nchains=64, niters=3, sc_target=30.0, slicing=True, max_levels=120),
    Case("sat40-slicing-max-init", "sat40", init="random", nchains=64, niters=3, sc_target=20.0, slicing=True,
         max_slices=4, init_slices=[1, 5, 9], max_levels=100),
    Case("sat40-pa-eval3", "sat40", nchains=64, eval_every=3, max_levels=150),
    Case("c3-sat70-slicing-pa", "sat70", nchains=64, niters=10, betas=linear_betas(0.01, 15.0, 20), sc_target=24.0,
         slicing=True),
    # at most 4 slices during the anneal and a target the annealed tree does not reach: the final greedy repair
    # (csrc/treesa_gpu.cu:1248-1274) adds dozens of labels
    Case("sat70-slicing-repair", "sat70", nchains=64, niters=3, sc_target=18.0, slicing=True, max_slices=4,
         max_levels=40, min_repair=3),
]


def tree_path(c):
    if c.init != "greedy":
        return None
    return os.path.join(common.DATA, "sat70_greedy.tree") if c.inst == "sat70" else common.tree_file(c.inst, "greedy")


def run_binary(c, tmp_path):
    bf = tmp_path / "betas.txt"
    bf.write_text("\n".join(repr(float(b)) for b in c.betas) + "\n")
    out, log = str(tmp_path / "out.json"), str(tmp_path / "levels.jsonl")
    args = [capi.BIN_PATH, "-i", common.inst_path(c.inst)]
    if tree_path(c):
        args += ["--tree", tree_path(c)]
    if c.stage2:
        b2 = tmp_path / "betas2.txt"
        b2.write_text("\n".join(repr(float(b)) for b in c.stage2[1]) + "\n")
        args += ["--stage2-betas", "file:" + str(b2), "--stage2-niters", str(c.niters), "--stage2-mode", c.stage2[0]]
    args += ["--betas", "file:" + str(bf), "--nchains", str(c.nchains), "--niters", str(c.niters),
             "--sc-target", str(c.sc_target), "--sc-weight", str(c.sc_weight), "--mode", c.mode,
             "--scheme", c.scheme, "--order", c.order, "--seed", str(c.seed), "--eval-every", str(c.eval_every),
             "--out", out, "--level-log", log, "--quiet"]
    if c.slicing:
        args += ["--slicing", "--slice-moves", "1", "--slice-every", "1"]
        if c.max_slices:
            args += ["--max-slices", str(c.max_slices)]
        if c.init_slices:
            args += ["--init-slices", ",".join(map(str, c.init_slices))]
    if c.select_sc:
        args += ["--select-sc"]
    if c.host_select:
        args += ["--host-select"]
    print("[binary]", c.name, flush=True)
    p = subprocess.run(args, capture_output=True, text=True, timeout=600)
    assert p.returncode == 0, p.stderr[-2000:]
    with open(out) as f:
        res = json.load(f)
    with open(log) as f:
        levels = [json.loads(x) for x in f]
    return res, levels


def run_oracle(c):
    m, nlab, ixs, iy = common.load_instance(c.inst)
    O = orc.Oracle(m, nlab, ixs, iy)
    lay = capi.layout(m, nlab)
    trees = orc.read_trees_py(tree_path(c), m) if tree_path(c) else None
    pop = common.oracle_population(O, lay, m, c.nchains, c.seed, trees)
    if c.init_slices:
        for l in c.init_slices:
            pop[:, lay.s_off + (l >> 6)] |= np.uint64(1) << np.uint64(l & 63)
    betas = f32(c.betas)
    mode0 = capi.MODES[c.mode]
    lmode = [mode0] * len(betas)
    lniters = [c.niters] * len(betas)
    if c.stage2:
        betas += f32(c.stage2[1])
        lmode += [capi.MODES[c.stage2[0]]] * len(c.stage2[1])
        lniters += [c.niters] * len(c.stage2[1])
    cfg = capi.make_config(mode=c.mode, sc_target=c.sc_target, sc_weight=c.sc_weight, seed=c.seed,
                           slicing=c.slicing, slice_moves=1, slice_every=1, max_slices=c.max_slices)
    P = orc.params_from_config(cfg, max(len(x) for x in ixs), nlab)
    print("[oracle]", c.name, flush=True)
    r = O.anneal(P, lay, pop, betas, lmode, lniters, capi.ORDER_PAR if c.order == "par" else capi.ORDER_PREORDER,
                 scheme=c.scheme, eval_every=c.eval_every, select_sc=c.select_sc, sc_target=c.sc_target,
                 sc_weight=c.sc_weight, seed=c.seed)
    # the binary's final verification: labels from the topology, greedy repair with slicing, host energy
    best = r["best_rec"].copy()
    ch = np.ascontiguousarray(best[lay.ch_off:]).view(np.uint32)[:m - 1]
    lab = O.labels(ch, lay.W)
    assert lab is not None
    best[:lay.nint * lay.W] = lab.reshape(-1)
    n_repair = O.repair(lay, best, c.sc_target) if c.slicing else 0
    tc, sc, t1, t2, ns = O.host_energy(lay, best, c.slicing, orc.DEFAULT_GM, orc.DEFAULT_H100)
    r.update(tc=tc, sc=sc, ns=ns, n_repair=n_repair, final=best, lay=lay, m=m, nlab=nlab)
    return r


def f32_bits(x):
    return int(np.float32(x).view(np.uint32))


@pytest.mark.parametrize("c", CASES, ids=[c.name for c in CASES])
def test_level_loop_matches_oracle(c, tmp_path):
    res, blev = run_binary(c, tmp_path)
    r = run_oracle(c)
    olev = r["levels"]
    evaluated = [i for i in range(len(olev)) if olev[i]["evaluated"]]
    device_loop = c.scheme == "indep" and not c.stage2 and not c.host_select
    assert [b["level"] for b in blev] == evaluated
    for b in blev:
        L = b["level"]
        o = olev[L]
        where = f"{c.name} level {L}"
        assert b["best"] == o["best"], where
        assert b["lc_bits"] == f32_bits(o["lc"]), where
        assert (b["sc"], b["ns"]) == (int(o["sc"]), int(o["ns"])), where
        assert b["score"] == float(o["score"]), where
        if device_loop:  # the device sums the energies in its own order
            assert abs(b["meanE"] - float(o["meanE"])) <= 1e-12 * abs(float(o["meanE"])), where
        else:
            assert b["meanE"] == float(o["meanE"]), where
        assert b["families"] == int(o["families"]), where
        assert b["resampled"] == bool(o["resampled"]), where
        if b["resampled"]:
            assert b["anc"] == [int(x) for x in r["anc"][L]], where
    lay, m = r["lay"], r["m"]
    tree = [[int(w & 0xFFFF), int(w >> 16)] for w in np.ascontiguousarray(r["final"][lay.ch_off:]).view(np.uint32)[:m - 1]]
    assert res["tree"] == tree
    assert res["best_chain"] == r["best_chain"]
    assert res["nresample"] == r["nresample"]
    assert res["total_sweeps"] == r["total_sweeps"]
    assert res["valid"] and res["labels_ok"]
    assert abs(res["tc_exact"] - r["tc"]) <= 1e-9 and res["sc"] == r["sc"]
    if c.slicing:
        S = r["final"][lay.s_off:lay.s_off + lay.W]
        sliced = [l for l in range(r["nlab"]) if int(S[l >> 6]) >> (l & 63) & 1]
        assert res["sliced"] == sliced and res["nsliced"] == r["ns"] == len(sliced)
        assert res["n_repair"] == r["n_repair"] >= c.min_repair
        if c.max_slices:
            assert all(b["ns"] <= c.max_slices for b in blev)
    if c.stage2:
        assert r["staged"]
        assert abs(res["stage1_tc_exact"] - r["h1"][0]) <= 1e-9 and res["stage1_sc"] == int(r["h1"][1])
    print("[ok]", c.name, f"tc {res['tc']:.4f} sc {res['sc']} |S| {res['nsliced']} resampled {res['nresample']}",
          flush=True)


def test_c3_full_size_properties(tmp_path):
    """The sat70 slicing workload at its benchmark size -- 2048 chains, 20 levels of 10 sweeps, one slice move
    per sweep, population annealing after every level -- beyond what the oracle replays in test time: the
    returned tree is valid over the sliced network, its label sets are the ones its topology gives, the tc / sc
    / |S| the binary reports equal the driver's recomputation in Python from the tree and the sliced labels,
    population annealing resampled after every level but the last (between 1 and 2048 families per level), and
    the repaired result meets the sc target."""
    c = Case("c3-full", "sat70", nchains=2048, niters=10, betas=linear_betas(0.01, 15.0, 20), sc_target=24.0,
             slicing=True)
    res, blev = run_binary(c, tmp_path)
    assert res["valid"] and res["labels_ok"]
    assert res["total_sweeps"] == 200 and res["nchains"] == 2048
    m, nlab, ixs, iy = common.load_instance("sat70")
    tree, info = formats.result_tree(res, ixs, iy)
    assert abs(info["tc_py"] - res["tc"]) < 1e-4 and info["sc_py"] == res["sc"]
    assert res["nsliced"] == len(res["sliced"]) == len(set(res["sliced"]))
    assert abs(info["tc_total_py"] - (res["tc"] + res["nsliced"])) < 1e-4
    assert res["sc"] <= c.sc_target
    assert [b["level"] for b in blev] == list(range(20))
    assert all(1 <= b["families"] <= 2048 for b in blev)
    assert [b["resampled"] for b in blev] == [True] * 19 + [False]
    assert res["slice_proposals"] > 0
    print("[ok] c3 full size", f"tc {res['tc']:.4f} sc {res['sc']} |S| {res['nsliced']} resampled {res['nresample']}",
          flush=True)
