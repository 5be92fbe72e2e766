"""The reference's end-to-end known answers as runnable cases (shared by the fixture script, CPU and GPU tests).

tests/golden/test_python_results_{par,preorder}.txt are the outputs of the reference's tests/test_python.py
(sweep order par / preorder).  Every printed run is rebuilt here with the arguments test_python.py passed to
treesa_gpu.optimize and the argv driver.optimize builds from them (treesa_gpu/driver.py:204-296):

  lines  5-56  schemes indep / pa / trunc, greedy and random starts, energy modes tc, gpu, h100 and the
               two-stage tc+gpu / tc+h100 (tests/test_python.py:48-65): 128 chains x 4 sweeps, sc_target 30,
               seed 1, betas 0.01:0.05:15, stage 2 on 1.0 + 0.1 i (i < 40);
  lines 57-62  slicing with pa, tc and tc+h100 (tests/test_python.py:67-90): 128 chains x 3 sweeps, greedy
               start, one slice move per sweep, stage 2 on 3.0 + 0.5 i (i < 26);
  lines 63-66  init="spectral" with spectral_k=3 (tests/test_python.py:105): 96 chains x 3 sweeps, betas
               1.0:0.05:15;
  lines 67-69  select="sc" against "score" (tests/test_python.py:118-130): 192 chains x 3 sweeps, sc_weight 4,
               seed 3, and the unconstrained pair (96 x 2, sc_target 1000, seed 5), spectral starts.

Greedy starts are the reference's committed omeco trees (tests/golden/data/<inst>.tree).  Spectral starts are
computed as treesa_gpu/spectral.py:136-199 computes them: the clique-expansion Laplacian (each tensor pair
once, weight 1/(k-1) per shared label of k holders), numpy.linalg.eigh, numpy.random.default_rng(seed)
directions, and the candidate search of treesa_gpu_amd.host.spectral_search (pinned against the reference's
printed orders in tests/test_starts.py).
"""
import json
import math
import os
import re

import numpy as np

import common
import oracle as orc

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "level_loop_answers.json")


def julia_betas(a=0.01, step=0.05, b=15.0):
    n = int(math.floor((b - a) / step + 1e-9)) + 1
    return [a + i * step for i in range(n)]


RUN_PAT = re.compile(r"ok   (\w+) (indep|pa|trunc)\s+(greedy|random) ([\w+]+)\s*: valid=True iy=True tc ([\d.]+)==.* "
                     r"sc (\d+)==\d+ time ([\d.e+-]+)==([\d.e+-]+) time2 ([\d.e+-]+)==([\d.e+-]+)")
SLICE_PAT = re.compile(r"ok   slicing (\w+) ([\w+]+)\s+T=(\d+): .*\|S\|=(\d+) tc/slice ([\d.]+)==.* sc (\d+)==.* "
                       r"total time ([\d.e+-]+)==")
SPEC_PAT = re.compile(r"ok   spectral (\w+): .* init=spectral tc ([\d.]+)==")
SEL_PAT = re.compile(r"ok   select (\w+) T=(\d+): sc-first \(sc (\d+), tc ([\d.]+)\) vs score \(sc (\d+), tc ([\d.]+)\); "
                     r"unconstrained tc ([\d.]+)==([\d.]+)")


def base(order, line, inst, **kw):
    c = dict(id=f"{order}:{line}", order=order, line=line, inst=inst, init="greedy", nchains=128, niters=4,
             betas=julia_betas(), scheme="indep", mode="tc", stage2=None, sc_target=30.0, sc_weight=1.0, seed=1,
             slicing=False, select_sc=False, spectral_k=0)
    c.update(kw)
    return c


def known_answer_cases(order):
    """Every run of the reference's log for one sweep order, with its printed values under "ref"."""
    out = []
    with open(os.path.join(HERE, "golden", f"test_python_results_{order}.txt")) as f:
        lines = f.readlines()
    for ln, text in enumerate(lines, 1):
        m = RUN_PAT.match(text)
        if m:
            inst, scheme, init, mode = m.group(1), m.group(2), m.group(3), m.group(4)
            stage2 = None
            if "+" in mode:
                stage2 = (mode.split("+")[1], [1.0 + 0.1 * i for i in range(40)])
                mode = "tc"
            out.append(base(order, ln, inst, scheme=scheme, init=init, mode=mode, stage2=stage2, kind="run",
                            ref=dict(tc=float(m.group(5)), tc_digits=4, sc=int(m.group(6)), gpu_time=m.group(8),
                                     h100_time=m.group(10))))
            continue
        m = SLICE_PAT.match(text)
        if m:
            inst, mode, T = m.group(1), m.group(2), float(m.group(3))
            stage2 = ("h100", [3.0 + 0.5 * i for i in range(26)]) if mode == "tc+h100" else None
            out.append(base(order, ln, inst, scheme="pa", niters=3, sc_target=T, slicing=True, stage2=stage2,
                            kind="slicing", ref=dict(ns=int(m.group(4)), tc=float(m.group(5)), tc_digits=3,
                                                     sc=int(m.group(6)), h100_time_total=m.group(7))))
            continue
        m = SPEC_PAT.match(text)
        if m:
            out.append(base(order, ln, m.group(1), init="spectral", spectral_k=3, nchains=96, niters=3,
                            betas=julia_betas(1.0, 0.05, 15.0), kind="spectral",
                            ref=dict(tc=float(m.group(2)), tc_digits=4)))
            continue
        m = SEL_PAT.match(text)
        if m:
            inst, T = m.group(1), float(m.group(2))
            common_kw = dict(init="spectral", spectral_k=4, betas=julia_betas(1.0, 0.05, 15.0), kind="select")
            out.append(base(order, ln, inst, nchains=192, niters=3, sc_target=T, sc_weight=4.0, seed=3,
                            select_sc=True, **common_kw, ref=dict(sc=int(m.group(3)), tc=float(m.group(4)),
                                                                    tc_digits=3)))
            out[-1]["id"] += "/sc"
            out.append(base(order, ln, inst, nchains=192, niters=3, sc_target=T, sc_weight=4.0, seed=3,
                            **common_kw, ref=dict(sc=int(m.group(5)), tc=float(m.group(6)), tc_digits=3)))
            out[-1]["id"] += "/score"
            for sel in (False, True):
                out.append(base(order, ln, inst, nchains=96, niters=2, sc_target=1000.0, seed=5, select_sc=sel,
                                **common_kw, ref=dict(tc=float(m.group(7)), tc_digits=4)))
                out[-1]["id"] += "/free-sc" if sel else "/free-score"
    return out


# ---- start trees ---------------------------------------------------------------------------------------
def reference_laplacian(ixs):
    """The Laplacian of the reference's tensor_graph (treesa_gpu/spectral.py:22-44, 56-68): pairs merged in
    first-seen order, degrees accumulated pair by pair."""
    n = len(ixs)
    occ = {}
    for t, ix in enumerate(ixs):
        for l in ix:
            occ.setdefault(l, []).append(t)
    acc = {}
    for ts in occ.values():
        k = len(ts)
        if k < 2:
            continue
        w = 1.0 / (k - 1)
        for i in range(k):
            for j in range(i + 1, k):
                a, b = ts[i], ts[j]
                key = (a, b) if a < b else (b, a)
                acc[key] = acc.get(key, 0.0) + w
    keys = np.array(list(acc.keys()), dtype=np.int64)
    rows, cols, w = keys[:, 0], keys[:, 1], np.array(list(acc.values()))
    deg = np.zeros(n)
    np.add.at(deg, rows, w)
    np.add.at(deg, cols, w)
    L = np.zeros((n, n))
    L[rows, cols] -= w
    L[cols, rows] -= w
    L[np.arange(n), np.arange(n)] += deg
    return L


def spectral_trees(inst, k, seed, nangles=24, nrandom=24):
    """The path trees of the reference's k best spectral orderings for this seed (children words, k x (m-1))."""
    from treesa_gpu_amd import host as S
    m, nlab, ixs, iy = common.load_instance(inst)
    _, V = np.linalg.eigh(reference_laplacian(ixs))
    V = V[:, 1:4]
    rng = np.random.default_rng(seed)
    dirs = []
    for _ in range(nrandom):
        v = rng.standard_normal(3)
        dirs.append(v / np.linalg.norm(v))
    so = S.spectral_search(ixs, iy, V, np.array(dirs), k=k, nangles=nangles)
    return np.array([S.path_tree(o) for _, _, o in so], np.uint32)


SPECTRAL_DIR = os.path.join(HERE, "golden", "spectral_starts")


def spectral_tree_path(inst, k, seed):
    """The committed spectral start trees of a case: computed once, here, by spectral_trees.  numpy's eigh on
    another machine may return other vectors for the degenerate eigenvalues of the lattices, hence other
    start trees, so every run of a case reads these."""
    return os.path.join(SPECTRAL_DIR, f"{inst}_k{k}_seed{seed}.tree")


def write_spectral_starts(cases):
    os.makedirs(SPECTRAL_DIR, exist_ok=True)
    for c in cases:
        if c["init"] != "spectral":
            continue
        p = spectral_tree_path(c["inst"], c["spectral_k"], c["seed"])
        if os.path.exists(p):
            continue
        trees = spectral_trees(c["inst"], c["spectral_k"], c["seed"])
        assert trees.shape[1] + 1 == common.load_instance(c["inst"])[0]
        with open(p, "w") as f:
            for t in trees:
                for w in t:
                    f.write(f"{int(w) & 0xFFFF} {int(w) >> 16}\n")


def tree_file_for(c, tmpdir):
    """Path of the case's start-tree file (None: random trees)."""
    if c["init"] == "greedy":
        return common.tree_file(c["inst"], "greedy")
    if c["init"] == "spectral":
        p = spectral_tree_path(c["inst"], c["spectral_k"], c["seed"])
        assert os.path.exists(p), f"{p} missing (tests/golden/make_level_loop_answers.py writes it)"
        return p
    return None


# ---- the two runs ---------------------------------------------------------------------------------------
def binary_args(c, binary, tmpdir, out, extra=()):
    """driver.optimize's argv for the case (treesa_gpu/driver.py:252-296)."""
    bf = os.path.join(tmpdir, "betas.txt")
    with open(bf, "w") as f:
        f.write("\n".join(repr(float(b)) for b in c["betas"]) + "\n")
    args = [binary, "-i", common.inst_path(c["inst"])]
    tf = tree_file_for(c, tmpdir)
    if tf:
        args += ["--tree", tf]
    if c["stage2"]:
        b2 = os.path.join(tmpdir, "betas2.txt")
        with open(b2, "w") as f:
            f.write("\n".join(repr(float(b)) for b in c["stage2"][1]) + "\n")
        args += ["--stage2-betas", "file:" + b2, "--stage2-niters", str(c["niters"]), "--stage2-mode", c["stage2"][0]]
    args += ["--betas", "file:" + bf, "--nchains", str(c["nchains"]), "--niters", str(c["niters"]),
             "--sc-target", str(c["sc_target"]), "--sc-weight", str(c["sc_weight"]), "--mode", c["mode"],
             "--scheme", c["scheme"], "--order", c["order"], "--kernel", "auto", "--seed", str(c["seed"]),
             "--trunc-frac", "0.25", "--eval-every", "1", "--out", out,
             "--gm", "11900000000000000.0,16000000000000.0,6,6,8,4e-06",
             "--h100-model", "4e-06,12300000000000.0,5.44e-14,7.68e-15,6.37e-14,2.02e-16,1.77e-13,14,1e-12"]
    if c["slicing"]:
        args += ["--slicing", "--slice-moves", "1", "--slice-every", "1"]
    if c["select_sc"]:
        args += ["--select-sc"]
    return args + ["--quiet"] + list(extra)


MODES = {"tc": 0, "gpu": 1, "h100": 2}


def oracle_run(c, tmpdir):
    """The case on the oracle: the reference's level loop from the same start population, then the binary's
    final verification (labels from the topology, greedy repair with slicing, host energy)."""
    from treesa_gpu_amd import capi
    m, nlab, ixs, iy = common.load_instance(c["inst"])
    O = orc.Oracle(m, nlab, ixs, iy)
    lay = capi.layout(m, nlab)
    tf = tree_file_for(c, tmpdir)
    trees = orc.read_trees_py(tf, m) if tf else None
    pop = common.oracle_population(O, lay, m, c["nchains"], c["seed"], trees)
    betas = [float(np.float32(b)) for b in c["betas"]]
    lmode = [MODES[c["mode"]]] * len(betas)
    lniters = [c["niters"]] * len(betas)
    if c["stage2"]:
        betas += [float(np.float32(b)) for b in c["stage2"][1]]
        lmode += [MODES[c["stage2"][0]]] * len(c["stage2"][1])
        lniters += [c["niters"]] * len(c["stage2"][1])
    cfg = capi.make_config(mode=c["mode"], sc_target=c["sc_target"], sc_weight=c["sc_weight"], seed=c["seed"],
                           slicing=c["slicing"], slice_moves=1, slice_every=1)
    P = orc.params_from_config(cfg, max(len(x) for x in ixs), nlab)
    r = O.anneal(P, lay, pop, betas, lmode, lniters, 0 if c["order"] == "par" else 1, scheme=c["scheme"],
                 select_sc=c["select_sc"], sc_target=c["sc_target"], sc_weight=c["sc_weight"], seed=c["seed"])
    best = r["best_rec"].copy()
    ch = np.ascontiguousarray(best[lay.ch_off:]).view(np.uint32)[:m - 1]
    best[:lay.nint * lay.W] = O.labels(ch, lay.W).reshape(-1)
    n_repair = O.repair(lay, best, c["sc_target"]) if c["slicing"] else 0
    tc, sc, t1, t2, ns = O.host_energy(lay, best, c["slicing"], orc.DEFAULT_GM, orc.DEFAULT_H100)
    S = best[lay.s_off:lay.s_off + lay.W]
    sliced = [l for l in range(nlab) if c["slicing"] and int(S[l >> 6]) >> (l & 63) & 1]
    return dict(tc=tc, sc=sc, ns=ns, gpu_time=t1, h100_time=t2, h100_time_total=t2 * 2.0 ** ns, n_repair=n_repair,
                tree=[[int(w & 0xFFFF), int(w >> 16)] for w in ch], sliced=sliced, best_chain=r["best_chain"],
                nresample=r["nresample"], levels=r["levels"], anc=r["anc"])


def tree_hash(tree):
    return common.fnv64(np.array([a | (b << 16) for a, b in tree], "<u4").tobytes())


def agrees_with_reference(c, got):
    """The printed values of the reference's log reproduce: tc to the printed digits, sc, |S| with slicing."""
    ref = c["ref"]
    ok = round(got["tc"], ref["tc_digits"]) == round(ref["tc"], ref["tc_digits"]) or \
        abs(got["tc"] - ref["tc"]) < 0.6 * 10.0 ** -ref["tc_digits"]
    if "sc" in ref:
        ok = ok and got["sc"] == ref["sc"]
    if "ns" in ref:
        ok = ok and got["ns"] == ref["ns"]
    return ok


def load_fixture():
    with open(FIXTURE) as f:
        return json.load(f)
