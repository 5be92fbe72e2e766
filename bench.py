#!/usr/bin/env python3
"""Throughput of the TreeSA sweep path on one MI355X (node visits/s), with its roofline and a CPU baseline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--reps R] [--config c2] [--no-cpu]

Workload (default c2, the headline): random 3-SAT n=100 (m=426 clause tensors, 100 labels,
tests/golden/data/sat100.txt), par-order sweeps of 8192 independent chains starting from the reference's three
spectral path trees (tests/golden/data/sat100_multi.tree, trees 1-3, chain c from tree c % 3), beta linear
1.0 -> 15 over 200 levels of one sweep each, tc energy with sc_target 20, best-of-N selection.  One step is one
level exactly as the drop-in binary runs it: one sweep kernel over all chains, the energy kernel, the host
score loop, and a download of the best chain when it improves.  The population is uploaded before the timed
region; K steps run levels 0..K-1 of the schedule (wrapping after 200).

The timed region is the drop-in binary's own level loop (bin/treesa_gpu, t_anneal: after the population is
resident in HBM, until the last level's energies are back), after --bench-warmup W untimed levels.
value = K * nchains * (m - 1) / that wall time (whole job), of the median of R runs (default 5; their results are
identical, their spread is reported as "repetitions").
kernel_visits_per_s = the reference's own definition (bench/throughput.py:64-70): node visits over the
event-timed sweep kernels only.

roofline: of the sweep kernel, per launch, with the resource that bounds it.  Where the binary runs the level
loop in one launch (scheme indep with every chain resident at once: c1) a launch is the whole schedule
(levels_per_launch); where it sweeps blocks of K levels per launch (scheme indep with more than twice the chains
the device holds at once: c2, "anneal=level_blocksK") a launch is K levels (the schedule's last block may be
shorter: the figures are averages over the run's launches, and the HBM traffic is the committed summary's per
level times the levels per launch); else one level.  Chains staged in LDS (c1-c3):
bound "lds", achieved = the algorithmic bytes of the proposals (5 label sets of W words + 8 B of children per
proposal, W words + 8 B written per accept, 4 B per visit without a rule, plus the slice steps' tree passes;
from the kernel's own counters), all served from LDS, over the average event-timed launch, against the LDS read
peak measured on this GPU by bin/lds_peak; beside it the same kernel's measured HBM traffic against 8 TB/s and
its VALUBusy from the committed rocprof summary.  Label sets streamed from HBM (c4, c5 --no-sum): bound "hbm",
the algorithmic bytes against 8 TB/s.  The chunk-summary kernel (c5 default) reads only the nonzero 16-byte
chunks: achieved = the bytes it loaded (its chunk counters), never the dense per-proposal figure.
cpu_baseline: the reference's own CPU port (csrc/cpu_ref.h, oracle/_ref/ref_harness) under OpenMP on the host's
cores (up to 16, the GPU's share of the host), over a bounded sample of the same workload (a subset of the
chains -- half from each end of the population, so that both launches of a split level are sampled -- every
level); the one-core rate beside it.  Slicing runs (c3) time the oracle port's whole level loop (the reference's
CPU port has no slice moves).
parity: the same CPU runs double as the full-size check.  The binary's final population of the whole schedule
(of the timed run, or of full_schedule when --steps is shorter; written after its timed loop) must equal the
reference harness's final trees chain by chain -- children words and label sets of every sampled chain, and
with the whole population sampled the proposal and accept totals -- or, for c3, every word of every record of
the oracle port's level loop: {"chains": N, "mismatches": 0, ...}.
full_schedule (when --steps is shorter than the workload's schedule): the whole schedule, once.
quality: best log2 tc at fixed wall time on random 3-SAT n=100 against the reference's published figure
(docs/REPORT.md:399-400: population annealing, 576 chains x 200 sweeps per level, tc 66.51 in 2.1 s, sc target
30, Quadro RTX 6000, one run): the same instance, start tree (its omeco greedy tree), schedule (0.01:0.05:15, 300
levels) and sc target, as mean +- sd over 5 seeds of 1152 chains with as many sweeps per level as fit in 2.1 s
of end-to-end wall time (the binary's whole process, as the reference's figure includes its process start and
I/O), and of the reference's own 576 x 200 configuration on this GPU.
long_variant (c1 and c5, whose literal runs are 1.1e7 and 5.9e6 node visits): the same workload with its schedule
repeated ten times, so that the level loop's fixed costs are spread over more levels; reported beside value.
reference_workload (c1): the reference's own sweep-rate benchmark (bench/throughput.py:21-37: sat100, its greedy
tree, 4 sweeps per level over 0.01:0.05:15, sc target 30, energies every 50 levels, pre-order) at 72 and 576
chains, sweeps/s per chain and node visits/s from the sweep kernels' time as that script computes them, beside
its published pre-order figures (bench/results/throughput_rtx6000.txt:26-27, Quadro RTX 6000).
"""
import argparse
import json
import os
import platform
import re
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from treesa_gpu_amd import capi, host  # noqa: E402

DATA = os.path.join(ROOT, "tests", "golden", "data")
METRIC = "node visits/sec on 1 MI355X, random 3-SAT n=100; best log2 tc at fixed wall time"
HBM_PEAK_GBS = 8000.0


def linear_betas(a, b, n):
    return [float(np.float32(a + i * (b - a) / (n - 1))) for i in range(n)]


CONFIGS = {
    # the reference's CPU-runnable check case: greedy start, pre-order, 256 chains x 100 sweeps
    "c1": dict(long=10, cpu_chains=256, inst="sat100", trees=("sat100.tree", None), order="preorder", nchains=256, levels=100, niters=1,
               betas=(0.01, 15.0), sc_target=20.0, scheme="indep", slicing=False,
               desc="random 3-SAT n=100 (m=426), greedy start, pre-order, 256 chains x 100 sweeps, beta 0.01->15"),
    "c2": dict(cpu_chains=256, inst="sat100", trees=("sat100_multi.tree", (1, 2, 3)), order="par", nchains=8192, levels=200, niters=1,
               betas=(1.0, 15.0), sc_target=20.0, scheme="indep", slicing=False,
               desc="random 3-SAT n=100 (m=426), spectral path starts, par order, 8192 chains x 200 sweeps, "
                    "beta 1->15, best-of-N"),
    "c3": dict(cpu_chains=128, inst="sat70", trees=("sat70_greedy.tree", None), order="par", nchains=2048, levels=20, niters=10,
               betas=(0.01, 15.0), sc_target=24.0, scheme="pa", slicing=True,
               desc="random 3-SAT n=70 (m=298), greedy start, par order, slicing (1 slice move per sweep), "
                    "2048 chains x 200 sweeps, population annealing every 10 sweeps, beta 0.01->15"),
    "c4": dict(cpu_chains=24, inst="reg3_2000", trees=("reg3_2000_spectral.tree", None), order="par", nchains=512, levels=100,
               niters=1, betas=(1.0, 15.0), sc_target=40.0, scheme="indep", slicing=False,
               desc="random 3-regular graph n=2000 (3000 labels, 47 words), spectral path starts, par order, "
                    "512 chains x 100 sweeps, beta 1->15"),
    "c5": dict(long=10, cpu_chains=72, inst="sq64", trees=("sq64_row.tree", None), order="par", nchains=72, levels=20, niters=1,
               betas=(0.01, 15.0), sc_target=70.0, scheme="indep", slicing=False,
               desc="64x64 open lattice (4096 tensors, 8064 labels, 126 words), row-major path start, par order, "
                    "72 chains x 20 sweeps, beta 0.01->15"),
}


def score_tc(lc, sc, sc_target, sc_weight=1.0):
    """Selection score of the reference in tc mode (csrc/treesa_gpu.cu:1740-1746), vectorised."""
    lc = lc.astype(np.float64)
    sc = sc.astype(np.float64)
    out = lc.copy()
    over = (sc > sc_target) & (sc_weight > 0)
    if over.any():
        pen = np.log2(sc_weight) + sc[over] + np.log2(1.0 - np.exp2(sc_target - sc[over]))
        mx = np.maximum(lc[over], pen)
        mn = np.minimum(lc[over], pen)
        out[over] = mx + np.log2(1.0 + np.exp2(mn - mx))
    return out


def setup(cfgname, population=True):
    """The workload: its config, instance, layout, start trees, initial population (None without population),
    sweep configuration, betas and order."""
    C = CONFIGS[cfgname]
    inst = host.Instance(os.path.join(DATA, C["inst"] + ".txt"))
    lay = capi.layout(inst.m, inst.nlab)
    tf, pick = C["trees"]
    trees = inst.read_trees(os.path.join(DATA, tf))
    if pick is not None:
        trees = trees[list(pick)]
    pop = inst.population(lay, trees, C["nchains"], seed=1) if population else None
    cfg = capi.make_config(mode="tc", sc_target=C["sc_target"], seed=1)
    betas = linear_betas(C["betas"][0], C["betas"][1], C["levels"])
    order = capi.ORDER_PAR if C["order"] == "par" else capi.ORDER_PREORDER
    return C, inst, lay, trees, pop, cfg, betas, order


def algorithmic_bytes(st, W, nint, slicing=False, slice_steps=0):
    """From the sweep kernel's counters, per unit of work: a proposal reads 5 label sets (+ S when slicing) and
    8 B of children, an accept writes one set and 8 B, a visit without a rule reads 4 B; a slice step evaluates
    the whole chain once plus once per slice proposal (3 sets + 4 B per node, + S) and scans the internal sets
    once per slice proposal.  The same figure for every kernel, whatever it skips."""
    prop, acc, visits, sprop = st[0], st[1], st[3], st[4]
    b = prop * (40 * W + 8 + (8 * W if slicing else 0)) + acc * (8 * W + 8) + (visits - prop) * 4
    evals = slice_steps + sprop
    b += evals * (24 * W * nint + 4 * nint + 8 * W) + sprop * 8 * W * nint
    return b


def loaded_bytes(st, chunks):
    """What a chunk-summary kernel moves in tc mode: per proposal only the 16-byte chunks of D, O, K and M that
    lie in their union's summary (chunks[0] positions, 64 B each; P's set is not read, its cost and size before
    the move come from the node-cost cache), 8 B of children and 10 B of cache, per accept only P's nonzero
    chunks (chunks[1] x 16 B), 8 B of children and 10 B of cache, per visit without a rule 4 B."""
    prop, acc, visits = st[0], st[1], st[3]
    return chunks[0] * 64 + prop * (8 + 10) + chunks[1] * 16 + acc * (8 + 10) + (visits - prop) * 4


def cached_loaded_bytes(st, W):
    """What the dense wide kernel moves in tc mode, where a visit takes P's cost and size before the move from the
    node-cost cache instead of counting P's set: per proposal 4 label sets, 8 B of children and 10 B of cache
    (two costs, one size), per accept P's set, 8 B of children and 10 B of cache, per visit without a rule 4 B."""
    prop, acc, visits = st[0], st[1], st[3]
    return prop * (32 * W + 8 + 10) + acc * (8 * W + 8 + 10) + (visits - prop) * 4


# committed rocprofv3 summaries by (workload, label-set path: "dense" streaming or chunk "sums")
PROFILES = {("c1", "dense"): "k_sweep_c1_sat100_preorder.md", ("c2", "dense"): "k_sweep_c2_sat100_par.md",
            ("c3", "dense"): "k_sweep_c3_sat70_par_slicing.md", ("c4", "dense"): "k_wide_c4_reg3_2000_par.md",
            ("c5", "dense"): "k_wide_c5_sq64_par.md", ("c5", "sums"): "k_wide_sums_c5_sq64_par.md"}


def label_path(desc):
    """"sums" when the sweep kernel read label sets through chunk summaries, else "dense"."""
    return "sums" if desc.startswith("wide") and " sums=0 " not in desc else "dense"


def measured_traffic(cfgname, path="dense", levels_per_launch=1.0):
    """HBM bytes per sweep-kernel dispatch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary of the
    same workload and path (None when there is none): its traffic_bytes_per_launch, or its
    traffic_bytes_per_level times the levels of a launch."""
    f = PROFILES.get((cfgname, path))
    if not f or not os.path.exists(os.path.join(ROOT, "profiles", f)):
        return None
    with open(os.path.join(ROOT, "profiles", f)) as fh:
        for line in fh:
            if line.strip().startswith("traffic_bytes_per_launch:"):
                return float(line.split(":")[1])
            if line.strip().startswith("traffic_bytes_per_level:"):
                return float(line.split(":")[1]) * levels_per_launch
    return None


def launch_count(desc, steps):
    """Sweep launches of a run of `steps` levels, from the binary's kernel description: one for the level loop in
    one launch, one per block of K levels for "anneal=level_blocksK", else one per level."""
    if desc.endswith("anneal=level_loop"):
        return 1
    m = re.search(r"anneal=level_blocks(\d+)$", desc)
    if m:
        k = int(m.group(1))
        return (steps + k - 1) // k
    return steps


def profile_value(cfgname, key, path="dense"):
    """A "key: value" line of the committed rocprof summary of this workload and path (None when absent)."""
    f = PROFILES.get((cfgname, path))
    if not f or not os.path.exists(os.path.join(ROOT, "profiles", f)):
        return None
    with open(os.path.join(ROOT, "profiles", f)) as fh:
        for line in fh:
            if line.strip().startswith(key + ":"):
                return float(line.split(":")[1])
    return None


_lds_peak = None


def lds_peak_gbs():
    """LDS read bandwidth of this GPU, measured once per run by bin/lds_peak (ds_read_b128 on every compute
    unit)."""
    global _lds_peak
    if _lds_peak is None:
        p = subprocess.run([os.path.join(ROOT, "treesa_gpu_amd", "bin", "lds_peak")], check=True, capture_output=True,
                           text=True)
        _lds_peak = json.loads(p.stdout.strip().splitlines()[-1])
    return _lds_peak


def host_facts():
    """CPU model, logical CPUs and the C library of this host."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    libc = " ".join(platform.libc_ver()) or "unknown"
    return {"cpu_model": model, "nproc": os.cpu_count(), "usable_cpus": len(os.sched_getaffinity(0)), "libc": libc}


def cpu_threads():
    """Threads for the CPU baseline: the CPUs this process may use, at most 16 (one GPU's share of its host)."""
    return max(1, min(16, len(os.sched_getaffinity(0))))


def cpu_port_worker(cfgname, nsample, level_loop_out=None):
    """Timing of the oracle port (slice moves included; threads from OMP_NUM_THREADS) on nsample chains' sweeps;
    prints seconds.  With level_loop_out: the workload's whole level loop instead (every chain, its population
    scheme, the oracle's restatement of csrc/treesa_gpu.cu:1756-1877), the final population saved there."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle as orc
    from common import oracle_population
    C, inst, lay, trees, pop, cfg, betas, order = setup(cfgname, population=False)
    m, nlab, ixs, iy = orc.read_instance_py(os.path.join(DATA, C["inst"] + ".txt"))
    O = orc.Oracle(m, nlab, ixs, iy)
    ocfg = capi.make_config(mode="tc", sc_target=C["sc_target"], seed=1, slicing=C["slicing"], slice_moves=1)
    P = orc.params_from_config(ocfg, inst.leaf_sc, nlab)
    if level_loop_out:
        p0 = oracle_population(O, lay, m, C["nchains"], 1, trees)
        nlev = len(betas)
        t0 = time.perf_counter()
        O.anneal(P, lay, p0, betas, [0] * nlev, [C["niters"]] * nlev, order, scheme=C["scheme"], eval_every=1,
                 sc_target=C["sc_target"], seed=1)
        secs = time.perf_counter() - t0
        np.save(level_loop_out, p0)
        print(secs)
        return
    p0 = oracle_population(O, lay, m, nsample, 1, trees)
    t0 = time.perf_counter()
    for lev, b in enumerate(betas):
        O.sweeps(P, lay, p0, order, b, lev * C["niters"], C["niters"])
    print(time.perf_counter() - t0)


def sample_slots(nchains, n):
    """Chain slots of a CPU sample of n of nchains chains: all of them, or n/2 from each end of the population
    (the split sweep launches of a level take chains [0, h) and [h, nchains) with h about nchains / 2), as
    (first slot, count) ranges."""
    if n >= nchains:
        return [(0, nchains)]
    a = n // 2
    return [(0, a), (nchains - (n - a), n - a)]


def ref_harness_run(C, trees, betas, c0, count, threads):
    """The reference's CPU port (oracle/_ref/ref_harness) on chain slots c0 .. c0 + count - 1 of the workload over
    every level: its JSON (per chain: children, label-set hash, proposal and accept counts; sweep seconds)."""
    ref = os.path.join(ROOT, "oracle", "_ref", "ref_harness")
    with tempfile.TemporaryDirectory() as td:
        tf = os.path.join(td, "trees.txt")
        with open(tf, "w") as f:
            for t in trees:
                for w in t:
                    f.write(f"{int(w) & 0xFFFF} {int(w) >> 16}\n")
        bs = ",".join(repr(b) for b in betas)
        args = [ref, "-i", os.path.join(DATA, C["inst"] + ".txt"), "--tree", tf, "--chains", str(count),
                "--chain0", str(c0), "--niters", str(C["niters"]), "--betas", bs, "--order", C["order"], "--mode",
                "tc", "--sc-target", str(C["sc_target"]), "--seed", "1", "--timing", "--threads", str(threads)]
        return json.loads(subprocess.run(args, check=True, capture_output=True, text=True).stdout)


def port_run(cfgname, nsample, threads, level_loop_out=None):
    """Seconds of the oracle port in a worker process on `threads` threads (see cpu_port_worker)."""
    env = dict(os.environ, OMP_NUM_THREADS=str(threads))
    args = [sys.executable, os.path.abspath(__file__), "--cpu-port-worker", cfgname, "--cpu-chains", str(nsample)]
    if level_loop_out:
        args += ["--cpu-level-loop-out", level_loop_out]
    p = subprocess.run(args, check=True, capture_output=True, text=True, env=env)
    return float(p.stdout.strip().splitlines()[-1])


def load_population(path, nchains, lay):
    """A population file the binary wrote with --dump-population."""
    return np.fromfile(path, dtype="<u8").reshape(nchains, lay.chain_words)


def parity_of(lay, nlab, pop, ref_chains=None, port_pop=None):
    """A final population (nchains x chain_words: the binary's --dump-population file) against the CPU runs of
    the same chains: per chain of the reference harness's output its children and the hash of its label sets
    (ceil(nlab/64) words per set, as the harness hashes them), or whole records against the oracle port's level
    loop."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle as orc
    nchains = pop.shape[0]
    bad = []
    if port_pop is not None:
        bad = [c for c in range(nchains) if not np.array_equal(pop[c], port_pop[c])]
        return {"chains": nchains, "mismatches": len(bad), "first_mismatches": bad[:8],
                "compared": "every word of every chain's record (label sets, children, slice set)"}
    wn = (nlab + 63) // 64
    for ch in ref_chains:
        c = ch["chain"]
        words = np.ascontiguousarray(pop[c, lay.ch_off:]).view(np.uint32)[:lay.nint]
        got = np.stack([words & 0xFFFF, words >> 16], axis=1).reshape(-1)
        lab = pop[c, :lay.nint * lay.W].reshape(lay.nint, lay.W)[:, :wn]
        if not np.array_equal(got, np.array(ch["children"], np.uint32)) or \
                orc.fnv64_bytes(lab.astype("<u8")) != ch["labels_fnv"]:
            bad.append(c)
    return {"chains": len(ref_chains), "mismatches": len(bad), "first_mismatches": bad[:8],
            "compared": "children words and label sets of every sampled chain"}


def cpu_baseline(cfgname, C, inst, lay, trees, betas, nsample, dump=None, gpu=None):
    """The reference's own CPU port (oracle/_ref, csrc/cpu_ref.h) over a sample of the workload's chains and every
    level: under OpenMP on every usable core (up to 16) with nsample chains per core, and on one core with nsample
    chains.  Its trajectories double as the parity check: with dump (the binary's final population of the same
    schedule) every sampled chain must equal the reference's.  Configurations with slice moves (which the
    reference's CPU port lacks) run the oracle port's whole level loop -- every chain, population annealing --
    and compare every record."""
    threads = cpu_threads()
    per_level = len(betas) * C["niters"] * (inst.m - 1)
    ref = os.path.join(ROOT, "oracle", "_ref", "ref_harness")
    parity = None
    if os.path.exists(ref) and not C["slicing"]:
        n_all = min(C["nchains"], nsample * threads)
        ranges = sample_slots(C["nchains"], n_all)
        outs = [ref_harness_run(C, trees, betas, c0, k, threads) for c0, k in ranges]
        secs = sum(o["seconds"] for o in outs)
        kind = "reference"
        secs1 = ref_harness_run(C, trees, betas, 0, nsample, 1)["seconds"]
        chains = [ch for o in outs for ch in o["chains"]]
        if dump:
            parity = parity_of(lay, inst.nlab, load_population(dump, C["nchains"], lay), ref_chains=chains)
            if n_all == C["nchains"] and gpu is not None:
                # the whole population: the proposal and accept counts of every chain add up to the binary's
                parity["proposals"] = [sum(ch["nprop"] for ch in chains), gpu["proposals"]]
                parity["accepts"] = [sum(ch["nacc"] for ch in chains), gpu["accepts"]]
                parity["mismatches"] += (parity["proposals"][0] != parity["proposals"][1]) + \
                    (parity["accepts"][0] != parity["accepts"][1])
        where = " and ".join(f"{c0}..{c0 + k - 1}" for c0, k in ranges)
        sample = (f"{n_all} chains (chain slots {where} of this workload's start) x {len(betas) * C['niters']} "
                  f"sweeps on {threads} threads: {n_all * per_level:.3e} visits in {secs:.1f} s")
    else:
        kind = "port"
        with tempfile.TemporaryDirectory() as td:
            out = os.path.join(td, "port_pop.npy")
            secs = port_run(cfgname, C["nchains"], threads, out if dump else None) if dump else \
                port_run(cfgname, min(C["nchains"], nsample * threads), threads)
            n_all = C["nchains"] if dump else min(C["nchains"], nsample * threads)
            if dump:
                parity = parity_of(lay, inst.nlab, load_population(dump, C["nchains"], lay), port_pop=np.load(out))
        secs1 = port_run(cfgname, nsample, 1)
        sample = (f"{'the whole level loop (every chain, population annealing after every level)' if dump else ''}"
                  f" {n_all} chains x {len(betas) * C['niters']} sweeps with slice moves on {threads} threads: "
                  f"{n_all * per_level:.3e} visits in {secs:.1f} s").strip()
    res = dict(value=n_all * per_level / secs, unit="node visits/s", cores=threads, kind=kind, sample=sample,
               one_core={"value": nsample * per_level / secs1, "sample": f"{nsample} chains, {secs1:.1f} s"},
               host=host_facts())
    if parity is not None:
        res["parity"] = parity
    return res


def copy_calibration(cfgname, reps=10):
    """reps population copies with identity ancestors through the C ABI (tsa_resample, then tsa_wait, whose
    copy kernel k_copy makes the resampling no sweep takes over): every launch reads and writes exactly
    nchains * chain_words * 8 bytes once, the reference point for the FETCH_SIZE / WRITE_SIZE counters."""
    C, inst, lay, trees, pop, cfg, betas, order = setup(cfgname)
    with capi.Context(lay, inst.leaf(lay.W), inst.leaf_sc, cfg, C["nchains"]) as ctx:
        ctx.upload(pop)
        anc = np.arange(C["nchains"], dtype=np.int32)
        for _ in range(reps):
            ctx.resample(anc)
            ctx.wait()
    print(json.dumps({"config": cfgname, "kernel": "k_copy", "launches": reps,
                      "bytes_read_per_launch": C["nchains"] * lay.chain_words * 8,
                      "bytes_written_per_launch": C["nchains"] * lay.chain_words * 8}))


def kernel_label(desc, order):
    """Name of the sweep kernel the binary ran, from its hip_kernel description."""
    o = "par" if order == capi.ORDER_PAR else "pre-order"
    if desc.startswith("wide") and order == capi.ORDER_PAR:
        how = "nonzero 16-byte chunks only (chunk summaries)" if " sums=0 " not in desc else "dense streaming"
        return f"k_wide par, label sets in HBM, {how}, " + desc.split(" ", 1)[1]
    loop = ", the whole level loop in one launch" if desc.endswith("anneal=level_loop") else ""
    m = re.search(r"anneal=level_blocks(\d+)$", desc)
    if m:
        loop = f", blocks of {m.group(1)} levels per launch"
    return f"k_sweep {o}, " + ("chain in LDS" if desc.startswith("lds") else "chain in HBM") + loop


def run_binary(C, trees, betas, steps, warmup, scheme=None, extra=(), dump=None, seed=1):
    """The drop-in binary's level loop on the workload; returns its JSON result.  With dump, the binary also
    writes the final population there (after its timed loop)."""
    with tempfile.TemporaryDirectory() as td:
        tf = os.path.join(td, "trees.txt")
        with open(tf, "w") as f:
            for t in trees:
                for w in t:
                    f.write(f"{int(w) & 0xFFFF} {int(w) >> 16}\n")
        bf = os.path.join(td, "betas.txt")
        with open(bf, "w") as f:
            f.write("\n".join(repr(betas[k % len(betas)]) for k in range(steps)) + "\n")
        out = os.path.join(td, "out.json")
        args = [capi.BIN_PATH, "-i", os.path.join(DATA, C["inst"] + ".txt"), "--tree", tf, "--betas", "file:" + bf,
                "--nchains", str(C["nchains"]), "--niters", str(C["niters"]), "--sc-target", str(C["sc_target"]),
                "--mode", "tc", "--order", C["order"], "--kernel", "auto", "--scheme", scheme or C["scheme"],
                "--seed", str(seed), "--eval-every", "1", "--bench-warmup", str(warmup), "--out", out, "--quiet"]
        if C["slicing"]:
            args += ["--slicing", "--slice-moves", "1", "--slice-every", "1"]
        args += list(extra)
        if dump:
            args += ["--dump-population", dump]
        p = subprocess.run(args, capture_output=True, text=True)
        if p.returncode != 0:
            raise RuntimeError(f"treesa_gpu failed ({p.returncode}): {p.stderr[-2000:]}")
        with open(out) as f:
            return json.load(f)


def reference_workload():
    """The reference's sweep-rate benchmark on sat100 (bench/throughput.py:21-37, 64-70), pre-order."""
    inst = host.Instance(os.path.join(DATA, "sat100.txt"))
    C = dict(inst="sat100", niters=4, sc_target=30.0, order="preorder", scheme="indep", slicing=False)
    trees = inst.read_trees(os.path.join(DATA, "sat100.tree"))
    nlev = 300
    betas = [0.01 + i * 0.05 for i in range(nlev)]  # the binary parses "0.01:0.05:15" into the same floats
    out = []
    published = {72: {"sweeps_per_s_per_chain": 4.48e4, "node_visits_per_s": 1.372e9, "kernel": "warp",
                      "source": "bench/results/throughput_rtx6000.txt:26"},
                 576: {"sweeps_per_s_per_chain": 3.19e4, "node_visits_per_s": 7.805e9, "kernel": "warp",
                       "source": "bench/results/throughput_rtx6000.txt:27"}}
    for nc in (72, 576):
        C["nchains"] = nc
        r = run_binary(C, trees, betas, nlev, 0, "indep", ["--eval-every", "50"])
        ks = r["kernel_s"]
        out.append({"nchains": nc, "sweeps_per_s_per_chain": r["total_sweeps"] / ks,
                    "node_visits_per_s": r["total_sweeps"] * nc * (inst.m - 1) / ks, "kernel_s": ks,
                    "kernel": r.get("hip_kernel"), "best_tc": r["tc"], "reference_rtx6000": published[nc]})
    return out


def quality_at_wall(budget_s, visits_per_s, seeds=(1, 2, 3, 4, 5)):
    """Best log2 tc reached within budget_s of end-to-end wall time on random 3-SAT n=100 (population annealing,
    sc target 30, the omeco greedy start, the 300-level schedule 0.01:0.05:15), as a statistic over seeds:
    * chosen: 1152 chains with as many sweeps per level as fit in the budget (calibrated on the first seed,
      then every seed at that count).  Measured on MI355X over 5 seeds each at this budget: 1152 chains
      66.87 +- 0.35, 2304 chains 67.04 +- 0.33, 576 chains 67.03 +- 0.59, 4608 chains 67.35 +- 0.17,
      truncation 67.46 +- 0.49, independent chains 67.57 +- 0.17;
    * reference_config: the reference's own configuration (576 chains x 200 sweeps per level) on this GPU;
    beside them the reference's single published run (docs/REPORT.md:399-400)."""
    inst = host.Instance(os.path.join(DATA, "sat100.txt"))
    nlev = 300
    betas = [float(np.float32(0.01 + i * 0.05)) for i in range(nlev)]
    trees = inst.read_trees(os.path.join(DATA, "sat100.tree"))

    def one(nchains, niters, seed):
        C = dict(inst="sat100", nchains=nchains, niters=niters, sc_target=30.0, order="par", scheme="pa",
                 slicing=False)
        t0 = time.perf_counter()
        r = run_binary(C, trees, betas, nlev, 0, "pa", seed=seed)
        wall = time.perf_counter() - t0
        return {"seed": seed, "niters": niters, "wall_s": round(wall, 4), "tc": r["tc"], "sc": r["sc"]}

    def stats(runs):
        tcs = [x["tc"] for x in runs]
        mean = sum(tcs) / len(tcs)
        sd = (sum((t - mean) ** 2 for t in tcs) / (len(tcs) - 1)) ** 0.5 if len(tcs) > 1 else 0.0
        return {"tc_mean": mean, "tc_sd": sd, "tc_min": min(tcs), "tc_max": max(tcs), "seeds": len(tcs),
                "wall_max_s": max(x["wall_s"] for x in runs),
                "within_budget": all(x["wall_s"] <= budget_s for x in runs), "runs": runs}

    nchains = 1152
    # sweeps per level from the measured sweep rate, leaving about 0.5 s for the process, the device set-up and
    # the population steps; then up to three corrections towards 90-97 % of the budget
    niters = max(1, int((budget_s - 0.5) * visits_per_s / (nchains * nlev * (inst.m - 1))))
    tries = []
    for _ in range(4):
        t = one(nchains, niters, seeds[0])
        tries.append(t)
        if 0.9 * budget_s <= t["wall_s"] <= 0.97 * budget_s:
            break
        nxt = max(1, int(niters * 0.94 * budget_s / t["wall_s"]))
        if nxt == niters or any(x["niters"] == nxt for x in tries):
            break
        niters = nxt
    fits = [x for x in tries if x["wall_s"] <= budget_s]
    niters = max(x["niters"] for x in fits) if fits else min(x["niters"] for x in tries)
    chosen = [next(x for x in tries if x["niters"] == niters)] + [one(nchains, niters, sd) for sd in seeds[1:]]
    refcfg = [one(576, 200, sd) for sd in seeds]
    return {"metric": "best log2 tc at fixed wall time", "instance": "random 3-SAT n=100 (sat100.txt)",
            "budget_s": budget_s,
            "chosen": dict(stats(chosen), config=f"population annealing, {nchains} chains x {niters} sweeps per "
                           "level, 300 levels 0.01:0.05:15, sc target 30, omeco greedy start (end-to-end wall of "
                           "the binary)", calibration=tries),
            "reference_config": dict(stats(refcfg), config="the reference's configuration on this GPU: population "
                                     "annealing, 576 chains x 200 sweeps per level, same schedule, sc target and "
                                     "start"),
            "reference": {"tc": 66.51, "sc": 62, "wall_s": 2.1, "hardware": "Quadro RTX 6000", "seeds": 1,
                          "config": "population annealing, 576 chains x 200 sweeps per level, same schedule, "
                                    "sc target and start", "source": "docs/REPORT.md:399-400"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="levels timed (default: the workload's schedule)")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--reps", type=int, default=5, help="runs of the workload; the median run is reported")
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-chains", type=int, default=None, help="chains in the CPU sample (default per workload)")
    ap.add_argument("--cpu-port-worker", default=None, help=argparse.SUPPRESS)
    ap.add_argument("--cpu-level-loop-out", default=None, help=argparse.SUPPRESS)
    ap.add_argument("--scheme", default=None, choices=("indep", "pa", "trunc"),
                    help="population scheme (pa resamples every level: its copy kernel moves a known number of "
                         "bytes, which calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--wide-waves", type=int, default=0, help="wide kernel: waves per workgroup (0: automatic)")
    ap.add_argument("--wide-wgs", type=int, default=0, help="wide kernel: workgroups per chain (0: automatic)")
    ap.add_argument("--wide-lanes", type=int, default=0, help="wide kernel: lanes per proposal (0: automatic)")
    ap.add_argument("--sums", default="auto", choices=("auto", "on", "off"),
                    help="wide kernel: chunk summaries (the binary's --sums / --no-sum; auto: on from 64 words)")
    ap.add_argument("--long", type=int, default=None,
                    help="also run the workload over this many times its levels (default: 10 for the short c1 and "
                         "c5, none otherwise; 0 or 1: none)")
    ap.add_argument("--no-overlap", action="store_true",
                    help="fold and selection of a level on the sweep's stream, not beside the next sweep")
    ap.add_argument("--draw-waves", type=int, default=0, choices=(-1, 0, 1),
                    help="pre-order: helper waves draw ahead (1), each visit draws (-1), automatic (0)")
    ap.add_argument("--level-launches", action="store_true",
                    help="scheme indep: one sweep launch and one selection per level instead of the level loop in one "
                         "launch")
    ap.add_argument("--level-loop", action="store_true",
                    help="scheme indep: the level loop in one launch also with more chains than are resident at once")
    ap.add_argument("--no-full", action="store_true", help="no full-schedule record when --steps is shorter")
    ap.add_argument("--no-quality", action="store_true", help="no best-tc-at-fixed-wall-time run (c2)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run identity population copies of the workload (counter calibration)")
    a = ap.parse_args()
    if a.copy_calibration:
        copy_calibration(a.config)
        return
    if a.cpu_port_worker:
        cpu_port_worker(a.cpu_port_worker, a.cpu_chains or 1, a.cpu_level_loop_out)
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        sys.exit("bench.py measures one GPU: chains are independent, and a multi-GPU run would shard them across "
                 "processes (see DESIGN.md); run with --gpus 1")
    C, inst, lay, trees, pop, cfg, betas, order = setup(a.config)
    steps = a.steps or C["levels"]
    nchains = C["nchains"]
    extra = (["--wpc", str(2 * a.wide_waves)] if a.wide_waves else []) + \
        (["--wide-wgs", str(a.wide_wgs)] if a.wide_wgs else []) + \
        (["--wide-lanes", str(a.wide_lanes)] if a.wide_lanes else []) + \
        {"auto": [], "on": ["--sums"], "off": ["--no-sum"]}[a.sums] + (["--no-overlap"] if a.no_overlap else []) + \
        (["--draw-waves", str(a.draw_waves)] if a.draw_waves else []) + \
        (["--level-launches"] if a.level_launches else []) + (["--level-loop"] if a.level_loop else [])
    visits = steps * C["niters"] * nchains * (inst.m - 1)

    # the final population of one run of the whole schedule, for the parity check of the CPU baseline's leg
    tmpdir = tempfile.TemporaryDirectory()
    dump = os.path.join(tmpdir.name, "population.u64") if not a.no_cpu else None

    def measure(extra_args, dump_to=None):
        """a.reps runs of the binary; of the run with the median wall time: its JSON, the sweep kernel's
        algorithmic bytes and mean duration per launch, and the roofline block of that kernel.  The results of
        the runs are identical (same seed); only their timings differ."""
        runs = [run_binary(C, trees, betas, steps, a.warmup, a.scheme, extra_args, dump_to if k == 0 else None)
                for k in range(max(1, a.reps))]
        assert all(x["tc"] == runs[0]["tc"] and x["tree"] == runs[0]["tree"] for x in runs), "runs disagree"
        runs.sort(key=lambda x: x["t_anneal"])
        r = runs[len(runs) // 2]
        r["_spread"] = {"reps": len(runs), "value_min": visits / runs[-1]["t_anneal"],
                        "value_max": visits / runs[0]["t_anneal"]}
        assert r["node_visits"] == visits, (r["node_visits"], visits)
        st = [r["proposals"], r["accepts"], r["warp_steps"], r["node_visits"], r["slice_proposals"]]
        slice_steps = steps * C["niters"] * nchains if C["slicing"] else 0
        desc = r.get("hip_kernel") or ""
        # the level loop in one launch runs every level of the schedule, a block K levels; else one level
        launches = launch_count(desc, steps)
        B = algorithmic_bytes(st, lay.W, inst.m - 1, C["slicing"], slice_steps) / launches
        dur = r["kernel_s"] / launches
        path = label_path(desc)
        traffic = measured_traffic(a.config, path, steps / launches)
        roof = {"kernel": kernel_label(desc, order), "levels_per_launch": steps / launches,
                "algorithmic_bytes_per_launch": B, "avg_launch_ms": dur * 1e3, "traffic": traffic}
        if desc.startswith("lds"):
            # label sets served from LDS: the LDS read peak of this GPU bounds the proposals' reads; HBM carries
            # only the staging of the records, and VALU issue is the resource the kernel actually saturates
            peak = lds_peak_gbs()
            roof.update(bound="lds", achieved=B / dur / 1e9, peak=peak["lds_read_GBps"], unit="GB/s",
                        frac=B / dur / 1e9 / peak["lds_read_GBps"],
                        peak_source="bin/lds_peak on this GPU: ds_read_b128 from every wave of every compute unit")
            if traffic is not None:
                roof["hbm"] = {"achieved": traffic / dur / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                               "frac": traffic / dur / 1e9 / HBM_PEAK_GBS}
            vb = profile_value(a.config, "valu_busy", path)
            if vb is not None:
                roof["valu_busy"] = vb / 100.0
        elif r.get("sum_chunks", 0) > 0:
            # the chunk-summary kernel reads only the nonzero chunks of its sets: what it loaded, from its counters
            L = loaded_bytes(st, (r["sum_chunks"], r["sum_xchunks"])) / launches
            roof.update(bound="hbm", achieved=L / dur / 1e9, peak=HBM_PEAK_GBS, unit="GB/s",
                        frac=L / dur / 1e9 / HBM_PEAK_GBS, loaded_bytes_per_launch=L)
        elif desc.startswith("wide"):
            # dense streaming in tc mode: P's set is never read (its cost and size come from the node-cost cache)
            L = cached_loaded_bytes(st, lay.W) / launches
            roof.update(bound="hbm", achieved=L / dur / 1e9, peak=HBM_PEAK_GBS, unit="GB/s",
                        frac=L / dur / 1e9 / HBM_PEAK_GBS, loaded_bytes_per_launch=L)
        else:
            roof.update(bound="hbm", achieved=B / dur / 1e9, peak=HBM_PEAK_GBS, unit="GB/s",
                        frac=B / dur / 1e9 / HBM_PEAK_GBS)
        return r, roof

    full = steps == C["levels"]  # the timed levels are the whole schedule (else they start it)
    r, roof = measure(extra, dump if full else None)
    dumped = r if full else None
    wall = r["t_anneal"]
    res = {
        "metric": METRIC, "value": visits / wall, "unit": "node visits/s", "n_gpus": 1, "steps": steps,
        "warmup": a.warmup, "ms_per_step": wall * 1e3 / steps, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u64",
        "data": "synthetic: the reference's committed instance and start-tree fixtures, seed 1",
        "config": {"workload": C["desc"], "config": a.config, "nchains": nchains, "levels_timed": steps,
                   "sweeps_per_level": C["niters"], "label_words64": lay.W, "kernel": r.get("hip_kernel"),
                   "scheme": a.scheme or C["scheme"]},
        "kernel_visits_per_s": visits / r["kernel_s"], "sweeps_per_s_per_chain": steps * C["niters"] / r["kernel_s"],
        "slice_proposals": r["slice_proposals"], "slice_accepts": r["slice_accepts"], "nsliced": r["nsliced"],
        "proposals": r["proposals"], "accepts": r["accepts"], "phases": r["warp_steps"],
        "best_tc": r["tc"], "best_sc": r["sc"], "wall_s": wall, "repetitions": r["_spread"],
        "roofline": roof,
    }
    if label_path(r.get("hip_kernel") or "") == "sums" and a.sums == "auto":
        # the summary path reads a few chunks per proposal and is bound by phase latency, not by HBM; the
        # dense streaming kernel on the same workload is the HBM-bound one, measured beside it
        rd, roofd = measure(extra + ["--no-sum"])
        assert rd["tc"] == r["tc"] and rd["tree"] == r["tree"], "dense and summary paths disagree"
        res["dense_streaming"] = {"value": visits / rd["t_anneal"], "ms_per_step": rd["t_anneal"] * 1e3 / steps,
                                  "kernel_visits_per_s": visits / rd["kernel_s"], "kernel": rd.get("hip_kernel"),
                                  "repetitions": rd["_spread"], "roofline": roofd}
    long_k = a.long if a.long is not None else C.get("long", 0)
    if long_k > 1 and a.steps is None:
        # the literal workload is short enough that the level loop's fixed costs (first-level set-up, the final
        # copies) weigh on the rate: the same workload over long_k times the levels, the schedule repeated
        lsteps = steps * long_k
        lv = lsteps * C["niters"] * nchains * (inst.m - 1)
        lruns = sorted((run_binary(C, trees, betas, lsteps, a.warmup, a.scheme, extra) for _ in range(3)),
                       key=lambda x: x["t_anneal"])
        lr = lruns[1]
        res["long_variant"] = {"levels": lsteps, "value": lv / lr["t_anneal"], "ms_per_step": lr["t_anneal"] * 1e3 / lsteps,
                               "kernel_visits_per_s": lv / lr["kernel_s"], "best_tc": lr["tc"],
                               "repetitions": {"reps": 3, "value_min": lv / lruns[-1]["t_anneal"],
                                               "value_max": lv / lruns[0]["t_anneal"]},
                               "note": f"the same workload with its {steps}-level schedule run {long_k} times in a row "
                                       "(median of three runs)"}
    if steps < C["levels"] and not a.no_full:
        # the timed steps are the first levels of the schedule: the whole schedule, once, beside them
        fsteps = C["levels"]
        fv = fsteps * C["niters"] * nchains * (inst.m - 1)
        fr = run_binary(C, trees, betas, fsteps, a.warmup, a.scheme, extra, dump)
        dumped = fr
        res["full_schedule"] = {"levels": fsteps, "value": fv / fr["t_anneal"], "ms_per_step": fr["t_anneal"] * 1e3 / fsteps,
                                "kernel_visits_per_s": fv / fr["kernel_s"], "best_tc": fr["tc"], "best_sc": fr["sc"]}
    if a.config == "c1" and a.steps is None:
        res["reference_workload"] = reference_workload()
    if a.config == "c2" and not a.no_quality:
        res["quality"] = quality_at_wall(2.1, res["kernel_visits_per_s"])
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_baseline(a.config, C, inst, lay, trees, betas,
                                           min(a.cpu_chains or C["cpu_chains"], nchains),
                                           dump if dumped is not None else None, dumped)
        if "parity" in res["cpu_baseline"]:
            res["parity"] = dict(res["cpu_baseline"]["parity"],
                                 run=("the timed run" if full else f"the full_schedule run ({C['levels']} levels)"),
                                 against=res["cpu_baseline"]["kind"])
    tmpdir.cleanup()
    print(json.dumps(res))


if __name__ == "__main__":
    main()
