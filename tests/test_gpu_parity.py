"""GPU parity: the HIP kernels (through the C ABI) against the oracle, bit for bit.

Every golden case of the reference's validation matrix (tests/run_checks.sh parameters, 48 chains) runs on
the GPU and in the oracle from the same initial records; the final records (children, label sets, slice
sets) and the proposal / accept counts must be identical, the first four chains must also match the
reference CPU port's hashes (tests/golden/ref_sweeps.json), and the energy kernel must return exactly the
oracle's 32-lane fold.  Slice moves (no reference CPU twin) are compared with the oracle's mirror.
"""
import numpy as np
import pytest

import common
import oracle as orc
from treesa_gpu_amd import capi

pytestmark = pytest.mark.gpu

NCHAINS = 48


def leaf_sets(m, ixs, W):
    leaf = np.zeros((m, W), np.uint64)
    for i, ix in enumerate(ixs):
        for l in ix:
            leaf[i, l >> 6] |= np.uint64(1) << np.uint64(l & 63)
    return leaf


class Case:
    def __init__(self, inst, order, mode, init="greedy", random_slices=0, par_follow=False, par_band=0, slicing=False,
                 slice_moves=1, slice_every=1, nchains=NCHAINS, kernel=capi.KERNEL_AUTO, wide=False, seed=None,
                 sc_target=None, wide_waves=0, wide_wgs=0, sums=0, lanes=0, data=None, draw_waves=0, wide_join=0):
        """inst names a fixture; data = (m, nlab, ixs, iy) gives an instance directly (then init must be a
        start-tree kind without fixture, e.g. "random")."""
        self.inst, self.order = inst, order
        m, nlab, ixs, iy = common.load_instance(inst) if data is None else data
        self.m, self.nlab, self.ixs = m, nlab, ixs
        self.O = orc.Oracle(m, nlab, ixs, iy)
        self.lay = capi.layout(m, nlab, wide)
        seed = common.CHECK_SEED if seed is None else seed
        tf = common.tree_file(inst, init) if data is None else None
        trees = orc.read_trees_py(tf, m) if tf else None
        self.pop0 = common.oracle_population(self.O, self.lay, m, nchains, seed, trees, random_slices)
        sl = slicing or random_slices > 0
        self.cfg = capi.make_config(mode=mode, sc_target=common.CHECK_SC_TARGET if sc_target is None else sc_target,
                                    seed=seed, slicing=sl, slice_moves=slice_moves if slicing else 0,
                                    slice_every=slice_every, par_follow=par_follow, par_band=par_band, kernel=kernel,
                                    wide_waves=wide_waves, wide_wgs=wide_wgs, sums=sums, wide_lanes=lanes,
                                    draw_waves=draw_waves, wide_join=wide_join)
        self.leaf_sc = max(len(x) for x in ixs)
        self.P = orc.params_from_config(self.cfg, self.leaf_sc, nlab)
        self.leaf = leaf_sets(m, ixs, self.lay.W)
        self.nchains = nchains
        self.ord = capi.ORDER_PAR if order == "par" else capi.ORDER_PREORDER

    def run_gpu(self, betas=common.CHECK_BETAS, niters=common.CHECK_NITERS):
        print(f"[gpu] {self.inst} {self.order} mode={self.cfg.mode} slicing={self.cfg.slicing} "
              f"kernel={self.cfg.kernel} W={self.lay.W} chains={self.nchains} wide_waves={self.cfg.wide_waves} "
              f"wide_wgs={self.cfg.wide_wgs} sums={self.cfg.sums} lanes={self.cfg.wide_lanes} "
              f"draw_waves={self.cfg.draw_waves} wide_join={self.cfg.wide_join}", flush=True)
        with capi.Context(self.lay, self.leaf, self.leaf_sc, self.cfg, self.nchains) as ctx:
            ctx.upload(self.pop0)
            for lev, b in enumerate(betas):
                ctx.sweeps(self.ord, b, lev * niters, niters)
            ctx.sweeps_ms()
            pop = ctx.download()
            st = ctx.stats()
            en = ctx.energy()
            desc = ctx.describe()
        return pop, st, en, desc

    def run_oracle(self, betas=common.CHECK_BETAS, niters=common.CHECK_NITERS):
        pop = self.pop0.copy()
        tot = [0] * 6
        for lev, b in enumerate(betas):
            st = self.O.sweeps(self.P, self.lay, pop, self.ord, b, lev * niters, niters)
            tot = [a + x for a, x in zip(tot, st)]
        return pop, tot, self.O.energy(self.P, self.lay, pop)


def compare(case, gpu, ora):
    gpop, gst, gen, desc = gpu
    opop, ost, oen = ora
    bad = [c for c in range(case.nchains) if not np.array_equal(gpop[c], opop[c])]
    assert not bad, f"{len(bad)}/{case.nchains} chains differ from the oracle (first {bad[:5]}) [{desc}]"
    assert gst[0] == ost[0] and gst[1] == ost[1], f"proposals/accepts gpu {gst[:2]} oracle {ost[:2]}"
    assert gst[3] == ost[3], "node visits"
    assert gst[4] == ost[4] and gst[5] == ost[5], "slice proposals/accepts"
    glc, gsc, gns = gen
    olc, osc, ons = oen
    assert np.array_equal(glc.view(np.uint32), olc.view(np.uint32)), "energy kernel lcost differs from the oracle"
    assert np.array_equal(gsc, osc) and np.array_equal(gns, ons)


@pytest.mark.parametrize("golden", common.golden_cases(), ids=common.case_id)
def test_sweeps_match_oracle_and_reference(golden):
    rs, pf, pb = common.case_options(golden)
    case = Case(golden["inst"], golden["order"], golden["mode"], golden["init"], random_slices=rs, par_follow=pf,
                par_band=pb)
    gpu = case.run_gpu()
    compare(case, gpu, case.run_oracle())
    for c, want in enumerate(golden["chains"]):
        chf, labf = common.record_hashes(gpu[0][c], case.lay, case.nlab)
        assert (chf, labf) == (want["children_fnv"], want["labels_fnv"]), f"chain {c} vs the reference CPU port"


@pytest.mark.parametrize("inst,order,mode", [("sat100", "par", "tc"), ("sat100", "preorder", "h100"),
                                             ("lat14", "par", "gpu"), ("reg3_250", "preorder", "tc")])
def test_lds_and_global_kernels_agree(inst, order, mode):
    a = Case(inst, order, mode, kernel=capi.KERNEL_LDS)
    b = Case(inst, order, mode, kernel=capi.KERNEL_GLOBAL)
    ga, gb = a.run_gpu(), b.run_gpu()
    assert ga[3].startswith("lds") and gb[3].startswith("global")
    assert np.array_equal(ga[0], gb[0])
    compare(a, ga, a.run_oracle())


# Pre-order sweeps with helper waves drawing each sweep's Philox words and Metropolis thresholds ahead
# (accept iff -beta*dE >= threshold) against each visit drawing its own and evaluating expf: both equal the
# oracle bit for bit, with the helpers forced on beyond one chain per compute unit and off below it, in every
# energy mode, on LDS and global-memory records, with slice moves.
@pytest.mark.parametrize("inst,mode,nchains,draw,kernel,slicing", [
    ("sat100", "tc", 300, 1, capi.KERNEL_AUTO, False), ("sat100", "tc", 300, -1, capi.KERNEL_AUTO, False),
    ("sat100", "gpu", 40, -1, capi.KERNEL_AUTO, False), ("lat14", "h100", 40, 1, capi.KERNEL_AUTO, False),
    ("reg3_250", "tc", 40, 1, capi.KERNEL_GLOBAL, False), ("sat60", "tc", 40, 1, capi.KERNEL_AUTO, True)])
def test_draw_waves_match_oracle(inst, mode, nchains, draw, kernel, slicing):
    case = Case(inst, "preorder", mode, nchains=nchains, kernel=kernel, draw_waves=draw, slicing=slicing,
                sc_target=20 if slicing else None)
    gpu = case.run_gpu()
    compare(case, gpu, case.run_oracle())


@pytest.mark.parametrize("inst,order,mode,moves,every", [("sat100", "par", "tc", 1, 1), ("sat100", "preorder", "tc", 2, 1),
                                                         ("grid24", "par", "h100", 1, 2), ("sat60", "par", "tc", 3, 1),
                                                         ("reg3_250", "par", "gpu", 1, 1)])
def test_slice_moves_match_oracle_mirror(inst, order, mode, moves, every):
    case = Case(inst, order, mode, slicing=True, slice_moves=moves, slice_every=every, sc_target=20)
    gpu = case.run_gpu()
    assert gpu[1][4] > 0, "no slice proposals"
    compare(case, gpu, case.run_oracle())


# The wide kernel (runtime-width chains, par order): every plan -- one workgroup per chain, or K co-resident
# workgroups per chain with chain barriers; dense streaming (sums -1) or chunk summaries (sums 1) with 1, 2,
# 4, 8 or 16 lanes per proposal -- gives the oracle's phase-by-phase sweep bit for bit, and so does its
# two-step energy kernel.
@pytest.mark.parametrize("inst,mode,waves,wgs,follow,band,sums,lanes", [
    ("sq46", "tc", 0, 0, False, 0, -1, 0), ("sq46", "tc", 16, 1, False, 0, -1, 0), ("sq46", "tc", 4, 1, True, 0, -1, 0),
    ("sq46", "gpu", 8, 3, False, 3, -1, 0), ("sq46", "h100", 16, 5, True, 0, -1, 0), ("grid24", "tc", 8, 2, False, 0, -1, 0),
    ("grid24", "gpu", 4, 1, True, 4, -1, 0), ("grid45", "tc", 16, 4, False, 0, -1, 0), ("lat14", "tc", 2, 2, False, 0, -1, 0),
    ("sq46", "tc", 0, 0, False, 0, 0, 0), ("sq46", "tc", 8, 1, False, 0, 1, 4), ("sq46", "tc", 4, 3, True, 0, 1, 16),
    ("sq46", "gpu", 8, 2, False, 3, 1, 8), ("sq46", "h100", 2, 5, True, 0, 1, 4), ("grid24", "tc", 8, 2, False, 0, 1, 8),
    ("grid45", "tc", 8, 4, False, 0, 1, 16), ("lat14", "tc", 2, 2, False, 0, 1, 4), ("lat14", "gpu", 8, 1, True, 2, 1, 8),
    ("sq46", "tc", 8, 2, False, 0, 1, 1), ("sq46", "gpu", 4, 1, True, 0, 1, 2), ("grid45", "h100", 8, 3, False, 2, 1, 1)])
def test_wide_kernel_matches_oracle(inst, mode, waves, wgs, follow, band, sums, lanes):
    case = Case(inst, "par", mode, wide=True, kernel=capi.KERNEL_WIDE, wide_waves=waves, wide_wgs=wgs,
                par_follow=follow, par_band=band, sums=sums, lanes=lanes)
    gpu = case.run_gpu()
    assert gpu[3].startswith("wide"), gpu[3]
    if wgs:
        assert f"blocks/chain={wgs}" in gpu[3], gpu[3]
    if sums:
        assert (" sums=0 " in gpu[3]) == (sums < 0), gpu[3]
    if lanes:
        assert f" G={lanes} " in gpu[3], gpu[3]
    compare(case, gpu, case.run_oracle())


# Several workgroups per chain check in before they sweep it; a chain whose check-in runs out of polls is swept
# by one of its workgroups alone.  Forced: every chain claimed at once (-1), or after a single poll (1, a mix of
# claimed and shared chains): the result is the oracle's bit for bit either way, and the next launch (whose
# check-in words the last workgroup of each chain reset) is too.
@pytest.mark.parametrize("inst,mode,waves,wgs,join", [("sq46", "tc", 8, 3, -1), ("sq46", "gpu", 16, 5, 1),
                                                      ("grid45", "tc", 16, 4, -1), ("grid24", "h100", 8, 2, 1),
                                                      ("lat14", "tc", 2, 2, 1)])
def test_wide_check_in_and_lone_sweeps_match_oracle(inst, mode, waves, wgs, join):
    case = Case(inst, "par", mode, wide=True, kernel=capi.KERNEL_WIDE, wide_waves=waves, wide_wgs=wgs,
                wide_join=join)
    gpu = case.run_gpu()
    assert f"blocks/chain={wgs}" in gpu[3], gpu[3]
    compare(case, gpu, case.run_oracle())


@pytest.mark.parametrize("inst,init,nchains,sums,lanes", [("reg3_2000", None, 6, 0, 0), ("sq64", None, 4, -1, 0),
                                                          ("sq64", None, 4, 0, 0), ("sq64", None, 4, 1, 4),
                                                          ("reg3_2000", None, 6, 1, 8), ("sq64", None, 4, 1, 1),
                                                          ("sq64", None, 4, 1, 2)])
def test_wide_kernel_at_benchmark_widths(inst, init, nchains, sums, lanes):
    # the 3-regular n=2000 graph (48 words) and the 64 x 64 lattice (126 words) from random trees, three
    # levels of one sweep; random trees give unions of up to all 63 chunks, so the summary path also runs
    # its later rounds (more than 2G chunks per proposal)
    case = Case(inst, "par", "tc", init=init, nchains=nchains, kernel=capi.KERNEL_WIDE, sc_target=40, sums=sums,
                lanes=lanes)
    betas = [0.5, 2.0, 8.0]
    gpu = case.run_gpu(betas=betas, niters=1)
    assert gpu[3].startswith("wide"), gpu[3]
    compare(case, gpu, case.run_oracle(betas=betas, niters=1))


# Chunk summaries stay exact across everything that rewrites label sets outside the sweep kernel: an upload,
# a population step (resample) and pre-order sweeps (the one-wave kernel), each followed by more par sweeps.
def test_wide_summaries_across_upload_resample_and_preorder():
    case = Case("sq46", "par", "tc", kernel=capi.KERNEL_WIDE, nchains=24, sums=1, lanes=8, wide_wgs=2)
    rng = np.random.default_rng(5)
    anc = rng.integers(0, case.nchains, case.nchains).astype(np.int32)
    opop = case.pop0.copy()
    print("[gpu] summaries across upload / resample / preorder sq46", flush=True)
    with capi.Context(case.lay, case.leaf, case.leaf_sc, case.cfg, case.nchains) as ctx:
        assert " sums=1 " in ctx.describe()
        ctx.upload(case.pop0)
        ctx.sweeps(capi.ORDER_PAR, 1.0, 0, 2)
        case.O.sweeps(case.P, case.lay, opop, capi.ORDER_PAR, 1.0, 0, 2)
        ctx.resample(anc)
        opop = opop[anc].copy()
        ctx.sweeps(capi.ORDER_PAR, 2.0, 2, 1)
        case.O.sweeps(case.P, case.lay, opop, capi.ORDER_PAR, 2.0, 2, 1)
        ctx.sweeps(capi.ORDER_PREORDER, 3.0, 3, 1)
        case.O.sweeps(case.P, case.lay, opop, capi.ORDER_PREORDER, 3.0, 3, 1)
        ctx.sweeps(capi.ORDER_PAR, 4.0, 4, 1)
        case.O.sweeps(case.P, case.lay, opop, capi.ORDER_PAR, 4.0, 4, 1)
        assert np.array_equal(ctx.download(), opop), "after resample / preorder"
        ctx.upload(case.pop0)
        opop = case.pop0.copy()
        ctx.sweeps(capi.ORDER_PAR, 5.0, 5, 2)
        case.O.sweeps(case.P, case.lay, opop, capi.ORDER_PAR, 5.0, 5, 2)
        assert np.array_equal(ctx.download(), opop), "after a second upload"
        glc, gsc, gns = ctx.energy()
        olc, osc, ons = case.O.energy(case.P, case.lay, opop)
        assert np.array_equal(glc.view(np.uint32), olc.view(np.uint32))
        ck = ctx.chunk_stats()
    assert ck[0] > 0 and ck[1] > 0, ck


# A tc-mode wide visit takes the costs of P and v before the move and P's size from the node-cost cache instead
# of P's set; the cache is rebuilt before the first sweep after an upload, a resample and a switch back from
# another energy mode (whose sweeps neither read nor keep tc costs).  Dense and summary paths, two workgroups
# per chain, no energy call between the steps: the records after every step and the final energies equal the
# oracle's.
@pytest.mark.parametrize("sums", [-1, 1])
def test_wide_cost_cache_across_resample_and_mode_switch(sums):
    case = Case("sq46", "par", "tc", kernel=capi.KERNEL_WIDE, nchains=24, sums=sums, wide_wgs=2)
    Pg = orc.params_from_config(case.cfg, case.leaf_sc, case.nlab)
    Pg.mode = capi.MODES["gpu"]
    rng = np.random.default_rng(11)
    anc = rng.integers(0, case.nchains, case.nchains).astype(np.int32)
    opop = case.pop0.copy()
    print(f"[gpu] cost cache across resample / mode switch sq46 sums={sums}", flush=True)
    with capi.Context(case.lay, case.leaf, case.leaf_sc, case.cfg, case.nchains) as ctx:
        assert ctx.describe().startswith("wide") and (" sums=0 " in ctx.describe()) == (sums < 0)
        ctx.upload(case.pop0)
        ctx.sweeps(capi.ORDER_PAR, 1.0, 0, 2)
        case.O.sweeps(case.P, case.lay, opop, capi.ORDER_PAR, 1.0, 0, 2)
        assert np.array_equal(ctx.download(), opop), "after an upload"
        ctx.resample(anc)
        opop = opop[anc].copy()
        ctx.sweeps(capi.ORDER_PAR, 2.0, 2, 1)
        case.O.sweeps(case.P, case.lay, opop, capi.ORDER_PAR, 2.0, 2, 1)
        assert np.array_equal(ctx.download(), opop), "after a resample"
        ctx.set_mode("gpu")
        ctx.sweeps(capi.ORDER_PAR, 3.0, 3, 1)
        case.O.sweeps(Pg, case.lay, opop, capi.ORDER_PAR, 3.0, 3, 1)
        ctx.set_mode("tc")
        ctx.sweeps(capi.ORDER_PAR, 4.0, 4, 2)
        case.O.sweeps(case.P, case.lay, opop, capi.ORDER_PAR, 4.0, 4, 2)
        assert np.array_equal(ctx.download(), opop), "after a gpu-mode sweep and the switch back"
        glc, gsc, gns = ctx.energy()
        olc, osc, ons = case.O.energy(case.P, case.lay, opop)
        assert np.array_equal(glc.view(np.uint32), olc.view(np.uint32))
        assert np.array_equal(gsc, osc) and np.array_equal(gns, ons)


# Energies from the node-cost cache the wide sweep kernel keeps: after every level the fold of the cached
# costs equals the oracle's evaluation of the same population, in every energy mode, also with a GPU model
# whose m0 != n0 (node costs that depend on the order of the two children).  With one workgroup per chain
# (wgs 1) the sweep launch folds the energies itself once the cache is exact (tc mode: from the first launch;
# the other modes: after the first energy call's full pass); with several, the fold kernel does.
@pytest.mark.parametrize("mode,gm,wgs", [("tc", capi.DEFAULT_GM, 0), ("h100", capi.DEFAULT_GM, 0),
                                         ("gpu", (11.9e15, 1.6e13, 3, 9, 8, 4e-6), 0), ("tc", capi.DEFAULT_GM, 1),
                                         ("h100", capi.DEFAULT_GM, 1), ("gpu", (11.9e15, 1.6e13, 3, 9, 8, 4e-6), 1)])
def test_wide_cached_energies_every_level(mode, gm, wgs):
    case = Case("sq46", "par", mode, kernel=capi.KERNEL_WIDE, nchains=24, wide_wgs=wgs, sums=-1)
    if gm is not capi.DEFAULT_GM:
        case.cfg = capi.make_config(mode=mode, sc_target=common.CHECK_SC_TARGET, seed=common.CHECK_SEED,
                                    kernel=capi.KERNEL_WIDE, gm=gm, wide_wgs=wgs, sums=-1)
        case.P = orc.params_from_config(case.cfg, case.leaf_sc, case.nlab)
    opop = case.pop0.copy()
    print(f"[gpu] cached energies sq46 mode={mode} gm={gm} wgs={wgs}", flush=True)
    with capi.Context(case.lay, case.leaf, case.leaf_sc, case.cfg, case.nchains) as ctx:
        desc = ctx.describe()
        assert " sums=0 " in desc and ("blocks/chain=1 " in desc) == (wgs == 1), desc
        ctx.upload(case.pop0)
        for lev, b in enumerate([0.3, 1.0, 3.0, 10.0]):
            if lev != 1:  # level 1 runs two launches between energies
                ctx.energy()
            ctx.sweeps(case.ord, b, 2 * lev, 2)
            case.O.sweeps(case.P, case.lay, opop, case.ord, b, 2 * lev, 2)
            glc, gsc, gns = ctx.energy()
            olc, osc, ons = case.O.energy(case.P, case.lay, opop)
            assert np.array_equal(glc.view(np.uint32), olc.view(np.uint32)), f"level {lev}: lcost"
            assert np.array_equal(gsc, osc) and np.array_equal(gns, ons), f"level {lev}: sc / ns"
        assert np.array_equal(ctx.download(), opop)


# Fused energies (every sweep launch also leaves the energies of the swept population): after every level
# tsa_energy returns exactly the oracle's evaluation, on the LDS, HBM and wide kernels and both wide plans, with
# the fold in the sweep kernel (fused 1 at these chain counts) or in the fold kernel (fused 2), also with
# fixed slice sets.
@pytest.mark.parametrize("inst,kernel,wgs,mode,fused,rs", [
    ("sat100", capi.KERNEL_LDS, 0, "tc", 1, 0), ("sat60", capi.KERNEL_GLOBAL, 0, "h100", 1, 0),
    ("sat100", capi.KERNEL_LDS, 0, "tc", 2, 0), ("sat60", capi.KERNEL_LDS, 0, "gpu", 2, 0),
    ("sat40", capi.KERNEL_LDS, 0, "tc", 2, 8), ("sat60", capi.KERNEL_GLOBAL, 0, "h100", 2, 0),
    ("sq46", capi.KERNEL_WIDE, 0, "tc", 1, 0), ("sq46", capi.KERNEL_WIDE, 1, "gpu", 1, 0),
    ("grid24", capi.KERNEL_WIDE, 3, "h100", 1, 0)])
def test_fused_energies_every_level(inst, kernel, wgs, mode, fused, rs):
    case = Case(inst, "par", mode, kernel=kernel, nchains=24, wide=kernel == capi.KERNEL_WIDE, random_slices=rs)
    case.cfg = capi.make_config(mode=mode, sc_target=common.CHECK_SC_TARGET, seed=common.CHECK_SEED, kernel=kernel,
                                wide_wgs=wgs, fused_energy=fused, slicing=rs > 0, slice_moves=0)
    opop = case.pop0.copy()
    print(f"[gpu] fused energies {inst} kernel={kernel} wgs={wgs} mode={mode}", flush=True)
    with capi.Context(case.lay, case.leaf, case.leaf_sc, case.cfg, case.nchains) as ctx:
        ctx.upload(case.pop0)
        for lev, b in enumerate([0.3, 1.0, 3.0, 10.0]):
            ctx.sweeps(case.ord, b, 2 * lev, 2)
            case.O.sweeps(case.P, case.lay, opop, case.ord, b, 2 * lev, 2)
            glc, gsc, gns = ctx.energy()
            olc, osc, ons = case.O.energy(case.P, case.lay, opop)
            assert np.array_equal(glc.view(np.uint32), olc.view(np.uint32)), f"level {lev}: lcost"
            assert np.array_equal(gsc, osc) and np.array_equal(gns, ons), f"level {lev}: sc / ns"
        assert np.array_equal(ctx.download(), opop)
        desc = ctx.describe()
    if kernel == capi.KERNEL_WIDE:
        assert desc.startswith("wide") and "fold_stage=" in desc, desc
    else:
        assert ("fold=apart" in desc) == (fused == 2), desc


def test_fold_kernel_at_benchmark_size():
    """8192 chains of the 3-SAT n=100 instance: more than the device holds at once, so the automatic plan
    leaves node costs to the fold kernel; one level against the oracle (records, counts, energies)."""
    case = Case("sat100", "par", "tc", init="multi", nchains=8192)
    case.cfg = capi.make_config(mode="tc", sc_target=20.0, seed=1, fused_energy=True)
    case.P = orc.params_from_config(case.cfg, case.leaf_sc, case.nlab)
    print("[gpu] fold kernel at 8192 chains", flush=True)
    with capi.Context(case.lay, case.leaf, case.leaf_sc, case.cfg, case.nchains) as ctx:
        ctx.upload(case.pop0)
        ctx.sweeps(case.ord, 2.0, 0, 1)
        gen = ctx.energy()
        gpop = ctx.download()
        desc = ctx.describe()
    assert "fold=apart" in desc, desc
    opop = case.pop0.copy()
    case.O.sweeps(case.P, case.lay, opop, case.ord, 2.0, 0, 1)
    oen = case.O.energy(case.P, case.lay, opop)
    assert np.array_equal(gpop, opop)
    assert np.array_equal(gen[0].view(np.uint32), oen[0].view(np.uint32))
    assert np.array_equal(gen[1], oen[1]) and np.array_equal(gen[2], oen[2])


@pytest.mark.parametrize("inst,nchains", [("sq46", 48), ("reg3_2000", 512), ("sq64", 72), ("grid45", 8)])
def test_automatic_plan_takes_the_wide_kernel(inst, nchains):
    # runtime-width chains without slicing must get the wide kernel from the automatic choice (a failed plan
    # would fall back to the one-wave HBM kernel, correct but slow)
    case = Case(inst, "par", "tc", init=None, nchains=nchains)
    with capi.Context(case.lay, case.leaf, case.leaf_sc, case.cfg, case.nchains) as ctx:
        desc = ctx.describe()
    assert case.lay.runtime_width == 1 and desc.startswith("wide"), desc


def test_resample_copies_ancestors():
    case = Case("sat40", "par", "tc")
    rng = np.random.default_rng(3)
    anc = rng.integers(0, case.nchains, case.nchains).astype(np.int32)
    with capi.Context(case.lay, case.leaf, case.leaf_sc, case.cfg, case.nchains) as ctx:
        ctx.upload(case.pop0)
        ctx.sweeps(case.ord, 1.0, 0, 2)
        before = ctx.download()
        ctx.resample(anc)
        after = ctx.download()
    assert np.array_equal(after, before[anc])


# tsa_resample's copy is made by the next sweep launch of the LDS kernels (each chain staged from its ancestor's
# record in the previous population buffer) or by a copy kernel before any other call: a resampling followed by
# sweeps, two resamplings in a row, and one followed by an energy call all give the oracle's records and
# energies, for both orders (pre-order with and without helper waves) and with slice moves.
@pytest.mark.parametrize("order,kw", [("par", {}), ("preorder", {}), ("preorder", {"draw_waves": -1}),
                                      ("par", {"slicing": True})])
def test_resample_taken_over_by_the_next_sweep(order, kw):
    case = Case("sat40", order, "tc", nchains=96, **kw)
    rng = np.random.default_rng(8)
    a1, a2, a3 = (rng.integers(0, case.nchains, case.nchains).astype(np.int32) for _ in range(3))
    opop = case.pop0.copy()
    print(f"[gpu] resample taken over by the next sweep sat40 {order} {kw}", flush=True)
    with capi.Context(case.lay, case.leaf, case.leaf_sc, case.cfg, case.nchains) as ctx:
        ctx.upload(case.pop0)
        ctx.sweeps(case.ord, 1.0, 0, 2)
        case.O.sweeps(case.P, case.lay, opop, case.ord, 1.0, 0, 2)
        ctx.resample(a1)  # taken over by the sweep launch
        opop = opop[a1].copy()
        ctx.sweeps(case.ord, 2.0, 2, 1)
        case.O.sweeps(case.P, case.lay, opop, case.ord, 2.0, 2, 1)
        assert np.array_equal(ctx.download(), opop), "a resampling, then sweeps"
        ctx.resample(a2)  # two in a row: the first copied before the second is staged
        ctx.resample(a3)
        opop = opop[a2][a3].copy()
        ctx.sweeps(case.ord, 3.0, 3, 2)
        case.O.sweeps(case.P, case.lay, opop, case.ord, 3.0, 3, 2)
        assert np.array_equal(ctx.download(), opop), "two resamplings, then sweeps"
        ctx.resample(a1)  # an energy call makes the copy
        opop = opop[a1].copy()
        glc, gsc, gns = ctx.energy()
        olc, osc, ons = case.O.energy(case.P, case.lay, opop)
        assert np.array_equal(glc.view(np.uint32), olc.view(np.uint32)) and np.array_equal(gsc, osc)
        assert np.array_equal(gns, ons)
        assert np.array_equal(ctx.download(), opop), "a resampling, then an energy call"


def test_upload_rejects_invalid_tree():
    case = Case("sat40", "par", "tc", nchains=4)
    bad = case.pop0.copy()
    bad[2, case.lay.ch_off:].view(np.uint32)[5] = 0xFFFF  # node id out of range
    with capi.Context(case.lay, case.leaf, case.leaf_sc, case.cfg, case.nchains) as ctx:
        with pytest.raises(capi.TsaError, match="not a valid tree"):
            ctx.upload(bad)
