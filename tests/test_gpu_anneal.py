"""GPU: the level loop in one launch (tsa_anneal) against one sweep launch and one selection per level
(tsa_sweeps + tsa_track), through the C ABI, bit for bit.

Both runs start from the same oracle-built population and sweep the same schedule; the final records, the
statistics, every trace row (lc, sc, |S|, chain, score, mean E, mean |S|: the level loop reduces in k_track's
order, so the means agree to the last bit) and the best chain, level, score and tree must be identical.  The
cases cover both sweep orders, pre-order with and without helper waves, one group of 256 chains and several
with a ragged last one, every energy mode, slicing, the sc-first selection, sparse evaluation, a schedule
split over two calls, the one-launch loop forced on more chains than are resident at once, and the per-level
launches tsa_anneal runs itself (too many chains, a session begun with tsa_track, the wide path).  The per-level
launches of the headline workload (8192 chains, the sweep of each level split over two streams) are compared
with the oracle's level loop directly.  That the
selection itself is the reference's is covered by the level-loop tests, which run the binary (whose indep loop
is this launch) against the oracle's level loop.
"""
import numpy as np
import pytest

import common
import oracle as orc
from test_gpu_parity import leaf_sets
from treesa_gpu_amd import capi

pytestmark = pytest.mark.gpu


class Setup:
    def __init__(self, inst, order, mode="tc", nchains=256, draw_waves=0, slicing=False, random_slices=0,
                 select_sc=False, seed=3, init="greedy", level_loop=0):
        m, nlab, ixs, iy = common.load_instance(inst)
        O = orc.Oracle(m, nlab, ixs, iy)
        self.lay = capi.layout(m, nlab)
        tf = common.tree_file(inst, init)
        trees = orc.read_trees_py(tf, m) if tf else None
        self.pop0 = common.oracle_population(O, self.lay, m, nchains, seed, trees, random_slices)
        sl = slicing or random_slices > 0
        self.cfg = capi.make_config(mode=mode, sc_target=common.CHECK_SC_TARGET, seed=seed, slicing=sl,
                                    slice_moves=1 if slicing else 0, draw_waves=draw_waves, kernel=capi.KERNEL_LDS,
                                    level_loop=level_loop)
        self.leaf_sc = max(len(x) for x in ixs)
        self.leaf = leaf_sets(m, ixs, self.lay.W)
        self.nchains, self.mode, self.sl, self.select_sc = nchains, mode, sl, select_sc
        self.ord = capi.ORDER_PAR if order == "par" else capi.ORDER_PREORDER
        self.name = (f"{inst} {order} {mode} chains={nchains} draw_waves={draw_waves} slicing={sl} sc={select_sc} "
                     f"level_loop={level_loop}")

    def context(self):
        ctx = capi.Context(self.lay, self.leaf, self.leaf_sc, self.cfg, self.nchains)
        ctx.upload(self.pop0)
        return ctx

    def begin(self, ctx, nlev):
        ctx.track_begin(mode=self.mode, slicing=self.sl, select_sc=self.select_sc, sc_target=common.CHECK_SC_TARGET,
                        max_levels=nlev)

    def finish(self, ctx):
        best = ctx.track_end()
        ctx.sweeps_ms()
        return {"pop": ctx.download(), "stats": ctx.stats(), "best": best, "desc": ctx.describe()}

    def per_level(self, betas, niters, evaluated):
        print(f"[gpu] per-level launches: {self.name}", flush=True)
        with self.context() as ctx:
            self.begin(ctx, len(betas))
            sweep = 0
            for lev, (b, k) in enumerate(zip(betas, niters)):
                ctx.sweeps(self.ord, b, sweep, k)
                sweep += k
                if evaluated[lev]:
                    ctx.track(lev)
            return self.finish(ctx)

    def level_loop(self, betas, niters, evaluated, split=None):
        print(f"[gpu] level loop: {self.name} split={split}", flush=True)
        with self.context() as ctx:
            self.begin(ctx, len(betas))
            parts = [(0, len(betas))] if split is None else [(0, split), (split, len(betas))]
            for l0, l1 in parts:
                ctx.anneal(self.ord, betas[l0:l1], niters[l0:l1], evaluated[l0:l1], level0=l0,
                           sweep0=int(sum(niters[:l0])))
            return self.finish(ctx)


def schedule(nlev, niters=1, every=1, b0=0.1, b1=6.0):
    betas = np.linspace(b0, b1, nlev).astype(np.float32)
    ev = [int(l % every == every - 1 or l == nlev - 1) for l in range(nlev)]
    return betas, [niters] * nlev, ev


def compare(s, a, b, evaluated):
    lay = s.lay
    bad = [c for c in range(s.nchains) if not np.array_equal(a["pop"][c], b["pop"][c])]
    assert not bad, f"{len(bad)} chains differ after the schedule (first {bad[:5]}) [{b['desc']}]"
    assert a["stats"] == b["stats"]
    (ac, al, asc, arec, arows, _, _), (bc, bl, bsc, brec, brows, _, _) = a["best"], b["best"]
    assert (ac, al) == (bc, bl) and asc == bsc, ((ac, al, asc), (bc, bl, bsc))
    for lev, e in enumerate(evaluated):
        ra, rb = arows[lev], brows[lev]
        if not e:
            assert rb["chain"] == 0 and rb["ticks"] == 0, f"level {lev} is not evaluated"
            continue
        for f in ("lc", "sc", "ns", "chain", "score", "meanE", "meanNs"):
            assert ra[f].tobytes() == rb[f].tobytes(), f"level {lev} {f}: {ra[f]} vs {rb[f]}"
        assert rb["ticks"] > 0
    span = slice(lay.ch_off, lay.s_off + lay.W)
    assert ac >= 0 and np.array_equal(arec[span], brec[span]), "best tree"


CASES = [
    # inst, order, mode, chains, draw_waves, slicing, random_slices, select_sc, levels, sweeps/level, eval every
    ("sat100", "preorder", "tc", 256, 1, False, 0, False, 12, 2, 3),   # helper waves, one group
    ("sat100", "preorder", "h100", 300, -1, False, 0, False, 10, 1, 1),  # one wave per chain, two groups
    ("sat100", "par", "tc", 600, 0, False, 0, False, 10, 1, 1),       # three groups, ragged last
    ("lat14", "par", "gpu", 130, 0, False, 0, True, 8, 3, 2),         # sc-first selection, gpu model
    ("sat60", "par", "tc", 200, 0, True, 0, False, 8, 2, 1),          # annealed slice set
    ("sat60", "preorder", "gpu", 64, 1, False, 3, False, 6, 2, 1),    # fixed random slices, helper waves
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(x) for x in c[:8]))
def test_level_loop_matches_level_launches(case):
    inst, order, mode, n, dw, slicing, rs, ssc, nlev, nit, every = case
    s = Setup(inst, order, mode, n, dw, slicing, rs, ssc)
    betas, niters, ev = schedule(nlev, nit, every)
    a = s.per_level(betas, niters, ev)
    b = s.level_loop(betas, niters, ev)
    if dw == 1:
        assert "preorder_draw_waves=3" in b["desc"], b["desc"]
    assert b["desc"].endswith("anneal=level_loop"), b["desc"]
    compare(s, a, b, ev)


@pytest.mark.parametrize("level_loop,want", [(1, "anneal=level_loop"), (0, "anneal=level_launches")])
def test_many_chains(level_loop, want):
    """8192 chains: more than are resident at once, so tsa_anneal runs per-level launches unless the one-launch
    loop is forced, whose later chains then start after earlier ones have run every level."""
    s = Setup("sat100", "par", "tc", 8192, level_loop=level_loop, init="multi")
    betas, niters, ev = schedule(5, 1, 2)
    a = s.per_level(betas, niters, ev)
    b = s.level_loop(betas, niters, ev)
    assert b["desc"].endswith(want), b["desc"]
    compare(s, a, b, ev)


@pytest.mark.parametrize("blocks,want", [(0, "anneal=level_blocks8"), (3, "anneal=level_blocks3"),
                                         (1, "anneal=level_launches")])
def test_level_blocks(blocks, want):
    """8192 chains with the overlapped selection and the fold apart (the benchmark's headline path): tsa_anneal
    sweeps several levels per launch (blocks of 8 by default, here 8 + 3 levels; or of 3: 3 + 3 + 3 + 2), each
    evaluated level leaving a snapshot of its own, whose fold and selection run as one launch each per block
    (the selection keeping the best in level order), beside the next block's sweeps; each block is split over two
    launches on two streams.  Sweeps per level vary and some levels are not evaluated; the records of all chains,
    the statistics, every trace row and the best equal the per-level launches (tsa_sweeps + tsa_track, pinned to
    the oracle's level loop by test_split_sweeps_match_oracle_level_loop)."""
    s = Setup("sat100", "par", "tc", 8192, init="multi")
    s.cfg.fused_energy = 1  # as the binary sets it when every level is evaluated
    s.cfg.level_blocks = blocks
    nlev = 11
    betas = np.linspace(1.0, 4.0, nlev).astype(np.float32)
    niters = [1, 2, 1, 1, 1, 1, 2, 1, 1, 1, 1]
    ev = [1, 0, 1, 1, 1, 0, 1, 1, 1, 0, 1]
    a = s.per_level(betas, niters, ev)
    b = s.level_loop(betas, niters, ev)
    assert b["desc"].endswith(want), b["desc"]
    assert "split_levels=" in b["desc"], b["desc"]
    compare(s, a, b, ev)


def test_level_loop_split_over_two_calls():
    s = Setup("sat100", "preorder", "tc", 256, 1)
    betas, niters, ev = schedule(10, 2, 2)
    a = s.level_loop(betas, niters, ev)
    b = s.level_loop(betas, niters, ev, split=4)
    compare(s, a, b, ev)
    c = s.per_level(betas, niters, ev)
    compare(s, c, b, ev)


def test_level_loop_refusals():
    s = Setup("sat100", "par", "tc", 64)
    betas, niters, ev = schedule(4)
    with s.context() as ctx:
        with pytest.raises(capi.TsaError):
            ctx.anneal(s.ord, betas, niters, ev)  # no tsa_track_begin
        s.begin(ctx, 4)
        with pytest.raises(capi.TsaError):
            ctx.anneal(s.ord, betas, [1, 0, 1, 1], ev)  # a level without a sweep
        with pytest.raises(capi.TsaError):
            ctx.anneal(s.ord, betas, niters, ev, level0=1)  # beyond max_levels
        ctx.anneal(s.ord, betas[:2], niters[:2], ev[:2])
        assert ctx.describe().endswith("anneal=level_loop")
        with pytest.raises(capi.TsaError):
            ctx.track(2)  # this session runs its levels in one launch
        ctx.track_end()
        s.begin(ctx, 4)
        ctx.track(0)
        ctx.anneal(s.ord, betas[1:], niters[1:], ev[1:], level0=1)  # after tsa_track: per-level launches
        assert ctx.describe().endswith("anneal=level_launches")
        ctx.track_end()
        ctx.sweeps_ms()


def test_wide_path_runs_level_launches():
    m, nlab, ixs, iy = common.load_instance("sat100")
    lay = capi.layout(m, nlab, wide=True)
    O = orc.Oracle(m, nlab, ixs, iy)
    pop = common.oracle_population(O, lay, m, 8, 3, orc.read_trees_py(common.tree_file("sat100", "greedy"), m))
    cfg = capi.make_config(mode="tc", sc_target=20.0, seed=3, kernel=capi.KERNEL_WIDE, level_loop=1)
    out = []
    for anneal in (False, True):
        print(f"[gpu] wide path, tsa_anneal={anneal}", flush=True)
        with capi.Context(lay, leaf_sets(m, ixs, lay.W), max(len(x) for x in ixs), cfg, 8) as ctx:
            ctx.upload(pop)
            ctx.track_begin(max_levels=3)
            if anneal:
                ctx.anneal(capi.ORDER_PAR, [1.0, 2.0, 3.0], [2, 1, 2], [1, 0, 1])
                assert ctx.describe().endswith("anneal=level_launches")
            else:
                for lev, (b, k, sw) in enumerate(zip([1.0, 2.0, 3.0], [2, 1, 2], [0, 2, 3])):
                    ctx.sweeps(capi.ORDER_PAR, b, sw, k)
                    if lev != 1:
                        ctx.track(lev)
            bc, bl, bs, rec, rows, _, _ = ctx.track_end()
            ctx.sweeps_ms()
            cols = b"".join(rows[f].tobytes() for f in ("lc", "sc", "ns", "chain", "score", "meanE", "meanNs"))
            out.append((bc, bl, bs, rec, cols, ctx.download()))
    (a, b) = out
    assert a[:3] == b[:3] and np.array_equal(a[3], b[3]) and np.array_equal(a[5], b[5])
    assert a[4] == b[4]


def test_async_download_keeps_the_record_of_its_point_in_the_stream():
    """tsa_download_async copies the record as it is at its place in the stream, into page-locked memory, and
    tsa_wait completes it: the copy enqueued between two sweep launches equals a waiting download made at the
    same point, not the record after the later sweep."""
    import ctypes
    s = Setup("sat100", "par", "tc", 64)
    lib = capi.load()
    words = s.lay.chain_words
    with s.context() as a:
        a.sweeps(s.ord, 2.0, 0, 2)
        ref = a.download(5, 1)[0]
    buf = lib.tsa_host_alloc(words * 8)
    assert buf
    try:
        with s.context() as b:
            b.sweeps(s.ord, 2.0, 0, 2)
            b._check(lib.tsa_download_async(b.h, 5, 1, buf))
            b.sweeps(s.ord, 4.0, 2, 3)
            b._check(lib.tsa_wait(b.h))
            got = np.ctypeslib.as_array((ctypes.c_uint64 * words).from_address(buf)).copy()
            after = b.download(5, 1)[0]
            b.sweeps_ms()
    finally:
        lib.tsa_host_free(buf)
    assert np.array_equal(got, ref)
    assert not np.array_equal(after, ref)  # the later sweeps moved the chain


def test_split_sweeps_match_oracle_level_loop():
    """The headline path as the benchmark runs it: 8192 chains of sat100 from the multi-tree starts with every
    level evaluated, so each level's node costs are folded and the chains selected on a second stream beside the
    next level's sweep, and each level's sweep runs as two launches on two streams (chains [0, h) and
    [h, 8192)).  The records of all 8192 chains (both halves), every trace row and the best chain and tree equal
    the oracle's level loop (the reference's run_anneal with scheme indep, csrc/treesa_gpu.cu:1788-1832)."""
    s = Setup("sat100", "par", "tc", 8192, init="multi")
    s.cfg.fused_energy = 1  # as the binary sets it when every level is evaluated
    nlev = 6
    betas, niters, ev = schedule(nlev, 1, 1, b0=1.0, b1=3.0)
    a = s.per_level(betas, niters, ev)
    assert "fold=apart" in a["desc"] and f"split_levels={nlev}" in a["desc"], a["desc"]
    m, nlab, ixs, iy = common.load_instance("sat100")
    O = orc.Oracle(m, nlab, ixs, iy)
    P = orc.params_from_config(s.cfg, s.leaf_sc, nlab)
    pop = s.pop0.copy()
    print("[oracle] level loop, 8192 chains", flush=True)
    r = O.anneal(P, s.lay, pop, [float(b) for b in betas], [0] * nlev, niters, capi.ORDER_PAR, scheme="indep",
                 eval_every=1, sc_target=common.CHECK_SC_TARGET, seed=3)
    bad = [c for c in range(s.nchains) if not np.array_equal(a["pop"][c], pop[c])]
    assert not bad, f"{len(bad)} chains differ from the oracle (first {bad[:5]}, split at {s.nchains // 2})"
    chain, level, score, rec, rows, _, _ = a["best"]
    for lev in range(nlev):
        o, g = r["levels"][lev], rows[lev]
        assert int(g["chain"]) == int(o["best"]), lev
        assert g["lc"].tobytes() == np.float32(o["lc"]).tobytes(), lev
        assert (int(g["sc"]), int(g["ns"])) == (int(o["sc"]), int(o["ns"])), lev
        assert float(g["score"]) == float(o["score"]), lev
    assert chain == r["best_chain"]
    span = slice(s.lay.ch_off, s.lay.s_off + s.lay.W)
    assert np.array_equal(rec[span], r["best_rec"][span]), "best tree"
