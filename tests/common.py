"""Shared helpers of the parity tests: instances, oracle-built initial populations, record hashes."""
import json
import math
import os

import numpy as np

import oracle as orc

HERE = os.path.dirname(os.path.abspath(__file__))
DATA = os.path.join(HERE, "golden", "data")
GOLDEN = os.path.join(HERE, "golden", "ref_sweeps.json")


def inst_path(name):
    return os.path.join(DATA, name + ".txt")


def load_instance(name):
    return orc.read_instance_py(inst_path(name))


def julia_range(a, step, b):
    """The reference's a:step:b betas (csrc/treesa_gpu.cu:1311-1315): count floor((b-a)/step + 1e-9) + 1,
    values a + i*step in double, stored as float."""
    n = int(math.floor((b - a) / step + 1e-9)) + 1
    return [float(np.float32(a + i * step)) for i in range(n)]


def tree_file(name, init):
    if init == "greedy":
        return os.path.join(DATA, name + ".tree")
    if init == "multi":
        return os.path.join(DATA, name + "_multi.tree")
    return None


def oracle_population(O, lay, m, nchains, seed, trees=None, random_slices=0, first=0):
    """Initial records built by the oracle alone: chain c from trees[c % K] or from the Julia random tree
    seeded splitmix64(seed * 1000003 + c), topology labels, optional fixed random slice sets; row k is chain
    slot first + k."""
    pop = np.zeros((nchains, lay.chain_words), np.uint64)
    cache = {}
    for k_row in range(nchains):
        c = first + k_row
        if trees is not None and len(trees):
            k = c % len(trees)
            ch = trees[k]
        else:
            k = None
            ch = orc.random_tree(m, orc.load().oracle_splitmix64((seed * 1000003 + c) & 0xFFFFFFFFFFFFFFFF))
        if k is None or k not in cache:
            lab = O.labels(ch, lay.W)
            assert lab is not None, "invalid initial tree"
            if k is not None:
                cache[k] = lab
        else:
            lab = cache[k]
        pop[k_row, :lay.nint * lay.W] = lab.reshape(-1)
        pop[k_row, lay.ch_off:].view(np.uint32)[:m - 1] = ch
        if random_slices:
            S = np.zeros(lay.W, np.uint64)
            orc.load().oracle_random_slices(O.nlab, seed, c, random_slices, lay.W, S.ctypes.data)
            pop[k_row, lay.s_off:lay.s_off + lay.W] = S
    return pop


def fnv64(b):
    h = 1469598103934665603
    for x in b:
        h ^= x
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return "%016x" % h


def record_hashes(rec, lay, nlab):
    """(children_fnv, labels_fnv) of one record, as the reference harness hashes them: children words, and the
    internal label sets as ceil(nlab/64) little-endian 64-bit words per node."""
    ch = np.ascontiguousarray(rec[lay.ch_off:]).view(np.uint32)[:lay.nint]
    wn = (nlab + 63) // 64
    lab = np.ascontiguousarray(rec[:lay.nint * lay.W]).reshape(lay.nint, lay.W)[:, :wn]
    return fnv64(ch.astype("<u4").tobytes()), fnv64(np.ascontiguousarray(lab).astype("<u8").tobytes())


def golden_cases():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


def case_id(c):
    return "-".join([c["inst"], c["order"], c["mode"], c["init"]] + [x.lstrip("-") for x in c["extra"]])


def case_options(c):
    """(random_slices, par_follow, par_band) of a golden case."""
    ex = c["extra"]
    rs = int(ex[ex.index("--random-slices") + 1]) if "--random-slices" in ex else 0
    pf = "--par-follow" in ex
    pb = int(ex[ex.index("--par-band") + 1]) if "--par-band" in ex else 0
    return rs, pf, pb


# the validation-matrix parameters of the reference (tests/run_checks.sh:13)
CHECK_BETAS = julia_range(0.2, 0.7, 7.0)
CHECK_NITERS = 4
CHECK_SC_TARGET = 24.0
CHECK_SEED = 7
