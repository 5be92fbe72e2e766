"""Small synthetic instances at the edges of the input space (shared by the CPU and GPU edge-case tests).

* pair: m = 2, which the binary and the library reject as the reference does (csrc/treesa_gpu.cu:2073);
* triple: m = 3, the smallest instance (two internal nodes);
* mixed40: an empty tensor, a label held by one tensor only, open labels (one of them the dangling label),
  labels held by two and by three tensors;
* deg3_<L>: L labels each held by two tensors, three labels per tensor, at the label-count boundaries of the
  register widths (64 | 65, 128 | 129, 256 | 257 labels -> 1, 2, 4, 8 words) and of the runtime width
  (513 labels);
* wide_<L>: 300 tensors and L labels each held by two tensors: 16384 labels is the widest chain the wide
  kernel takes (256 words), 16385 falls back to the one-wave kernel with runtime width;
* sparse_<m>: m tensors over 256 labels (register width 4: the chain stays in LDS), each label on two random
  tensors and every tensor without one given one more: 513 tensors are 512 internal nodes, the most whose
  par scan keeps the list of unvisited nodes; 514 tensors scan every node in two batches of 512.
"""
import numpy as np


def _deg3(nlab, seed):
    # 2 * nlab label slots dealt to m = 2 nlab / 3 tensors, three per tensor, no label twice on one tensor
    m = (2 * nlab + 2) // 3
    rng = np.random.default_rng(seed)
    for _ in range(1000):
        slots = np.repeat(np.arange(nlab), 2)
        rng.shuffle(slots)
        ixs = [[] for _ in range(m)]
        ok = True
        for k, l in enumerate(slots):
            t = k % m
            if l in ixs[t]:
                ok = False
                break
            ixs[t].append(int(l))
        if ok:
            return m, nlab, ixs, []
    raise RuntimeError("no simple assignment found")


def _mixed40():
    rng = np.random.default_rng(11)
    m, nlab = 40, 70
    ixs = [[] for _ in range(m)]
    for l in range(68):
        k = 2 if l % 4 else 3
        for t in rng.choice([t for t in range(m) if t != 5], k, replace=False):
            ixs[int(t)].append(l)
    ixs[7].append(69)  # label 69: one holder; label 68: none (an unused id)
    return m, nlab, [sorted(ix) for ix in ixs], [0, 13, 69]


def _wide(nlab, seed):
    m = 300
    rng = np.random.default_rng(seed)
    ixs = [[] for _ in range(m)]
    for l in range(nlab):
        a, b = rng.choice(m, 2, replace=False)
        ixs[int(a)].append(l)
        ixs[int(b)].append(l)
    return m, nlab, ixs, []


def _sparse(m, seed, nlab=256):
    rng = np.random.default_rng(seed)
    ixs = [set() for _ in range(m)]
    for l in range(nlab):
        a, b = rng.choice(m, 2, replace=False)
        ixs[int(a)].add(l)
        ixs[int(b)].add(l)
    for t in range(m):
        if not ixs[t]:
            ixs[t].add(int(rng.integers(nlab)))
    return m, nlab, [sorted(ix) for ix in ixs], []


def instance(name):
    if name == "pair":
        return 2, 3, [[0, 1], [1, 2]], [0]
    if name == "triple":
        return 3, 2, [[0], [0, 1], [1]], []
    if name == "mixed40":
        return _mixed40()
    if name.startswith("deg3_"):
        return _deg3(int(name[5:]), 3)
    if name.startswith("wide_"):
        return _wide(int(name[5:]), 5)
    if name.startswith("sparse_"):
        return _sparse(int(name[7:]), 9)
    raise KeyError(name)


NAMES = ["triple", "mixed40", "deg3_64", "deg3_65", "deg3_129", "deg3_257", "deg3_513", "sparse_513", "sparse_514"]
WIDE = ["wide_16384", "wide_16385"]
