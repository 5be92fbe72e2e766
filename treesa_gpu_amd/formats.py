"""Tree and result formats of the reference's Python layer, in this package's own code.

* Tree dicts (omeco's NestedEinsum.to_dict(), the format the reference's driver returns): a leaf is
  {"tensor_index": i}, an internal node {"args": [left, right], "eins": {"ixs": [labels_left,
  labels_right], "iy": labels_out}} (treesa_gpu/trees.py:8-11).
* Children lists: (left, right) of internal nodes m..2m-2 in post-order, root last -- the binary's tree file
  and its JSON "tree" (treesa_gpu/driver.py:80-108).
* leaf_ids, recompute_outputs, contractions, complexity (treesa_gpu/trees.py:17-80); the two time models
  gpu_time / h100_time and their tree sums (treesa_gpu/trees.py:87-149); label_map / write_instance
  (treesa_gpu/driver.py:60-77); runner_json (treesa_gpu/driver.py:351-353); result_tree, the driver's
  reading of the binary's JSON (treesa_gpu/driver.py:313-328).

Every traversal is iterative, so path trees over thousands of tensors need no recursion limit.  All indices
have dimension 2: log2 sizes are label counts.
"""
import json
import math

from . import capi
from .instances import label_map  # noqa: F401  (re-exported: the driver's label numbering)

GPU_KEYS = ("peak_ops", "bw_bits", "m0", "n0", "k0", "launch")
H100_KEYS = ("launch", "perm_bw_bits", "cc_bit", "cc_cell", "tc_bit", "tc_pad_cell", "tc_out_bit", "small_rank",
             "small_cell")
GPU_MODEL = dict(zip(GPU_KEYS, capi.DEFAULT_GM))
H100_MODEL = dict(zip(H100_KEYS, capi.DEFAULT_H100))


def _postorder(d):
    """Nodes of a tree dict with their children's positions: list of (node, left_pos, right_pos), leaves
    with (node, -1, -1), children before parents, left subtree first."""
    out = []
    stack = [(d, False)]
    pos = []  # positions of finished subtrees, in completion order
    while stack:
        t, done = stack.pop()
        if "tensor_index" in t:
            out.append((t, -1, -1))
            pos.append(len(out) - 1)
        elif done:
            r = pos.pop()
            l = pos.pop()
            out.append((t, l, r))
            pos.append(len(out) - 1)
        else:
            stack.append((t, True))
            stack.append((t["args"][1], False))
            stack.append((t["args"][0], False))
    return out


def leaf_ids(d):
    """Tensor indices of the leaves, left to right."""
    return [t["tensor_index"] for t, l, _ in _postorder(d) if l < 0]


def dict_to_children(d, m):
    """Tree dict -> [(left, right)] of internal nodes m..2m-2 (post-order ids, root last)."""
    ids = []
    ch = []
    for t, l, r in _postorder(d):
        if l < 0:
            ids.append(int(t["tensor_index"]))
        else:
            ch.append((ids[l], ids[r]))
            ids.append(m + len(ch) - 1)
    if len(ch) != m - 1 or ids[-1] != 2 * m - 2 or sorted(i for i in ids if i < m) != list(range(m)):
        raise ValueError("tree must be binary over all m tensors")
    return ch


def children_to_dict(ch, m, ixs, iy):
    """Children list (node ids, root 2m-2; pairs or the binary's [l, r] lists) -> tree dict with
    topology-derived internal labels."""
    if m == 1:
        return recompute_outputs({"tensor_index": 0}, ixs, iy)
    ch = [(int(l), int(r)) for l, r in ch]
    if len(ch) != m - 1:
        raise ValueError("a tree over m tensors has m - 1 internal nodes")
    node = {}
    seen = set()
    stack = [2 * m - 2]  # internal nodes may be numbered in any order: build from the root down
    while stack:
        v = stack[-1]
        if v < m:
            node[v] = {"tensor_index": v}
            stack.pop()
            continue
        l, r = ch[v - m]
        if l in node and r in node:
            node[v] = {"args": [node[l], node[r]], "eins": {"ixs": [[], []], "iy": []}}
            stack.pop()
            continue
        if v in seen:
            raise ValueError("children list is not a binary tree over all m tensors")
        seen.add(v)
        for u in (r, l):
            if not 0 <= u < 2 * m - 1 or u in seen or u in node:
                raise ValueError("children list is not a binary tree over all m tensors")
            stack.append(u)
    if len(node) != 2 * m - 1:
        raise ValueError("children list is not a binary tree over all m tensors")
    return recompute_outputs(node[2 * m - 2], ixs, iy)


def recompute_outputs(d, ixs, iy):
    """A new tree whose internal output labels follow from the topology: a label is kept iff a tensor outside
    the node's subtree holds it or it is open.  A node's iy lists the kept labels in the order of their first
    appearance in its left input's labels followed by its right input's."""
    total = {}
    for ix in ixs:
        for l in ix:
            total[l] = total.get(l, 0) + 1
    final = set(iy)
    built = []  # per post-order position: (new node, label counts in the subtree, output labels)
    for t, li, ri in _postorder(d):
        if li < 0:
            labs = list(ixs[t["tensor_index"]])
            cnt = {}
            for l in labs:
                cnt[l] = cnt.get(l, 0) + 1
            built.append(({"tensor_index": t["tensor_index"]}, cnt, labs))
            continue
        (ln, lc, la), (rn, rc, lb) = built[li], built[ri]
        cnt = dict(lc)
        for k, v in rc.items():
            cnt[k] = cnt.get(k, 0) + v
        out, seen = [], set()
        for x in la + lb:
            if x not in seen:
                seen.add(x)
                if x in final or cnt[x] < total[x]:
                    out.append(x)
        built.append(({"args": [ln, rn], "eins": {"ixs": [la, lb], "iy": out}}, cnt, out))
    return built[-1][0]


def contractions(d, ixs):
    """(B, M, N, K) label counts of every pairwise contraction, post-order: B batch (both inputs and the
    output), M / N only in the left / right input and the output, K summed (both inputs, not the output)."""
    sets = []
    acc = []
    for t, li, ri in _postorder(d):
        if li < 0:
            sets.append(frozenset(ixs[t["tensor_index"]]))
            continue
        a, b, y = sets[li], sets[ri], frozenset(t["eins"]["iy"])
        acc.append((len(a & b & y), len((a - b) & y), len((b - a) & y), len((a & b) - y)))
        sets.append(y)
    return acc


def _log2_sum_pow2(xs):
    if not xs:
        return 0.0
    mx = max(xs)
    return mx + math.log2(sum(2.0 ** (x - mx) for x in xs))


def complexity(d, ixs):
    """(tc, sc) in log2: tc = log2 of the sum over contractions of 2^(B+M+N+K), sc = the largest tensor (inputs
    and intermediates)."""
    cs = contractions(d, ixs)
    tc = _log2_sum_pow2([b + m + n + k for b, m, n, k in cs])
    sc = max([b + m + n for b, m, n, _ in cs] + [len(set(ix)) for ix in ixs])
    return tc, sc


def gpu_time(B, M, N, K, model=None):
    """Modeled seconds of one contraction on bit-packed tensor cores: the larger of the padded AND-popcount
    work at peak_ops and the bits of both inputs and the output at bw_bits, plus a launch."""
    g = GPU_MODEL if model is None else model
    ops = 2.0 ** (1 + B + max(M, g["m0"]) + max(N, g["n0"]) + max(K, g["k0"]))
    bits = 2.0 ** (B + M + K) + 2.0 ** (B + N + K) + 2.0 ** (B + M + N)
    return max(ops / g["peak_ops"], bits / g["bw_bits"]) + g["launch"]


def h100_time(B, M, N, K, model=None, small=False):
    """Modeled seconds of one contraction with the fitted H100 model: batched small contractions cost
    small_cell per output-bit x summed combination; others three launches, the permutes of both inputs and the
    cheaper of the CUDA-core and the tensor-core (K >= 7 and max(M, N) >= 5) GEMM."""
    h = H100_MODEL if model is None else model
    if small:
        return h["small_cell"] * 2.0 ** (B + M + N + K)
    a, b, c = 2.0 ** (B + M + K), 2.0 ** (B + N + K), 2.0 ** (B + M + N)
    moved = a + b + c
    cc = h["cc_bit"] * moved + h["cc_cell"] * 2.0 ** (B + M + N + K)
    best = cc
    if K >= 7 and max(M, N) >= 5:
        tcore = (h["tc_bit"] * moved + h["tc_pad_cell"] * 2.0 ** (B + max(M, 6) + max(N, 6) + max(K, 8))
                 + h["tc_out_bit"] * c)
        best = min(cc, tcore)
    return 3 * h["launch"] + 2 * (a + b) / h["perm_bw_bits"] + best


def tree_gpu_time(d, ixs, model=None):
    return sum(gpu_time(*c, model=model) for c in contractions(d, ixs))


def tree_h100_time(d, ixs, model=None):
    """Modeled seconds of one slice: contractions whose output rank is at most small_rank are batched."""
    h = H100_MODEL if model is None else model
    return sum(h100_time(B, M, N, K, h, small=(B + M + N) <= h["small_rank"]) for B, M, N, K in contractions(d, ixs))


def write_instance(path, ixs, iy):
    """The instance file (m nlab / per tensor: k l1..lk / ny y1..) with labels numbered by label_map; returns
    the map."""
    from .instances import instance_text
    mp = label_map(ixs, iy)
    with open(path, "w") as f:
        f.write(instance_text(ixs, iy))
    return mp


def write_tree_file(path, trees, m):
    """Tree file of one or more start trees (tree dicts or children lists): m-1 lines "left right" each."""
    with open(path, "w") as f:
        for t in trees:
            if isinstance(t, dict):
                ch = dict_to_children(t, m)
            else:  # (left, right) pairs, or children words left | right << 16
                ch = [tuple(w) if isinstance(w, (tuple, list)) else (int(w) & 0xFFFF, int(w) >> 16) for w in t]
            for a, b in ch:
                f.write(f"{int(a)} {int(b)}\n")


def result_tree(res, ixs, iy, lmap=None, gpu_model=None, h100_model=None):
    """The binary's JSON result (a dict or a path) -> (tree dict, info), as the driver reads it: sliced label
    ids mapped back to the caller's labels, the tree over the sliced network, and tc / sc / model times of
    that tree recomputed in Python (keys *_py)."""
    if isinstance(res, str):
        with open(res) as f:
            res = json.load(f)
    lmap = label_map(ixs, iy) if lmap is None else lmap
    inv = {v: k for k, v in lmap.items()}
    sliced = [inv[i] for i in res["sliced"]]
    sl = set(sliced)
    ixs_s = [[l for l in ix if l not in sl] for ix in ixs] if sl else ixs
    iy_s = [l for l in iy if l not in sl]
    m = len(ixs)
    tree = children_to_dict(res["tree"], m, ixs_s, iy_s)
    if sorted(leaf_ids(tree)) != list(range(m)):
        raise ValueError("result tree does not contain every leaf exactly once")
    tc, sc = complexity(tree, ixs_s)
    info = {k: v for k, v in res.items() if k != "tree"}
    t1 = tree_gpu_time(tree, ixs_s, gpu_model)
    t2 = tree_h100_time(tree, ixs_s, h100_model)
    info.update(sliced=sliced, tc_py=tc, sc_py=sc, gpu_time_py=t1, h100_time_py=t2, tc_total_py=tc + len(sliced),
                h100_time_total_py=t2 * 2.0 ** len(sliced))
    return tree, info


def runner_json(tree, info):
    """{"tree": tree dict on the sliced network, "sliced": [the caller's labels]}."""
    return {"tree": tree, "sliced": list(info.get("sliced", []))}
