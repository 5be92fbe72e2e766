"""Write the inputs of the larger benchmark workloads as fixtures under tests/golden/data/.

* sat70.txt + sat70_greedy.tree: random 3-SAT n=70, m=round(4.26*70)=298, seed 1 (the reference's generator,
  treesa_gpu_amd/instances.py) and the native greedy start tree, best of 10 runs, seed 1
  (treesa_gpu_amd/host.py; the reference commits no greedy tree for this instance).
* reg3_2000.txt + reg3_2000_spectral.tree: a 3-regular graph with 2000 vertices from the seeded configuration
  model (seed 1) and its 4 best native spectral path trees (seed 1).
* sq64.txt + sq64_row.tree: the 64 x 64 lattice and its row-major path tree.
Committed so that every run of the benchmarks starts from the same trees.  Usage:
python tests/golden/make_inputs.py
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from treesa_gpu_amd import instances as I  # noqa: E402
from treesa_gpu_amd import host as S  # noqa: E402

DATA = os.path.join(HERE, "data")


def mapped(ixs, iy):
    mp = I.label_map(ixs, iy)
    return [[mp[l] for l in ix] for ix in ixs], [mp[l] for l in iy]


def write(name, ixs, iy, trees, suffix):
    with open(os.path.join(DATA, name + ".txt"), "w") as f:
        f.write(I.instance_text(ixs, iy))
    S.write_trees(os.path.join(DATA, f"{name}_{suffix}.tree"), trees)


def main():
    ixs, iy = I.sat(70)
    mx, my = mapped(ixs, iy)
    write("sat70", ixs, iy, [S.greedy_tree(mx, my, nrepeat=10, seed=1)], "greedy")
    ixs, iy = I.reg3(2000, seed=1)
    mx, my = mapped(ixs, iy)
    so = S.spectral_orders(mx, my, k=4, seed=1)
    print("reg3_2000 spectral path tc:", [round(t, 3) for t, _, _ in so])
    write("reg3_2000", ixs, iy, [S.path_tree(o) for _, _, o in so], "spectral")
    ixs, iy = I.sq(64)
    write("sq64", ixs, iy, [S.path_tree(range(len(ixs)))], "row")


if __name__ == "__main__":
    main()
