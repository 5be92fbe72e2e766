"""bench.py's byte accounting, on the CPU: the per-unit figures the roofline divides by the launch time.

* algorithmic_bytes: per proposal five label sets of W words and 8 B of children, per accept one set and 8 B,
  per visit without a rule 4 B (plus the slice step's passes with slicing);
* cached_loaded_bytes (the dense wide kernel in tc mode): four sets per proposal, P's cost and size from the
  node-cost cache (10 B read per proposal, 10 B written per accept);
* loaded_bytes (the chunk-summary kernel in tc mode): 64 B per union chunk (four sets), P's nonzero chunks
  written per accept.
Each is checked against a count written out by hand and against the others' differences, so that a dropped term
or a wrong set count fails.
"""
import pytest

import bench


@pytest.mark.parametrize("W", [1, 2, 48, 126])
def test_algorithmic_and_cached_bytes(W):
    prop, acc, visits = 1000, 370, 1300
    st = [prop, acc, 11, visits, 0]
    alg = bench.algorithmic_bytes(st, W, nint=425)
    assert alg == prop * (5 * 8 * W + 8) + acc * (8 * W + 8) + (visits - prop) * 4
    cached = bench.cached_loaded_bytes(st, W)
    assert cached == prop * (4 * 8 * W + 8 + 10) + acc * (8 * W + 8 + 10) + (visits - prop) * 4
    # the cache replaces one set read per proposal by 10 B, and adds 10 B of writes per accept
    assert alg - cached == prop * (8 * W - 10) - acc * 10


def test_slicing_adds_the_slice_passes():
    W, nint = 2, 297
    st = [500, 200, 9, 600, 40]
    # 40 slice proposals: each evaluates the chain (3 sets + 4 B per node, + S) and scans the internal sets
    none = bench.algorithmic_bytes(st[:4] + [0], W, nint)
    base = bench.algorithmic_bytes(st, W, nint)
    assert base - none == 40 * (24 * W * nint + 4 * nint + 8 * W) + 40 * 8 * W * nint
    # slicing on, 100 slice steps: S read by every proposal, and each step evaluates the chain once more
    sl = bench.algorithmic_bytes(st, W, nint, slicing=True, slice_steps=100)
    assert sl - base == 500 * 8 * W + 100 * (24 * W * nint + 4 * nint + 8 * W)


def test_summary_path_bytes():
    prop, acc, visits = 800, 300, 900
    chunks, xchunks = 2400, 500
    got = bench.loaded_bytes([prop, acc, 0, visits, 0], (chunks, xchunks))
    assert got == chunks * 4 * 16 + prop * (8 + 10) + xchunks * 16 + acc * (8 + 10) + (visits - prop) * 4
    # a union of every chunk of the five-set figure's W words reads four fifths of it, plus the cache
    W = 126
    full = bench.loaded_bytes([prop, 0, 0, prop, 0], (prop * W // 2, 0))
    alg = bench.algorithmic_bytes([prop, 0, 0, prop, 0], W, nint=4095)
    assert full == alg * 4 // 5 - prop * 8 * 4 // 5 + prop * (8 + 10)


def test_launch_count_follows_the_kernel_description():
    """Levels per sweep launch, from the binary's kernel description: the level loop in one launch, blocks of K
    levels (the schedule's last block shorter), or one launch per level."""
    d = "lds W=2 waves/block=4 lds_bytes/wave=11104 fold=apart split_levels=6"
    assert bench.launch_count(d + " anneal=level_blocks8", 20) == 3  # 8 + 8 + 4
    assert bench.launch_count(d + " anneal=level_blocks8", 16) == 2
    assert bench.launch_count(d + " anneal=level_blocks3", 200) == 67
    assert bench.launch_count("lds W=2 waves/block=1 anneal=level_loop", 100) == 1
    assert bench.launch_count(d + " anneal=level_launches", 20) == 20
    assert bench.launch_count("wide W=48 G=8 anneal=level_launches", 100) == 100
    assert "blocks of 8 levels" in bench.kernel_label(d + " anneal=level_blocks8", 0)
