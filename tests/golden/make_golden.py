"""Write tests/golden/ref_sweeps.json from the reference's own CPU port.

Runs oracle/_ref/ref_harness (csrc/cpu_ref.h + csrc/common.h compiled where they lie by `make -C oracle`)
on the reference's test instances with the parameters of its kernel validation matrix
(tests/run_checks.sh:13: 4 reference chains, --niters 4, --betas 0.2:0.7:7, --sc-target 24, --seed 7) over
both sweep orders, the three energy modes, greedy / random / multi-tree starts, fixed random slice sets
and the par-order options.  For every chain it stores the proposal and accept counts and FNV-1a hashes of
the final children words and label sets, which is what tests/test_oracle_golden.py checks the oracle
against.  Usage: python tests/golden/make_golden.py
"""
import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(HERE))
DATA = os.path.join(HERE, "data")
REF = os.path.join(ROOT, "oracle", "_ref", "ref_harness")

BASE = ["--chains", "4", "--niters", "4", "--betas", "0.2:0.7:7", "--sc-target", "24", "--seed", "7"]


def cases():
    out = []
    for inst in ("sat40", "sat100", "reg3_250", "lat14", "grid24"):
        for order in ("par", "preorder"):
            for mode in ("tc", "h100"):
                out.append(dict(inst=inst, order=order, mode=mode, init="greedy", extra=[]))
    for order in ("par", "preorder"):
        out.append(dict(inst="sat100", order=order, mode="gpu", init="greedy", extra=[]))
        out.append(dict(inst="sat100", order=order, mode="tc", init="random", extra=[]))
        out.append(dict(inst="sat100", order=order, mode="tc", init="multi", extra=[]))
        out.append(dict(inst="sat100", order=order, mode="tc", init="greedy", extra=["--random-slices", "8"]))
        out.append(dict(inst="grid24", order=order, mode="h100", init="greedy", extra=["--random-slices", "8"]))
        out.append(dict(inst="sq46", order=order, mode="tc", init="greedy", extra=[]))
    out.append(dict(inst="sat100", order="par", mode="tc", init="greedy", extra=["--par-band", "4"]))
    out.append(dict(inst="reg3_250", order="par", mode="tc", init="greedy", extra=["--par-follow"]))
    out.append(dict(inst="lat14", order="par", mode="h100", init="greedy", extra=["--par-band", "8", "--par-follow"]))
    return out


def fnv64(data):
    h = 1469598103934665603
    for b in data:
        h ^= b
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return "%016x" % h


def run(case):
    inst = os.path.join(DATA, case["inst"] + ".txt")
    args = [REF, "-i", inst] + BASE + ["--order", case["order"], "--mode", case["mode"]] + case["extra"]
    if case["init"] == "greedy":
        args += ["--tree", os.path.join(DATA, case["inst"] + ".tree")]
    elif case["init"] == "multi":
        args += ["--tree", os.path.join(DATA, case["inst"] + "_multi.tree")]
    else:
        args += ["--random-trees"]
    res = json.loads(subprocess.run(args, check=True, capture_output=True, text=True).stdout)
    chains = []
    for ch in res["chains"]:
        words = ch["children"]
        b = bytearray()
        for i in range(0, len(words), 2):
            b += ((words[i] | (words[i + 1] << 16)) & 0xFFFFFFFF).to_bytes(4, "little")
        chains.append(dict(nprop=ch["nprop"], nacc=ch["nacc"], labels_fnv=ch["labels_fnv"], children_fnv=fnv64(b)))
    return chains


def main():
    if not os.path.exists(REF):
        sys.exit(f"{REF} missing: run `make -C oracle` where /root/reference exists")
    out = {"params": BASE, "cases": []}
    for c in cases():
        c2 = dict(c)
        c2["chains"] = run(c)
        out["cases"].append(c2)
        print(c["inst"], c["order"], c["mode"], c["init"], " ".join(c["extra"]), [x["nacc"] for x in c2["chains"]])
    with open(os.path.join(HERE, "ref_sweeps.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
