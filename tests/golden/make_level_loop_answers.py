"""Writes tests/golden/level_loop_answers.json: the oracle's level loop on every run of the reference's logged
Python test (tests/level_loop_cases.py), for both sweep orders.

Per case: the oracle's final tc / sc / |S| / repair / tree hash / best chain, and whether the reference's printed
values reproduce.  For every case that does not reproduce: the levels whose sweeps made a Metropolis decision within two ulp of
expf (u lies between expf's neighbours two ulp down and up: an expf within two ulp of this host's could decide
otherwise), and the same run again under seven perturbations of the float arithmetic (oracle.set_variant): the
lse of the energy fold (and in the float energy modes the sweeps' models) evaluated in double and rounded once,
then six runs (seeds 1..6) in which exp2f / log2f results move by one ulp and Metropolis's expf by up to two ulp
at hash-chosen operands -- devices whose functions stay within those bounds (the reference's GPU documents expf
within two ulp) but round differently from this host's libm.  Per perturbation it records the first level whose
decision (best chain or ancestors) changes, the decision margins the unperturbed oracle measured there, the final
answer and whether it reproduces the reference: a run whose answer moves under such a perturbation cannot be
expected to reproduce a device whose functions round differently, and one that then lands on the reference's
printed answer shows that the difference is that rounding.

Usage: python tests/golden/make_level_loop_answers.py [case-id-prefix ...]   (several minutes per order)
"""
import json
import os
import sys
import tempfile
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import level_loop_cases as K  # noqa: E402
import oracle as orc  # noqa: E402


def summary(got):
    return dict(tc=round(got["tc"], 9), sc=got["sc"], ns=got["ns"], n_repair=got["n_repair"],
                tree_fnv=K.tree_hash(got["tree"]), sliced=got["sliced"], best_chain=got["best_chain"],
                nresample=got["nresample"], gpu_time=got["gpu_time"], h100_time=got["h100_time"],
                h100_time_total=got["h100_time_total"])


def first_divergence(a, b):
    la, lb = a["levels"], b["levels"]
    for L in range(len(la)):
        if la[L]["best"] != lb[L]["best"] or (la[L]["resampled"] and list(a["anc"][L]) != list(b["anc"][L])):
            return L
    return None


def main():
    only = sys.argv[1:]
    out = {"cases": []}
    if os.path.exists(K.FIXTURE) and only:
        out = K.load_fixture()
    done = {c["id"]: i for i, c in enumerate(out["cases"])}
    K.write_spectral_starts([c for order in ("par", "preorder") for c in K.known_answer_cases(order)])
    for order in ("par", "preorder"):
        for c in K.known_answer_cases(order):
            if only and not any(c["id"].startswith(p) for p in only):
                continue
            t0 = time.time()
            with tempfile.TemporaryDirectory() as tmp:
                orc.set_variant(0)
                got = K.oracle_run(c, tmp)
                rec = dict(id=c["id"], kind=c["kind"], ref=c["ref"], oracle=summary(got),
                           reproduces=K.agrees_with_reference(c, got))
                if not rec["reproduces"]:
                    tc_only = c["mode"] == "tc" and not c["stage2"]
                    lv = got["levels"]
                    rec["metropolis_near_levels"] = [L for L in range(len(lv)) if lv[L]["metropolis_near"] > 0][:20]
                    rec["perturbed"] = []
                    runs = [(1 if tc_only else 3, 0)] + [((4 if tc_only else 12) | 16, s) for s in range(1, 7)]
                    for variant, seed in runs:
                        orc.set_variant(variant, seed)
                        alt = K.oracle_run(c, tmp)
                        orc.set_variant(0)
                        L = first_divergence(got, alt)
                        lev = got["levels"][L] if L is not None else None
                        rec["perturbed"].append(dict(
                            variant=variant, noise_seed=seed, first_level=L, answer=summary(alt),
                            answer_changes=K.tree_hash(alt["tree"]) != K.tree_hash(got["tree"]) or
                            alt["sliced"] != got["sliced"],
                            sel_margin=float(lev["sel_margin"]) if lev is not None else None,
                            pop_margin=float(lev["pop_margin"]) if lev is not None else None,
                            reproduces=K.agrees_with_reference(c, alt)))
            if c["id"] in done:
                out["cases"][done[c["id"]]] = rec
            else:
                out["cases"].append(rec)
            ps = rec.get("perturbed") or []
            note = ""
            if ps:
                moved = sum(p["answer_changes"] for p in ps)
                hit = sum(p["reproduces"] for p in ps)
                firsts = [p["first_level"] for p in ps if p["first_level"] is not None]
                note = (f"; perturbed x{len(ps)}: answer moves in {moved}, reproduces the reference in {hit}, "
                        f"first diverging level {min(firsts) if firsts else None}")
            print(f"{c['id']:22s} {c['kind']:8s} ref {c['ref'].get('tc')} oracle {got['tc']:.4f}/{got['sc']}/{got['ns']} "
                  f"{'reproduces' if rec['reproduces'] else 'differs'}{note} [{time.time() - t0:.0f} s]", flush=True)
            with open(K.FIXTURE, "w") as f:
                json.dump(out, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
