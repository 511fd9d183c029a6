"""Write the golden words of pythia_base2.py's plate and order switches (run here, in the build container).

foundation0/pythia_base2.py:21-27, 40-58: plates=finished|start picks which checkpoint's plates, biases, norms and
word tables the machine runs (the converter keeps both on one grid), plates=built runs their difference (finished
- start, digit for digit), and order=shuffle runs the stream's lanes in the order
default_rng(12345).permutation(768), every plate permuted to match.  This script converts a seeded
finished checkpoint (random_pythia(seed=5, vocab=1000)) with a different start checkpoint (seed 6) by this
repository's converter, executes pythia_base2.py's definitions with each switch, and records the greedy words
and the hashes of the last position's intermediates.  The reference source is read and executed here only;
modes_golden.json holds words and hashes.  Cases already in the file for the same model are kept.
Usage:  python tests/golden/make_golden_modes.py [/root/reference]
"""
from __future__ import annotations

import importlib.util
import json
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
OUT = os.path.join(HERE, "modes_golden.json")


def _module(name):
    spec = importlib.util.spec_from_file_location(name, os.path.join(HERE, name + ".py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main():
    g2 = _module("make_golden")
    gp = _module("make_golden_pythia")
    gf = _module("make_golden_float")
    sm = g2.load_pkg()
    from streaming_machine_amd import pythia
    t0 = time.time()
    fin, cfg = pythia.random_pythia(seed=5, vocab=1000)
    start, _ = pythia.random_pythia(seed=6, vocab=1000)
    npz = pythia.convert_pythia(fin, cfg, start=start)
    del fin, start
    out = {"generator": "tests/golden/make_golden_modes.py",
           "reference": "foundation0/pythia_base2.py (definitions) with plates= and order=",
           "hash": "sha256 of int64 little-endian bytes",
           "model": dict(recipe=dict(finished_seed=5, start_seed=6, vocab=1000), digest=sm.array_digest(npz)),
           "cases": []}
    if os.path.exists(OUT):
        old = json.load(open(OUT))
        if old.get("model") == out["model"]:
            out["cases"] = old["cases"]
    have = {tuple(c["switches"]) for c in out["cases"]}
    work = tempfile.mkdtemp(prefix="sm_golden_modes_")
    np.savez(os.path.join(work, "base2_pythia-modes.npz"), **npz)
    prompt = sm.prompt_ids(50, 8, 1000)
    for switches in (["plates=finished"], ["plates=start"], ["order=shuffle"], ["plates=built"],
                     ["plates=built", "gauge=float"]):
        if tuple(switches) in have:
            continue
        ns = gf.namespace(os.path.join(REF, "foundation0", "pythia_base2.py"), work,
                          ["pythia_base2.py", "size=modes"] + switches, file_as=os.path.join(work, "pythia_base2.py"))
        rc = gp.Recorder(ns)
        words, rec = gp.run_words(ns, rc, prompt, 8)
        out["cases"].append(dict(name="_".join(s.replace("=", "_") for s in switches), switches=switches,
                                 prompt=prompt, words=words, records={"last": rec}))
        print(f"[{time.time() - t0:6.1f}s] {switches}: {words}", flush=True)
        del ns, rc
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote {OUT} in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
