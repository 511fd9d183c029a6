"""Write the float-stage golden words from the reference itself (run here, in the build container).

base2.py's switches gauge= / edge= / arrival= (base2.py:10-11) and pythia_base2.py's gauge= / turn= / edge= /
arrival= (foundation0/pythia_base2.py:21-27) put one stage back to float64.  This script executes both scripts'
definitions with those switches on the seeded models converted by this repository's converters (the recipes of
make_golden.py and make_golden_pythia.py) and records, per case, the greedy words (full recompute per word, as
the scripts run) and the hashes of the last position's intermediates (the same recorders as the integer goldens).
The reference source is read and executed here only; float_golden.json holds words and hashes.
Usage:  python tests/golden/make_golden_float.py [/root/reference]
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
OUT = os.path.join(HERE, "float_golden.json")


def _module(name):
    spec = importlib.util.spec_from_file_location(name, os.path.join(HERE, name + ".py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def namespace(path: str, cwd: str, argv: list, file_as: str | None = None, cut: str | None = None) -> dict:
    """Execute a reference script's definitions (up to `cut` when given) with argv and cwd as its command line."""
    src = open(path).read()
    if cut:
        src = src[:src.index(cut)]
    ns: dict = {"__name__": "float_golden", "__file__": file_as or path}
    old_cwd, old_argv = os.getcwd(), sys.argv
    os.chdir(cwd)
    sys.argv = argv
    try:
        exec(compile(src, path, "exec"), ns)
    finally:
        os.chdir(old_cwd)
        sys.argv = old_argv
    return ns


def save(out):
    with open(OUT + ".tmp", "w") as f:
        json.dump(out, f, indent=1)
    os.replace(OUT + ".tmp", OUT)


GPT2_MODES = [("gauge",), ("edge",), ("arrival",), ("gauge", "edge", "arrival")]
PYTHIA_MODES = [("gauge",), ("turn",), ("edge",), ("arrival",), ("gauge", "turn", "edge", "arrival")]


def main():
    g2 = _module("make_golden")
    gp = _module("make_golden_pythia")
    sm = g2.load_pkg()
    from streaming_machine_amd import pythia
    t0 = time.time()
    out = {"generator": "tests/golden/make_golden_float.py",
           "reference": {"gpt2": "base2.py (definitions up to its tokenizer line) with gauge=/edge=/arrival=float",
                         "pythia": "foundation0/pythia_base2.py (definitions) with gauge=/turn=/edge=/arrival=float"},
           "hash": "sha256 of int64 little-endian bytes", "models": {}, "cases": []}
    work = tempfile.mkdtemp(prefix="sm_golden_float_")

    for mname, kw, cases in (("gpt2_small", dict(seed=0, vocab=1000, n_ctx=64), [("p8_w8", sm.prompt_ids(1, 8, 1000), 8)]),
                             ("gpt2_124m", dict(seed=0, vocab=50257, n_ctx=1024), [("p8_w16", sm.prompt_ids(1, 8), 16)])):
        npz = sm.convert(sm.random_gpt2(**kw))
        out["models"][mname] = dict(recipe=kw, digest=sm.array_digest(npz))
        d = os.path.join(work, mname)
        os.makedirs(d, exist_ok=True)
        np.savez(os.path.join(d, "base2_gpt2.npz"), **npz)
        del npz
        for modes in GPT2_MODES:
            ns = namespace(os.path.join(REF, "base2.py"), d, ["base2.py"] + [f"{k}=float" for k in modes],
                           cut="tok = GPT2Tokenizer")
            rc = g2.Recorder(ns, kw["vocab"])
            for cname, prompt, nw in cases:
                words, recs = g2.run_words(ns, rc, prompt, nw, False)
                out["cases"].append(dict(name=f"{mname}_{cname}_{'_'.join(modes)}", model=mname, float=list(modes),
                                         prompt=prompt, words=words, records=recs))
                print(f"[{time.time() - t0:7.1f}s] {mname} {cname} {modes}: {words}", flush=True)
                save(out)
            del ns, rc
        os.remove(os.path.join(d, "base2_gpt2.npz"))

    for mname, kw, cases in (("pythia_small", dict(seed=5, vocab=1000), [("p8_w8", sm.prompt_ids(50, 8, 1000), 8)]),
                             ("pythia_160m", dict(seed=5, vocab=50304), [("p64_w4", sm.prompt_ids(5, 64, 50304), 4)])):
        sd, cfg = pythia.random_pythia(**kw)
        npz = pythia.convert_pythia(sd, cfg)
        del sd
        out["models"][mname] = dict(recipe=kw, digest=sm.array_digest(npz))
        d = os.path.join(work, mname)
        os.makedirs(d, exist_ok=True)
        np.savez(os.path.join(d, f"base2_pythia-{mname}.npz"), **npz)
        del npz
        for modes in PYTHIA_MODES:
            path = os.path.join(REF, "foundation0", "pythia_base2.py")
            ns = namespace(path, d, ["pythia_base2.py", f"size={mname}"] + [f"{k}=float" for k in modes],
                           file_as=os.path.join(d, "pythia_base2.py"))
            rc = gp.Recorder(ns)
            for cname, prompt, nw in cases:
                words, rec = gp.run_words(ns, rc, prompt, nw)
                out["cases"].append(dict(name=f"{mname}_{cname}_{'_'.join(modes)}", model=mname, float=list(modes),
                                         prompt=prompt, words=words, records={"last": rec}))
                print(f"[{time.time() - t0:7.1f}s] {mname} {cname} {modes}: {words}", flush=True)
                save(out)
            del ns, rc
        os.remove(os.path.join(d, f"base2_pythia-{mname}.npz"))
    print(f"wrote {OUT} in {time.time() - t0:.0f}s", flush=True)


if __name__ == "__main__":
    main()
