"""Write the full-length golden words of the batched workloads from the reference itself (run here, in the build
container, once; about an hour of CPU).

The batched workloads decode far past the contexts the short golden cases reach: 64 streams of 32-token prompts
and 128 words (context to 160) for GPT-2 124M, and 32 streams of 64-token prompts and 256 words (context to 320)
for the Pythia-160m-shaped machine.  This script runs base2.py's forward (full recompute per word, base2.py:123)
and pythia_base2.py's forward (foundation0/pythia_base2.py:151-160) for streams 0 and 1 of each, over the whole
length, on the seeded models converted by this repository's converters (the same recipes as make_golden.py and
make_golden_pythia.py), and records the words and the converted arrays' digests.  The reference source is read
and executed here only; the fixture (long_golden.json) holds words.  Usage:
    python tests/golden/make_golden_long.py [/root/reference]
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
OUT = os.path.join(HERE, "long_golden.json")


def _module(name):
    spec = importlib.util.spec_from_file_location(name, os.path.join(HERE, name + ".py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def save(out):
    with open(OUT + ".tmp", "w") as f:
        json.dump(out, f, indent=1)
    os.replace(OUT + ".tmp", OUT)


def main():
    g2 = _module("make_golden")
    gp = _module("make_golden_pythia")
    sm = g2.load_pkg()
    from streaming_machine_amd import pythia
    t0 = time.time()
    out = {"generator": "tests/golden/make_golden_long.py",
           "reference": {"gpt2": "base2.py forward (definitions up to its tokenizer line)",
                         "pythia": "foundation0/pythia_base2.py forward (plates=finished, all stages int)"},
           "models": {}, "cases": []}
    work = tempfile.mkdtemp(prefix="sm_golden_long_")

    # GPT-2 124M, 64 streams: stream s prompt default_rng(4 + s), 32 tokens; 128 words
    kw = dict(seed=0, vocab=50257, n_ctx=1024)
    npz = sm.convert(sm.random_gpt2(**kw))
    out["models"]["gpt2_124m"] = dict(recipe=kw, digest=sm.array_digest(npz))
    d = os.path.join(work, "gpt2")
    os.makedirs(d, exist_ok=True)
    np.savez(os.path.join(d, "base2_gpt2.npz"), **npz)
    del npz
    ns = g2.base2_namespace(d)
    for s in (0, 1):
        prompt = sm.prompt_ids(4 + s, 32)
        got = []
        for i in range(128):
            got.append(int(ns["forward"](list(prompt) + got)))
            if i % 16 == 15:
                print(f"[{time.time() - t0:7.1f}s] c4 stream {s}: {i + 1} words", flush=True)
        out["cases"].append(dict(name=f"c4_stream{s}_p32_w128", model="gpt2_124m", prompt=prompt, words=got))
        save(out)
    del ns
    os.remove(os.path.join(d, "base2_gpt2.npz"))

    # Pythia-160m-shaped, 32 streams: stream s prompt default_rng(5 + s), 64 tokens of vocab 50304; 256 words
    kw = dict(seed=5, vocab=50304)
    sd, cfg = pythia.random_pythia(**kw)
    npz = pythia.convert_pythia(sd, cfg)
    del sd
    out["models"]["pythia_160m"] = dict(recipe=kw, digest=sm.array_digest(npz))
    d = os.path.join(work, "pythia")
    os.makedirs(d, exist_ok=True)
    np.savez(os.path.join(d, "base2_pythia-pythia_160m.npz"), **npz)
    del npz
    ns = gp.pythia_namespace(d, "pythia_160m")
    for s in (0, 1):
        prompt = sm.prompt_ids(5 + s, 64, 50304)
        got = []
        for i in range(256):
            words, _ = ns["forward"](list(prompt) + got)
            got.append(int(words[0]))
            if i % 32 == 31:
                print(f"[{time.time() - t0:7.1f}s] c5 stream {s}: {i + 1} words", flush=True)
        out["cases"].append(dict(name=f"py_c5_stream{s}_p64_w256", model="pythia_160m", prompt=prompt, words=got))
        save(out)
    print(f"wrote {OUT} in {time.time() - t0:.0f}s", flush=True)


if __name__ == "__main__":
    main()
