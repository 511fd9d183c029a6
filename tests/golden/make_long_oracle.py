"""Write the long-context fixtures of the batched workloads with the C oracle (oracle/, test infrastructure).

The oracle is pinned against the reference's own words and intermediates (base2_golden.json, pythia_golden.json,
and the full-length words of streams 0 and 1 in long_golden.json, compared by tests/test_oracle_long.py); this
script extends those checks to more streams and to the KV cache deep into the context, where running the
reference for every stream would take hours.  Everything written here is labelled as the oracle's.
  * GPT-2 124M, 64 streams of 32-token prompts (stream s: default_rng(4 + s)), 128 words: the words of streams
    0, 1, 31 and 63; the key rows, their water levels and the value rows of stream 63 at layers 0 and 11 and
    positions 0, 128 and 158; the stream row after the last position.
  * the Pythia-160m-shaped machine, 32 streams of 64-token prompts (stream s: default_rng(5 + s)), 256 words:
    the words of streams 0, 1 and 31; the cache of stream 31 at layers 0 and 11, positions 0, 200 and 318.
  * GPT-2 124M with a 1000-token prompt (default_rng(77)) and 8 words, and the same for Pythia (default_rng(78)):
    every attention of the prompt pass and of the decode steps runs past 999 positions; words, the cache at
    positions 0, 500, 998, 1005 of layers 0 and 11, and the stream row.
Usage:  python tests/golden/make_long_oracle.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)


def h64(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(np.asarray(a, dtype=np.int64)).tobytes()).hexdigest()


def run(session, prompt, n_words):
    """prompt then n_words words, each fed back (the last word is not stepped): words and the positions stepped"""
    words, tok = [], None
    for i, t in enumerate(prompt):
        tok = session.step(t, want_head=i == len(prompt) - 1)
    for _ in range(n_words):
        words.append(tok)
        if len(words) == n_words:
            break
        tok = session.step(tok)
    return words


def cache(session, layers, positions):
    out = {}
    for l in layers:
        for p in positions:
            k16, ek, v = session.read_kv(l, p)
            out[f"{l}.{p}"] = dict(k16=h64(k16), ek=h64(ek), v=h64(v))
    return out


def main():
    sys.path.insert(0, HERE)
    from make_golden import load_pkg
    sm = load_pkg()
    import oracle
    from oracle.pythia import PythiaOracle
    t0 = time.time()
    out = {"generator": "tests/golden/make_long_oracle.py", "source": "the C oracle (oracle/base2_oracle.c, "
           "oracle/pythia_oracle.c), pinned against the reference's goldens", "hash": "sha256 of int64 little-endian bytes",
           "models": {}, "cases": []}

    npz = sm.convert(sm.random_gpt2(seed=0, vocab=50257, n_ctx=1024))
    out["models"]["gpt2_124m"] = dict(recipe=dict(seed=0, vocab=50257, n_ctx=1024), digest=sm.array_digest(npz))
    orc = oracle.Oracle(npz)
    for s in (0, 1, 31, 63):
        prompt = sm.prompt_ids(4 + s, 32)
        ses = orc.session(160)
        words = run(ses, prompt, 128)
        c = dict(name=f"c4_stream{s}_p32_w128", model="gpt2_124m", prompt=prompt, words=words)
        if s == 63:
            c["cache"] = cache(ses, (0, 11), (0, 128, 158))
            c["resid"] = h64(ses.resid())
        out["cases"].append(c)
        print(f"[{time.time() - t0:6.1f}s] c4 stream {s}: {words[:8]}", flush=True)
    prompt = sm.prompt_ids(77, 1000)
    ses = orc.session(1008)
    words = run(ses, prompt, 8)
    out["cases"].append(dict(name="gpt2_p1000_w8", model="gpt2_124m", prompt=prompt, words=words,
                             cache=cache(ses, (0, 11), (0, 500, 998, 1005)), resid=h64(ses.resid())))
    print(f"[{time.time() - t0:6.1f}s] gpt2 1000-token prompt: {words}", flush=True)
    del orc, ses, npz

    sd, cfg = sm.pythia.random_pythia(seed=5, vocab=50304)
    npz = sm.pythia.convert_pythia(sd, cfg)
    del sd
    out["models"]["pythia_160m"] = dict(recipe=dict(seed=5, vocab=50304), digest=sm.array_digest(npz))
    orc = PythiaOracle(npz)
    for s in (0, 1, 31):
        prompt = sm.prompt_ids(5 + s, 64, 50304)
        ses = orc.session(320)
        words = run(ses, prompt, 256)
        c = dict(name=f"py_c5_stream{s}_p64_w256", model="pythia_160m", prompt=prompt, words=words)
        if s == 31:
            c["cache"] = cache(ses, (0, 11), (0, 200, 318))
            c["resid"] = h64(ses.resid())
        out["cases"].append(c)
        print(f"[{time.time() - t0:6.1f}s] c5 stream {s}: {words[:8]}", flush=True)
    prompt = sm.prompt_ids(78, 1000, 50304)
    ses = orc.session(1008)
    words = run(ses, prompt, 8)
    out["cases"].append(dict(name="pythia_p1000_w8", model="pythia_160m", prompt=prompt, words=words,
                             cache=cache(ses, (0, 11), (0, 500, 998, 1005)), resid=h64(ses.resid())))
    print(f"[{time.time() - t0:6.1f}s] pythia 1000-token prompt: {words}", flush=True)
    with open(os.path.join(HERE, "long_oracle.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote long_oracle.json in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
