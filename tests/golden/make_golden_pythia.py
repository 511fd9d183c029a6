"""Write golden vectors from the reference's own foundation0/pythia_base2.py (run here, in the build container).

Why: the Pythia machine's stages compose into a forward pass that no fixture of the reference pins for
random-init weights (its words_pythia-*.json need the real checkpoints, which are not available offline).  So
this script executes pythia_base2.py's definitions (its __main__ block is not run) with __file__ placed in a
temporary directory that holds this repository's converted npz (the reference loads base2_pythia-<size>.npz
from its own directory), on seeded models, and records:
  * the converted arrays' SHA-256 (a test proves the same model was rebuilt),
  * the greedy words of each case (forward(prompt + words)[0][0], word by word, as its run-on loop does),
  * SHA-256 of every intermediate row of the last position of the last forward call (the stream entering each
    layer, both gauges, each plate's light, water level, pile and output, the attention output, the edge
    output; the head's gauge, light, pile and logits),
  * attention outputs on synthetic QKV matrices (per-head interleaved q, k, v) at 300 and 1100 positions.
The fixtures (pythia_golden.json) are data; the reference source is only read and executed here and never
copied.  Usage:  python tests/golden/make_golden_pythia.py [/root/reference]
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from make_golden import h64, load_pkg  # noqa: E402

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"


def pythia_namespace(npz_dir: str, size: str) -> dict:
    """Execute pythia_base2.py's definitions as if the file sat in npz_dir (where the npz is)."""
    path = os.path.join(REF, "foundation0", "pythia_base2.py")
    src = open(path).read()
    ns: dict = {"__name__": "pythia_golden", "__file__": os.path.join(npz_dir, "pythia_base2.py")}
    argv = sys.argv
    sys.argv = ["pythia_base2.py", f"size={size}"]
    try:
        exec(compile(src, path, "exec"), ns)
    finally:
        sys.argv = argv
    return ns


class Recorder:
    """Wraps pythia_base2.py's stage functions in its namespace; keeps the last row of each stage's numbers."""

    def __init__(self, ns: dict):
        self.ns, self.on, self.rec, self.layer, self.head = ns, False, {}, 0, False
        self.orig = {k: ns[k] for k in ("gauge", "plain", "attention", "edge", "to16", "product")}
        for k in self.orig:
            ns[k] = getattr(self, k)

    def put(self, key, row):
        if self.on:
            self.rec[key] = h64(row)

    def put_int(self, key, v):
        if self.on:
            self.rec[key] = int(v)

    def gauge(self, R, name):
        if name.startswith("ln1."):
            self.layer = int(name.split(".")[1])
            self.put(f"stream.{self.layer}", R[-1])
        if name == "lnf":
            self.put("stream.final", R[-1])
        out = self.orig["gauge"](R, name)
        self.put(f"gauge.{name}", out[-1])
        self.head = name == "lnf"
        return out

    def plain(self, X, name):
        out = self.orig["plain"](X, name)
        if self.on:
            w, e, b, wmax = self.ns["PL"][name]
            x16, ex = self.orig["to16"](X[-1:])
            pile = self.orig["product"](x16, w, wmax)
            self.put(f"x16.{name}", x16[-1])
            self.put_int(f"ex.{name}", ex[-1])
            self.put(f"pile.{name}", pile[-1])
            self.put(f"out.{name}", out[-1])
        return out

    def attention(self, QKV):
        out = self.orig["attention"](QKV)
        self.put(f"att.{self.layer}", out[-1])
        return out

    def edge(self, H):
        out = self.orig["edge"](H)
        self.put(f"hid.{self.layer}", out[-1])
        return out

    def to16(self, X):
        x16, ex = self.orig["to16"](X)
        if self.head:
            self.put("x16.head", x16[-1])
            self.put_int("ex.head", ex[-1])
        return x16, ex

    def product(self, x16, w, wmax):
        p = self.orig["product"](x16, w, wmax)
        if self.head:
            self.put("pile.head", p[-1])
            self.head = False
        return p


def run_words(ns, rc: Recorder, prompt, n_words):
    got, rec = [], {}
    for i in range(n_words):
        rc.on = i == n_words - 1
        rc.rec = {}
        words, lg = ns["forward"](list(prompt) + got)
        got.append(int(words[0]))
        if rc.on:
            row = lg[-1]
            order = np.argsort(-row, kind="stable")[:5]
            rec = dict(rc.rec, position=len(prompt) + i - 1, logits=h64(row),
                       top5=[[int(j), int(row[j])] for j in order])
        rc.on = False
    return got, rec


def synth_qkv(seed: int, P: int, std: float) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return np.round(rng.standard_normal((P, 2304)) * std * 65536).astype(np.int64)


def main():
    sm = load_pkg()
    from streaming_machine_amd import pythia
    t0 = time.time()
    out = {"generator": "tests/golden/make_golden_pythia.py",
           "reference": "foundation0/pythia_base2.py (definitions; plates=finished, all stages int)",
           "hash": "sha256 of int64 little-endian bytes", "models": {}, "cases": [], "attention": []}
    work = tempfile.mkdtemp(prefix="sm_golden_py_")
    specs = [("pythia_small", dict(seed=5, vocab=1000)), ("pythia_160m", dict(seed=5, vocab=50304))]
    for mname, kw in specs:
        sd, cfg = pythia.random_pythia(**kw)
        npz = pythia.convert_pythia(sd, cfg)
        del sd
        out["models"][mname] = dict(recipe=kw, digest=sm.array_digest(npz))
        d = os.path.join(work, mname)
        os.makedirs(d, exist_ok=True)
        np.savez(os.path.join(d, f"base2_pythia-{mname}.npz"), **npz)
        del npz
        ns = pythia_namespace(d, mname)
        rc = Recorder(ns)
        print(f"[{time.time() - t0:7.1f}s] {mname}: pythia_base2.py loaded", flush=True)
        if mname == "pythia_small":
            cases = [("py_small_p8_w8", sm.prompt_ids(50, 8, kw["vocab"]), 8),
                     ("py_small_p1_w6", sm.prompt_ids(51, 1, kw["vocab"]), 6)]
        else:
            cases = [(f"py_c5_stream{s}_p64_w4", sm.prompt_ids(5 + s, 64, kw["vocab"]), 4) for s in range(2)]
        for cname, prompt, nw in cases:
            words, rec = run_words(ns, rc, prompt, nw)
            out["cases"].append(dict(name=cname, model=mname, prompt=prompt, words=words, records={"last": rec}))
            print(f"[{time.time() - t0:7.1f}s] {cname}: {words}", flush=True)
        if mname == "pythia_160m":
            att = rc.orig["attention"]
            for seed, P, std in ((6, 300, 2.0), (6, 1100, 4.0)):
                Q = synth_qkv(seed, P, std)
                A = att(Q)
                out["attention"].append(dict(seed=seed, P=P, std=std, out_sha256=h64(A),
                                             row_sha16=[h64(r)[:16] for r in A], last_row=[int(v) for v in A[-1]]))
                print(f"[{time.time() - t0:7.1f}s] attention P={P} std={std}", flush=True)
        del ns, rc
        os.remove(os.path.join(d, f"base2_pythia-{mname}.npz"))
    with open(os.path.join(HERE, "pythia_golden.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote pythia_golden.json in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
