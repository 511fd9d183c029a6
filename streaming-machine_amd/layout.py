"""The device-image directory: base2_gpu.py's format, unchanged (base2_gpu.py:9-17).

  {name}.wc   int16 [nin][nout], input-major       for name in qkv.l, proj.l, fc.l, mproj.l (l = 0..11), head
  {name}.e    int32 [nout]  per-column power of two
  {name}.b    int64 [nout]  per-column bias at the stream's scale
  wte.bin, wpe.bin, phi.bin, arrival.bin, log2.bin, exp2.bin   int64
  manifest.json  {"banks": [{"name", "nin", "nout"}, ...], "log2_768", "eps40", "arrival_len"}

A directory written by the reference's own base2_gpu.py loads unchanged, and so does one written here.
The HIP library (sm_create) reads this directory and lays the banks out for the GPU itself.
"""
from __future__ import annotations

import json
import os

import numpy as np

from .convert import BANKS


def bank_names(n_layer: int = 12):
    return [f"{b}.{l}" for l in range(n_layer) for b in BANKS] + ["head"]


def layout(npz: dict, out_dir: str, n_layer: int = 12) -> str:
    """Write the npz dictionary as a device-image directory; returns the directory."""
    os.makedirs(out_dir, exist_ok=True)
    banks = []
    for name in bank_names(n_layer):
        w = np.ascontiguousarray(npz[name + ".w"]).astype(np.int16)
        nin, nout = w.shape
        w.tofile(os.path.join(out_dir, f"{name}.wc"))
        np.asarray(npz[name + ".e"]).astype(np.int32).tofile(os.path.join(out_dir, f"{name}.e"))
        np.asarray(npz[name + ".b"]).astype(np.int64).tofile(os.path.join(out_dir, f"{name}.b"))
        banks.append(dict(name=name, nin=int(nin), nout=int(nout)))
    for k in ("wte", "wpe", "phi", "arrival", "log2", "exp2"):
        np.asarray(npz[k]).astype(np.int64).tofile(os.path.join(out_dir, f"{k}.bin"))
    man = dict(banks=banks, log2_768=int(npz["log2_768"]), eps40=int(npz["eps40"]), arrival_len=int(len(npz["arrival"])))
    with open(os.path.join(out_dir, "manifest.json"), "w") as f:
        json.dump(man, f)
    return out_dir


def load_layout(dirname: str) -> dict:
    """Read a device-image directory back into the npz dictionary (memory-mapped where large)."""
    with open(os.path.join(dirname, "manifest.json")) as f:
        man = json.load(f)
    out = {}
    for b in man["banks"]:
        name, nin, nout = b["name"], b["nin"], b["nout"]
        out[name + ".w"] = np.fromfile(os.path.join(dirname, f"{name}.wc"), dtype=np.int16).reshape(nin, nout)
        out[name + ".e"] = np.fromfile(os.path.join(dirname, f"{name}.e"), dtype=np.int32).astype(np.int64)
        out[name + ".b"] = np.fromfile(os.path.join(dirname, f"{name}.b"), dtype=np.int64)
    for k in ("phi", "arrival", "log2", "exp2"):
        out[k] = np.fromfile(os.path.join(dirname, f"{k}.bin"), dtype=np.int64)
    out["wte"] = np.fromfile(os.path.join(dirname, "wte.bin"), dtype=np.int64).reshape(-1, 768)
    out["wpe"] = np.fromfile(os.path.join(dirname, "wpe.bin"), dtype=np.int64).reshape(-1, 768)
    out["log2_768"] = np.array(man["log2_768"])
    out["eps40"] = np.array(man["eps40"])
    return out


def rewire(npz: dict, seed: int, n_layer: int = 12):
    """The random wiring of base2_stream.swift:161-190 (its seed= test): the stream's 768 channels (one order for
    every layer), each layer's heads, the dimensions inside each head (one order shared by q and k, another for
    v), each layer's 3072 neurons and the words at the top, all shuffled; every bank's rows and columns, its
    powers and biases, and the word and position tables follow.  Every sum is of whole numbers, so every pile is
    the same number in its new place and the machine's words are the same (ties between equal top logits aside,
    which go to the lowest slot).  The permutations come from numpy's default_rng(seed) (the reference's own
    generator is not needed: any shuffle must give the same words).

    Returns (the rewired npz, the permutations): slot j of the word table holds word perms["words"][j], so a
    prompt goes in as slots (perms["slot_of"][word]) and the machine's slots come back as perms["words"][slot].
    """
    rng = np.random.default_rng(seed)
    d, vocab = 768, len(npz["wte"])
    chan = rng.permutation(d)
    out = dict(npz)
    perms = {"chan": chan, "layers": []}
    for l in range(n_layer):
        hp, dqk, dv, neu = rng.permutation(12), rng.permutation(64), rng.permutation(64), rng.permutation(3072)
        qkv_cols = np.array([part * 768 + hp[h] * 64 + (dqk[k] if part < 2 else dv[k])
                             for part in range(3) for h in range(12) for k in range(64)])
        proj_rows = np.array([hp[h] * 64 + dv[k] for h in range(12) for k in range(64)])
        for name, rp, cp in ((f"qkv.{l}", chan, qkv_cols), (f"proj.{l}", proj_rows, chan),
                             (f"fc.{l}", chan, neu), (f"mproj.{l}", neu, chan)):
            out[name + ".w"] = np.ascontiguousarray(np.asarray(npz[name + ".w"])[np.ix_(rp, cp)])
            out[name + ".e"] = np.asarray(npz[name + ".e"])[cp]
            out[name + ".b"] = np.asarray(npz[name + ".b"])[cp]
        perms["layers"].append({"qkv_cols": qkv_cols, "proj_rows": proj_rows, "neurons": neu})
    words = rng.permutation(vocab)
    out["head.w"] = np.ascontiguousarray(np.asarray(npz["head.w"])[np.ix_(chan, words)])
    out["head.e"] = np.asarray(npz["head.e"])[words]
    out["head.b"] = np.asarray(npz["head.b"])[words]
    out["wte"] = np.ascontiguousarray(np.asarray(npz["wte"])[np.ix_(words, chan)])
    out["wpe"] = np.ascontiguousarray(np.asarray(npz["wpe"])[:, chan])
    slot_of = np.empty(vocab, dtype=np.int64)
    slot_of[words] = np.arange(vocab)
    perms["words"], perms["slot_of"] = words, slot_of
    return out, perms
