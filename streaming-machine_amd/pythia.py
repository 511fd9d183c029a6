"""The Pythia-160m-shaped integer machine's numbers: a seeded random checkpoint and its conversion.

Restates foundation0/pythia_convert.py (the only place a float exists) for one checkpoint:
  * every plate [in][out] as int16 with one power of two per output neuron, the smallest that holds the
    neuron's largest weight in 16 places (pythia_convert.py:57-68, 75-77); the head per word column, the embed
    table per word row (:104-106);
  * biases and the norms' offsets as whole numbers at the stream's scale 2^-16 (:72, 79, 89-90);
  * each norm's gain on 16 places with one power of two for the vector, NOT folded into the plate after it
    (:85-90);
  * tables: PHI and the arrival (as base2_convert.py builds them), LOG2/EXP2, cos/sin of the turns at 2^-30 for
    every position (rotary on the first quarter of each head, pairs (i, i + quarter/2)), eps40 = eps d^2 2^40
    and half_log2_hs = log2(head size)/2 at 2^-16 (:109-120).
The reference converts a finished and a start checkpoint onto one grid (X.w / X.s): each neuron's power of two is
the smallest that holds the larger of the two checkpoints' largest values (shared16, pythia_convert.py:51-60), the
norms' gain power likewise (:83-86).  Given no start, the finished checkpoint is written under both names, so the
reference's machine loads the file unchanged.  As in convert.py, ceil(log2(mx / 32767)) is evaluated exactly
through frexp.
"""
from __future__ import annotations

import json
import math
import os

import numpy as np

from .convert import _ceil_log2, stream, tables

PYTHIA_SHAPE = dict(n_layer=12, d=768, n_head=12, d_ff=3072, vocab=50304, n_ctx=2048, rotary_pct=0.25,
                    rotary_emb_base=10000, layer_norm_eps=1e-5)
P_BANKS = ("qkv", "proj", "fc", "mproj")
P_NORMS = ("ln1", "ln2")


def random_pythia(seed: int = 5, vocab: int = 50304, n_layer: int = 12, std: float = 0.02):
    """HF GPTNeoX-named float32 state dict of a Pythia-160m-shaped model (d=768, 12 heads of 64, FFN 3072,
    rotary on 25% of each head, parallel residual, untied embed_in / embed_out) and its config.

    One default_rng(seed) walks the state dict in GPTNeoXForCausalLM order; weights, biases and norm offsets are
    N(0, 0.02); norm gains are 1 + N(0, 0.02) (a literal N(0, 0.02) gain would shrink every normalised row about
    fifty times)."""
    rng = np.random.default_rng(seed)
    d, f = 768, 3072

    def nrm(*shape):
        return (rng.standard_normal(shape) * std).astype(np.float32)

    def gain(n):
        return (1.0 + rng.standard_normal(n) * std).astype(np.float32)

    sd = {"gpt_neox.embed_in.weight": nrm(vocab, d)}
    for l in range(n_layer):
        p = f"gpt_neox.layers.{l}."
        sd[p + "input_layernorm.weight"] = gain(d)
        sd[p + "input_layernorm.bias"] = nrm(d)
        sd[p + "post_attention_layernorm.weight"] = gain(d)
        sd[p + "post_attention_layernorm.bias"] = nrm(d)
        sd[p + "attention.query_key_value.weight"] = nrm(3 * d, d)     # torch Linear [out][in]
        sd[p + "attention.query_key_value.bias"] = nrm(3 * d)
        sd[p + "attention.dense.weight"] = nrm(d, d)
        sd[p + "attention.dense.bias"] = nrm(d)
        sd[p + "mlp.dense_h_to_4h.weight"] = nrm(f, d)
        sd[p + "mlp.dense_h_to_4h.bias"] = nrm(f)
        sd[p + "mlp.dense_4h_to_h.weight"] = nrm(d, f)
        sd[p + "mlp.dense_4h_to_h.bias"] = nrm(d)
    sd["gpt_neox.final_layer_norm.weight"] = gain(d)
    sd["gpt_neox.final_layer_norm.bias"] = nrm(d)
    sd["embed_out.weight"] = nrm(vocab, d)
    cfg = dict(PYTHIA_SHAPE, vocab=vocab, n_layer=n_layer)
    return sd, cfg


def q16(W: np.ndarray, axis: int, Ws: np.ndarray | None = None):
    """int16 values with one power of two per neuron along `axis` (0: per column, 1: per row), the smallest that
    holds the larger of W's and (given) Ws's largest values in 16 places; returns W's values, Ws's values (None
    when not given) and the powers (pythia_convert.py:51-60)."""
    mx = np.abs(W).max(axis)
    if Ws is not None:
        mx = np.maximum(mx, np.abs(Ws).max(axis))
    e = _ceil_log2(np.maximum(mx, 1e-30) / 32767)
    sh = np.exp2(np.expand_dims(e, axis).astype(np.float64))
    q = np.round(W / sh).astype(np.int64)
    qs = None if Ws is None else np.round(Ws / sh).astype(np.int64)
    if np.abs(q).max() > 32767 or (qs is not None and np.abs(qs).max() > 32767):
        raise ValueError("q16: a value does not fit 16 places")
    return q.astype(np.int16), (None if qs is None else qs.astype(np.int16)), e


def pythia_tables(d: int, hs: int, rot: int, n_pos: int, base: float, eps: float) -> dict:
    """The Pythia machine's tables (pythia_convert.py:109-120)."""
    t = tables()
    inv = float(base) ** (-np.arange(0, rot, 2) / rot)
    ang = np.arange(n_pos)[:, None] * inv[None, :]
    half = round(math.log2(hs) / 2 * 65536)
    if half * 2 != math.log2(hs) * 65536:
        raise ValueError("head size must be a power of two")
    return {"phi": t["phi"], "arrival": t["arrival"], "log2": t["log2"], "exp2": t["exp2"],
            "cos": np.round(np.cos(ang) * 2 ** 30).astype(np.int64), "sin": np.round(np.sin(ang) * 2 ** 30).astype(np.int64),
            "eps40": np.array(round(eps * d * d * 2 ** 40)), "half_log2_hs": np.array(half)}


def convert_pythia(sd: dict, cfg: dict, start: dict | None = None) -> dict:
    """GPTNeoX-named finished state dict (numpy or torch) + config, and optionally the start checkpoint's state
    dict, -> the npz dictionary pythia_base2.py loads (X.w finished, X.s start on the same per-neuron power X.e;
    X.b / X.bs, lnN.g / .gs / .ge / .b / .bs; pythia_convert.py:64-107).  Without a start the finished checkpoint
    stands for both."""
    def arr(d, k):
        v = d[k]
        if hasattr(v, "detach"):
            v = v.detach().cpu().numpy()
        return np.asarray(v, dtype=np.float64)

    def get(k):
        return arr(sd, k)

    def get0(k):
        return arr(sd if start is None else start, k)

    d, L, nh = cfg["d"], cfg["n_layer"], cfg["n_head"]
    hs = d // nh
    rot = int(hs * cfg["rotary_pct"])
    out = {}

    def plate(name, key, bias=True):
        w, ws, e = q16(get(key + ".weight").T, 0, get0(key + ".weight").T)
        out[name + ".w"], out[name + ".s"], out[name + ".e"] = w, ws, e
        if bias:
            out[name + ".b"], out[name + ".bs"] = stream(get(key + ".bias")), stream(get0(key + ".bias"))

    def norm(name, key):
        g, gs = get(key + ".weight"), get0(key + ".weight")
        ge = int(_ceil_log2(np.array([max(np.abs(g).max(), np.abs(gs).max(), 1e-30) / 32767]))[0])
        out[name + ".g"] = np.round(g / 2.0 ** ge).astype(np.int64)
        out[name + ".gs"] = np.round(gs / 2.0 ** ge).astype(np.int64)
        out[name + ".ge"] = np.array(ge)
        out[name + ".b"], out[name + ".bs"] = stream(get(key + ".bias")), stream(get0(key + ".bias"))

    for l in range(L):
        p = f"gpt_neox.layers.{l}."
        norm(f"ln1.{l}", p + "input_layernorm")
        norm(f"ln2.{l}", p + "post_attention_layernorm")
        plate(f"qkv.{l}", p + "attention.query_key_value")
        plate(f"proj.{l}", p + "attention.dense")
        plate(f"fc.{l}", p + "mlp.dense_h_to_4h")
        plate(f"mproj.{l}", p + "mlp.dense_4h_to_h")
    norm("lnf", "gpt_neox.final_layer_norm")
    plate("head", "embed_out", bias=False)
    out["embed.w"], out["embed.s"], out["embed.e"] = q16(get("gpt_neox.embed_in.weight"), 1, get0("gpt_neox.embed_in.weight"))
    out.update(pythia_tables(d, hs, rot, cfg["n_ctx"], cfg["rotary_emb_base"], cfg["layer_norm_eps"]))
    for k, v in dict(d=d, L=L, heads=nh, hs=hs, rot=rot, vocab=cfg["vocab"]).items():
        out[k] = np.array(v)
    return out


def select_plates(npz: dict, plates: str = "finished") -> dict:
    """foundation0/pythia_base2.py:44-46's `plates=`: "finished" (the converted checkpoint's plates, biases, norms
    and word tables), "start" (the start checkpoint's, which the converter keeps beside them as .s / .bs / .gs on
    the same powers of two) or "built" (finished - start, digit for digit: every plate, bias, gain, offset and word
    row, on the same powers of two).  A built digit takes 17 bits (int64 arrays here); pythia_layout writes such
    plates as two int16 halves whose difference is the digit."""
    if plates not in ("finished", "start", "built"):
        raise ValueError(f"plates={plates}: finished, start or built")
    out = dict(npz)
    if plates == "finished":
        return out
    for k in npz:
        for tail, start in ((".w", ".s"), (".b", ".bs"), (".g", ".gs")):
            if k.endswith(tail) and k[:-len(tail)] + start in npz:
                s0 = np.asarray(npz[k[:-len(tail)] + start])
                out[k] = s0 if plates == "start" else np.asarray(npz[k]).astype(np.int64) - s0.astype(np.int64)
    return out


def split_digits(w: np.ndarray):
    """A plate of digits within +-65535 as two int16 halves a - b = w: a = w clipped to int16, b = a - w (both
    within int16 since |w| <= 32767 + 32768)."""
    w = np.asarray(w, dtype=np.int64)
    if w.size and np.abs(w).max() > 65535:
        raise ValueError("split_digits: a digit past 17 bits")
    a = np.clip(w, -32768, 32767)
    return a.astype(np.int16), (a - w).astype(np.int16)


def shuffle_order(npz: dict, seed: int = 12345) -> dict:
    """foundation0/pythia_base2.py:42, 48-58's `order=shuffle` (an order-free check): the stream's 768 lanes in the
    order default_rng(seed).permutation(768); every plate that reads the stream (qkv, fc, the head) takes its rows
    in that order, every plate that writes it (proj, mproj) its columns, powers and biases, the norms their gains
    and offsets, the embed table its columns.  Every sum is of whole numbers, so every pile is the same number in
    its new place: the words and the head's piles are the plain machine's."""
    d = int(npz["d"])
    perm = np.random.default_rng(seed).permutation(d)
    out = dict(npz)
    for l in range(int(npz["L"])):
        for nm in P_NORMS:
            k = f"{nm}.{l}"
            out[k + ".g"], out[k + ".b"] = np.asarray(npz[k + ".g"])[perm], np.asarray(npz[k + ".b"])[perm]
        for nm in ("qkv", "fc"):
            out[f"{nm}.{l}.w"] = np.ascontiguousarray(np.asarray(npz[f"{nm}.{l}.w"])[perm])
        for nm in ("proj", "mproj"):
            k = f"{nm}.{l}"
            out[k + ".w"] = np.ascontiguousarray(np.asarray(npz[k + ".w"])[:, perm])
            out[k + ".e"], out[k + ".b"] = np.asarray(npz[k + ".e"])[perm], np.asarray(npz[k + ".b"])[perm]
    out["lnf.g"], out["lnf.b"] = np.asarray(npz["lnf.g"])[perm], np.asarray(npz["lnf.b"])[perm]
    out["head.w"] = np.ascontiguousarray(np.asarray(npz["head.w"])[perm])
    out["embed.w"] = np.ascontiguousarray(np.asarray(npz["embed.w"])[:, perm])
    return out


def pythia_layout(npz: dict, out_dir: str) -> str:
    """Write a converted Pythia model as a device-image directory for the HIP library.  The reference runs this
    machine on the CPU only and has no device format for it; this one extends base2_gpu.py's:

      {qkv,proj,fc,mproj}.{l}.wc / .e / .b   int16 [nin][nout], int32 [nout], int64 [nout] (as base2_gpu.py)
      head.wc / head.e                       int16 [768][vocab], int32 [vocab] (no bias)
      embed.wc / embed.e                     int16 [vocab][768], int32 [vocab] (a power of two per word)
      X.wsc (split digits only)              int16, the subtracted half of plate / word table X (digit = wc - wsc)
      {ln1,ln2}.{l}.g / .b, lnf.g / .b       int32 [768] gain on 16 places, int64 [768] offset at 2^-16
      phi.bin arrival.bin log2.bin exp2.bin cos.bin sin.bin   int64 (cos / sin [positions][rot / 2] at 2^-30)
      cosf.bin sinf.bin                      float64 [positions][rot / 2]: the float turn's cos and sin
      manifest.json  {"kind": "pythia", "banks": [...], "norms": [{"name", "ge"}, ...], "hs", "rot",
                      "half_log2_hs", "log2_768", "eps40", "arrival_len", "vocab", "split"}
    Plates whose digits leave int16 (plates=built) are written split: X.wc - X.wsc is the digit ("split": 1; the
    machine then runs at one stream, position by position).
    """
    os.makedirs(out_dir, exist_ok=True)
    L = int(npz["L"])
    banks, norms = [], []
    plates = [f"{b}.{l}" for l in range(L) for b in P_BANKS] + ["head", "embed"]
    split = any(int(np.max(npz[n + ".w"])) > 32767 or int(np.min(npz[n + ".w"])) < -32768 for n in plates)

    def write_plate(name):
        if split:
            a, b = split_digits(npz[name + ".w"])
            np.ascontiguousarray(b).tofile(os.path.join(out_dir, f"{name}.wsc"))
        else:
            a = np.asarray(npz[name + ".w"]).astype(np.int16)
        np.ascontiguousarray(a).tofile(os.path.join(out_dir, f"{name}.wc"))
        return a.shape

    for name in plates[:-1]:
        w_shape = write_plate(name)
        np.asarray(npz[name + ".e"]).astype(np.int32).tofile(os.path.join(out_dir, f"{name}.e"))
        if name != "head":
            np.asarray(npz[name + ".b"]).astype(np.int64).tofile(os.path.join(out_dir, f"{name}.b"))
        banks.append(dict(name=name, nin=int(w_shape[0]), nout=int(w_shape[1])))
    for name in [f"{n}.{l}" for l in range(L) for n in P_NORMS] + ["lnf"]:
        np.asarray(npz[name + ".g"]).astype(np.int32).tofile(os.path.join(out_dir, f"{name}.g"))
        np.asarray(npz[name + ".b"]).astype(np.int64).tofile(os.path.join(out_dir, f"{name}.b"))
        norms.append(dict(name=name, ge=int(npz[name + ".ge"])))
    write_plate("embed")
    np.asarray(npz["embed.e"]).astype(np.int32).tofile(os.path.join(out_dir, "embed.e"))
    for k in ("phi", "arrival", "log2", "exp2", "cos", "sin"):
        np.ascontiguousarray(npz[k]).astype(np.int64).tofile(os.path.join(out_dir, f"{k}.bin"))
    # turn=float (foundation0/pythia_base2.py:118-119): numpy's float64 cos and sin of position x 10000^(-2i/rot)
    rot = int(npz["rot"])
    ang = np.arange(len(npz["cos"]))[:, None] * (10000.0 ** (-np.arange(0, rot, 2) / rot))[None, :]
    np.cos(ang).astype(np.float64).tofile(os.path.join(out_dir, "cosf.bin"))
    np.sin(ang).astype(np.float64).tofile(os.path.join(out_dir, "sinf.bin"))
    man = dict(kind="pythia", banks=banks, norms=norms, hs=int(npz["hs"]), rot=int(npz["rot"]),
               half_log2_hs=int(npz["half_log2_hs"]), log2_768=round(math.log2(768) * 65536), eps40=int(npz["eps40"]),
               arrival_len=int(len(npz["arrival"])), vocab=int(npz["vocab"]), split=int(split))
    with open(os.path.join(out_dir, "manifest.json"), "w") as f:
        json.dump(man, f)
    return out_dir
