"""The Pythia oracle (oracle/pythia_oracle.c) against the golden vectors written from foundation0/pythia_base2.py
itself, plus negative controls that plant mistakes in the oracle's inputs and show the goldens catch them."""
from __future__ import annotations

import hashlib
import os

import numpy as np
import pytest

from conftest import REPO
from oracle.pythia import PythiaOracle


def h64(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(np.asarray(a, dtype=np.int64)).tobytes()).hexdigest()


def record_hashes(rec) -> dict:
    got = {}
    for l in range(12):
        got[f"stream.{l}"] = h64(rec["stream"][l])
        got[f"gauge.ln1.{l}"] = h64(rec["g1"][l])
        got[f"gauge.ln2.{l}"] = h64(rec["g2"][l])
        for k, b in enumerate(("qkv", "proj", "fc", "mproj")):
            nin, nout = (768, 768, 768, 3072)[k], (2304, 768, 3072, 768)[k]
            got[f"x16.{b}.{l}"] = h64(rec["x16"][l, k, :nin])
            got[f"ex.{b}.{l}"] = int(rec["ex"][l, k])
            got[f"pile.{b}.{l}"] = h64(rec["pile"][l, k, :nout])
            got[f"out.{b}.{l}"] = h64(rec["out"][l, k, :nout])
        got[f"att.{l}"] = h64(rec["att"][l])
        got[f"hid.{l}"] = h64(rec["hid"][l])
    got["stream.final"] = h64(rec["stream_final"])
    got["gauge.lnf"] = h64(rec["glnf"])
    got["x16.head"] = h64(rec["hx16"])
    got["ex.head"] = int(rec["hex"][0])
    got["pile.head"] = h64(rec["hpile"])
    got["logits"] = h64(rec["logits"])
    return got


def run_case(orc, case):
    """the case's words through the KV-cached oracle, recording the last position"""
    from oracle.pythia import new_record
    P, W = case["prompt"], case["words"]
    s = orc.session(len(P) + len(W))
    rec = new_record(orc.vocab)
    seq = P + W
    words = []
    for i in range(len(seq) - 1):
        w = s.step(seq[i], want_head=i >= len(P) - 1, rec=rec if i == len(seq) - 2 else None)
        if i >= len(P) - 1:
            words.append(w)
    return words, record_hashes(rec)


def small_cases(pgolden):
    return [c for c in pgolden["cases"] if c["model"] == "pythia_small"]


def test_converter_fingerprint(sm, py_small_npz, pgolden):
    """the converter rebuilds exactly the arrays the goldens were written from"""
    want = pgolden["models"]["pythia_small"]["digest"]
    assert sm.array_digest(py_small_npz) == want


def test_small_model_words_and_records(py_small_oracle, pgolden):
    for case in small_cases(pgolden):
        words, got = run_case(py_small_oracle, case)
        assert words == case["words"], case["name"]
        want = case["records"]["last"]
        keys = [k for k in want if k in got]
        assert len(keys) == 258
        bad = [k for k in keys if got[k] != want[k]]
        assert not bad, f"{case['name']}: {len(bad)} intermediates differ, first {sorted(bad)[:6]}"


def synth_qkv(seed: int, P: int, std: float) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return np.round(rng.standard_normal((P, 2304)) * std * 65536).astype(np.int64)


@pytest.mark.parametrize("which", [0, 1])
def test_attention_golden(py_small_oracle, pgolden, which):
    """turns, water levels, scores, arrival and the exact power at 300 and 1100 positions"""
    a = pgolden["attention"][which]
    A = py_small_oracle.attention(synth_qkv(a["seed"], a["P"], a["std"]))
    assert [h64(r)[:16] for r in A] == a["row_sha16"]
    assert h64(A) == a["out_sha256"]


def test_kv_cache_equals_recompute_position_by_position(py_small_oracle, pgolden):
    """the golden words come from full recomputes; the oracle's cache gives the same at every prefix"""
    case = small_cases(pgolden)[0]
    P = case["prompt"]
    for n in range(1, len(P) + 1):
        w = py_small_oracle.generate(P[:n], 1)
        if n == len(P):
            assert w == case["words"][:1]


# ---- negative controls: a planted mistake in the oracle's inputs must move the goldens ----

def _planted(npz, **changes):
    from oracle.pythia import PythiaOracle
    m = dict(npz)
    m.update(changes)
    return PythiaOracle(m)


def test_planted_turn_sign_is_caught(py_small_npz, pgolden):
    a = pgolden["attention"][0]
    orc = _planted(py_small_npz, sin=-py_small_npz["sin"])
    A = orc.attention(synth_qkv(a["seed"], a["P"], a["std"]))
    assert h64(A[0]) [:16] == a["row_sha16"][0]          # position 0 turns by angle 0: unchanged
    assert h64(A) != a["out_sha256"]


def test_planted_half_log2_is_caught(py_small_npz, pgolden):
    a = pgolden["attention"][0]
    orc = _planted(py_small_npz, half_log2_hs=np.array(int(py_small_npz["half_log2_hs"]) + 65536))
    assert h64(orc.attention(synth_qkv(a["seed"], a["P"], a["std"]))) != a["out_sha256"]


def test_planted_gain_offset_is_caught(py_small_npz, pgolden):
    case = small_cases(pgolden)[0]
    g = py_small_npz["ln2.3.g"].copy()
    g[5] += 1
    _, got = run_case(_planted(py_small_npz, **{"ln2.3.g": g}), case)
    want = case["records"]["last"]
    assert got["gauge.ln2.2"] == want["gauge.ln2.2"] and got["gauge.ln2.3"] != want["gauge.ln2.3"]


def _modes():
    import json
    path = os.path.join(REPO, "tests", "golden", "modes_golden.json")
    return json.load(open(path)) if os.path.exists(path) else None


def modes_npz(sm, case):
    """the plate / order switch of a modes_golden.json case applied to the finished-and-start model"""
    fin, cfg = sm.pythia.random_pythia(seed=5, vocab=1000)
    start, _ = sm.pythia.random_pythia(seed=6, vocab=1000)
    npz = sm.pythia.convert_pythia(fin, cfg, start=start)
    sw = dict(s.split("=") for s in case["switches"])
    npz = sm.pythia.select_plates(npz, sw.get("plates", "finished"))
    return sm.pythia.shuffle_order(npz) if sw.get("order") == "shuffle" else npz


def test_plate_and_order_switches(sm):
    """pythia_base2.py's plates=start and order=shuffle (its order-free check) as package transforms of the
    converted model: the oracle on them gives the words the reference gave with those switches.  plates=built's
    17-bit digits the oracle does not hold (it refuses them); the device's run is pinned to the reference's words
    and records by the GPU test."""
    g = _modes()
    if g is None:
        pytest.skip("modes_golden.json not written")
    fin, cfg = sm.pythia.random_pythia(seed=5, vocab=1000)
    start, _ = sm.pythia.random_pythia(seed=6, vocab=1000)
    assert sm.array_digest(sm.pythia.convert_pythia(fin, cfg, start=start)) == g["model"]["digest"]
    assert {tuple(c["switches"]) for c in g["cases"]} >= {("plates=start",), ("plates=built",), ("order=shuffle",)}
    for case in g["cases"]:
        if any(s.endswith("=float") for s in case["switches"]):
            continue                                  # (the oracle runs every stage in integers)
        if "plates=built" in case["switches"]:
            with pytest.raises(ValueError):
                PythiaOracle(modes_npz(sm, case))
            continue
        assert PythiaOracle(modes_npz(sm, case)).generate(case["prompt"], len(case["words"])) == case["words"], case["name"]
    with pytest.raises(ValueError):
        sm.pythia.select_plates({}, "other")


def test_built_plates_and_split_digits(sm, tmp_path):
    """plates=built (foundation0/pythia_base2.py:44-46): every plate, bias, gain, offset and word row is finished -
    start; the layout writes digits past int16 as two int16 halves whose difference is the digit"""
    fin, cfg = sm.pythia.random_pythia(seed=5, vocab=200, n_layer=12)
    start, _ = sm.pythia.random_pythia(seed=6, vocab=200, n_layer=12)
    npz = sm.pythia.convert_pythia(fin, cfg, start=start)
    built = sm.pythia.select_plates(npz, "built")
    for k, ks in (("qkv.3.w", "qkv.3.s"), ("head.w", "head.s"), ("embed.w", "embed.s"), ("fc.0.b", "fc.0.bs"),
                  ("ln2.5.g", "ln2.5.gs"), ("lnf.b", "lnf.bs")):
        assert np.array_equal(built[k], np.asarray(npz[k], np.int64) - np.asarray(npz[ks], np.int64)), k
    assert np.array_equal(built["qkv.3.e"], npz["qkv.3.e"])          # the same powers of two
    assert int(np.abs(built["qkv.0.w"]).max()) > 32767               # the seeded pair reaches 17 bits
    w = np.array([-65535, -32769, -32768, -1, 0, 1, 32767, 32768, 65535], np.int64)
    a, b = sm.pythia.split_digits(w)
    assert a.dtype == np.int16 and b.dtype == np.int16
    assert np.array_equal(a.astype(np.int64) - b.astype(np.int64), w)
    with pytest.raises(ValueError):
        sm.pythia.split_digits(np.array([65536]))
    d = sm.pythia.pythia_layout(built, str(tmp_path / "built"))
    import json
    assert json.load(open(os.path.join(d, "manifest.json")))["split"] == 1
    for name, shape in (("qkv.7", (768, 2304)), ("head", (768, 200)), ("embed", (200, 768))):
        hi = np.fromfile(os.path.join(d, f"{name}.wc"), np.int16).astype(np.int64)
        lo = np.fromfile(os.path.join(d, f"{name}.wsc"), np.int16).astype(np.int64)
        assert np.array_equal((hi - lo).reshape(shape), built[f"{name}.w"]), name
    plain = sm.pythia.pythia_layout(npz, str(tmp_path / "plain"))
    assert json.load(open(os.path.join(plain, "manifest.json")))["split"] == 0
    assert not os.path.exists(os.path.join(plain, "qkv.0.wsc"))
