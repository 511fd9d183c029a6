"""GPU parity of the Pythia-shaped machine (foundation0/pythia_base2.py) through the C ABI: words, every recorded
intermediate and the KV cache, bit-exact against the reference's golden vectors and the Pythia oracle."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import h64
from test_oracle_pythia import run_case, small_cases

pytestmark = pytest.mark.gpu

BANKS = ("qkv", "proj", "fc", "mproj")
NIN = (768, 768, 768, 3072)
NOUT = (2304, 768, 3072, 768)


def machine_record(m, stream0) -> dict:
    """the device record of one position keyed like the golden fixture; stream0 is the row entering layer 0
    (the device records the stream after each half layer, so out.proj.0 needs it)"""
    x16, exls, pile = m.read("x16"), m.read("exls"), m.read("pile")
    qkv, att, hid, rr = m.read("qkv"), m.read("att"), m.read("hid"), m.read("rresid")
    gauge, fcpre = m.read("gauge"), m.read("fcpre")
    out = {}
    for l in range(12):
        entering = stream0 if l == 0 else rr[l - 1, 1]
        out[f"stream.{l}"] = h64(entering)
        out[f"gauge.ln1.{l}"] = h64(gauge[l, 0])
        out[f"gauge.ln2.{l}"] = h64(gauge[l, 1])
        for k, b in enumerate(BANKS):
            out[f"x16.{b}.{l}"] = h64(x16[l, k, :NIN[k]])
            out[f"ex.{b}.{l}"] = int(exls[l, k, 0])
            out[f"pile.{b}.{l}"] = h64(pile[l, k, :NOUT[k]])
        out[f"out.qkv.{l}"] = h64(qkv[l])
        out[f"out.proj.{l}"] = h64(rr[l, 0] - entering)           # the attention half's addition (int64 wraps)
        out[f"out.fc.{l}"] = h64(fcpre[l])
        out[f"out.mproj.{l}"] = h64(rr[l, 1] - rr[l, 0])
        out[f"att.{l}"] = h64(att[l])
        out[f"hid.{l}"] = h64(hid[l])
    out["stream.final"] = h64(rr[11, 1])
    out["gauge.lnf"] = h64(m.read("hgauge"))
    out["x16.head"] = h64(m.read("hx16"))
    out["ex.head"] = int(m.read("hexls")[0])
    out["pile.head"] = h64(m.read("hpile"))
    out["logits"] = h64(m.read("logits"))
    return out


def oracle_stream0(orc, case):
    from oracle.pythia import new_record
    s = orc.session(len(case["prompt"]) + len(case["words"]))
    seq = case["prompt"] + case["words"]
    rec = new_record(orc.vocab)
    for i in range(len(seq) - 1):
        s.step(seq[i], want_head=False, rec=rec if i == len(seq) - 2 else None)
    return rec["stream"][0].copy()


@pytest.mark.parametrize("use_graph,att_split", [(True, 0), (False, 0), (True, 1)])
def test_small_model_words_and_records(sm, py_small_dir, py_small_oracle, pgolden, use_graph, att_split):
    """att_split 1: every step's attention spread over chunks of positions (the turns and exact power there)"""
    m = sm.Machine(py_small_dir, max_ctx=64, use_graph=use_graph, att_split=att_split)
    assert m.kind == "pythia"
    for case in small_cases(pgolden):
        last = case["records"]["last"]
        m.reset()
        m.record_at(last["position"])
        m.prefill(case["prompt"])
        assert [int(w) for w in m.generate(len(case["words"]))[0]] == case["words"], case["name"]
        got = machine_record(m, oracle_stream0(py_small_oracle, case))
        keys = [k for k in last if k in got]
        assert len(keys) == 258
        bad = [k for k in keys if got[k] != last[k]]
        assert not bad, f"{case['name']}: {len(bad)} intermediates differ, first {sorted(bad)[:6]}"
    m.close()


def test_pythia_32_streams_golden_words(sm, py_full_dir, pgolden):
    """the two golden streams of the 160m-shaped workload: 64-word prompts, 4 words each"""
    m = sm.Machine(py_full_dir, max_ctx=128)
    for c in [c for c in pgolden["cases"] if c["model"] == "pythia_160m"]:
        assert m.stream(c["prompt"], len(c["words"])) == c["words"], c["name"]
    m.close()


def test_kv_cache_matches_oracle(sm, py_small_dir, py_small_oracle):
    m = sm.Machine(py_small_dir, max_ctx=64)
    prompt = sm.prompt_ids(60, 6, 1000)
    words = m.stream(prompt, 6)
    s = py_small_oracle.session(32)
    seq = prompt + words
    ow = []
    for i, t in enumerate(seq[:-1]):
        w = s.step(t, want_head=i >= len(prompt) - 1)
        if i >= len(prompt) - 1:
            ow.append(w)
    assert ow == words
    for l in (0, 5, 11):
        for p in (0, 3, len(seq) - 2):
            k16, ek, v = s.read_kv(l, p)
            assert np.array_equal(m.read("k16", l, 0, p), k16)
            assert np.array_equal(m.read("ek", l, 0, p), ek)
            assert np.array_equal(m.read("v", l, 0, p), v)
    assert np.array_equal(m.read("resid"), s.resid())
    m.close()


@pytest.mark.parametrize("att_split", [0, -1, 310])
def test_long_context_against_oracle(sm, py_small_dir, py_small_oracle, att_split):
    """a 300-word prompt and 24 words: turns at positions past 256, context 324; the attention spread over chunks
    of positions (the default), one block a head, and switching inside the decode steps"""
    m = sm.Machine(py_small_dir, max_ctx=400, att_split=att_split)
    prompt = sm.prompt_ids(61, 300, 1000)
    assert m.stream(prompt, 24) == py_small_oracle.generate(prompt, 24, 400)
    m.close()


@pytest.mark.parametrize("use_graph,rows", [(True, 64), (False, 64), (True, 0)])
def test_profiled_machine(sm, py_small_dir, pgolden, use_graph, rows):
    c = small_cases(pgolden)[0]
    m = sm.Machine(py_small_dir, max_ctx=64, profile=True, graph_steps=4, use_graph=use_graph, prefill_rows=rows)
    assert m.stream(c["prompt"], len(c["words"])) == c["words"]
    n, us = m.profile()
    assert n == len(c["words"]) + (len(c["prompt"]) - 1 if rows == 0 else 0) and us > 0
    m.close()


# ---- batched streams (int8 MFMA contraction, per-stream race) ----

@pytest.mark.parametrize("B", [3, 20])
def test_small_model_streams(sm, py_small_dir, py_small_oracle, B):
    prompts = [sm.prompt_ids(80 + b, 8, 1000) for b in range(B)]
    prompts[B - 1] = prompts[0]
    m = sm.Machine(py_small_dir, max_ctx=64, max_streams=B)
    got = m.streams(prompts, 10)
    m.close()
    assert got[B - 1] == got[0]
    for b in range(B):
        assert got[b] == py_small_oracle.generate(prompts[b], 10, 64), f"stream {b}"


@pytest.mark.parametrize("use_graph", [True, False])
def test_small_model_batched_record(sm, py_small_dir, py_small_oracle, pgolden, use_graph):
    case = small_cases(pgolden)[0]
    last = case["records"]["last"]
    m = sm.Machine(py_small_dir, max_ctx=64, max_streams=5, use_graph=use_graph)
    m.reset()
    m.record_at(last["position"])
    prompts = [case["prompt"]] + [sm.prompt_ids(90 + b, len(case["prompt"]), 1000) for b in range(4)]
    for b, p in enumerate(prompts):
        m.prefill(p, b)
    assert [int(w) for w in m.generate(len(case["words"]))[0]] == case["words"]
    got = machine_record(m, oracle_stream0(py_small_oracle, case))
    bad = [k for k in last if k in got and got[k] != last[k]]
    assert not bad, f"{len(bad)} intermediates differ, first {sorted(bad)[:6]}"
    m.close()


def test_pythia_32_streams_64_token_prompts(sm, py_full_dir, py_full_npz, pgolden):
    """32 streams of 64-word prompts: the two golden streams, a sample against the oracle, a late stream's cache"""
    from oracle.pythia import PythiaOracle
    cs = [c for c in pgolden["cases"] if c["model"] == "pythia_160m"]
    prompts = [cs[0]["prompt"], cs[1]["prompt"]] + [sm.prompt_ids(500 + b, 64, 50304) for b in range(2, 32)]
    m = sm.Machine(py_full_dir, max_ctx=96, max_streams=32)
    got = m.streams(prompts, 4)
    assert got[0] == cs[0]["words"] and got[1] == cs[1]["words"]
    orc = PythiaOracle(py_full_npz)
    for b in (13, 31):
        assert got[b] == orc.generate(prompts[b], 4, 96), f"stream {b}"
    s = orc.session(96)
    seq = prompts[31] + got[31]
    for t in seq[:-1]:
        s.step(t, want_head=False)
    for l in (0, 11):
        for p in (0, 63, len(seq) - 2):
            k16, ek, v = s.read_kv(l, p)
            assert np.array_equal(m.read("k16", l, 31, p), k16)
            assert np.array_equal(m.read("ek", l, 31, p), ek)
            assert np.array_equal(m.read("v", l, 31, p), v)
    m.close()


@pytest.mark.parametrize("streams", [1, 3])
def test_rshift_assert(sm, py_small_npz, tmp_path, streams):
    """foundation0/pythia_base2.py:63: a left shift past 2^(62 + s) stops the reference.  A planted head power of
    two (word 5: 2^40) turns the head's plain shift into a left shift of 40 and more places: the oracle stops, and
    the device reports SM_E_OVERFLOW (batch 1: the GEMV head; 3 streams: the MFMA head)"""
    from oracle.pythia import PythiaOracle
    npz = dict(py_small_npz)
    e = np.array(npz["head.e"]).copy()
    e[5] = 40
    npz["head.e"] = e
    prompt = sm.prompt_ids(50, 8, 1000)
    with pytest.raises(ArithmeticError):
        PythiaOracle(npz).generate(prompt, 4)
    d = str(tmp_path / f"py_shift_{streams}")
    sm.pythia.pythia_layout(npz, d)
    m = sm.Machine(d, max_ctx=32, max_streams=streams)
    with pytest.raises(sm.SmError) as ex:
        m.streams([prompt] * streams, 4)
    assert ex.value.code == -6
    m.close()


@pytest.mark.parametrize("streams,att_split", [(1, 0), (2, 0), (1, 1)])
def test_plate_and_order_switches(sm, tmp_path, streams, att_split):
    """pythia_base2.py's plates=finished|start|built and order=shuffle (the finished-and-start model of
    modes_golden.json): words and every recorded intermediate of the last position against the reference run
    with each switch (the shuffled machine's intermediates in their shuffled places; plates=built's 17-bit digits
    as split plates, one stream only); att_split 1: one stream with every step's attention spread over chunks of
    positions and its output row formed in proj's blocks"""
    from test_oracle_pythia import _modes, modes_npz
    g = _modes()
    if g is None:
        pytest.skip("modes_golden.json not written")
    for case in g["cases"]:
        d = str(tmp_path / f"{case['name']}_{streams}")
        sm.pythia.pythia_layout(modes_npz(sm, case), d)
        kw = {s.split("=")[0]: "float" for s in case["switches"] if s.endswith("=float")}
        kw["att_split"] = att_split
        if "plates=built" in case["switches"] or len(kw) > 1:  # split digits, float stages: one stream, position by position
            if streams > 1:
                with pytest.raises(sm.SmError):
                    sm.Machine(d, max_ctx=32, max_streams=streams, **kw)
                continue
            kw["prefill_rows"] = 0
        m = sm.Machine(d, max_ctx=32, max_streams=streams, **kw)
        last = case["records"]["last"]
        m.reset()
        m.record_at(last["position"])
        for s in range(streams):
            m.prefill(case["prompt"], s)
        got = m.generate(len(case["words"]))
        assert all([int(w) for w in row] == case["words"] for row in got), case["name"]
        rec = machine_record(m, np.zeros(768, dtype=np.int64))
        m.close()
        keys = [k for k in last if k in rec and k not in ("stream.0", "out.proj.0")]
        assert len(keys) > 200
        bad = sorted(k for k in keys if rec[k] != last[k])
        assert not bad, f"{case['name']}: {len(bad)} intermediates differ, first {bad[:6]}"
