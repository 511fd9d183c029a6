"""GPU parity of the whole decode step through the C ABI: emitted words, every recorded intermediate and the KV
cache, bit-exact against base2.py's golden vectors and the oracle."""
from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import REPO, golden_case, h64

pytestmark = pytest.mark.gpu

BANKS = ("qkv", "proj", "fc", "mproj")
NIN = (768, 768, 768, 3072)
NOUT = (2304, 768, 3072, 768)


def machine_record(m) -> dict:
    """the device record of one position, keyed like the golden fixture"""
    x16, exls, pile = m.read("x16"), m.read("exls"), m.read("pile")
    qkv, att, hid, rr = m.read("qkv"), m.read("att"), m.read("hid"), m.read("rresid")
    out = {}
    for l in range(12):
        for k, b in enumerate(BANKS):
            out[f"x16.{b}.{l}"] = h64(x16[l, k, :NIN[k]])
            out[f"pile.{b}.{l}"] = h64(pile[l, k, :NOUT[k]])
            out[f"ex.{b}.{l}"] = int(exls[l, k, 0])
            if b in ("qkv", "fc"):
                out[f"ls.{b}.{l}"] = int(exls[l, k, 1])
        out[f"out.qkv.{l}"] = h64(qkv[l])
        out[f"att.{l}"] = h64(att[l])
        out[f"hid.{l}"] = h64(hid[l])
        out[f"resid_attn.{l}"] = h64(rr[l, 0])
        out[f"resid_mlp.{l}"] = h64(rr[l, 1])
        out[f"out.mproj.{l}"] = h64(rr[l, 1] - rr[l, 0])             # the MLP half's addition
        if l:
            out[f"out.proj.{l}"] = h64(rr[l, 0] - rr[l - 1, 1])      # the attention half's addition
    hexls = m.read("hexls")
    out["x16.head"] = h64(m.read("hx16"))
    out["ex.head"], out["ls.head"] = int(hexls[0]), int(hexls[1])
    out["pile.head"] = h64(m.read("hpile"))
    out["logits"] = h64(m.read("logits"))
    return out


def compare_record(got: dict, want: dict):
    keys = [k for k in want if k in got]
    assert len(keys) > 200
    bad = [k for k in keys if got[k] != want[k]]
    assert not bad, f"{len(bad)} intermediates differ, first: {sorted(bad)[:8]}"


@pytest.mark.parametrize("use_graph,verify_tables", [(True, False), (False, False), (True, True)])
def test_small_model_words(sm, small_dir, golden, use_graph, verify_tables):
    c = golden_case(golden, "small_p8_w8")
    m = sm.Machine(small_dir, max_ctx=64, use_graph=use_graph, verify_tables=verify_tables)
    assert m.tables_verified          # the layout's tables are base2_convert.py's
    assert m.stream(c["prompt"], len(c["words"])) == c["words"]
    m.close()


def test_verify_tables_refuses_a_changed_table(sm, small_dir, small_npz, tmp_path):
    """verify_tables=True refuses a layout whose tables differ from their formulas; the default reads them as given"""
    d = sm.layout(small_npz, str(tmp_path))
    e = np.fromfile(os.path.join(d, "exp2.bin"), dtype=np.int64)
    e[777] += 1
    e.tofile(os.path.join(d, "exp2.bin"))
    with pytest.raises(sm.SmError):
        sm.Machine(d, max_ctx=64, verify_tables=True)
    m = sm.Machine(d, max_ctx=64)
    assert not m.tables_verified
    m.close()


@pytest.mark.parametrize("streams,att_split", [(1, 0), (3, 0), (1, 1)])
def test_changed_arrival_table_is_read_as_given(sm, small_npz, tmp_path, streams, att_split):
    """with the reference's tables the machine computes each arrival from its formula (the create-time check found
    them equal entry for entry); a layout whose arrival table differs is read as given: the attention rows of the
    recorded position, at batch 1 (one block a head, and spread over chunks of positions) and with three streams,
    equal the oracle's run with the same table"""
    import oracle
    npz = dict(small_npz)
    arr = npz["arrival"].copy()
    arr[1:2048] = arr[1:2048] * 3 // 4                  # every arrival within 2 units of the maximum
    npz["arrival"] = arr
    d = sm.layout(npz, str(tmp_path))
    prompt = sm.prompt_ids(2, 8, 1000)
    want, base = oracle.new_record(1000), oracle.new_record(1000)
    oracle.Oracle(npz).forward(prompt, rec=want)          # the last position's intermediates
    oracle.Oracle(small_npz).forward(prompt, rec=base)
    assert not np.array_equal(want["att"], base["att"])  # the change reaches the attention
    m = sm.Machine(d, max_ctx=64, max_streams=streams, att_split=att_split)
    assert not m.tables_verified
    m.reset()
    m.record_at(len(prompt) - 1)
    for b in range(streams):
        m.prefill(prompt, b)
    m.generate(1)
    np.testing.assert_array_equal(m.read("att"), want["att"])
    m.close()


def test_small_model_record(sm, small_dir, golden):
    c = golden_case(golden, "small_p8_w8")
    m = sm.Machine(small_dir, max_ctx=64)
    last = c["records"]["last"]
    m.reset()
    m.record_at(last["position"])
    m.prefill(c["prompt"])
    m.generate(len(c["words"]))
    compare_record(machine_record(m), last)
    m.close()


@pytest.fixture(scope="module")
def full_machine(sm, full_dir):
    m = sm.Machine(full_dir, max_ctx=1024)
    yield m
    m.close()


def test_batch1_8_token_prompt_words_and_records(full_machine, golden):
    """GPT-2 124M, batch 1, 8-token prompt, 16 greedy words: the words and every intermediate of the first and
    the last position against base2.py"""
    m = full_machine
    c = golden_case(golden, "c1_p8_w16")
    for which in ("first", "last"):
        rec = c["records"][which]
        m.reset()
        m.record_at(rec["position"])
        m.prefill(c["prompt"])
        assert [int(w) for w in m.generate(len(c["words"]))[0]] == c["words"]
        compare_record(machine_record(m), rec)


@pytest.mark.parametrize("stream", [0, 1])
def test_gpt2_32_token_prompts(full_machine, golden, stream):
    """32-token prompts of the batched config, one stream at a time"""
    c = golden_case(golden, f"c4_stream{stream}_p32_w4")
    assert full_machine.stream(c["prompt"], len(c["words"])) == c["words"]


def test_kv_cache_matches_oracle(full_machine, full_oracle, sm):
    """the cache the device keeps equals the oracle's (k16, ek, v at every layer and position)"""
    m = full_machine
    prompt = sm.prompt_ids(7, 5)
    words = m.stream(prompt, 6)
    s = full_oracle.session(32)
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


def test_long_context_against_oracle(full_machine, full_oracle, sm):
    """a 200-token prompt and 40 words (context 240; the attention spread over chunks of positions, the machine's
    default past position 128): words equal the KV-cached oracle's"""
    prompt = sm.prompt_ids(9, 200)
    assert full_machine.stream(prompt, 40) == full_oracle.generate(prompt, 40, 256)


@pytest.mark.parametrize("att_split", [-1, 1, 150])
def test_attention_structures_give_the_same_machine(sm, full_dir, full_oracle, golden, att_split):
    """the batch-1 attention one block a head (att_split -1), spread over chunks from position 1 on, and switching
    at position 150 inside a run: the same words as the oracle over a 200-token prompt (prompt positions through
    the decode step, so every position 0..239 runs one of the two), the KV cache late in the context, and base2.py's
    words and every recorded intermediate of the golden sequence"""
    m = sm.Machine(full_dir, max_ctx=256, att_split=att_split, prefill_rows=0)
    prompt = sm.prompt_ids(9, 200)
    words = m.stream(prompt, 40)
    assert words == full_oracle.generate(prompt, 40, 256)
    s = full_oracle.session(256)
    seq = prompt + words
    for i, t in enumerate(seq[:-1]):
        s.step(t, want_head=False)
    for l in (0, 11):
        for p in (149, 150, 238):
            k16, ek, v = s.read_kv(l, p)
            assert np.array_equal(m.read("k16", l, 0, p), k16)
            assert np.array_equal(m.read("ek", l, 0, p), ek)
            assert np.array_equal(m.read("v", l, 0, p), v)
    c = golden_case(golden, "c1_p8_w16")
    for which in ("first", "last"):
        rec = c["records"][which]
        m.reset()
        m.record_at(rec["position"])
        m.prefill(c["prompt"])
        assert [int(w) for w in m.generate(len(c["words"]))[0]] == c["words"]
        compare_record(machine_record(m), rec)
    m.record_at(-1)
    m.close()


def test_thousand_token_prompt_batch1(sm, full_dir):
    """batch 1, a 1000-token prompt and 8 words: the attention spread over 16 chunks a head (positions 999..1006)"""
    import json as _json
    with open(os.path.join(REPO, "tests", "golden", "long_oracle.json")) as f:
        case = {c["name"]: c for c in _json.load(f)["cases"]}["gpt2_p1000_w8"]
    m = sm.Machine(full_dir, max_ctx=1008)
    assert m.stream(case["prompt"], 8) == case["words"]
    m.close()


def test_prompt_of_one_word_and_continuation(full_machine, full_oracle, sm):
    m = full_machine
    m.reset()
    m.prefill([464])
    a = [int(w) for w in m.generate(3)[0]]
    b = [int(w) for w in m.generate(2)[0]]        # continues where it stopped
    assert a + b == full_oracle.generate([464], 5)


def test_errors(full_machine, sm):
    m = full_machine
    m.reset()
    with pytest.raises(sm.SmError) as e:
        m.prefill([50257])
    assert e.value.code == -1
    with pytest.raises(sm.SmError) as e:
        m.generate(2)                             # no prompt
    assert e.value.code == -7
    m.prefill(list(range(1000)))
    with pytest.raises(sm.SmError) as e:
        m.generate(100)                           # 1000 + 100 - 1 > 1024
    assert e.value.code == -5


@pytest.mark.parametrize("use_graph,rows", [(True, 64), (False, 64), (True, 0)])
def test_profiled_machine_gives_the_same_words(sm, full_dir, golden, use_graph, rows):
    """one timed head per decode step: the steps after the prompt pass (rows > 0), or every position (rows = 0)"""
    c = golden_case(golden, "c1_p8_w16")
    m = sm.Machine(full_dir, max_ctx=64, profile=True, graph_steps=4, use_graph=use_graph, prefill_rows=rows)
    assert m.stream(c["prompt"], len(c["words"])) == c["words"]
    n, us = m.profile()
    assert n == len(c["words"]) + (len(c["prompt"]) - 1 if rows == 0 else 0) and us > 0
    m.close()


@pytest.mark.parametrize("kind,streams,use_graph", [("gpt2", 1, True), ("gpt2", 1, False), ("gpt2", 3, True),
                                                    ("pythia", 1, True), ("pythia", 3, True)])
def test_runs_of_steps(sm, small_dir, small_oracle, py_small_dir, py_small_oracle, kind, streams, use_graph):
    """a generation cut into calls of 5, 1, 4 and 7 words, with graphs of 3 steps and a recorded position part way:
    runs of one, two and three steps, chunk ends inside a call and a run split by the recorded step.  A run's later
    steps take the race of the step before into their first kernel and the run ends with the race, so every cut
    is a place where the machine must hold a raced position; the words are the oracle's"""
    d, orc = (small_dir, small_oracle) if kind == "gpt2" else (py_small_dir, py_small_oracle)
    prompts = [sm.prompt_ids(70 + b, 6, 1000) for b in range(streams)]
    m = sm.Machine(d, max_ctx=64, max_streams=streams, graph_steps=3, use_graph=use_graph)
    m.reset()
    m.record_at(6 + 7)
    for b, p in enumerate(prompts):
        m.prefill(p, b)
    got = [[] for _ in range(streams)]
    for n in (5, 1, 4, 7):
        for b, row in enumerate(m.generate(n)):
            got[b] += [int(w) for w in row]
    m.close()
    for b in range(streams):
        assert got[b] == orc.generate(prompts[b], 17, 64), f"stream {b}"
