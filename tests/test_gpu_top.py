"""The collapsing top read (base2_stream_fr.swift:4-15, top=fr) on the GPU, batch 1.

The head reads the high-byte plane (w >> 8) of every word, bounds each word's score exactly from the light alone,
and reads the low bytes (w & 255) of the words whose upper bound reaches the best lower bound.  Checked here:
the words are the full read's (base2.py's golden words, and the plain machine over a long context); every
survivor's exact pile and score are the oracle's; every word set aside scores below the winner (from the oracle's
full logits); a recorded step (which reads the full table) still records every intermediate.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden_case
from test_gpu_machine import compare_record, machine_record

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def top_machine(sm, full_dir):
    m = sm.Machine(full_dir, max_ctx=256, top="fr")
    yield m
    m.close()


def _oracle_head(full_oracle, prompt, words):
    """the oracle's head piles and logits at the position that gave the last word"""
    from oracle import new_record
    s = full_oracle.session(len(prompt) + len(words))
    seq = list(prompt) + list(words)
    rec = new_record(full_oracle.vocab)
    for i in range(len(seq) - 1):
        last = i == len(seq) - 2
        w = s.step(seq[i], want_head=last, rec=rec if last else None)
    assert w == words[-1]
    return rec["head_pile"], rec["logits"]


def _check_survivors(m, full_oracle, prompt, words):
    n, rows = m.top()
    pile, logits = _oracle_head(full_oracle, prompt, words)
    assert 1 <= n <= 1024
    assert len(rows) == n
    surv = {w for w, _, _ in rows}
    assert words[-1] in surv
    for w, p, y in rows:
        assert p == pile[w] and y == logits[w], f"word {w}"
    out = np.ones(len(logits), bool)
    out[list(surv)] = False
    assert (logits[out] < logits[words[-1]]).all()      # every word set aside is below the winner
    return n


def test_top_read_8_token_prompt(top_machine, full_oracle, golden):
    c = golden_case(golden, "c1_p8_w16")
    got = top_machine.stream(c["prompt"], len(c["words"]))
    assert got == c["words"]
    n = _check_survivors(top_machine, full_oracle, c["prompt"], got)
    print(f"survivors at the last step: {n} of 50257")


def test_top_read_long_context(top_machine, full_oracle, sm, full_dir):
    prompt = sm.prompt_ids(9, 200)
    got = top_machine.stream(prompt, 40)
    plain = sm.Machine(full_dir, max_ctx=256)
    assert got == plain.stream(prompt, 40)
    plain.close()
    _check_survivors(top_machine, full_oracle, prompt, got)


def test_top_read_records_a_full_step(top_machine, golden):
    c = golden_case(golden, "c1_p8_w16")
    rec = c["records"]["last"]
    m = top_machine
    m.reset()
    m.record_at(rec["position"])
    m.prefill(c["prompt"])
    assert [int(w) for w in m.generate(len(c["words"]))[0]] == c["words"]
    compare_record(machine_record(m), rec)
    m.record_at(-1)


@pytest.mark.parametrize("kw", [dict(max_streams=2), dict(head_grid=256), dict(inv=True, prefill_rows=0)])
def test_top_read_limits(sm, full_dir, kw):
    """asked for where it does not apply, the top read is refused; "auto" takes the full read there"""
    with pytest.raises(sm.SmError) as e:
        sm.Machine(full_dir, max_ctx=64, top="fr", **kw)
    assert e.value.code == -1
    m = sm.Machine(full_dir, max_ctx=64, top="auto", **kw)
    assert not m.top_read
    m.close()


def test_full_read_is_the_default_auto_takes_the_top_read(sm, full_dir, py_small_dir):
    m = sm.Machine(full_dir, max_ctx=64)
    assert not m.top_read
    m.close()
    m = sm.Machine(full_dir, max_ctx=64, top="auto")
    assert m.top_read
    m.close()
    m = sm.Machine(py_small_dir, max_ctx=64, top="auto")   # the Pythia machine has no top read
    assert not m.top_read
    m.close()
