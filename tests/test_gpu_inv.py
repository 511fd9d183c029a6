"""The complement machine (base2_stream.swift:26 `inv`, "the whole machine on the negative") on the GPU.

The stream row, every plate and every light are held bit-complemented on the device; each pile is corrected by the
plate's column sum, the light's sum and the input count; the stream updates subtract; the race takes the smallest
complemented logit.  The reference's claim for it (base2_stream.swift:296) is that the words are the plain
machine's; here every word, every recorded intermediate (base2.py's golden records) and the KV cache must equal
the plain machine's, and the stream row the device holds must be the bitwise complement of the plain one.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden_case
from test_gpu_machine import compare_record, machine_record

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def inv_machine(sm, full_dir):
    m = sm.Machine(full_dir, max_ctx=256, prefill_rows=0, inv=True)
    yield m
    m.close()


@pytest.fixture(scope="module")
def plain_machine(sm, full_dir):
    m = sm.Machine(full_dir, max_ctx=256, prefill_rows=0)
    yield m
    m.close()


def test_complement_words_and_records(inv_machine, golden):
    """GPT-2 124M, 8-token prompt, 16 words: the words and every intermediate of the first and the last position
    against base2.py's golden records"""
    m = inv_machine
    c = golden_case(golden, "c1_p8_w16")
    for which in ("first", "last"):
        rec = c["records"][which]
        m.reset()
        m.record_at(rec["position"])
        m.prefill(c["prompt"])
        assert [int(w) for w in m.generate(len(c["words"]))[0]] == c["words"]
        compare_record(machine_record(m), rec)
    m.record_at(-1)


def test_complement_stream_and_cache(inv_machine, plain_machine, sm):
    """a 200-token prompt and 40 words: the same words and KV cache as the plain machine; the stream row is its
    complement"""
    prompt = sm.prompt_ids(9, 200)
    want = plain_machine.stream(prompt, 40)
    assert inv_machine.stream(prompt, 40) == want
    for l in (0, 6, 11):
        for p in (0, 100, 238):
            for name in ("k16", "ek", "v"):
                assert np.array_equal(inv_machine.read(name, l, 0, p), plain_machine.read(name, l, 0, p)), (name, l, p)
    r_inv, r = inv_machine.read("resid"), plain_machine.read("resid")
    assert np.array_equal(r_inv, ~r)
    assert not np.array_equal(r_inv, r)


def test_complement_plain_launches(sm, full_dir, golden):
    """kernel by kernel (no graphs), and continuing a run"""
    c = golden_case(golden, "c4_stream1_p32_w4")
    m = sm.Machine(full_dir, max_ctx=64, prefill_rows=0, inv=True, use_graph=False)
    m.reset()
    m.prefill(c["prompt"])
    a = [int(w) for w in m.generate(2)[0]]
    b = [int(w) for w in m.generate(2)[0]]
    assert a + b == c["words"]
    m.close()


@pytest.mark.parametrize("kw", [dict(max_streams=2, prefill_rows=0), dict(prefill_rows=64)])
def test_complement_limits(sm, full_dir, kw):
    """the complement machine is the batch-1 GEMV path with the prompt position by position"""
    with pytest.raises(sm.SmError) as e:
        sm.Machine(full_dir, max_ctx=64, inv=True, **kw)
    assert e.value.code == -1


def test_complement_not_pythia(sm, py_small_dir):
    with pytest.raises(sm.SmError) as e:
        sm.Machine(py_small_dir, max_ctx=64, prefill_rows=0, inv=True)
    assert e.value.code == -1
