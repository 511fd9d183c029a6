"""The value cache at 64 bits (GPU).  base2.py's attention weighs each cached value as the raw int64 the qkv bank gave
(base2.py:85-99).  The machine keeps every value's low 32 bits and, beside them, the whole value; a head that holds a
value past 32 bits reads its values whole.  Checked two ways:
* with v64 = 1 every head reads whole values from the start, so the 64-bit reading runs on the golden workloads:
  the same words and recorded intermediates as base2.py (GPT-2, Pythia; one stream, the attention spread over chunks,
  batched streams, the prompt pass);
* a model whose layer-0 head-0 values are planted past 2^33 (its qkv bias): the words equal the oracle's exact int64
  run (past base2.py's 2^52 float64 bound the reference itself is not exact there, so the pin is the oracle's integer
  arithmetic), and the cached values read back whole;
* the Pythia machine with layer 0's head-0 values scaled by 2^16 (their column exponents; pythia_base2.py's integer
  attention is exact up to its 2^62 assert, which these stay below): the oracle's words, layer 0's attention row and
  the whole cached values.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden_case
from test_gpu_machine import compare_record, machine_record

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("att_split", [0, 1])
def test_whole_values_batch1_golden(sm, full_dir, golden, att_split):
    """GPT-2 124M, batch 1: base2.py's words and every recorded intermediate with every head reading whole values
    (att_split 1: through the attention spread over chunks)"""
    m = sm.Machine(full_dir, max_ctx=64, v64=True, att_split=att_split)
    c = golden_case(golden, "c1_p8_w16")
    for which in ("first", "last"):
        rec = c["records"][which]
        m.reset()
        m.record_at(rec["position"])
        m.prefill(c["prompt"])
        assert [int(w) for w in m.generate(len(c["words"]))[0]] == c["words"]
        compare_record(machine_record(m), rec)
    m.close()


@pytest.mark.parametrize("prefill_rows", [64, 0])
def test_whole_values_streams(sm, small_dir, small_oracle, prefill_rows):
    """three streams of the small model (and the prompt pass through the MFMA banks) reading whole values"""
    prompts = [sm.prompt_ids(50 + b, 8, 1000) for b in range(3)]
    m = sm.Machine(small_dir, max_ctx=64, max_streams=3, v64=True, prefill_rows=prefill_rows)
    got = m.streams(prompts, 10)
    m.close()
    for b in range(3):
        assert got[b] == small_oracle.generate(prompts[b], 10, 64), f"stream {b}"


def test_whole_values_long_context(sm, full_dir, full_oracle):
    """GPT-2 124M, batch 1, a 200-token prompt: the one-block attention (positions 64..159) and the spread one
    (from 160) reading whole values"""
    prompt = sm.prompt_ids(9, 200)
    m = sm.Machine(full_dir, max_ctx=256, v64=True)
    assert m.stream(prompt, 16) == full_oracle.generate(prompt, 16, 256)
    m.close()


@pytest.mark.parametrize("streams", [1, 3])
def test_whole_values_pythia(sm, py_small_dir, py_small_oracle, streams):
    """the Pythia machine (its turns, exact power and |v| sum(a) assert) reading whole values"""
    prompts = [sm.prompt_ids(80 + b, 8, 1000) for b in range(streams)]
    m = sm.Machine(py_small_dir, max_ctx=64, max_streams=streams, v64=True)
    got = m.streams(prompts, 10)
    m.close()
    for b in range(streams):
        assert got[b] == py_small_oracle.generate(prompts[b], 10, 64), f"stream {b}"


@pytest.fixture(scope="module")
def wide(sm, small_npz, tmp_path_factory):
    """the small model with layer 0's head-0 values past 2^33 (qkv bias of its 64 value columns), laid out"""
    import oracle
    npz = dict(small_npz)
    b = npz["qkv.0.b"].copy()
    b[1536:1600] += np.arange(64, dtype=np.int64) * (1 << 26) + (1 << 33)
    npz["qkv.0.b"] = b
    d = sm.layout(npz, str(tmp_path_factory.mktemp("wide_layout")))
    return d, oracle.Oracle(npz, bound=False)


@pytest.mark.parametrize("streams,att_split,prefill_rows", [(1, 0, 64), (1, 1, 64), (1, 0, 0), (3, 0, 64)],
                         ids=["one_block", "spread", "position_by_position", "three_streams"])
def test_values_past_32_bits(sm, wide, streams, att_split, prefill_rows):
    """values past 2^33 at every position of one head: the machine continues with them whole (no overflow error)
    and gives the oracle's exact int64 words; the cache holds them whole"""
    d, orc = wide
    prompts = [sm.prompt_ids(60 + b, 8, 1000) for b in range(streams)]
    m = sm.Machine(d, max_ctx=64, max_streams=streams, att_split=att_split, prefill_rows=prefill_rows)
    got = m.streams(prompts, 8)
    for b in range(streams):
        assert got[b] == orc.generate(prompts[b], 8, 64), f"stream {b}"
    s = orc.session(64)
    seq = prompts[0] + got[0]
    for t in seq[:-1]:
        s.step(t, want_head=False)
    for p in (0, 5, len(seq) - 2):
        v = s.read_kv(0, p)[2]
        assert np.abs(v[:64]).min() > 2 ** 31                 # the planted head: every value past 32 bits
        assert np.array_equal(m.read("v64", 0, 0, p), v)
        assert np.array_equal(m.read("v", 0, 0, p), v.astype(np.int32))   # the low 32 bits beside them
    m.close()


@pytest.fixture(scope="module")
def py_wide(sm, py_small_npz, tmp_path_factory):
    """the small Pythia model with layer 0's head-0 value columns (128-191 of the interleaved q, k, v) scaled by
    2^16 through their exponents, laid out: about a third of those values past 32 bits, varying with the position,
    while the attention sum stays below the reference's 2^62 assert (pythia_base2.py:139)"""
    from oracle.pythia import PythiaOracle
    npz = dict(py_small_npz)
    e = np.array(npz["qkv.0.e"]).copy()
    e[128:192] += 16
    npz["qkv.0.e"] = e
    d = sm.pythia.pythia_layout(npz, str(tmp_path_factory.mktemp("py_wide_layout")))
    return d, PythiaOracle(npz)


@pytest.mark.parametrize("streams,att_split", [(1, 0), (1, 1), (3, 0)], ids=["one_block", "spread", "three_streams"])
def test_pythia_values_past_32_bits(sm, py_wide, streams, att_split):
    """the Pythia machine with values past 32 bits in one head: the oracle's words, layer 0's attention row at the
    last step (stream 0) and the cache's whole values"""
    from oracle.pythia import new_record
    d, orc = py_wide
    prompts = [sm.prompt_ids(60 + b, 8, 1000) for b in range(streams)]
    m = sm.Machine(d, max_ctx=64, max_streams=streams, att_split=att_split)
    m.reset()
    m.record_at(len(prompts[0]) + 8 - 2)
    for b, p in enumerate(prompts):
        m.prefill(p, b)
    got = [[int(w) for w in row] for row in m.generate(8)]
    for b in range(streams):
        assert got[b] == orc.generate(prompts[b], 8, 64), f"stream {b}"
    s = orc.session(64)
    seq = prompts[0] + got[0]
    rec = new_record(orc.vocab)
    for i, t in enumerate(seq[:-1]):
        s.step(t, want_head=False, rec=rec if i == len(seq) - 2 else None)
    assert np.array_equal(m.read("att")[0], rec["att"][0])
    wide = 0
    for p in range(len(seq) - 1):
        v = s.read_kv(0, p)[2]
        wide += int((np.abs(v[:64]) > 2 ** 31).any())
        assert np.array_equal(m.read("v64", 0, 0, p), v)
        assert np.array_equal(m.read("v", 0, 0, p), v.astype(np.int32))
    assert wide >= 8                                            # most positions hold a value past 32 bits
    m.close()
