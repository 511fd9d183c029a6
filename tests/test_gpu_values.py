"""The value cache at 64 bits (GPU).  base2.py's attention weighs each cached value as the raw int64 the qkv bank gave
(base2.py:85-99).  The machine keeps every value's low 32 bits and, beside them, the whole value; a head that holds a
value past 32 bits reads its values whole.  Checked two ways:
* with v64 = 1 every head reads whole values from the start, so the 64-bit reading runs on the golden workloads:
  the same words and recorded intermediates as base2.py (GPT-2, Pythia; one stream, the attention spread over chunks,
  batched streams, the prompt pass);
* a model whose layer-0 head-0 values are planted past 2^33 (its qkv bias): the words equal the oracle's exact int64
  run (past base2.py's 2^52 float64 bound the reference itself is not exact there, so the pin is the oracle's integer
  arithmetic), and the cached values read back whole.
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
