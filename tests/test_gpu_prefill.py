"""GPU parity of the prompt passes: with prefill_rows > 0 every prompt position but the last goes through the
int8 MFMA banks that many rows at a time (base2_stream.swift:74-91, 274-275: the prompt through each layer at
once), the rows of a pass drawn stream by stream in position order.  The words equal the oracle's, and the
whole KV cache, every layer and position, equals the one the position-by-position machine (prefill_rows = 0)
keeps."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden_case
from test_gpu_machine import compare_record, machine_record

pytestmark = pytest.mark.gpu


def kv_cache(m, streams: int, npos: int) -> dict:
    out = {}
    for name in ("k16", "ek", "v"):
        out[name] = np.stack([np.stack([np.stack([m.read(name, l, s, p) for p in range(npos)]) for s in range(streams)])
                              for l in range(12)])
    return out


def run(sm, d, prompts, n, rows, max_ctx=64):
    m = sm.Machine(d, max_ctx=max_ctx, max_streams=len(prompts), prefill_rows=rows)
    if len(prompts) == 1:
        words = [m.stream(prompts[0], n)]
    else:
        words = m.streams(prompts, n)
    kv = kv_cache(m, len(prompts), len(prompts[0]) + n - 1)
    m.close()
    return words, kv


def same_kv(a: dict, b: dict):
    for name in a:
        bad = np.argwhere(np.any(a[name] != b[name], axis=-1))
        assert bad.size == 0, f"{name} differs at (layer, stream, position) {bad[:4].tolist()}"


@pytest.mark.parametrize("rows", [1, 5, 16, 64])
def test_gpt2_one_stream(sm, small_dir, small_oracle, rows):
    """40-token prompt: passes of 1, 5, 16 and 64 rows (one, partial and several row tiles; 39 rows in one pass)"""
    prompt = sm.prompt_ids(11, 40, 1000)
    want = small_oracle.generate(prompt, 4)
    w0, kv0 = run(sm, small_dir, [prompt], 4, 0)
    w1, kv1 = run(sm, small_dir, [prompt], 4, rows)
    assert w0 == [want] and w1 == [want]
    same_kv(kv0, kv1)


@pytest.mark.parametrize("rows", [16, 64])
def test_gpt2_three_streams(sm, small_dir, small_oracle, rows):
    """three streams, 20-token prompts: 57 prompt rows, passes that cross from one stream into the next"""
    prompts = [sm.prompt_ids(20 + s, 20, 1000) for s in range(3)]
    want = [small_oracle.generate(p, 5) for p in prompts]
    w0, kv0 = run(sm, small_dir, prompts, 5, 0)
    w1, kv1 = run(sm, small_dir, prompts, 5, rows)
    assert w0 == want and w1 == want
    same_kv(kv0, kv1)


def test_gpt2_full_model_prompt_past_128(sm, full_dir, full_oracle):
    """GPT-2 124M, a 150-token prompt (prompt rows past position 128 read their keys in the attention's loop)"""
    prompt = sm.prompt_ids(12, 150)
    m = sm.Machine(full_dir, max_ctx=160, prefill_rows=64)
    assert m.stream(prompt, 3) == full_oracle.generate(prompt, 3, 160)
    k = [m.read("k16", 11, 0, p) for p in (0, 100, 148)]
    m.close()
    m0 = sm.Machine(full_dir, max_ctx=160, prefill_rows=0)
    m0.stream(prompt, 3)
    assert all(np.array_equal(a, m0.read("k16", 11, 0, p)) for a, p in zip(k, (0, 100, 148)))
    m0.close()


def test_record_inside_the_prompt(sm, small_dir, golden):
    """a record asked for at a prompt position: the pass stops short of it and the steps record it (the layers'
    intermediates; no head runs at a prompt position whose word is known)"""
    c = golden_case(golden, "small_p8_w8")
    recs = []
    for rows in (0, 64):
        m = sm.Machine(small_dir, max_ctx=64, prefill_rows=rows)
        m.reset()
        m.record_at(5)
        m.prefill(c["prompt"])
        assert [int(w) for w in m.generate(len(c["words"]))[0]] == c["words"]
        recs.append({k: v for k, v in machine_record(m).items() if not k.endswith(".head") and k != "logits"})
        m.close()
    compare_record(recs[1], recs[0])


@pytest.mark.parametrize("streams,rows", [(1, 64), (1, 7), (3, 16)])
def test_pythia(sm, py_small_dir, py_small_oracle, streams, rows):
    """the Pythia machine (turned keys by position in the pass, parallel residual): words and cache"""
    prompts = [sm.prompt_ids(30 + s, 24, 1000) for s in range(streams)]
    want = [py_small_oracle.generate(p, 4) for p in prompts]
    w0, kv0 = run(sm, py_small_dir, prompts, 4, 0)
    w1, kv1 = run(sm, py_small_dir, prompts, 4, rows)
    assert w0 == want and w1 == want
    same_kv(kv0, kv1)


def test_rejects_pass_sizes(sm, small_dir):
    for rows in (-1, 65):
        with pytest.raises(sm.SmError) as e:
            sm.Machine(small_dir, max_ctx=64, prefill_rows=rows)
        assert e.value.code == -1
