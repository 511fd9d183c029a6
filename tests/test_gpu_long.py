"""Full-length parity of the batched workloads and the attention block path deep into the context (GPU).

* 64 streams of GPT-2 124M (32-token prompts, 128 words, context to 160) and 32 streams of the Pythia-160m-shaped
  machine (64-token prompts, 256 words, context to 320): every word of several streams, and the KV cache and
  stream row of the last stream late in the context, against the long fixtures.  Streams 0 and 1 are checked
  against the reference's own words (long_golden.json, written by executing base2.py / pythia_base2.py), the
  others against the oracle's (long_oracle.json; the oracle is pinned to the reference's words by
  tests/test_oracle_long.py).
* A 1000-token prompt on a two-stream machine of each model: the prompt pass and the decode steps attend over
  999 to 1006 positions with the batched attention kernel (the block path).
* The batched attention kernel on the attention workload's synthetic rows (T = 128, 512, 1024) against base2.py's
  attention.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from conftest import REPO, h64, synth_qkv

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

GOLD = os.path.join(REPO, "tests", "golden")


def _cases(name):
    path = os.path.join(GOLD, name)
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return {c["name"]: c for c in json.load(f)["cases"]}


ORC = _cases("long_oracle.json")
REF = _cases("long_golden.json")


def _check_cache(m, case, stream):
    for key, want in case["cache"].items():
        l, p = (int(x) for x in key.split("."))
        assert h64(m.read("k16", l, stream, p)) == want["k16"], f"k16 layer {l} position {p}"
        assert h64(m.read("ek", l, stream, p)) == want["ek"], f"ek layer {l} position {p}"
        assert h64(m.read("v", l, stream, p)) == want["v"], f"v layer {l} position {p}"
    assert h64(m.read("resid", 0, stream)) == case["resid"]


def test_gpt2_64_streams_128_words_full_length(sm, full_dir):
    """64 streams, 128 words each: streams 0, 1, 31, 63 word for word, stream 63's cache at 0, 128, 158"""
    m = sm.Machine(full_dir, max_ctx=160, max_streams=64)
    prompts = [sm.prompt_ids(4 + s, 32) for s in range(64)]
    got = m.streams(prompts, 128)
    for s in (0, 1, 31, 63):
        assert got[s] == ORC[f"c4_stream{s}_p32_w128"]["words"], f"stream {s}"
    for s in (0, 1):
        if f"c4_stream{s}_p32_w128" in REF:
            assert got[s] == REF[f"c4_stream{s}_p32_w128"]["words"], f"stream {s} against base2.py"
    _check_cache(m, ORC["c4_stream63_p32_w128"], 63)
    m.close()


def test_pythia_32_streams_256_words_full_length(sm, py_full_dir):
    """32 Pythia streams, 256 words each: streams 0, 1, 31 word for word, stream 31's cache at 0, 200, 318"""
    m = sm.Machine(py_full_dir, max_ctx=320, max_streams=32)
    prompts = [sm.prompt_ids(5 + s, 64, 50304) for s in range(32)]
    got = m.streams(prompts, 256)
    for s in (0, 1, 31):
        assert got[s] == ORC[f"py_c5_stream{s}_p64_w256"]["words"], f"stream {s}"
    for s in (0, 1):
        if f"py_c5_stream{s}_p64_w256" in REF:
            assert got[s] == REF[f"py_c5_stream{s}_p64_w256"]["words"], f"stream {s} against pythia_base2.py"
    _check_cache(m, ORC["py_c5_stream31_p64_w256"], 31)
    m.close()


@pytest.mark.parametrize("model", ["gpt2", "pythia"])
def test_thousand_token_prompt_two_streams(sm, full_dir, py_full_dir, model):
    """a 1000-token prompt on both streams of a two-stream machine, 8 words: attention over 999..1006 positions"""
    case = ORC[f"{model}_p1000_w8"]
    m = sm.Machine(full_dir if model == "gpt2" else py_full_dir, max_ctx=1008, max_streams=2)
    got = m.streams([case["prompt"], case["prompt"]], 8)
    assert got[0] == case["words"] and got[1] == case["words"]
    for s in (0, 1):
        _check_cache(m, case, s)
    m.close()


def test_batched_attention_kernel_golden(sm, golden):
    """the attention workload (T = 128, 512, 1024) through the batched attention kernel, two streams at once: every row of both
    against base2.py's own attention"""
    t = sm.Tables(sm.tables())
    ctx, rows = 1024, 2
    for case in golden["attention"]:
        Q = synth_qkv(case["seed"], case["P"], case["std"])
        P = len(Q)
        k16 = torch.zeros((rows, 12, ctx, 64), dtype=torch.int16, device="cuda")
        km = torch.zeros((rows, 12, ctx), dtype=torch.int64, device="cuda")
        ek = torch.zeros((rows, 12, ctx), dtype=torch.int32, device="cuda")
        v = torch.zeros((rows, 12, ctx, 64), dtype=torch.int32, device="cuda")
        out = torch.zeros((P, rows, 768), dtype=torch.int64, device="cuda")
        q = torch.from_numpy(np.ascontiguousarray(np.stack([Q, Q], axis=1))).cuda()     # [P][rows][2304]
        for p in range(P):
            sm.stages.attend_rows(t, q[p].data_ptr(), rows, k16.data_ptr(), km.data_ptr(), ek.data_ptr(),
                                  v.data_ptr(), p, ctx, out[p].data_ptr())
        A = out.cpu().numpy()
        for r in range(rows):
            got = [h64(row)[:16] for row in A[:, r]]
            bad = [i for i, (x, y) in enumerate(zip(got, case["row_sha16"])) if x != y]
            assert not bad, f"P={P} stream {r}: first differing rows {bad[:5]}"
            assert h64(A[:, r]) == case["out_sha256"]
    t.close()
