"""The oracle against base2.py's own golden vectors (tests/golden/base2_golden.json): the converted model's
fingerprint, greedy words, every intermediate of recorded positions, attention at 128-1024 positions, and the
KV-cached step against the full recompute."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden_case, h64, synth_qkv

BANKS = ("qkv", "proj", "fc", "mproj")
NIN = (768, 768, 768, 3072)
NOUT = (2304, 768, 3072, 768)


def oracle_record_keys(rec) -> dict:
    out = {}
    for l in range(12):
        for k, b in enumerate(BANKS):
            out[f"x16.{b}.{l}"] = h64(rec["x16"][l, k, :NIN[k]])
            out[f"pile.{b}.{l}"] = h64(rec["pile"][l, k, :NOUT[k]])
            out[f"ex.{b}.{l}"] = int(rec["ex"][l, k])
            if b in ("qkv", "fc"):
                out[f"ls.{b}.{l}"] = int(rec["ls"][l, k])
        out[f"out.qkv.{l}"] = h64(rec["qkv"][l])
        out[f"att.{l}"] = h64(rec["att"][l])
        out[f"hid.{l}"] = h64(rec["hid"][l])
        out[f"resid_attn.{l}"] = h64(rec["resid"][l, 0])
        out[f"resid_mlp.{l}"] = h64(rec["resid"][l, 1])
        out[f"out.mproj.{l}"] = h64(rec["resid"][l, 1] - rec["resid"][l, 0])
        if l:
            out[f"out.proj.{l}"] = h64(rec["resid"][l, 0] - rec["resid"][l - 1, 1])
    out["x16.head"] = h64(rec["head_x16"])
    out["ex.head"], out["ls.head"] = int(rec["head_ex"][0]), int(rec["head_ls"][0])
    out["pile.head"] = h64(rec["head_pile"])
    out["logits"] = h64(rec["logits"])
    return out


def run_recorded(orc, case, which):
    import oracle
    want = case["records"][which]
    s = orc.session(len(case["prompt"]) + len(case["words"]))
    seq = case["prompt"] + case["words"]
    rec, words = None, []
    for i, t in enumerate(seq[:-1]):
        r = oracle.new_record(orc.vocab) if i == want["position"] else None
        w = s.step(t, want_head=i >= len(case["prompt"]) - 1, rec=r)
        if i >= len(case["prompt"]) - 1:
            words.append(w)
        rec = r if r is not None else rec
    return words, oracle_record_keys(rec), want


def test_small_model_fingerprint(sm, small_npz, golden):
    assert sm.array_digest(small_npz) == golden["models"]["gpt2_small"]["digest"]


def test_full_model_fingerprint(sm, full_npz, golden):
    assert sm.array_digest(full_npz) == golden["models"]["gpt2_124m"]["digest"]


def test_small_words_and_record(small_oracle, golden):
    c = golden_case(golden, "small_p8_w8")
    assert small_oracle.generate(c["prompt"], len(c["words"])) == c["words"]
    for which in c["records"]:
        words, got, want = run_recorded(small_oracle, c, which)
        assert words == c["words"]
        keys = [k for k in want if k in got]
        assert len(keys) > 250
        assert [k for k in keys if got[k] != want[k]] == []


def test_small_full_recompute_words(small_oracle, golden):
    c = golden_case(golden, "small_p8_w8")
    got = []
    for _ in range(len(c["words"])):
        got.append(small_oracle.forward(c["prompt"] + got))
    assert got == c["words"]


def test_numpy_port_words(small_npz, golden):
    from oracle.base2_np import Base2Numpy
    c = golden_case(golden, "small_p8_w8")
    assert Base2Numpy(small_npz).generate(c["prompt"], 4) == c["words"][:4]


def test_batch1_8_token_prompt_words_and_records(full_oracle, golden):
    c = golden_case(golden, "c1_p8_w16")
    for which in ("first", "last"):
        words, got, want = run_recorded(full_oracle, c, which)
        assert words == c["words"]
        keys = [k for k in want if k in got]
        assert len(keys) > 250
        assert [k for k in keys if got[k] != want[k]] == []


@pytest.mark.parametrize("stream", [0, 1])
def test_gpt2_32_token_prompt_words(full_oracle, golden, stream):
    c = golden_case(golden, f"c4_stream{stream}_p32_w4")
    assert full_oracle.generate(c["prompt"], len(c["words"])) == c["words"]


def test_attention_golden(full_oracle, golden):
    for case in golden["attention"]:
        A = full_oracle.attention(synth_qkv(case["seed"], case["P"], case["std"]))
        assert [h64(r)[:16] for r in A] == case["row_sha16"]
        assert h64(A) == case["out_sha256"] and [int(v) for v in A[-1]] == case["last_row"]


def test_kv_step_equals_full_recompute(small_oracle, sm):
    for seed in (20, 21, 22):
        prompt = sm.prompt_ids(seed, 3 + seed % 5, 1000)
        kv = small_oracle.generate(prompt, 5)
        full = []
        for _ in range(5):
            full.append(small_oracle.forward(prompt + full))
        assert kv == full


def test_attention_over_a_cache(full_oracle, golden, sm):
    """the oracle's attention of the newest row over a given cache (the device attention's contract): a cache
    filled from the golden QKV rows (each head's k through to16, v raw) gives base2.py's own rows at several
    positions, and a cache with one value changed does not (it is read)"""
    import oracle
    st = oracle.Stages(sm.tables())
    case = golden["attention"][0]
    Q = synth_qkv(case["seed"], case["P"], case["std"])
    P = len(Q)
    k16 = np.zeros((12, P, 64), np.int64)
    ek = np.zeros((12, P), np.int64)
    v = np.zeros((12, P, 64), np.int64)
    for h in range(12):
        x16, ex = st.to16(Q[:, 768 + 64 * h: 768 + 64 * h + 64])
        k16[h], ek[h] = x16, ex
        v[h] = Q[:, 1536 + 64 * h: 1536 + 64 * h + 64]
    for p in (0, 1, 63, 64, P - 1):
        got = full_oracle.attend_cached(Q[p], k16, ek, v, p)
        assert h64(got)[:16] == case["row_sha16"][p], p
    v[3, 10, 5] += 1 << 14
    assert h64(full_oracle.attend_cached(Q[P - 1], k16, ek, v, P - 1))[:16] != case["row_sha16"][P - 1]


def test_bound_switch_keeps_the_exact_integers(sm, small_npz):
    """past base2.py's 2^52 exactness bound (here: one head's values planted past 2^33) the oracle reports the bound;
    with bound=False its KV-cached steps give the exact int64 result instead, the same as with the bound where the
    bound holds"""
    import oracle
    prompt = sm.prompt_ids(60, 8, 1000)
    assert oracle.Oracle(small_npz, bound=False).generate(prompt, 6, 64) == oracle.Oracle(small_npz).generate(prompt, 6, 64)
    npz = dict(small_npz)
    b = npz["qkv.0.b"].copy()
    b[1536:1600] += np.arange(64, dtype=np.int64) * (1 << 26) + (1 << 33)
    npz["qkv.0.b"] = b
    with pytest.raises(ArithmeticError):
        oracle.Oracle(npz).generate(prompt, 6, 64)
    words = oracle.Oracle(npz, bound=False).generate(prompt, 6, 64)
    assert words != oracle.Oracle(small_npz).generate(prompt, 6, 64)     # the planted head reaches the words
