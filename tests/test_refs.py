"""The tools for the reference's real-weight fixtures (streaming-machine_amd/refs.py): FNV-1a 64 against its
specification's published test vectors, the plate hash against a byte-by-byte restatement, the refs_many.json
report on a stand-in machine, and the record hashes of the GPU machine against the oracle's record."""
from __future__ import annotations

import numpy as np
import pytest


def test_fnv1a64_published_vectors(sm):
    # FNV-1a 64-bit test vectors (the FNV specification's test suite)
    assert sm.refs.fnv1a64(b"") == 0xCBF29CE484222325
    assert sm.refs.fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert sm.refs.fnv1a64(b"foobar") == 0x85944171F73967E8


def _bytewise(pile, x16, ex) -> str:
    """the plate hash as base2_stream_fr2.swift:990-993 writes it: mix(v) feeds v's 8 bytes, lowest first"""
    h = 0xCBF29CE484222325

    def mix(v):
        nonlocal h
        for _ in range(8):
            h ^= v & 0xFF
            h = (h * 0x100000001B3) & ((1 << 64) - 1)
            v >>= 8

    for v in pile:
        mix(int(v) & ((1 << 64) - 1))
    for v in x16:
        mix(int(v) & 0xFFFFFFFF)
    mix(int(ex) & 0xFFFFFFFF)
    return format(h, "x")


def test_plate_hash_matches_bytewise(sm):
    rng = np.random.default_rng(9)
    pile = rng.integers(-(2 ** 62), 2 ** 62, 37)
    x16 = rng.integers(-32768, 32769, 23)
    x16[0], x16[1] = 32768, -32768
    assert sm.refs.plate_hash(pile, x16, -17) == _bytewise(pile, x16, -17)
    assert sm.refs.plate_hash(pile, x16, 5) == _bytewise(pile, x16, 5)


class _Stand:
    """a machine stand-in that answers stream() from a table"""

    def __init__(self, answers):
        self.answers = answers

    def stream(self, ids, n):
        return self.answers[tuple(ids)][:n]


def test_run_refs_report(sm):
    refs = [{"prompt": "a", "ids": [1, 2], "ref": [5, 6, 7], "margins": [0.1, 0.2, 0.3]},
            {"prompt": "b", "ids": [3], "ref": [8, 9, 10], "margins": [0.4, 0.5, 0.6]}]
    m = _Stand({(1, 2): [5, 6, 7], (3,): [8, 1, 10]})
    r = sm.refs.run_refs(m, refs)
    assert r["identical"] == 1 and r["prompts"] == 2
    d = r["per_prompt"][1]
    assert d["first_differs_at"] == 2 and d["machine_word"] == 1 and d["model_word"] == 9 and d["model_lead"] == 0.5


@pytest.mark.gpu
def test_rec_hash_matches_the_oracle(sm, small_dir, small_npz, small_oracle):
    """the 48 plate hashes of two new positions from the GPU's record equal those of the oracle's record"""
    from oracle import new_record
    ids, n = sm.prompt_ids(13, 6, 1000), 3
    m = sm.Machine(small_dir, max_ctx=64)
    got = sm.refs.rec_hash(m, ids, n)
    words = m.stream(ids, n)
    m.close()
    assert len(got) == n - 1 and all(len(r) == 48 for r in got)
    seq = ids + words
    want = []
    for q in range(len(ids), len(ids) + n - 1):
        s = small_oracle.session(64)
        rec = new_record(small_oracle.vocab)
        for i in range(q + 1):
            s.step(seq[i], want_head=False, rec=rec if i == q else None)
        want.append(sm.refs.plate_hashes(rec["x16"], rec["ex"], rec["pile"]))
    assert got == want
