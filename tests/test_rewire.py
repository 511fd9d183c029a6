"""The random wiring (base2_stream.swift:161-190, its seed= test): channels, heads, in-head dimensions, neurons
and words shuffled; whole-number sums make every pile the same number in its new place.  CPU: the oracle's words
and piles under the wiring equal the plain machine's.  GPU: the same on the device, for both launch paths."""
from __future__ import annotations

import numpy as np
import pytest


def _words(orc, perms, ids, n):
    slots = orc.generate([int(perms["slot_of"][t]) for t in ids], n)
    return [int(perms["words"][s]) for s in slots]


def test_oracle_words_and_piles_under_wiring(sm, small_npz, small_oracle):
    import oracle
    wired, perms = sm.rewire(small_npz, seed=3)
    orc = oracle.Oracle(wired)
    ids = sm.prompt_ids(17, 6, 1000)
    assert _words(orc, perms, ids, 5) == small_oracle.generate(ids, 5)
    # the piles of one position, in their new places
    r0, r1 = oracle.new_record(1000), oracle.new_record(1000)
    small_oracle.forward(ids, rec=r0)
    orc.forward([int(perms["slot_of"][t]) for t in ids], rec=r1)
    for l in (0, 7):
        L = perms["layers"][l]
        assert np.array_equal(r1["pile"][l, 0, :2304], r0["pile"][l, 0, L["qkv_cols"]])
        assert np.array_equal(r1["pile"][l, 1, :768], r0["pile"][l, 1, perms["chan"]])
        assert np.array_equal(r1["pile"][l, 2, :3072], r0["pile"][l, 2, L["neurons"]])
        assert np.array_equal(r1["pile"][l, 3, :768], r0["pile"][l, 3, perms["chan"]])
    assert np.array_equal(r1["head_pile"], r0["head_pile"][perms["words"]])


@pytest.mark.gpu
@pytest.mark.parametrize("streams", [1, 3])
def test_device_words_under_wiring(sm, small_npz, small_oracle, tmp_path, streams):
    wired, perms = sm.rewire(small_npz, seed=11)
    d = sm.layout(wired, str(tmp_path / "wired"))
    prompts = [sm.prompt_ids(40 + s, 12, 1000) for s in range(streams)]
    m = sm.Machine(d, max_ctx=64, max_streams=streams)
    got = m.streams([[int(perms["slot_of"][t]) for t in p] for p in prompts], 6)
    m.close()
    assert [[int(perms["words"][s]) for s in row] for row in got] == [small_oracle.generate(p, 6) for p in prompts]
