"""The converters and the device-image layout against the reference's own scripts (CPU).

converter_pins.json holds the digests of what base2_convert.py, base2_gpu.py and foundation0/pythia_convert.py
wrote for seeded inputs (tests/golden/make_converter_pins.py ran them in the build container): every array of
their npz files and every file of the base2_gpu/ directory.  convert(), layout() and convert_pythia() must give
the same bytes on the same seeded inputs.
"""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import pytest

from conftest import REPO


@pytest.fixture(scope="module")
def pins():
    with open(os.path.join(REPO, "tests", "golden", "converter_pins.json")) as f:
        return json.load(f)


def _diff(got: dict, want: dict):
    return sorted(k for k in set(got) | set(want) if got.get(k) != want.get(k))


def test_convert_small_matches_base2_convert(sm, pins, small_npz):
    p = pins["gpt2_small"]
    assert p["recipe"] == dict(seed=0, vocab=1000, n_ctx=64)
    assert _diff(sm.array_digest(small_npz), p["npz_digest"]) == []


def test_convert_124m_matches_base2_convert(sm, pins, full_npz):
    assert _diff(sm.array_digest(full_npz), pins["gpt2_124m"]["npz_digest"]) == []


@pytest.mark.parametrize("which", ["gpt2_small", "gpt2_124m"])
def test_layout_matches_base2_gpu(sm, pins, small_npz, full_npz, which, tmp_path):
    npz = small_npz if which == "gpt2_small" else full_npz
    d = sm.layout(npz, str(tmp_path / "base2_gpu"))
    files = {f: hashlib.sha256(open(os.path.join(d, f), "rb").read()).hexdigest() for f in sorted(os.listdir(d))}
    want = pins[which]["layout_files"]
    # every file base2_gpu.py writes, byte for byte; the manifest by content (its JSON spacing is the writer's)
    assert _diff({k: v for k, v in files.items() if k != "manifest.json"},
                 {k: v for k, v in want.items() if k != "manifest.json"}) == []
    with open(os.path.join(d, "manifest.json")) as f:
        assert json.load(f) == pins[which]["layout_manifest"]


def test_convert_pythia_matches_pythia_convert(sm, pins):
    p = pins["pythia_160m"]
    fin, cfg = sm.pythia.random_pythia(seed=p["recipe"]["finished_seed"], vocab=p["recipe"]["vocab"])
    start, _ = sm.pythia.random_pythia(seed=p["recipe"]["start_seed"], vocab=p["recipe"]["vocab"])
    npz = sm.pythia.convert_pythia(fin, cfg, start=start)
    assert p["start_sets_power"] > 0              # the pin exercises the shared power of two
    assert _diff(sm.array_digest(npz), p["npz_digest"]) == []


def test_shared_power_is_set_by_the_larger_checkpoint(sm):
    """pythia_convert.py's shared16: one power of two per neuron for both checkpoints, from the larger maximum"""
    fin = np.array([[1.0, -3.0], [0.5, 1.0]])      # column maxima 1.0 and 3.0
    start = np.array([[4.0, 1.0], [0.0, -1.0]])    # column maxima 4.0 and 1.0
    q, qs, e = sm.pythia.q16(fin, 0, start)
    # column 0: the start's 4.0 sets the power (2^-13 holds 4.0 as 32768 > 32767, so 2^-12); column 1: 3.0
    assert list(e) == [int(np.ceil(np.log2(4.0 / 32767))), int(np.ceil(np.log2(3.0 / 32767)))]
    assert np.array_equal(q.astype(np.int64) * 2.0 ** e[None, :], np.round(fin / 2.0 ** e[None, :]) * 2.0 ** e[None, :])
    assert np.abs(qs).max() <= 32767 and qs[0, 0] == 4.0 / 2.0 ** e[0]
    q1, _, e1 = sm.pythia.q16(fin, 0)               # the finished checkpoint alone sits one place finer on column 0
    assert e1[0] == e[0] - 2 and e1[1] == e[1]
