"""The float-stage switches on the GPU (base2.py:10-11 gauge= / edge= / arrival=; foundation0/pythia_base2.py:21-27
gauge= / turn= / edge= / arrival=), against the reference run with the same switches (float_golden.json, written
by executing base2.py and pythia_base2.py).

The switches are diagnostics, compared at the word level (every word of every case is the reference's), and
here also every recorded intermediate of the last position, bit for bit.  For the gauge and the turn that is by
construction: the device performs numpy's own sequence of correctly rounded float64 operations (numpy's pairwise
sums, then division and square root; the turn's cos and sin are numpy's, written into the layout).  For the
edge (tanh, erf, pow from the device library against numpy's and libm's) and the arrival (exp, and this kernel's
summation order against numpy's BLAS) it is measured, not guaranteed: the float64 results can differ in the last
bit, and every stage rounds to a whole number at 2^-16, so a difference shows only when a value falls within
that last bit of a rounding boundary.  A failure of the record check alone, with the words equal, is that case.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from conftest import REPO
import test_gpu_machine as g2rec
import test_gpu_pythia as pyrec

pytestmark = pytest.mark.gpu

PATH = os.path.join(REPO, "tests", "golden", "float_golden.json")
CASES = json.load(open(PATH))["cases"] if os.path.exists(PATH) else []


def _record(m, model):
    if model.startswith("gpt2"):
        return g2rec.machine_record(m)
    got = pyrec.machine_record(m, np.zeros(768, dtype=np.int64))
    for k in ("stream.0", "out.proj.0"):      # need the row entering layer 0, which the device does not record
        got.pop(k)
    return got


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_float_stage_words(sm, small_dir, full_dir, py_small_dir, py_full_dir, case):
    d = dict(gpt2_small=small_dir, gpt2_124m=full_dir, pythia_small=py_small_dir, pythia_160m=py_full_dir)[case["model"]]
    kw = {k: "float" for k in case["float"]}
    m = sm.Machine(d, max_ctx=len(case["prompt"]) + len(case["words"]) + 8, prefill_rows=0, **kw)
    last = case["records"]["last"]
    m.reset()
    m.record_at(last["position"])
    m.prefill(case["prompt"])
    words = [int(w) for w in m.generate(len(case["words"]))[0]]
    got = _record(m, case["model"])
    m.close()
    assert words == case["words"], f"words {words} != the reference's {case['words']}"
    keys = [k for k in last if k in got]
    assert len(keys) > 200
    bad = sorted(k for k in keys if got[k] != last[k])
    assert not bad, f"{len(bad)} of {len(keys)} intermediates differ, first: {bad[:8]}"
