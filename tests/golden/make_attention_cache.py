"""Writes tests/golden/attention_cache.json: the attention workload's expected outputs (12 heads x 64, uniform int16
caches at T = 128, 512, 1024, the new position p = T - 1; bench.attention_workload() draws the inputs), computed by
the oracle's attention over a given cache (oracle.Oracle.attend_cached, pinned against base2.py's own attention rows
by tests/test_oracle_golden.py::test_attention_over_a_cache).  The fixture is the oracle's, labelled so; bench.py
and the GPU tests compare both device attention kernels with it.

    python tests/golden/make_attention_cache.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, REPO)


def main():
    import bench
    import oracle
    sm = bench.load_sm()
    orc = oracle.Oracle(sm.convert(sm.random_gpt2(seed=0, vocab=1000, n_ctx=64)))   # (only its tables are used)
    cases = []
    for T, k16, ek, v, qkv in bench.attention_workload():
        out = orc.attend_cached(qkv, k16.astype(np.int64), ek.astype(np.int64), v.astype(np.int64), T - 1)
        cases.append({"name": f"attention_cache_T{T}", "T": T, "p": T - 1, "source": "oracle (attend_cached)",
                      "out_sha256": hashlib.sha256(np.ascontiguousarray(out, np.int64).tobytes()).hexdigest(),
                      "out_head0": [int(x) for x in out[:64]]})
    with open(os.path.join(REPO, "tests", "golden", "attention_cache.json"), "w") as f:
        json.dump({"note": "expected outputs of the attention workload (bench.attention_workload), written by "
                           "tests/golden/make_attention_cache.py with the oracle", "cases": cases}, f, indent=1)


if __name__ == "__main__":
    main()
