"""Host logic on the CPU: the converter's numbers (base2_convert.py), the layout directory (base2_gpu.py) and the
benchmark's byte accounting."""
from __future__ import annotations

import importlib.util
import os

import numpy as np

from conftest import REPO


def test_cols16_is_the_smallest_power_holding_each_column(sm):
    rng = np.random.default_rng(0)
    W = rng.standard_normal((300, 200)) * rng.choice([1e-3, 0.02, 3.0], 200)[None, :]
    W[:, 5] = 0.0
    q, e = sm.cols16(W)
    assert q.dtype == np.int16 and np.abs(q.astype(np.int64)).max() <= 32767
    mx = np.abs(q.astype(np.int64)).max(0)
    assert np.all(mx[np.arange(200) != 5] >= 16384)            # one power smaller would not hold the column
    deq = q * np.exp2(e.astype(np.float64))[None, :]
    assert np.all(np.abs(deq - W) <= np.exp2(e.astype(np.float64))[None, :] / 2 + 1e-300)


def test_fold_is_centring_with_the_gain(sm):
    sd = sm.random_gpt2(seed=3, vocab=300, n_ctx=16)
    npz = sm.convert(sd)
    g1 = sd["transformer.h.0.ln_1.weight"].astype(np.float64)
    Wq = sd["transformer.h.0.attn.c_attn.weight"].astype(np.float64)
    C = np.eye(768) - 1.0 / 768
    ref = C @ (g1[:, None] * Wq)                                  # base2_convert.py:36
    deq = npz["qkv.0.w"] * np.exp2(npz["qkv.0.e"].astype(np.float64))[None, :]
    assert np.abs(deq - ref).max() <= np.exp2(npz["qkv.0.e"].astype(np.float64)).max() * 0.5 + 1e-12
    b1, bq = sd["transformer.h.0.ln_1.bias"].astype(np.float64), sd["transformer.h.0.attn.c_attn.bias"].astype(np.float64)
    assert np.abs(npz["qkv.0.b"] - np.round((b1 @ Wq + bq) * 65536)).max() <= 1


def test_layout_round_trip(sm, small_npz, tmp_path):
    d = sm.layout(small_npz, str(tmp_path / "lay"))
    back = sm.load_layout(d)
    for k in ("qkv.3.w", "mproj.11.b", "head.w", "head.e", "wte", "wpe", "phi", "arrival", "log2", "exp2"):
        assert np.array_equal(np.asarray(back[k]), np.asarray(small_npz[k]).astype(np.asarray(back[k]).dtype)), k
    assert int(back["eps40"]) == int(small_npz["eps40"])
    names = sorted(os.listdir(d))
    assert "manifest.json" in names and "qkv.0.wc" in names and "head.b" in names


def test_step_bytes_match_the_published_accounting():
    spec = importlib.util.spec_from_file_location("bench", os.path.join(REPO, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    assert bench.WORKLOAD_FIXED == 248_662_476        # weights + exponents/biases, per token
    assert bench.KV_WORKLOAD == 73_728                # k and v at 4 B each, 12 layers x 768, per cached position
    # what this layout reads per cached position: 12 layers x (768 int16 keys + 768 int32 values + per head an
    # int32 key water level and an int64 mask of the +32768 dimensions)
    assert bench.KV_LAYOUT == 12 * (768 * 6 + 12 * 12) == 57_024
    assert bench.bank_bytes(768, 50257) == 2 * 768 * 50257 + 12 * 50257
    assert sum(bench.b1_kernel_bytes(k, 16) for k in ("qkv", "proj", "fc", "mproj")) * 12 + \
        bench.b1_kernel_bytes("head", 16) + 12 * bench.b1_kernel_bytes("attend", 16) == 248_662_476 + 73_728 * 16