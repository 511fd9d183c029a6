"""GPU parity of base2.py's stage functions through the C ABI (sm_stage_*, sm_plate_product, sm_stage_attend):
bit-exact against the oracle on seeded random inputs and on the edge values each stage has."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from conftest import REPO, h64, synth_qkv

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.fixture(scope="module")
def tabs(sm):
    return sm.tables()


@pytest.fixture(scope="module")
def dtabs_obj(sm, tabs):
    return sm.Tables(tabs)


@pytest.fixture(scope="module")
def dtabs(dtabs_obj):
    """the device tables (every stage reads its entries from memory)"""
    return dtabs_obj


def test_tables_verified_against_their_formulas(dtabs_obj):
    """every loaded entry equals its defining formula evaluated on the device"""
    assert dtabs_obj.verified() is True


@pytest.mark.parametrize("name,at", [("exp2", 12345), ("log2", 0), ("log2", 65535)])
def test_tampered_table_is_found(sm, tabs, name, at):
    """one changed entry: the device check finds it (the stages still read what was loaded)"""
    bad = dict(tabs)
    bad[name] = tabs[name].copy()
    bad[name][at] += 1
    t = sm.Tables(bad)
    assert t.verified() is False
    t.close()


@pytest.fixture(scope="module")
def orc(tabs):
    import oracle
    return oracle.Stages(tabs)


def edge_values():
    v = [0, 1, -1, 2, -2, 3, -3, 32767, -32768, 32768, -32769, 65535, -65535, 65536, 2 ** 31 - 1, -2 ** 31,
         2 ** 40 + 12345, -(2 ** 40) - 99, 2 ** 62, -(2 ** 62), 2 ** 63 - 1, -(2 ** 63)]
    return np.array(v, dtype=np.int64)


def test_rshift(sm, orc):
    rng = np.random.default_rng(10)
    x = np.concatenate([rng.integers(-2 ** 40, 2 ** 40, 20000), np.repeat(edge_values(), 9)])
    s = np.concatenate([rng.integers(-20, 70, 20000), np.tile(np.array([-70, -64, -63, -1, 0, 1, 15, 63, 64], np.int64), len(edge_values()))])
    dx, ds, do = dev(x), dev(s), torch.empty(len(x), dtype=torch.int64, device="cuda")
    sm.stages.rshift(dx.data_ptr(), ds.data_ptr(), do.data_ptr(), len(x))
    assert np.array_equal(host(do), orc.rshift(x, s))


def test_log2fix(sm, orc, dtabs):
    rng = np.random.default_rng(11)
    v = np.concatenate([rng.integers(1, 2 ** 62, 20000), 2 ** rng.integers(0, 62, 500), rng.integers(1, 70000, 3000),
                        np.array([1, 2, 3, 65535, 65536, 65537, 2 ** 62, 2 ** 63 - 1, 0, -5, -(2 ** 63)], np.int64)])
    dv, do = dev(v), torch.empty(len(v), dtype=torch.int64, device="cuda")
    sm.stages.log2fix(dtabs, dv.data_ptr(), do.data_ptr(), len(v))
    assert np.array_equal(host(do), orc.log2fix(v))


def test_power(sm, orc, dtabs):
    rng = np.random.default_rng(12)
    n = 30000
    x = np.concatenate([rng.integers(-2 ** 45, 2 ** 45, n), rng.integers(-2 ** 62, 2 ** 62, 2000)])   # the second part wraps
    F = np.concatenate([rng.integers(-40 * 65536, 20 * 65536, n), rng.integers(-70 * 65536, 70 * 65536, 2000)])
    dx, dF, do = dev(x), dev(F), torch.empty(len(x), dtype=torch.int64, device="cuda")
    sm.stages.power(dtabs, dx.data_ptr(), dF.data_ptr(), do.data_ptr(), len(x))
    assert np.array_equal(host(do), orc.power(x, F))


def test_edge(sm, orc, dtabs):
    rng = np.random.default_rng(13)
    h = np.concatenate([rng.integers(-2 ** 20, 2 ** 20, 30000), np.arange(-(2 ** 19) - 40, -(2 ** 19) + 40),
                        np.arange(2 ** 19 - 40, 2 ** 19 + 40), edge_values()[:-2]])
    dh, do = dev(h), torch.empty(len(h), dtype=torch.int64, device="cuda")
    sm.stages.edge(dtabs, dh.data_ptr(), do.data_ptr(), len(h))
    assert np.array_equal(host(do), orc.edge(h))


@pytest.mark.parametrize("n", [64, 768, 3072])
def test_to16(sm, orc, n):
    rng = np.random.default_rng(14 + n)
    X = rng.integers(-2 ** 30, 2 ** 30, (40, n)) >> rng.integers(0, 30, (40, 1))
    X[3] = 0
    X[4, 5] = 65535                    # rounds up to +32768 after the shift
    X[5] = rng.integers(-32767, 32768, n)
    dX = dev(X)
    dx16 = torch.empty_like(dX)
    dex = torch.empty(len(X), dtype=torch.int64, device="cuda")
    sm.stages.to16(dX.data_ptr(), len(X), n, dx16.data_ptr(), dex.data_ptr())
    x16, ex = orc.to16(X)
    assert np.array_equal(host(dx16), x16) and np.array_equal(host(dex), ex)
    assert host(dx16).max() <= 32768


def test_gauge_log(sm, orc, dtabs):
    rng = np.random.default_rng(15)
    R = (rng.standard_normal((64, 768)) * rng.choice([100.0, 3000.0, 2.0 ** 20], (64, 1))).astype(np.int64)
    R[0] = 7                           # a flat row: the variance is the eps term alone
    dR = dev(R)
    dx16 = torch.empty_like(dR)
    dex = torch.empty(len(R), dtype=torch.int64, device="cuda")
    dls = torch.empty(len(R), dtype=torch.int64, device="cuda")
    sm.stages.gauge_log(dtabs, dR.data_ptr(), len(R), dx16.data_ptr(), dex.data_ptr(), dls.data_ptr())
    x16, ex, LS = orc.gauge_log(R)
    assert np.array_equal(host(dx16), x16) and np.array_equal(host(dex), ex) and np.array_equal(host(dls), LS)


@pytest.mark.parametrize("n", [1, 5, 50257, 300000])
def test_race(sm, orc, n):
    rng = np.random.default_rng(16 + n)
    v = rng.integers(-1000, 1000, n)
    if n > 10:
        v[[7, n - 3, n // 2]] = 5000    # ties: the lowest index wins
    dv, do = dev(v), torch.zeros(1, dtype=torch.int64, device="cuda")
    sm.stages.race(dv.data_ptr(), n, do.data_ptr())
    assert int(host(do)[0]) == orc.race(v) == int(np.argmax(v))


SHAPES = [(768, 2304, 2), (768, 768, 2), (768, 3072, 2), (3072, 768, 1), (768, 50257, 8), (768, 50257, 4), (3072, 768, 2),
          (768, 2304, 8)]


@pytest.mark.parametrize("nin,nout,tc", SHAPES)
def test_plate_product(sm, nin, nout, tc):
    """The integer GEMV at GPT-2 shapes: uniform int16 weights (both extremes), uniform lights with the
    +-32768 edge values, exact against an int64 matrix product."""
    rng = np.random.default_rng(2)
    w = rng.integers(-32768, 32768, (nin, nout)).astype(np.int16)
    e = rng.integers(-16, -7, nout).astype(np.int32)
    b = np.zeros(nout, np.int64)
    x = rng.integers(-32768, 32768, nin).astype(np.int64)
    x[:4] = [32768, -32768, 32767, 0]
    w[0, :3] = [-32768, 32767, -1]
    plate = sm.Plate(w, e, b, tile_cols=tc)
    dx = dev(x)
    dp = torch.empty(nout, dtype=torch.int64, device="cuda")
    plate.product(dx.data_ptr(), dp.data_ptr())
    want = x @ w.astype(np.int64)
    assert np.array_equal(host(dp), want)
    plate.product(dx.data_ptr(), dp.data_ptr(), grid=37)     # fewer blocks than tiles: the tile loop
    assert np.array_equal(host(dp), want)
    plate.close()


ATTEND = ["attend", "attend_split"]       # one block a head; spread over chunks of 64 positions


def _attend_all(sm, dtabs, QKV, ctx, fn="attend"):
    """run the device attention (stage entry point `fn`) position by position over QKV rows (the cache fills as it
    goes)"""
    P = len(QKV)
    k16 = torch.zeros((ctx, 768), dtype=torch.int16, device="cuda")
    km = torch.zeros((ctx, 12), dtype=torch.int64, device="cuda")
    ek = torch.zeros((ctx, 12), dtype=torch.int32, device="cuda")
    v = torch.zeros((ctx, 768), dtype=torch.int32, device="cuda")
    dq = dev(QKV)
    out = torch.zeros((P, 768), dtype=torch.int64, device="cuda")
    f = getattr(sm.stages, fn)
    for p in range(P):
        f(dtabs, dq[p].data_ptr(), k16.data_ptr(), km.data_ptr(), ek.data_ptr(), v.data_ptr(), p, ctx, out[p].data_ptr())
    return host(out)


@pytest.mark.parametrize("fn", ATTEND)
def test_attention_golden(sm, dtabs, golden, fn):
    """the attention workload's shapes (T = 128, 512, 1024): every row against base2.py's own attention (golden
    vectors), through the one-block kernel and through the kernels spread over chunks of positions"""
    for case in golden["attention"]:
        Q = synth_qkv(case["seed"], case["P"], case["std"])
        A = _attend_all(sm, dtabs, Q, 1024, fn)
        rows = [h64(r)[:16] for r in A]
        bad = [i for i, (a, b) in enumerate(zip(rows, case["row_sha16"])) if a != b]
        assert not bad, f"P={case['P']}: first differing row {bad[:5]}"
        assert h64(A) == case["out_sha256"]


@pytest.mark.parametrize("fn", ATTEND)
def test_attention_extreme_keys(sm, dtabs, small_oracle, fn):
    """keys at the ends of the 16-bit range, +32768 (held as 32767 with its mask bit) and -32768, in the
    short path (p < 64), the general one and the long-context ring (p >= 128), against the oracle; spread over
    chunks: one to four chunks, the new position first, inside and last in its chunk"""
    rng = np.random.default_rng(21)
    P = 200
    Q = np.round(rng.standard_normal((P, 2304)) * 0.5 * 65536).astype(np.int64)
    for p in range(0, P, 3):
        for h in range(0, 12, 1 + p % 4):
            k = Q[p, 768 + 64 * h: 768 + 64 * h + 64]
            k[:] = rng.integers(-2 ** 19, 2 ** 19, 64)
            k[(p + h) % 64] = 2 ** 21 - 1               # to16 (shift 6): +32768
            k[(p + 3 * h + 1) % 64] = 1 - 2 ** 21       # -32768
            if p % 2:
                k[(p + 7) % 64] = 2 ** 21 - 1            # two +32768 in one row
            if p % 5 == 0:
                q = Q[p, 64 * h: 64 * h + 64]          # q at +32768 and -32768 too
                q[:] = rng.integers(-2 ** 19, 2 ** 19, 64)
                q[(p + h) % 64] = 2 ** 21 - 1
                q[(p + 3 * h + 1) % 64] = 1 - 2 ** 21
    want = small_oracle.attention(Q)
    got = _attend_all(sm, dtabs, Q, 256, fn)
    bad = [i for i in range(P) if not np.array_equal(got[i], want[i])]
    assert not bad, f"first differing positions {bad[:5]}"


@pytest.mark.parametrize("fn", ATTEND)
def test_attention_overflow_flag(sm, dtabs, fn):
    """a value past 32 bits cannot enter the int32 V cache: the call reports SM_E_OVERFLOW"""
    Q = np.zeros((1, 2304), np.int64)
    Q[0, 1536] = 2 ** 33
    with pytest.raises(sm.SmError) as ei:
        _attend_all(sm, dtabs, Q, 16, fn)
    assert ei.value.code == -6


@pytest.mark.parametrize("fn", ATTEND)
def test_attention_workload_caches(sm, dtabs, small_oracle, fn):
    """the attention microbenchmark's own inputs (uniform int16 caches at T = 128, 512, 1024, bench.attention_workload):
    both kernels' outputs against the oracle on the same caches and against the committed fixture bench gates on"""
    import hashlib
    import bench
    want = {c["T"]: c for c in json.load(open(os.path.join(REPO, "tests", "golden", "attention_cache.json")))["cases"]}
    f = getattr(sm.stages, fn)
    for T, k16, ek, v, qkv in bench.attention_workload():
        dk, de, dv = dev(k16), dev(ek), dev(v)
        km = torch.zeros((12, T), dtype=torch.int64, device="cuda")
        dq = dev(qkv)
        o = torch.zeros(768, dtype=torch.int64, device="cuda")
        f(dtabs, dq.data_ptr(), dk.data_ptr(), km.data_ptr(), de.data_ptr(), dv.data_ptr(), T - 1, T, o.data_ptr())
        got = host(o)
        assert np.array_equal(got, small_oracle.attend_cached(qkv, k16, ek, v, T - 1)), T
        assert hashlib.sha256(got.tobytes()).hexdigest() == want[T]["out_sha256"], T
