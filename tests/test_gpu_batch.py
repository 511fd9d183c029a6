"""GPU parity of the batched streams (several streams decoded in lockstep, every bank an int8 MFMA contraction
over byte planes): the rows product against an exact matrix product, then whole machines stream by stream
against the oracle and base2.py's golden words."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import golden_case
from test_gpu_machine import compare_record, machine_record

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def exact_rows(x, w):
    """x @ w exactly: every partial sum is an integer below 2^53, so float64 products and sums are exact"""
    return (x.astype(np.float64) @ w.astype(np.float64)).astype(np.int64)


def light_rows(rng, nin):
    """64 rows of lights with the edges of the byte split: +32768 (the correction plane), -32768, 32767, 0,
    rows entirely at an extreme, and rows 16-31 free of +32768 (a row tile that needs no correction)"""
    x = rng.integers(-32768, 32769, (64, nin)).astype(np.int64)
    x[0, :4] = [32768, -32768, 32767, 0]
    x[1] = 32768
    x[2] = -32768
    x[3] = 0
    x[4] = 32767
    x[5, ::2] = 32768
    x[16:32] = np.minimum(x[16:32], 32767)
    x[40] = 32768
    return x


ROW_SHAPES = [(768, 2304), (768, 768), (768, 3072), (3072, 768), (768, 1000), (768, 50257)]


@pytest.mark.parametrize("nin,nout", ROW_SHAPES)
def test_rows_product(sm, nin, nout):
    """the MFMA contraction at the GPT-2 shapes (and a vocabulary that is no multiple of 16) for 1..64 rows"""
    rng = np.random.default_rng(3)
    w = rng.integers(-32768, 32768, (nin, nout)).astype(np.int16)
    w[0, :4] = [-32768, 32767, -1, 0]
    w[:, 1] = -32768                    # a column entirely at the negative extreme
    w[:, 2] = 32767
    e = rng.integers(-16, -7, nout).astype(np.int32)
    b = np.zeros(nout, np.int64)
    x = light_rows(rng, nin)
    want = exact_rows(x, w)
    plate = sm.Plate(w, e, b, tile_cols=0)
    assert plate.bytes == ((nout + 15) // 16) * 16 * nin * 2
    dx = dev(x)
    for rows in (64, 1, 2, 17, 33, 16, 40):     # 16 and 17: the row-tile boundary; then fewer rows than before
        dp = torch.full((rows, nout), -7, dtype=torch.int64, device="cuda")
        plate.product_rows(dx.data_ptr(), rows, dp.data_ptr())
        assert np.array_equal(host(dp), want[:rows]), f"rows={rows}"
    plate.close()


def producer_rows(rng, rows, nin, nparts):
    """int64 rows as a producing phase leaves them, each with its own water level (shift 0 .. 40), lights at the
    byte split's edges after the shift (values that round up to +32768, down to -32768, to 32767), planted at
    different k so that different waves' steps hold them, and the OR words of the rows' nparts equal parts"""
    shifts = [1, 0, 7, 20, 40, 3, 12]
    X = np.zeros((rows, nin), np.int64)
    for r in range(rows):
        sh = shifts[r % len(shifts)]
        top = 1 << (15 + sh)                          # |x| < top: the water level stays at sh
        X[r] = rng.integers(-(top - 1), top, nin, dtype=np.int64)
        if sh >= 1 and not 16 <= r < 32:
            half = 1 << (sh - 1)
            k = (r * 97) % nin
            X[r, k] = top - half                      # +32768
            X[r, (k + 1) % nin] = -top + half - 1     # -32768
            X[r, (k + nin // 2) % nin] = top - half   # +32768 in another wave's steps
            X[r, (k + 5) % nin] = top - 3 * half      # 32767
    parts = np.abs(X).reshape(rows, nparts, nin // nparts)
    orw = np.bitwise_or.reduce(parts, axis=2).astype(np.int64)
    return X, orw


@pytest.fixture(scope="module")
def orc(sm):
    import oracle
    return oracle.Stages(sm.tables())


@pytest.mark.parametrize("nin,nout", [(768, 768), (768, 2304), (3072, 768)])
def test_rows_product_from_producer_rows(sm, orc, nin, nout):
    """the light formed inside the bank (the machine's proj and mproj) from int64 rows and their OR words: the
    piles equal the exact product of the oracle's lights, +32768 corrections included, for 1..64 rows"""
    rng = np.random.default_rng(11)
    w = rng.integers(-32768, 32768, (nin, nout)).astype(np.int16)
    w[:, 1] = -32768
    w[:, 2] = 32767
    e = rng.integers(-16, -7, nout).astype(np.int32)
    b = np.zeros(nout, np.int64)
    nparts = 12 if nin == 768 else 192
    X, orw = producer_rows(rng, 64, nin, nparts)
    x16, _ = orc.to16(X)
    assert (x16 == 32768).any(axis=1).sum() >= 30 and (x16 == -32768).any()
    want = exact_rows(x16, w)
    plate = sm.Plate(w, e, b, tile_cols=0)
    dX, dorw = dev(X), dev(orw)
    for rows in (64, 1, 17, 40):
        dp = torch.full((rows, nout), -7, dtype=torch.int64, device="cuda")
        plate.product_rows_from(dX.data_ptr(), dorw.data_ptr(), rows, dp.data_ptr())
        assert np.array_equal(host(dp), want[:rows]), f"rows={rows}"
    plate.close()


def test_rows_product_rejects(sm):
    w = np.zeros((768, 32), np.int16)
    e = np.zeros(32, np.int32)
    b = np.zeros(32, np.int64)
    rows_plate, gemv_plate = sm.Plate(w, e, b, tile_cols=0), sm.Plate(w, e, b, tile_cols=2)
    x = torch.zeros((65, 768), dtype=torch.int64, device="cuda")
    p = torch.zeros((65, 32), dtype=torch.int64, device="cuda")
    for plate, rows in ((rows_plate, 65), (rows_plate, 0), (gemv_plate, 1)):
        with pytest.raises(sm.SmError) as err:
            plate.product_rows(x.data_ptr(), rows, p.data_ptr())
        assert err.value.code == -1
    with pytest.raises(sm.SmError):
        rows_plate.product(x.data_ptr(), p.data_ptr())
    for plate, rows in ((rows_plate, 65), (rows_plate, 0), (gemv_plate, 1)):
        with pytest.raises(sm.SmError) as err:
            plate.product_rows_from(x.data_ptr(), x.data_ptr(), rows, p.data_ptr())
        assert err.value.code == -1
    rows_plate.close()
    gemv_plate.close()


@pytest.mark.parametrize("B", [3, 20])
def test_small_model_streams(sm, small_dir, small_oracle, B):
    """B streams of the small model (one and two row tiles), every stream's words equal the oracle's"""
    prompts = [sm.prompt_ids(50 + b, 8, 1000) for b in range(B)]
    prompts[B - 1] = prompts[0]                     # two streams with one prompt give one answer
    m = sm.Machine(small_dir, max_ctx=64, max_streams=B)
    got = m.streams(prompts, 10)
    m.close()
    assert got[B - 1] == got[0]
    for b in range(B):
        assert got[b] == small_oracle.generate(prompts[b], 10, 64), f"stream {b}"


@pytest.mark.parametrize("kw", [dict(graph_steps=3), dict(graph_steps=1), dict(use_graph=False), {}],
                         ids=["graphs_of_3", "graphs_of_1", "plain", "graphs_of_16"])
def test_small_model_position_slots(sm, small_dir, small_oracle, kw):
    """the batched step reads the position from one of two slots and its race writes the next position into the
    other: graphs of an odd number of steps are replayed from either slot, words asked for in several calls
    continue where the last call stopped (each call checks the device position), and a reset starts over"""
    B = 3
    prompts = [sm.prompt_ids(60 + b, 5, 1000) for b in range(B)]
    want = [small_oracle.generate(p, 19, 64) for p in prompts]
    m = sm.Machine(small_dir, max_ctx=64, max_streams=B, **kw)
    for _ in range(2):
        m.reset()
        for b, p in enumerate(prompts):
            m.prefill(p, b)
        got = np.concatenate([m.generate(n) for n in (4, 1, 7, 3, 4)], axis=1)
        for b in range(B):
            assert [int(w) for w in got[b]] == want[b], f"stream {b}"
    m.close()


@pytest.mark.parametrize("use_graph", [True, False])
def test_small_model_batched_record(sm, small_dir, golden, use_graph):
    """stream 0 of a batch keeps base2.py's record: every intermediate of the last position"""
    c = golden_case(golden, "small_p8_w8")
    last = c["records"]["last"]
    m = sm.Machine(small_dir, max_ctx=64, max_streams=5, use_graph=use_graph)
    m.reset()
    m.record_at(last["position"])
    prompts = [c["prompt"]] + [sm.prompt_ids(70 + b, len(c["prompt"]), 1000) for b in range(4)]
    for b, p in enumerate(prompts):
        m.prefill(p, b)
    words = m.generate(len(c["words"]))
    assert [int(w) for w in words[0]] == c["words"]
    compare_record(machine_record(m), last)
    m.close()


@pytest.fixture(scope="module")
def batch_machine(sm, full_dir):
    m = sm.Machine(full_dir, max_ctx=160, max_streams=64)
    yield m
    m.close()


def test_gpt2_64_streams_two_golden_streams(sm, full_dir, golden):
    """the batched machine's two golden streams of the 64-stream workload, decoded together"""
    cs = [golden_case(golden, f"c4_stream{s}_p32_w4") for s in (0, 1)]
    m = sm.Machine(full_dir, max_ctx=160, max_streams=2)
    assert m.streams([c["prompt"] for c in cs], 4) == [c["words"] for c in cs]
    m.close()


def test_gpt2_64_streams_32_token_prompts(sm, batch_machine, full_oracle, golden):
    """64 streams with 32-word prompts: the golden streams and a sample of the rest against the oracle, and the
    KV cache of a late stream"""
    cs = [golden_case(golden, f"c4_stream{s}_p32_w4") for s in (0, 1)]
    prompts = [cs[0]["prompt"], cs[1]["prompt"]] + [sm.prompt_ids(200 + b, 32) for b in range(2, 64)]
    m = batch_machine
    got = m.streams(prompts, 4)
    assert got[0] == cs[0]["words"] and got[1] == cs[1]["words"]
    for b in (2, 17, 47, 63):
        assert got[b] == full_oracle.generate(prompts[b], 4, 64), f"stream {b}"
    s = full_oracle.session(64)
    seq = prompts[63] + got[63]
    for t in seq[:-1]:
        s.step(t, want_head=False)
    for l in (0, 11):
        for p in (0, 31, len(seq) - 2):
            k16, ek, v = s.read_kv(l, p)
            assert np.array_equal(m.read("k16", l, 63, p), k16)
            assert np.array_equal(m.read("ek", l, 63, p), ek)
            assert np.array_equal(m.read("v", l, 63, p), v)


def test_batched_continuation_and_errors(sm, batch_machine, full_oracle):
    m = batch_machine
    prompts = [sm.prompt_ids(300 + b, 6) for b in range(64)]
    m.reset()
    for b, p in enumerate(prompts):
        m.prefill(p, b)
    a = m.generate(2)
    c = m.generate(3)                               # continues where it stopped
    assert [int(w) for w in a[9]] + [int(w) for w in c[9]] == full_oracle.generate(prompts[9], 5, 16)
    m.reset()
    m.prefill(prompts[0], 0)
    with pytest.raises(sm.SmError) as e:
        m.generate(1)                               # the other 63 streams have no prompt
    assert e.value.code == -7
    m.reset()
    for b in range(64):
        m.prefill(prompts[b][: 5 if b == 7 else 6], b)
    with pytest.raises(sm.SmError) as e:
        m.generate(1)                               # prompts of different lengths
    assert e.value.code == -7


def test_stream_on_a_multi_stream_machine(sm, small_dir, small_oracle):
    """Machine.stream(prompt, n, stream=k) on a three-stream machine: every stream takes the prompt, row k's words"""
    prompt = sm.prompt_ids(21, 8, 1000)
    m = sm.Machine(small_dir, max_ctx=64, max_streams=3)
    want = small_oracle.generate(prompt, 5)
    assert m.stream(prompt, 5, stream=2) == want
    assert m.stream(prompt, 5) == want
    with pytest.raises(sm.SmError):
        m.stream(prompt, 5, stream=3)
    m.close()
