"""Decode benchmark of the integer ("all base 2") GPT-2 124M machine on one MI355X.

Workload (the batch-1 configuration the metric is quoted on): GPT-2 124M shape, random-init N(0, 0.02) weights
from seed 0 converted to int16 plates with per-column powers of two; batch 1; an 8-token prompt drawn from
default_rng(1); 16 greedy words per sequence, i.e. the prompt pass plus 15 decode steps at context 9..23.
A "step" is one decode position (one new word).  The timed region covers exactly --steps decode steps, in
sequences of 15 (each sequence's prompt pass runs untimed first), with the weights, tables and KV cache resident
in HBM.  Before any number is printed the emitted words are checked against the golden words that base2.py
(and pythia_base2.py for the Pythia leg) gave for the same prompts (tests/golden, written by executing the
reference itself); the CPU baseline's own words are checked against the GPU's.

Printed: one JSON line with the driver's fields plus
  roofline      the head kernel (the largest single launch: the 768 x 50257 plate read), its mean
                duration from HIP event pairs recorded around every head launch inside the timed region
  step_roofline the whole decode step's algorithmic bytes over its measured time
  prompt_included  words per second counting the prompt pass (every prompt position but the last through the
                int8 MFMA banks in passes of up to 64 rows, then the first word's step), as the reference also
                reports beside the after-the-prompt rate
  batched       the same machine with 64 streams in lockstep (int8 MFMA contraction), 32-token prompts,
                128 words each (tokens/s over all streams)
  pythia        the Pythia-160m-shaped machine with 32 streams, 64-token prompts, 256 words each
  cpu_baseline  base2.py's CPU path restated in numpy (full recompute per word, float64 products, the
                top-down race loop), timed on a bounded sample of the same sequence on the host cores
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import tempfile
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
METRIC = "decode tokens/s, GPT-2-124M int base-2, B=1 & B=64; % HBM roofline"
HBM_PEAK_GBS = 8000.0
WORDS = 16          # words per sequence (the prompt pass gives the first)
PROMPT = 8
B_STREAMS, B_PROMPT, B_WORDS = 64, 32, 128     # the batched workload: 64 streams, 32-token prompts, 128 words
P_STREAMS, P_PROMPT, P_WORDS = 32, 64, 256     # the Pythia-160m-shaped workload: 32 streams, 64-token prompts, 256 words
PREFILL_ROWS = 64   # prompt rows a pass through the int8 MFMA banks (0: position by position)


def load_sm():
    if "streaming_machine_amd" in sys.modules:
        return sys.modules["streaming_machine_amd"]
    root = os.path.join(REPO, "streaming-machine_amd")
    spec = importlib.util.spec_from_file_location("streaming_machine_amd", os.path.join(root, "__init__.py"),
                                                  submodule_search_locations=[root])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["streaming_machine_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def golden_words(fname: str) -> dict:
    """case name -> words, from the golden fixtures written by executing the reference itself"""
    with open(os.path.join(REPO, "tests", "golden", fname)) as f:
        return {c["name"]: c["words"] for c in json.load(f)["cases"]}


def head_bytes(vocab: int) -> int:
    """algorithmic bytes of one head launch: the int16 plate plus an int32 exponent and an int64 bias per word"""
    return 2 * 768 * vocab + 12 * vocab


# the KV cache read per cached position of a stream: 12 layers x (int16 k16 and int32 v per dimension, and per
# head an int32 key water level and an int64 mask of the key's +32768 dimensions)
KV_BYTES = 12 * (768 * 6 + 12 * 12)


def step_bytes(vocab: int, ctx: float) -> float:
    """algorithmic bytes of one decode step: every plate once (int16), the per-column exponents and biases,
    and the KV cache read at context ctx"""
    layer_w = 2 * (768 * 2304 + 768 * 768 + 768 * 3072 + 3072 * 768)
    layer_cols = 12 * (2304 + 768 + 3072 + 768)
    return 12 * (layer_w + layer_cols) + head_bytes(vocab) + KV_BYTES * ctx


def batched_leg(sm, lay):
    """64 independent streams decoded in lockstep (every bank an int8 MFMA contraction): one sequence of
    32-token prompts and 128 words per stream, KV cache up to 160.  Timed: the 127 decode steps after the
    prompt pass; the head launches are timed with their own event pairs.  Streams 0 and 1 begin with the golden
    words base2.py gives for their prompts."""
    import torch
    if lay is None:
        lay = tempfile.mkdtemp(prefix="sm_bench_")
        sm.layout(sm.convert(sm.random_gpt2(seed=0)), lay)
    prompts = [sm.prompt_ids(4 + b, B_PROMPT) for b in range(B_STREAMS)]     # stream s: default_rng(4 + s)
    gw = golden_words("base2_golden.json")
    want = {b: gw[f"c4_stream{b}_p32_w4"] for b in (0, 1)}
    m = sm.Machine(lay, max_ctx=B_PROMPT + B_WORDS, max_streams=B_STREAMS, graph_steps=B_WORDS - 1, profile=True,
                   prefill_rows=PREFILL_ROWS)
    res = None
    for it in range(2):                     # the first sequence warms up (graph instantiation)
        m.reset()
        torch.cuda.synchronize()
        t = time.perf_counter()
        for b, p in enumerate(prompts):
            m.prefill(p, b)
        first = m.generate(1)               # the prompt pass and the first word
        torch.cuda.synchronize()
        tp = time.perf_counter() - t
        m.profile(clear=True)
        t = time.perf_counter()
        rest = m.generate(B_WORDS - 1)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t
        n, us = m.profile(clear=True)
        words = np.concatenate([first, rest], axis=1)
        for b, w in want.items():
            if [int(x) for x in words[b][:len(w)]] != w:
                raise RuntimeError(f"batched stream {b}: GPU words differ from base2.py's golden words")
        res = (dt, n, us, tp)
    m.close()
    dt, n, us, tp = res
    steps = B_WORDS - 1
    ms = 1000.0 * dt / steps
    hb = head_bytes(m.vocab)
    ach = hb / (us * 1e-6) / 1e9
    # int8 MFMA work of one head launch: 4 byte-plane products of 64 x 768 x vocab (2 ops per multiply-add)
    ops = 4 * 2 * B_STREAMS * 768 * m.vocab
    ctx_mean = B_PROMPT + B_WORDS / 2.0
    sb = step_bytes(m.vocab, 0) + B_STREAMS * KV_BYTES * ctx_mean
    return {"streams": B_STREAMS, "value": round(B_STREAMS * steps / dt, 1), "unit": "tokens/s",
            "ms_per_step": round(ms, 4), "steps": steps,
            "workload": f"{B_STREAMS} streams, {B_PROMPT}-token random prompts, {B_WORDS} greedy words each "
                        f"(context to {B_PROMPT + B_WORDS}); streams 0 and 1 checked against base2.py's golden words",
            "prompt_included": {"value": round(B_STREAMS * B_WORDS / (tp + dt), 1), "unit": "tokens/s",
                                "prompt_ms": round(1000.0 * tp, 3)},
            "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "kernel": "k_head_rows<4,EPI_HEAD>",
                         "mean_launch_us": round(us, 3), "launches_timed": n,
                         "int8_tops": round(ops / (us * 1e-6) / 1e12, 1), "int8_frac": round(ops / (us * 1e-6) / 5.0e15, 4)},
            "step_roofline": {"bytes_per_step": int(sb), "achieved": round(sb / (ms * 1e-3) / 1e9, 1),
                              "frac": round(sb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}}


def pythia_leg(sm):
    """The Pythia-160m-shaped machine (random N(0, 0.02) weights from default_rng(5), vocab 50304, rotary on a
    quarter of each head, parallel residual): 32 streams decoded in lockstep, 64-token prompts (stream s:
    default_rng(5 + s)), 256 greedy words each, context to 320.  Timed: the 255 decode steps after the prompt
    pass.  Streams 0 and 1 begin with the golden words pythia_base2.py gives for their prompts."""
    import torch
    t0 = time.time()
    sd, cfg = sm.pythia.random_pythia(seed=5)
    npz = sm.pythia.convert_pythia(sd, cfg)
    del sd
    lay = tempfile.mkdtemp(prefix="sm_bench_py_")
    sm.pythia.pythia_layout(npz, lay)
    prompts = [sm.prompt_ids(5 + b, P_PROMPT, 50304) for b in range(P_STREAMS)]
    gw = golden_words("pythia_golden.json")
    want = {b: gw[f"py_c5_stream{b}_p64_w4"] for b in (0, 1)}
    del npz
    log(f"pythia: model converted and laid out in {time.time() - t0:.1f}s")
    m = sm.Machine(lay, max_ctx=P_PROMPT + P_WORDS, max_streams=P_STREAMS, graph_steps=P_WORDS - 1, profile=True,
                   prefill_rows=PREFILL_ROWS)
    res = None
    for it in range(2):                     # the first sequence warms up (graph instantiation)
        m.reset()
        torch.cuda.synchronize()
        t = time.perf_counter()
        for b, p in enumerate(prompts):
            m.prefill(p, b)
        first = m.generate(1)               # the prompt pass and the first word
        torch.cuda.synchronize()
        tp = time.perf_counter() - t
        m.profile(clear=True)
        t = time.perf_counter()
        rest = m.generate(P_WORDS - 1)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t
        n, us = m.profile(clear=True)
        words = np.concatenate([first, rest], axis=1)
        for b, w in want.items():
            if [int(x) for x in words[b][:len(w)]] != w:
                raise RuntimeError(f"pythia stream {b}: GPU words differ from pythia_base2.py's golden words")
        res = (dt, n, us, tp)
    vocab = m.vocab
    m.close()
    dt, n, us, tp = res
    steps = P_WORDS - 1
    ms = 1000.0 * dt / steps
    hb = head_bytes(vocab) - 8 * vocab                 # no bias on Pythia's head
    ctx_mean = P_PROMPT + P_WORDS / 2.0
    layer_w = 12 * (2 * (768 * 2304 + 768 * 768 + 768 * 3072 + 3072 * 768) + 12 * (2304 + 768 + 3072 + 768))
    sb = layer_w + hb + P_STREAMS * KV_BYTES * ctx_mean
    return {"streams": P_STREAMS, "value": round(P_STREAMS * steps / dt, 1), "unit": "tokens/s",
            "ms_per_step": round(ms, 4), "steps": steps,
            "workload": f"Pythia-160m-shaped integer machine, {P_STREAMS} streams, {P_PROMPT}-token random prompts, "
                        f"{P_WORDS} greedy words each (context to {P_PROMPT + P_WORDS}); streams 0 and 1 checked "
                        f"against pythia_base2.py's golden words",
            "prompt_included": {"value": round(P_STREAMS * P_WORDS / (tp + dt), 1), "unit": "tokens/s",
                                "prompt_ms": round(1000.0 * tp, 3)},
            "roofline": {"bound": "hbm", "achieved": round(hb / (us * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(hb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "kernel": "k_head_rows<2,EPI_PHEAD>",
                         "mean_launch_us": round(us, 3), "launches_timed": n},
            "step_roofline": {"bytes_per_step": int(sb), "achieved": round(sb / (ms * 1e-3) / 1e9, 1),
                              "frac": round(sb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}}


def cpu_baseline(npz, prompt, want, budget_s: float = 20.0):
    """base2.py's CPU path (numpy restatement): forward(ids + got) per word, as base2.py:123 does."""
    sys.path.insert(0, REPO)
    from oracle.base2_np import Base2Numpy
    try:
        from threadpoolctl import threadpool_info
        blas = [i for i in threadpool_info() if i.get("user_api") == "blas"]
        cores = int(blas[0]["num_threads"]) if blas else 1
    except Exception:
        cores = 1
    nb = Base2Numpy(npz)
    got, t_total, n = [], 0.0, 0
    for i in range(len(want)):
        t0 = time.perf_counter()
        w = nb.forward(list(prompt) + got)
        dt = time.perf_counter() - t0
        got.append(w)
        if i > 0:                       # decode words only (the first word is the prompt pass)
            t_total += dt
            n += 1
        if t_total > budget_s and n >= 2:
            break
    if got != want[:len(got)]:
        raise RuntimeError(f"cpu baseline words differ from the GPU's: {got} vs {want[:len(got)]}")
    return {"value": n / t_total, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"words 2..{n + 1} of the 8-token-prompt sequence, full recompute per word (context 9..{8 + n}), "
                      f"numpy float64-BLAS products and the top-down race loop"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=150)
    ap.add_argument("--warmup", type=int, default=15)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-batched", action="store_true", help="skip the 64-stream leg")
    ap.add_argument("--no-pythia", action="store_true", help="skip the Pythia 32-stream leg")
    ap.add_argument("--head-grid", type=int, default=0)
    ap.add_argument("--only", choices=("b1", "b64", "pythia"), default="",
                    help="profiling: run one leg and print only its result (not the bench line)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MB",
                    help="profiling: first copy MB MiB device to device (calibrates HBM byte counters)")
    ap.add_argument("--layout", default="", help="reuse a layout directory (else one is built in a temp dir)")
    ap.add_argument("--prefill-rows", type=int, default=64,
                    help="prompt rows a pass through the MFMA banks (0: the prompt position by position)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported (the batched streams would "
              f"shard as independent replicas, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    if args.steps <= 0 or args.warmup < 0:
        sys.exit("bench.py: --steps must be positive and --warmup non-negative")

    global PREFILL_ROWS
    PREFILL_ROWS = args.prefill_rows
    sm = load_sm()
    if args.copy_probe:
        import torch
        src = torch.ones(args.copy_probe << 18, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: {args.copy_probe} MiB device to device")
        del src, dst
    if args.only == "b64":
        print(json.dumps(batched_leg(sm, None)), flush=True)
        return
    if args.only == "pythia":
        print(json.dumps(pythia_leg(sm)), flush=True)
        return
    t0 = time.time()
    sd = sm.random_gpt2(seed=0)
    npz = sm.convert(sd)
    del sd
    lay = args.layout or tempfile.mkdtemp(prefix="sm_bench_")
    if not os.path.exists(os.path.join(lay, "manifest.json")):
        sm.layout(npz, lay)
    log(f"model converted and laid out in {time.time() - t0:.1f}s")
    prompt = sm.prompt_ids(1, PROMPT)

    # the parity gate: base2.py's own words for this sequence (golden fixture written from the reference)
    want = golden_words("base2_golden.json")["c1_p8_w16"]

    import torch
    m = sm.Machine(lay, max_ctx=64, head_grid=args.head_grid, graph_steps=WORDS - 1, profile=True,
                   prefill_rows=PREFILL_ROWS)
    vocab = m.vocab

    def sequence(timed: bool):
        m.reset()
        torch.cuda.synchronize()
        t = time.perf_counter()
        m.prefill(prompt)
        first = int(m.generate(1)[0, 0])        # the prompt pass and the first word
        torch.cuda.synchronize()
        tp = time.perf_counter() - t
        m.profile(clear=True)
        t = time.perf_counter()
        rest = [int(w) for w in m.generate(WORDS - 1)[0]]
        torch.cuda.synchronize()
        dt = time.perf_counter() - t
        words = [first] + rest
        if words != want:
            raise RuntimeError(f"GPU words differ from base2.py's golden words: {words} vs {want}")
        n, us = m.profile(clear=True)
        return dt, n, us, tp

    for _ in range(max(1, -(-args.warmup // (WORDS - 1)))):
        sequence(False)
    total, steps, head_n, head_us_sum, prompt_s, nseq = 0.0, 0, 0, 0.0, 0.0, 0
    while steps < args.steps:
        dt, n, us, tp = sequence(True)
        prompt_s += tp
        nseq += 1
        k = min(WORDS - 1, args.steps - steps)
        total += dt * k / (WORDS - 1)
        steps += k
        head_n += n
        head_us_sum += us * n
    head_us = head_us_sum / head_n
    ms_per_step = 1000.0 * total / steps
    tok_s = steps / total
    hb = head_bytes(vocab)
    ach = hb / (head_us * 1e-6) / 1e9
    ctx_mean = PROMPT + WORDS / 2.0
    sb = step_bytes(vocab, ctx_mean)
    step_ach = sb / (ms_per_step * 1e-3) / 1e9

    traffic = None
    tfile = os.path.join(REPO, "profiles", "head_gemv_traffic.txt")
    if os.path.exists(tfile):
        for line in open(tfile):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = int(float(line.split(":")[1]))

    m.close()
    if args.only == "b1":
        print(json.dumps({"value": round(tok_s, 2), "ms_per_step": round(ms_per_step, 4), "head_us": round(head_us, 3),
                          "prompt_ms": round(1000.0 * prompt_s / nseq, 3)}), flush=True)
        return
    batched = None if args.no_batched else batched_leg(sm, lay)
    if batched:
        log(f"batched: {batched['value']} tokens/s, {batched['ms_per_step']} ms/step, head {batched['roofline']['mean_launch_us']} us")
    pyleg = None if args.no_pythia else pythia_leg(sm)
    if pyleg:
        log(f"pythia: {pyleg['value']} tokens/s, {pyleg['ms_per_step']} ms/step, head {pyleg['roofline']['mean_launch_us']} us")
    cpu = None if args.no_cpu else cpu_baseline(npz, prompt, want)
    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tokens/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int64", "data": "synthetic",
        "config": {"workload": "GPT-2 124M integer base-2 decode, batch 1, 8-token random prompt, 16 greedy words "
                               "per sequence (15 decode steps, context 9..23), random-init N(0,0.02) seed 0",
                   "batch": 1, "prompt": PROMPT, "words": WORDS, "vocab": vocab},
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "k_gemv<768,4,4,PRO_GAUGE,EPI_HEAD> (head plate read; the race is its own launch)",
                     "bytes_per_launch": hb, "mean_launch_us": round(head_us, 3), "launches_timed": head_n},
        "step_roofline": {"bytes_per_step": int(sb), "achieved": round(step_ach, 1), "frac": round(step_ach / HBM_PEAK_GBS, 4)},
        "prompt_included": {"value": round(WORDS / (prompt_s / nseq + ms_per_step * 1e-3 * (WORDS - 1)), 2), "unit": "tokens/s",
                            "prompt_ms": round(1000.0 * prompt_s / nseq, 3),
                            "note": "16 words per sequence over the prompt pass (7 prompt rows through the int8 MFMA "
                                    "banks, then the first word's step) plus 15 decode steps"},
        "batched": batched,
        "pythia": pyleg,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
