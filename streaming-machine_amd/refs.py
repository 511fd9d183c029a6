"""The reference's real-weight fixtures, for use when the real GPT-2 weights are at hand.

* refs_many.json (the fp32 model's words for 30 prompts; base2_stream.swift:262-298 reads it and reports how many
  prompts come out identical, and for the others the first differing word and the model's own lead there):
  `run_refs(machine, refs)` gives the same report for the MI355X machine.
* gpu_fr2/rec_*.json "rec_hash" (base2_stream_fr2.swift:985-995): for every new position of a prompt and each of
  the 48 plates (slot 4 l + b, banks qkv, proj, fc, mproj), FNV-1a 64 over the plate's pile (its nout int64
  values), the light entering it (its nin values, each as the unsigned 32-bit word of the int32 light) and the
  light's water level (the same), every value fed as 8 little-endian bytes; written as lowercase hex without
  leading zeros.  `plate_hashes(x16, ex, pile)` forms the 48 hashes of one recorded position and
  `rec_hash(machine, ids, n_words)` the whole per-prompt list, through the machine's own record.

With random weights none of these fixtures applies (their words and hashes come from GPT-2's real weights);
the functions are checked here on the FNV-1a specification and on records the oracle computes.
"""
from __future__ import annotations

import numpy as np

FNV_OFFSET = 0xCBF29CE484222325
FNV_PRIME = 0x100000001B3
MASK64 = (1 << 64) - 1
NIN = (768, 768, 768, 3072)
NOUT = (2304, 768, 3072, 768)


def fnv1a64(data: bytes, h: int = FNV_OFFSET) -> int:
    """FNV-1a, 64 bits: for each byte, h ^= byte, h *= 0x100000001b3 (mod 2^64)."""
    for b in data:
        h = ((h ^ b) * FNV_PRIME) & MASK64
    return h


def _words(values, as_u32: bool) -> bytes:
    """values as 8-byte little-endian words; as_u32: each an int32 taken as its unsigned 32-bit pattern"""
    v = np.asarray(values, dtype=np.int64)
    if as_u32:
        v = v.astype(np.int32).view(np.uint32).astype(np.uint64)
    else:
        v = v.view(np.uint64)
    return v.astype("<u8").tobytes()


def plate_hash(pile, x16, ex) -> str:
    """one plate's record hash: its pile, then its light, then the light's water level"""
    h = fnv1a64(_words(pile, False))
    h = fnv1a64(_words(x16, True), h)
    h = fnv1a64(_words([ex], True), h)
    return format(h, "x")


def plate_hashes(x16, ex, pile) -> list:
    """the 48 hashes of one position from a record: x16 [12][4][3072], ex [12][4], pile [12][4][3072]"""
    out = []
    for slot in range(48):
        l, b = slot // 4, slot % 4
        out.append(plate_hash(pile[l, b, :NOUT[b]], x16[l, b, :NIN[b]], int(ex[l, b])))
    return out


def rec_hash(machine, ids, n_words: int) -> list:
    """the rec_hash list of one prompt: for each new position q = len(ids) .. len(ids) + n_words - 2 (every
    position whose word entered from the machine itself, base2_stream_fr2.swift:989), the 48 plate hashes, from
    the machine's record of stream 0"""
    S = len(ids)
    rows = []
    for q in range(S, S + n_words - 1):
        machine.reset()
        machine.record_at(q)
        machine.prefill(ids)
        machine.generate(n_words)
        rows.append(plate_hashes(machine.read("x16"), machine.read("exls")[:, :, 0], machine.read("pile")))
    return rows


def run_refs(machine, refs: list, n_words: int | None = None) -> dict:
    """base2_stream.swift's report over a refs_many.json list: each case's words against the fp32 model's
    ("ref"), the count of identical prompts, and for the others the first differing word and the model's lead
    there ("margins")"""
    report, same = [], 0
    for case in refs:
        want = list(case["ref"])[: n_words or len(case["ref"])]
        got = machine.stream(list(case["ids"]), len(want))
        if got == want:
            same += 1
            report.append({"prompt": case.get("prompt", ""), "identical": True})
            continue
        j = next(i for i in range(len(want)) if got[i] != want[i])
        margins = case.get("margins")
        report.append({"prompt": case.get("prompt", ""), "identical": False, "first_differs_at": j + 1,
                       "machine_word": got[j], "model_word": want[j],
                       "model_lead": None if margins is None else margins[j]})
    return {"identical": same, "prompts": len(refs), "per_prompt": report}
