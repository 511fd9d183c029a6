"""Pin the converters and the device-image layout to the reference's own scripts (run here, in the build container).

Writes tests/golden/converter_pins.json with digests only (SHA-256 of each converted array's dtype, shape and
bytes; SHA-256 of each file of a device-image directory):
  * base2_convert.py run on seeded GPT-2 state dicts (the 124M shape and a 1000-word, 64-position one): its
    transformers import is served by a stub module whose GPT2LMHeadModel.from_pretrained returns the seeded
    weights as torch tensors (the script's only input), and its npz is hashed array by array;
  * base2_gpu.py run on that npz: every file of its base2_gpu/ directory, and its manifest;
  * foundation0/pythia_convert.py run on seeded Pythia-160m-shaped checkpoints written as model.safetensors +
    config.json under a models/ tree beside the script's stand-in location (a finished checkpoint from
    random_pythia(seed=5) and a different start checkpoint from seed 6, so that the shared per-neuron power of
    two is set by the start on some neurons), and its npz is hashed array by array.
The reference source is read from /root/reference and executed here only; nothing of it is kept.
Usage:  python tests/golden/make_converter_pins.py [/root/reference]
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import tempfile
import time
import types

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"


def run_script(path: str, cwd: str, argv: list, file_as: str | None = None):
    src = open(path).read()
    old_cwd, old_argv = os.getcwd(), sys.argv
    os.chdir(cwd)
    sys.argv = argv
    try:
        exec(compile(src, path, "exec"), {"__name__": "__main__", "__file__": file_as or path})
    finally:
        os.chdir(old_cwd)
        sys.argv = old_argv


def file_digests(d: str) -> dict:
    out = {}
    for f in sorted(os.listdir(d)):
        with open(os.path.join(d, f), "rb") as fh:
            out[f] = hashlib.sha256(fh.read()).hexdigest()
    return out


def gpt2_pins(sm, kw):
    import torch
    sd = sm.random_gpt2(**kw)

    class _Model:
        def state_dict(self):
            return {k: torch.from_numpy(v) for k, v in sd.items()}

    stub = types.ModuleType("transformers")
    stub.GPT2LMHeadModel = types.SimpleNamespace(from_pretrained=lambda name: _Model())
    saved = sys.modules.get("transformers")
    sys.modules["transformers"] = stub
    work = tempfile.mkdtemp(prefix="sm_pin_gpt2_")
    try:
        run_script(os.path.join(REF, "base2_convert.py"), work, ["base2_convert.py"])
    finally:
        if saved is None:
            del sys.modules["transformers"]
        else:
            sys.modules["transformers"] = saved
    with np.load(os.path.join(work, "base2_gpt2.npz")) as z:
        npz = {k: z[k] for k in z.files}
    digest = sm.array_digest(npz)
    run_script(os.path.join(REF, "base2_gpu.py"), work, ["base2_gpu.py"])
    d = os.path.join(work, "base2_gpu")
    files = file_digests(d)
    with open(os.path.join(d, "manifest.json")) as f:
        manifest = json.load(f)
    return dict(recipe=kw, npz_digest=digest, layout_files=files, layout_manifest=manifest)


def pythia_pins(sm):
    from safetensors.numpy import save_file
    from streaming_machine_amd import pythia
    fin, cfg = pythia.random_pythia(seed=5)
    start, _ = pythia.random_pythia(seed=6)
    work = tempfile.mkdtemp(prefix="sm_pin_py_")
    hf_cfg = dict(hidden_size=cfg["d"], num_hidden_layers=cfg["n_layer"], num_attention_heads=cfg["n_head"],
                  intermediate_size=cfg["d_ff"], rotary_pct=cfg["rotary_pct"], rotary_emb_base=cfg["rotary_emb_base"],
                  max_position_embeddings=cfg["n_ctx"], layer_norm_eps=cfg["layer_norm_eps"], vocab_size=cfg["vocab"],
                  use_parallel_residual=True, hidden_act="gelu", tie_word_embeddings=False)
    for step, sd in (("step143000", fin), ("step0", start)):
        d = os.path.join(work, "models", f"pythia-160m-{step}")
        os.makedirs(d)
        save_file({k: np.ascontiguousarray(v) for k, v in sd.items()}, os.path.join(d, "model.safetensors"))
        with open(os.path.join(d, "config.json"), "w") as f:
            json.dump(hf_cfg, f)
    run_script(os.path.join(REF, "foundation0", "pythia_convert.py"), work, ["pythia_convert.py", "size=160m"],
               file_as=os.path.join(work, "pythia_convert.py"))
    with np.load(os.path.join(work, "base2_pythia-160m.npz")) as z:
        npz = {k: z[k] for k in z.files}
    with open(os.path.join(work, "convert_pythia-160m.json")) as f:
        report = json.load(f)
    start_sets = sum(r["start_sets_power"] for r in report)
    return dict(recipe=dict(finished_seed=5, start_seed=6, vocab=cfg["vocab"]), npz_digest=sm.array_digest(npz),
                start_sets_power=start_sets)


def main():
    sys.path.insert(0, HERE)
    from make_golden import load_pkg
    sm = load_pkg()
    t0 = time.time()
    out = {"generator": "tests/golden/make_converter_pins.py",
           "reference": "base2_convert.py, base2_gpu.py, foundation0/pythia_convert.py (run with seeded inputs)",
           "digest": "array_digest: sha256 of dtype, shape and C-order bytes; files: sha256 of the bytes"}
    out["gpt2_small"] = gpt2_pins(sm, dict(seed=0, vocab=1000, n_ctx=64))
    print(f"[{time.time() - t0:6.1f}s] gpt2 small", flush=True)
    out["gpt2_124m"] = gpt2_pins(sm, dict(seed=0, vocab=50257, n_ctx=1024))
    print(f"[{time.time() - t0:6.1f}s] gpt2 124m", flush=True)
    out["pythia_160m"] = pythia_pins(sm)
    print(f"[{time.time() - t0:6.1f}s] pythia 160m (start sets the power on {out['pythia_160m']['start_sets_power']} neurons)",
          flush=True)
    with open(os.path.join(HERE, "converter_pins.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote converter_pins.json in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
