"""streaming-machine on MI355X: the integer ("all base 2") GPT-2 decode step as hand-written gfx950 HIP.

Host API, after the reference's "convert -> layout -> stream" (base2_convert.py, base2_gpu.py, base2.py):
    sd   = random_gpt2(seed)                    # or any HF-named GPT-2 state dict
    npz  = convert(sd)                          # base2_convert.py's numbers
    layout(npz, "base2_gpu")                    # base2_gpu.py's directory format
    m    = Machine("base2_gpu")                 # the HIP library owns weights, tables and the KV cache
    ids  = m.stream(prompt_ids, n_words)        # greedy words, decoded on the GPU
    word = m.forward(ids)                       # base2.py:forward's contract
"""
from .convert import convert, tables, cols16, stream, array_digest  # noqa: F401
from .model import random_gpt2, prompt_ids, GPT2_SHAPE  # noqa: F401
from .layout import layout, load_layout, bank_names, rewire  # noqa: F401
from . import pythia  # noqa: F401
from . import refs  # noqa: F401


def __getattr__(name):
    # the ctypes binding is loaded on first use so that CPU-only callers never need the HIP runtime
    if name in ("Machine", "Tables", "Plate", "lib", "LIB_PATH", "SmError", "stages", "check", "profile_stages",
                "kernel_times"):
        from . import machine
        return getattr(machine, name)
    raise AttributeError(name)
