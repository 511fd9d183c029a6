"""Conversion: float GPT-2 weights -> the integer ("all base 2") machine's numbers, run once on the host.

Restates base2_convert.py (base2_convert.py:18-61):
  * each layer norm's mean removal (C = I - 1/n), gain and offset are folded into the bank after it:
        W' = C diag(g) W,   b' = offset . W + b            (base2_convert.py:31-41, 43-45)
  * every bank is stored as int16 with one power of two per output column, the smallest that holds the
    column's largest weight (cols16, base2_convert.py:20-26)
  * biases, the token table and the position table become whole numbers at the stream's scale 2^-16
    (base2_convert.py:28, 41, 45-46)
  * the tables: PHI (the GELU share), ARR (the arrival e^-d), LOG2 and EXP2 (fine parts) and the two
    constants log2(768) and eps (base2_convert.py:48-61)

Two deliberate differences, both for cross-machine determinism (the result is checked by hash):
  * C @ Y is computed as Y minus its column sums / n, and offset @ W as a column sum of offset[:, None] * W,
    instead of BLAS products whose rounding depends on the CPU's BLAS kernel.  The two are equal in exact
    arithmetic; in float64 they can differ in the last bit, which after rounding to 16 bits changes a weight
    by one step at most on a measure-zero set of inputs.
  * ceil(log2(mx / 32767)) is evaluated exactly through frexp instead of a libm log2.
The machine itself never sees a float: it reads only this module's output.
"""
from __future__ import annotations

import math

import numpy as np

ES = 16          # the stream's scale is 2^-ES (base2_convert.py:15)
SC = 10          # scores on a scale of 2^-SC (base2_convert.py:50)
N_EMBD = 768
BANKS = ("qkv", "proj", "fc", "mproj")


def _fold_center(Y: np.ndarray) -> np.ndarray:
    """C @ Y with C = I - 1/n: each column minus its mean (column sums accumulated row by row)."""
    n = Y.shape[0]
    return Y - (Y.sum(axis=0) / n)[None, :]


def _vec_mat(v: np.ndarray, W: np.ndarray) -> np.ndarray:
    """v @ W as a deterministic column sum."""
    return (v[:, None] * W).sum(axis=0)


def _ceil_log2(r: np.ndarray) -> np.ndarray:
    """Exact ceil(log2(r)) for r > 0: r = m 2^k with m in [0.5, 1) gives k, or k - 1 when m == 0.5."""
    m, k = np.frexp(r)
    return np.where(m == 0.5, k - 1, k).astype(np.int64)


def cols16(W: np.ndarray):
    """int16 weights, one power of two per column (base2_convert.py:20-26)."""
    mx = np.maximum(np.abs(W).max(axis=0), 1e-30)
    e = _ceil_log2(mx / 32767)
    q = np.round(W / np.exp2(e.astype(np.float64))[None, :]).astype(np.int64)
    if np.abs(q).max() > 32767:
        raise ValueError("cols16: a weight does not fit 16 bits")
    return q.astype(np.int16), e


def stream(v: np.ndarray) -> np.ndarray:
    """Whole numbers at the stream's scale 2^-16 (base2_convert.py:28)."""
    return np.round(np.asarray(v, dtype=np.float64) * 2.0 ** ES).astype(np.int64)


_TABLES: dict | None = None


def tables() -> dict:
    """The machine's tables (base2_convert.py:48-61).  The float expressions are kept term for term so the
    rounded integers are the reference's."""
    global _TABLES
    if _TABLES is None:
        root2 = math.sqrt(2)
        phi = np.array([round(0.5 * (1 + math.erf(((i - 32768) / 4096) / root2)) * 65536) for i in range(65536)],
                       dtype=np.int64)
        arr = []
        d = 0
        while True:
            a = round(math.exp(-d / 2 ** SC) * 2 ** 24)
            if a == 0:
                break
            arr.append(a)
            d += 1
        log2t = np.array([round(math.log2(1 + m / 65536) * 65536) for m in range(65536)], dtype=np.int64)
        exp2t = np.array([round(2 ** (f / 65536) * 65536) for f in range(65536)], dtype=np.int64)
        _TABLES = {
            "phi": phi,
            "arrival": np.array(arr, dtype=np.int64),
            "log2": log2t,
            "exp2": exp2t,
            "log2_768": np.array(round(math.log2(768) * 65536)),
            "eps40": np.array(round(1e-5 * 768 * 768 * 2 ** 40)),
        }
    return {k: v.copy() for k, v in _TABLES.items()}


def convert(sd: dict, n_layer: int = 12) -> dict:
    """HF-named GPT-2 state dict (numpy or torch, any float dtype) -> the npz dictionary base2.py loads
    (keys {qkv,proj,fc,mproj}.{l}.{w,e,b}, head.{w,e,b}, wte, wpe, phi, arrival, log2, exp2, log2_768, eps40)."""
    def get(k):
        v = sd[k]
        if hasattr(v, "detach"):
            v = v.detach().cpu().numpy()
        return np.asarray(v, dtype=np.float64)

    out = {}
    for k in range(n_layer):
        p = f"transformer.h.{k}."
        g1, b1, g2, b2 = get(p + "ln_1.weight"), get(p + "ln_1.bias"), get(p + "ln_2.weight"), get(p + "ln_2.bias")
        Wq, bq = get(p + "attn.c_attn.weight"), get(p + "attn.c_attn.bias")
        Wf, bf = get(p + "mlp.c_fc.weight"), get(p + "mlp.c_fc.bias")
        plates = (
            ("qkv", _fold_center(g1[:, None] * Wq), _vec_mat(b1, Wq) + bq),
            ("proj", get(p + "attn.c_proj.weight"), get(p + "attn.c_proj.bias")),
            ("fc", _fold_center(g2[:, None] * Wf), _vec_mat(b2, Wf) + bf),
            ("mproj", get(p + "mlp.c_proj.weight"), get(p + "mlp.c_proj.bias")),
        )
        for name, W, b in plates:
            out[f"{name}.{k}.w"], out[f"{name}.{k}.e"] = cols16(W)
            out[f"{name}.{k}.b"] = stream(b)
    wte = get("transformer.wte.weight")
    gf, bfin = get("transformer.ln_f.weight"), get("transformer.ln_f.bias")
    wteT = np.ascontiguousarray(wte.T)
    out["head.w"], out["head.e"] = cols16(_fold_center(gf[:, None] * wteT))
    out["head.b"] = stream(_vec_mat(bfin, wteT))
    out["wte"], out["wpe"] = stream(wte), stream(get("transformer.wpe.weight"))
    out.update(tables())
    return out


def array_digest(npz: dict) -> dict:
    """SHA-256 of every converted array (bytes in C order plus dtype and shape): the conversion's fingerprint."""
    import hashlib
    dig = {}
    for k in sorted(npz):
        a = np.ascontiguousarray(npz[k])
        h = hashlib.sha256()
        h.update(f"{a.dtype.str}{a.shape}".encode())
        h.update(a.tobytes())
        dig[k] = h.hexdigest()
    return dig
