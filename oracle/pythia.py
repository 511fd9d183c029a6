"""ctypes binding of pythia_oracle.c: the CPU restatement of foundation0/pythia_base2.py.

TEST INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke(), bench.py's cpu_baseline leg).

  PythiaOracle(npz).generate(prompt, n)      KV-cached greedy words (pythia_base2.py:forward's words)
  PythiaOracle(npz).session(max_ctx).step()  one position at a time, with an optional record of its numbers
  PythiaOracle(npz).attention(QKV)           pythia_base2.py:attention on a whole [P][3d] matrix

Parity pins: the golden vectors of tests/golden/make_golden_pythia.py (written by executing pythia_base2.py on
the same converted arrays): words, every intermediate of the last position, and attention at 300 and 1100
positions.  The stage functions it shares with the GPT-2 oracle (rshift, to16, log2fix, race, edge) are pinned
by tests/test_oracle_stages.py.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import build, _p, i16p, i64p

ERRORS = {1: "product passed 2^53 (pythia_base2.py:75)", 2: "position past the cache or word out of range",
          3: "rshift left shift past 2^62 (pythia_base2.py:63)", 4: "turn input past 2^31 (pythia_base2.py:121)",
          5: "attention sum passed 2^62 (pythia_base2.py:139)", 6: "power result past int64 (pythia_base2.py:90)"}


class PyModel(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in ("L", "d", "heads", "hs", "rot", "vocab", "npos", "alen")] + [
        ("w", (i16p * 4) * 12), ("e", (i64p * 4) * 12), ("b", (i64p * 4) * 12),
        ("ng", (i64p * 2) * 12), ("nge", (ctypes.c_int64 * 2) * 12), ("nb", (i64p * 2) * 12),
        ("fg", i64p), ("fge", ctypes.c_int64), ("fb", i64p),
        ("hw", i16p), ("he", i64p), ("ew", i16p), ("ee", i64p),
        ("phi", i64p), ("arr", i64p), ("log2t", i64p), ("exp2t", i64p), ("cosT", i64p), ("sinT", i64p),
        ("eps40", ctypes.c_int64), ("half", ctypes.c_int64),
        ("wmax", (ctypes.c_double * 4) * 12), ("hwmax", ctypes.c_double)]


class PyRec(ctypes.Structure):
    _fields_ = [(n, i64p) for n in ("stream", "g1", "g2", "x16", "ex", "pile", "out", "att", "hid",
                                    "stream_final", "glnf", "hx16", "hex", "hpile", "logits")]


def new_record(vocab: int, L: int = 12) -> dict:
    shapes = {"stream": (L, 768), "g1": (L, 768), "g2": (L, 768), "x16": (L, 4, 3072), "ex": (L, 4),
              "pile": (L, 4, 3072), "out": (L, 4, 3072), "att": (L, 768), "hid": (L, 3072), "stream_final": (768,),
              "glnf": (768,), "hx16": (768,), "hex": (1,), "hpile": (vocab,), "logits": (vocab,)}
    return {k: np.zeros(s, dtype=np.int64) for k, s in shapes.items()}


def _check(st: int):
    if st:
        raise ArithmeticError("pythia oracle: " + ERRORS.get(st, f"status {st}"))


class PythiaOracle:
    def __init__(self, npz: dict):
        self.lib = ctypes.CDLL(build())
        L = self.lib
        L.pyo_prepare.argtypes = [ctypes.POINTER(PyModel)]
        L.pyo_kv_new.restype = ctypes.c_void_p
        L.pyo_kv_new.argtypes = [ctypes.POINTER(PyModel), ctypes.c_int64]
        L.pyo_kv_free.argtypes = [ctypes.c_void_p]
        L.pyo_step.restype = ctypes.c_int64
        L.pyo_step.argtypes = [ctypes.POINTER(PyModel), ctypes.c_void_p, ctypes.c_int32, ctypes.c_int,
                               ctypes.POINTER(PyRec), ctypes.POINTER(ctypes.c_int)]
        L.pyo_read_kv.argtypes = [ctypes.POINTER(PyModel), ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, i64p, i64p, i64p]
        L.pyo_resid.argtypes = [ctypes.POINTER(PyModel), ctypes.c_void_p, i64p]
        L.pyo_attention.restype = ctypes.c_int
        L.pyo_attention.argtypes = [ctypes.POINTER(PyModel), i64p, ctypes.c_int64, i64p]
        self._keep = []
        m = PyModel()

        def keep(a, dtype):
            if dtype == np.int16:          # plates and word rows: plates=built's 17-bit digits are not held here
                a = np.asarray(a)
                if a.size and (int(a.max()) > 32767 or int(a.min()) < -32768):
                    raise ValueError("the oracle holds int16 plates: a digit past 16 bits (plates=built)")
            a = np.ascontiguousarray(a, dtype=dtype)
            self._keep.append(a)
            return a

        m.L, m.d, m.heads, m.hs, m.rot, m.vocab = (int(npz[k]) for k in ("L", "d", "heads", "hs", "rot", "vocab"))
        if m.d != 768 or m.heads * m.hs != 768 or m.hs > 64 or m.L > 12:
            raise ValueError("the oracle is sized for d = 768, head size <= 64, at most 12 layers")
        for l in range(m.L):
            for k, bn in enumerate(("qkv", "proj", "fc", "mproj")):
                m.w[l][k] = _p(keep(npz[f"{bn}.{l}.w"], np.int16), i16p)
                m.e[l][k] = _p(keep(npz[f"{bn}.{l}.e"], np.int64))
                m.b[l][k] = _p(keep(npz[f"{bn}.{l}.b"], np.int64))
            for j, nn in enumerate(("ln1", "ln2")):
                m.ng[l][j] = _p(keep(npz[f"{nn}.{l}.g"], np.int64))
                m.nge[l][j] = int(npz[f"{nn}.{l}.ge"])
                m.nb[l][j] = _p(keep(npz[f"{nn}.{l}.b"], np.int64))
        m.fg, m.fge, m.fb = _p(keep(npz["lnf.g"], np.int64)), int(npz["lnf.ge"]), _p(keep(npz["lnf.b"], np.int64))
        m.hw, m.he = _p(keep(npz["head.w"], np.int16), i16p), _p(keep(npz["head.e"], np.int64))
        m.ew, m.ee = _p(keep(npz["embed.w"], np.int16), i16p), _p(keep(npz["embed.e"], np.int64))
        cos = keep(npz["cos"], np.int64)
        m.npos = cos.shape[0]
        arr = keep(npz["arrival"], np.int64)
        m.alen = len(arr)
        m.phi, m.arr = _p(keep(npz["phi"], np.int64)), _p(arr)
        m.log2t, m.exp2t = _p(keep(npz["log2"], np.int64)), _p(keep(npz["exp2"], np.int64))
        m.cosT, m.sinT = _p(cos), _p(keep(npz["sin"], np.int64))
        m.eps40, m.half = int(npz["eps40"]), int(npz["half_log2_hs"])
        L.pyo_prepare(ctypes.byref(m))
        self.m = m
        self.vocab, self.n_pos, self.L = int(m.vocab), int(m.npos), int(m.L)

    def _rec(self, rec):
        if rec is None:
            return None
        r = PyRec()
        for name, _ in PyRec._fields_:
            if name in rec:
                setattr(r, name, _p(rec[name]))
        return ctypes.byref(r)

    def session(self, max_ctx: int = 2048) -> "PythiaSession":
        return PythiaSession(self, max_ctx)

    def generate(self, prompt, n_words: int, max_ctx: int | None = None) -> list:
        """KV-cached greedy decode: the prompt, then n_words words (each fed back)."""
        s = self.session(max_ctx or (len(prompt) + n_words))
        out, tok = [], None
        for i, t in enumerate(prompt):
            tok = s.step(t, want_head=(i == len(prompt) - 1))
        for _ in range(n_words):
            out.append(tok)
            if len(out) == n_words:
                break
            tok = s.step(tok)
        return out

    def attention(self, QKV: np.ndarray) -> np.ndarray:
        QKV = np.ascontiguousarray(QKV, dtype=np.int64)
        out = np.zeros((QKV.shape[0], 768), dtype=np.int64)
        _check(self.lib.pyo_attention(ctypes.byref(self.m), _p(QKV), QKV.shape[0], _p(out)))
        return out


class PythiaSession:
    def __init__(self, orc: PythiaOracle, max_ctx: int):
        self.o = orc
        self.h = orc.lib.pyo_kv_new(ctypes.byref(orc.m), max_ctx)
        self.max_ctx = max_ctx

    def __del__(self):
        if getattr(self, "h", None):
            self.o.lib.pyo_kv_free(self.h)
            self.h = None

    def step(self, tok: int, want_head: bool = True, rec=None) -> int:
        st = ctypes.c_int(0)
        r = self.o.lib.pyo_step(ctypes.byref(self.o.m), self.h, int(tok), int(want_head), self.o._rec(rec), ctypes.byref(st))
        _check(st.value)
        return int(r)

    def read_kv(self, layer: int, pos: int):
        k16, ek, v = np.zeros(768, np.int64), np.zeros(12, np.int64), np.zeros(768, np.int64)
        self.o.lib.pyo_read_kv(ctypes.byref(self.o.m), self.h, layer, pos, _p(k16), _p(ek), _p(v))
        return k16, ek, v

    def resid(self):
        R = np.zeros(768, np.int64)
        self.o.lib.pyo_resid(ctypes.byref(self.o.m), self.h, _p(R))
        return R
