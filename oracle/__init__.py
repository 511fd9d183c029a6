"""CPU oracle for the integer GPT-2 machine of base2.py.

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
package, as the checker (or the timed CPU baseline).  The HIP product path never imports it.

  oracle.C         ctypes binding of base2_oracle.c (exact int64 restatement: stage functions, full-recompute
                   forward, KV-cached step)
  oracle.base2_np  numpy restatement with base2.py's own structure (float64 products under the 2^52 bound,
                   the top-down race loop, full recompute per word): the CPU baseline

Parity pins, per function (see tests/test_oracle_stages.py, tests/test_oracle_golden.py):
  rshift, to16, log2fix, power, race, edge, gauge_log   closed forms + brute force with Python big ints
  product                                              exact integer GEMM (brute force)
  tables                                               closed-form constants (ALEN 17745, LOG768, EPS40) + monotonicity
  attention, forward, KV-cached step                    golden vectors written from base2.py itself
                                                        (tests/golden/make_golden.py) + KV == recompute
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

i64p = ctypes.POINTER(ctypes.c_int64)
i16p = ctypes.POINTER(ctypes.c_int16)
i32p = ctypes.POINTER(ctypes.c_int32)


def build(force: bool = False) -> str:
    """Compile base2_oracle.c with gcc (make -C oracle)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE] + (["-B"] if force else []), check=True)
    return LIB_PATH


class OrcModel(ctypes.Structure):
    _fields_ = [
        ("n_layer", ctypes.c_int64), ("d", ctypes.c_int64), ("n_head", ctypes.c_int64), ("hd", ctypes.c_int64),
        ("d_ff", ctypes.c_int64), ("vocab", ctypes.c_int64), ("n_ctx", ctypes.c_int64),
        ("w", (i16p * 4) * 12), ("e", (i64p * 4) * 12), ("b", (i64p * 4) * 12),
        ("head_w", i16p), ("head_e", i64p), ("head_b", i64p),
        ("wte", i64p), ("wpe", i64p),
        ("phi", i64p), ("arr", i64p), ("alen", ctypes.c_int64),
        ("log2t", i64p), ("exp2t", i64p),
        ("log768", ctypes.c_int64), ("eps40", ctypes.c_int64),
    ]


class OrcRec(ctypes.Structure):
    _fields_ = [(n, i64p) for n in ("x16", "ex", "ls", "pile", "qkv", "att", "hid", "resid",
                                    "head_x16", "head_ex", "head_ls", "head_pile", "logits")]


REC_SHAPES = {
    "x16": (12, 4, 3072), "ex": (12, 4), "ls": (12, 4), "pile": (12, 4, 3072), "qkv": (12, 2304),
    "att": (12, 768), "hid": (12, 3072), "resid": (12, 2, 768), "head_x16": (768,), "head_ex": (1,),
    "head_ls": (1,),
}


def new_record(vocab: int) -> dict:
    r = {k: np.zeros(s, dtype=np.int64) for k, s in REC_SHAPES.items()}
    r["head_pile"] = np.zeros(vocab, dtype=np.int64)
    r["logits"] = np.zeros(vocab, dtype=np.int64)
    return r


def _p(a, t=i64p):
    return a.ctypes.data_as(t)


class Oracle:
    """The C oracle bound to one converted model (an npz dictionary; arrays are kept alive here)."""

    def __init__(self, npz: dict, bound: bool = True):
        """bound: report base2.py's 2^52 exactness bound (its float64 products are exact only below it) as an error;
        False: the KV-cached steps return the exact int64 result past it (the device's contract)"""
        self.bound = bound
        self.lib = ctypes.CDLL(build())
        L = self.lib
        L.orc_forward.restype = ctypes.c_int64
        L.orc_forward.argtypes = [ctypes.POINTER(OrcModel), i32p, ctypes.c_int64, ctypes.POINTER(OrcRec), ctypes.POINTER(ctypes.c_int)]
        L.orc_kv_new.restype = ctypes.c_void_p
        L.orc_kv_new.argtypes = [ctypes.c_int64]
        L.orc_kv_free.argtypes = [ctypes.c_void_p]
        L.orc_kv_step.restype = ctypes.c_int64
        L.orc_kv_step.argtypes = [ctypes.POINTER(OrcModel), ctypes.c_void_p, ctypes.c_int32, ctypes.c_int, ctypes.POINTER(OrcRec), ctypes.POINTER(ctypes.c_int)]
        L.orc_kv_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, i64p, i64p, i64p]
        L.orc_kv_read_resid.argtypes = [ctypes.c_void_p, i64p]
        L.orc_attention.restype = ctypes.c_int
        L.orc_attention.argtypes = [ctypes.POINTER(OrcModel), i64p, ctypes.c_int64, i64p]
        L.orc_attend_cached.restype = ctypes.c_int
        L.orc_attend_cached.argtypes = [ctypes.POINTER(OrcModel), i64p, i64p, i64p, i64p, ctypes.c_int64, ctypes.c_int64, i64p]
        self._keep = []
        m = OrcModel()

        def keep(a, dtype):
            a = np.ascontiguousarray(a, dtype=dtype)
            self._keep.append(a)
            return a

        m.n_layer, m.d, m.n_head, m.hd, m.d_ff = 12, 768, 12, 64, 3072
        wte = keep(npz["wte"], np.int64)
        wpe = keep(npz["wpe"], np.int64)
        m.vocab = wte.shape[0]
        m.n_ctx = wpe.shape[0]
        for l in range(12):
            for k, bn in enumerate(("qkv", "proj", "fc", "mproj")):
                m.w[l][k] = _p(keep(npz[f"{bn}.{l}.w"], np.int16), i16p)
                m.e[l][k] = _p(keep(npz[f"{bn}.{l}.e"], np.int64))
                m.b[l][k] = _p(keep(npz[f"{bn}.{l}.b"], np.int64))
        m.head_w = _p(keep(npz["head.w"], np.int16), i16p)
        m.head_e = _p(keep(npz["head.e"], np.int64))
        m.head_b = _p(keep(npz["head.b"], np.int64))
        m.wte, m.wpe = _p(wte), _p(wpe)
        self.phi = keep(npz["phi"], np.int64)
        self.arr = keep(npz["arrival"], np.int64)
        self.log2t = keep(npz["log2"], np.int64)
        self.exp2t = keep(npz["exp2"], np.int64)
        m.phi, m.arr, m.alen = _p(self.phi), _p(self.arr), len(self.arr)
        m.log2t, m.exp2t = _p(self.log2t), _p(self.exp2t)
        m.log768, m.eps40 = int(npz["log2_768"]), int(npz["eps40"])
        self.m = m
        self.vocab = int(m.vocab)
        self.n_ctx = int(m.n_ctx)

    def _rec(self, rec):
        if rec is None:
            return None
        r = OrcRec()
        for name, _ in OrcRec._fields_:
            if name in rec:
                setattr(r, name, _p(rec[name]))
        return ctypes.byref(r)

    def forward(self, ids, rec=None) -> int:
        """base2.py:forward: recompute every position of `ids`; the next word."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        st = ctypes.c_int(0)
        tok = self.lib.orc_forward(ctypes.byref(self.m), _p(ids, i32p), len(ids), self._rec(rec), ctypes.byref(st))
        if st.value:
            raise ArithmeticError("oracle: a product passed the 2^52 bound of base2.py:31")
        return int(tok)

    def attention(self, QKV: np.ndarray) -> np.ndarray:
        QKV = np.ascontiguousarray(QKV, dtype=np.int64)
        out = np.zeros((QKV.shape[0], 768), dtype=np.int64)
        if self.lib.orc_attention(ctypes.byref(self.m), _p(QKV), QKV.shape[0], _p(out)):
            raise ArithmeticError("oracle: attention sum passed 2^52")
        return out

    def attend_cached(self, qkv: np.ndarray, k16: np.ndarray, ek: np.ndarray, v: np.ndarray, p: int) -> np.ndarray:
        """the newest row p's attention over a given cache (k16 [12][ctx][64], ek [12][ctx], v [12][ctx][64]; rows
        s < p used) and its own q, k, v from qkv [2304]: the device attention's contract (sm_stage_attend)"""
        qkv = np.ascontiguousarray(qkv, dtype=np.int64)
        k16 = np.ascontiguousarray(k16, dtype=np.int64)
        ek = np.ascontiguousarray(ek, dtype=np.int64)
        v = np.ascontiguousarray(v, dtype=np.int64)
        ctx = k16.shape[1]
        assert k16.shape == (12, ctx, 64) and ek.shape == (12, ctx) and v.shape == (12, ctx, 64) and 0 <= p < ctx
        out = np.zeros(768, dtype=np.int64)
        if self.lib.orc_attend_cached(ctypes.byref(self.m), _p(qkv), _p(k16), _p(ek), _p(v), ctx, p, _p(out)):
            raise ArithmeticError("oracle: attention sum passed 2^52")
        return out

    def session(self, max_ctx: int = 1024) -> "KVSession":
        return KVSession(self, max_ctx)

    def generate(self, prompt, n_words: int, max_ctx: int | None = None) -> list:
        """KV-cached greedy decode: the prompt, then n_words words (each fed back)."""
        s = self.session(max_ctx or (len(prompt) + n_words))
        out = []
        tok = None
        for i, t in enumerate(prompt):
            tok = s.step(t, want_head=(i == len(prompt) - 1))
        for _ in range(n_words):
            out.append(tok)
            if len(out) == n_words:
                break
            tok = s.step(tok)
        return out


class KVSession:
    def __init__(self, orc: Oracle, max_ctx: int):
        self.o = orc
        self.h = orc.lib.orc_kv_new(max_ctx)
        self.max_ctx = max_ctx

    def __del__(self):
        if getattr(self, "h", None):
            self.o.lib.orc_kv_free(self.h)
            self.h = None

    def step(self, tok: int, want_head: bool = True, rec=None) -> int:
        st = ctypes.c_int(0)
        r = self.o.lib.orc_kv_step(ctypes.byref(self.o.m), self.h, int(tok), int(want_head), self.o._rec(rec), ctypes.byref(st))
        if st.value == 2:
            raise ValueError("oracle: position past the cache or token out of range")
        if st.value and self.o.bound:
            raise ArithmeticError("oracle: a product passed the 2^52 bound of base2.py:31")
        return int(r)

    def read_kv(self, layer: int, pos: int):
        k16 = np.zeros(768, np.int64)
        ek = np.zeros(12, np.int64)
        v = np.zeros(768, np.int64)
        self.o.lib.orc_kv_read(self.h, layer, pos, _p(k16), _p(ek), _p(v))
        return k16, ek, v

    def resid(self):
        R = np.zeros(768, np.int64)
        self.o.lib.orc_kv_read_resid(self.h, _p(R))
        return R


def set_threads(n: int) -> int:
    """OpenMP threads of the C oracle's parallel loops (0: every processor); returns the count in force"""
    L = ctypes.CDLL(build())
    L.orc_set_threads.argtypes = [ctypes.c_int]
    L.orc_get_threads.restype = ctypes.c_int
    L.orc_set_threads(int(n))
    return int(L.orc_get_threads())


def stage_lib():
    """The C oracle's stage functions with argtypes set (rshift, log2fix, power, edge, to16, gauge_log, product, race)."""
    L = ctypes.CDLL(build())
    L.orc_rshift.argtypes = [i64p, i64p, i64p, ctypes.c_int64]
    L.orc_log2fix.argtypes = [i64p, i64p, ctypes.c_int64, i64p]
    L.orc_power.argtypes = [i64p, i64p, i64p, ctypes.c_int64, i64p]
    L.orc_edge.argtypes = [i64p, i64p, ctypes.c_int64, i64p]
    L.orc_to16.argtypes = [i64p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, i64p, i64p]
    L.orc_gauge_log.argtypes = [i64p, ctypes.c_int64, ctypes.c_int64, i64p, i64p, i64p, ctypes.c_int64, ctypes.c_int64, i64p]
    L.orc_product.restype = ctypes.c_int
    L.orc_product.argtypes = [i64p, ctypes.c_int64, ctypes.c_int64, i16p, ctypes.c_int64, i64p]
    L.orc_race.restype = ctypes.c_int64
    L.orc_race.argtypes = [i64p, ctypes.c_int64]
    return L


class Stages:
    """numpy-in / numpy-out wrappers of the C oracle's stage functions."""

    def __init__(self, tabs: dict):
        self.L = stage_lib()
        self.log2t = np.ascontiguousarray(tabs["log2"], np.int64)
        self.exp2t = np.ascontiguousarray(tabs["exp2"], np.int64)
        self.phi = np.ascontiguousarray(tabs["phi"], np.int64)
        self.log768 = int(tabs["log2_768"])
        self.eps40 = int(tabs["eps40"])

    @staticmethod
    def _c(a, dt=np.int64):
        return np.ascontiguousarray(a, dtype=dt)

    def rshift(self, x, s):
        x = self._c(x)
        s = self._c(np.broadcast_to(s, x.shape))
        out = np.empty_like(x)
        self.L.orc_rshift(_p(x), _p(s), _p(out), x.size)
        return out

    def log2fix(self, v):
        v = self._c(v)
        out = np.empty_like(v)
        self.L.orc_log2fix(_p(v), _p(out), v.size, _p(self.log2t))
        return out

    def power(self, x, F):
        x = self._c(x)
        F = self._c(np.broadcast_to(F, x.shape))
        out = np.empty_like(x)
        self.L.orc_power(_p(x), _p(F), _p(out), x.size, _p(self.exp2t))
        return out

    def edge(self, h):
        h = self._c(h)
        out = np.empty_like(h)
        self.L.orc_edge(_p(h), _p(out), h.size, _p(self.phi))
        return out

    def to16(self, X, e=-16):
        X = self._c(np.atleast_2d(X))
        x16 = np.empty_like(X)
        ex = np.empty(X.shape[0], np.int64)
        self.L.orc_to16(_p(X), X.shape[0], X.shape[1], e, _p(x16), _p(ex))
        return x16, ex

    def gauge_log(self, R):
        R = self._c(np.atleast_2d(R))
        x16 = np.empty_like(R)
        ex = np.empty(R.shape[0], np.int64)
        LS = np.empty(R.shape[0], np.int64)
        self.L.orc_gauge_log(_p(R), R.shape[0], R.shape[1], _p(x16), _p(ex), _p(LS), self.log768, self.eps40, _p(self.log2t))
        return x16, ex, LS

    def product(self, x16, w):
        x16 = self._c(np.atleast_2d(x16))
        w = self._c(w, np.int16)
        pile = np.empty((x16.shape[0], w.shape[1]), np.int64)
        if self.L.orc_product(_p(x16), x16.shape[0], x16.shape[1], _p(w, i16p), w.shape[1], _p(pile)):
            raise ArithmeticError("product passed 2^52")
        return pile

    def race(self, v):
        v = self._c(v)
        return int(self.L.orc_race(_p(v), v.size))
