"""numpy restatement of base2.py with the reference's own structure.

TEST INFRASTRUCTURE ONLY (the CPU baseline that bench.py times, and a second restatement for the tests).

It keeps what makes base2.py's CPU path cost what it costs:
  * forward(ids) recomputes every position of the sequence for each new word (base2.py:102-106, 123);
  * products are float64 matrix products, exact under the |p| < 2^52 guard (base2.py:29-32);
  * the race is the top-down bit elimination, one numpy pass per bit (base2.py:34-40), and attention runs it
    once per row per head (base2.py:95-96);
  * log2fix is a Python loop per value (base2.py:42-48).
Only the integer stages are restated (the float switches are diagnostics, not parity targets).
"""
from __future__ import annotations

import numpy as np

ES, SC = 16, 10
BANK_NAMES = ("qkv", "proj", "fc", "mproj")


class Base2Numpy:
    def __init__(self, npz: dict, n_layer: int = 12):
        self.n_layer = n_layer
        self.PHI, self.ARR = np.asarray(npz["phi"], np.int64), np.asarray(npz["arrival"], np.int64)
        self.LOG2, self.EXP2 = np.asarray(npz["log2"], np.int64), np.asarray(npz["exp2"], np.int64)
        self.LOG768, self.EPS40 = int(npz["log2_768"]), int(npz["eps40"])
        self.wte, self.wpe = np.asarray(npz["wte"], np.int64), np.asarray(npz["wpe"], np.int64)
        names = [f"{b}.{l}" for l in range(n_layer) for b in BANK_NAMES] + ["head"]
        # plates held as float64 like base2.py:16, so each product is one BLAS call
        self.W = {k: (np.asarray(npz[k + ".w"]).astype(np.float64), np.asarray(npz[k + ".e"], np.int64),
                      np.asarray(npz[k + ".b"], np.int64)) for k in names}

    # -- base2.py:18-22
    @staticmethod
    def rshift(X, s):
        s = np.asarray(s, dtype=np.int64)
        shifted = np.left_shift(X, np.maximum(-s, 0))
        pos = np.maximum(s, 0)
        half = np.where(pos > 0, np.left_shift(np.int64(1), np.maximum(pos - 1, 0)), 0)
        return np.right_shift(shifted + half, pos)

    # -- base2.py:24-27
    def to16(self, X, e):
        orr = np.bitwise_or.reduce(np.abs(X), axis=1)
        top = np.array([int(v).bit_length() for v in orr])
        sh = np.maximum(top - 15, 0)
        return self.rshift(X, sh[:, None]), e + sh

    # -- base2.py:29-32
    @staticmethod
    def product(x16, w):
        p = x16.astype(np.float64) @ w
        assert np.abs(p).max() < 2 ** 52
        return p.astype(np.int64)

    # -- base2.py:34-40
    @staticmethod
    def race(vals):
        u = vals.astype(np.int64).view(np.uint64) ^ np.uint64(1 << 63)
        alive = np.ones(len(u), dtype=bool)
        for bit in range(63, -1, -1):
            lit = alive & (((u >> np.uint64(bit)) & np.uint64(1)) == 1)
            if lit.any():
                alive = lit
        return int(np.flatnonzero(alive)[0])

    # -- base2.py:42-48
    def log2fix(self, V):
        res = []
        for v in V:
            v = int(v)
            t = v.bit_length() - 1
            m = (v >> (t - 16)) & 0xFFFF if t >= 16 else (v << (16 - t)) & 0xFFFF
            res.append(t * 65536 + int(self.LOG2[m]))
        return np.array(res, dtype=np.int64)

    # -- base2.py:50-53
    def power(self, X, F):
        F = np.asarray(F, dtype=np.int64)
        return self.rshift(X * self.EXP2[np.bitwise_and(F, 0xFFFF)], 16 - np.right_shift(F, 16))

    # -- base2.py:55-60
    def gauge_log(self, R):
        x16, ex = self.to16(R, -ES)
        S1, S2 = x16.sum(1), (x16 * x16).sum(1)
        eps = np.array([self.EPS40 >> (40 + 2 * int(e)) if 40 + 2 * int(e) >= 0 else self.EPS40 << -(40 + 2 * int(e))
                        for e in ex])
        V = 768 * S2 - S1 * S1 + eps
        return x16, ex, np.right_shift(self.log2fix(V), 1) - self.LOG768 + ex * 65536

    # -- base2.py:62-71 (integer gauge)
    def gauged_bank(self, R, name):
        w, we, b = self.W[name]
        x16, ex, LS = self.gauge_log(R)
        return self.power(self.product(x16, w), (we[None, :] + ex[:, None] + ES) * 65536 - LS[:, None]) + b

    # -- base2.py:73-76
    def plain_bank(self, X, name):
        w, we, b = self.W[name]
        x16, ex = self.to16(X, -ES)
        return self.rshift(self.product(x16, w), -(we[None, :] + ex[:, None] + ES)) + b

    # -- base2.py:78-83 (integer edge)
    def edge(self, H):
        idx = self.rshift(H, ES - 12) + 32768
        share = np.where(idx < 0, 0, np.where(idx > 65535, 65536, self.PHI[np.clip(idx, 0, 65535)]))
        return self.rshift(H * share, 16)

    # -- base2.py:85-100 (integer arrival)
    def attention(self, QKV):
        P = QKV.shape[0]
        out = np.zeros((P, 768), dtype=np.int64)
        alen = len(self.ARR)
        for h in range(12):
            q = QKV[:, h * 64:(h + 1) * 64]
            k = QKV[:, 768 + h * 64:768 + (h + 1) * 64]
            v = QKV[:, 1536 + h * 64:1536 + (h + 1) * 64]
            q16, eq = self.to16(q, -ES)
            k16, ek = self.to16(k, -ES)
            sc = self.rshift(self.product(q16, k16.T.astype(np.float64)), -(eq[:, None] + ek[None, :] - 3 + SC))
            for p in range(P):
                row = sc[p, :p + 1]
                d = row[self.race(row)] - row
                a = np.where(d < alen, self.ARR[np.minimum(d, alen - 1)], 0)
                num = self.product(a[None, :], v[:p + 1].astype(np.float64))[0]
                out[p, h * 64:(h + 1) * 64] = self.power(num, -self.log2fix([a.sum()])[0])
        return out

    # -- base2.py:102-114
    def forward(self, ids):
        P = len(ids)
        R = self.wte[ids] + self.wpe[:P]
        for l in range(self.n_layer):
            R = R + self.plain_bank(self.attention(self.gauged_bank(R, f"qkv.{l}")), f"proj.{l}")
            R = R + self.plain_bank(self.edge(self.gauged_bank(R, f"fc.{l}")), f"mproj.{l}")
        w, we, b = self.W["head"]
        x16, ex, LS = self.gauge_log(R[-1:])
        pile = self.product(x16, w)
        return self.race(self.power(pile, (we[None, :] + ex[:, None] + ES) * 65536 - LS[:, None])[0] + b)

    def generate(self, prompt, n_words):
        """base2.py:123's loop: each word recomputes the whole sequence."""
        got = []
        for _ in range(n_words):
            got.append(self.forward(list(prompt) + got))
        return got
