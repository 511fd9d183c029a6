"""ctypes binding of libsm_base2.so (include/sm_base2.h) and the host-side machine API.

Machine mirrors the reference's machine (base2.py:forward and base2_stream.swift's run loop): it owns the
device image of a base2_gpu.py directory and decodes greedy words on the GPU.  There is no CPU fallback:
if the HIP library is missing or the device call fails, an SmError is raised.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsm_base2.so")

SM_OK, SM_E_ARG, SM_E_IO, SM_E_HIP, SM_E_OOM, SM_E_CTX, SM_E_OVERFLOW, SM_E_STATE = 0, -1, -2, -3, -4, -5, -6, -7
CODES = {SM_E_ARG: "SM_E_ARG", SM_E_IO: "SM_E_IO", SM_E_HIP: "SM_E_HIP", SM_E_OOM: "SM_E_OOM", SM_E_CTX: "SM_E_CTX",
         SM_E_OVERFLOW: "SM_E_OVERFLOW", SM_E_STATE: "SM_E_STATE"}

READ = dict(k16=1, ek=2, v=3, resid=4, seq=5, x16=10, exls=11, pile=12, qkv=13, att=14, hid=15, rresid=16,
            hx16=17, hexls=18, hpile=19, logits=20, gauge=21, fcpre=22, hgauge=23, top=24, v64=25)


class SmError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{CODES.get(code, code)}: {msg}")
        self.code = code


class SmConfig(ctypes.Structure):
    _fields_ = [("max_streams", ctypes.c_int32), ("max_ctx", ctypes.c_int32), ("use_graph", ctypes.c_int32),
                ("head_grid", ctypes.c_int32), ("graph_steps", ctypes.c_int32), ("profile", ctypes.c_int32),
                ("table_mode", ctypes.c_int32), ("prefill_rows", ctypes.c_int32), ("inv", ctypes.c_int32),
                ("float_stages", ctypes.c_int32), ("top_read", ctypes.c_int32), ("att_split", ctypes.c_int32),
                ("v64", ctypes.c_int32)]


FLOAT_STAGES = dict(gauge=1, edge=2, arrival=4, turn=8)     # SM_FLOAT_* of include/sm_base2.h


_LIB = None
vp = ctypes.c_void_p
i32, i64 = ctypes.c_int32, ctypes.c_int64
i32p, i64p = ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int64)


def lib():
    """Load the HIP library (built by __graft_entry__.build()); raises if it is not there."""
    global _LIB
    if _LIB is None:
        # The library binds whichever HIP runtime (libamdhip64.so.7) the process already holds.  torch bundles its
        # own copy under that soname and finds no GPU when initialised on top of the other one, so a process that
        # uses torch imports it before this first load (the tests and bench.py do); the library itself never
        # imports torch.
        if not os.path.exists(LIB_PATH):
            raise SmError(SM_E_IO, f"{LIB_PATH} is missing: build it (python -c 'import __graft_entry__ as g; g.build()')")
        L = ctypes.CDLL(LIB_PATH)
        L.sm_last_error.restype = ctypes.c_char_p
        L.sm_create.argtypes = [ctypes.c_char_p, ctypes.POINTER(SmConfig), ctypes.POINTER(vp)]
        L.sm_destroy.argtypes = [vp]
        L.sm_reset.argtypes = [vp]
        L.sm_prefill.argtypes = [vp, i32, i32p, i32]
        L.sm_generate.argtypes = [vp, i32, i32p]
        L.sm_record_at.argtypes = [vp, i32]
        L.sm_read.argtypes = [vp, i32, i32, i32, i32, vp, ctypes.c_size_t]
        L.sm_info.argtypes = [vp, i32p, i32p, i32p, i32p, i32p]
        L.sm_model_kind.argtypes = [vp]
        L.sm_top_read.argtypes = [vp]
        L.sm_tables_verified.argtypes = [vp]
        L.sm_profile.argtypes = [vp, i64p, ctypes.POINTER(ctypes.c_double), i32]
        L.sm_profile_stages.argtypes = [i32]
        L.sm_profile_kernels.argtypes = [ctypes.c_char_p, i32, i64p, ctypes.POINTER(ctypes.c_double), i32, i32p, i32]
        L.sm_tables_create.argtypes = [i64p, i64p, i32, i64p, i64p, i64, i64, ctypes.POINTER(vp)]
        L.sm_tables_destroy.argtypes = [vp]
        L.sm_stage_rshift.argtypes = [vp, vp, vp, i64, vp]
        L.sm_stage_log2fix.argtypes = [vp, vp, vp, i64, vp]
        L.sm_stage_power.argtypes = [vp, vp, vp, vp, i64, vp]
        L.sm_stage_edge.argtypes = [vp, vp, vp, i64, vp]
        L.sm_stage_to16.argtypes = [vp, i32, i32, vp, vp, vp]
        L.sm_stage_gauge_log.argtypes = [vp, vp, i32, vp, vp, vp, vp]
        L.sm_stage_race.argtypes = [vp, i64, vp, vp]
        L.sm_stage_attend.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, vp, vp]
        L.sm_stage_attend_split.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, vp, vp]
        L.sm_stage_attend_rows.argtypes = [vp, vp, i32, vp, vp, vp, vp, i32, i32, vp, vp]
        L.sm_plate_create.argtypes = [ctypes.POINTER(ctypes.c_int16), i32p, i64p, i32, i32, i32, ctypes.POINTER(vp)]
        L.sm_plate_destroy.argtypes = [vp]
        L.sm_plate_product.argtypes = [vp, vp, vp, i32, vp]
        L.sm_plate_product_rows.argtypes = [vp, vp, i32, vp, vp]
        L.sm_plate_product_rows_from.argtypes = [vp, vp, vp, i32, vp, vp]
        L.sm_plate_product_rows_noalloc.argtypes = [vp, vp, i32, vp, vp]
        L.sm_plate_bytes.restype = i64
        L.sm_plate_bytes.argtypes = [vp]
        _LIB = L
    return _LIB


def check(rc: int):
    if rc != SM_OK:
        raise SmError(rc, lib().sm_last_error().decode(errors="replace"))


def _np(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


class Machine:
    """The integer GPT-2 machine on one MI355X.

    Machine(layout_dir, max_ctx=1024, max_streams=1, use_graph=True, prefill_rows=64, gauge="int", edge="int",
            arrival="int")
      prefill_rows: every prompt position but the last goes through the int8 MFMA banks that many rows a pass
      (base2_stream.swift:274: the prompt through each layer at once); 0 runs it position by position.
      inv: the complement machine (base2_stream.swift:26 `inv`): stream, plates and lights held bit-complemented on
      the device; the same words (GPT-2, one stream, prefill_rows=0).
      top: "fr" (base2_stream_fr.swift's collapsing top read: the high bytes of every word, then the low bytes of
      the words that can still win; the same words; GPT-2, one stream, no inv or float stages), "plain" (the
      default: the whole word table read a step, measured faster at batch 1), or "auto" (the collapsing read
      where it applies).  .top_read says which runs; .top() gives the last step's survivors.
      .stream(prompt_ids, n_words) -> list of words        (base2.py:123's loop, KV-cached on the device)
      .forward(ids) -> word                                 (base2.py:forward's contract)
      .reset(); .prefill(ids, stream=0); .generate(n_words) -> int32 [n_streams][n_words]
      .record_at(pos); .read(name, layer=0, stream=0, pos=0)
      att_split: batch 1, the position from which a step's attention runs spread over the GPU (chunks of 64
      positions, one block a chunk; 0: from position 160, -1: never); the same words either way.
      v64: every head reads its cached values whole (64-bit) from the start; by default a head does so once it holds
      a value past 32 bits (every value's low 32 bits are kept, and a row holding a value past them also whole);
      the same words either way.
    gauge / edge / arrival ("int" or "float"; base2.py:10-11) and turn (the Pythia machine,
    foundation0/pythia_base2.py:21-27) put that stage back to float64 on the device, as the reference's switches
    do: diagnostics, compared with the reference at the word level (one stream, prefill_rows=0).  With
    arrival="float" the cache holds each key as float64 (read("k16") / read("ek") are not kept).
    """

    def __init__(self, layout_dir: str, max_ctx: int = 1024, max_streams: int = 1, use_graph: bool = True,
                 head_grid: int = 0, graph_steps: int = 16, profile: bool = False, verify_tables: bool = False,
                 prefill_rows: int = 64, gauge: str = "int", edge: str = "int", arrival: str = "int", turn: str = "int",
                 inv: bool = False, top: str = "plain", att_split: int = 0, v64: bool = False):
        fs = 0
        for name, v in (("gauge", gauge), ("edge", edge), ("arrival", arrival), ("turn", turn)):
            if v not in ("int", "float"):
                raise ValueError(f"{name}={v}: each stage is int or float")
            fs |= FLOAT_STAGES[name] if v == "float" else 0
        if top not in ("plain", "fr", "auto"):
            raise ValueError(f"top={top}: plain, fr or auto")
        self.L = lib()
        cfg = SmConfig(max_streams, max_ctx, 1 if use_graph else 0, head_grid, graph_steps, 1 if profile else 0,
                       1 if verify_tables else 0, prefill_rows, 1 if inv else 0, fs,
                       dict(plain=0, fr=1, auto=2)[top], att_split, 1 if v64 else 0)
        h = vp()
        check(self.L.sm_create(os.fsencode(layout_dir), ctypes.byref(cfg), ctypes.byref(h)))
        self.h = h
        v, c, s, n, ar = i32(), i32(), i32(), i32(), i32()
        check(self.L.sm_info(self.h, ctypes.byref(v), ctypes.byref(c), ctypes.byref(s), ctypes.byref(n), ctypes.byref(ar)))
        self.vocab, self.max_ctx, self.max_streams, self.n_pos = v.value, c.value, s.value, n.value
        self.tables_verified = bool(ar.value)          # every table entry equals its formula (base2_convert.py:48-61)
        k = self.L.sm_model_kind(self.h)
        check(min(k, 0))
        self.kind = ("gpt2", "pythia")[k]
        t = self.L.sm_top_read(self.h)
        check(min(t, 0))
        self.top_read = bool(t)

    def close(self):
        if getattr(self, "h", None):
            self.L.sm_destroy(self.h)
            self.h = None

    __del__ = close

    def reset(self):
        check(self.L.sm_reset(self.h))

    def prefill(self, ids, stream: int = 0):
        a = _np(ids, np.int32)
        check(self.L.sm_prefill(self.h, stream, a.ctypes.data_as(i32p), len(a)))

    def generate(self, n_words: int) -> np.ndarray:
        out = np.zeros((self.max_streams, n_words), dtype=np.int32)
        check(self.L.sm_generate(self.h, n_words, out.ctypes.data_as(i32p)))
        return out

    def streams(self, prompts, n_words: int) -> list:
        """every stream at once: prompts[b] (all of one length) then n_words words each"""
        self.reset()
        for b, p in enumerate(prompts):
            self.prefill(p, b)
        return [[int(w) for w in row] for row in self.generate(n_words)]

    def stream(self, prompt, n_words: int, stream: int = 0) -> list:
        """base2.py:123's loop for one prompt: its n_words greedy words.  Every stream of the machine takes the
        prompt (all streams of a run decode in lockstep from prompts of one length), and stream `stream`'s words
        are returned."""
        if not 0 <= stream < self.max_streams:
            raise SmError(SM_E_ARG, f"stream {stream} outside [0, {self.max_streams})")
        self.reset()
        for b in range(self.max_streams):
            self.prefill(prompt, b)
        return [int(w) for w in self.generate(n_words)[stream]]

    def forward(self, ids) -> int:
        """base2.py:forward: the word that follows ids."""
        return self.stream(ids, 1)[0]

    def profile(self, clear: bool = True):
        """(head launches timed, their mean duration in microseconds) since the last clear"""
        n, us = ctypes.c_int64(), ctypes.c_double()
        check(self.L.sm_profile(self.h, ctypes.byref(n), ctypes.byref(us), 1 if clear else 0))
        return n.value, (us.value / n.value if n.value else float("nan"))

    def kernels(self, clear: bool = True) -> dict:
        """per kernel name: (launches, mean microseconds) of every timed launch since the last clear (profile=True
        machines; stage entry points after profile_stages(True)); process-wide"""
        return kernel_times(clear)

    def record_at(self, pos: int):
        check(self.L.sm_record_at(self.h, pos))

    def read(self, name: str, layer: int = 0, stream: int = 0, pos: int = 0) -> np.ndarray:
        shapes = {"k16": ((768,), np.int32), "ek": ((12,), np.int32), "v": ((768,), np.int32), "v64": ((768,), np.int64),
                  "resid": ((768,), np.int64), "seq": ((self.max_ctx + 1,), np.int32),
                  "x16": ((12, 4, 3072), np.int64), "exls": ((12, 4, 2), np.int64), "pile": ((12, 4, 3072), np.int64),
                  "qkv": ((12, 2304), np.int64), "att": ((12, 768), np.int64), "hid": ((12, 3072), np.int64),
                  "rresid": ((12, 2, 768), np.int64), "hx16": ((768,), np.int64), "hexls": ((2,), np.int64),
                  "hpile": ((self.vocab,), np.int64), "logits": ((self.vocab,), np.int64),
                  "gauge": ((12, 2, 768), np.int64), "fcpre": ((12, 3072), np.int64), "hgauge": ((768,), np.int64)}
        shape, dt = shapes[name]
        out = np.zeros(shape, dtype=dt)
        check(self.L.sm_read(self.h, READ[name], layer, stream, pos, out.ctypes.data, out.nbytes))
        return out

    def top(self) -> tuple:
        """the collapsing top read's last step: (survivor count, [(word, exact pile, score)] of the first 1024)"""
        out = np.zeros(1 + 3 * 1024, dtype=np.int64)
        check(self.L.sm_read(self.h, READ["top"], 0, 0, 0, out.ctypes.data, out.nbytes))
        n = int(out[0])
        rows = out[1:].reshape(1024, 3)[:min(n, 1024)]
        return n, [tuple(int(v) for v in r) for r in rows]


def profile_stages(on: bool = True):
    """stamp every launch of the stage and plate entry points with its own HIP event pair"""
    check(lib().sm_profile_stages(1 if on else 0))


def kernel_times(clear: bool = True, symbols: bool = False) -> dict:
    """kernel name -> (launches, mean microseconds) of the timed launches since the last clear (process-wide);
    symbols=True: (launches, mean microseconds, the device function's demangled name as a kernel trace gives it)"""
    cap = 256
    names = ctypes.create_string_buffer(cap * 256)
    n_l = np.zeros(cap, np.int64)
    us = np.zeros(cap, np.float64)
    n = i32()
    check(lib().sm_profile_kernels(names, len(names), n_l.ctypes.data_as(i64p), us.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                                   cap, ctypes.byref(n), 1 if clear else 0))
    rows = [r.split("\t", 1) for r in names.value.decode().split("\n")[:n.value]]
    if symbols:
        return {r[0]: (int(n_l[i]), float(us[i] / n_l[i]), r[1] if len(r) > 1 else "") for i, r in enumerate(rows)}
    return {r[0]: (int(n_l[i]), float(us[i] / n_l[i])) for i, r in enumerate(rows)}


class Tables:
    """Device tables for the stage entry points (base2_convert.py:48-61)."""

    def __init__(self, tabs: dict):
        self.L = lib()
        self._keep = [_np(tabs[k], np.int64) for k in ("phi", "arrival", "log2", "exp2")]
        phi, arr, lg, ep = self._keep
        h = vp()
        check(self.L.sm_tables_create(phi.ctypes.data_as(i64p), arr.ctypes.data_as(i64p), len(arr),
                                      lg.ctypes.data_as(i64p), ep.ctypes.data_as(i64p), int(tabs["log2_768"]),
                                      int(tabs["eps40"]), ctypes.byref(h)))
        self.h = h

    def verified(self) -> bool:
        """every entry equals its defining formula (base2_convert.py:48-61), checked on the device at create"""
        v = self.L.sm_tables_verified(self.h)
        check(min(v, 0))
        return bool(v)

    def close(self):
        if getattr(self, "h", None):
            self.L.sm_tables_destroy(self.h)
            self.h = None

    __del__ = close


class Plate:
    """A plate on the device (input-major int16 [nin][nout] on the host): tile_cols > 0 lays it out for the
    one-row GEMV (.product), tile_cols == 0 as int8 MFMA byte planes for rows of lights (.product_rows)."""

    def __init__(self, w, e, b, tile_cols: int = 8):
        self.L = lib()
        w = _np(w, np.int16)
        self.nin, self.nout = w.shape
        e = _np(e, np.int32)
        b = _np(b, np.int64)
        h = vp()
        check(self.L.sm_plate_create(w.ctypes.data_as(ctypes.POINTER(ctypes.c_int16)), e.ctypes.data_as(i32p),
                                     b.ctypes.data_as(i64p), self.nin, self.nout, tile_cols, ctypes.byref(h)))
        self.h = h
        self.bytes = int(self.L.sm_plate_bytes(self.h))

    def product(self, x16_ptr: int, pile_ptr: int, grid: int = 0, stream: int = 0):
        check(self.L.sm_plate_product(self.h, x16_ptr, pile_ptr, grid, stream))

    def product_rows(self, x16_ptr: int, rows: int, pile_ptr: int, stream: int = 0):
        check(self.L.sm_plate_product_rows(self.h, x16_ptr, rows, pile_ptr, stream))

    def product_rows_noalloc(self, x16_ptr: int, rows: int, pile_ptr: int, stream: int = 0):
        """product_rows with the light planes in the library's static device scratch: no allocation on any call
        (calls that overlap on one GPU race)"""
        check(self.L.sm_plate_product_rows_noalloc(self.h, x16_ptr, rows, pile_ptr, stream))

    def product_rows_from(self, x_ptr: int, orw_ptr: int, rows: int, pile_ptr: int, stream: int = 0):
        """the light formed in the bank from int64 rows and their OR words (12 a row for nin 768, 192 for 3072)"""
        check(self.L.sm_plate_product_rows_from(self.h, x_ptr, orw_ptr, rows, pile_ptr, stream))

    def close(self):
        if getattr(self, "h", None):
            self.L.sm_plate_destroy(self.h)
            self.h = None

    __del__ = close


class stages:
    """base2.py's stage functions on device buffers (pointers to device memory; stream = hipStream_t or 0)."""

    @staticmethod
    def rshift(x, s, out, n, stream=0):
        check(lib().sm_stage_rshift(x, s, out, n, stream))

    @staticmethod
    def log2fix(t: Tables, v, out, n, stream=0):
        check(lib().sm_stage_log2fix(t.h, v, out, n, stream))

    @staticmethod
    def power(t: Tables, x, F, out, n, stream=0):
        check(lib().sm_stage_power(t.h, x, F, out, n, stream))

    @staticmethod
    def edge(t: Tables, h, out, n, stream=0):
        check(lib().sm_stage_edge(t.h, h, out, n, stream))

    @staticmethod
    def to16(X, rows, n, x16, ex, stream=0):
        check(lib().sm_stage_to16(X, rows, n, x16, ex, stream))

    @staticmethod
    def gauge_log(t: Tables, R, rows, x16, ex, LS, stream=0):
        check(lib().sm_stage_gauge_log(t.h, R, rows, x16, ex, LS, stream))

    @staticmethod
    def race(v, n, out, stream=0):
        check(lib().sm_stage_race(v, n, out, stream))

    @staticmethod
    def attend(t: Tables, qkv, k16, km, ek, v, pos, ctx, out, stream=0):
        """k16: int16 [12][ctx][64] keys (+32768 held as 32767), km: int64 [12][ctx] masks of the +32768
        dimensions, ek: int32 [12][ctx], v: int32 [12][ctx][64] (device pointers; zeroed = empty)"""
        check(lib().sm_stage_attend(t.h, qkv, k16, km, ek, v, pos, ctx, out, stream))

    @staticmethod
    def attend_split(t: Tables, qkv, k16, km, ek, v, pos, ctx, out, stream=0):
        """the same attention (same caches and result) spread over the GPU: each head's positions in chunks of 64,
        one block a chunk, as the batch-1 machine runs it from its att_split position on (ctx <= 8192)"""
        check(lib().sm_stage_attend_split(t.h, qkv, k16, km, ek, v, pos, ctx, out, stream))

    @staticmethod
    def attend_rows(t: Tables, qkv, rows, k16, km, ek, v, pos, ctx, out, stream=0):
        """the same for `rows` streams through the batched machine's kernel: qkv [rows][2304], caches stream-major
        ([rows][12][ctx][64] keys and values, [rows][12][ctx] masks and water levels), out [rows][768]"""
        check(lib().sm_stage_attend_rows(t.h, qkv, rows, k16, km, ek, v, pos, ctx, out, stream))
