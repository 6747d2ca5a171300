"""CPU oracle for the decode hot path -- TEST INFRASTRUCTURE ONLY.

A ctypes wrapper over ``oracle/_build/liboracle.so`` (built from
``oracle/oracle.c`` by ``oracle/Makefile``), a plain-C restatement of the
reference's CPU decode path (crates/atlas-quant/src/lib.rs:43-168 and
crates/atlas-model/src/lib.rs:335-1732; see oracle.c for the line map).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker or the
timed CPU baseline.  The product package ``atlas_amd`` never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle.so")

F32, BF16, INT8, INT4 = 0, 1, 2, 3


def build() -> str:
    """Compile the oracle with its Makefile (gcc, seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        _lib = C.CDLL(_SO)
        _declare(_lib)
    return _lib


class Mat(C.Structure):
    _fields_ = [("fmt", C.c_int), ("data", C.c_void_p), ("scales", C.c_void_p),
                ("rows", C.c_int64), ("cols", C.c_int64), ("block", C.c_int64)]


class RopeScaling(C.Structure):
    _fields_ = [("yarn", C.c_int), ("factor", C.c_float), ("orig_max_pos", C.c_int),
                ("attn_factor", C.c_float), ("beta_fast", C.c_float),
                ("beta_slow", C.c_float)]


class Config(C.Structure):
    _fields_ = [("vocab", C.c_int), ("d_model", C.c_int), ("n_layers", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("ffn_hidden", C.c_int),
                ("max_seq", C.c_int), ("rope_theta", C.c_float), ("rms_eps", C.c_float),
                ("rope", RopeScaling), ("sliding_window", C.c_int),
                ("layer_sliding", C.c_void_p), ("post_norm", C.c_int)]


class Layer(C.Structure):
    _fields_ = [("wq", Mat), ("wk", Mat), ("wv", Mat), ("wo", Mat),
                ("w_gate", Mat), ("w_up", Mat), ("w_down", Mat),
                ("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p),
                ("q_norm", C.c_void_p), ("k_norm", C.c_void_p)]


class Sampling(C.Structure):
    _fields_ = [("temperature", C.c_float), ("repetition_penalty", C.c_float),
                ("repetition_window", C.c_int), ("frequency_penalty", C.c_float),
                ("presence_penalty", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int),
                ("min_p", C.c_float), ("suppress", C.c_void_p), ("n_suppress", C.c_int)]


def sampling(temperature=1.0, top_p=1.0, top_k=0, min_p=0.0, repetition_penalty=1.0,
             repetition_window=64, frequency_penalty=0.0, presence_penalty=0.0, suppress=()):
    """A Sampling struct; the suppress array is kept alive on the struct."""
    su = np.ascontiguousarray(list(suppress) or [0], np.uint32)
    s = Sampling(temperature, repetition_penalty, repetition_window, frequency_penalty,
                 presence_penalty, top_p, top_k, min_p, su.ctypes.data, len(suppress))
    s._keep = su
    return s


def _declare(L):
    P, I, I64, F, U64, SZ = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_uint64, C.c_size_t
    sig = {
        "orc_splitmix64_at": (U64, [U64, U64]),
        "orc_fill_normal": (None, [P, SZ, U64, F, F]),
        "orc_fill_uniform": (None, [P, SZ, U64, F, F]),
        "orc_bf16_from_f32": (None, [P, P, SZ]),
        "orc_bf16_to_f32": (None, [P, P, SZ]),
        "orc_int8_quantize": (None, [P, SZ, SZ, P, P]),
        "orc_int8_dequantize": (None, [P, P, SZ, SZ, P]),
        "orc_int4_quantize": (None, [P, SZ, SZ, SZ, P, P]),
        "orc_int4_dequantize": (None, [P, P, SZ, SZ, SZ, P]),
        "orc_mat_row": (None, [C.POINTER(Mat), I64, P]),
        "orc_linear": (None, [C.POINTER(Mat), P, P]),
        "orc_linear_rows": (None, [C.POINTER(Mat), P, P, I64, I64, I]),
        "orc_linear_batch": (None, [C.POINTER(Mat), P, P, I]),
        "orc_rmsnorm": (None, [P, P, I, F]),
        "orc_silu": (F, [F]),
        "orc_softmax": (None, [P, I]),
        "orc_qk_norm": (None, [P, P, I, I, F]),
        "orc_add": (None, [P, P, I]),
        "orc_rope_tables": (None, [I, I, F, C.POINTER(RopeScaling), P, P, P]),
        "orc_rope_apply": (None, [P, I, P, P]),
        "orc_attention": (None, [P, P, P, P, I, I, I, I, F, I]),
        "orc_model_new": (P, [C.POINTER(Config), C.POINTER(Mat), P, P, C.POINTER(Mat), I]),
        "orc_model_new_slots": (P, [C.POINTER(Config), C.POINTER(Mat), P, P,
                                    C.POINTER(Mat), I, I]),
        "orc_model_free": (None, [P]),
        "orc_model_reset": (None, [P]),
        "orc_model_pos": (I, [P]),
        "orc_model_attn_scale": (F, [P]),
        "orc_model_forward_one": (None, [P, C.c_uint32, P, P]),
        "orc_model_select_slot": (None, [P, I]),
        "orc_model_set_kv_rows": (I, [P, I, I, I, P, P]),
        "orc_model_set_pos": (I, [P, I]),
        "orc_argmax": (I, [P, I]),
        "orc_repetition_penalty": (None, [P, I, P, I, F]),
        "orc_generate_greedy": (I, [P, P, I, I, P, I, F, I, I64, P, I, P]),
        "orc_rng_next": (F, [C.POINTER(U64)]),
        "orc_frequency_penalty": (None, [P, I, P, P, I, F]),
        "orc_presence_penalty": (None, [P, I, P, I, F]),
        "orc_top_k": (None, [P, I, I]),
        "orc_top_p": (None, [P, I, F]),
        "orc_min_p": (None, [P, I, F]),
        "orc_sample_from_probs": (I, [P, I, F]),
        "orc_sample_step": (I, [P, I, P, I, I, C.POINTER(Sampling), C.POINTER(U64)]),
        "orc_generate_sampled": (I, [P, P, I, I, C.POINTER(Sampling), U64, I64, P, I, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


# ---- generator -------------------------------------------------------------

def normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_normal(_p(out), n, seed & (2**64 - 1), mean, std)
    return out


def uniform(n: int, seed: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_uniform(_p(out), n, seed & (2**64 - 1), lo, hi)
    return out


# ---- formats -----------------------------------------------------------------

def bf16_from_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_bf16_from_f32(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.uint16)
    out = np.empty(x.shape, np.float32)
    lib().orc_bf16_to_f32(_p(x), _p(out), x.size)
    return out


def int8_quantize(w: np.ndarray):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    data = np.empty((rows, cols), np.int8)
    scales = np.empty(rows, np.float32)
    lib().orc_int8_quantize(_p(w), rows, cols, _p(data), _p(scales))
    return data, scales


def int8_dequantize(data: np.ndarray, scales: np.ndarray) -> np.ndarray:
    rows, cols = data.shape
    out = np.empty((rows, cols), np.float32)
    lib().orc_int8_dequantize(_p(np.ascontiguousarray(data)), _p(np.ascontiguousarray(scales)),
                              rows, cols, _p(out))
    return out


def int4_quantize(w: np.ndarray, block: int):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    n = rows * cols
    data = np.empty((n + 1) // 2, np.uint8)
    scales = np.empty((n + block - 1) // block, np.float32)
    lib().orc_int4_quantize(_p(w), rows, cols, block, _p(data), _p(scales))
    return data, scales


def int4_dequantize(data, scales, rows, cols, block) -> np.ndarray:
    out = np.empty((rows, cols), np.float32)
    lib().orc_int4_dequantize(_p(np.ascontiguousarray(data)), _p(np.ascontiguousarray(scales)),
                              rows, cols, block, _p(out))
    return out


# ---- matrices ----------------------------------------------------------------

class MatView:
    """Keeps numpy storage alive next to the C view struct."""

    def __init__(self, fmt, data, rows, cols, scales=None, block=0):
        self.fmt, self.rows, self.cols, self.block = fmt, rows, cols, block
        self.data = np.ascontiguousarray(data)
        self.scales = None if scales is None else np.ascontiguousarray(scales, np.float32)
        self.c = Mat(fmt, self.data.ctypes.data,
                     0 if self.scales is None else self.scales.ctypes.data,
                     rows, cols, block)

    @staticmethod
    def f32(w):
        w = np.ascontiguousarray(w, np.float32)
        return MatView(F32, w, w.shape[0], w.shape[1])

    @staticmethod
    def bf16(bits, rows, cols):
        return MatView(BF16, np.ascontiguousarray(bits, np.uint16), rows, cols)

    @staticmethod
    def int8(data, scales):
        return MatView(INT8, data, data.shape[0], data.shape[1], scales)

    @staticmethod
    def int4(data, scales, rows, cols, block):
        return MatView(INT4, data, rows, cols, scales, block)


def linear(m: MatView, x: np.ndarray, threads: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(m.rows, np.float32)
    lib().orc_linear_rows(C.byref(m.c), _p(x), _p(y), 0, m.rows, threads)
    return y


def linear_batch(m: MatView, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    n = x.shape[0]
    y = np.empty((n, m.rows), np.float32)
    lib().orc_linear_batch(C.byref(m.c), _p(x), _p(y), n)
    return y


def rmsnorm(x, w, eps):
    x = np.array(x, np.float32, copy=True)
    w = np.ascontiguousarray(w, np.float32)
    lib().orc_rmsnorm(_p(x), _p(w), x.size, eps)
    return x


def silu(x: float) -> float:
    return lib().orc_silu(x)


def softmax(x):
    x = np.array(x, np.float32, copy=True)
    lib().orc_softmax(_p(x), x.size)
    return x


def qk_norm(x, w, n_heads, head_dim, eps=1e-6):
    x = np.array(x, np.float32, copy=True)
    lib().orc_qk_norm(_p(x), _p(np.ascontiguousarray(w, np.float32)), n_heads, head_dim, eps)
    return x


def rope_tables(head_dim, max_seq, theta, yarn=None):
    """yarn: None or dict(factor, orig_max_pos, attn_factor, beta_fast, beta_slow)."""
    sc = RopeScaling(0, 1.0, 0, 1.0, 32.0, 1.0)
    if yarn:
        sc = RopeScaling(1, yarn["factor"], yarn["orig_max_pos"], yarn["attn_factor"],
                         yarn["beta_fast"], yarn["beta_slow"])
    half = head_dim // 2
    cos = np.empty((max_seq, half), np.float32)
    sin = np.empty((max_seq, half), np.float32)
    freqs = np.empty(half, np.float32)
    lib().orc_rope_tables(head_dim, max_seq, theta, C.byref(sc), _p(cos), _p(sin), _p(freqs))
    return cos, sin, freqs


def rope_apply(x, cos_row, sin_row):
    x = np.array(x, np.float32, copy=True)
    lib().orc_rope_apply(_p(x), x.size, _p(np.ascontiguousarray(cos_row, np.float32)),
                         _p(np.ascontiguousarray(sin_row, np.float32)))
    return x


def attention(q, k_cache, v_cache, n_heads, n_kv, head_dim, pos, scale, window):
    q = np.ascontiguousarray(q, np.float32)
    out = np.empty(n_heads * head_dim, np.float32)
    lib().orc_attention(_p(q), _p(np.ascontiguousarray(k_cache, np.float32)),
                        _p(np.ascontiguousarray(v_cache, np.float32)), _p(out),
                        n_heads, n_kv, head_dim, pos, scale, window)
    return out


def argmax(x) -> int:
    x = np.ascontiguousarray(x, np.float32)
    return lib().orc_argmax(_p(x), x.size)


def repetition_penalty(logits, toks, theta):
    logits = np.array(logits, np.float32, copy=True)
    t = np.ascontiguousarray(toks, np.uint32)
    lib().orc_repetition_penalty(_p(logits), logits.size, _p(t), t.size, theta)
    return logits


# ---- sampling ----------------------------------------------------------------

class Rng:
    """Rng::from_seed / next_f32 (XorShift64), lib.rs:1203-1214."""

    def __init__(self, seed: int):
        self.state = C.c_uint64((seed | 1) & (2**64 - 1))

    def next_f32(self) -> float:
        return lib().orc_rng_next(C.byref(self.state))


def frequency_penalty(logits, toks, counts, penalty):
    logits = np.array(logits, np.float32, copy=True)
    t = np.ascontiguousarray(toks, np.uint32)
    c = np.ascontiguousarray(counts, np.uint32)
    lib().orc_frequency_penalty(_p(logits), logits.size, _p(t), _p(c), t.size, penalty)
    return logits


def presence_penalty(logits, toks, penalty):
    logits = np.array(logits, np.float32, copy=True)
    t = np.ascontiguousarray(toks, np.uint32)
    lib().orc_presence_penalty(_p(logits), logits.size, _p(t), t.size, penalty)
    return logits


def _filter(fn, logits, arg):
    logits = np.array(logits, np.float32, copy=True)
    getattr(lib(), fn)(_p(logits), logits.size, arg)
    return logits


def top_k(logits, k):
    return _filter("orc_top_k", logits, k)


def top_p(logits, p):
    return _filter("orc_top_p", logits, p)


def min_p(logits, mp):
    return _filter("orc_min_p", logits, mp)


def sample_from_probs(probs, rand) -> int:
    p = np.ascontiguousarray(probs, np.float32)
    return lib().orc_sample_from_probs(_p(p), p.size, rand)


def sample_step(logits, hist, step, s: Sampling, rng: Rng) -> int:
    lg = np.ascontiguousarray(logits, np.float32)
    h = np.ascontiguousarray(list(hist) or [0], np.uint32)
    return lib().orc_sample_step(_p(lg), lg.size, _p(h), len(hist), step, C.byref(s),
                                 C.byref(rng.state))


# ---- model ---------------------------------------------------------------------

class Model:
    """OlmoModel CPU path over caller-held weights (MatView / numpy arrays).

    ``cfg`` is a dict with the ModelConfig fields; ``weights`` a dict:
    embed (MatView), lm_head (MatView), final_norm (f32), layers: list of dicts
    with wq wk wv wo w_gate w_up w_down (MatView), attn_norm, ffn_norm,
    q_norm, k_norm (f32 or None).
    """

    def __init__(self, cfg: dict, weights: dict, threads: int = 1, slots: int = 1):
        self._keep = []
        y = cfg.get("yarn")
        sc = RopeScaling(0, 1.0, 0, 1.0, 32.0, 1.0)
        if y:
            sc = RopeScaling(1, y["factor"], y["orig_max_pos"], y["attn_factor"],
                             y["beta_fast"], y["beta_slow"])
        sl = np.ascontiguousarray(cfg.get("layer_sliding") or [0] * cfg["n_layers"], np.uint8)
        self._keep.append(sl)
        self.cfg = Config(cfg["vocab"], cfg["d_model"], cfg["n_layers"], cfg["n_heads"],
                          cfg["n_kv_heads"], cfg["ffn_hidden"], cfg["max_seq"],
                          cfg["rope_theta"], cfg["rms_eps"], sc,
                          cfg.get("sliding_window") or 0, sl.ctypes.data,
                          1 if cfg.get("post_norm", True) else 0)
        self.vocab = cfg["vocab"]
        self.d = cfg["d_model"]
        self.n_layers = cfg["n_layers"]
        layers = (Layer * cfg["n_layers"])()

        def vec(a):
            if a is None:
                return 0
            a = np.ascontiguousarray(a, np.float32)
            self._keep.append(a)
            return a.ctypes.data

        for i, lw in enumerate(weights["layers"]):
            for k in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
                self._keep.append(lw[k])
                setattr(layers[i], k, lw[k].c)
            layers[i].attn_norm = vec(lw["attn_norm"])
            layers[i].ffn_norm = vec(lw["ffn_norm"])
            layers[i].q_norm = vec(lw.get("q_norm"))
            layers[i].k_norm = vec(lw.get("k_norm"))
        self._layers = layers
        self._keep += [weights["embed"], weights["lm_head"]]
        fn = vec(weights["final_norm"])
        self.h = lib().orc_model_new_slots(C.byref(self.cfg), C.byref(weights["embed"].c),
                                           C.cast(layers, C.c_void_p), fn,
                                           C.byref(weights["lm_head"].c), threads, slots)

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_model_free(self.h)
            self.h = None

    def reset(self):
        lib().orc_model_reset(self.h)

    def select(self, slot: int):
        lib().orc_model_select_slot(self.h, slot)

    @property
    def pos(self) -> int:
        return lib().orc_model_pos(self.h)

    def set_kv_rows(self, layer: int, pos0: int, k, v) -> None:
        """Test seeding: cache rows pos0.. of one layer (k, v: [n][n_kv*hd] f32)."""
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        assert k.shape == v.shape and k.ndim == 2
        if lib().orc_model_set_kv_rows(self.h, layer, pos0, k.shape[0], _p(k), _p(v)) != 0:
            raise ValueError("set_kv_rows: rows outside the cache")

    def set_pos(self, pos: int) -> None:
        if lib().orc_model_set_pos(self.h, pos) != 0:
            raise ValueError(f"set_pos: {pos} outside the cache")

    @property
    def attn_scale(self) -> float:
        return lib().orc_model_attn_scale(self.h)

    def forward_one(self, token: int, hidden: bool = False):
        logits = np.empty(self.vocab, np.float32)
        hid = np.empty((self.n_layers, self.d), np.float32) if hidden else None
        lib().orc_model_forward_one(self.h, token, _p(logits), _p(hid) if hidden else None)
        return (logits, hid) if hidden else logits

    def generate_greedy(self, prompt, max_new, suppress=(), rep_penalty=1.0,
                        rep_window=64, eos=None, extra_stop=()):
        pr = np.ascontiguousarray(prompt, np.uint32)
        su = np.ascontiguousarray(list(suppress) or [0], np.uint32)
        ex = np.ascontiguousarray(list(extra_stop) or [0], np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        n = lib().orc_generate_greedy(self.h, _p(pr), pr.size, max_new, _p(su), len(suppress),
                                      rep_penalty, rep_window, -1 if eos is None else eos,
                                      _p(ex), len(extra_stop), _p(out))
        return [int(t) for t in out[:n]]

    def generate_sampled(self, prompt, max_new, s: Sampling, seed: int, eos=None,
                         extra_stop=()):
        pr = np.ascontiguousarray(prompt, np.uint32)
        ex = np.ascontiguousarray(list(extra_stop) or [0], np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        n = lib().orc_generate_sampled(self.h, _p(pr), pr.size, max_new, C.byref(s), seed,
                                       -1 if eos is None else eos, _p(ex), len(extra_stop),
                                       _p(out))
        return [int(t) for t in out[:n]]
