"""Host mirror of the reference's `atlas-model` decode surface on the MI355X engine.

``ModelConfig`` (crates/atlas-model/src/lib.rs:58-329), ``SamplingConfig``
(lib.rs:1223-1295) and ``OlmoModel`` (lib.rs:1298-2009): ``reset``,
``forward_one`` / ``forward_one_gpu`` (both run the HIP engine),
``forward_one_hooked``, ``generate``, ``generate_with_sampling``,
``generate_with_sampling_hooked``, ``generate_streaming``,
``set_rng_seed``; plus ``generate_batch`` (ragged micro-batch, extension).
The engine is include/atlas_engine.h; nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence

import numpy as np

from ._lib import HOOK_FN, TOKEN_FN, AtlasError, ModelConfigC, SamplingC, check, load

W_BF16, W_INT8, W_INT4 = 1, 2, 3
T_WQ, T_WK, T_WV, T_WO, T_W_GATE, T_W_UP, T_W_DOWN = range(7)
T_ATTN_NORM, T_FFN_NORM, T_Q_NORM, T_K_NORM, T_EMBED, T_LM_HEAD, T_FINAL_NORM = range(7, 14)


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


@dataclass
class RopeYarn:
    """RopeScaling::Yarn (lib.rs:35-53)."""
    factor: float = 8.0
    orig_max_pos: int = 8192
    attn_factor: float = 1.2079441541679836
    beta_fast: float = 32.0
    beta_slow: float = 1.0


@dataclass
class ModelConfig:
    vocab_size: int
    d_model: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    ffn_hidden: int
    max_seq_len: int
    rope_theta: float = 500000.0
    rms_norm_eps: float = 1e-6
    layer_types: List[str] = field(default_factory=list)     # "sliding" / "full"
    sliding_window: Optional[int] = None
    rope_scaling: Optional[RopeYarn] = None
    eos_token_id: Optional[int] = None
    post_norm: bool = True
    qk_norm: bool = True

    def head_dim(self) -> int:
        return self.d_model // self.n_heads

    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim()

    @staticmethod
    def olmo3_actual_7b() -> "ModelConfig":
        """lib.rs:253-269 (post-norm + QK-norm), with the OLMo-3 SWA / YaRN
        settings load_model_from_dir reads from config.json (lib.rs:2367-2432):
        layers i % 4 != 3 sliding with window 4096, YaRN factor 8."""
        return ModelConfig(vocab_size=100278, d_model=4096, n_layers=32, n_heads=32,
                           n_kv_heads=32, ffn_hidden=11008, max_seq_len=4096,
                           rope_theta=500000.0, rms_norm_eps=1e-6,
                           layer_types=["full" if i % 4 == 3 else "sliding" for i in range(32)],
                           sliding_window=4096, rope_scaling=RopeYarn())

    @staticmethod
    def olmo3_1b() -> "ModelConfig":
        """lib.rs:109-126."""
        return ModelConfig(vocab_size=100352, d_model=2048, n_layers=16, n_heads=16, n_kv_heads=16,
                           ffn_hidden=8192, max_seq_len=4096, rope_theta=500000.0,
                           rms_norm_eps=1e-5)

    @staticmethod
    def llama32_1b() -> "ModelConfig":
        """lib.rs:128-145."""
        return ModelConfig(vocab_size=128256, d_model=2048, n_layers=16, n_heads=32, n_kv_heads=8,
                           ffn_hidden=8192, max_seq_len=131072, rope_theta=500000.0,
                           rms_norm_eps=1e-5)

    @staticmethod
    def smollm2_1b7() -> "ModelConfig":
        """lib.rs:148-165."""
        return ModelConfig(vocab_size=49152, d_model=2048, n_layers=24, n_heads=32, n_kv_heads=32,
                           ffn_hidden=8192, max_seq_len=8192, rope_theta=130000.0,
                           rms_norm_eps=1e-5)

    @staticmethod
    def smollm2_135m() -> "ModelConfig":
        """lib.rs:188-205."""
        return ModelConfig(vocab_size=49152, d_model=576, n_layers=30, n_heads=9, n_kv_heads=3,
                           ffn_hidden=1536, max_seq_len=8192, rope_theta=10000.0,
                           rms_norm_eps=1e-5)

    @staticmethod
    def tiny() -> "ModelConfig":
        """lib.rs:312-328."""
        return ModelConfig(vocab_size=256, d_model=64, n_layers=2, n_heads=4, n_kv_heads=2,
                           ffn_hidden=128, max_seq_len=128, rope_theta=10000.0, rms_norm_eps=1e-5)


@dataclass
class SamplingConfig:
    temperature: float = 1.0
    repetition_penalty: float = 1.0
    repetition_window: int = 64
    frequency_penalty: float = 0.0
    presence_penalty: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    min_p: float = 0.0
    suppress_initial_tokens: List[int] = field(default_factory=list)

    @staticmethod
    def greedy() -> "SamplingConfig":
        return SamplingConfig(temperature=0.0)

    @staticmethod
    def olmo3() -> "SamplingConfig":
        """lib.rs:1278-1294."""
        return SamplingConfig(temperature=0.6, repetition_penalty=1.15, repetition_window=256,
                              top_p=0.95, top_k=50, min_p=0.05, suppress_initial_tokens=[14023])


def sample_host(logits, hist: Sequence[int], step: int, cfg: SamplingConfig,
                rng_state: int):
    """One token choice of generate_with_sampling (lib.rs:1623-1711) on the
    host: returns (token, new XorShift64 state).  ``rng_state`` is the raw
    state (Rng::from_seed stores seed | 1, lib.rs:1203-1206)."""
    lg = np.ascontiguousarray(logits, np.float32)
    h = np.ascontiguousarray(list(hist) or [0], np.uint32)
    sup = np.ascontiguousarray(cfg.suppress_initial_tokens or [0], np.uint32)
    s = SamplingC(cfg.temperature, cfg.repetition_penalty, cfg.repetition_window,
                  cfg.frequency_penalty, cfg.presence_penalty, cfg.top_p, cfg.top_k, cfg.min_p,
                  sup.ctypes.data, len(cfg.suppress_initial_tokens), -1, None, 0, 0)
    st = C.c_uint64(rng_state & (2**64 - 1))
    tok = C.c_uint32(0)
    check(load().atlas_sample_host(_p(lg), lg.size, _p(h), len(hist), step, C.byref(s),
                                   C.byref(st), C.byref(tok)))
    return int(tok.value), int(st.value)


class OlmoModel:
    """Decode engine handle: weights in HBM, one captured step per token."""

    def __init__(self, cfg: ModelConfig, weight_format: int = W_BF16, int4_block: int = 32,
                 max_batch: int = 1):
        lib = load()
        self.config = cfg
        self.weight_format = weight_format
        self.eos_token_id = cfg.eos_token_id
        self.extra_stop_tokens: List[int] = []
        self._rng_seed = 0
        sl = np.zeros(cfg.n_layers, np.uint8)
        for i, t in enumerate(cfg.layer_types[:cfg.n_layers]):
            sl[i] = 1 if t == "sliding" else 0
        self._sl = sl
        y = cfg.rope_scaling
        c = ModelConfigC(cfg.vocab_size, cfg.d_model, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads,
                         cfg.ffn_hidden, cfg.max_seq_len, cfg.rope_theta, cfg.rms_norm_eps,
                         1 if y else 0, y.factor if y else 1.0, y.orig_max_pos if y else 0,
                         y.attn_factor if y else 1.0, y.beta_fast if y else 32.0,
                         y.beta_slow if y else 1.0, cfg.sliding_window or 0,
                         sl.ctypes.data, 1 if cfg.post_norm else 0, 1 if cfg.qk_norm else 0,
                         weight_format, int4_block, max_batch)
        self._h = lib.atlas_model_create(C.byref(c))
        if not self._h:
            raise AtlasError(lib.atlas_last_error_code(), lib.atlas_last_error().decode())

    def close(self):
        if getattr(self, "_h", None):
            load().atlas_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- weights -------------------------------------------------------------
    def init_random(self, seed: int) -> None:
        check(load().atlas_model_init_random(self._h, seed))

    def set_tensor(self, kind: int, layer: int, data: np.ndarray,
                   scales: Optional[np.ndarray] = None) -> None:
        data = np.ascontiguousarray(data)
        sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
        check(load().atlas_model_set_tensor(self._h, kind, layer, _p(data),
                                            None if sc is None else _p(sc)))

    def get_tensor(self, kind: int, layer: int, shape, dtype, n_scales: int = 0):
        out = np.empty(shape, dtype)
        sc = np.empty(max(n_scales, 1), np.float32) if n_scales else None
        check(load().atlas_model_get_tensor(self._h, kind, layer, _p(out),
                                            None if sc is None else _p(sc)))
        return (out, sc) if n_scales else out

    # ---- state -----------------------------------------------------------------
    def reset(self) -> None:
        """lib.rs:1389-1392."""
        check(load().atlas_model_reset(self._h))

    @property
    def pos(self) -> int:
        return load().atlas_model_pos(self._h)

    def set_kv_rows(self, layer: int, pos0: int, k, v, seq: int = 0) -> None:
        """Test helper (no reference counterpart): cache rows pos0.. of one
        layer of sequence slot seq; k, v are [n][n_kv * head_dim] f32."""
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        if k.shape != v.shape or k.ndim != 2:
            raise ValueError("set_kv_rows: k and v must be [n][kv_dim] arrays of one shape")
        check(load().atlas_model_set_kv_rows(self._h, seq, layer, pos0, k.shape[0], _p(k), _p(v)))

    def set_pos(self, pos: int) -> None:
        """Test helper: the position the next decode step writes."""
        check(load().atlas_model_set_pos(self._h, pos))

    @property
    def attn_scale(self) -> float:
        return load().atlas_model_attn_scale(self._h)

    def set_rng_seed(self, seed: int) -> None:
        """lib.rs:1961-1963; used by the next generate call."""
        self._rng_seed = seed

    def set_long_context(self, from_pos: int) -> None:
        """Position from which decode steps use the long-context attention
        path (extension; default: never, the fused step is faster at every
        measured context)."""
        check(load().atlas_model_set_long_context(self._h, from_pos))

    def prefill(self, tokens: Sequence[int]) -> None:
        """Feed tokens at the current position without choosing, several per
        step (extension; the reference feeds one per forward)."""
        t = np.ascontiguousarray(list(tokens) or [0], np.uint32)
        check(load().atlas_model_prefill(self._h, _p(t), len(tokens)))

    def set_prefill_chunk(self, chunk: int) -> None:
        """Tokens per prefill step, 1..1024 (default 1024; 1 = token by token; above
        16 needs GEMM inner dims that are multiples of 128, else 16 is used)."""
        check(load().atlas_model_set_prefill_chunk(self._h, chunk))

    def use_graph(self, enable: bool) -> None:
        check(load().atlas_model_use_graph(self._h, 1 if enable else 0))

    @property
    def stream(self) -> int:
        return load().atlas_model_stream(self._h) or 0

    def weight_bytes(self) -> int:
        return load().atlas_model_weight_bytes(self._h)

    # ---- forward ---------------------------------------------------------------
    def forward_one_gpu(self, token: int) -> np.ndarray:
        """lib.rs:1463-1505: logits [vocab] downloaded to the host."""
        out = np.empty(self.config.vocab_size, np.float32)
        check(load().atlas_model_forward_one(self._h, token, _p(out)))
        return out

    forward_one = forward_one_gpu

    def forward_one_hooked(self, token: int, hook: Callable[[int, np.ndarray], Optional[float]]):
        """lib.rs:1425-1445: hook(layer_idx, hidden) after every layer."""
        d = self.config.d_model

        def _cb(user, li, hidden, n, delta):
            h = np.ctypeslib.as_array(hidden, shape=(n,)).copy()
            r = hook(li, h)
            return 0 if r is None else 1

        cb = HOOK_FN(_cb)
        out = np.empty(self.config.vocab_size, np.float32)
        check(load().atlas_model_forward_one_hooked(self._h, token, _p(out), None, cb, None))
        return out

    def forward_one_hidden(self, token: int):
        """Logits plus the post-residual hidden state after every layer."""
        out = np.empty(self.config.vocab_size, np.float32)
        hid = np.empty((self.config.n_layers, self.config.d_model), np.float32)
        check(load().atlas_model_forward_one_hooked(self._h, token, _p(out), _p(hid),
                                                    HOOK_FN(0), None))
        return out, hid

    # ---- generation --------------------------------------------------------------
    def _sampling(self, s: SamplingConfig, keep: list):
        sup = np.ascontiguousarray(s.suppress_initial_tokens or [0], np.uint32)
        ex = np.ascontiguousarray(self.extra_stop_tokens or [0], np.uint32)
        keep += [sup, ex]
        eos = -1 if self.eos_token_id is None else int(self.eos_token_id)
        return SamplingC(s.temperature, s.repetition_penalty, s.repetition_window,
                         s.frequency_penalty, s.presence_penalty, s.top_p, s.top_k, s.min_p,
                         sup.ctypes.data, len(s.suppress_initial_tokens), eos, ex.ctypes.data,
                         len(self.extra_stop_tokens), self._rng_seed)

    def generate(self, prompt: Sequence[int], max_new: int, temperature: float) -> List[int]:
        """lib.rs:1574-1580."""
        return self.generate_with_sampling(prompt, max_new, SamplingConfig(temperature=temperature))

    def generate_with_sampling(self, prompt: Sequence[int], max_new: int,
                               cfg: SamplingConfig) -> List[int]:
        """lib.rs:1599-1732."""
        keep: list = []
        s = self._sampling(cfg, keep)
        pr = np.ascontiguousarray(list(prompt) or [0], np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        n = C.c_int(0)
        check(load().atlas_model_generate(self._h, _p(pr), len(prompt), max_new, C.byref(s),
                                          _p(out), C.byref(n)))
        return [int(t) for t in out[:n.value]]

    def generate_with_sampling_hooked(self, prompt, max_new, cfg: SamplingConfig,
                                      hook: Callable[[int, np.ndarray], Optional[float]]):
        """lib.rs:1745-1846: (tokens, [(token, total_delta, layers_fired)])."""
        keep: list = []
        s = self._sampling(cfg, keep)

        def _cb(user, li, hidden, n, delta):
            h = np.ctypeslib.as_array(hidden, shape=(n,))
            r = hook(li, h)
            if r is None:
                return 0
            delta[0] = float(r)
            return 1

        cb = HOOK_FN(_cb)
        pr = np.ascontiguousarray(list(prompt) or [0], np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        tot = np.empty(max(max_new, 1), np.float32)
        fired = np.empty(max(max_new, 1), np.uint32)
        n = C.c_int(0)
        check(load().atlas_model_generate_hooked(self._h, _p(pr), len(prompt), max_new, C.byref(s),
                                                 cb, None, _p(out), _p(tot), _p(fired), C.byref(n)))
        toks = [int(t) for t in out[:n.value]]
        return toks, [(toks[i], float(tot[i]), int(fired[i])) for i in range(n.value)]

    def generate_streaming(self, prompt, max_new, cfg: SamplingConfig,
                           on_token: Callable[[int], bool]) -> List[int]:
        """lib.rs:1853-1955: on_token returning False stops early."""
        keep: list = []
        s = self._sampling(cfg, keep)
        got: List[int] = []

        def _cb(user, tok):
            got.append(int(tok))
            return 1 if on_token(int(tok)) else 0

        cb = TOKEN_FN(_cb)
        pr = np.ascontiguousarray(list(prompt) or [0], np.uint32)
        n = C.c_int(0)
        check(load().atlas_model_generate_streaming(self._h, _p(pr), len(prompt), max_new,
                                                    C.byref(s), cb, None, C.byref(n)))
        return got[:n.value]

    def generate_batch(self, prompts: Sequence[Sequence[int]], max_new: int,
                       cfg: Optional[SamplingConfig] = None) -> List[List[int]]:
        """Ragged micro-batch of independent sequences (extension)."""
        cfg = cfg or SamplingConfig.greedy()
        keep: list = []
        s = self._sampling(cfg, keep)
        lens = np.ascontiguousarray([len(p) for p in prompts], np.int32)
        flat = np.ascontiguousarray([t for p in prompts for t in p] or [0], np.uint32)
        out = np.zeros((len(prompts), max(max_new, 1)), np.uint32)
        nout = np.zeros(len(prompts), np.int32)
        check(load().atlas_model_generate_batch(self._h, _p(flat), _p(lens), len(prompts), max_new,
                                                C.byref(s), _p(out), _p(nout)))
        return [[int(t) for t in out[i, :nout[i]]] for i in range(len(prompts))]

    def decode_greedy(self, first_token: int, n_steps: int) -> np.ndarray:
        """Replays the captured step n_steps times with no host sync in between."""
        toks = np.empty(max(n_steps, 1), np.uint32)
        check(load().atlas_model_decode_greedy(self._h, first_token, n_steps, _p(toks)))
        return toks[:n_steps]

    def decode_greedy_timed(self, first_token: int, n_steps: int):
        """decode_greedy plus each step's GPU time in ms (HIP events on the
        engine stream after every step): (tokens, step_ms)."""
        toks = np.empty(max(n_steps, 1), np.uint32)
        ms = np.zeros(max(n_steps, 1), np.float32)
        check(load().atlas_model_decode_greedy_timed(self._h, first_token, n_steps, _p(toks), _p(ms)))
        return toks[:n_steps], ms[:n_steps]
