"""Checkpoint loading: the reference's ``SafetensorsFile``, ``f16_to_f32``,
``patch_config_from_hf_json``, ``load_model_from_safetensors`` and
``load_model_from_dir`` (crates/atlas-model/src/lib.rs:2048-2570) over the
native loader (include/atlas_loader.h).

Parsing, name mapping and architecture detection run in the library (C++);
the weights go from a memory map through pinned buffers to the device, which
converts them into the model's weight format.  This module only wraps the
calls and returns numpy arrays / ``OlmoModel`` objects.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import os
import struct
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import numpy as np

from ._lib import AtlasError, ModelConfigC, check, load
from .model import W_BF16, ModelConfig, OlmoModel, RopeYarn


@dataclass
class TensorDesc:
    """lib.rs:2051-2061."""
    name: str
    dtype: str
    shape: List[int]
    offsets: Tuple[int, int]


class SafetensorsFile:
    """lib.rs:2063-2241: header parsed once; tensor data read on demand."""

    def __init__(self, handle):
        self._h = handle

    @staticmethod
    def open(path: str) -> "SafetensorsFile":
        h = C.c_void_p()
        check(load().atlas_st_open(os.fsencode(path), C.byref(h)))
        return SafetensorsFile(h)

    @staticmethod
    def from_bytes(data: bytes) -> "SafetensorsFile":
        h = C.c_void_p()
        buf = C.create_string_buffer(bytes(data), len(data)) if data else None
        check(load().atlas_st_from_bytes(buf, len(data), C.byref(h)))
        return SafetensorsFile(h)

    def close(self) -> None:
        if getattr(self, "_h", None):
            load().atlas_st_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return load().atlas_st_count(self._h)

    def len(self) -> int:
        return len(self)

    def is_empty(self) -> bool:
        return len(self) == 0

    def _desc(self, i: int) -> TensorDesc:
        name, dtype = C.c_char_p(), C.c_char_p()
        nd, shape = C.c_int(), C.POINTER(C.c_uint64)()
        off = (C.c_uint64 * 2)()
        check(load().atlas_st_desc(self._h, i, C.byref(name), C.byref(dtype), C.byref(nd),
                                   C.byref(shape), off))
        return TensorDesc(name.value.decode(), dtype.value.decode(),
                          [int(shape[k]) for k in range(nd.value)], (int(off[0]), int(off[1])))

    @property
    def tensors(self) -> List[TensorDesc]:
        return [self._desc(i) for i in range(len(self))]

    def tensor_names(self) -> List[str]:
        return [t.name for t in self.tensors]

    def contains(self, name: str) -> bool:
        return load().atlas_st_find(self._h, name.encode()) >= 0

    def get_desc(self, name: str) -> Optional[TensorDesc]:
        i = load().atlas_st_find(self._h, name.encode())
        return None if i < 0 else self._desc(i)

    def get_f32(self, name: str) -> np.ndarray:
        n = C.c_size_t()
        lib = load()
        check(lib.atlas_st_get_f32(self._h, name.encode(), None, 0, C.byref(n)))
        out = np.empty(n.value, np.float32)
        check(lib.atlas_st_get_f32(self._h, name.encode(), out.ctypes.data_as(C.c_void_p),
                                   out.size, C.byref(n)))
        return out

    def get_bf16(self, name: str) -> np.ndarray:
        n = C.c_size_t()
        lib = load()
        check(lib.atlas_st_get_bf16(self._h, name.encode(), None, 0, C.byref(n)))
        out = np.empty(n.value, np.uint16)
        check(lib.atlas_st_get_bf16(self._h, name.encode(), out.ctypes.data_as(C.c_void_p),
                                    out.size, C.byref(n)))
        return out

    @staticmethod
    def build_f32(tensors: Sequence[Tuple[str, Sequence[int], Sequence[float]]]) -> bytes:
        """lib.rs:2152-2185: F32 tensors in the given order, offsets packed,
        header written without whitespace."""
        data = bytearray()
        entries = []
        for name, shape, values in tensors:
            start = len(data)
            data += np.asarray(values, dtype="<f4").tobytes()
            entries.append(f'"{name}":{{"dtype":"F32","shape":[{",".join(str(int(s)) for s in shape)}],'
                           f'"data_offsets":[{start},{len(data)}]}}')
        header = ("{" + ",".join(entries) + "}").encode()
        return struct.pack("<Q", len(header)) + header + bytes(data)


def f16_to_f32(h: int) -> float:
    """lib.rs:2243-2263."""
    return float(load().atlas_f16_to_f32(h & 0xFFFF))


# ---- configuration -----------------------------------------------------------

def _to_c(cfg: ModelConfig, weight_format: int, int4_block: int, max_batch: int, keep: list):
    sl = np.zeros(max(cfg.n_layers, 1), np.uint8)
    for i, t in enumerate(cfg.layer_types[:cfg.n_layers]):
        sl[i] = 1 if t == "sliding" else 0
    keep.append(sl)
    y = cfg.rope_scaling
    return ModelConfigC(cfg.vocab_size, cfg.d_model, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads,
                        cfg.ffn_hidden, cfg.max_seq_len, cfg.rope_theta, cfg.rms_norm_eps,
                        1 if y else 0, y.factor if y else 1.0, y.orig_max_pos if y else 0,
                        y.attn_factor if y else 1.0, y.beta_fast if y else 32.0,
                        y.beta_slow if y else 1.0, cfg.sliding_window or 0, sl.ctypes.data,
                        1 if cfg.post_norm else 0, 1 if cfg.qk_norm else 0, weight_format,
                        int4_block, max_batch)


def _from_c(c: ModelConfigC, base: ModelConfig) -> ModelConfig:
    types = list(base.layer_types)
    if c.layer_sliding:
        p = C.cast(c.layer_sliding, C.POINTER(C.c_uint8))
        types = ["sliding" if p[i] else "full" for i in range(c.n_layers)]
    y = RopeYarn(c.yarn_factor, c.yarn_orig_max_pos, c.yarn_attn_factor, c.yarn_beta_fast,
                 c.yarn_beta_slow) if c.yarn else None
    return dataclasses.replace(base, vocab_size=c.vocab, d_model=c.d_model, n_layers=c.n_layers,
                               n_heads=c.n_heads, n_kv_heads=c.n_kv_heads,
                               ffn_hidden=c.ffn_hidden, max_seq_len=c.max_seq,
                               rope_theta=c.rope_theta, rms_norm_eps=c.rms_eps,
                               layer_types=types, sliding_window=c.sliding_window or None,
                               rope_scaling=y, post_norm=bool(c.post_norm),
                               qk_norm=bool(c.qk_norm))


def patch_config_from_hf_json(cfg: ModelConfig, config_path: str) -> ModelConfig:
    """lib.rs:2367-2432: a copy of ``cfg`` with layer_types, sliding_window,
    rope_scaling (YaRN), rope_theta, rms_norm_eps and eos_token_id taken from
    the file where present."""
    keep: list = []
    c = _to_c(cfg, W_BF16, 32, 1, keep)
    cap = 4096
    types = np.zeros(cap, np.uint8)
    n_types, eos = C.c_int(-1), C.c_int64(-1)
    check(load().atlas_config_patch_hf_json(os.fsencode(config_path), C.byref(c),
                                            types.ctypes.data_as(C.c_void_p), cap,
                                            C.byref(n_types), C.byref(eos)))
    c.layer_sliding = None
    out = _from_c(c, cfg)
    if n_types.value >= 0:
        if n_types.value > cap:
            raise AtlasError(-1, f"config.json: {n_types.value} layer_types exceed {cap}")
        out.layer_types = ["sliding" if t else "full" for t in types[:n_types.value]]
    if eos.value >= 0:
        out.eos_token_id = int(eos.value)
    return out


# ---- models --------------------------------------------------------------------

def _wrap(h, cfg: ModelConfig, weight_format: int, eos: Optional[int]) -> OlmoModel:
    c = ModelConfigC()
    check(load().atlas_model_get_config(h, C.byref(c)))
    m = OlmoModel.__new__(OlmoModel)
    m._h = h
    m.config = _from_c(c, cfg)
    if eos is not None:
        m.config.eos_token_id = eos
    m.weight_format = weight_format
    m.eos_token_id = m.config.eos_token_id
    m.extra_stop_tokens = []
    m._rng_seed = 0
    m._sl = None
    return m


def load_model_from_safetensors(path: str, cfg: ModelConfig, weight_format: int = W_BF16,
                                int4_block: int = 32, max_batch: int = 1) -> OlmoModel:
    """lib.rs:2283-2359.  ``weight_format`` picks the device residency: bf16
    (bf16 tensors bit-exact, f32/f16 truncated) or int8 / int4 quantised on
    the device by the atlas-quant rules."""
    keep: list = []
    c = _to_c(cfg, weight_format, int4_block, max_batch, keep)
    h = C.c_void_p()
    check(load().atlas_model_load_safetensors(os.fsencode(path), C.byref(c), C.byref(h)))
    return _wrap(h, cfg, weight_format, None)


def load_model_from_dir(dir_path: str, cfg: ModelConfig, weight_format: int = W_BF16,
                        int4_block: int = 32, max_batch: int = 1) -> OlmoModel:
    """lib.rs:2437-2570: config.json overlay, then the shards of
    model.safetensors.index.json or model.safetensors."""
    keep: list = []
    c = _to_c(cfg, weight_format, int4_block, max_batch, keep)
    h, eos = C.c_void_p(), C.c_int64(-1)
    check(load().atlas_model_load_dir(os.fsencode(dir_path), C.byref(c), C.byref(h),
                                      C.byref(eos)))
    return _wrap(h, cfg, weight_format, int(eos.value) if eos.value >= 0 else None)
