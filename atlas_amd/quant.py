"""Host mirror of the reference's `atlas-quant` formats.

``Int8Tensor`` (crates/atlas-quant/src/lib.rs:32-89) and ``Int4Tensor``
(lib.rs:93-180) with the same fields, quantisation rules and packing: int8
per-row absmax / 127, int4 per-block absmax / 7 over the flattened index,
two nibbles per byte with the even element in the high nibble; scales
1.0 for all-zero rows/blocks; v * (1/scale), clamp, round half away from
zero.  Quantisation runs in the library's host code
(atlas_quantize_int8_host / atlas_quantize_int4_host); the same rules run on
the device in atlas_quantize_int8_dev / atlas_quantize_int4_dev.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import check, load

INT4_BLOCK_SIZE = 64          # lib.rs:93 default


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


@dataclass
class Int8Tensor:
    data: np.ndarray      # int8 [rows * cols]
    scales: np.ndarray    # f32 [rows]
    rows: int
    cols: int

    @staticmethod
    def quantize(t: np.ndarray) -> "Int8Tensor":
        t = np.ascontiguousarray(t, np.float32)
        if t.ndim != 2:
            raise ValueError("Int8Tensor::quantize requires 2D tensor")
        rows, cols = t.shape
        data = np.empty(rows * cols, np.int8)
        scales = np.empty(rows, np.float32)
        check(load().atlas_quantize_int8_host(_p(t), rows, cols, _p(data), _p(scales)))
        return Int8Tensor(data, scales, rows, cols)

    def dequantize(self) -> np.ndarray:
        d = self.data.reshape(self.rows, self.cols).astype(np.float32)
        return (d * self.scales[:, None]).astype(np.float32)

    def memory_bytes(self) -> int:
        return self.data.size + self.scales.size * 4

    def compression_ratio(self) -> float:
        return self.rows * self.cols * 4 / self.memory_bytes()


@dataclass
class Int4Tensor:
    data: np.ndarray      # uint8 [ceil(n / 2)]
    scales: np.ndarray    # f32 [ceil(n / block_size)]
    rows: int
    cols: int
    block_size: int

    @staticmethod
    def quantize(t: np.ndarray, block_size: int = INT4_BLOCK_SIZE) -> "Int4Tensor":
        t = np.ascontiguousarray(t, np.float32)
        if t.ndim != 2:
            raise ValueError("Int4Tensor::quantize requires 2D tensor")
        rows, cols = t.shape
        n = rows * cols
        data = np.empty((n + 1) // 2, np.uint8)
        scales = np.empty((n + block_size - 1) // block_size, np.float32)
        check(load().atlas_quantize_int4_host(_p(t), rows, cols, block_size, _p(data), _p(scales)))
        return Int4Tensor(data, scales, rows, cols, block_size)

    def dequantize(self) -> np.ndarray:
        n = self.rows * self.cols
        i = np.arange(n)
        byte = self.data[i // 2]
        nib = np.where(i % 2 == 0, byte >> 4, byte & 0x0F).astype(np.int32)
        sv = np.where(nib >= 8, nib - 16, nib).astype(np.float32)
        return (sv * self.scales[i // self.block_size]).astype(np.float32).reshape(self.rows, self.cols)

    def memory_bytes(self) -> int:
        return self.data.size + self.scales.size * 4

    def compression_ratio(self) -> float:
        return self.rows * self.cols * 4 / self.memory_bytes()
