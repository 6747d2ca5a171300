"""Host mirror of the reference's `atlas-tensor` GPU surface.

Same names and argument meaning as crates/atlas-tensor/src/lib.rs:
``GpuBuf`` (178-237), ``GpuBufBf16`` (242-280), ``GpuBufKind`` (284-292),
``GpuMatrix`` (309-436), ``GpuVec`` (460-556), ``GpuRopeTables`` (662-693),
``GpuKvCache`` (701-785) and the free functions (97-142, 570-654), over the
C ABI of include/atlas_kernels.h.  Extensions: ``GpuBufKind.INT8`` /
``GpuBufKind.INT4`` and ``GpuMatrix.upload_int8`` / ``upload_int4`` for the
dequant-fused GEMVs.

Error behaviour follows the reference's Option/bool contract where it has
one (allocation -> None, ``sgemm`` -> False when no device is present), but
there is no CPU compute fallback: an op called on a vector that is not on the
GPU raises ``AtlasError`` instead of silently computing on the host.
"""
from __future__ import annotations

import ctypes as C
from enum import Enum
from typing import Optional

import numpy as np

from ._lib import AtlasError, check, check_void, load


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def cuda_available() -> bool:
    """lib.rs:129-135 -- a HIP device is reachable."""
    return load().atlas_cuda_available() != 0


def cuda_device_count() -> int:
    """lib.rs:137-142."""
    return load().atlas_cuda_device_count()


def device_sync() -> None:
    """lib.rs:97-100 -- drain the device."""
    load().atlas_sync()
    check_void()


class _DevMem:
    """Owns one device allocation (RAII like GpuBuf's Drop, lib.rs:226-237)."""

    def __init__(self, nbytes: int, sync_alloc: bool):
        self.ptr = None
        self.nbytes = nbytes
        self._sync = sync_alloc
        p = C.c_void_p()
        fn = load().atlas_dev_malloc_sync if sync_alloc else load().atlas_dev_malloc
        rc = fn(C.byref(p), nbytes)
        if rc < 0:
            # delivered here (GpuBuf.alloc turns it into None): not left
            # recorded for the next call's check
            msg = load().atlas_last_error().decode()
            load().atlas_clear_error()
            raise MemoryError(msg)
        self.ptr = p.value or 0

    def free(self):
        if self.ptr:
            lib = load()
            (lib.atlas_dev_free_sync if self._sync else lib.atlas_dev_free)(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class GpuBuf:
    """f32 device buffer (lib.rs:178-237): alloc / upload / download."""

    def __init__(self, mem: _DevMem, length: int):
        self._mem = mem
        self.len = length

    @property
    def ptr(self) -> int:
        return self._mem.ptr

    @staticmethod
    def alloc(length: int) -> Optional["GpuBuf"]:
        try:
            return GpuBuf(_DevMem(max(length, 1) * 4, sync_alloc=False), length)
        except MemoryError:
            return None

    @staticmethod
    def upload(data) -> Optional["GpuBuf"]:
        a = np.ascontiguousarray(data, np.float32)
        b = GpuBuf.alloc(a.size)
        if b is None:
            return None
        if check(load().atlas_memcpy_h2d(b.ptr, _p(a), a.nbytes)) < 0:
            return None
        return b

    def download(self) -> np.ndarray:
        out = np.empty(self.len, np.float32)
        check(load().atlas_memcpy_d2h(_p(out), self.ptr, out.nbytes))
        return out


class GpuBufBf16:
    """bf16-bits device buffer for weights (lib.rs:242-280)."""

    def __init__(self, mem: _DevMem, length: int):
        self._mem = mem
        self.len = length

    @property
    def ptr(self) -> int:
        return self._mem.ptr

    @staticmethod
    def alloc(length: int) -> Optional["GpuBufBf16"]:
        try:
            return GpuBufBf16(_DevMem(max(length, 1) * 2, sync_alloc=True), length)
        except MemoryError:
            return None

    @staticmethod
    def upload(data) -> Optional["GpuBufBf16"]:
        a = np.ascontiguousarray(data, np.uint16)
        b = GpuBufBf16.alloc(a.size)
        if b is None:
            return None
        check(load().atlas_memcpy_h2d(b.ptr, _p(a), a.nbytes))
        return b


class _QuantBuf:
    """int8 / int4 weight buffer: packed data + f32 scales (extension)."""

    def __init__(self, data: np.ndarray, scales: np.ndarray, block: int):
        self.block = block
        self._d = _DevMem(max(data.nbytes, 1), sync_alloc=True)
        self._s = _DevMem(max(scales.nbytes, 4), sync_alloc=True)
        check(load().atlas_memcpy_h2d(self._d.ptr, _p(data), data.nbytes))
        check(load().atlas_memcpy_h2d(self._s.ptr, _p(scales), scales.nbytes))

    @property
    def ptr(self) -> int:
        return self._d.ptr

    @property
    def scales_ptr(self) -> int:
        return self._s.ptr


class GpuBufKind(Enum):
    """lib.rs:284-292 (F32, BF16) plus the INT8 / INT4 extensions."""
    F32 = 0
    BF16 = 1
    INT8 = 2
    INT4 = 3

    def is_bf16(self) -> bool:
        return self is GpuBufKind.BF16


class GpuMatrix:
    """Weight matrix resident in HBM (lib.rs:309-436)."""

    def __init__(self, kind: Optional[GpuBufKind], buf, rows: int, cols: int):
        self.kind = kind
        self.buf = buf
        self.rows = rows
        self.cols = cols

    @staticmethod
    def upload(data, rows: int, cols: int) -> "GpuMatrix":
        buf = GpuBuf.upload(data) if cuda_available() else None
        return GpuMatrix(GpuBufKind.F32 if buf else None, buf, rows, cols)

    @staticmethod
    def upload_bf16(data, rows: int, cols: int) -> "GpuMatrix":
        buf = GpuBufBf16.upload(data) if cuda_available() else None
        return GpuMatrix(GpuBufKind.BF16 if buf else None, buf, rows, cols)

    @staticmethod
    def upload_int8(t) -> "GpuMatrix":
        """From an ``atlas_amd.quant.Int8Tensor`` (extension)."""
        buf = _QuantBuf(np.ascontiguousarray(t.data, np.int8), np.ascontiguousarray(t.scales, np.float32), 0) \
            if cuda_available() else None
        return GpuMatrix(GpuBufKind.INT8 if buf else None, buf, t.rows, t.cols)

    @staticmethod
    def upload_int4(t) -> "GpuMatrix":
        """From an ``atlas_amd.quant.Int4Tensor`` (extension)."""
        buf = _QuantBuf(np.ascontiguousarray(t.data, np.uint8), np.ascontiguousarray(t.scales, np.float32),
                        t.block_size) if cuda_available() else None
        return GpuMatrix(GpuBufKind.INT4 if buf else None, buf, t.rows, t.cols)

    def is_on_gpu(self) -> bool:
        return self.buf is not None

    def is_bf16(self) -> bool:
        return self.kind is GpuBufKind.BF16

    def _launch(self, x_ptr: int, y_ptr: int, n: int) -> None:
        lib = load()
        m, k = self.rows, self.cols
        if self.kind is GpuBufKind.F32:
            lib.atlas_matmul_f32(self.buf.ptr, x_ptr, y_ptr, m, n, k)
            check_void()
        elif self.kind is GpuBufKind.BF16:
            lib.atlas_sgemm_bf16_f32(self.buf.ptr, x_ptr, y_ptr, m, n, k)
            check_void()
        else:
            fmt = 2 if self.kind is GpuBufKind.INT8 else 3
            if n == 1:
                check(lib.atlas_gemv_f32(fmt, self.buf.ptr, self.buf.scales_ptr, self.buf.block,
                                         x_ptr, y_ptr, m, k))
            else:
                raise AtlasError(-4, "quantised GpuMatrix: use sgemm_rows for n > 1")

    def sgemm(self, rhs, k: int, n: int, out: np.ndarray) -> bool:
        """out[m x n] = self[m x k] rhs[k x n]; H2D rhs, D2H out (lib.rs:371-400)."""
        if self.buf is None:
            return False
        assert self.cols == k
        b = GpuBuf.upload(np.ascontiguousarray(rhs, np.float32).reshape(-1))
        c = GpuBuf.alloc(self.rows * n)
        if b is None or c is None:
            return False
        self._launch(b.ptr, c.ptr, n)
        out[...] = c.download().reshape(out.shape)
        return True

    def sgemm_vec(self, x: "GpuVec", n: int = 1) -> Optional["GpuVec"]:
        """Device-to-device GEMV; returns a new GpuVec (lib.rs:409-435)."""
        if self.buf is None or x.buf is None:
            return None
        out = GpuBuf.alloc(self.rows * n)
        if out is None:
            return None
        self._launch(x.buf.ptr, out.ptr, n)
        return GpuVec(out, np.zeros(self.rows * n, np.float32), self.rows * n)

    def sgemm_rows(self, x: "GpuVec", n: int) -> "GpuVec":
        """Ragged micro-batch: x holds n activation rows [n x cols]; returns
        [n x rows] (extension, skinny MFMA GEMM)."""
        if self.buf is None or x.buf is None:
            raise AtlasError(-1, "sgemm_rows: operands are not on the GPU")
        out = GpuBuf.alloc(self.rows * n)
        fmt = {GpuBufKind.BF16: 1, GpuBufKind.INT8: 2, GpuBufKind.INT4: 3}[self.kind]
        scales = getattr(self.buf, "scales_ptr", None)
        block = getattr(self.buf, "block", 0)
        check(load().atlas_gemm_skinny_f32(fmt, self.buf.ptr, scales, block, x.buf.ptr, out.ptr,
                                           self.rows, n, self.cols))
        return GpuVec(out, np.zeros(self.rows * n, np.float32), self.rows * n)

    def __repr__(self):
        kind = "cpu" if self.kind is None else self.kind.name.lower()
        return f"GpuMatrix({self.rows}x{self.cols}, {kind})"


class GpuVec:
    """Activation vector in HBM (lib.rs:460-556); ``cpu`` mirrors the field."""

    def __init__(self, buf: Optional[GpuBuf], cpu: np.ndarray, length: int):
        self.buf = buf
        self.cpu = cpu
        self.len = length

    @staticmethod
    def zeros(length: int) -> "GpuVec":
        buf = GpuBuf.alloc(length) if cuda_available() else None
        if buf is not None:
            check(load().atlas_memset_zero(buf.ptr, max(length, 1) * 4))
        return GpuVec(buf, np.zeros(length, np.float32), length)

    @staticmethod
    def from_slice(data) -> "GpuVec":
        a = np.ascontiguousarray(data, np.float32).reshape(-1)
        buf = GpuBuf.upload(a) if cuda_available() else None
        return GpuVec(buf, a.copy(), a.size)

    def download(self) -> np.ndarray:
        if self.buf is not None:
            return self.buf.download()
        return self.cpu.copy()

    def is_on_gpu(self) -> bool:
        return self.buf is not None

    def gpu_ptr(self) -> Optional[int]:
        return self.buf.ptr if self.buf is not None else None

    def gpu_ptr_mut(self) -> Optional[int]:
        return self.gpu_ptr()

    def _need(self, *others: "GpuVec") -> None:
        if self.buf is None or any(o.buf is None for o in others):
            raise AtlasError(-1, "GpuVec op on a vector that is not on the GPU (no CPU fallback)")

    def add_inplace(self, other: "GpuVec") -> None:
        """lib.rs:506-519: self += other (device, new buffer swapped in)."""
        self._need(other)
        out = GpuBuf.alloc(self.len)
        load().atlas_vec_add_f32(self.buf.ptr, other.buf.ptr, out.ptr, self.len)
        check_void()
        self.buf = out

    def rmsnorm_inplace(self, w: "GpuVec", eps: float) -> None:
        """lib.rs:522-543: self = rmsnorm(self) * w."""
        self._need(w)
        out = GpuBuf.alloc(self.len)
        load().atlas_rmsnorm_f32(self.buf.ptr, w.buf.ptr, out.ptr, self.len, eps)
        check_void()
        self.buf = out

    def residual_rmsnorm_inplace(self, y: "GpuVec", w: "GpuVec", eps: float) -> None:
        """self += rmsnorm(y) * w in one launch (post-norm block, extension)."""
        self._need(y, w)
        check(load().atlas_residual_rmsnorm_f32(self.buf.ptr, y.buf.ptr, w.buf.ptr, self.len, 1, eps))

    def __repr__(self):
        return f"GpuVec(len={self.len}, gpu={self.is_on_gpu()})"


def gpu_argmax(x: GpuVec) -> Optional[int]:
    """lib.rs:107-126: index of the maximum (last one on ties)."""
    if x.buf is None:
        raise AtlasError(-1, "gpu_argmax: vector is not on the GPU (no CPU fallback)")
    out = GpuBuf.alloc(1)
    load().atlas_gpu_argmax(x.buf.ptr, out.ptr, x.len)
    check_void()
    return int(out.download()[0])


def rope_apply_gpu(x: GpuVec, pos: int, head_dim: int, theta_base: float) -> None:
    """lib.rs:570-587."""
    x._need()
    load().atlas_rope_apply_f32(x.buf.ptr, pos, head_dim, theta_base)
    check_void()


def silu_mul_gpu(gate: GpuVec, up: GpuVec) -> GpuVec:
    """lib.rs:590-609: silu(gate) * up into a new GpuVec."""
    gate._need(up)
    out = GpuBuf.alloc(gate.len)
    load().atlas_silu_mul_f32(gate.buf.ptr, up.buf.ptr, out.ptr, gate.len)
    check_void()
    return GpuVec(out, np.zeros(gate.len, np.float32), gate.len)


def adamw_step_gpu(param: int, m: int, v: int, grad: int, lr: float, beta1: float, beta2: float,
                   eps: float, wd: float, bc1: float, bc2: float, n: int) -> bool:
    """lib.rs:612-628 (training kernel, kept for ABI completeness)."""
    if not cuda_available():
        return False
    load().atlas_adamw_step(param, m, v, grad, lr, beta1, beta2, eps, wd, bc1, bc2, n)
    check_void()
    return True


def qk_norm_inplace_gpu(x: GpuVec, w: GpuVec, n_heads: int, head_dim: int, eps: float) -> None:
    """lib.rs:633-654."""
    x._need(w)
    load().atlas_qk_norm_inplace(x.buf.ptr, w.buf.ptr, n_heads, head_dim, eps)
    check_void()


class GpuRopeTables:
    """lib.rs:662-693: cos/sin [max_seq x half_dim] in HBM."""

    def __init__(self, cos: GpuVec, sin: GpuVec, max_seq: int, half_dim: int):
        self.cos, self.sin, self.max_seq, self.half_dim = cos, sin, max_seq, half_dim

    @staticmethod
    def upload(cos_flat, sin_flat, max_seq: int, half_dim: int) -> Optional["GpuRopeTables"]:
        if not cuda_available():
            return None
        return GpuRopeTables(GpuVec.from_slice(cos_flat), GpuVec.from_slice(sin_flat), max_seq, half_dim)

    def apply_to(self, x: GpuVec, n_heads: int, head_dim: int, pos: int) -> None:
        x._need(self.cos, self.sin)
        load().atlas_rope_precomputed(x.buf.ptr, self.cos.buf.ptr, self.sin.buf.ptr, n_heads,
                                      head_dim, pos, self.max_seq)
        check_void()


class GpuKvCache:
    """lib.rs:701-785: keys/values [max_seq x n_kv_heads x head_dim] f32."""

    def __init__(self, keys: GpuVec, values: GpuVec, max_seq: int, n_kv_heads: int, head_dim: int):
        self.keys, self.values = keys, values
        self.max_seq, self.n_kv_heads, self.head_dim = max_seq, n_kv_heads, head_dim

    @staticmethod
    def new(max_seq: int, n_kv_heads: int, head_dim: int) -> Optional["GpuKvCache"]:
        if not cuda_available():
            return None
        total = max_seq * n_kv_heads * head_dim
        return GpuKvCache(GpuVec.zeros(total), GpuVec.zeros(total), max_seq, n_kv_heads, head_dim)

    def write(self, pos: int, new_k: GpuVec, new_v: GpuVec) -> None:
        if not 0 <= pos < self.max_seq:
            raise AtlasError(-1, f"GpuKvCache.write: pos {pos} outside [0, {self.max_seq})")
        self.keys._need(self.values, new_k, new_v)
        load().atlas_kv_cache_write(self.keys.buf.ptr, self.values.buf.ptr, new_k.buf.ptr,
                                    new_v.buf.ptr, pos, self.n_kv_heads, self.head_dim)
        check_void()

    def decode_attention(self, q: GpuVec, n_heads: int, pos: int, scale: float,
                         window_size: int) -> Optional[GpuVec]:
        if q.buf is None:
            return None
        if not 0 <= pos < self.max_seq:
            raise AtlasError(-1, f"decode_attention: pos {pos} outside [0, {self.max_seq})")
        n = n_heads * self.head_dim
        out = GpuBuf.alloc(n)
        load().atlas_decode_attention(q.buf.ptr, self.keys.buf.ptr, self.values.buf.ptr, out.ptr,
                                      n_heads, self.n_kv_heads, self.head_dim, pos, scale, window_size)
        check_void()
        return GpuVec(out, np.zeros(n, np.float32), n)

    def reset(self) -> None:
        """No-op by design (lib.rs:772-784): positions beyond pos are never read."""
