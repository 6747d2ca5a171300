"""Kernel parity on the MI355X: every HIP entry point against the oracle.

Tolerances: GEMV outputs max-abs <= 1e-3 * max|y_ref|;
attention outputs <= 2e-3 * max|o_ref|; quantisation and indexing bit-exact.
Inputs are seeded N(0, 0.02) weights and N(0, 1) activations, as the configs ask.
"""
import ctypes as C
import math

import numpy as np
import pytest

from atlas_amd._lib import check_void
from tests.gpu_util import Dev, lib, rel_err, sync

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3
ATTN_TOL = 2e-3


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import atlas_amd
    atlas_amd.load()
    if not lib().atlas_cuda_available():
        pytest.fail("no HIP device visible: GPU tests need an MI355X")


def _w(shape, seed):
    return (np.random.default_rng(seed).standard_normal(shape) * 0.02).astype(np.float32)


def _x(n, seed):
    return np.random.default_rng(seed).standard_normal(n).astype(np.float32)


# ---------------------------------------------------------------------------
# batch-1 GEMV: bf16 / int8 / int4 / f32
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M,K", [(4096, 4096), (11008, 4096), (4096, 11008), (100, 64),
                                 (37, 200), (4, 3)])
def test_gemv_bf16(orc, M, K):
    print(f"gemv_bf16 M={M} K={K}", flush=True)
    bits = orc.bf16_from_f32(_w((M, K), M + K))
    x = _x(K, 1)
    y_ref = orc.linear(orc.MatView.bf16(bits, M, K), x, threads=8)
    dw, dx, dy = Dev(bits), Dev(x), Dev.empty(M)
    assert lib().atlas_gemv_bf16_f32(dw.ptr, dx.ptr, dy.ptr, M, K) == 0
    assert rel_err(dy.get(), y_ref) <= GEMV_TOL


@pytest.mark.parametrize("M,K", [(11008, 4096), (4096, 11008), (64, 48), (5, 7)])
def test_gemv_int8(orc, M, K):
    print(f"gemv_int8 M={M} K={K}", flush=True)
    q, s = orc.int8_quantize(_w((M, K), 3 * M + K))
    x = _x(K, 2)
    y_ref = orc.linear(orc.MatView.int8(q, s), x, threads=8)
    dw, ds, dx, dy = Dev(q), Dev(s), Dev(x), Dev.empty(M)
    assert lib().atlas_gemv_i8_f32(dw.ptr, ds.ptr, dx.ptr, dy.ptr, M, K) == 0
    assert rel_err(dy.get(), y_ref) <= GEMV_TOL


@pytest.mark.parametrize("M,K,bs", [(4096, 4096, 32), (11008, 4096, 32), (4096, 11008, 32),
                                    (256, 4096, 64), (3, 96, 64), (7, 50, 32)])
def test_gemv_int4(orc, M, K, bs):
    print(f"gemv_int4 M={M} K={K} bs={bs}", flush=True)
    q, s = orc.int4_quantize(_w((M, K), 5 * M + K), bs)
    x = _x(K, 3)
    y_ref = orc.linear(orc.MatView.int4(q, s, M, K, bs), x, threads=8)
    dw, ds, dx, dy = Dev(q), Dev(s), Dev(x), Dev.empty(M)
    assert lib().atlas_gemv_i4_f32(dw.ptr, ds.ptr, bs, dx.ptr, dy.ptr, M, K) == 0
    assert rel_err(dy.get(), y_ref) <= GEMV_TOL


def test_gemv_f32_matmul_n1(orc):
    w = _w((300, 512), 9)
    x = _x(512, 4)
    y_ref = orc.linear(orc.MatView.f32(w), x)
    dw, dx, dy = Dev(w), Dev(x), Dev.empty(300)
    lib().atlas_matmul_f32(dw.ptr, dx.ptr, dy.ptr, 300, 1, 512)
    sync()
    assert rel_err(dy.get(), y_ref) <= GEMV_TOL


@pytest.mark.parametrize("fmt", ["bf16", "int8", "int4"])
def test_gemv_swiglu(orc, fmt):
    h, K = 512, 256
    g, u = _w((h, K), 11), _w((h, K), 12)
    x = _x(K, 5)
    inter = np.empty((2 * h, K), np.float32)
    inter[0::2], inter[1::2] = g, u
    if fmt == "bf16":
        stored = orc.bf16_from_f32(inter)
        gv, uv = orc.MatView.bf16(stored[0::2].copy(), h, K), orc.MatView.bf16(stored[1::2].copy(), h, K)
        args = (1, Dev(stored), None, 0)
    elif fmt == "int8":
        q, s = orc.int8_quantize(inter)
        gv, uv = orc.MatView.int8(q[0::2].copy(), s[0::2].copy()), orc.MatView.int8(q[1::2].copy(), s[1::2].copy())
        args = (2, Dev(q), Dev(s), 0)
    else:
        q, s = orc.int4_quantize(inter, 32)
        qg, qu = q.reshape(2 * h, K // 2)[0::2].copy(), q.reshape(2 * h, K // 2)[1::2].copy()
        sg, su = s.reshape(2 * h, K // 32)[0::2].copy(), s.reshape(2 * h, K // 32)[1::2].copy()
        gv, uv = orc.MatView.int4(qg, sg, h, K, 32), orc.MatView.int4(qu, su, h, K, 32)
        args = (3, Dev(q), Dev(s), 32)
    gr, ur = orc.linear(gv, x), orc.linear(uv, x)
    ref = np.array([orc.silu(float(a)) for a in gr], np.float32) * ur
    dx, dh = Dev(x), Dev.empty(h)
    fmt_id, dw, ds, bs = args
    assert lib().atlas_gemv_swiglu_f32(fmt_id, dw.ptr, ds.ptr if ds else None, bs, dx.ptr, dh.ptr,
                                       h, K) == 0
    assert rel_err(dh.get(), ref) <= GEMV_TOL


# ---------------------------------------------------------------------------
# skinny ragged batch: multi-row GEMV (2-3 rows) and MFMA tiles (4-8 rows)
# ---------------------------------------------------------------------------

def _stored(orc, fmt, w, block=32):
    """(oracle view, device weights, device scales, format id, block) of w."""
    M, K = w.shape
    if fmt == "bf16":
        b = orc.bf16_from_f32(w)
        return orc.MatView.bf16(b, M, K), Dev(b), None, 1, 0
    if fmt == "int8":
        q, s = orc.int8_quantize(w)
        return orc.MatView.int8(q, s), Dev(q), Dev(s), 2, 0
    q, s = orc.int4_quantize(w, block)
    return orc.MatView.int4(q, s, M, K, block), Dev(q), Dev(s), 3, block


def _skinny_check(orc, fmt, n, M, K, block=32, seed=0):
    w = _w((M, K), 21 + n + seed)
    x = np.random.default_rng(n + seed).standard_normal((n, K)).astype(np.float32)
    view, dw, ds, fid, bs = _stored(orc, fmt, w, block)
    ref = orc.linear_batch(view, x)
    dx, dy = Dev(x), Dev.empty((n, M))
    assert lib().atlas_gemm_skinny_f32(fid, dw.ptr, ds.ptr if ds else None, bs, dx.ptr, dy.ptr,
                                       M, n, K) == 0
    y = dy.get()
    for i in range(n):
        assert rel_err(y[i], ref[i]) <= GEMV_TOL, i


@pytest.mark.parametrize("n", [1, 3, 5, 8])
@pytest.mark.parametrize("fmt", ["bf16", "int8", "int4"])
def test_skinny(orc, fmt, n):
    M, K = (4096, 4096) if n in (1, 8) else (1000, 512)
    print(f"skinny {fmt} n={n} M={M} K={K}", flush=True)
    _skinny_check(orc, fmt, n, M, K)


# 9-16 rows: two MFMA A tiles share each weight tile (half the k tiles per
# wave, so K = 4096 already splits across blocks) -- bf16 with K <= 4096 and
# int8 with K <= 4096 and M > 8192 -- or two launches of the 2-8-row kernels
# (int4, int8 otherwise, bf16 with K > 4096), the second half's rows offset
@pytest.mark.parametrize("fmt,n,M,K", [
    ("bf16", 9, 1000, 512), ("bf16", 16, 4096, 4096), ("bf16", 13, 777, 11008),
    ("int8", 16, 1000, 4096), ("int8", 9, 4096, 11008), ("int8", 12, 9000, 1024),
    ("int4", 16, 2048, 4096), ("int4", 12, 1000, 11008), ("int4", 9, 4096, 4096)])
def test_skinny_two_a_tiles(orc, fmt, n, M, K):
    print(f"skinny two tiles {fmt} n={n} M={M} K={K}", flush=True)
    _skinny_check(orc, fmt, n, M, K, 32, seed=3)


# 17-128 rows: the tiled MFMA GEMM of prompt chunks.  Cases: one and eight
# 16-row tiles with a ragged last tile, K split across blocks (K = 11008: 344
# k steps) and unsplit (70 000 rows fill the grid), rows not a multiple of
# the 128-row block; int8 row scales, int4 blocks of 32 and 128.
@pytest.mark.parametrize("fmt,n,M,K,block", [
    ("bf16", 17, 1000, 512, 32), ("bf16", 32, 4096, 4096, 32), ("bf16", 61, 777, 11008, 32),
    ("bf16", 100, 2048, 1024, 32), ("bf16", 128, 4096, 4096, 32), ("bf16", 40, 70000, 128, 32),
    ("bf16", 128, 130, 256, 32),
    ("int8", 17, 1000, 512, 32), ("int8", 128, 4096, 4096, 32), ("int8", 70, 777, 11008, 32),
    ("int4", 20, 1000, 512, 32), ("int4", 128, 4096, 4096, 32), ("int4", 90, 777, 11008, 32),
    ("int4", 48, 2048, 1024, 128)])
def test_gemm_rows(orc, fmt, n, M, K, block):
    print(f"gemm rows {fmt} n={n} M={M} K={K} block={block}", flush=True)
    _skinny_check(orc, fmt, n, M, K, block, seed=5)


# Two and three rows take the multi-row GEMV: the 7B shapes (three rows of
# K = 11008 fill 132 KB of LDS), odd row counts, K not a multiple of one
# wave step, int4 blocks of 128, and a 3 x 32 matrix.
@pytest.mark.parametrize("fmt,n,M,K,block", [
    ("bf16", 2, 11008, 4096, 32), ("bf16", 3, 4096, 11008, 32), ("bf16", 2, 3, 32, 32),
    ("int8", 2, 4096, 11008, 32), ("int8", 3, 1001, 544, 32), ("int8", 3, 12288, 4096, 32),
    ("int4", 2, 11008, 4096, 32), ("int4", 3, 4096, 11008, 32), ("int4", 3, 777, 1024, 128),
    ("int4", 2, 64, 12288, 64)])
def test_skinny_multi_row(orc, fmt, n, M, K, block):
    print(f"skinny multi-row {fmt} n={n} M={M} K={K} block={block}", flush=True)
    _skinny_check(orc, fmt, n, M, K, block, seed=7)


# The ragged batch's 1/3/5/8-row GEMMs at the 7B decode shapes (BASELINE.json
# configs[2] asks for 1/3/5/8 rows of 11008 x 4096; at that shape the int4
# kernel hands 688 row groups to 256 blocks).
@pytest.mark.parametrize("M,K", [(4096, 4096), (11008, 4096)])
@pytest.mark.parametrize("n", [1, 3, 5, 8])
@pytest.mark.parametrize("fmt", ["bf16", "int8", "int4"])
def test_skinny_7b_rows(orc, fmt, n, M, K):
    print(f"skinny 7B {fmt} n={n} M={M} K={K}", flush=True)
    _skinny_check(orc, fmt, n, M, K, 32, seed=11)


# The 2-8-row skinny kernels: direct loads (int4; bf16 and int8 with
# K > 4096) and the LDS-staged tile (bf16 and int8 with K <= 4096): a ragged
# last 16-row group, K splits with a remainder slice, and two rows of int8
# on either side of K = 4096.
@pytest.mark.parametrize("fmt,n,M,K", [
    ("int8", 8, 777, 4096), ("int8", 2, 1000, 8192), ("int8", 4, 300, 11008), ("int8", 2, 33, 2048),
    ("bf16", 3, 1000, 4096),
    ("bf16", 8, 777, 8192), ("bf16", 5, 4096, 11008), ("bf16", 2, 100, 4224),
    ("int4", 8, 777, 8192), ("int4", 6, 33, 4224)])
def test_skinny_direct_loads(orc, fmt, n, M, K):
    print(f"skinny direct {fmt} n={n} M={M} K={K}", flush=True)
    _skinny_check(orc, fmt, n, M, K, 32, seed=13)


# SwiGLU epilogue over n rows: one row (batch-1 GEMV), two (multi-row GEMV),
# five (MFMA skinny tiles, split-K reduce applies SwiGLU), the direct-load
# kernels' own epilogue (int8 5 rows) and the split reduce after them (bf16
# 4 rows at K = 4224, int8 8 rows at K = 8192), twenty rows at
# K = 128 (the prompt GEMM's unsplit epilogue: gate/up pairs meet across
# lanes) and at K = 4096 (split, SwiGLU in the reduce); 9-16 rows as two
# launches (int4 12 rows, int8 13 rows at K = 8192) and as 16-row MFMA tiles
# (int8, 2h = 10 000 weight rows).
@pytest.mark.parametrize("fmt,n,h,K", [
    ("bf16", 1, 1000, 512), ("int8", 2, 700, 1024), ("int4", 5, 512, 2048),
    ("bf16", 20, 640, 128), ("int8", 20, 640, 128), ("int4", 20, 640, 128),
    ("bf16", 20, 2048, 4096), ("int4", 33, 1024, 4096),
    ("int8", 5, 512, 2048), ("bf16", 4, 256, 4224), ("int8", 8, 300, 8192),
    ("int4", 12, 512, 2048), ("int8", 13, 600, 8192), ("int8", 16, 5000, 1024)])
def test_gemm_skinny_swiglu(orc, fmt, n, h, K):
    print(f"skinny swiglu {fmt} n={n} h={h} K={K}", flush=True)
    w = _w((2 * h, K), 97 + n)
    x = np.random.default_rng(n).standard_normal((n, K)).astype(np.float32)
    view, dw, ds, fid, bs = _stored(orc, fmt, w, 32)
    y = orc.linear_batch(view, x)                     # [n, 2h]: gate_i, up_i interleaved
    ref = np.array([[orc.silu(float(g)) for g in row] for row in y[:, 0::2]], np.float32)
    ref *= y[:, 1::2]
    dx, dh = Dev(x), Dev.empty((n, h))
    assert lib().atlas_gemm_skinny_swiglu_f32(fid, dw.ptr, ds.ptr if ds else None, bs, dx.ptr,
                                              dh.ptr, h, n, K) == 0
    got = dh.get()
    for i in range(n):
        assert rel_err(got[i], ref[i]) <= GEMV_TOL, i


def test_sgemm_bf16_reference_layout(orc):
    # crates/atlas-tensor/src/lib.rs:44-47: B is [k x n] row-major, C [m x n]
    M, K = 256, 512
    b = orc.bf16_from_f32(_w((M, K), 31))
    view = orc.MatView.bf16(b, M, K)
    for n in (2, 5, 8, 12):
        X = np.random.default_rng(n).standard_normal((K, n)).astype(np.float32)
        ref = np.stack([orc.linear(view, X[:, j].copy()) for j in range(n)], axis=1)
        dw, dx, dc = Dev(b), Dev(X), Dev.empty((M, n))
        lib().atlas_sgemm_bf16_f32(dw.ptr, dx.ptr, dc.ptr, M, n, K)
        sync()
        assert rel_err(dc.get(), ref) <= GEMV_TOL, n


def test_tensor_mirrors_host_slices_rope_and_cache(orc):
    # GpuMatrix::sgemm with host slices (H2D rhs, D2H out; crates/atlas-tensor/
    # src/lib.rs:371-400) over f32 and bf16 weights, one and several columns;
    # GpuRopeTables::apply_to (lib.rs:681-692) and GpuKvCache::{write,
    # decode_attention} (lib.rs:722-770) against the oracle
    from atlas_amd.tensor import GpuKvCache, GpuMatrix, GpuRopeTables, GpuVec
    M, K = 768, 1024
    w = _w((M, K), 61)
    bits = orc.bf16_from_f32(w)
    for mat, view in ((GpuMatrix.upload(w, M, K), orc.MatView.f32(w)),
                      (GpuMatrix.upload_bf16(bits, M, K), orc.MatView.bf16(bits, M, K))):
        for n in (1, 3):
            rhs = np.random.default_rng(n).standard_normal((K, n)).astype(np.float32)
            out = np.empty((M, n), np.float32)
            assert mat.sgemm(rhs, K, n, out)
            ref = np.stack([orc.linear(view, rhs[:, j].copy()) for j in range(n)], axis=1)
            assert rel_err(out, ref) <= GEMV_TOL, (mat, n)
    H, KVH, hd, S = 8, 2, 128, 300
    cos, sin, _ = orc.rope_tables(hd, S, 500000.0, dict(factor=8.0, orig_max_pos=8192,
                                                        attn_factor=1.2079441541679836,
                                                        beta_fast=32.0, beta_slow=1.0))
    tabs = GpuRopeTables.upload(cos.reshape(-1), sin.reshape(-1), S, hd // 2)
    q = np.random.default_rng(3).standard_normal(H * hd).astype(np.float32)
    qd = GpuVec.from_slice(q)
    tabs.apply_to(qd, H, hd, 257)
    want = np.concatenate([orc.rope_apply(q[h * hd:(h + 1) * hd], cos[257], sin[257])
                           for h in range(H)])
    assert rel_err(qd.download(), want) <= 1e-6
    cache = GpuKvCache.new(S, KVH, hd)
    kc = np.random.default_rng(4).standard_normal((S, KVH * hd)).astype(np.float32)
    vc = np.random.default_rng(5).standard_normal((S, KVH * hd)).astype(np.float32)
    for p in range(S):
        cache.write(p, GpuVec.from_slice(kc[p]), GpuVec.from_slice(vc[p]))
    scale = 1.2079441541679836 / math.sqrt(hd)
    for pos, window in ((0, 0), (299, 0), (299, 64)):
        got = cache.decode_attention(qd, H, pos, scale, window).download()
        ref = orc.attention(qd.download(), kc, vc, H, KVH, hd, pos, scale, window)
        assert rel_err(got, ref) <= ATTN_TOL, (pos, window)


def test_sgemm_vec_ones_literal():
    # crates/atlas-tensor/src/lib.rs:1207-1220
    from atlas_amd.tensor import GpuMatrix, GpuVec
    gm = GpuMatrix.upload(np.ones(12, np.float32), 4, 3)
    out = gm.sgemm_vec(GpuVec.from_slice([1.0, 1.0, 1.0]), 1)
    assert out.len == 4
    assert np.allclose(out.download(), 3.0)


# ---------------------------------------------------------------------------
# attention (config 4: 32 q heads, 8 kv heads, hd 128)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("ctx,window", [(512, 0), (4096, 0), (16384, 0), (16384, 4096),
                                        (4096, 4096), (1, 0), (300, 64)])
def test_decode_attention_gqa(orc, ctx, window):
    H, KVH, hd = 32, 8, 128
    print(f"attention ctx={ctx} window={window}", flush=True)
    rng = np.random.default_rng(ctx + window)
    q = rng.standard_normal(H * hd).astype(np.float32)
    K = rng.standard_normal((ctx, KVH, hd)).astype(np.float32)
    V = rng.standard_normal((ctx, KVH, hd)).astype(np.float32)
    scale = 1.2079441541679836 / math.sqrt(hd)
    pos = ctx - 1
    ref = orc.attention(q, K, V, H, KVH, hd, pos, scale, window)
    dq, dk, dv, do = Dev(q), Dev(K), Dev(V), Dev.empty(H * hd)
    lib().atlas_decode_attention(dq.ptr, dk.ptr, dv.ptr, do.ptr, H, KVH, hd, pos, scale, window)
    sync()
    assert rel_err(do.get(), ref) <= ATTN_TOL


@pytest.mark.parametrize("H,KVH,hd", [(4, 2, 16), (8, 8, 64), (4, 1, 64), (32, 32, 128),
                                      (6, 3, 32), (8, 2, 256)])
def test_decode_attention_shapes(orc, H, KVH, hd):
    rng = np.random.default_rng(H * hd)
    ctx = 77
    q = rng.standard_normal(H * hd).astype(np.float32)
    K = rng.standard_normal((ctx, KVH, hd)).astype(np.float32)
    V = rng.standard_normal((ctx, KVH, hd)).astype(np.float32)
    for pos, window in ((ctx - 1, 0), (40, 7), (0, 0)):
        ref = orc.attention(q, K, V, H, KVH, hd, pos, 0.1, window)
        dq, dk, dv, do = Dev(q), Dev(K), Dev(V), Dev.empty(H * hd)
        lib().atlas_decode_attention(dq.ptr, dk.ptr, dv.ptr, do.ptr, H, KVH, hd, pos, 0.1, window)
        sync()
        assert rel_err(do.get(), ref) <= ATTN_TOL, (pos, window)


# ---------------------------------------------------------------------------
# fused norm / RoPE / KV write
# ---------------------------------------------------------------------------

def test_qkv_post_matches_oracle(orc):
    H, KVH, hd, max_seq, pos = 32, 8, 128, 64, 37
    yarn = dict(factor=8.0, orig_max_pos=8192, attn_factor=1.2079441541679836,
                beta_fast=32.0, beta_slow=1.0)
    cos, sin, _ = orc.rope_tables(hd, max_seq, 500000.0, yarn)
    rng = np.random.default_rng(8)
    qkv = rng.standard_normal((H + 2 * KVH) * hd).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, H * hd).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, KVH * hd).astype(np.float32)
    q_ref = orc.qk_norm(qkv[:H * hd], qn, H, hd, 1e-6)
    k_ref = orc.qk_norm(qkv[H * hd:(H + KVH) * hd], kn, KVH, hd, 1e-6)
    q_ref = np.concatenate([orc.rope_apply(q_ref[h * hd:(h + 1) * hd], cos[pos], sin[pos]) for h in range(H)])
    k_ref = np.concatenate([orc.rope_apply(k_ref[h * hd:(h + 1) * hd], cos[pos], sin[pos]) for h in range(KVH)])
    d_qkv, dqn, dkn = Dev(qkv), Dev(qn), Dev(kn)
    dcos, dsin = Dev(cos), Dev(sin)
    kc, vc = Dev.empty((max_seq, KVH, hd)), Dev.empty((max_seq, KVH, hd))
    assert lib().atlas_qkv_post_f32(d_qkv.ptr, dqn.ptr, dkn.ptr, 1e-6, dcos.ptr, dsin.ptr, kc.ptr,
                                    vc.ptr, H, KVH, hd, pos) == 0
    out = d_qkv.get()
    assert np.max(np.abs(out[:H * hd] - q_ref)) <= 1e-5 * np.max(np.abs(q_ref))
    assert np.max(np.abs(kc.get()[pos].reshape(-1) - k_ref)) <= 1e-5 * np.max(np.abs(k_ref))
    assert np.array_equal(vc.get()[pos].reshape(-1), qkv[(H + KVH) * hd:])
    assert np.all(kc.get()[pos + 1:] == 0) and np.all(kc.get()[:pos] == 0)


def test_reference_qk_norm_rope_kv_ops(orc):
    H, hd, max_seq, pos = 4, 64, 16, 5
    cos, sin, _ = orc.rope_tables(hd, max_seq, 10000.0)
    rng = np.random.default_rng(3)
    x = rng.standard_normal(H * hd).astype(np.float32)
    w = rng.uniform(0.5, 1.5, H * hd).astype(np.float32)
    ref = orc.qk_norm(x, w, H, hd, 1e-6)
    ref = np.concatenate([orc.rope_apply(ref[h * hd:(h + 1) * hd], cos[pos], sin[pos]) for h in range(H)])
    dx, dw, dc, ds = Dev(x), Dev(w), Dev(cos), Dev(sin)
    lib().atlas_qk_norm_inplace(dx.ptr, dw.ptr, H, hd, 1e-6)
    lib().atlas_rope_precomputed(dx.ptr, dc.ptr, ds.ptr, H, hd, pos, max_seq)
    sync()
    assert np.max(np.abs(dx.get() - ref)) <= 1e-5 * np.max(np.abs(ref))
    kc, vc = Dev.empty((max_seq, H * hd)), Dev.empty((max_seq, H * hd))
    nk, nv = Dev(x), Dev(w)
    lib().atlas_kv_cache_write(kc.ptr, vc.ptr, nk.ptr, nv.ptr, pos, H, hd)
    sync()
    assert np.array_equal(kc.get()[pos], x) and np.array_equal(vc.get()[pos], w)


def test_rmsnorm_and_residual(orc):
    # crates/atlas-tensor/src/lib.rs:1171-1181 literal
    from atlas_amd.tensor import GpuVec
    x = GpuVec.from_slice([1.0, 2.0, 3.0, 4.0])
    x.rmsnorm_inplace(GpuVec.from_slice([1.0] * 4), 1e-5)
    out = x.download()
    r = math.sqrt(7.5)
    assert abs(out[0] - 1 / r) < 1e-6 and abs(out[3] - 4 / r) < 1e-6
    rng = np.random.default_rng(4)
    for n in (4096, 11008, 77):
        xs, ys = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        ref = xs + orc.rmsnorm(ys, w, 1e-6)
        dx, dy, dw = Dev(xs), Dev(ys), Dev(w)
        assert lib().atlas_residual_rmsnorm_f32(dx.ptr, dy.ptr, dw.ptr, n, 1, 1e-6) == 0
        assert np.max(np.abs(dx.get() - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_reference_tensor_ops():
    # crates/atlas-tensor/src/lib.rs:1144-1205 (GpuVec tests)
    from atlas_amd import tensor as t
    assert t.cuda_available() and t.cuda_device_count() >= 1
    z = t.GpuVec.zeros(64)
    assert z.len == 64 and np.all(z.download() == 0)
    v = t.GpuVec.from_slice(np.arange(16, dtype=np.float32))
    assert np.array_equal(v.download(), np.arange(16, dtype=np.float32))
    a = t.GpuVec.from_slice([1.0, 2.0, 3.0, 4.0])
    a.add_inplace(t.GpuVec.from_slice([0.5] * 4))
    assert np.allclose(a.download(), [1.5, 2.5, 3.5, 4.5])
    s = t.silu_mul_gpu(t.GpuVec.from_slice([0.0, 1.0, -1.0, 2.0]), t.GpuVec.from_slice([1.0] * 4))
    assert abs(s.download()[0]) < 1e-6 and abs(s.download()[1] - 0.7310586) < 1e-6
    r = t.GpuVec.from_slice([1.0, 2.0, 3.0, 4.0])
    t.rope_apply_gpu(r, 0, 4, 10000.0)
    assert np.allclose(r.download(), [1.0, 2.0, 3.0, 4.0])


# ---------------------------------------------------------------------------
# the remaining reference-FFI exports (crates/atlas-tensor/src/lib.rs:17-92)
# ---------------------------------------------------------------------------

def _adamw_ref(p, m, v, g, lr, b1, b2, eps, wd, bc1, bc2):
    """kernels/matmul.cu:138-161 restated in float64 from float32 inputs.  The
    coefficients the kernel forms in float32 (1 - beta, 1 - lr * wd) are
    rounded to float32 first: 1 - 0.999f is 0.00099998713, not 0.001."""
    f = np.float32
    p, m, v, g = (np.asarray(a, np.float64) for a in (p, m, v, g))
    b1, b2, lr, eps = float(f(b1)), float(f(b2)), float(f(lr)), float(f(eps))
    c1, c2 = float(f(1) - f(b1)), float(f(1) - f(b2))
    decay = float(f(1) - f(lr) * f(wd))
    m = b1 * m + c1 * g
    v = b2 * v + c2 * g * g
    mh, vh = m * bc1, v * bc2
    return p * decay - lr * mh / (np.sqrt(vh) + eps), m, v


def test_adamw_step_reference_contract():
    # The caller passes bc = 1/(1 - beta^t) (crates/atlas-optim/src/lib.rs:203-204),
    # which the kernel multiplies by; decay is decoupled (p * (1 - lr*wd)).
    print("adamw_step", flush=True)
    rng = np.random.default_rng(17)
    n = 70001
    lr, b1, b2, eps, wd = 1e-3, 0.9, 0.999, 1e-8, 0.01
    p = rng.standard_normal(n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    dp, dm, dv = Dev(p), Dev(m), Dev(v)
    for t in range(1, 4):
        g = rng.standard_normal(n).astype(np.float32)
        bc1 = np.float32(1.0 / (1.0 - np.float32(b1) ** np.float32(t)))
        bc2 = np.float32(1.0 / (1.0 - np.float32(b2) ** np.float32(t)))
        dg = Dev(g)
        lib().atlas_adamw_step(dp.ptr, dm.ptr, dv.ptr, dg.ptr, lr, b1, b2, eps, wd,
                               float(bc1), float(bc2), n)
        check_void()
        p_ref, m_ref, v_ref = _adamw_ref(p, m, v, g, lr, b1, b2, eps, wd, float(bc1), float(bc2))
        gp, gm, gv = dp.get(), dm.get(), dv.get()
        assert np.max(np.abs(gm - m_ref)) <= 1e-6 * np.max(np.abs(m_ref))
        assert np.max(np.abs(gv - v_ref)) <= 1e-6 * np.max(np.abs(v_ref))
        assert np.max(np.abs(gp - p_ref)) <= 2e-6 * np.max(np.abs(p_ref))
        if t == 1:
            # closed form at step 1 from zero moments: m_hat = g, v_hat = g^2, so
            # every parameter moves by lr * sign(g) after decay (|g| >> eps)
            step = p.astype(np.float64) * (1 - lr * wd) - gp
            big = np.abs(g) > 1e-3
            # (a few float32 ulps of |p| <= 5; a divided bias correction is off by 9 lr)
            assert np.max(np.abs(step[big] - lr * np.sign(g[big]))) < 2e-6
        p, m, v = gp, gm, gv


def test_softmax_scale_relu_copy():
    print("softmax/scale/relu/vram_copy", flush=True)
    # crates/atlas-tensor/src/lib.rs:1109-1114 and 1132-1138 literals
    x = Dev(np.array([1.0, 2.0, 3.0], np.float32))
    o = Dev.empty(3)
    lib().atlas_softmax_f32(x.ptr, o.ptr, 1, 3)
    s = o.get()
    e = np.exp(np.array([1.0, 2.0, 3.0]) - 3.0)
    assert abs(float(np.sum(s)) - 1.0) < 1e-6
    assert np.max(np.abs(s - e / e.sum())) < 1e-7
    t = Dev(np.array([-2.0, -1.0, 0.0, 1.0, 2.0], np.float32))
    o5 = Dev.empty(5)
    lib().atlas_scale_f32(t.ptr, 2.0, o5.ptr, 5)
    assert np.array_equal(o5.get(), [-4.0, -2.0, 0.0, 2.0, 4.0])
    lib().atlas_relu_f32(t.ptr, o5.ptr, 5)
    assert np.array_equal(o5.get(), [0.0, 0.0, 0.0, 1.0, 2.0])
    rng = np.random.default_rng(23)
    # row softmax: against float64, rows summing to one, shift invariance
    for rows, cols in ((7, 100278), (33, 5), (4, 257), (1, 1)):
        a = (rng.standard_normal((rows, cols)) * 4).astype(np.float32)
        da, do = Dev(a), Dev.empty((rows, cols))
        lib().atlas_softmax_f32(da.ptr, do.ptr, rows, cols)
        got = do.get().astype(np.float64)
        a64 = a.astype(np.float64)
        ex = np.exp(a64 - a64.max(axis=1, keepdims=True))
        ref = ex / ex.sum(axis=1, keepdims=True)
        assert np.max(np.abs(got - ref)) <= 1e-6 * np.max(ref)
        assert np.max(np.abs(got.sum(axis=1) - 1.0)) < 1e-5
        da2 = Dev(a + np.float32(8.0))
        lib().atlas_softmax_f32(da2.ptr, do.ptr, rows, cols)
        assert np.max(np.abs(do.get() - got)) <= 2e-6 * np.max(ref)
    # scale and relu are one rounding each: bit-exact with numpy float32
    n = 1 << 20 | 3
    a = rng.standard_normal(n).astype(np.float32)
    da, do = Dev(a), Dev.empty(n)
    lib().atlas_scale_f32(da.ptr, np.float32(-0.3125), do.ptr, n)
    assert np.array_equal(do.get(), a * np.float32(-0.3125))
    lib().atlas_relu_f32(da.ptr, do.ptr, n)
    assert np.array_equal(do.get(), np.where(a > 0, a, np.float32(0)))
    # vram_copy is a bit copy (NaN payloads and -0.0 included)
    bits = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    bits[:4] = [0x7FC01234, 0xFF800001, 0x80000000, 0x00000001]
    db, dc = Dev(bits), Dev.empty(n, np.uint32)
    lib().atlas_vram_copy_f32(db.ptr, dc.ptr, n)
    assert np.array_equal(dc.get(), bits)
    check_void()


def _rope_apply_ref(x, pos, hd, theta):
    """crates/atlas-tensor/src/lib.rs:570-587 CPU form (float32 throughout)."""
    x = np.array(x, np.float32)
    half = hd // 2
    i = np.arange(half)
    freq = np.float32(1.0) / np.power(np.float32(theta), (2 * i).astype(np.float32) / np.float32(hd))
    ang = np.float32(pos) * freq.astype(np.float32)
    c, s = np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))
    x0, x1 = x[:half].astype(np.float64), x[half:].astype(np.float64)
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c])


@pytest.mark.parametrize("hd,theta", [(128, 500000.0), (64, 10000.0), (6, 10000.0)])
def test_rope_apply_positions(hd, theta):
    print(f"rope_apply hd={hd}", flush=True)
    rng = np.random.default_rng(hd)
    for pos in (1, 3, 17, 63):
        x = rng.standard_normal(hd).astype(np.float32)
        d = Dev(x)
        lib().atlas_rope_apply_f32(d.ptr, pos, hd, theta)
        got = d.get().astype(np.float64)
        ref = _rope_apply_ref(x, pos, hd, theta)
        assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref)), pos
        # rotate-half pairs (i, i + hd/2) keep their norm; adjacent pairs would not
        half = hd // 2
        n_in = x[:half].astype(np.float64) ** 2 + x[half:].astype(np.float64) ** 2
        n_out = got[:half] ** 2 + got[half:] ** 2
        assert np.max(np.abs(n_out - n_in)) <= 1e-5 * np.max(n_in)
    # position 1, dimension pair 0 turns by exactly one radian (freq_0 = 1)
    x = np.zeros(hd, np.float32)
    x[0] = 1.0
    d = Dev(x)
    lib().atlas_rope_apply_f32(d.ptr, 1, hd, theta)
    g = d.get()
    assert abs(g[0] - math.cos(1.0)) < 1e-6 and abs(g[hd // 2] - math.sin(1.0)) < 1e-6


# ---------------------------------------------------------------------------
# argmax, quantisers, initialisers
# ---------------------------------------------------------------------------

def test_argmax_tie_rule_and_values(orc):
    from atlas_amd.tensor import GpuVec, gpu_argmax
    assert gpu_argmax(GpuVec.from_slice([1.0, 3.0, 3.0, 2.0])) == 2
    rng = np.random.default_rng(0)
    for n in (100278, 1, 257, 300000):
        x = rng.standard_normal(n).astype(np.float32)
        if n > 10:
            x[n // 3] = x[n - 5] = x.max() + 1.0      # tie: the later index wins
        dx, do = Dev(x), Dev.empty(1, np.uint32)
        assert lib().atlas_argmax_u32(dx.ptr, n, do.ptr) == 0
        assert int(do.get()[0]) == orc.argmax(x)


def test_device_quantisers_bit_exact(orc):
    rng = np.random.default_rng(12)
    w = (rng.standard_normal((257, 192)) * 0.02).astype(np.float32)
    w[3] = 0.0                                      # all-zero row -> scale 1
    w[5, :10] = [127 * 0.01, 2.5 * 0.01, -2.5 * 0.01, 0, 0, 0, 0, 0, 0, 0]
    q_ref, s_ref = orc.int8_quantize(w)
    # every device buffer stays referenced until the results are read back
    dw, dq, ds = Dev(w), Dev.empty(w.shape, np.int8), Dev.empty(257)
    assert lib().atlas_quantize_int8_dev(dw.ptr, 0, 257, 192, dq.ptr, ds.ptr) == 0
    assert np.array_equal(dq.get(), q_ref) and np.array_equal(ds.get(), s_ref)
    for bs in (32, 64, 50):
        q4, s4 = orc.int4_quantize(w, bs)
        d4, d4s = Dev.empty(q4.shape, np.uint8), Dev.empty(s4.shape)
        assert lib().atlas_quantize_int4_dev(dw.ptr, 0, w.size, bs, d4.ptr, d4s.ptr) == 0
        assert np.array_equal(d4.get(), q4) and np.array_equal(d4s.get(), s4), bs
    # bf16-bits input quantises the widened values
    bits = orc.bf16_from_f32(w)
    q_ref, s_ref = orc.int8_quantize(orc.bf16_to_f32(bits))
    dbits = Dev(bits)
    assert lib().atlas_quantize_int8_dev(dbits.ptr, 1, 257, 192, dq.ptr, ds.ptr) == 0
    assert np.array_equal(dq.get(), q_ref) and np.array_equal(ds.get(), s_ref)


def test_fill_random_distribution():
    n = 1 << 20
    d = Dev.empty(n)
    assert lib().atlas_fill_random(0, d.ptr, n, 7, 0.0, 0.02) == 0
    v = d.get().astype(np.float64)
    assert abs(v.mean()) < 1e-4 and abs(v.std() - 0.02) < 1e-4
    assert lib().atlas_fill_random(2, d.ptr, n, 7, 0.5, 1.5) == 0
    u = d.get()
    assert u.min() >= 0.5 and u.max() < 1.5 and abs(u.mean() - 1.0) < 2e-3


def test_errors_are_reported():
    from atlas_amd._lib import AtlasError, check
    with pytest.raises(AtlasError):
        check(lib().atlas_gemv_i4_f32(None, None, 32, None, None, 4, 32))
    assert lib().atlas_gemv_f32(7, None, None, 0, None, None, 0, 0) == 0   # empty is a no-op


# ---------------------------------------------------------------------------
# fused-prologue GEMVs (residual RMSNorm, RMSNorm, SwiGLU folded into x)
# ---------------------------------------------------------------------------

def _stored(orc, fmt, w, bs=32):
    M, K = w.shape
    if fmt == "bf16":
        b = orc.bf16_from_f32(w)
        return orc.MatView.bf16(b, M, K), Dev(b), None, 1, 0
    if fmt == "int8":
        q, s = orc.int8_quantize(w)
        return orc.MatView.int8(q, s), Dev(q), Dev(s), 2, 0
    q, s = orc.int4_quantize(w, bs)
    return orc.MatView.int4(q, s, M, K, bs), Dev(q), Dev(s), 3, bs


@pytest.mark.parametrize("fmt", ["bf16", "int8", "int4"])
@pytest.mark.parametrize("M,K", [(12288, 4096), (100278, 4096), (333, 1024), (4096, 11008)])
def test_gemv_fused_prologues(orc, fmt, M, K):
    print(f"gemv_fused {fmt} M={M} K={K}", flush=True)
    rng = np.random.default_rng(M + K)
    view, dw, ds, fid, bs = _stored(orc, fmt, _w((M, K), M * 7 + K))
    x = rng.standard_normal(K).astype(np.float32)
    y = rng.standard_normal(K).astype(np.float32) * 3.0
    nw = rng.uniform(0.5, 1.5, K).astype(np.float32)
    dx, dyv, dnw = Dev(x), Dev(y), Dev(nw)
    out, xo = Dev.empty(M), Dev.empty(K)
    L = lib()
    # residual norm: x' = x + rmsnorm(y) * w
    xr = x + orc.rmsnorm(y, nw, 1e-6)
    assert L.atlas_gemv_fused_f32(fid, dw.ptr, ds.ptr if ds else None, bs, dx.ptr, out.ptr, M, K,
                                  1, dyv.ptr, dnw.ptr, 1e-6, xo.ptr) == 0
    assert np.max(np.abs(xo.get() - xr)) <= 1e-5 * np.max(np.abs(xr))
    assert rel_err(out.get(), orc.linear(view, xr, threads=8)) <= GEMV_TOL
    # rmsnorm prologue
    xn = orc.rmsnorm(x, nw, 1e-5)
    assert L.atlas_gemv_fused_f32(fid, dw.ptr, ds.ptr if ds else None, bs, dx.ptr, out.ptr, M, K,
                                  2, None, dnw.ptr, 1e-5, xo.ptr) == 0
    assert np.max(np.abs(xo.get() - xn)) <= 1e-5 * np.max(np.abs(xn))
    assert rel_err(out.get(), orc.linear(view, xn, threads=8)) <= GEMV_TOL
    # silu prologue over interleaved pairs
    pairs = rng.standard_normal(2 * K).astype(np.float32) * 2.0
    xs = np.array([orc.silu(float(g)) for g in pairs[0::2]], np.float32) * pairs[1::2]
    dp = Dev(pairs)
    assert L.atlas_gemv_fused_f32(fid, dw.ptr, ds.ptr if ds else None, bs, None, out.ptr, M, K,
                                  3, dp.ptr, None, 0.0, None) == 0
    assert rel_err(out.get(), orc.linear(view, xs, threads=8)) <= GEMV_TOL


@pytest.mark.parametrize("H,KVH,hd,ctx,window,splits,chunk", [
    (32, 8, 128, 512, 0, 0, 0), (32, 8, 128, 4096, 0, 0, 0), (32, 8, 128, 16384, 0, 0, 0),
    (32, 8, 128, 16384, 4096, 0, 0), (32, 8, 128, 1, 0, 0, 0), (32, 8, 128, 300, 64, 7, 0),
    (32, 32, 128, 200, 0, 4, 0), (8, 8, 64, 77, 0, 3, 0), (4, 1, 64, 50, 16, 1, 0),
    (8, 2, 256, 90, 0, 5, 0), (16, 2, 128, 1000, 0, 64, 0),
    # min_chunk: fewer active splits than the grid holds
    (32, 8, 128, 4096, 0, 64, 1024), (32, 32, 128, 200, 0, 16, 64), (32, 8, 128, 1, 0, 16, 256),
    (32, 32, 128, 700, 0, 16, 256), (8, 2, 256, 3000, 1000, 8, 300), (8, 8, 64, 129, 0, 4, 64)])
def test_attention_fused(orc, H, KVH, hd, ctx, window, splits, chunk):
    print(f"attention_fused H={H} KVH={KVH} hd={hd} ctx={ctx} w={window} s={splits} c={chunk}",
          flush=True)
    rng = np.random.default_rng(ctx * 7 + hd)
    max_seq = ctx + 2
    yarn = dict(factor=8.0, orig_max_pos=8192, attn_factor=1.2079441541679836,
                beta_fast=32.0, beta_slow=1.0)
    cos, sin, _ = orc.rope_tables(hd, max_seq, 500000.0, yarn)
    pos = ctx - 1
    K = np.zeros((max_seq, KVH, hd), np.float32)
    V = np.zeros((max_seq, KVH, hd), np.float32)
    K[:pos] = rng.standard_normal((pos, KVH, hd))
    V[:pos] = rng.standard_normal((pos, KVH, hd))
    qkv = rng.standard_normal((H + 2 * KVH) * hd).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, H * hd).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, KVH * hd).astype(np.float32)
    # oracle: QK-norm, RoPE, cache write at pos, attention
    q = orc.qk_norm(qkv[:H * hd], qn, H, hd, 1e-6)
    k = orc.qk_norm(qkv[H * hd:(H + KVH) * hd], kn, KVH, hd, 1e-6)
    q = np.concatenate([orc.rope_apply(q[h * hd:(h + 1) * hd], cos[pos], sin[pos]) for h in range(H)])
    k = np.concatenate([orc.rope_apply(k[h * hd:(h + 1) * hd], cos[pos], sin[pos]) for h in range(KVH)])
    Kr, Vr = K.copy(), V.copy()
    Kr[pos] = k.reshape(KVH, hd)
    Vr[pos] = qkv[(H + KVH) * hd:].reshape(KVH, hd)
    scale = 1.2079441541679836 / math.sqrt(hd)
    ref = orc.attention(q, Kr, Vr, H, KVH, hd, pos, scale, window)
    d_qkv, dqn, dkn, dc, ds = Dev(qkv), Dev(qn), Dev(kn), Dev(cos), Dev(sin)
    dk, dv, do = Dev(K), Dev(V), Dev.empty(H * hd)
    for rep in range(2):          # a second launch reuses the merge counters
        assert lib().atlas_attention_fused_f32(d_qkv.ptr, dqn.ptr, dkn.ptr, 1e-6, dc.ptr, ds.ptr,
                                               dk.ptr, dv.ptr, do.ptr, H, KVH, hd, pos, scale,
                                               window, splits, chunk) == 0
        assert rel_err(do.get(), ref) <= ATTN_TOL, rep
    assert np.max(np.abs(dk.get()[pos] - Kr[pos])) <= 1e-5 * np.max(np.abs(k))
    assert np.array_equal(dv.get()[pos], Vr[pos])


# ---------------------------------------------------------------------------
# the streaming-floor measurement entry (bench.py's gemv_vs_stream_floor)
# ---------------------------------------------------------------------------

def test_bench_stream_floor_runs_and_rejects_bad_sizes():
    lib().atlas_clear_error()                            # an earlier test's refusal may still be recorded
    buf = Dev.empty((16 << 20) // 4)                     # 16 MiB
    us = C.c_float(-1.0)
    # a graph of 8 launches of 4 MiB over the buffer, at 2 blocks per CU
    assert lib().atlas_bench_stream_floor(C.c_void_p(buf.ptr), 16 << 20, 4 << 20, 8, 2,
                                          C.byref(us)) == 0
    # 4 MiB at 8 TB/s would be 0.5 us; a launch also pays its fixed cost
    assert 0.5 < us.value < 1000.0, us.value
    assert lib().atlas_last_error_code() == 0, lib().atlas_last_error()
    # 0 bytes: an empty kernel of the same grid (the launch floor), cheaper
    # than a launch that streams 4 MiB; buf may be null
    empty = C.c_float(-1.0)
    assert lib().atlas_bench_stream_floor(None, 0, 0, 8, 2, C.byref(empty)) == 0
    assert 0.0 < empty.value < us.value, (empty.value, us.value)
    for nbytes in (4 << 20 | 4096, 32 << 20):            # not whole 16 KiB groups, past the buffer
        assert lib().atlas_bench_stream_floor(C.c_void_p(buf.ptr), 16 << 20, nbytes, 8, 2,
                                              C.byref(us)) < 0, nbytes
    assert lib().atlas_bench_stream_floor(C.c_void_p(buf.ptr), 16 << 20, 4 << 20, 0, 2,
                                          C.byref(us)) < 0
    lib().atlas_clear_error()                            # the refusals above recorded errors


# ---------------------------------------------------------------------------
# library scratch and graph capture
# ---------------------------------------------------------------------------

def _hip_runtime():
    """The HIP runtime this process's atlas library uses (the same loaded
    copy, found in /proc/self/maps), for stream capture from the test."""
    path = None
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64.so" in line:
                path = line.split()[-1]
                break
    assert path, "libamdhip64 is not loaded"
    hip = C.CDLL(path)
    for name in ("hipStreamCreate", "hipStreamDestroy", "hipStreamBeginCapture",
                 "hipStreamEndCapture", "hipGraphInstantiate", "hipGraphLaunch",
                 "hipStreamSynchronize", "hipGraphExecDestroy", "hipGraphDestroy"):
        getattr(hip, name).restype = C.c_int
    return hip


def test_scratch_growth_refused_under_capture():
    """A fresh thread's first atlas_gpu_argmax needs library scratch; under a
    stream capture that growth is refused (ATLAS_EUNSUPPORTED) instead of
    recording an allocation into the caller's graph.  After one eager call
    of the same shape the captured call works, and every replay matches the
    eager result."""
    import threading
    hip = _hip_runtime()
    n = 100278
    x = np.random.default_rng(41).standard_normal(n).astype(np.float32)
    x[777] = 9.0
    res = {}

    def capture(st, fn):
        """Capture fn() on stream st (global mode); returns the graph exec."""
        graph, exe = C.c_void_p(), C.c_void_p()
        assert hip.hipStreamBeginCapture(st, 0) == 0
        fn()
        assert hip.hipStreamEndCapture(st, C.byref(graph)) == 0
        assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, C.c_size_t(0)) == 0
        return graph, exe

    def worker():
        st = C.c_void_p()
        try:
            dx, d_eager, d_graph = Dev(x), Dev.empty(2), Dev.empty(2)
            assert hip.hipStreamCreate(C.byref(st)) == 0
            lib().atlas_set_thread_stream(st)
            res["bytes_before"] = lib().atlas_thread_scratch_bytes()
            g1, e1 = capture(st, lambda: lib().atlas_gpu_argmax(dx.ptr, d_graph.ptr, n))
            res["code"] = lib().atlas_last_error_code()
            res["msg"] = lib().atlas_last_error().decode()
            lib().atlas_clear_error()
            res["bytes_refused"] = lib().atlas_thread_scratch_bytes()
            hip.hipGraphExecDestroy(e1)
            hip.hipGraphDestroy(g1)
            # warm-up on the same thread, then capture
            lib().atlas_gpu_argmax(dx.ptr, d_eager.ptr, n)
            lib().atlas_stream_sync()
            check_void()
            res["bytes_warm"] = lib().atlas_thread_scratch_bytes()
            eager = d_eager.get()
            g2, e2 = capture(st, lambda: lib().atlas_gpu_argmax(dx.ptr, d_graph.ptr, n))
            check_void()
            replays = []
            for _ in range(3):
                lib().atlas_memset_zero(d_graph.ptr, 8)        # eager work between replays
                lib().atlas_stream_sync()
                assert hip.hipGraphLaunch(e2, st) == 0
                assert hip.hipStreamSynchronize(st) == 0
                replays.append(d_graph.get())
            hip.hipGraphExecDestroy(e2)
            hip.hipGraphDestroy(g2)
            res["eager"], res["replays"] = eager, replays
        except BaseException as e:          # reported on the main thread
            res["exc"] = e
        finally:
            lib().atlas_clear_thread_stream()
            if st.value:
                hip.hipStreamSynchronize(st)
                hip.hipStreamDestroy(st)

    t = threading.Thread(target=worker)
    t.start()
    t.join()
    if "exc" in res:
        raise res["exc"]
    assert res["bytes_before"] == 0
    assert res["code"] == -4, res          # ATLAS_EUNSUPPORTED
    assert "captured" in res["msg"]
    assert res["bytes_refused"] == 0
    assert res["bytes_warm"] > 0
    assert res["eager"][0] == 777.0          # the index, as a float (lib.rs:107-126)
    for r in res["replays"]:
        assert np.array_equal(r, res["eager"])
