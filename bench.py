"""Benchmark of the decode hot path on one MI355X.

Headline (BASELINE.json metric "decode GEMV HBM GB/s (% of peak) + tok/s,
7B OLMo-shape bf16/int8/int4"): greedy batch-1 decode of a random-init
OLMo-3-7B-shaped model (32 layers, d 4096, 32/32 heads of 128, SwiGLU 11008,
vocab 100278, post-norm, QK-norm, YaRN, 24 sliding-window layers) with bf16
weights, after a 128-token random prompt.  One step = one decoded token
(every weight GEMV, attention over the KV cache, lm_head, device argmax).
`value` = tok/s of the K timed steps (weights resident in HBM).

Also reported: the int8 model's tok/s, the GEMV/attention microbenchmarks of
BASELINE.json configs 1-4 (GB/s against the 8 TB/s HBM peak, each timed over
>= 1 GiB of rotating buffers so the 256 MB Infinity Cache cannot serve them),
the roofline of the dominant kernel (the bf16 decode GEMV) and the CPU
baseline: the oracle's restatement of the reference CPU path on one host
core, timed on one 7B decode step of the same weights.

Usage: python bench.py [--gpus 1] [--steps 256] [--warmup 16] [--quick]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of each bf16 decode GEMV kernel: rocprofv3 FETCH_SIZE x 2
# + WRITE_SIZE x 1 (the factors a 1 GiB copy reads on this part), measured by
# `bench.py --pmc-probe` (profiles/gemv_7b_counters.md).
TRAFFIC = {"gate_up": 180980000, "qkv": 101250000, "w_o": 33830000, "w_down": 90680000,
           "lm_head": 822270000}
ROOT = os.path.dirname(os.path.abspath(__file__))
SPREAD: dict = {}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


class DevBufs:
    """`count` rotating device copies of one host array (via the C ABI)."""

    def __init__(self, lib, host: np.ndarray, count: int):
        self.lib, self.ptrs, self.nbytes = lib, [], host.nbytes
        for _ in range(count):
            p = C.c_void_p()
            assert lib.atlas_dev_malloc_sync(C.byref(p), max(host.nbytes, 4)) == 0
            assert lib.atlas_memcpy_h2d(p.value, _p(host), host.nbytes) == 0
            self.ptrs.append(p.value)

    def free(self):
        for p in self.ptrs:
            self.lib.atlas_dev_free_sync(p)
        self.ptrs = []


def time_launches(torch, fn, n_iter: int, warm: int = 3) -> float:
    """Average ms per call of fn(i), HIP events on the library's stream."""
    for i in range(warm):
        fn(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(n_iter):
        fn(i)
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / n_iter


def time_graph(torch, lib, fn, n_launch: int, replays: int = 5) -> float:
    """Average ms per call of fn(i), i < n_launch, captured into one HIP graph on
    a torch capture stream (the library's launches follow it through
    atlas_set_thread_stream) and replayed: the launch gaps of a graph, as the
    decode step runs its kernels, without the host's per-call enqueue cost."""
    s = torch.cuda.Stream()
    fn(0)                                   # any first-use work outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        assert lib.atlas_set_thread_stream(C.c_void_p(s.cuda_stream)) == 0
        try:
            for i in range(n_launch):
                fn(i)
        finally:
            lib.atlas_clear_thread_stream()
    g.replay()
    torch.cuda.synchronize()
    best = None
    for _ in range(replays):
        # replay() launches on the current stream: the events go there too
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        e1.synchronize()
        ms = e0.elapsed_time(e1) / n_launch
        best = ms if best is None else min(best, ms)
    del g
    return best


def launch_spread(torch, fn, n_iter: int) -> dict:
    """p10 / median / p90 of the per-call time of fn(i) over n_iter >= 100
    back-to-back calls, from a HIP event recorded after every call.  This is a
    second pass: each event adds ~2.5 us to its call on MI355X (measured: the
    median sits that far above the plain pass's mean), so the spread's width
    is the information here and the plain pass's mean stays the time."""
    n_iter = max(100, n_iter)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n_iter + 1)]
    torch.cuda.synchronize()
    ev[0].record()
    for i in range(n_iter):
        fn(i)
        ev[i + 1].record()
    ev[-1].synchronize()
    d = np.array([ev[i].elapsed_time(ev[i + 1]) for i in range(n_iter)]) * 1e3
    return {"p10_us": round(float(np.percentile(d, 10)), 2),
            "median_us": round(float(np.median(d)), 2),
            "p90_us": round(float(np.percentile(d, 90)), 2), "launches": n_iter,
            "note": "an event after every call (~2.5 us each): read the width, not the level"}


def gemv_bench(torch, lib, orc_free_rng, quick: bool) -> dict:
    """Configs 1-3: batch-1 GEMVs and the int4 skinny GEMM, GB/s."""
    out = {}
    rng = orc_free_rng
    cases = [("bf16_4096x4096", 1, 4096, 4096, 0), ("int8_11008x4096", 2, 11008, 4096, 0),
             ("int8_4096x11008", 2, 4096, 11008, 0), ("int4_4096x4096_bs32", 3, 4096, 4096, 32),
             ("int4_11008x4096_bs32", 3, 11008, 4096, 32)]
    for name, fmt, M, K, bs in cases:
        if fmt == 1:
            data = rng.integers(0, 65535, (M, K), dtype=np.uint16)
            data = (data & 0x807F) | 0x3C00            # finite bf16 of modest size
            scales = None
            wbytes = M * K * 2
        elif fmt == 2:
            data = rng.integers(-127, 128, (M, K), dtype=np.int8)
            scales = rng.uniform(1e-4, 2e-4, M).astype(np.float32)
            wbytes = M * K + 4 * M
        else:
            data = rng.integers(0, 256, M * K // 2, dtype=np.uint8)
            scales = rng.uniform(1e-3, 2e-3, M * K // bs).astype(np.float32)
            wbytes = M * K // 2 + 4 * (M * K // bs)
        alg = wbytes + 4 * K + 4 * M
        copies = max(2, int(np.ceil(1.1e9 / wbytes)))
        if quick:
            copies = max(2, copies // 4)
        W = DevBufs(lib, data, copies)
        S = DevBufs(lib, scales, copies) if scales is not None else None
        X = DevBufs(lib, rng.standard_normal(K).astype(np.float32), 1)
        Y = DevBufs(lib, np.zeros(M, np.float32), 1)

        def run(i, W=W, S=S, X=X, Y=Y, fmt=fmt, M=M, K=K, bs=bs, copies=copies):
            j = i % copies
            rc = lib.atlas_gemv_f32(fmt, W.ptrs[j], S.ptrs[j] if S else None, bs, X.ptrs[0],
                                    Y.ptrs[0], M, K)
            assert rc == 0

        ms = time_launches(torch, run, copies * (3 if quick else 10))
        gbs = alg / (ms * 1e-3) / 1e9
        ms_g = time_graph(torch, lib, run, copies * 2)
        gbs_g = alg / (ms_g * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 2), "GB_s": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 3), "bytes": alg, "rotating_copies": copies,
                     "graph_us": round(ms_g * 1e3, 2), "graph_GB_s": round(gbs_g, 1),
                     "graph_frac": round(gbs_g / HBM_PEAK_GBS, 3),
                     "spread": launch_spread(torch, run, copies * (3 if quick else 10))}
        sp = out[name]["spread"]
        log(f"gemv {name}: {ms * 1e3:.2f} us  {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%}); "
            f"in a graph {ms_g * 1e3:.2f} us ({gbs_g / HBM_PEAK_GBS:.1%}); "
            f"per launch p10/median/p90 {sp['p10_us']}/{sp['median_us']}/{sp['p90_us']} us")
        W.free()
        if S:
            S.free()
        X.free()
        Y.free()
    # int4 skinny (ragged micro-batch) at 11008x4096
    M, K, bs = 11008, 4096, 32
    data = rng.integers(0, 256, M * K // 2, dtype=np.uint8)
    scales = rng.uniform(1e-3, 2e-3, M * K // bs).astype(np.float32)
    wbytes = M * K // 2 + 4 * (M * K // bs)
    copies = max(2, int(np.ceil(1.1e9 / wbytes)) // (4 if quick else 1))
    W, S = DevBufs(lib, data, copies), DevBufs(lib, scales, copies)
    for n in (1, 3, 5, 8):
        X = DevBufs(lib, rng.standard_normal((n, K)).astype(np.float32), 1)
        Y = DevBufs(lib, np.zeros((n, M), np.float32), 1)

        def run(i, X=X, Y=Y, n=n):
            j = i % copies
            assert lib.atlas_gemm_skinny_f32(3, W.ptrs[j], S.ptrs[j], bs, X.ptrs[0], Y.ptrs[0],
                                             M, n, K) == 0

        ms = time_launches(torch, run, copies * (2 if quick else 6))
        alg = wbytes + n * (4 * K + 4 * M)
        gbs = alg / (ms * 1e-3) / 1e9
        out[f"int4_skinny_n{n}_11008x4096_bs32"] = {
            "us": round(ms * 1e3, 2), "GB_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 3),
            "bytes": alg, "spread": launch_spread(torch, run, copies * (2 if quick else 6))}
        sp = out[f"int4_skinny_n{n}_11008x4096_bs32"]["spread"]
        log(f"skinny int4 n={n}: {ms * 1e3:.2f} us  {gbs:.0f} GB/s; per launch p10/median/p90 "
            f"{sp['p10_us']}/{sp['median_us']}/{sp['p90_us']} us")
        X.free()
        Y.free()
    W.free()
    S.free()
    return out


def attention_bench(torch, lib, rng, quick: bool) -> dict:
    """Config 4: GQA 32 q / 8 kv heads of 128, f32 cache, one query token."""
    H, KVH, hd = 32, 8, 128
    out = {}
    for ctx, window in ((512, 0), (4096, 0), (16384, 0), (16384, 4096)):
        eff = min(ctx, window) if window else ctx
        alg = 2 * eff * KVH * hd * 4 + 2 * H * hd * 4
        cache_bytes = ctx * KVH * hd * 4
        copies = max(2, int(np.ceil(1.1e9 / (2 * cache_bytes))) // (4 if quick else 1))
        kv = rng.standard_normal((ctx, KVH, hd)).astype(np.float32)
        Kc, Vc = DevBufs(lib, kv, copies), DevBufs(lib, kv, copies)
        Q = DevBufs(lib, rng.standard_normal(H * hd).astype(np.float32), 1)
        O = DevBufs(lib, np.zeros(H * hd, np.float32), 1)

        def run(i):
            j = i % copies
            lib.atlas_decode_attention(Q.ptrs[0], Kc.ptrs[j], Vc.ptrs[j], O.ptrs[0], H, KVH, hd,
                                       ctx - 1, 0.1067, window)

        ms = time_launches(torch, run, copies * (3 if quick else 10))
        assert lib.atlas_last_error_code() == 0, lib.atlas_last_error()
        gbs = alg / (ms * 1e-3) / 1e9
        key = f"ctx{ctx}" + (f"_w{window}" if window else "")
        out[key] = {"us": round(ms * 1e3, 2), "GB_s": round(gbs, 1),
                    "frac": round(gbs / HBM_PEAK_GBS, 3), "bytes": alg,
                    "spread": launch_spread(torch, run, copies * (3 if quick else 10))}
        sp = out[key]["spread"]
        log(f"attention {key}: {ms * 1e3:.2f} us  {gbs:.0f} GB/s; per launch p10/median/p90 "
            f"{sp['p10_us']}/{sp['median_us']}/{sp['p90_us']} us")
        Kc.free(); Vc.free(); Q.free(); O.free()
    return out


PREFILL = {}      # weight format -> prompt prefill timings of decode_bench


def host_slice_bench(rng) -> dict:
    """GpuMatrix::sgemm, the reference's host-slice path (crates/atlas-tensor/
    src/lib.rs:371-400): x uploaded, the GEMV, y downloaded, per call; beside
    it sgemm_vec on device-resident x.  bf16 4096 x 4096."""
    from atlas_amd.tensor import GpuMatrix, GpuVec
    M = K = 4096
    w = (rng.standard_normal(M * K) * 0.02).astype(np.float32)
    g = GpuMatrix.upload_bf16(w, M, K)
    x = rng.standard_normal(K).astype(np.float32)
    out = np.empty((M, 1), np.float32)
    xv = GpuVec.from_slice(x)
    for _ in range(5):
        g.sgemm(x.reshape(K, 1), K, 1, out)
        g.sgemm_vec(xv)
    iters = 200
    t0 = time.perf_counter()
    for _ in range(iters):
        g.sgemm(x.reshape(K, 1), K, 1, out)
    host_us = (time.perf_counter() - t0) / iters * 1e6
    t0 = time.perf_counter()
    for _ in range(iters):
        y = g.sgemm_vec(xv)
    y.download() if hasattr(y, "download") else None
    dev_us = (time.perf_counter() - t0) / iters * 1e6
    wbytes = M * K * 2
    log(f"GpuMatrix.sgemm (host slices in/out) bf16 4096x4096: {host_us:.1f} us/call "
        f"({wbytes / (host_us * 1e-6) / 1e9:.0f} GB/s of weights); sgemm_vec (device x): "
        f"{dev_us:.1f} us/call incl. host dispatch")
    return {"shape": "bf16 4096x4096", "host_slices_us_per_call": round(host_us, 2),
            "host_slices_weight_GB_s": round(wbytes / (host_us * 1e-6) / 1e9, 1),
            "device_vec_us_per_call": round(dev_us, 2)}


def decode_bench(model_mod, fmt: int, prompt, steps: int, warmup: int, seed: int):
    import dataclasses
    cfg = dataclasses.replace(model_mod.ModelConfig.olmo3_actual_7b(),
                              max_seq_len=len(prompt) + warmup + steps + 8)
    m = model_mod.OlmoModel(cfg, weight_format=fmt, int4_block=32)
    t0 = time.perf_counter()
    m.init_random(seed)
    log(f"fmt {fmt}: random init {time.perf_counter() - t0:.1f}s, "
        f"{m.weight_bytes() / 1e9:.2f} GB of weights in HBM")
    # the prompt: token by token (the reference's loop), then through the
    # multi-row prefill step; the second leaves the state the decode continues
    pre = {}
    # 128-row chunks take hipBLASLt (bf16, int8) or the tiled MFMA GEMM (int4)
    for chunk in (1, 16, 128):
        m.reset()
        m.set_prefill_chunk(chunk)
        # capture the step graphs (and, for 128, run the eager chunk once)
        m.prefill([int(t) for t in prompt[:4 if chunk <= 16 else -1]])
        m.reset()
        t0 = time.perf_counter()
        m.prefill([int(t) for t in prompt[:-1]])
        dt_p = time.perf_counter() - t0
        pre["token_by_token_s" if chunk == 1 else f"chunk{chunk}_s"] = round(dt_p, 4)
        log(f"fmt {fmt}: prompt of {len(prompt) - 1} tokens prefilled {chunk} per step in "
            f"{dt_p * 1e3:.1f} ms ({(len(prompt) - 1) / dt_p:.0f} tok/s)")
    pre["tokens"] = len(prompt) - 1
    for chunk in (16, 128):
        if f"chunk{chunk}_s" in pre:
            pre[f"chunk{chunk}_tok_s"] = round((len(prompt) - 1) / pre[f"chunk{chunk}_s"], 1)
    PREFILL[fmt] = pre
    # the timed region: `steps` greedy steps, one graph replay each, with the
    # stream idle on entry (the warm-up call synchronises) and synchronised on
    # exit; no event between the steps (each costs 6-10 us of stream time)
    toks = m.decode_greedy(int(prompt[-1]), warmup)
    first = int(toks[-1]) if warmup else int(prompt[-1])
    t0 = time.perf_counter()
    toks2 = m.decode_greedy(first, steps)
    dt = time.perf_counter() - t0
    assert len(toks2) == steps
    # the per-step spread: the same positions again, an event after every step
    m.reset()
    m.prefill([int(t) for t in prompt[:-1]])
    m.decode_greedy(int(prompt[-1]), warmup)
    toks3, step_ms = m.decode_greedy_timed(first, steps)
    SPREAD[fmt] = step_spread(step_ms)
    SPREAD[fmt]["same_tokens_as_timed_run"] = bool(np.array_equal(toks2, toks3))
    return m, dt


_FLOOR_BUF = []


def stream_floor(lib, m) -> dict:
    """Each decode GEMV role of model m (eager launches, atlas_model_bench_gemv)
    beside the streaming floor of a launch of the same bytes: a graph of
    read-only launches with the bf16 decode GEMV's work split and load pattern
    (atlas_bench_stream_floor, best of 2-4 blocks per CU).  The difference is
    what the GEMV's own work costs per launch."""
    if not _FLOOR_BUF:
        p = C.c_void_p()
        nbytes = 2 << 30
        assert lib.atlas_dev_malloc_sync(C.byref(p), nbytes) == 0
        assert lib.atlas_fill_random(2, p.value, nbytes // 4, 11, 0.0, 1.0) == 0
        _FLOOR_BUF.extend([p.value, nbytes])
    buf, nbytes = _FLOOR_BUF
    out = {}
    for which, role in ((4, "qkv"), (5, "w_o"), (3, "gate_up"), (2, "w_down"), (6, "lm_head")):
        ms, launches, b = C.c_float(), C.c_int(), C.c_int64()
        iters = 32 if which == 6 else 8
        assert lib.atlas_model_bench_gemv(m._h, 1, which, C.byref(ms), C.byref(launches), C.byref(b)) == 0
        assert lib.atlas_model_bench_gemv(m._h, iters, which, C.byref(ms), C.byref(launches),
                                          C.byref(b)) == 0
        gemv_us = ms.value / launches.value * 1e3
        per = b.value // (launches.value // iters)
        size = max(16384, per // 16384 * 16384)
        best = None
        for bpc in (2, 3, 4):
            us = C.c_float()
            n = 16 if size > 400e6 else 64
            assert lib.atlas_bench_stream_floor(C.c_void_p(buf), nbytes, size, n, bpc, C.byref(us)) == 0, \
                lib.atlas_last_error()
            best = us.value if best is None else min(best, us.value)
        out[role] = {"MB": round(per / 1e6, 2), "gemv_us": round(gemv_us, 2), "floor_us": round(best, 2),
                     "gemv_over_floor": round(gemv_us / best, 3)}
        log(f"stream floor {role}: {per / 1e6:.1f} MB, GEMV {gemv_us:.2f} us, floor {best:.2f} us "
            f"({gemv_us / best:.3f}x)")
    return out


def launch_floor(lib) -> dict:
    """What any launch costs in a graph of back-to-back launches on this part,
    before GEMV work: an empty kernel of a decode GEMV's grid, and read-only
    launches with the GEMV's work split at 10.5-180 MB, with a line fitted
    through the sizes from 33.6 MB (fixed microseconds + bytes / streaming
    rate).  A single launch of B bytes can reach at most B / floor(B) of HBM
    bandwidth; the 75% target needs launches of about 80 MB or more."""
    if not _FLOOR_BUF:
        p = C.c_void_p()
        nbytes = 2 << 30
        assert lib.atlas_dev_malloc_sync(C.byref(p), nbytes) == 0
        assert lib.atlas_fill_random(2, p.value, nbytes // 4, 11, 0.0, 1.0) == 0
        _FLOOR_BUF.extend([p.value, nbytes])
    buf, nbytes = _FLOOR_BUF
    us = C.c_float()
    empty = None
    for bpc in (2, 4):
        assert lib.atlas_bench_stream_floor(None, 0, 0, 64, bpc, C.byref(us)) == 0, lib.atlas_last_error()
        empty = us.value if empty is None else min(empty, us.value)
    sizes = (10518528, 33587200, 100728832, 180355072)
    pts = []
    for size in sizes:
        best = None
        for bpc in (2, 3, 4):
            assert lib.atlas_bench_stream_floor(C.c_void_p(buf), nbytes, size, 16, bpc, C.byref(us)) == 0, \
                lib.atlas_last_error()
            best = us.value if best is None else min(best, us.value)
        pts.append((size, best))
    xs = np.array([p[0] for p in pts if p[0] >= 30e6], dtype=np.float64)
    ys = np.array([p[1] for p in pts if p[0] >= 30e6], dtype=np.float64)
    slope, fixed = np.polyfit(xs, ys, 1)        # us per byte, us
    out = {"empty_kernel_us": round(empty, 3),
           "fit": {"fixed_us": round(float(fixed), 3), "stream_TB_s": round(1e-6 / float(slope), 3),
                   "from_MB": [round(x / 1e6, 2) for x in xs]},
           "by_size": {f"{s / 1e6:.2f}MB": {"us": round(t, 3), "GB_s": round(s / t / 1e3, 1),
                                            "max_frac_of_peak": round(s / t / 1e3 / HBM_PEAK_GBS, 3)}
                       for s, t in pts}}
    log(f"launch floor: empty kernel {empty:.2f} us; read floor {fixed:.2f} us + bytes / "
        f"{1e-6 / slope:.2f} TB/s; " + ", ".join(f"{s / 1e6:.1f} MB {t:.2f} us" for s, t in pts))
    return out


def step_spread(step_ms) -> dict:
    """Median and p10/p90 of the per-step GPU times (HIP events recorded on
    the engine stream after every step of a second run over the timed run's
    positions)."""
    a = np.asarray(step_ms, np.float64)
    return {"p10_ms": round(float(np.percentile(a, 10)), 4),
            "median_ms": round(float(np.median(a)), 4),
            "p90_ms": round(float(np.percentile(a, 90)), 4),
            "mean_ms": round(float(a.mean()), 4), "steps": int(a.size)}


def generate_rates(m, am) -> dict:
    """End-to-end rates of the reference's own forms on the loaded 7B model:
    n / elapsed(generate(&[1, 2, 3], n, 0.0)) with n = 30
    (crates/atlas-model/src/lib.rs:4312-4316; prompt, host loop and logits
    included), the same with SamplingConfig::default() (lib.rs:1223-1276)
    and SamplingConfig::olmo3() (lib.rs:1278-1294), and the greedy hooked
    generate (a host callback after every layer, lib.rs:1452-1461)."""
    from atlas_amd.model import SamplingConfig
    m.reset()
    m.generate([1, 2, 3], 4, 0.0)                   # captures, warm
    n = 30
    m.reset()
    t0 = time.perf_counter()
    out = m.generate([1, 2, 3], n, 0.0)
    ref_style = n / (time.perf_counter() - t0)
    assert len(out) == n
    seen = [0]

    def hook(li, h):
        seen[0] += 1
        return None

    # SamplingConfig::default() (temperature 1, top_k 0: the whole vocabulary)
    # and the OLMo-3 preset, both sampled on the device inside the step
    m.set_rng_seed(5)
    m.generate_with_sampling([1, 2, 3], 4, SamplingConfig())
    rates = {}
    for name, sc in (("default", SamplingConfig()), ("olmo3", SamplingConfig.olmo3())):
        m.set_rng_seed(7)
        t0 = time.perf_counter()
        got = m.generate_with_sampling([1, 2, 3], n, sc)
        rates[name] = len(got) / (time.perf_counter() - t0)
    nh = 16
    m.reset()
    m.generate_with_sampling_hooked([1, 2, 3], 2, SamplingConfig.greedy(), hook)
    m.reset()
    seen[0] = 0
    t0 = time.perf_counter()
    outh, _ = m.generate_with_sampling_hooked([1, 2, 3], nh, SamplingConfig.greedy(), hook)
    hooked = len(outh) / (time.perf_counter() - t0)
    log(f"generate([1,2,3], {n}, 0.0): {ref_style:.1f} tok/s; sampled with SamplingConfig::default(): "
        f"{rates['default']:.1f} tok/s, olmo3 preset: {rates['olmo3']:.1f} tok/s; hooked generate: "
        f"{hooked:.1f} tok/s ({seen[0]} hook calls for {len(outh)} tokens)")
    return {"reference_style_tok_s": round(ref_style, 2),
            "reference_style_form": "n / elapsed(generate([1,2,3], n=30, temperature 0.0))",
            "default_sampling_tok_s": round(rates["default"], 2),
            "olmo3_sampling_tok_s": round(rates["olmo3"], 2),
            "hooked_generate_tok_s": round(hooked, 2), "hooked_tokens": len(outh)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--quick", action="store_true", help="fewer microbenchmark iterations")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-micro", action="store_true")
    ap.add_argument("--no-ragged", action="store_true", help="skip the ragged batch of config 5")
    ap.add_argument("--loader", action="store_true",
                    help="also time the checkpoint loader on a 7B-shaped 4-layer bf16 "
                         "safetensors checkpoint (writes ~3.3 GB to a temporary directory)")
    ap.add_argument("--loader-only", action="store_true", help="only the loader measurement")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="short program for rocprofv3 --pmc passes: a 1 GiB device copy "
                         "(calibration), then one launch set of each decode GEMV kernel of the "
                         "bf16, int8 and int4 7B models and two decode steps each")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the decode path runs on a single MI355X and multi-GPU sharding is design-only",
              file=sys.stderr)
        return 2

    import torch
    import atlas_amd
    from atlas_amd import model as am

    lib = atlas_amd.load()
    if not lib.atlas_cuda_available():
        print("bench.py: no HIP device", file=sys.stderr)
        return 1
    torch.cuda.init()
    lib.atlas_set_stream(C.c_void_p(torch.cuda.current_stream().cuda_stream))
    rng = np.random.default_rng(2026)
    prompt = rng.integers(0, 100278, 128)
    if args.pmc_probe:
        return pmc_probe(torch, lib, am)
    if args.loader_only:
        print(json.dumps({"checkpoint_load": loader_bench(torch, am)}), flush=True)
        return 0

    micro = {}
    attn = {}
    host_slice = None
    if not args.no_micro:
        micro = gemv_bench(torch, lib, rng, args.quick)
        attn = attention_bench(torch, lib, rng, args.quick)
        host_slice = host_slice_bench(rng)

    # ---- headline: bf16 7B decode -------------------------------------------
    m, dt = decode_bench(am, am.W_BF16, prompt, args.steps, args.warmup, seed=7)
    ms_step = dt * 1e3 / args.steps
    tok_s = args.steps / dt
    wbytes = m.weight_bytes()
    log(f"bf16 decode: {ms_step:.3f} ms/token, {tok_s:.1f} tok/s, "
        f"weights {wbytes / 1e9:.2f} GB -> {wbytes / (ms_step * 1e-3) / 1e9:.0f} GB/s")

    # The step's bf16 GEMVs, role by role (QKV, W_o, gate/up, W_down and
    # lm_head launch the same kernel template at different shapes); the
    # roofline is reported for the role that takes the most time per step
    # (gate/up: 42% of the weight bytes), the others beside it.
    def gemv_set(which, iters=8):
        ms, launches, nbytes = C.c_float(), C.c_int(), C.c_int64()
        assert lib.atlas_model_bench_gemv(m._h, 1, which, C.byref(ms), C.byref(launches),
                                          C.byref(nbytes)) == 0
        assert lib.atlas_model_bench_gemv(m._h, iters, which, C.byref(ms), C.byref(launches),
                                          C.byref(nbytes)) == 0
        per_launch_ms = ms.value / launches.value
        per_launch_bytes = nbytes.value / (launches.value / iters)
        return (per_launch_ms, per_launch_bytes, ms.value / iters, launches.value // iters)

    kernels = {}
    for which, name, kern in (
            (3, "gate_up", "gemv_v4_kernel<bf16, rows 2, unroll 4> (RMSNorm+residual prologue, "
                           "SwiGLU epilogue)"),
            (4, "qkv", "gemv_v4_kernel<bf16, rows 2, unroll 4> (RMSNorm+residual prologue)"),
            (5, "w_o", "gemv_v4_kernel<bf16, rows 2, unroll 4>"),
            (2, "w_down", "gemv_v4_kernel<bf16, rows 1, unroll 4> (rows padded to 22272 B)"),
            (6, "lm_head", "gemv_v4_kernel<bf16, rows 2, unroll 4> (RMSNorm prologue)")):
        per_ms, per_bytes, step_ms, n = gemv_set(which, 8 if which != 6 else 32)
        gbs = per_bytes / (per_ms * 1e-3) / 1e9
        kernels[name] = {"kernel": kern, "launches_per_step": n, "ms_per_step": round(step_ms, 4),
                         "traffic": TRAFFIC.get(name),
                         "bytes_per_launch": int(per_bytes), "us_per_launch": round(per_ms * 1e3, 3),
                         "GB_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"decode GEMVs {name}: {n} launches/step, {step_ms:.3f} ms, {per_ms * 1e3:.2f} us and "
            f"{per_bytes / 1e6:.2f} MB per launch, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%})")
    step_gemv_ms = sum(k["ms_per_step"] for k in kernels.values())
    all_gbs = sum(k["bytes_per_launch"] * k["launches_per_step"] for k in kernels.values()) / (
        step_gemv_ms * 1e-3) / 1e9
    dom = max(kernels.values(), key=lambda k: k["ms_per_step"])
    log(f"decode GEMVs: {step_gemv_ms:.3f} ms/step, {all_gbs:.0f} GB/s")

    # roofline share of the whole step: weights + KV at 8 TB/s vs measured
    ctx_mid = len(prompt) + args.warmup + args.steps // 2
    kv_bytes = 0
    for li in range(32):
        eff = ctx_mid if li % 4 == 3 else min(ctx_mid, 4096)
        kv_bytes += 2 * eff * 32 * 128 * 4
    step_bytes = wbytes + kv_bytes + 100278 * 4
    step_floor_ms = step_bytes / (HBM_PEAK_GBS * 1e9) * 1e3

    floor = {"bf16": stream_floor(lib, m)}
    lfloor = launch_floor(lib)
    rates = generate_rates(m, am)
    # bench the GPU CPU-baseline inputs before freeing the model
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(m, am, prompt, "bf16")
    m.close()
    del m

    # ---- int8 and int4 models ------------------------------------------------
    quant = {}
    for fmt, name in ((am.W_INT8, "int8"), (am.W_INT4, "int4")):
        mq, dtq = decode_bench(am, fmt, prompt, args.steps, args.warmup, seed=7)
        wq = mq.weight_bytes()
        quant[name] = {"tok_s": round(args.steps / dtq, 2),
                       "ms_per_step": round(dtq * 1e3 / args.steps, 4),
                       "weight_bytes": int(wq),
                       "weight_GB_s": round(wq / (dtq / args.steps) / 1e9, 1)}
        quant[name]["step_spread"] = SPREAD.get(fmt)
        log(f"{name} decode: {dtq * 1e3 / args.steps:.3f} ms/token, {args.steps / dtq:.1f} tok/s, "
            f"weights {wq / 1e9:.2f} GB")
        if name == "int8" and cpu is not None:
            cpu["int8"] = cpu_baseline(mq, am, prompt, "int8")
        floor[name] = stream_floor(lib, mq)
        mq.close()
        del mq

    ragged = None
    if not args.no_ragged:
        ragged = ragged_bench(am, rng, args.quick)
    load_res = loader_bench(torch, am) if args.loader else None

    res = {
        "metric": "decode GEMV HBM GB/s (% of peak) + tok/s, 7B OLMo-shape bf16/int8/int4",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 weights, f32 activations/accumulation",
        "data": "synthetic: random-init weights N(0,0.02) (bf16 by truncation), norms U(0.5,1.5), "
                "128 random prompt ids",
        "config": {"workload": "OLMo-3-7B-shaped greedy decode, batch 1, bf16 weights "
                               "(BASELINE.json configs[4])",
                   "global_batch": 1, "seq_len": len(prompt) + args.warmup + args.steps,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": dom["GB_s"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": dom["frac"], "traffic": dom["traffic"],
                     "kernel": dom["kernel"],
                     "bytes_per_launch": dom["bytes_per_launch"],
                     "us_per_launch": dom["us_per_launch"]},
        "gemv_kernels": kernels,
        "gemv_vs_stream_floor": floor,
        "launch_floor": lfloor,
        "step_spread": SPREAD.get(am.W_BF16),
        "generate_rates": rates,
        "step_roofline": {"bytes_per_step": int(step_bytes),
                          "floor_ms": round(step_floor_ms, 4),
                          "frac_of_step_at_roofline": round(step_floor_ms / ms_step, 4),
                          "gemv_ms_per_step": round(step_gemv_ms, 4),
                          "gemv_all_GB_s": round(all_gbs, 1)},
        "int8": quant["int8"],
        "int4": quant["int4"],
        "ragged_batch": ragged,
        "prefill_bf16": PREFILL.get(am.W_BF16),
        "prefill_int8": PREFILL.get(am.W_INT8),
        "prefill_int4": PREFILL.get(am.W_INT4),
        "checkpoint_load": load_res,
        "gemv_microbench": micro,
        "attention_microbench": attn,
        "host_slice_sgemm": host_slice,
        "reference_published": {"olmo3_7b_bf16_tok_s": 61.7, "hardware": "A100-SXM4-40GB"},
    }
    if cpu:
        res["cpu_baseline"] = cpu
    print(json.dumps(res), flush=True)
    return 0


def ragged_bench(am, rng, quick: bool) -> dict:
    """Config 5's ragged batch: 8 greedy sequences with prompts of 16..2048
    random ids decoded together, bf16 weights.  Each step runs up to 8 rows:
    one per live sequence, the spare rows taking further prompt tokens of the
    sequences with the most prompt left (atlas_model_generate_batch)."""
    import dataclasses
    lens = [16, 64, 128, 256, 512, 1024, 1536, 2048]
    max_new = 64 if quick else 256
    cfg = dataclasses.replace(am.ModelConfig.olmo3_actual_7b(),
                              max_seq_len=max(lens) + max_new + 8)
    m = am.OlmoModel(cfg, weight_format=am.W_BF16, int4_block=32, max_batch=len(lens))
    m.init_random(7)
    prompts = [[int(t) for t in rng.integers(0, 100278, n)] for n in lens]
    t0 = time.perf_counter()
    out = m.generate_batch(prompts, max_new)
    dt = time.perf_counter() - t0
    gen = sum(len(o) for o in out)
    total = sum(lens) + gen
    res = {"sequences": len(lens), "prompt_lens": lens, "max_new": max_new,
           "generated_tokens": gen, "tokens_processed": total, "seconds": round(dt, 3),
           "tok_s_processed": round(total / dt, 1), "tok_s_generated": round(gen / dt, 1)}
    log(f"ragged batch: {len(lens)} sequences, {total} tokens ({gen} generated) in {dt:.2f} s "
        f"-> {total / dt:.0f} tok/s processed")
    m.close()
    return res


def loader_bench(torch, am, n_layers: int = 4) -> dict:
    """The checkpoint loader (load_model_from_dir) on a 7B-shaped bf16
    safetensors checkpoint cut to n_layers layers (embedding, lm_head and the
    layers' matrices at their real shapes) plus an OLMo-3 config.json,
    written to local disk first, so the load reads from the page cache.
    Roofline: the pinned host-to-device copy rate measured in the same run."""
    import dataclasses
    import json
    import shutil
    import struct
    import tempfile
    from atlas_amd import loader
    d, f, V = 4096, 11008, 100278
    cfg7 = am.ModelConfig.olmo3_actual_7b()
    cfg = dataclasses.replace(cfg7, n_layers=n_layers, layer_types=cfg7.layer_types[:n_layers],
                              max_seq_len=256)
    tensors = [("model.embed_tokens.weight", (V, d))]
    for li in range(n_layers):
        p = f"model.layers.{li}."
        tensors += [(p + "self_attn.q_proj.weight", (d, d)), (p + "self_attn.k_proj.weight", (d, d)),
                    (p + "self_attn.v_proj.weight", (d, d)), (p + "self_attn.o_proj.weight", (d, d)),
                    (p + "mlp.gate_proj.weight", (f, d)), (p + "mlp.up_proj.weight", (f, d)),
                    (p + "mlp.down_proj.weight", (d, f)),
                    (p + "post_attention_layernorm.weight", (d,)),
                    (p + "post_feedforward_layernorm.weight", (d,)),
                    (p + "self_attn.q_norm.weight", (d,)), (p + "self_attn.k_norm.weight", (d,))]
    tensors += [("model.norm.weight", (d,)), ("lm_head.weight", (V, d))]
    # one 64 MiB block of N(0, 0.02) bf16 values, repeated through every tensor
    blk = (np.random.default_rng(1).standard_normal(32 << 20) * 0.02).astype(np.float32)
    blk = (blk.view(np.uint32) >> 16).astype(np.uint16)
    hdr, off = {}, 0
    for name, shape in tensors:
        nb = int(np.prod(shape)) * 2
        hdr[name] = {"dtype": "BF16", "shape": list(shape), "data_offsets": [off, off + nb]}
        off += nb
    tmp = tempfile.mkdtemp(prefix="atlas_ckpt_")
    res = {}
    try:
        t0 = time.perf_counter()
        h = json.dumps(hdr).encode()
        with open(os.path.join(tmp, "model.safetensors"), "wb") as fo:
            fo.write(struct.pack("<Q", len(h)) + h)
            for name, shape in tensors:
                n = int(np.prod(shape))
                while n > 0:
                    k = min(n, blk.size)
                    fo.write(blk[:k].tobytes())
                    n -= k
        with open(os.path.join(tmp, "config.json"), "w") as fo:
            json.dump({"layer_types": ["sliding_attention" if t == "sliding" else "full_attention"
                                       for t in cfg.layer_types],
                       "sliding_window": 4096, "rope_theta": 500000.0, "rms_norm_eps": 1e-6,
                       "rope_scaling": {"rope_type": "yarn", "factor": 8.0,
                                        "original_max_position_embeddings": 8192,
                                        "attention_factor": 1.2079441541679836,
                                        "beta_fast": 32.0, "beta_slow": 1.0},
                       "eos_token_id": 100257}, fo)
        file_bytes = os.path.getsize(os.path.join(tmp, "model.safetensors"))
        log(f"loader: wrote {file_bytes / 1e9:.2f} GB checkpoint in {time.perf_counter() - t0:.1f} s")
        # pinned host -> device copy rate (the transfer roofline)
        src = torch.empty(1 << 30, dtype=torch.uint8, pin_memory=True)
        dst = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst.copy_(src, non_blocking=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(4):
            dst.copy_(src, non_blocking=True)
        torch.cuda.synchronize()
        h2d = 4 * (1 << 30) / (time.perf_counter() - t0) / 1e9
        del src, dst
        res = {"file_bytes": file_bytes, "layers": n_layers, "h2d_pinned_GB_s": round(h2d, 1)}
        log(f"loader: pinned host-to-device copy {h2d:.1f} GB/s")
        t0 = time.perf_counter()
        am.OlmoModel(cfg, weight_format=am.W_BF16).close()
        res["create_seconds"] = round(time.perf_counter() - t0, 3)
        log(f"loader: creating the model alone {res['create_seconds']:.3f} s")
        for fmt, name in ((am.W_BF16, "bf16"), (am.W_BF16, "bf16_again"), (am.W_INT8, "int8"),
                          (am.W_INT4, "int4")):
            t0 = time.perf_counter()
            m = loader.load_model_from_dir(tmp, cfg, weight_format=fmt)
            dt = time.perf_counter() - t0
            assert m.eos_token_id == 100257 and m.config.post_norm and m.config.qk_norm
            m.close()
            gbs = file_bytes / dt / 1e9
            res[name] = {"seconds": round(dt, 3), "GB_s": round(gbs, 2),
                         "frac_of_h2d": round(gbs / h2d, 3)}
            log(f"loader: {name} residency {dt:.2f} s, {gbs:.2f} GB/s ({gbs / h2d:.0%} of H2D)")
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return res


def pmc_probe(torch, lib, am) -> int:
    """Dispatches whose counters calibrate and measure the decode kernels:
    three copies of 1 GiB (2 GiB moved each: FETCH_SIZE and WRITE_SIZE of a
    plain copy of known size), then for the bf16, int8 and int4 7B models one
    launch of each GEMV set (bench_gemv which = 3 gate/up, 1 QKV + W_o +
    lm_head, 2 W_down) and two decode steps at positions 1 and 2 (attention,
    argmax) and a 127-token prompt in one 128-row chunk, twice (prompt GEMMs
    and prompt attention; the first chunk also times the library GEMM's
    candidates); then int4 11008 x 4096 as one batch-1 GEMV and the
    skinny GEMM at 4 and 8 rows; last, the reference-ABI decode attention of
    BASELINE config 4 (GQA 32/8/128, f32 cache) at ctx 512, 4096 and 16384.
    Kernels are told apart by name and grid size."""
    n = 1 << 28
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"pmc probe: copy of {n * 4} bytes x3 done")
    del src, dst
    for fmt, name in ((am.W_BF16, "bf16"), (am.W_INT8, "int8"), (am.W_INT4, "int4")):
        import dataclasses
        cfg = dataclasses.replace(am.ModelConfig.olmo3_actual_7b(), max_seq_len=256)
        m = am.OlmoModel(cfg, weight_format=fmt, int4_block=32)
        m.init_random(7)
        m.reset()
        m.forward_one(1)
        ms, launches, nbytes = C.c_float(), C.c_int(), C.c_int64()
        for which in (3, 1, 2):
            assert lib.atlas_model_bench_gemv(m._h, 1, which, C.byref(ms), C.byref(launches),
                                              C.byref(nbytes)) == 0
            log(f"pmc probe {name}: GEMV set {which}: {launches.value} launches, {nbytes.value} "
                f"algorithmic bytes, {ms.value:.3f} ms")
        m.forward_one(2)
        m.forward_one(3)
        torch.cuda.synchronize()
        m.set_prefill_chunk(128)
        # twice: the first chunk also times the library GEMM's candidates
        # (bf16, int8); the second is the steady state
        for _ in range(2):
            m.reset()
            m.prefill(list(range(100, 227)))
        torch.cuda.synchronize()
        log(f"pmc probe {name}: 127-token prompt chunk done (twice)")
        m.close()
    # int4 11008 x 4096 (block 32): batch-1 GEMV, then the skinny GEMM at 4
    # and 8 rows, each on its own copy of the weights
    M, K, bs = 11008, 4096, 32
    rng = np.random.default_rng(5)
    W = DevBufs(lib, rng.integers(0, 256, M * K // 2, dtype=np.uint8), 3)
    S = DevBufs(lib, rng.uniform(1e-3, 2e-3, M * K // bs).astype(np.float32), 3)
    X = DevBufs(lib, rng.standard_normal((8, K)).astype(np.float32), 1)
    Y = DevBufs(lib, np.zeros((8, M), np.float32), 1)
    assert lib.atlas_gemv_f32(3, W.ptrs[0], S.ptrs[0], bs, X.ptrs[0], Y.ptrs[0], M, K) == 0
    for j, n in ((1, 4), (2, 8)):
        assert lib.atlas_gemm_skinny_f32(3, W.ptrs[j], S.ptrs[j], bs, X.ptrs[0], Y.ptrs[0], M, n,
                                         K) == 0
    torch.cuda.synchronize()
    log(f"pmc probe int4 {M}x{K}: GEMV, skinny n=4, skinny n=8 done "
        f"({M * K // 2 + 4 * M * K // bs} algorithmic weight bytes each)")
    for b in (W, S, X, Y):
        b.free()
    H, KVH, hd = 32, 8, 128
    for ctx in (512, 4096, 16384):
        kv = rng.standard_normal((ctx, KVH, hd)).astype(np.float32)
        Kc, Vc = DevBufs(lib, kv, 1), DevBufs(lib, kv, 1)
        Q = DevBufs(lib, rng.standard_normal(H * hd).astype(np.float32), 1)
        O = DevBufs(lib, np.zeros(H * hd, np.float32), 1)
        for _ in range(2):
            lib.atlas_decode_attention(Q.ptrs[0], Kc.ptrs[0], Vc.ptrs[0], O.ptrs[0], H, KVH, hd, ctx - 1,
                                       C.c_float(0.1067), 0)
        torch.cuda.synchronize()
        assert lib.atlas_last_error_code() == 0, lib.atlas_last_error()
        log(f"pmc probe: decode attention GQA {H}/{KVH}/{hd} ctx {ctx} x2 done "
            f"({2 * ctx * KVH * hd * 4} K/V bytes each)")
        for b in (Kc, Vc, Q, O):
            b.free()
    return 0


def cpu_info() -> dict:
    """The host the CPU baseline ran on: its CPU model and core counts."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(),
            "cores_available": len(os.sched_getaffinity(0))}


CPU_POS = 140        # inside the timed decode's contexts (128-token prompt + steps)


def cpu_baseline(m, am, prompt, fmt: str) -> dict:
    """The oracle (restatement of the reference CPU path) on one 7B decode
    step of the same weights (bf16, or int8 with its row scales), downloaded
    from the GPU, at position CPU_POS: the oracle and the engine get the same
    seeded KV-cache rows for positions 0..CPU_POS-1, so the timed CPU step
    includes attention over CPU_POS + 1 positions in every layer, and the
    GPU step over the same state is compared with it.  The process is pinned
    to one host core for the timed step."""
    sys.path.insert(0, ROOT)
    import oracle as orc
    d, V, L, f = 4096, 100278, 32, 11008
    t0 = time.perf_counter()
    shapes = {am.T_WQ: (d, d), am.T_WK: (d, d), am.T_WV: (d, d), am.T_WO: (d, d),
              am.T_W_GATE: (f, d), am.T_W_UP: (f, d), am.T_W_DOWN: (d, f)}
    names = {am.T_WQ: "wq", am.T_WK: "wk", am.T_WV: "wv", am.T_WO: "wo", am.T_W_GATE: "w_gate",
             am.T_W_UP: "w_up", am.T_W_DOWN: "w_down"}

    def mat(k, li, shp):
        if fmt == "bf16":
            return orc.MatView.bf16(m.get_tensor(k, li, shp, np.uint16), *shp)
        q, sc = m.get_tensor(k, li, shp, np.int8, n_scales=shp[0])
        return orc.MatView.int8(q, sc)

    layers = []
    for li in range(L):
        ld = {names[k]: mat(k, li, shp) for k, shp in shapes.items()}
        ld["attn_norm"] = m.get_tensor(am.T_ATTN_NORM, li, (d,), np.float32)
        ld["ffn_norm"] = m.get_tensor(am.T_FFN_NORM, li, (d,), np.float32)
        ld["q_norm"] = m.get_tensor(am.T_Q_NORM, li, (d,), np.float32)
        ld["k_norm"] = m.get_tensor(am.T_K_NORM, li, (d,), np.float32)
        layers.append(ld)
    emb = orc.MatView.bf16(m.get_tensor(am.T_EMBED, 0, (V, d), np.uint16), V, d)
    lm = mat(am.T_LM_HEAD, 0, (V, d))
    fn = m.get_tensor(am.T_FINAL_NORM, 0, (d,), np.float32)
    log(f"cpu baseline ({fmt}): weights downloaded in {time.perf_counter() - t0:.1f}s")
    ocfg = dict(vocab=V, d_model=d, n_layers=L, n_heads=32, n_kv_heads=32, ffn_hidden=f,
                max_seq=CPU_POS + 8, rope_theta=500000.0, rms_eps=1e-6,
                yarn=dict(factor=8.0, orig_max_pos=8192, attn_factor=1.2079441541679836,
                          beta_fast=32.0, beta_slow=1.0),
                sliding_window=4096, layer_sliding=[0 if i % 4 == 3 else 1 for i in range(L)],
                post_norm=True)
    om = orc.Model(ocfg, dict(embed=emb, lm_head=lm, final_norm=fn, layers=layers), threads=1)
    # the same cache rows in both (K, V ~ N(0, 1)), then both at CPU_POS
    krng = np.random.default_rng(140)
    m.reset()
    for li in range(L):
        k = krng.standard_normal((CPU_POS, 32 * 128), dtype=np.float32)
        v = krng.standard_normal((CPU_POS, 32 * 128), dtype=np.float32)
        m.set_kv_rows(li, 0, k, v)
        om.set_kv_rows(li, 0, k, v)
    m.set_pos(CPU_POS)
    om.set_pos(CPU_POS)
    tok = int(prompt[0])
    info = cpu_info()
    # one core for the timed step (in-process: the affinity of this thread,
    # which runs the single-threaded oracle), restored afterwards
    saved = os.sched_getaffinity(0)
    core = min(saved)
    os.sched_setaffinity(0, {core})
    try:
        t0 = time.perf_counter()
        logits = om.forward_one(tok)
        dt = time.perf_counter() - t0
    finally:
        os.sched_setaffinity(0, saved)
    # the same token and state through the GPU engine (a sanity line; the
    # parity tests carry the parity claims)
    glog = m.forward_one(tok)
    agree = int(np.argmax(glog[::-1])) == int(np.argmax(logits[::-1]))
    rel = float(np.max(np.abs(glog - logits)) / np.max(np.abs(logits)))
    log(f"cpu baseline ({fmt}): one 7B decode step at pos {CPU_POS} on core {core} of "
        f"{info['cpu_model']} in {dt:.1f}s; GPU/CPU logits rel err {rel:.2e}, top-1 "
        f"{'agrees' if agree else 'DIFFERS'}")
    return {"value": round(1.0 / dt, 5), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"one OLMo-3-7B-shaped {fmt} decode step at position {CPU_POS} (all 32 "
                      f"layers with attention over {CPU_POS + 1} cached positions, lm_head) of "
                      "the same weights, oracle/oracle.c single-threaded, pinned to one core",
            "pinned_core": core, "position": CPU_POS, **info,
            "seconds": round(dt, 2), "gpu_vs_cpu_logit_rel_err": rel, "top1_agrees": agree}


if __name__ == "__main__":
    sys.exit(main())
