"""The no-allocation decode attention entry point against the allocating one.

atlas_decode_attention_noalloc takes the arguments of atlas_decode_attention
(crates/atlas-tensor/src/lib.rs:80-86) and the same split count, with its
split partials in the library's fixed device workspace.  Two calls in a row,
the second with a smaller input (the workspace keeps the first call's
contents), made first and from a fresh thread that must end them holding no
library scratch, must match the allocating entry point within the attention
tolerance (2e-3 * max|o|) and the oracle; a shape whose partials exceed the
workspace is refused with ATLAS_EINVAL.
"""
import math
import threading

import numpy as np
import pytest

from tests.gpu_util import Dev, lib, rel_err, sync

pytestmark = pytest.mark.gpu

ATTN_TOL = 2e-3


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import atlas_amd
    atlas_amd.load()
    if not lib().atlas_cuda_available():
        pytest.fail("no HIP device visible: GPU tests need an MI355X")


def _case(H, KVH, hd, rows, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(H * hd).astype(np.float32)
    kc = rng.standard_normal((rows, KVH * hd)).astype(np.float32)
    vc = rng.standard_normal((rows, KVH * hd)).astype(np.float32)
    return q, kc, vc


def test_decode_attention_noalloc_matches_allocating_entry(orc):
    H, KVH, hd = 32, 8, 128
    scale = 1.2079441541679836 / math.sqrt(hd)
    # the second call is smaller: fewer positions and a window
    cases = ((16383, 0, 1), (700, 256, 2))
    bufs = []
    for pos, window, seed in cases:
        q, kc, vc = _case(H, KVH, hd, pos + 1, seed)
        bufs.append((q, kc, vc, Dev(q), Dev(kc), Dev(vc), Dev.empty(H * hd), Dev.empty(H * hd)))
    # The no-allocation calls come first, from a fresh thread with no library
    # scratch: they must leave it without any (nothing allocated on its behalf).
    res = {}

    def worker():
        try:
            res["before"] = lib().atlas_thread_scratch_bytes()
            for (pos, window, _), (_, _, _, dq, dk, dv, _, db) in zip(cases, bufs):
                print(f"noalloc attention pos={pos} window={window}", flush=True)
                res[pos] = lib().atlas_decode_attention_noalloc(dq.ptr, dk.ptr, dv.ptr, db.ptr,
                                                                H, KVH, hd, pos, scale, window)
            lib().atlas_stream_sync()
            res["after"] = lib().atlas_thread_scratch_bytes()
        except BaseException as e:          # reported on the main thread
            res["exc"] = e

    t = threading.Thread(target=worker)
    t.start()
    t.join()
    if "exc" in res:
        raise res["exc"]
    assert res["before"] == 0 and res["after"] == 0, res
    for (pos, window, _), (q, kc, vc, dq, dk, dv, da, db) in zip(cases, bufs):
        assert res[pos] == 0, pos
        lib().atlas_decode_attention(dq.ptr, dk.ptr, dv.ptr, da.ptr, H, KVH, hd, pos, scale,
                                     window)
        sync()
        a, b = da.get(), db.get()
        assert rel_err(b, a) <= ATTN_TOL
        ref = orc.attention(q, kc, vc, H, KVH, hd, pos, scale, window)
        assert rel_err(b, ref) <= ATTN_TOL


def test_decode_attention_noalloc_refuses_oversize(orc):
    # one KV head of dim 256 shared by 64 query heads at 16384 positions: 256
    # splits of partials need 64 * 256 * 258 * 4 bytes, above the workspace
    H, KVH, hd, pos = 64, 1, 256, 16383
    need = H * 256 * (hd + 2) * 4
    assert need > lib().atlas_decode_attention_noalloc_max_bytes()
    q, kc, vc = _case(H, KVH, hd, pos + 1, 3)
    dq, dk, dv, do = Dev(q), Dev(kc), Dev(vc), Dev.empty(H * hd)
    rc = lib().atlas_decode_attention_noalloc(dq.ptr, dk.ptr, dv.ptr, do.ptr, H, KVH, hd, pos,
                                              1.0 / math.sqrt(hd), 0)
    assert rc == -1
    assert b"workspace" in lib().atlas_last_error()
    lib().atlas_clear_error()
