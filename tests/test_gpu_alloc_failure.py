"""Allocation failure, forced from the host (atlas_debug_fail_allocations).

The reference's contract for a failed device allocation is an Option / bool
that sends the caller to its CPU path (crates/atlas-tensor/src/lib.rs:
193-207, 371-400, 409-435).  Here every entry point that allocates returns
ATLAS_ENOMEM instead, frees what it had taken, and leaves the model usable.
The switch makes the chosen allocation fail before HIP is asked, so no
kernel ever runs out of memory for real.
"""
import ctypes as C
import threading

import numpy as np
import pytest

from atlas_amd._lib import AtlasError
from tests import modelgen
from tests.gpu_util import Dev, lib

pytestmark = pytest.mark.gpu

ENOMEM = -3


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import atlas_amd
    atlas_amd.load()
    if not lib().atlas_cuda_available():
        pytest.fail("no HIP device visible: GPU tests need an MI355X")
    yield
    lib().atlas_debug_fail_allocations(0, 0)


@pytest.fixture(autouse=True)
def _switch_off():
    lib().atlas_debug_fail_allocations(0, 0)
    lib().atlas_clear_error()
    yield
    lib().atlas_debug_fail_allocations(0, 0)
    lib().atlas_clear_error()


def _free_bytes():
    """hipMemGetInfo of the HIP runtime the library uses."""
    path = None
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64.so" in line:
                path = line.split()[-1]
                break
    hip = C.CDLL(path)
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipDeviceSynchronize() == 0
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def test_model_create_fails_cleanly_at_every_allocation():
    from atlas_amd import model as am
    cfg = am.ModelConfig.tiny()
    # one full create / forward / destroy first: the kernels' code objects and
    # HIP's own pools are then loaded, so the memory check below sees only
    # what the failed creates might have kept
    m = am.OlmoModel(cfg)
    m.init_random(3)
    m.forward_one(5)
    m.close()
    before = _free_bytes()
    failures = 0
    for k in range(400):
        print(f"create with allocation {k} failing", flush=True)
        lib().atlas_debug_fail_allocations(k, 1)
        try:
            m = am.OlmoModel(cfg)
        except AtlasError as e:
            assert e.code == ENOMEM, (k, e)
            failures += 1
            continue
        lib().atlas_debug_fail_allocations(0, 0)
        m.close()
        break
    else:
        pytest.fail("create never succeeded")
    assert failures == k and k > 20, k          # every allocation of create was tried
    # nothing the failed creates took is still held (HIP's own pools may keep
    # a little, so a few MiB of slack)
    after = _free_bytes()
    print(f"{k} allocations in create; free device memory {before} -> {after}", flush=True)
    assert after >= before - (16 << 20)
    m = am.OlmoModel(cfg)                       # and the next create works
    m.init_random(3)
    lg = m.forward_one(5)
    assert np.all(np.isfinite(lg))
    m.close()


def _small():
    cfg = modelgen.olmo3_small_config(n_layers=2)
    W = modelgen.make_weights(cfg, seed=9, fmt="bf16")
    return W, modelgen.engine_model(W)


def test_generate_enomem_then_usable(orc):
    from atlas_amd.model import SamplingConfig
    W, m = _small()
    # 100 suppressed tokens outgrow the model's 64-entry device list, so this
    # generate has to allocate
    s = SamplingConfig.greedy()
    s.suppress_initial_tokens = list(range(100, 200))
    prompt = [1, 2, 3]
    lib().atlas_debug_fail_allocations(0, 1)
    with pytest.raises(AtlasError) as e:
        m.generate_with_sampling(prompt, 8, s)
    assert e.value.code == ENOMEM
    lib().atlas_debug_fail_allocations(0, 0)
    toks = m.generate_with_sampling(prompt, 8, s)
    want = modelgen.oracle_model(W, threads=4).generate_greedy(prompt, 8, suppress=range(100, 200))
    assert toks == want, (toks, want)
    # and with the plain greedy settings again
    assert m.generate_with_sampling(prompt, 8, SamplingConfig.greedy()) == \
        modelgen.oracle_model(W, threads=4).generate_greedy(prompt, 8)


def test_hooked_forward_enomem_then_usable(orc):
    W, m = _small()
    o = modelgen.oracle_model(W, threads=4)
    m.reset()
    lib().atlas_debug_fail_allocations(0, 1)        # the per-layer hidden-state buffer
    with pytest.raises(AtlasError) as e:
        m.forward_one_hidden(7)
    assert e.value.code == ENOMEM
    lib().atlas_debug_fail_allocations(0, 0)
    m.reset()
    lg, hid = m.forward_one_hidden(7)
    ref, rhid = o.forward_one(7, hidden=True)
    assert np.max(np.abs(lg - ref)) <= 1e-3 * np.max(np.abs(ref))
    assert np.max(np.abs(hid - rhid)) <= 1e-3 * np.max(np.abs(rhid))


def test_tensor_mirror_option_contract():
    # lib.rs:193-207: a failed allocation is None / false, never an exception
    from atlas_amd import tensor as t
    lib().atlas_debug_fail_allocations(0, 1)
    assert t.GpuBuf.alloc(1024) is None
    lib().atlas_debug_fail_allocations(0, 1)
    mat = t.GpuMatrix.upload(np.ones(12, np.float32), 4, 3)
    assert not mat.is_on_gpu()
    out = np.zeros(4, np.float32)
    assert mat.sgemm(np.ones(3, np.float32), 3, 1, out) is False
    ok = t.GpuMatrix.upload(np.arange(12, dtype=np.float32), 4, 3)
    assert ok.is_on_gpu()
    lib().atlas_debug_fail_allocations(0, 1)        # the rhs upload inside sgemm
    assert ok.sgemm(np.ones(3, np.float32), 3, 1, out) is False
    assert ok.sgemm(np.ones(3, np.float32), 3, 1, out) is True
    assert out.tolist() == [3.0, 12.0, 21.0, 30.0]


def test_library_scratch_enomem_then_usable():
    # a fresh thread's first argmax grows its scratch: refused, then it works
    x = np.random.default_rng(5).standard_normal(5000).astype(np.float32)
    x[1234] = 50.0
    res = {}

    def worker():
        try:
            dx, do = Dev(x), Dev.empty(2)
            lib().atlas_debug_fail_allocations(0, 1)
            lib().atlas_gpu_argmax(dx.ptr, do.ptr, x.size)
            res["code"] = lib().atlas_last_error_code()
            lib().atlas_clear_error()
            lib().atlas_debug_fail_allocations(0, 0)
            res["bytes"] = lib().atlas_thread_scratch_bytes()
            lib().atlas_gpu_argmax(dx.ptr, do.ptr, x.size)
            lib().atlas_stream_sync()
            res["code2"] = lib().atlas_last_error_code()
            res["idx"] = do.get()[0]
        except BaseException as e:
            res["exc"] = e

    t = threading.Thread(target=worker)
    t.start()
    t.join()
    if "exc" in res:
        raise res["exc"]
    assert res["code"] == ENOMEM and res["bytes"] == 0
    assert res["code2"] == 0 and res["idx"] == 1234.0
