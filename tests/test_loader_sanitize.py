"""The checkpoint parsers under AddressSanitizer and UndefinedBehaviorSanitizer
(CPU only).

atlas_amd/csrc/st_format.cpp (safetensors headers and data ranges,
config.json, the shard index) has no device code, so it is built here with
g++ -fsanitize=address,undefined -fno-sanitize-recover=all together with the
error state (errors.cpp) and the driver tests/sanitize/st_fuzz.cpp.  The
driver first replays a corpus -- every malformed file test_loader.py's error
tests feed the library, its range-error file, a tiny OLMo-3 checkpoint in one
and two shards with its index and config.json (ckptgen), and a few broken
configs -- then runs a seeded mutation fuzz (bit flips, truncations, JSON
tokens, header-length changes, deep nesting) through every query a caller can
make.  Any out-of-bounds access, leak or undefined behaviour aborts the run.
"""
import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, HERE)

FUZZ_ITERS = 6000
FUZZ_SEED = 20261202


def _sanitizer_toolchain():
    gxx = shutil.which("g++")
    if not gxx:
        return None
    lib = subprocess.run([gxx, "-print-file-name=libasan.so"], capture_output=True,
                         text=True).stdout.strip()
    return gxx if lib and os.path.sep in lib and os.path.exists(lib) else None


@pytest.fixture(scope="module")
def st_fuzz(tmp_path_factory):
    gxx = _sanitizer_toolchain()
    if gxx is None:
        pytest.skip("g++ with the AddressSanitizer runtime is not available")
    out = tmp_path_factory.mktemp("san") / "st_fuzz"
    csrc = os.path.join(ROOT, "atlas_amd", "csrc")
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-I", os.path.join(ROOT, "include"),
           os.path.join(csrc, "errors.cpp"), os.path.join(csrc, "st_format.cpp"),
           os.path.join(HERE, "sanitize", "st_fuzz.cpp"), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return str(out)


def _corpus(d):
    import ckptgen
    import modelgen
    from test_loader import _hdr, header_error_cases, range_error_file
    files = []

    def put(name, blob):
        p = os.path.join(d, name)
        with open(p, "wb") as f:
            f.write(blob)
        files.append(p)

    for k, (blob, _) in enumerate(header_error_cases()):
        put(f"header_error_{k}.bin", blob)
    put("range_errors.bin", range_error_file())
    put("not_object.bin", _hdr("[1, 2]"))
    cfg = modelgen.olmo3_small_config(n_layers=2, vocab=128, d_model=64, ffn_hidden=128)
    W = modelgen.make_weights(cfg, seed=5, fmt="bf16")
    t = ckptgen.hf_tensors(W)
    ckdir = os.path.join(d, "ckpt")
    ckptgen.write_dir(ckdir, t, shards=2, config=ckptgen.olmo3_config_json(cfg, eos=7))
    for name in sorted(os.listdir(ckdir)):
        files.append(os.path.join(ckdir, name))
    put("one_shard.safetensors", ckptgen.safetensors_bytes(t))
    bad = [(n, dt, sh, raw[:-4]) for n, dt, sh, raw in t]
    put("short_tensors.safetensors", ckptgen.safetensors_bytes(bad))
    for k, text in enumerate(['{"rope_scaling": {"rope_type": "yarn", "factor": "x"}}',
                              '{"layer_types": [1, null, "sliding_attention"], '
                              '"sliding_window": -5}',
                              '{"sliding_window": 1e300, "eos_token_id": 1.5}',
                              '{"rope_theta": 5e5, "rms_norm_eps": 1e-6', '']):
        put(f"config_{k}.json", text.encode())
    return files


def test_parsers_clean_under_asan_ubsan(st_fuzz, tmp_path):
    corpus = _corpus(str(tmp_path))
    work = tmp_path / "work"
    work.mkdir()
    env = dict(os.environ,
               ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([st_fuzz, str(work), str(FUZZ_ITERS), str(FUZZ_SEED)] + corpus,
                       capture_output=True, text=True, env=env, timeout=600)
    report = (r.stdout + r.stderr)[-4000:]
    assert "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, report
    assert r.returncode == 0, report
    assert "st_fuzz ok" in r.stdout, report
    print(r.stdout.strip())
