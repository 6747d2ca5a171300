"""ctypes binding of libatlas_kernels.so (include/atlas_kernels.h, include/atlas_engine.h).

The library is loaded from the package directory only.  There is no CPU
fallback: if the HIP library is missing or cannot be loaded, every entry
point raises :class:`AtlasError` -- a silent CPU path would hide that the
hot path is not running.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libatlas_kernels.so")


class AtlasError(RuntimeError):
    """A C-ABI call returned a negative ATLAS_E* code."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"atlas error {code}: {msg}")
        self.code = code


class ModelConfigC(C.Structure):
    _fields_ = [("vocab", C.c_int), ("d_model", C.c_int), ("n_layers", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("ffn_hidden", C.c_int),
                ("max_seq", C.c_int), ("rope_theta", C.c_float), ("rms_eps", C.c_float),
                ("yarn", C.c_int), ("yarn_factor", C.c_float), ("yarn_orig_max_pos", C.c_int),
                ("yarn_attn_factor", C.c_float), ("yarn_beta_fast", C.c_float),
                ("yarn_beta_slow", C.c_float), ("sliding_window", C.c_int),
                ("layer_sliding", C.c_void_p), ("post_norm", C.c_int), ("qk_norm", C.c_int),
                ("weight_format", C.c_int), ("int4_block", C.c_int), ("max_batch", C.c_int)]


class SamplingC(C.Structure):
    _fields_ = [("temperature", C.c_float), ("repetition_penalty", C.c_float),
                ("repetition_window", C.c_int), ("frequency_penalty", C.c_float),
                ("presence_penalty", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int),
                ("min_p", C.c_float), ("suppress_initial_tokens", C.c_void_p),
                ("n_suppress", C.c_int), ("eos_token_id", C.c_int64),
                ("extra_stop_tokens", C.c_void_p), ("n_extra_stop", C.c_int),
                ("rng_seed", C.c_uint64)]


HOOK_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.POINTER(C.c_float), C.c_int,
                      C.POINTER(C.c_float))
TOKEN_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_uint32)

P, I, F, SZ, I64, U64, U32 = (C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_int64,
                              C.c_uint64, C.c_uint32)

# name -> (restype, argtypes); int-returning calls are status codes
SIGNATURES = {
    # Part 1: reference FFI (crates/atlas-tensor/src/lib.rs:17-92)
    "atlas_matmul_f32": (None, [P, P, P, I, I, I]),
    "atlas_vec_add_f32": (None, [P, P, P, I]),
    "atlas_scale_f32": (None, [P, F, P, I]),
    "atlas_relu_f32": (None, [P, P, I]),
    "atlas_softmax_f32": (None, [P, P, I, I]),
    "atlas_cuda_available": (I, []),
    "atlas_cuda_device_count": (I, []),
    "atlas_rmsnorm_f32": (None, [P, P, P, I, F]),
    "atlas_rope_apply_f32": (None, [P, I, I, F]),
    "atlas_silu_mul_f32": (None, [P, P, P, I]),
    "atlas_vram_copy_f32": (None, [P, P, I]),
    "atlas_adamw_step": (None, [P, P, P, P, F, F, F, F, F, F, F, I]),
    "atlas_sgemm_bf16_f32": (None, [P, P, P, I, I, I]),
    "atlas_sync": (None, []),
    "atlas_qk_norm_inplace": (None, [P, P, I, I, F]),
    "atlas_rope_precomputed": (None, [P, P, P, I, I, I, I]),
    "atlas_kv_cache_write": (None, [P, P, P, P, I, I, I]),
    "atlas_decode_attention": (None, [P, P, P, P, I, I, I, I, F, I]),
    "atlas_gpu_argmax": (None, [P, P, I]),
    # Part 2: memory / runtime
    "atlas_last_error_code": (I, []),
    "atlas_last_error": (C.c_char_p, []),
    "atlas_clear_error": (None, []),
    "atlas_dev_malloc": (I, [C.POINTER(C.c_void_p), SZ]),
    "atlas_dev_free": (I, [P]),
    "atlas_dev_malloc_sync": (I, [C.POINTER(C.c_void_p), SZ]),
    "atlas_dev_free_sync": (I, [P]),
    "atlas_memcpy_h2d": (I, [P, P, SZ]),
    "atlas_memcpy_d2h": (I, [P, P, SZ]),
    "atlas_memcpy_d2d": (I, [P, P, SZ]),
    "atlas_memset_zero": (I, [P, SZ]),
    "atlas_set_device": (I, [I]),
    "atlas_set_stream": (I, [P]),
    "atlas_set_thread_stream": (I, [P]),
    "atlas_clear_thread_stream": (I, []),
    "atlas_get_stream": (P, []),
    "atlas_stream_sync": (I, []),
    "atlas_thread_scratch_bytes": (I64, []),
    "atlas_debug_fail_allocations": (I, [I, I]),
    "atlas_device_cu_count": (I, []),
    # Part 3: extensions
    "atlas_gemv_f32": (I, [I, P, P, I, P, P, I, I]),
    "atlas_gemv_bf16_f32": (I, [P, P, P, I, I]),
    "atlas_gemv_i8_f32": (I, [P, P, P, P, I, I]),
    "atlas_gemv_i4_f32": (I, [P, P, I, P, P, I, I]),
    "atlas_gemv_swiglu_f32": (I, [I, P, P, I, P, P, I, I]),
    "atlas_gemv_fused_f32": (I, [I, P, P, I, P, P, I, I, I, P, P, F, P]),
    "atlas_gemm_skinny_f32": (I, [I, P, P, I, P, P, I, I, I]),
    "atlas_gemm_skinny_swiglu_f32": (I, [I, P, P, I, P, P, I, I, I]),
    "atlas_rmsnorm_rows_f32": (I, [P, P, P, I, I, F]),
    "atlas_residual_rmsnorm_f32": (I, [P, P, P, I, I, F]),
    "atlas_qkv_post_f32": (I, [P, P, P, F, P, P, P, P, I, I, I, I]),
    "atlas_attention_fused_f32": (I, [P, P, P, F, P, P, P, P, P, I, I, I, I, F, I, I, I]),
    "atlas_decode_attention_noalloc": (I, [P, P, P, P, I, I, I, I, F, I]),
    "atlas_decode_attention_noalloc_max_bytes": (I64, []),
    "atlas_bench_stream_floor": (I, [P, I64, I64, I, I, P]),
    "atlas_argmax_u32": (I, [P, I, P]),
    "atlas_quantize_int8_dev": (I, [P, I, I, I, P, P]),
    "atlas_quantize_int4_dev": (I, [P, I, I64, I, P, P]),
    "atlas_quantize_int8_host": (I, [P, I64, I64, P, P]),
    "atlas_quantize_int4_host": (I, [P, I64, I64, I64, P, P]),
    "atlas_fill_random": (I, [I, P, I64, U64, F, F]),
    # engine (include/atlas_engine.h)
    "atlas_model_create": (P, [C.POINTER(ModelConfigC)]),
    "atlas_model_destroy": (None, [P]),
    "atlas_model_set_tensor": (I, [P, I, I, P, P]),
    "atlas_model_get_tensor": (I, [P, I, I, P, P]),
    "atlas_model_init_random": (I, [P, U64]),
    "atlas_model_reset": (I, [P]),
    "atlas_model_pos": (I, [P]),
    "atlas_model_set_kv_rows": (I, [P, I, I, I, I, P, P]),
    "atlas_model_set_pos": (I, [P, I]),
    "atlas_model_attn_scale": (F, [P]),
    "atlas_model_forward_one": (I, [P, U32, P]),
    "atlas_model_forward_one_hooked": (I, [P, U32, P, P, HOOK_FN, P]),
    "atlas_model_generate": (I, [P, P, I, I, C.POINTER(SamplingC), P, C.POINTER(C.c_int)]),
    "atlas_model_generate_hooked": (I, [P, P, I, I, C.POINTER(SamplingC), HOOK_FN, P, P, P, P,
                                        C.POINTER(C.c_int)]),
    "atlas_model_generate_streaming": (I, [P, P, I, I, C.POINTER(SamplingC), TOKEN_FN, P,
                                           C.POINTER(C.c_int)]),
    "atlas_model_generate_batch": (I, [P, P, P, I, I, C.POINTER(SamplingC), P, P]),
    "atlas_model_decode_greedy": (I, [P, U32, I, P]),
    "atlas_model_decode_greedy_timed": (I, [P, U32, I, P, P]),
    "atlas_model_set_long_context": (I, [P, I]),
    "atlas_model_prefill": (I, [P, P, I]),
    "atlas_model_set_prefill_chunk": (I, [P, I]),
    "atlas_model_get_config": (I, [P, C.POINTER(ModelConfigC)]),
    "atlas_model_set_tensor_dev": (I, [P, I, I, P, I, I64, P]),
    "atlas_load_scratch_create": (P, []),
    "atlas_load_scratch_destroy": (None, [P]),
    # include/atlas_loader.h (crates/atlas-model/src/lib.rs:2048-2570)
    "atlas_st_open": (I, [C.c_char_p, P]),
    "atlas_st_from_bytes": (I, [P, SZ, P]),
    "atlas_st_close": (None, [P]),
    "atlas_st_count": (I, [P]),
    "atlas_st_find": (I, [P, C.c_char_p]),
    "atlas_st_desc": (I, [P, I, P, P, P, P, P]),
    "atlas_st_get_f32": (I, [P, C.c_char_p, P, SZ, P]),
    "atlas_st_get_bf16": (I, [P, C.c_char_p, P, SZ, P]),
    "atlas_f16_to_f32": (F, [C.c_uint16]),
    "atlas_config_patch_hf_json": (I, [C.c_char_p, C.POINTER(ModelConfigC), P, I, P, P]),
    "atlas_model_load_safetensors": (I, [C.c_char_p, C.POINTER(ModelConfigC), P]),
    "atlas_model_load_dir": (I, [C.c_char_p, C.POINTER(ModelConfigC), P, P]),
    "atlas_sample_host": (I, [P, I, P, I, I, C.POINTER(SamplingC), C.POINTER(C.c_uint64), P]),
    "atlas_sample_device": (I, [P, I, P, I, I, C.POINTER(SamplingC), C.POINTER(C.c_uint64), P]),
    "atlas_model_bench_gemv": (I, [P, I, I, P, P, P]),
    "atlas_model_use_graph": (I, [P, I]),
    "atlas_model_stream": (P, [P]),
    "atlas_model_logits_dev": (P, [P]),
    "atlas_model_weight_bytes": (I64, [P]),
}

_lib = None
_load_error = None


def load():
    """Load the HIP library (raises AtlasError if it is not built)."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise AtlasError(-4, f"{LIB_PATH} is not built: run `python -m atlas_amd.build` "
                             "(there is no CPU fallback)")
    try:
        lib = C.CDLL(LIB_PATH)
    except OSError as e:            # missing HIP runtime, wrong arch, ...
        _load_error = e
        raise AtlasError(-2, f"cannot load {LIB_PATH}: {e}") from e
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int) -> int:
    """Raise AtlasError for a negative status code.  The library's recorded
    error is cleared once it is raised, so a later `void` call's check_void
    does not report it again."""
    if rc is not None and rc < 0:
        lib = load()
        msg = lib.atlas_last_error()
        text = msg.decode() if msg else ""
        lib.atlas_clear_error()
        raise AtlasError(rc, text)
    return rc


def check_void() -> None:
    """For the reference's void entry points: raise if one recorded an error."""
    lib = load()
    code = lib.atlas_last_error_code()
    if code < 0:
        msg = lib.atlas_last_error().decode()
        lib.atlas_clear_error()
        raise AtlasError(code, msg)


def exported_symbols() -> list[str]:
    return sorted(SIGNATURES)
