// common.hpp -- shared helpers for the gfx950 decode kernels.
//
// Error model (errors.hpp): every C-ABI entry point returns 0 on success or a
// negative ATLAS_E* code and records a message retrievable with
// atlas_last_error() (thread-local).  Launches go to the library-wide stream
// (atlas_set_stream; default: the null stream, as the reference uses) unless
// the calling thread set its own (atlas_set_thread_stream).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>

#include "errors.hpp"

namespace atlas {

hipStream_t stream();          // the calling thread's override, else the library-wide stream
int device_cu_count();         // CUs of the current device (cached)

// Device scratch owned by the calling thread on the current device, for entry
// points that are not handed a workspace (split partials of the reference-ABI
// attention, split-K partials of the skinny GEMMs, argmax partials).  Each
// slot grows stream-ordered on the thread's current stream (the old buffer is
// freed after the work already queued there; a thread that switched streams
// waits for the previous one first) and is kept until the thread exits.  Two
// threads never share a slot; calls of one thread on two streams at once do.
// zero_new: a grown slot is cleared (fill kernel) before it is returned.
enum ScratchSlot {
    SCR_ATTN = 0,       // atlas_decode_attention split partials
    SCR_GEMM,           // skinny / prompt-GEMM split-K partials
    SCR_ARGMAX,         // argmax per-block keys
    SCR_FUSED_PART,     // atlas_attention_fused_f32 split partials
    SCR_FUSED_CNT,      // ... its merge counters (kept at zero by the kernel)
    SCR_FUSED_POS,      // ... its position word
    SCR_ATTN_CNT,       // atlas_decode_attention merge counters (kept at zero)
    SCR_N
};
// A slot that must grow while its stream is being captured is refused with
// ATLAS_EUNSUPPORTED (no allocation is recorded into the caller's graph).  A
// thread's slots are freed when the thread exits.
int thread_scratch(int slot, size_t bytes, void** out, bool zero_new = false);
size_t thread_scratch_bytes();   // bytes the calling thread holds on the current device

// Check a HIP call; on failure record the error and return ATLAS_EHIP.
#define ATLAS_HIP(call)                                                        \
    do {                                                                       \
        hipError_t e_ = (call);                                                \
        if (e_ != hipSuccess) {                                                \
            ::atlas::set_error(ATLAS_EHIP, "%s: %s (%s:%d)", #call,            \
                               hipGetErrorString(e_), __FILE__, __LINE__);     \
            return ATLAS_EHIP;                                                 \
        }                                                                      \
    } while (0)

// Check a kernel launch.
#define ATLAS_LAUNCH_CHECK(name)                                               \
    do {                                                                       \
        hipError_t e_ = hipGetLastError();                                     \
        if (e_ != hipSuccess) {                                                \
            ::atlas::set_error(ATLAS_EHIP, "launch %s: %s", name,              \
                               hipGetErrorString(e_));                         \
            return ATLAS_EHIP;                                                 \
        }                                                                      \
    } while (0)

// Every device and pinned-host allocation of the library goes through these:
// they fail with hipErrorOutOfMemory while the allocation-failure switch says
// so (atlas_debug_fail_allocations), and otherwise call HIP.
template <typename T>
inline hipError_t dev_malloc(T** p, size_t bytes) {
    if (alloc_should_fail()) { *p = nullptr; return hipErrorOutOfMemory; }
    return hipMalloc(reinterpret_cast<void**>(p), bytes);
}
template <typename T>
inline hipError_t dev_malloc_async(T** p, size_t bytes, hipStream_t st) {
    if (alloc_should_fail()) { *p = nullptr; return hipErrorOutOfMemory; }
    return hipMallocAsync(reinterpret_cast<void**>(p), bytes, st);
}
template <typename T>
inline hipError_t host_malloc_pinned(T** p, size_t bytes, unsigned flags = hipHostMallocDefault) {
    if (alloc_should_fail()) { *p = nullptr; return hipErrorOutOfMemory; }
    return hipHostMalloc(reinterpret_cast<void**>(p), bytes, flags);
}

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

// bf16 bits -> f32 is a 16-bit left shift (kernels/matmul.cu:321-323).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Sign-extended byte i of w as f32 (one v_cvt_f32_i32 with SDWA byte select).
__device__ __forceinline__ float s8_at(uint32_t w, int i) {
    return (float)(int8_t)(w >> (8 * i));
}

// Wave64 all-lanes sum through DPP: quad swaps, half-row and row mirrors,
// then row broadcasts 15 and 31 fold the four rows into lane 63, which is
// read back into every lane.
__device__ __forceinline__ float wave_sum(float v) {
    int x = __float_as_int(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));  // quad [1,0,3,2]
    x = __float_as_int(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));  // quad [2,3,0,1]
    x = __float_as_int(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false)); // row_half_mirror
    x = __float_as_int(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false)); // row_mirror
    x = __float_as_int(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false)); // row_bcast15
    x = __float_as_int(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false)); // row_bcast31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum over the 16 lanes of each DPP row; every lane of the row gets it.
__device__ __forceinline__ float row16_sum(float v) {
    int x = __float_as_int(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));
    x = __float_as_int(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));
    x = __float_as_int(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false));
    x = __float_as_int(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false));
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Nontemporal 128-bit load: weights are streamed once per token, so keep
// them from displacing the activations and KV tiles that are re-read.
__device__ __forceinline__ u32x4 ldg_stream(const u32x4* p) {
    return __builtin_nontemporal_load(p);
}

// A block-uniform pointer made visible as uniform (readfirstlane of both
// halves).  Buffer descriptors built from it live in SGPRs; built from a
// VGPR pointer, every buffer load would be wrapped in a waterfall loop.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(const T* p) {
    const uint64_t u = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
    return (T*)(((uint64_t)hi << 32) | lo);
}

}  // namespace atlas
