// runtime.cpp -- device, stream, memory and error handling behind the C ABI.
//
// Replaces the CUDA runtime calls the reference makes directly from Rust
// (crates/atlas-tensor/src/lib.rs:151-161: cudaMalloc, cudaFree, cudaMemcpy,
// cudaMallocAsync, cudaFreeAsync) and the device queries of
// kernels/matmul.cu:580-595.
#include <atomic>
#include <mutex>

#include "common.hpp"
#include "fused.hpp"

namespace atlas {

// The launch stream: one library-wide stream (atlas_set_stream; the null
// stream until set, as in the reference), which a thread may override for
// its own calls (atlas_set_thread_stream).  Every call of a thread without
// an override goes to the library-wide stream, whichever thread set it.
static std::atomic<hipStream_t> g_stream{nullptr};
static thread_local bool t_has_stream = false;
static thread_local hipStream_t t_stream = nullptr;

hipStream_t stream() { return t_has_stream ? t_stream : g_stream.load(std::memory_order_acquire); }

namespace {
constexpr int kScratchDevices = 16;
struct ScratchBuf {
    void* p = nullptr;
    size_t cap = 0;
    hipStream_t last = nullptr;   // stream of the most recent use
};
struct ThreadScratch {
    ScratchBuf b[kScratchDevices][SCR_N];
    // a thread's slots go with it: each buffer is freed once the work queued
    // on the stream of its last use is done (hipFree waits for the device)
    ~ThreadScratch() {
        bool any = false;
        for (int d = 0; d < kScratchDevices; ++d)
            for (int i = 0; i < SCR_N; ++i) any = any || b[d][i].p;
        if (!any) return;
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess) return;
        for (int d = 0; d < kScratchDevices; ++d)
            for (int i = 0; i < SCR_N; ++i)
                if (b[d][i].p && hipSetDevice(d) == hipSuccess) {
                    (void)hipFree(b[d][i].p);
                    b[d][i].p = nullptr;
                }
        (void)hipSetDevice(cur);
        (void)hipGetLastError();
    }
};
thread_local ThreadScratch t_scratch;
}  // namespace

size_t thread_scratch_bytes() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) return 0;
    size_t n = 0;
    for (int i = 0; i < SCR_N; ++i) n += t_scratch.b[dev][i].cap;
    return n;
}

int thread_scratch(int slot, size_t bytes, void** out, bool zero_new) {
    ATLAS_REQUIRE(out && slot >= 0 && slot < SCR_N, "scratch: bad slot %d", slot);
    *out = nullptr;
    int dev = 0;
    ATLAS_HIP(hipGetDevice(&dev));
    ATLAS_REQUIRE(dev >= 0 && dev < kScratchDevices, "scratch: device %d", dev);
    ScratchBuf& s = t_scratch.b[dev][slot];
    hipStream_t st = stream();
    if (bytes > s.cap) {
        // Growing under a stream capture would record an allocation node
        // whose address is not backed until the graph runs (and the
        // synchronisation below would break the capture): refuse instead.
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        ATLAS_HIP(hipStreamIsCapturing(st, &cs));
        if (cs != hipStreamCaptureStatusNone) {
            set_error(ATLAS_EUNSUPPORTED,
                      "scratch: this call needs %zu bytes of library scratch on this thread and "
                      "the stream is being captured; make one call of the same shape on this "
                      "thread before the capture, or use a *_noalloc entry point", bytes);
            return ATLAS_EUNSUPPORTED;
        }
        if (s.p) {
            // the old buffer may still be read by work queued on the stream
            // of its last use: free it after that work
            if (s.last != st) ATLAS_HIP(hipStreamSynchronize(s.last));
            ATLAS_HIP(hipFreeAsync(s.p, st));
            s.p = nullptr;
            s.cap = 0;
        }
        const size_t cap = (bytes + 65535) / 65536 * 65536;
        void* p = nullptr;
        if (dev_malloc_async(&p, cap, st) != hipSuccess || !p) {
            (void)hipGetLastError();
            set_error(ATLAS_ENOMEM, "scratch: device allocation of %zu bytes failed", cap);
            return ATLAS_ENOMEM;
        }
        if (zero_new) {
            const int rc = ew_launch(EW_FILL, nullptr, nullptr, reinterpret_cast<float*>(p), 0.0f,
                                     (long)(cap / 4), st);
            if (rc) {
                (void)hipFreeAsync(p, st);
                return rc;
            }
        }
        s.p = p;
        s.cap = cap;
    }
    s.last = st;
    *out = s.p;
    return ATLAS_OK;
}

int device_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

}  // namespace atlas

using namespace atlas;

ATLAS_API int atlas_cuda_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

ATLAS_API int atlas_cuda_available(void) { return atlas_cuda_device_count() > 0 ? 1 : 0; }

ATLAS_API void atlas_sync(void) {
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) set_error(ATLAS_EHIP, "hipDeviceSynchronize: %s", hipGetErrorString(e));
}

ATLAS_API int atlas_set_device(int device) {
    ATLAS_HIP(hipSetDevice(device));
    return ATLAS_OK;
}

ATLAS_API int atlas_set_stream(void* s) {
    g_stream.store(reinterpret_cast<hipStream_t>(s), std::memory_order_release);
    return ATLAS_OK;
}

ATLAS_API int atlas_set_thread_stream(void* s) {
    t_stream = reinterpret_cast<hipStream_t>(s);
    t_has_stream = true;
    return ATLAS_OK;
}

ATLAS_API int atlas_clear_thread_stream(void) {
    t_has_stream = false;
    t_stream = nullptr;
    return ATLAS_OK;
}

ATLAS_API void* atlas_get_stream(void) { return reinterpret_cast<void*>(stream()); }

ATLAS_API int atlas_stream_sync(void) {
    ATLAS_HIP(hipStreamSynchronize(stream()));
    return ATLAS_OK;
}

ATLAS_API int64_t atlas_thread_scratch_bytes(void) { return (int64_t)thread_scratch_bytes(); }

ATLAS_API int atlas_device_cu_count(void) { return device_cu_count(); }

ATLAS_API int atlas_dev_malloc(void** ptr, size_t bytes) {
    ATLAS_REQUIRE(ptr, "atlas_dev_malloc: null out pointer");
    *ptr = nullptr;
    if (bytes == 0) return ATLAS_OK;
    // one allocation: the switch is asked once, then stream-ordered with a
    // plain hipMalloc as the fallback
    if (alloc_should_fail()) {
        set_error(ATLAS_ENOMEM, "device allocation of %zu bytes failed (injected)", bytes);
        return ATLAS_ENOMEM;
    }
    if (hipMallocAsync(ptr, bytes, stream()) == hipSuccess && *ptr) return ATLAS_OK;
    (void)hipGetLastError();
    if (hipMalloc(ptr, bytes) != hipSuccess || !*ptr) {
        (void)hipGetLastError();
        *ptr = nullptr;
        set_error(ATLAS_ENOMEM, "device allocation of %zu bytes failed", bytes);
        return ATLAS_ENOMEM;
    }
    return ATLAS_OK;
}

ATLAS_API int atlas_dev_free(void* ptr) {
    if (!ptr) return ATLAS_OK;
    if (hipFreeAsync(ptr, stream()) == hipSuccess) return ATLAS_OK;
    (void)hipGetLastError();
    ATLAS_HIP(hipFree(ptr));
    return ATLAS_OK;
}

ATLAS_API int atlas_dev_malloc_sync(void** ptr, size_t bytes) {
    ATLAS_REQUIRE(ptr, "atlas_dev_malloc_sync: null out pointer");
    *ptr = nullptr;
    if (bytes == 0) return ATLAS_OK;
    if (dev_malloc(ptr, bytes) != hipSuccess || !*ptr) {
        (void)hipGetLastError();
        *ptr = nullptr;
        set_error(ATLAS_ENOMEM, "device allocation of %zu bytes failed", bytes);
        return ATLAS_ENOMEM;
    }
    return ATLAS_OK;
}

ATLAS_API int atlas_dev_free_sync(void* ptr) {
    if (!ptr) return ATLAS_OK;
    ATLAS_HIP(hipFree(ptr));
    return ATLAS_OK;
}

ATLAS_API int atlas_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return ATLAS_OK;
    ATLAS_REQUIRE(dst && src, "memcpy_h2d: null pointer");
    ATLAS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream()));
    ATLAS_HIP(hipStreamSynchronize(stream()));
    return ATLAS_OK;
}

ATLAS_API int atlas_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return ATLAS_OK;
    ATLAS_REQUIRE(dst && src, "memcpy_d2h: null pointer");
    ATLAS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream()));
    ATLAS_HIP(hipStreamSynchronize(stream()));
    return ATLAS_OK;
}

ATLAS_API int atlas_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return ATLAS_OK;
    ATLAS_REQUIRE(dst && src, "memcpy_d2d: null pointer");
    ATLAS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream()));
    return ATLAS_OK;
}

ATLAS_API int atlas_memset_zero(void* dst, size_t bytes) {
    if (bytes == 0) return ATLAS_OK;
    ATLAS_REQUIRE(dst && bytes % 4 == 0, "memset_zero: needs a 4-byte multiple");
    return ew_launch(EW_FILL, nullptr, nullptr, reinterpret_cast<float*>(dst), 0.0f,
                     (long)(bytes / 4), stream());
}
