// runtime.cpp -- device, stream, memory and error handling behind the C ABI.
//
// Replaces the CUDA runtime calls the reference makes directly from Rust
// (crates/atlas-tensor/src/lib.rs:151-161: cudaMalloc, cudaFree, cudaMemcpy,
// cudaMallocAsync, cudaFreeAsync) and the device queries of
// kernels/matmul.cu:580-595.
#include <cstdarg>
#include <mutex>

#include "common.hpp"
#include "fused.hpp"

namespace atlas {

static thread_local int t_err_code = ATLAS_OK;
static thread_local char t_err_msg[512] = "";

void set_error(int code, const char* fmt, ...) {
    t_err_code = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_err_msg, sizeof(t_err_msg), fmt, ap);
    va_end(ap);
}

void clear_error() {
    t_err_code = ATLAS_OK;
    t_err_msg[0] = 0;
}

// Each host thread launches on its own current stream (the null stream until
// atlas_set_stream), so two threads driving the library never share one.
static thread_local hipStream_t g_stream = nullptr;

hipStream_t stream() { return g_stream; }

namespace {
constexpr int kScratchDevices = 16;
struct ScratchBuf {
    void* p = nullptr;
    size_t cap = 0;
    hipStream_t last = nullptr;   // stream of the most recent use
};
struct ThreadScratch {
    ScratchBuf b[kScratchDevices][SCR_N];
};
thread_local ThreadScratch t_scratch;
}  // namespace

int thread_scratch(int slot, size_t bytes, void** out, bool zero_new) {
    ATLAS_REQUIRE(out && slot >= 0 && slot < SCR_N, "scratch: bad slot %d", slot);
    *out = nullptr;
    int dev = 0;
    ATLAS_HIP(hipGetDevice(&dev));
    ATLAS_REQUIRE(dev >= 0 && dev < kScratchDevices, "scratch: device %d", dev);
    ScratchBuf& s = t_scratch.b[dev][slot];
    hipStream_t st = g_stream;
    if (bytes > s.cap) {
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
        if (hipMallocAsync(&p, cap, st) != hipSuccess || !p) {
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

ATLAS_API int atlas_last_error_code(void) { return t_err_code; }
ATLAS_API const char* atlas_last_error(void) { return t_err_msg; }
ATLAS_API void atlas_clear_error(void) { clear_error(); }

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
    g_stream = reinterpret_cast<hipStream_t>(s);
    return ATLAS_OK;
}

ATLAS_API void* atlas_get_stream(void) { return reinterpret_cast<void*>(g_stream); }

ATLAS_API int atlas_stream_sync(void) {
    ATLAS_HIP(hipStreamSynchronize(g_stream));
    return ATLAS_OK;
}

ATLAS_API int atlas_device_cu_count(void) { return device_cu_count(); }

ATLAS_API int atlas_dev_malloc(void** ptr, size_t bytes) {
    ATLAS_REQUIRE(ptr, "atlas_dev_malloc: null out pointer");
    *ptr = nullptr;
    if (bytes == 0) return ATLAS_OK;
    if (hipMallocAsync(ptr, bytes, g_stream) == hipSuccess && *ptr) return ATLAS_OK;
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
    if (hipFreeAsync(ptr, g_stream) == hipSuccess) return ATLAS_OK;
    (void)hipGetLastError();
    ATLAS_HIP(hipFree(ptr));
    return ATLAS_OK;
}

ATLAS_API int atlas_dev_malloc_sync(void** ptr, size_t bytes) {
    ATLAS_REQUIRE(ptr, "atlas_dev_malloc_sync: null out pointer");
    *ptr = nullptr;
    if (bytes == 0) return ATLAS_OK;
    if (hipMalloc(ptr, bytes) != hipSuccess || !*ptr) {
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
    ATLAS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
    ATLAS_HIP(hipStreamSynchronize(g_stream));
    return ATLAS_OK;
}

ATLAS_API int atlas_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return ATLAS_OK;
    ATLAS_REQUIRE(dst && src, "memcpy_d2h: null pointer");
    ATLAS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
    ATLAS_HIP(hipStreamSynchronize(g_stream));
    return ATLAS_OK;
}

ATLAS_API int atlas_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return ATLAS_OK;
    ATLAS_REQUIRE(dst && src, "memcpy_d2d: null pointer");
    ATLAS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
    return ATLAS_OK;
}

ATLAS_API int atlas_memset_zero(void* dst, size_t bytes) {
    if (bytes == 0) return ATLAS_OK;
    ATLAS_REQUIRE(dst && bytes % 4 == 0, "memset_zero: needs a 4-byte multiple");
    return ew_launch(EW_FILL, nullptr, nullptr, reinterpret_cast<float*>(dst), 0.0f,
                     (long)(bytes / 4), g_stream);
}
