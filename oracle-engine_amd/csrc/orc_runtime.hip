// C-ABI runtime plumbing: device selection, error reporting, memory, streams,
// graph capture and events. The reference is CPU-only; the closest
// counterparts are its RAM preload of the GGUF data section
// (core/gguf_parser.cpp:112-138) and the anonymous allocations of
// core/platform.cpp:337-341, which orc_upload / orc_malloc replace.
#include "orc_internal.hpp"

#include <cstdio>
#include <cstring>
#include <mutex>

namespace orc {

static thread_local std::string g_err;
static hipStream_t g_stream = nullptr;
static int g_device = -1;
static std::mutex g_mu;

int set_error(int code, const std::string& msg) {
    g_err = msg;
    return code;
}
hipStream_t resolve_stream(orc_stream_t s) { return s ? (hipStream_t)s : g_stream; }
bool initialized() { return g_device >= 0; }

__global__ void k_fill(uint8_t* p, uint8_t v, size_t n) {
    size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16;
    const size_t stride = (size_t)gridDim.x * blockDim.x * 16;
    uint32_t w = v * 0x01010101u;
    for (; i < n; i += stride) {
        if (i + 16 <= n && (((uintptr_t)(p + i)) & 15) == 0) *(u32x4*)(p + i) = u32x4{w, w, w, w};
        else
            for (size_t k = i; k < n && k < i + 16; ++k) p[k] = v;
    }
}

}  // namespace orc

using namespace orc;

extern "C" const char* orc_last_error(void) { return g_err.c_str(); }

extern "C" int orc_init(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_device == device) return ORC_OK;
    int n = 0;
    ORC_HIP_CHECK(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return set_error(ORC_E_INVALID, "orc_init: no such device");
    ORC_HIP_CHECK(hipSetDevice(device));
    if (g_stream) (void)hipStreamDestroy(g_stream);
    ORC_HIP_CHECK(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    if (int rc = gemm_device_init(device)) return rc;
    if (int rc = argmax_noalloc_device_init(device)) return rc;
    g_device = device;
    return ORC_OK;
}

extern "C" int orc_shutdown(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_stream) {
        (void)hipStreamSynchronize(g_stream);
        (void)hipStreamDestroy(g_stream);
    }
    g_stream = nullptr;
    gemm_device_release();
    g_device = -1;
    return ORC_OK;
}

extern "C" int orc_device_info(char* name, int cap, int* n_cu, size_t* hbm) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    hipDeviceProp_t pr;
    ORC_HIP_CHECK(hipGetDeviceProperties(&pr, g_device));
    if (name && cap > 0) std::snprintf(name, (size_t)cap, "%s (%s)", pr.name, pr.gcnArchName);
    if (n_cu) *n_cu = pr.multiProcessorCount;
    if (hbm) *hbm = pr.totalGlobalMem;
    return ORC_OK;
}

extern "C" int orc_malloc(void** d_ptr, size_t bytes) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_ptr) return set_error(ORC_E_INVALID, "orc_malloc: null out pointer");
    *d_ptr = nullptr;
    ORC_HIP_CHECK(hipMalloc(d_ptr, bytes ? bytes : 1));
    return ORC_OK;
}

extern "C" int orc_free(void* d_ptr) {
    if (!d_ptr) return ORC_OK;
    ORC_HIP_CHECK(hipFree(d_ptr));
    return ORC_OK;
}

extern "C" int orc_memcpy_h2d(void* dst, const void* src, size_t bytes, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!bytes) return ORC_OK;
    ORC_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, resolve_stream(s)));
    ORC_HIP_CHECK(hipStreamSynchronize(resolve_stream(s)));
    return ORC_OK;
}

extern "C" int orc_memcpy_d2h(void* dst, const void* src, size_t bytes, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!bytes) return ORC_OK;
    ORC_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, resolve_stream(s)));
    ORC_HIP_CHECK(hipStreamSynchronize(resolve_stream(s)));
    return ORC_OK;
}

extern "C" int orc_memcpy_d2d(void* dst, const void* src, size_t bytes, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!bytes) return ORC_OK;
    ORC_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, resolve_stream(s)));
    return ORC_OK;
}

extern "C" int orc_fill(void* dst, int v, size_t bytes, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!bytes) return ORC_OK;
    size_t chunks = (bytes + 15) / 16;
    unsigned grid = (unsigned)std::min<size_t>((chunks + 255) / 256, 4096);
    hipLaunchKernelGGL(k_fill, dim3(grid), dim3(256), 0, resolve_stream(s), (uint8_t*)dst, (uint8_t)v, bytes);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_upload(const void* h_src, size_t bytes, void** d_ptr) {
    if (int rc = orc_malloc(d_ptr, bytes)) return rc;
    // large copies in 256 MiB pieces through the default stream
    const size_t piece = 256ull << 20;
    for (size_t off = 0; off < bytes; off += piece) {
        size_t n = std::min(piece, bytes - off);
        ORC_HIP_CHECK(hipMemcpyAsync((uint8_t*)*d_ptr + off, (const uint8_t*)h_src + off, n, hipMemcpyHostToDevice,
                                     g_stream));
    }
    ORC_HIP_CHECK(hipStreamSynchronize(g_stream));
    return ORC_OK;
}

extern "C" int orc_stream_create(orc_stream_t* s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    hipStream_t st;
    ORC_HIP_CHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    *s = (orc_stream_t)st;
    return ORC_OK;
}
extern "C" int orc_stream_destroy(orc_stream_t s) {
    if (s) ORC_HIP_CHECK(hipStreamDestroy((hipStream_t)s));
    return ORC_OK;
}
extern "C" int orc_stream_sync(orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    ORC_HIP_CHECK(hipStreamSynchronize(resolve_stream(s)));
    return ORC_OK;
}
extern "C" int orc_device_sync(void) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    ORC_HIP_CHECK(hipDeviceSynchronize());
    return ORC_OK;
}

extern "C" int orc_graph_begin(orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    ORC_HIP_CHECK(hipStreamBeginCapture(resolve_stream(s), hipStreamCaptureModeThreadLocal));
    return ORC_OK;
}
extern "C" int orc_graph_end(orc_stream_t s, orc_graph_t* out) {
    hipGraph_t g = nullptr;
    ORC_HIP_CHECK(hipStreamEndCapture(resolve_stream(s), &g));
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return set_error(ORC_E_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    *out = (orc_graph_t)ex;
    return ORC_OK;
}
extern "C" int orc_graph_launch(orc_graph_t g, orc_stream_t s) {
    ORC_HIP_CHECK(hipGraphLaunch((hipGraphExec_t)g, resolve_stream(s)));
    return ORC_OK;
}
extern "C" int orc_graph_destroy(orc_graph_t g) {
    if (g) ORC_HIP_CHECK(hipGraphExecDestroy((hipGraphExec_t)g));
    return ORC_OK;
}

extern "C" int orc_event_create(orc_event_t* ev) {
    hipEvent_t e;
    ORC_HIP_CHECK(hipEventCreate(&e));
    *ev = (orc_event_t)e;
    return ORC_OK;
}
extern "C" int orc_event_destroy(orc_event_t ev) {
    if (ev) ORC_HIP_CHECK(hipEventDestroy((hipEvent_t)ev));
    return ORC_OK;
}
extern "C" int orc_event_record(orc_event_t ev, orc_stream_t s) {
    ORC_HIP_CHECK(hipEventRecord((hipEvent_t)ev, resolve_stream(s)));
    return ORC_OK;
}
extern "C" int orc_event_elapsed_ms(orc_event_t a, orc_event_t b, float* ms) {
    ORC_HIP_CHECK(hipEventSynchronize((hipEvent_t)b));
    ORC_HIP_CHECK(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return ORC_OK;
}
