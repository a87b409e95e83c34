// Context, memory, transfer and graph entry points of the C ABI, plus the
// hipBLAS GEMM. Semantics follow kernels/kernels.cu:8-107 of nano-vllm-rs:
// one context owns a device, a non-blocking stream and a BLAS handle; every
// call re-activates the context's device; errors land in a thread-local
// buffer read by nv_last_error().
#include <stdarg.h>
#include <stdio.h>

#include <new>

#include "../../include/nano_hip.h"
#include "nvr_internal.h"

namespace {
thread_local char g_last_error[1024];
}

namespace nvr {

int hip_status(hipError_t status, const char* operation) {
    if (status == hipSuccess) return 0;
    snprintf(g_last_error, sizeof(g_last_error), "%s: %s (%d)", operation, hipGetErrorString(status),
             int(status));
    return int(status);
}

int blas_status(hipblasStatus_t status, const char* operation) {
    if (status == HIPBLAS_STATUS_SUCCESS) return 0;
    snprintf(g_last_error, sizeof(g_last_error), "%s: hipBLAS status %d", operation, int(status));
    return int(status) + 10000;
}

int fail(int code, const char* fmt, ...) {
    va_list args;
    va_start(args, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
    va_end(args);
    return code;
}

}  // namespace nvr

namespace {
// Allocation, transfer and synchronisation are not capturable; the reference
// relies on its Rust wrapper for this, here the library refuses by itself.
int refuse_if_capturing(nv_context* c, const char* what) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    int error = nvr::hip_status(hipStreamIsCapturing(c->stream, &status), "hipStreamIsCapturing");
    if (error) return error;
    if (status != hipStreamCaptureStatusNone)
        return nvr::fail(-2, "%s is forbidden during graph capture", what);
    return 0;
}
}  // namespace

extern "C" {

const char* nv_last_error(void) { return g_last_error; }

int nv_stream(nv_context* c, void** output) {
    NVR_ACTIVATE(c);
    *output = reinterpret_cast<void*>(c->stream);
    return 0;
}

int nv_sm_count(nv_context* c, int* output) {
    NVR_ACTIVATE(c);
    NVR_HIP(hipDeviceGetAttribute(output, hipDeviceAttributeMultiprocessorCount, c->device));
    return 0;
}

int nv_create(int device, nv_context** output) {
    NVR_HIP(hipSetDevice(device));
    nv_context* c = new (std::nothrow) nv_context{device, nullptr, nullptr, 0, nullptr, nullptr};
    if (!c) return nvr::fail(-1, "host context allocation failed");
    int error = nvr::hip_status(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking),
                                "hipStreamCreateWithFlags");
    if (error) { delete c; return error; }
    error = nvr::hip_status(hipDeviceGetAttribute(&c->cu_count, hipDeviceAttributeMultiprocessorCount, device),
                            "hipDeviceGetAttribute");
    if (error) { (void)hipStreamDestroy(c->stream); delete c; return error; }
    error = nvr::blas_status(hipblasCreate(&c->blas), "hipblasCreate");
    if (error) { (void)hipStreamDestroy(c->stream); delete c; return error; }
    error = nvr::blas_status(hipblasSetStream(c->blas, c->stream), "hipblasSetStream");
    // No atomics: every GEMM gives the same bits on every run, as the
    // reference's cuBLAS GEMMs do (graph replays equal eager launches).
    if (!error) error = nvr::blas_status(hipblasSetAtomicsMode(c->blas, HIPBLAS_ATOMICS_NOT_ALLOWED),
                                         "hipblasSetAtomicsMode");
    if (!error) error = nvr::bind_static_partials(c);
    if (!error) error = nvr::create_pair_state(c);
    if (error) {
        if (c->pair_state) (void)hipFree(c->pair_state);
        hipblasDestroy(c->blas);
        (void)hipStreamDestroy(c->stream);
        delete c;
        return error;
    }
    *output = c;
    return 0;
}

void nv_destroy(nv_context* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    if (c->pair_state) (void)hipFree(c->pair_state);
    hipblasDestroy(c->blas);
    (void)hipStreamDestroy(c->stream);
    delete c;
}

int nv_alloc(nv_context* c, size_t bytes, void** output) {
    NVR_ACTIVATE(c);
    if (int error = refuse_if_capturing(c, "allocation")) return error;
    NVR_HIP(hipMalloc(output, bytes));
    int error = nvr::hip_status(hipMemsetAsync(*output, 0, bytes, c->stream), "hipMemsetAsync");
    if (error) { (void)hipFree(*output); *output = nullptr; }
    return error;
}

void nv_free(nv_context* c, void* buffer) {
    (void)hipSetDevice(c->device);
    (void)hipFree(buffer);
}

int nv_upload(nv_context* c, void* dst, const void* src, size_t bytes) {
    NVR_ACTIVATE(c);
    if (int error = refuse_if_capturing(c, "upload")) return error;
    NVR_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
    return nvr::hip_status(hipStreamSynchronize(c->stream), "host upload synchronize");
}

int nv_download(nv_context* c, const void* src, void* dst, size_t bytes) {
    NVR_ACTIVATE(c);
    if (int error = refuse_if_capturing(c, "download")) return error;
    NVR_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
    return nvr::hip_status(hipStreamSynchronize(c->stream), "host download synchronize");
}

int nv_sync(nv_context* c) {
    NVR_ACTIVATE(c);
    if (int error = refuse_if_capturing(c, "synchronization")) return error;
    return nvr::hip_status(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

int nv_mem_info(nv_context* c, size_t* free_bytes, size_t* total_bytes) {
    NVR_ACTIVATE(c);
    return nvr::hip_status(hipMemGetInfo(free_bytes, total_bytes), "hipMemGetInfo");
}

int nv_capture_begin(nv_context* c) {
    NVR_ACTIVATE(c);
    return nvr::hip_status(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal),
                           "hipStreamBeginCapture");
}

int nv_capture_end(nv_context* c, void** output) {
    NVR_ACTIVATE(c);
    hipGraph_t graph = nullptr;
    int error = nvr::hip_status(hipStreamEndCapture(c->stream, &graph), "hipStreamEndCapture");
    if (error) {
        if (graph) (void)hipGraphDestroy(graph);
        return error;
    }
    hipGraphExec_t exec = nullptr;
    error = nvr::hip_status(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void)hipGraphDestroy(graph);
    if (!error) *output = reinterpret_cast<void*>(exec);
    return error;
}

void nv_capture_abort(nv_context* c) {
    (void)hipSetDevice(c->device);
    hipGraph_t graph = nullptr;
    (void)hipStreamEndCapture(c->stream, &graph);
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipGetLastError();
}

int nv_graph_replay(nv_context* c, void* graph) {
    NVR_ACTIVATE(c);
    return nvr::hip_status(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph), c->stream), "hipGraphLaunch");
}

void nv_graph_destroy(nv_context* c, void* graph) {
    (void)hipSetDevice(c->device);
    (void)hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph));
}

int nv_gemm(nv_context* c, const void* x, const void* w, void* y, int m, int n, int k) {
    NVR_ACTIVATE(c);
    const float alpha = 1.0f, beta = 0.0f;
    // Row-major Y[m,n] = X[m,k] W[n,k]^T is column-major Y'[n,m] = A' B with
    // A = W seen as column-major [k,n] (lda = k, transposed) and B = X seen as
    // column-major [k,m] (ldb = k).
    NVR_BLAS(hipblasGemmEx(c->blas, HIPBLAS_OP_T, HIPBLAS_OP_N, n, m, k, &alpha, w, HIP_R_16BF, k, x,
                           HIP_R_16BF, k, &beta, y, HIP_R_16BF, n, HIPBLAS_COMPUTE_32F, HIPBLAS_GEMM_DEFAULT));
    return 0;
}

uint64_t nv_sampling_seed(uint64_t base, uint64_t request_id, uint64_t generated) {
    auto mix = [](uint64_t v) {
        v += 0x9e3779b97f4a7c15ull;
        v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
        v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
        return v ^ (v >> 31);
    };
    return mix(mix(base) ^ mix(request_id) ^ mix(generated));
}

}  // extern "C"
