// Host-side internals of the nano-vllm-rs HIP library: the context object,
// status plumbing and launch checks shared by every translation unit.
#pragma once

#include <hip/hip_runtime.h>
#include <hipblas/hipblas.h>
#include <stdint.h>

struct nv_context {
    int device;
    hipStream_t stream;
    hipblasHandle_t blas;
    int cu_count;
    // Device address of this device's copy of the sampler's static partials
    // (sample.hip), for nv_sample_parallel_static.
    void* static_partials;
    // The paired sampler's per-row exchange words (sample.hip): two uint64
    // per row, zero between launches (every launch leaves them zero).
    void* pair_state;
};

namespace nvr {

// Records "<operation>: <message> (<code>)" in the calling thread's error
// buffer and returns the status unchanged (0 leaves the buffer untouched).
int hip_status(hipError_t status, const char* operation);
int blas_status(hipblasStatus_t status, const char* operation);
int fail(int code, const char* fmt, ...);

// Looks up this device's copy of the sampler's static partials (called by
// nv_create with the context's device current).
int bind_static_partials(nv_context* c);

// Allocates and zeroes the paired sampler's exchange words (nv_create);
// released by nv_destroy.
int create_pair_state(nv_context* c);

// Status of the most recent launch on this thread.
inline int launch_status() { return hip_status(hipGetLastError(), "HIP kernel launch"); }

inline bool aligned(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0; }

}  // namespace nvr

#define NVR_HIP(call)                                                  \
    do {                                                               \
        int nvr_error_ = ::nvr::hip_status((call), #call);             \
        if (nvr_error_) return nvr_error_;                             \
    } while (0)
#define NVR_BLAS(call)                                                 \
    do {                                                               \
        int nvr_error_ = ::nvr::blas_status((call), #call);            \
        if (nvr_error_) return nvr_error_;                             \
    } while (0)
#define NVR_ACTIVATE(c) NVR_HIP(hipSetDevice((c)->device))
