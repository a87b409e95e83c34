// SiLU-gate-mul (nv_silu).
//
// Semantics: kernels/kernels.cu:356-365 of nano-vllm-rs. packed is
// [rows, 2, intermediate] (gate half, then up half, per token):
//   out[r,i] = bf16( (g / (1 + exp(-g))) * u ),  g = gate[r,i], u = up[r,i]
// with a single rounding at the store.
//
// Numerics: exp uses the hardware base-2 exponential (v_exp_f32 on -g*log2 e)
// and the division uses v_rcp_f32, which keeps the fp32 result within a few
// ulp of the correctly rounded expression and so the bf16 output within one
// bf16 ulp. When 1 + exp(-g) >= 2^126 the quotient is subnormal, where the
// reciprocal would flush; those lanes take the IEEE division instead.
//
// Layout: one thread per 16-byte chunk (8 elements) over all rows, 256-thread
// blocks on a flat grid: a block may straddle rows, so no lane idles when a
// row's chunk count is not a multiple of 256 (3072/8 = 384 at Qwen3-0.6B,
// where per-row blocks left a quarter of the lanes idle; 10% faster). The
// row index is one 32-bit division per thread.
#include "../../include/nano_hip.h"
#include "nvr_device.h"
#include "nvr_internal.h"

namespace {

using nvr::silu_mul;

// Eight elements on the reciprocal path, with one branch for the whole chunk
// into the exact division (only taken when some gate is below about -87).
__device__ __forceinline__ void silu_mul8(const float* g, const float* u, float* o) {
    float d[8];
    bool slow = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        d[i] = 1.0f + __builtin_amdgcn_exp2f(-g[i] * 1.44269504088896340736f);
        slow |= !(d[i] < 0x1.0p126f);
    }
    if (__builtin_expect(slow, 0)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = silu_mul(g[i], u[i]);
        return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (g[i] * __builtin_amdgcn_rcpf(d[i])) * u[i];
}

__global__ __launch_bounds__(256) void silu16(const uint16_t* __restrict__ packed, uint16_t* __restrict__ out,
                                              int intermediate, int64_t total_chunks) {
    const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (c >= total_chunks) return;
    const uint32_t chunks = uint32_t(intermediate) / 8u;
    const uint32_t row32 = uint32_t(c) / chunks;  // the host keeps total_chunks below 2^32
    const int chunk = int(uint32_t(c) - row32 * chunks);
    const int64_t row = row32;
    const int64_t gate_base = row * 2 * intermediate + 8 * chunk;
    const uint4 gw = nvr::load_stream(packed + gate_base);
    const uint4 uw = nvr::load_stream(packed + gate_base + intermediate);
    float g[8], u[8], o[8];
    nvr::unpack8(gw, g);
    nvr::unpack8(uw, u);
    silu_mul8(g, u, o);
    nvr::store_stream(out + 8 * c, nvr::pack8_split(o));
}

__global__ __launch_bounds__(256) void silu_generic(const uint16_t* __restrict__ packed, uint16_t* __restrict__ out,
                                                    int rows, int intermediate) {
    const int64_t total = int64_t(rows) * intermediate;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
        const int64_t r = i / intermediate, col = i - r * intermediate;
        const int64_t base = r * 2 * intermediate + col;
        out[i] = nvr::f32_to_bf16(silu_mul(nvr::bf16_to_f32(packed[base]), nvr::bf16_to_f32(packed[base + intermediate])));
    }
}

}  // namespace

extern "C" int nv_silu(nv_context* c, const void* packed, void* out, int rows, int intermediate) {
    NVR_ACTIVATE(c);
    if (rows <= 0 || intermediate <= 0) return nvr::fail(-2, "silu: dimensions must be positive");
    auto in16 = static_cast<const uint16_t*>(packed);
    auto out16 = static_cast<uint16_t*>(out);
    const int64_t total_chunks = int64_t(rows) * (intermediate / 8);
    const int64_t grid = (total_chunks + 255) / 256;
    if (intermediate % 8 == 0 && nvr::aligned(packed, 16) && nvr::aligned(out, 16) && total_chunks <= 0xffffffffLL) {
        hipLaunchKernelGGL(silu16, dim3(unsigned(grid)), dim3(256), 0, c->stream, in16, out16, intermediate,
                           total_chunks);
    } else {
        const int64_t want = (int64_t(rows) * intermediate + 255) / 256;
        const unsigned g = unsigned(want > 65535 ? 65535 : want);
        hipLaunchKernelGGL(silu_generic, dim3(g), dim3(256), 0, c->stream, in16, out16, rows, intermediate);
    }
    return nvr::launch_status();
}
