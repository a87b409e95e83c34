// Row copies: embedding gather (nv_embedding), last-token gather (nv_gather)
// and the standalone paged KV-cache slot write (nv_kv_write).
//
// Semantics: kernels/kernels.cu:139-144 (embedding) and :366-371 (gather) of
// nano-vllm-rs — out[r,:] = src[index[r],:] when 0 <= index[r] < src_rows,
// else +0 — and the K/V half of kernels/kernels.cu:188-190,206-209 for the KV
// write — rows whose slot lies outside [0, bs*blocks) are skipped.
//
// Fast path (row bytes a multiple of 16, 16-byte aligned): four rows per wave,
// 16-byte chunks strided by 64 lanes, all loads of a lane issued before its
// stores. Indices are read once per row instead of once per element, and there
// is no per-element 64-bit division.
#include "../../include/nano_hip.h"
#include "nvr_device.h"
#include "nvr_internal.h"

namespace {

using nvr::kWave;

constexpr int kUnroll = 4;  // 16-byte chunks in flight per lane

__device__ __forceinline__ void copy_row16(const uint4* __restrict__ src, uint4* __restrict__ dst, int chunks,
                                           int lane) {
    for (int c0 = lane; c0 < chunks; c0 += kWave * kUnroll) {
        uint4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int c = c0 + u * kWave;
            if (c < chunks) v[u] = nvr::load_stream(src + c);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int c = c0 + u * kWave;
            if (c < chunks) nvr::store_stream(dst + c, v[u]);
        }
    }
}

__device__ __forceinline__ void zero_row16(uint4* __restrict__ dst, int chunks, int lane) {
    for (int c = lane; c < chunks; c += kWave) nvr::store_stream(dst + c, make_uint4(0, 0, 0, 0));
}

// out[r] = src[index[r]] (or zeros); rows of `hidden` bf16, `hidden % 8 == 0`.
// Each wave copies kGatherRows rows: their indices arrive with one load, then
// every chunk load of those rows is in flight before the first store. Fewer,
// fatter waves measured faster than more, thinner ones on MI355X (16384 rows
// of 2 KiB: 12.5 us at 8 rows a wave, 12.9 at 4 or 16, 14.1 at 1 or 2; KV
// writes of 4 KiB rows: 22.5 us at 16 rows a wave, 23.4 at 8, 24.5 at 4,
// 26.3 at 1).
constexpr int kGatherRows = 8;
constexpr int kKvRows = 16;
constexpr int kMaxChunksPerLane = 4;  // rows up to 64 * 4 * 8 = 2048 bf16 take the unrolled path

__global__ __launch_bounds__(256) void gather_rows16(const int* __restrict__ index, const uint16_t* __restrict__ src,
                                                     uint16_t* __restrict__ out, int rows, int hidden, int src_rows) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row0 = (int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave) * kGatherRows;
    if (row0 >= rows) return;
    const int chunks = hidden / 8;
    int idx[kGatherRows];
#pragma unroll
    for (int r = 0; r < kGatherRows; ++r) idx[r] = row0 + r < rows ? index[row0 + r] : -1;
    if (chunks <= kWave * kMaxChunksPerLane) {
        uint4 v[kGatherRows][kMaxChunksPerLane];
#pragma unroll
        for (int r = 0; r < kGatherRows; ++r) {
            const bool ok = idx[r] >= 0 && idx[r] < src_rows;
            const uint4* s = reinterpret_cast<const uint4*>(src + int64_t(ok ? idx[r] : 0) * hidden);
#pragma unroll
            for (int u = 0; u < kMaxChunksPerLane; ++u) {
                const int c = lane + u * kWave;
                v[r][u] = make_uint4(0, 0, 0, 0);
                if (ok && c < chunks) v[r][u] = nvr::load_stream(s + c);
            }
        }
#pragma unroll
        for (int r = 0; r < kGatherRows; ++r) {
            if (row0 + r >= rows) break;
            uint4* d = reinterpret_cast<uint4*>(out + (row0 + r) * hidden);
#pragma unroll
            for (int u = 0; u < kMaxChunksPerLane; ++u) {
                const int c = lane + u * kWave;
                if (c < chunks) nvr::store_stream(d + c, v[r][u]);
            }
        }
        return;
    }
    for (int r = 0; r < kGatherRows && row0 + r < rows; ++r) {
        uint4* dst = reinterpret_cast<uint4*>(out + (row0 + r) * hidden);
        if (idx[r] >= 0 && idx[r] < src_rows)
            copy_row16(reinterpret_cast<const uint4*>(src + int64_t(idx[r]) * hidden), dst, chunks, lane);
        else
            zero_row16(dst, chunks, lane);
    }
}

__global__ __launch_bounds__(256) void gather_rows_generic(const int* __restrict__ index,
                                                           const uint16_t* __restrict__ src,
                                                           uint16_t* __restrict__ out, int rows, int hidden,
                                                           int src_rows) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;
    const int i = index[row];
    const bool ok = i >= 0 && i < src_rows;
    for (int j = lane; j < hidden; j += kWave) out[row * hidden + j] = ok ? src[int64_t(i) * hidden + j] : uint16_t(0);
}

// kc[slot[r]] = k[r], vc[slot[r]] = v[r]; each row is `width` = kvh*dim bf16.
// kKvRows rows per wave with their slots loaded together, as for gathers.
__global__ __launch_bounds__(256) void kv_write16(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                  const int* __restrict__ slots, uint16_t* __restrict__ kc,
                                                  uint16_t* __restrict__ vc, int rows, int width, int64_t capacity) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row0 = (int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave) * kKvRows;
    if (row0 >= rows) return;
    const int chunks = width / 8;
    int slot[kKvRows];
#pragma unroll
    for (int r = 0; r < kKvRows; ++r) slot[r] = row0 + r < rows ? slots[row0 + r] : -1;
    constexpr int U = 2;  // chunks per lane per row on the unrolled path (width <= 1024)
    if (chunks <= kWave * U) {
        uint4 a[kKvRows][U], b[kKvRows][U];
#pragma unroll
        for (int r = 0; r < kKvRows; ++r) {
            const bool ok = slot[r] >= 0 && int64_t(slot[r]) < capacity;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = lane + u * kWave;
                if (ok && c < chunks) {
                    a[r][u] = nvr::load_stream(k + (row0 + r) * width + 8 * c);
                    b[r][u] = nvr::load_stream(v + (row0 + r) * width + 8 * c);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < kKvRows; ++r) {
            const bool ok = slot[r] >= 0 && int64_t(slot[r]) < capacity;
            if (!ok) continue;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = lane + u * kWave;
                if (c < chunks) {
                    nvr::store_stream(kc + int64_t(slot[r]) * width + 8 * c, a[r][u]);
                    nvr::store_stream(vc + int64_t(slot[r]) * width + 8 * c, b[r][u]);
                }
            }
        }
        return;
    }
    for (int r = 0; r < kKvRows && row0 + r < rows; ++r) {
        if (slot[r] < 0 || int64_t(slot[r]) >= capacity) continue;
        const uint4* ks = reinterpret_cast<const uint4*>(k + (row0 + r) * width);
        const uint4* vs = reinterpret_cast<const uint4*>(v + (row0 + r) * width);
        copy_row16(ks, reinterpret_cast<uint4*>(kc + int64_t(slot[r]) * width), chunks, lane);
        copy_row16(vs, reinterpret_cast<uint4*>(vc + int64_t(slot[r]) * width), chunks, lane);
    }
}

__global__ __launch_bounds__(256) void kv_write_generic(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                        const int* __restrict__ slots, uint16_t* __restrict__ kc,
                                                        uint16_t* __restrict__ vc, int rows, int width,
                                                        int64_t capacity) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;
    const int slot = slots[row];
    if (slot < 0 || int64_t(slot) >= capacity) return;
    for (int j = lane; j < width; j += kWave) {
        kc[int64_t(slot) * width + j] = k[row * width + j];
        vc[int64_t(slot) * width + j] = v[row * width + j];
    }
}

int launch_gather(nv_context* c, const void* index, const void* src, void* out, int rows, int hidden, int src_rows,
                  const char* name) {
    NVR_ACTIVATE(c);
    if (rows <= 0 || hidden <= 0 || src_rows <= 0) return nvr::fail(-2, "%s: dimensions must be positive", name);
    auto idx = static_cast<const int*>(index);
    auto s = static_cast<const uint16_t*>(src);
    auto o = static_cast<uint16_t*>(out);
    if (hidden % 8 == 0 && nvr::aligned(src, 16) && nvr::aligned(out, 16)) {
        const unsigned blocks = unsigned((int64_t(rows) + 4 * kGatherRows - 1) / (4 * kGatherRows));
        hipLaunchKernelGGL(gather_rows16, dim3(blocks), dim3(256), 0, c->stream, idx, s, o, rows, hidden, src_rows);
    } else {
        const unsigned blocks = unsigned((int64_t(rows) + 3) / 4);
        hipLaunchKernelGGL(gather_rows_generic, dim3(blocks), dim3(256), 0, c->stream, idx, s, o, rows, hidden,
                           src_rows);
    }
    return nvr::launch_status();
}

}  // namespace

extern "C" {

int nv_embedding(nv_context* c, const void* tokens, const void* weight, void* out, int rows, int hidden, int vocab) {
    return launch_gather(c, tokens, weight, out, rows, hidden, vocab, "embedding");
}

int nv_gather(nv_context* c, const void* x, const void* indices, void* out, int rows, int hidden, int input_rows) {
    return launch_gather(c, indices, x, out, rows, hidden, input_rows, "gather");
}

int nv_kv_write(nv_context* c, const void* k, const void* v, const void* slots, void* kc, void* vc, int rows, int kvh,
                int dim, int bs, int blocks) {
    NVR_ACTIVATE(c);
    if (rows <= 0 || kvh <= 0 || dim <= 0 || bs <= 0 || blocks <= 0)
        return nvr::fail(-2, "kv_write: dimensions must be positive");
    const int64_t width = int64_t(kvh) * dim;
    if (width > 0x7fffffff) return nvr::fail(-2, "kv_write: kvh * dim exceeds int32");
    const int64_t capacity = int64_t(bs) * blocks;
    auto k16 = static_cast<const uint16_t*>(k);
    auto v16 = static_cast<const uint16_t*>(v);
    auto sl = static_cast<const int*>(slots);
    auto kc16 = static_cast<uint16_t*>(kc);
    auto vc16 = static_cast<uint16_t*>(vc);
    if (width % 8 == 0 && nvr::aligned(k, 16) && nvr::aligned(v, 16) && nvr::aligned(kc, 16) && nvr::aligned(vc, 16)) {
        const unsigned nblocks = unsigned((int64_t(rows) + 4 * kKvRows - 1) / (4 * kKvRows));
        hipLaunchKernelGGL(kv_write16, dim3(nblocks), dim3(256), 0, c->stream, k16, v16, sl, kc16, vc16, rows,
                           int(width), capacity);
    } else {
        const unsigned nblocks = unsigned((int64_t(rows) + 3) / 4);
        hipLaunchKernelGGL(kv_write_generic, dim3(nblocks), dim3(256), 0, c->stream, k16, v16, sl, kc16, vc16, rows,
                           int(width), capacity);
    }
    return nvr::launch_status();
}

}  // extern "C"
