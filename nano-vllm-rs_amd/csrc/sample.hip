// Greedy / Gumbel-max sampling (nv_sample, nv_sample_parallel).
//
// Semantics: kernels/kernels.cu:372-466,488-501 of nano-vllm-rs. For row r with
// temperature T = temps[r] and seed = seeds[r], every token t scores
//   T > 0:  f32(logit) / T - ln(-ln(u)),  u = ((splitmix64(seed ^ t*K) >> 41) + 0.5) * 2^-23
//   else:   f32(logit)
// and the row's output is the argmax under the total order "higher score,
// then lower index"; NaN never wins; a row where nothing wins yields 0.
// Because that order is total, any partitioning of the vocabulary returns the
// same token as the serial scan (kernels/kernels.cu:409-411).
//
// ln is nvr_logf, a fixed-bits logarithm shared with the host oracle, so CPU
// and GPU agree on every Gumbel index.
//
// Layout: stage 1 gives each (row, partition) one 256-thread block; every lane
// loads kChunksPerLane 16-byte chunks (8 logits each) up front, keeps its own
// best (score, index), the wave folds with butterfly shuffles and the four
// waves through LDS. Stage 2 folds a row's partials in one wave. Partitions
// are a multiple of the reference's 2048 tokens, so the caller's scratch
// (batch x ceil(vocab/2048) entries) always suffices.
#include "../../include/nano_hip.h"
#include "nvr_device.h"
#include "nvr_internal.h"

namespace {

using nvr::kWave;
constexpr int kRefPartition = 2048;
// 16-byte chunks of logits per lane in a partition (partition width
// 2048 * kChunksPerLane tokens). Measured on MI355X at 256 x 151936: 2 is the
// best for Gumbel and mixed batches (4 favours all-greedy batches by ~7%).
constexpr int kChunksPerLane = 2;

struct Best {
    float score;
    int index;
};

__device__ __forceinline__ void consider(Best& b, float s, int i) {
    if (nvr::better(s, i, b.score, b.index)) { b.score = s; b.index = i; }
}

__device__ __forceinline__ Best wave_argmax(Best b) {
#pragma unroll
    for (int mask = kWave / 2; mask > 0; mask >>= 1) {
        const float s = nvr::xor_lane(b.score, mask);
        const int i = nvr::xor_lane(b.index, mask);
        consider(b, s, i);
    }
    return b;
}

// Fold a 256-thread block; the result is valid in thread 0.
__device__ __forceinline__ Best block_argmax(Best b) {
    __shared__ float scores[4];
    __shared__ int indices[4];
    b = wave_argmax(b);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) { scores[wave] = b.score; indices[wave] = b.index; }
    __syncthreads();
    if (threadIdx.x == 0) {
        b = Best{scores[0], indices[0]};
        for (int w = 1; w < int(blockDim.x / kWave); ++w) consider(b, scores[w], indices[w]);
    }
    return b;
}

template <bool GUMBEL>
__device__ __forceinline__ void scan_chunk(Best& b, const uint4& w, int token0, float temperature, uint64_t seed) {
    float f[8];
    nvr::unpack8(w, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float s = GUMBEL ? nvr::gumbel_score(f[i], temperature, seed, uint32_t(token0 + i)) : f[i];
        consider(b, s, token0 + i);
    }
}

// Scans tokens [begin, end) of one row with 256 threads (serial and generic
// paths); begin and end are multiples of 8 when VEC.
template <bool VEC>
__device__ __forceinline__ Best scan_range(const uint16_t* __restrict__ row, int begin, int end, float temperature,
                                           uint64_t seed) {
    Best b{-__builtin_inff(), nvr::kNoIndex};
    const bool gumbel = temperature > 0.0f;
    if constexpr (VEC) {
        constexpr int kLoads = 4;
        const int64_t step = 8 * int64_t(blockDim.x);
        for (int64_t t0 = begin + 8 * int64_t(threadIdx.x); t0 < end; t0 += kLoads * step) {
            uint4 w[kLoads];
#pragma unroll
            for (int u = 0; u < kLoads; ++u) {
                const int64_t t = t0 + u * step;  // 64-bit: vocab may sit close to INT_MAX
                if (t < end) w[u] = nvr::load_stream(row + t);
            }
#pragma unroll
            for (int u = 0; u < kLoads; ++u) {
                const int64_t t = t0 + u * step;
                if (t < end) {
                    if (gumbel) scan_chunk<true>(b, w[u], int(t), temperature, seed);
                    else scan_chunk<false>(b, w[u], int(t), temperature, seed);
                }
            }
        }
    } else {
        for (int64_t t = begin + int64_t(threadIdx.x); t < end; t += int64_t(blockDim.x)) {
            const float logit = nvr::bf16_to_f32(row[t]);
            const float s = gumbel ? nvr::gumbel_score(logit, temperature, seed, uint32_t(t)) : logit;
            consider(b, s, int(t));
        }
    }
    return b;
}

template <bool VEC>
__global__ __launch_bounds__(256) void sample_rows(const uint16_t* __restrict__ logits, const float* __restrict__ temps,
                                                   const uint64_t* __restrict__ seeds, int* __restrict__ out,
                                                   int vocab) {
    const int r = blockIdx.x;
    Best b = scan_range<VEC>(logits + int64_t(r) * vocab, 0, vocab, temps[r], seeds[r]);
    b = block_argmax(b);
    if (threadIdx.x == 0) out[r] = b.index == nvr::kNoIndex ? 0 : b.index;
}

// One partition of one row per 256-thread block. Each lane keeps C chunks of
// 8 logits in registers (partition width 2048*C tokens) with every load issued
// before any is scored; greedy rows compare, Gumbel rows score all 8*C tokens
// with the 8 independent hash/log chains of a chunk interleaved.
template <int C>
__global__ __launch_bounds__(256) void sample_partitions_vec(const uint16_t* __restrict__ logits,
                                                             const float* __restrict__ temps,
                                                             const uint64_t* __restrict__ seeds,
                                                             float* __restrict__ partial_scores,
                                                             int* __restrict__ partial_ids, int vocab, int parts) {
    constexpr int W = 2048 * C;
    const int r = blockIdx.x / parts;
    const int p = blockIdx.x - r * parts;
    const int begin = p * W;
    const int end = int(min(int64_t(begin) + W, int64_t(vocab)));
    const uint16_t* row = logits + int64_t(r) * vocab;

    uint4 w[C];
    int t0[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        t0[c] = begin + 8 * int(threadIdx.x) + 2048 * c;
        if (t0[c] < end) w[c] = nvr::load_stream(row + t0[c]);
    }
    const float temperature = temps[r];
    const uint64_t seed = seeds[r];
    Best b{-__builtin_inff(), nvr::kNoIndex};
    if (temperature > 0.0f) {
#pragma unroll
        for (int c = 0; c < C; ++c)
            if (t0[c] < end) scan_chunk<true>(b, w[c], t0[c], temperature, seed);
    } else {
#pragma unroll
        for (int c = 0; c < C; ++c)
            if (t0[c] < end) scan_chunk<false>(b, w[c], t0[c], temperature, seed);
    }
    b = block_argmax(b);
    if (threadIdx.x == 0) {
        partial_scores[blockIdx.x] = b.score;
        partial_ids[blockIdx.x] = b.index;
    }
}

// Generic partitions (unaligned rows or vocab % 8 != 0): 2048-token
// partitions scanned element by element.
__global__ __launch_bounds__(256) void sample_partitions_generic(const uint16_t* __restrict__ logits,
                                                                 const float* __restrict__ temps,
                                                                 const uint64_t* __restrict__ seeds,
                                                                 float* __restrict__ partial_scores,
                                                                 int* __restrict__ partial_ids, int vocab, int width,
                                                                 int parts) {
    const int r = blockIdx.x / parts;
    const int p = blockIdx.x - r * parts;
    const int begin = p * width;
    const int end = int(min(int64_t(begin) + width, int64_t(vocab)));
    Best b = scan_range<false>(logits + int64_t(r) * vocab, begin, end, temps[r], seeds[r]);
    b = block_argmax(b);
    if (threadIdx.x == 0) {
        partial_scores[blockIdx.x] = b.score;
        partial_ids[blockIdx.x] = b.index;
    }
}

__global__ __launch_bounds__(64) void sample_combine(const float* __restrict__ partial_scores,
                                                     const int* __restrict__ partial_ids, int* __restrict__ out,
                                                     int parts) {
    const int64_t base = int64_t(blockIdx.x) * parts;
    Best b{-__builtin_inff(), nvr::kNoIndex};
    for (int p = threadIdx.x; p < parts; p += kWave) consider(b, partial_scores[base + p], partial_ids[base + p]);
    b = wave_argmax(b);
    if (threadIdx.x == 0) out[blockIdx.x] = b.index == nvr::kNoIndex ? 0 : b.index;
}

// 16-byte row accesses need rows that start 16-byte aligned; token offsets
// inside a partition stay below INT_MAX when vocab leaves 8192 of headroom.
bool vector_rows(const void* logits, int vocab) {
    return vocab % 8 == 0 && vocab <= 0x7fffffff - 8192 && nvr::aligned(logits, 16);
}

int launch_serial(nv_context* c, const void* logits, const void* temps, const void* seeds, void* out, int batch,
                  int vocab) {
    auto l16 = static_cast<const uint16_t*>(logits);
    auto t = static_cast<const float*>(temps);
    auto s = static_cast<const uint64_t*>(seeds);
    auto o = static_cast<int*>(out);
    if (vector_rows(logits, vocab))
        hipLaunchKernelGGL(sample_rows<true>, dim3(batch), dim3(256), 0, c->stream, l16, t, s, o, vocab);
    else
        hipLaunchKernelGGL(sample_rows<false>, dim3(batch), dim3(256), 0, c->stream, l16, t, s, o, vocab);
    return nvr::launch_status();
}

}  // namespace

extern "C" {

int nv_sample(nv_context* c, const void* logits, const void* temps, const void* seeds, void* out, int batch,
              int vocab) {
    NVR_ACTIVATE(c);
    if (batch <= 0 || vocab <= 0) return nvr::fail(-2, "sample: dimensions must be positive");
    return launch_serial(c, logits, temps, seeds, out, batch, vocab);
}

int nv_sample_parallel(nv_context* c, const void* logits, const void* temps, const void* seeds, void* out,
                       void* partial_scores, void* partial_ids, int batch, int vocab) {
    NVR_ACTIVATE(c);
    if (batch <= 0 || vocab <= 0) return nvr::fail(-2, "sample_parallel: dimensions must be positive");
    const int64_t ref_parts = (int64_t(vocab) + kRefPartition - 1) / kRefPartition;
    if (ref_parts <= 1 || int64_t(batch) * ref_parts > 0x7fffffff)
        return launch_serial(c, logits, temps, seeds, out, batch, vocab);
    auto l16 = static_cast<const uint16_t*>(logits);
    auto t = static_cast<const float*>(temps);
    auto s = static_cast<const uint64_t*>(seeds);
    auto ps = static_cast<float*>(partial_scores);
    auto pi = static_cast<int*>(partial_ids);
    int parts;
    if (vector_rows(logits, vocab)) {
        // Never more partitions than the scratch holds (ceil(vocab / 2048)).
        parts = int((int64_t(vocab) + 2048 * kChunksPerLane - 1) / (2048 * kChunksPerLane));
        hipLaunchKernelGGL(sample_partitions_vec<kChunksPerLane>, dim3(unsigned(int64_t(batch) * parts)), dim3(256), 0,
                           c->stream, l16, t, s, ps, pi, vocab, parts);
    } else {
        parts = int(ref_parts);
        hipLaunchKernelGGL(sample_partitions_generic, dim3(unsigned(int64_t(batch) * parts)), dim3(256), 0, c->stream,
                           l16, t, s, ps, pi, vocab, kRefPartition, parts);
    }
    NVR_HIP(hipGetLastError());
    hipLaunchKernelGGL(sample_combine, dim3(batch), dim3(64), 0, c->stream, ps, pi, static_cast<int*>(out), parts);
    return nvr::launch_status();
}

}  // extern "C"
