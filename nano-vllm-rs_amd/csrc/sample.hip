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
// Layout of nv_sample_parallel (16-byte aligned rows, vocab % 8 == 0):
//   1. sample_partitions_vec: one 256-thread block per (row, partition of
//      2048 * kChunksPerLane tokens); every lane loads its chunks of 8 logits
//      up front; the block stores the partition's greedy maximum (greedy rows)
//      or the exact Gumbel score of that token (Gumbel rows).
//   2. sample_refine: Gumbel rows only. Exact pruning against the row's best
//      partial, then the surviving tokens are scored (see the kernel).
//   3. sample_combine: one wave folds a row's partials.
// Partitions are a multiple of the reference's 2048 tokens, so the caller's
// scratch (batch x ceil(vocab/2048) entries) always suffices. Other rows take
// 2048-token partitions scanned element by element, then stage 3.
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

// First pass, every row: one partition of one row per 256-thread block. Each
// lane keeps C chunks of 8 logits in registers (partition width 2048*C tokens)
// with every load issued before any is compared. The block stores the
// partition's greedy maximum, which is final for greedy rows; for Gumbel rows
// it stores the exact Gumbel score of that maximum's token instead, which seeds
// the pruning bound of sample_refine.
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
    Best b{-__builtin_inff(), nvr::kNoIndex};
#pragma unroll
    for (int c = 0; c < C; ++c)
        if (t0[c] < end) scan_chunk<false>(b, w[c], t0[c], 0.0f, 0);
    b = block_argmax(b);
    if (threadIdx.x == 0) {
        const float temperature = temps[r];
        float score = b.score;
        if (temperature > 0.0f && b.index != nvr::kNoIndex)
            score = nvr::gumbel_score(b.score, temperature, seeds[r], uint32_t(b.index));
        partial_scores[blockIdx.x] = score;
        partial_ids[blockIdx.x] = b.index;
    }
}

// Largest value the Gumbel term -ln(-ln(u)) takes over every u the hash can
// produce (exhaustive over all 2^23 uniforms with nvr_logf): 16.6355324.
constexpr float kNoiseMax = 0x1.0a2b24p+4f;

// Upper bound of a token's Gumbel score from its logit: logit * (1/T) is
// within a few ulp of the correctly rounded logit / T, and the 2^-18
// relative-plus-absolute margin covers that and the final rounding.
__device__ __forceinline__ float score_bound(float logit, float inv_t) {
    const float est = logit * inv_t;
    return (est + kNoiseMax) + (__builtin_fabsf(est) + 17.0f) * 0x1.0p-18f;
}

// Second pass, same grid as the first; blocks of greedy rows exit at once.
// (Striding a grid of eight blocks per CU over the items instead was measured
// no faster for greedy rows: their cost is the dependent launch itself.)
//
// Gumbel rows: exact branch-and-bound over the partition. S0 = the largest
// partial score of the row is the exact score of a real token (the first pass
// stored the score of each partition's largest logit; refined blocks overwrite
// theirs with their best), so a token whose score_bound is below S0 cannot be
// the row's winner. Partials read while other blocks overwrite them are still
// scores of real tokens, so the race only changes how much is pruned, never
// the result. Each wave compacts its own candidates into LDS (ballot + mbcnt,
// no block barrier) and scores them with every lane busy. The block then
// overwrites its partial. (A last-block combine through a ticket counter was
// measured 7x slower: publishing a partial at agent scope writes back and
// invalidates the L2 of the block's XCD.)
template <int C>
__global__ __launch_bounds__(256) void sample_refine(const uint16_t* __restrict__ logits,
                                                     const float* __restrict__ temps,
                                                     const uint64_t* __restrict__ seeds,
                                                     float* __restrict__ partial_scores, int* __restrict__ partial_ids,
                                                     int vocab, int parts) {
    constexpr int W = 2048 * C;
    constexpr int kLaneTokens = 8 * C;
    __shared__ uint32_t queue[4][kWave * kLaneTokens];
    const int r = blockIdx.x / parts;
    const int p = blockIdx.x - r * parts;
    const float temperature = temps[r];
    if (!(temperature > 0.0f)) return;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const uint64_t seed = seeds[r];
    const int64_t first = int64_t(r) * parts;
    const int begin = p * W;
    const int end = int(min(int64_t(begin) + W, int64_t(vocab)));
    const uint16_t* row = logits + int64_t(r) * vocab;

    // Every wave folds the row's partial scores itself (no block barrier). The
    // first 64 are loaded before the logits so the fold need not wait for them.
    float s0 = lane < parts ? __hip_atomic_load(partial_scores + first + lane, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT)
                            : -__builtin_inff();
    uint4 w[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int t = begin + 8 * int(threadIdx.x) + 2048 * c;
        w[c] = t < end ? nvr::load_stream(row + t) : make_uint4(0, 0, 0, 0);
    }
    for (int q = lane + kWave; q < parts; q += kWave)
        s0 = fmaxf(s0, __hip_atomic_load(partial_scores + first + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
#pragma unroll
    for (int m = kWave / 2; m > 0; m >>= 1) s0 = fmaxf(s0, nvr::xor_lane(s0, m));
    const float inv_t = 1.0f / temperature;

    // Compaction: entry = token offset in the partition (low 16 bits) | logit
    // bits (high 16 bits). A wave holds at most kWave * kLaneTokens entries.
    uint32_t* wq = queue[wave];
    int n = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const bool live = begin + 8 * int(threadIdx.x) + 2048 * c < end;
        float f[8];
        nvr::unpack8(w[c], f);
        const uint32_t words[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const bool take = live && !(score_bound(f[i], inv_t) < s0);
            const uint64_t ballot = __ballot(take);
            if (take) {
                const int pos = n + int(__builtin_amdgcn_mbcnt_hi(uint32_t(ballot >> 32),
                                                                  __builtin_amdgcn_mbcnt_lo(uint32_t(ballot), 0u)));
                const uint32_t bits = (i & 1) ? (words[i / 2] >> 16) : (words[i / 2] & 0xffffu);
                wq[pos] = uint32_t(8 * int(threadIdx.x) + 2048 * c + i) | (bits << 16);
            }
            n += __popcll(ballot);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // Two entries per lane per iteration; an odd tail scores one entry twice.
    Best best{-__builtin_inff(), nvr::kNoIndex};
    for (int q = lane; q < n; q += 2 * kWave) {
        const uint32_t e0 = wq[q];
        const uint32_t e1 = wq[q + kWave < n ? q + kWave : q];
        const int ta = begin + int(e0 & 0xffffu), tb = begin + int(e1 & 0xffffu);
        const float sa = nvr::gumbel_score(nvr::bf16_to_f32(uint16_t(e0 >> 16)), temperature, seed, uint32_t(ta));
        const float sb = nvr::gumbel_score(nvr::bf16_to_f32(uint16_t(e1 >> 16)), temperature, seed, uint32_t(tb));
        consider(best, sa, ta);
        consider(best, sb, tb);
    }
    best = block_argmax(best);
    if (threadIdx.x == 0) {
        __hip_atomic_store(partial_scores + blockIdx.x, best.score, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(partial_ids + blockIdx.x, best.index, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
        const int items = batch * parts;
        hipLaunchKernelGGL(sample_partitions_vec<kChunksPerLane>, dim3(unsigned(items)), dim3(256), 0, c->stream, l16,
                           t, s, ps, pi, vocab, parts);
        NVR_HIP(hipGetLastError());
        hipLaunchKernelGGL(sample_refine<kChunksPerLane>, dim3(unsigned(items)), dim3(256), 0, c->stream, l16, t, s,
                           ps, pi, vocab, parts);
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
