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
// Layout of nv_sample_parallel (16-byte aligned rows, vocab % 8 == 0) from
// 17 rows (up to 16: sample_partitions_full scores every token of 2048-token
// partitions, then stage 3):
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
//
// Large batches (at least one row per CU, rows of at most 20 * 8192 tokens)
// take one launch instead, in which a 1024-thread block keeps a row's worth
// of logits in registers (Qwen3's 151936 logits are 76 VGPRs a lane), so every
// logit is read from HBM once and no partials or second launch are needed.
// sample_paired (up to 16384 rows, with the context's exchange words) gives
// each block half of its own row and half of a partner row of the other kind,
// a greedy row with a Gumbel row; sample_resident (otherwise) gives each block
// one whole row.
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
// Batches of at most this many rows score every token exactly in one pass
// (sample_partitions_full) instead of pruning in a second one. Measured on
// MI355X at 151936 tokens, half greedy / half T = 0.6 and all T = 0.6: 8 rows
// 7.8 / 8.5 us against 10.7 / 11.1 us, 16 rows 9.7 / 11.0 against
// 11.6 / 12.4 us; at 32 rows the two paths are even.
constexpr int kFullScoreRows = 16;

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

// Small batches: one pass in which Gumbel rows score every token of the
// partition exactly (the greedy rows as sample_partitions_vec), then
// sample_combine. At a few rows the batch's whole scoring is a few million
// hashes and logarithms spread over every CU, cheaper than the pruning pass
// and its extra dependent launch.
template <int C>
__global__ __launch_bounds__(256) void sample_partitions_full(const uint16_t* __restrict__ logits,
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
            if (t0[c] < end) scan_chunk<false>(b, w[c], t0[c], 0.0f, 0);
    }
    b = block_argmax(b);
    if (threadIdx.x == 0) {
        partial_scores[blockIdx.x] = b.score;
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

// ------------------------------------------------------ row-resident ----
// Threads per resident block; a row takes 1024 / kResThreads blocks. Two
// 512-thread blocks per row (halves folded by sample_combine; parity-tested)
// measured slower at 256 rows of 151936 on MI355X: greedy 20.1 vs 15.9 us,
// T = 0.6 52.4 vs 37.6 us (each half prunes against its own, weaker s0),
// half and half 40.8 vs 37.2 us.
constexpr int kResThreads = 1024;
constexpr int kResMaxChunks = 20;  // 16-byte chunks per lane: a part holds at most 20 * 8 * TPB tokens
constexpr int kXFloors = 1024;     // tabulated per-logit hash floors (see sample_resident)
// Noise thresholds at D_k = -4 + k/16, k < kFloorSteps; the last lies above kNoiseMax.
constexpr int kFloorSteps = 336;
// Block geometry: TPB threads per block (1024: one block per CU holding a
// whole row; 512: two blocks per CU, each holding half a row). Candidate
// queues per wave fill the block's share of the CU's 160 KiB of LDS.
template <int TPB>
struct ResGeometry {
    static constexpr int kWaves = TPB / kWave;
    static constexpr int kQueue = TPB == 1024 ? 2432 : 2304;
    static constexpr size_t kLdsBytes = sizeof(uint32_t) * (size_t(kWaves) * kQueue + kFloorSteps + kXFloors) +
                                        3 * kWaves * (sizeof(float) + sizeof(int));
    static_assert(kLdsBytes * (1024 / TPB) <= 160 * 1024, "the resident sampler's blocks must fit one CU's LDS");
};

// Lower bound of the hash values whose Gumbel noise -ln(-ln(u)) reaches D_k:
// every m (the top 23 hash bits) with noise(m) >= D_k has m >= noise_floor(k).
// The noise is increasing in m with inverse u = exp(-exp(-D)); it is evaluated
// at D_k - 2^-12 and 64 units are subtracted: slack that covers the error of
// the noise's two nvr_logf calls (below 2e-6 in D) and of nvr_expf (a few
// units in m) many times over. Above kNoiseMax no m qualifies.
__device__ __forceinline__ uint32_t noise_floor(int k) {
    const float d = float(k) * 0.0625f - 4.0f;
    if (d > kNoiseMax) return 1u << 23;
    const float u = nvr::nvr_expf(-nvr::nvr_expf(-(d - 0x1.0p-12f)));
    const float m = floorf(u * 8388608.0f) - 64.0f;
    return m > 0.0f ? uint32_t(m) : 0u;
}

// Exact pruning of a candidate against s0, the score of a real token of the
// row. With q = logit/T and est = logit * (1/T) within 2^-22 of q, the score
// RN(q + noise) is below s0 whenever noise < dc = (s0 - est) - (|s0| + |est| +
// 17) * 2^-17; the margin covers est's error, the roundings of dc and of the
// score, and one ulp of s0. noise(m) < D_k <= dc for every m < noise_floor(k),
// so a candidate needs its exact score only when m >= hash_floor(...), which
// is 0 (always score) when pruning is off or dc is below the table.
struct Pruner {
    float s0, inv_t, temperature;
    uint64_t seed;
    bool on;  // s0 and 1/T finite
    const uint32_t* floors;
};
__device__ __forceinline__ uint32_t hash_floor(const Pruner& p, float logit) {
    const float est = logit * p.inv_t;
    const float dc = (p.s0 - est) - (__builtin_fabsf(p.s0) + __builtin_fabsf(est) + 17.0f) * 0x1.0p-17f;
    const bool use = p.on & (dc >= -4.0f);  // false for NaN
    int k = use ? int(fminf((dc + 4.0f) * 16.0f, float(kFloorSteps - 1))) : 0;
    k -= (float(k) * 0.0625f - 4.0f > dc) ? 1 : 0;  // (dc + 4) rounded up across a grid point
    const uint32_t f = p.floors[k < 0 ? 0 : k];
    return use ? f : 0u;
}
// The top 23 bits of the token's hash (the uniform's numerator).
__device__ __forceinline__ uint32_t hash_m(uint64_t seed, uint32_t token) {
    return uint32_t(nvr::splitmix64(seed ^ (uint64_t(token) * nvr::kTokenMix)) >> 41);
}
// gumbel_score from the hash's top bits.
__device__ __forceinline__ float score_from_m(float logit, float temperature, uint32_t m) {
    const float u = (float(m) + 0.5f) * (1.0f / 8388608.0f);
    return logit / temperature - nvr::nvr_logf(-nvr::nvr_logf(u));
}

// Scores queue entries [begin, count), two per lane per iteration (an odd
// tail scores one entry twice). Entry = f32 bits of the logit (low 16 bits
// zero) | chunk round k << 9 | lane << 3 | element; chunk = k * stride + base +
// lane, base being the compacting wave's first chunk of round 0. TAB: the
// hash floor of a logit is read from xfloors, indexed by its bf16 bits minus
// lxb, instead of computed.
template <bool TAB>
__device__ __forceinline__ void score_queue(const uint32_t* queue, int begin, int count, int lane, int base,
                                            int stride, const Pruner& p, const uint32_t* xfloors, int lxb,
                                            Best& best) {
    for (int j = begin + lane; j < count; j += 2 * kWave) {
        const uint32_t e0 = queue[j];
        const uint32_t e1 = queue[j + kWave < count ? j + kWave : j];
        // Chunk k * stride + base + lane (k < 32 and stride, base below 2^24:
        // a full-rate 24-bit multiply).
        const int ta = 8 * int(__umul24(e0 >> 9 & 31u, uint32_t(stride)) + uint32_t(base) + (e0 >> 3 & 63u)) +
                       int(e0 & 7u);
        const int tb = 8 * int(__umul24(e1 >> 9 & 31u, uint32_t(stride)) + uint32_t(base) + (e1 >> 3 & 63u)) +
                       int(e1 & 7u);
        const float xa = __uint_as_float(e0 & 0xffff0000u), xb = __uint_as_float(e1 & 0xffff0000u);
        // Floors and both hashes before one rare branch, so the two hash
        // chains interleave; a token below its floor scores below s0 and is
        // skipped (its score would not change `best`).
        const uint32_t fa = TAB ? xfloors[int(e0 >> 16) - lxb] : hash_floor(p, xa);
        const uint32_t fb = TAB ? xfloors[int(e1 >> 16) - lxb] : hash_floor(p, xb);
        const uint32_t ma = hash_m(p.seed, uint32_t(ta)), mb = hash_m(p.seed, uint32_t(tb));
        if ((ma >= fa) | (mb >= fb)) {
            if (ma >= fa) consider(best, score_from_m(xa, p.temperature, ma), ta);
            if (mb >= fb) consider(best, score_from_m(xb, p.temperature, mb), tb);
        }
    }
}

// Argmax over a block of W waves; the result is valid in every thread. Each
// call needs its own W slots in `scores` / `ids`.
template <int W>
__device__ __forceinline__ Best block_fold(Best b, float* scores, int* ids) {
    b = wave_argmax(b);
    if ((threadIdx.x & (kWave - 1)) == 0) {
        scores[threadIdx.x / kWave] = b.score;
        ids[threadIdx.x / kWave] = b.index;
    }
    __syncthreads();
    Best r{scores[0], ids[0]};
#pragma unroll
    for (int w = 1; w < W; ++w) consider(r, scores[w], ids[w]);
    return r;
}

// Phase 1 of the resident samplers, as the chunks arrive: the lane's best
// chunk under "higher maximum wins; an equal maximum only while there is
// none" (the lane sees its tokens in increasing order, so that keeps the
// lowest index, and a lane of -inf logits picks its first chunk), then the
// lowest token of that chunk holding the maximum. Chunk k of the lane is
// k * stride + first; chunks past the row end become NaN, which fmaxf skips
// and which never wins or becomes a candidate. Branch-free.
constexpr uint32_t kNaN2 = 0x7fc07fc0u;
template <int C>
__device__ __forceinline__ Best lane_best(uint4 (&w)[C], int stride, int first, int chunks) {
    float bv = -__builtin_inff();
    int bk = -1;
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const bool valid = k * stride + first < chunks;
        w[k].x = valid ? w[k].x : kNaN2;
        w[k].y = valid ? w[k].y : kNaN2;
        w[k].z = valid ? w[k].z : kNaN2;
        w[k].w = valid ? w[k].w : kNaN2;
        float f[8];
        nvr::unpack8(w[k], f);
        const float m = fmaxf(fmaxf(fmaxf(f[0], f[1]), fmaxf(f[2], f[3])), fmaxf(fmaxf(f[4], f[5]), fmaxf(f[6], f[7])));
        const bool take = (m > bv) | ((bk < 0) & (m == bv));
        bv = take ? m : bv;
        bk = take ? k : bk;
    }
    // The lowest token of the best chunk holding bv (select over the chunks,
    // no dynamic register indexing).
    uint4 bw = make_uint4(kNaN2, kNaN2, kNaN2, kNaN2);
#pragma unroll
    for (int k = 0; k < C; ++k) {
        bw.x = bk == k ? w[k].x : bw.x;
        bw.y = bk == k ? w[k].y : bw.y;
        bw.z = bk == k ? w[k].z : bw.z;
        bw.w = bk == k ? w[k].w : bw.w;
    }
    Best lb{bv, nvr::kNoIndex};
    float f[8];
    nvr::unpack8(bw, f);
    int e = 8;
#pragma unroll
    for (int i = 7; i >= 0; --i) e = f[i] == bv ? i : e;
    if (bk >= 0) lb.index = 8 * (bk * stride + first) + e;
    // Keep only the packed words live into the later phases (without this the
    // compiler keeps the unpacked floats instead, twice the registers).
#pragma unroll
    for (int k = 0; k < C; ++k) __asm__ volatile("" : "+v"(w[k].x), "+v"(w[k].y), "+v"(w[k].z), "+v"(w[k].w));
    return lb;
}

// The candidates of a Gumbel row pruned against s0 are exactly the logits
// x >= lx, lx the smallest bf16 value with x * (1/T) >= (s0 - kNoiseMax) -
// (|s0| + 34) * 2^-17 (x * (1/T) is nondecreasing in x; the margin covers
// 1/T's and the score's roundings), in the order-preserving 16-bit keys of
// the bf16 values (-inf .. +inf). bound * T lies within a few fp32 ulps of
// that threshold, so its key (rounded toward -inf) is at most a step from
// lx's: two steps up while the predicate fails, two down while the key below
// passes, and the key is exact once it passes and the one below does not
// (tests/cpp/candidate_floor_check.cpp compares it with the full search on
// millions of (s0, T) pairs, edge cases included). Past the range
// where that holds, or if the steps do not settle, a binary search over all
// keys (16 dependent steps) decides. -inf when pruning is off.
__device__ __forceinline__ float candidate_floor(float s0, float inv_t, float t, bool on) {
    if (!on) return -__builtin_inff();
    const float bound = (s0 - kNoiseMax) - (__builtin_fabsf(s0) + 34.0f) * 0x1.0p-17f;
    auto value = [](int key) { return nvr::bf16_to_f32(uint16_t(key >= 0x8000 ? key - 0x8000 : 0xffff - key)); };
    auto pass = [&](int key) { return value(key) * inv_t >= bound; };
    const float v0 = bound * t;
    const uint32_t u = __float_as_uint(v0);
    int key = (u & 0x80000000u) ? 0xffff - int((u >> 16) + ((u & 0xffffu) != 0u)) : int(u >> 16) + 0x8000;
    if (__builtin_fabsf(v0) >= 0x1.0p-100f && __builtin_fabsf(v0) <= 0x1.0p+100f) {
        key += !pass(key);
        key += !pass(key);
        key -= pass(key - 1);
        key -= pass(key - 1);
        if (pass(key) && !pass(key - 1)) return value(key);
    }
    int lo = 0x007f, hi = 0xff80;  // -inf, +inf; +inf always qualifies
    if (pass(lo)) hi = lo;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (pass(mid)) hi = mid;
        else lo = mid;
    }
    return value(hi);
}

// One window of a wave's compaction: the candidates (x >= lx) of the lane's
// chunks, in chunk and element order across the wave, from queue position
// `window` on, at most `capacity` of them (ballot + mbcnt). Entry = f32 bits
// of the logit (low 16 bits zero) | chunk round k << 9 | lane << 3 |
// element. Returns the wave's candidate count minus `window`.
template <int C>
__device__ __forceinline__ int compact_window(uint4 (&w)[C], float lx, uint32_t* queue, int window, int capacity,
                                              uint32_t lane_code) {
    int n = -window;  // queue position of the next candidate
#pragma unroll
    for (int k = 0; k < C; ++k) {
        // Opaque per window, so the compiler recomputes the keys from the
        // packed words instead of hoisting 8 C of them out of the loop.
        __asm__ volatile("" : "+v"(w[k].x), "+v"(w[k].y), "+v"(w[k].z), "+v"(w[k].w));
        const uint32_t words[4] = {w[k].x, w[k].y, w[k].z, w[k].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t xb = (i & 1) ? (words[i / 2] & 0xffff0000u) : (words[i / 2] << 16);
            const bool take = __uint_as_float(xb) >= lx;
            const uint64_t ballot = __ballot(take);
            const uint32_t pos = __builtin_amdgcn_mbcnt_hi(uint32_t(ballot >> 32),
                                                           __builtin_amdgcn_mbcnt_lo(uint32_t(ballot), uint32_t(n)));
            if (take & (pos < uint32_t(capacity))) queue[pos] = xb | lane_code | uint32_t(k << 9 | i);
            n += int(__popcll(ballot));
        }
    }
    return n;
}

// compact_window for waves that run two to a SIMD, with the same entries
// in the same order: a chunk's eight ballots are taken before any position,
// so no element waits on the previous one's scalar count. Where a chunk's
// every position lies inside the window, each element is one store under
// exec = its ballot. Otherwise every lane stores: the queue holds
// `capacity` entries followed by one spare per lane; a non-candidate stores
// into its lane's spare, a candidate past the window into min(position,
// capacity + lane), a spare too (each of those slots holds junk).
typedef __attribute__((address_space(3))) uint32_t lds_word;
template <int C>
__device__ __forceinline__ int compact_window_dense(uint4 (&w)[C], float lx, uint32_t* queue, int window,
                                                    int capacity, uint32_t lane_code) {
    const uint32_t spare = uint32_t(capacity) + (lane_code >> 3);
    // The queue's LDS byte address (wave-uniform, so scalar).
    const uint32_t qbase =
        __builtin_amdgcn_readfirstlane(uint32_t(reinterpret_cast<size_t>((lds_word*)queue)));
    int n = -window;
#pragma unroll
    for (int k = 0; k < C; ++k) {
        __asm__ volatile("" : "+v"(w[k].x), "+v"(w[k].y), "+v"(w[k].z), "+v"(w[k].w));
        const uint32_t words[4] = {w[k].x, w[k].y, w[k].z, w[k].w};
        uint32_t xb[8];
        uint64_t bal[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            xb[i] = (i & 1) ? (words[i / 2] & 0xffff0000u) : (words[i / 2] << 16);
            bal[i] = __ballot(__uint_as_float(xb[i]) >= lx);
        }
        if (n >= 0 && n + 8 * kWave <= capacity) {
            // Every position of this chunk lies in [0, capacity): a candidate's
            // address is qn (the queue's address of entry n, scalar) plus 4
            // times the candidates below it.
            // The round's code in a register of its own, so that each entry is
            // one or3 with the element index as an inline constant (no scalar
            // move per element).
            uint32_t code = lane_code | uint32_t(k << 9);
            __asm__("" : "+v"(code));
            uint32_t qn = qbase + 4 * uint32_t(n);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t below = __builtin_amdgcn_mbcnt_hi(uint32_t(bal[i] >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo(uint32_t(bal[i]), 0u));
                // Only the candidate lanes write: exec is the ballot for the one
                // LDS store (restored at once), so no per-lane select. The
                // compiler's wait counting does not see this store. Reads by
                // the same wave need no wait (a wave's LDS operations complete
                // in order); a caller that hands the queue to other waves
                // waits for it explicitly before the barrier.
                uint64_t saved;
                __asm__ volatile(
                    "s_and_saveexec_b64 %0, %3\n\t"
                    "ds_write_b32 %1, %2\n\t"
                    "s_mov_b64 exec, %0"
                    : "=&s"(saved)
                    : "v"(qn + 4 * below), "v"(xb[i] | code | uint32_t(i)), "s"(bal[i])
                    : "memory", "scc");
                // qn += 4 * popcount, one scalar shift-add
                __asm__("s_lshl2_add_u32 %0, %1, %0" : "+s"(qn) : "s"(uint32_t(__popcll(bal[i]))) : "scc");
            }
            n = int((qn - qbase) / 4);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t pos = __builtin_amdgcn_mbcnt_hi(
                    uint32_t(bal[i] >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(bal[i]), uint32_t(n)));
                // the ballot is the candidate lanes' mask: select on it directly
                // (as a plain select the compiler masks exec around the position)
                uint32_t to;
                __asm__("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(to) : "v"(spare), "v"(min(pos, spare)), "s"(bal[i]));
                queue[to] = xb[i] | lane_code | uint32_t(k << 9 | i);
                n += int(__popcll(bal[i]));
            }
        }
    }
    return n;
}

// Most tokens are candidates (high temperature, flat rows): queue windows
// would cost more than they save, so every lane scores its own candidates,
// re-reading its chunks k * stride + first (cache hits).
__device__ __forceinline__ void score_in_place(const uint16_t* row, int first, int stride, int chunks, float lx,
                                               const Pruner& p, Best& best) {
    const uint32_t* words = reinterpret_cast<const uint32_t*>(row);
#pragma unroll 1
    for (int c = first; c < chunks; c += stride) {
        const uint4 v = *reinterpret_cast<const uint4*>(words + 4 * c);
        const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float x = __uint_as_float((i & 1) ? (vw[i / 2] & 0xffff0000u) : (vw[i / 2] << 16));
            if (x >= lx) {
                const uint32_t f = hash_floor(p, x), m = hash_m(p.seed, uint32_t(8 * c + i));
                if (m >= f) consider(best, score_from_m(x, p.temperature, m), 8 * c + i);
            }
        }
    }
}

// One row (parts == 1) or one half of a row (parts == 2) per block, resident
// in registers: lane t of part p holds chunks k * parts * TPB + p * TPB + t
// (k < C) of 8 logits, all loads issued first. A whole row writes out[row];
// a half writes its (score, index) to the partials, for sample_combine. Phase 1 (as the chunks arrive): the lane's greedy maximum. Greedy rows
// end with the block's maximum. Gumbel rows: every lane scores its maximum's
// token exactly; the best of those real scores (of this part) is s0, a lower
// bound for the part's own winner. A token whose
// logit * (1/T) is below E = (s0 - kNoiseMax) - (|s0| + 34) * 2^-17 cannot
// reach s0 (the noise never exceeds kNoiseMax; the margin covers 1/T's and the
// score's roundings), so each wave compacts the others into its LDS queue
// (ballot + mbcnt) and scores them; a test of the token's hash rejects
// almost all without the two logarithms and the division (hash_floor).
//
// Cost model: every row sits on one CU, so each VALU instruction spent per
// logit costs the whole batch about 1 us (151936 logits / 64 lanes per
// wave-instruction at one wave-instruction per cycle per CU); the compaction
// is therefore kept at a handful of instructions per logit.
template <int C, int TPB>
__global__ __launch_bounds__(TPB) void sample_resident(const uint16_t* __restrict__ logits,
                                                       const float* __restrict__ temps,
                                                       const uint64_t* __restrict__ seeds, int* __restrict__ out,
                                                       float* __restrict__ partial_scores,
                                                       int* __restrict__ partial_ids, int vocab, int parts,
                                                       int partial_stride) {
    using G = ResGeometry<TPB>;
    constexpr int kW = G::kWaves, kQ = G::kQueue;
    extern __shared__ __align__(16) uint32_t lds[];
    uint32_t* floors = lds + kW * kQ;
    uint32_t* xfloors = floors + kFloorSteps;
    float* fold_s = reinterpret_cast<float*>(xfloors + kXFloors);
    int* fold_i = reinterpret_cast<int*>(fold_s + 3 * kW);
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int r = blockIdx.x / parts, part = blockIdx.x - r * parts;
    const int chunks = vocab / 8;
    const int stride = parts * TPB;       // chunks between a lane's rounds
    const int first = part * TPB + tid;   // the lane's round-0 chunk
    const uint16_t* row = logits + int64_t(r) * vocab;
    auto finish = [&](const Best& b) {
        if (tid != 0) return;
        if (parts == 1) {
            out[r] = b.index == nvr::kNoIndex ? 0 : b.index;
        } else {
            partial_scores[int64_t(r) * partial_stride + part] = b.score;
            partial_ids[int64_t(r) * partial_stride + part] = b.index;
        }
    };

    uint4 w[C];
#pragma unroll
    for (int k = 0; k < C; ++k) w[k] = nvr::load_stream(row + 8 * int64_t(min(k * stride + first, chunks - 1)));
    const float temperature = temps[r];
    const uint64_t seed = seeds[r];
    const bool gumbel = temperature > 0.0f;
    if (gumbel)
        for (int k = tid; k < kFloorSteps; k += TPB) floors[k] = noise_floor(k);

    const Best lb = lane_best<C>(w, stride, first, chunks);
    const Best top = block_fold<kW>(lb, fold_s, fold_i);
    if (!gumbel) {
        finish(top);
        return;
    }

    // Phase 2: s0 from the lanes' maxima (each the score of a real token).
    Best own{-__builtin_inff(), nvr::kNoIndex};
    if (lb.index != nvr::kNoIndex) own = Best{nvr::gumbel_score(lb.score, temperature, seed, uint32_t(lb.index)), lb.index};
    const Best seeded = block_fold<kW>(own, fold_s + kW, fold_i + kW);
    const float s0 = seeded.score, inv_t = 1.0f / temperature;
    const bool on = __builtin_fabsf(s0) < __builtin_inff() && inv_t < __builtin_inff();
    const float lx = candidate_floor(s0, inv_t, temperature, on);

    // Phase 3: each wave compacts its candidates into its LDS queue (ballot +
    // mbcnt) and scores them, in rounds of kQ entries when there are
    // more (a round re-runs the compaction from the registers and keeps the
    // next window). Entry = f32 bits of the logit (low 16 bits zero) | chunk
    // round k << 9 | lane << 3 | element. Chunks past the row end are NaN and
    // never candidates. The counts vary between rows far more than between
    // the waves of a row (measured), so each wave scores its own queue.
    uint32_t* queue = lds + wave * kQ;
    const uint32_t lane_code = uint32_t(lane) << 3;
    const int base = part * TPB + wave * kWave;
    const Pruner p{s0, inv_t, temperature, seed, on, floors};
    Best best = seeded;
    // When every candidate is positive (lx > 0) and the candidates span at
    // most kXFloors bf16 values (lx up to the row maximum), hash_floor is
    // tabulated once per value (a few hundred at low temperatures) instead of
    // computed per candidate. Positive bf16 values order like their bits.
    const int lxb = int(__float_as_uint(lx) >> 16);
    const int span = (on & (lx > 0.0f) & (top.score >= lx)) ? int(__float_as_uint(top.score) >> 16) - lxb + 1 : 0;
    const bool tab = span > 0 && span <= kXFloors;
    if (tab) {
        for (int j = tid; j < span; j += TPB) xfloors[j] = hash_floor(p, nvr::bf16_to_f32(uint16_t(lxb + j)));
        __syncthreads();
    }
    for (int window = 0;; window += kQ) {
        const int n = compact_window<C>(w, lx, queue, window, kQ, lane_code);
        if (window == 0 && n > 2 * kQ) {
            score_in_place(row, first, stride, chunks, lx, p, best);
            break;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int count = min(n, kQ);
        if (tab) score_queue<true>(queue, 0, count, lane, base, stride, p, xfloors, lxb, best);
        else score_queue<false>(queue, 0, count, lane, base, stride, p, xfloors, lxb, best);
        if (n <= kQ) break;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    best = block_fold<kW>(best, fold_s + 2 * kW, fold_i + 2 * kW);
    finish(best);
}

// ------------------------------------------------------- paired halves ----
// One 1024-thread block per row, like sample_resident, but each block holds
// two half rows: waves 0-7 (slot 0) take half 0 of row b = blockIdx.x and
// waves 8-15 (slot 1) half 1 of row partner_row(b). Half h of a row is its
// chunks k * 1024 + 512 h + t (t < 512, k < C). Partners pair each Gumbel
// row (T > 0) with a greedy row, so with one row per CU a mixed batch puts
// half a Gumbel row and half a greedy row on every CU instead of a whole
// Gumbel row on half of them: once the greedy half is done (its maximum
// needs no second pass), its waves score the back halves of the Gumbel
// half's candidate queues. Rows left without a partner hold both halves in
// one block, which then works as sample_resident does.
//
// A row split over two blocks needs two exchanges, through the context's
// per-row words (two uint64, zero between launches): X, the halves' s0 (the
// best exact score of their lane maxima), each half ORing its order key into
// its 32 bits and waiting a bounded time for the other's, so that both prune
// against the better s0 (a real token's score, so pruning stays exact); and
// Y, the halves' (score, index) keys met in a 64-bit atomic maximum, whose
// returned value tells the second half that it holds both: it writes the
// token and zeroes X and Y. A half that waits in vain (its partner's block
// not yet resident, when rows outnumber CUs) prunes against its own s0.
constexpr int kPairThreads = 1024, kPairWaves = 16, kSlotThreads = 512, kSlotWaves = 8;
constexpr int kPairQueue = 2304;   // queue entries per wave: kPairCap, then a spare per lane
constexpr int kPairCap = kPairQueue - kWave;
constexpr int kPairRows = 16384;   // rows of the context's exchange words
constexpr int kPairWaitTicks = 400;  // 4 us of the 100 MHz realtime counter
constexpr size_t kPairLdsBytes =
    sizeof(uint32_t) * (size_t(kPairWaves) * kPairQueue + kFloorSteps + 2 * kXFloors) +
    3 * kPairWaves * (sizeof(float) + sizeof(int)) + kPairWaves * sizeof(int) + 2 * sizeof(float) + sizeof(int);
static_assert(kPairLdsBytes <= 160 * 1024, "the paired sampler's block must fit one CU's LDS");

// Order key of a score for the exchanges: increasing in the score, -0 and +0
// equal, at least 0x007fffff (-inf) for every non-NaN score, so 0 means absent.
__device__ __forceinline__ uint32_t score_key(float s) {
    const uint32_t u = __float_as_uint(s == 0.0f ? 0.0f : s);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_score(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
// (score, index) as one key ordered like `better`: higher score, then lower
// index. "No winner" is the smallest key that is not zero.
__device__ __forceinline__ uint64_t result_key(const Best& b) {
    if (b.index == nvr::kNoIndex) return uint64_t(1) << 32;
    return (uint64_t(score_key(b.score)) << 32) | uint32_t(0x7fffffff - b.index);
}

// The row whose half 1 block b's slot 1 holds: the k-th Gumbel row and the
// k-th greedy row (in row order) are partners; rows beyond the shorter list
// are their own partners. partner_row(partner_row(b)) == b, so every half is
// taken once. Wave-uniform; every lane of the wave takes part. Up to
// 64 * kDealLoads rows it works on temperatures loaded by load_deal, which
// the kernel issues before any logit load of the block: behind those (152 KB
// per CU) a load would wait for the CU's share of the memory bandwidth.
constexpr int kDealLoads = 16;
struct DealTemps {
    float t[kDealLoads];  // temps[64 c + lane] (clamped to the last row)
    float own;            // temps[b]
};
__device__ __forceinline__ DealTemps load_deal(const float* temps, int batch, int b, int lane) {
    DealTemps d;
    d.own = temps[b];
#pragma unroll
    for (int c = 0; c < kDealLoads; ++c) d.t[c] = temps[min(c * kWave + lane, batch - 1)];
    return d;
}
__device__ __forceinline__ int partner_row(const float* temps, const DealTemps& d, int batch, int b, int lane) {
    // Every value below is wave-uniform; taking the row's own temperature
    // from the first lane lets the compiler keep the rank and both walks in
    // scalar registers instead of running them as per-lane divergent loops.
    const bool gum = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(d.own))) > 0.0f;
    const bool one_round = batch <= kWave * kDealLoads;
    uint64_t kinds[kDealLoads];  // bit l of kinds[c]: row 64 c + l is Gumbel
#pragma unroll
    for (int c = 0; c < kDealLoads; ++c) kinds[c] = __ballot(c * kWave + lane < batch && d.t[c] > 0.0f);
    auto kind_mask = [&](int c) {  // Gumbel rows among 64 c .. 64 c + 63
        if (one_round) {
            uint64_t m = 0;
#pragma unroll
            for (int k = 0; k < kDealLoads; ++k) m = k == c ? kinds[k] : m;
            return m;
        }
        const int i = c * kWave + lane;
        return uint64_t(__ballot(i < batch && temps[i] > 0.0f));
    };
    const int nc = (batch + kWave - 1) / kWave;
    int before = 0, total = 0;  // Gumbel rows before b, and in all
    for (int c = 0; c < nc; ++c) {
        const uint64_t g = kind_mask(c);
        total += __popcll(g);
        const int off = b - c * kWave;
        if (off >= 0) before += __popcll(off >= kWave ? g : g & ((uint64_t(1) << off) - 1));
    }
    const int rank = gum ? before : b - before;
    if (rank >= (gum ? batch - total : total)) return b;
    int seen = 0;
    for (int c = 0; c < nc; ++c) {
        const uint64_t valid = c * kWave + kWave <= batch ? ~uint64_t(0) : (uint64_t(1) << (batch - c * kWave)) - 1;
        const uint64_t m = (gum ? ~kind_mask(c) : kind_mask(c)) & valid;  // rows of the other kind
        const int n = __popcll(m);
        if (rank < seen + n) {
            // The (rank - seen)-th set bit of m: the one lane whose bit is set
            // and which counts exactly that many set bits of m below itself.
            const uint32_t below = __builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u));
            const uint64_t at = __ballot(((m >> lane) & 1) != 0 && int(below) == rank - seen);
            return c * kWave + __builtin_ctzll(at);
        }
        seen += n;
    }
    return b;
}

// Best over waves [w0, w0 + n) of a fold array (n <= 16), in every lane (all
// lanes active): lane l of each 16-lane row takes entry l, then a butterfly
// inside the row (DPP moves). `better` orders (score, index) pairs totally
// and no NaN score reaches a fold, so the winner is the one a left-to-right
// fold finds, in 4 dependent steps instead of n - 1.
__device__ __forceinline__ Best fold_waves(const float* s, const int* i, int w0, int n) {
    const int l = int(threadIdx.x) & 15;
    Best r{-__builtin_inff(), nvr::kNoIndex};
    if (l < n) r = Best{s[w0 + l], i[w0 + l]};
#pragma unroll
    for (int mask = 8; mask > 0; mask >>= 1) consider(r, nvr::xor_lane(r.score, mask), nvr::xor_lane(r.index, mask));
    return r;
}

// X exchange of half `half` of row r (one thread): publish s0's key, wait for
// the other half's, return the better of the two.
__device__ __forceinline__ float exchange_s0(uint64_t* state, int r, int half, float s0) {
    uint64_t* x = state + 2 * int64_t(r);
    const uint64_t old = __hip_atomic_fetch_or(x, uint64_t(score_key(s0)) << (32 * half), __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
    uint32_t other = uint32_t(old >> (32 * (1 - half)));
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (other == 0 && int64_t(__builtin_amdgcn_s_memrealtime() - t0) < kPairWaitTicks) {
        __builtin_amdgcn_s_sleep(1);
        other = uint32_t(__hip_atomic_load(x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >> (32 * (1 - half)));
    }
    return other != 0 ? fmaxf(s0, key_score(other)) : s0;
}

// Y exchange (one thread): meet the other half's result; the second half to
// arrive writes the token and leaves both words zero for the next launch.
__device__ __forceinline__ void deposit(uint64_t* state, int r, const Best& b, int* out) {
    uint64_t* x = state + 2 * int64_t(r);
    const uint64_t key = result_key(b);
    const uint64_t old = __hip_atomic_fetch_max(x + 1, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == 0) return;
    const uint64_t m = old > key ? old : key;
    out[r] = (m >> 32) == 1 ? 0 : int(0x7fffffff - uint32_t(m));
    __hip_atomic_store(x + 1, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(x, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Queue entries [0, split(n)) are scored by their compacting wave, the rest
// by its helper in the other slot (a multiple of two entries per lane).
__device__ __forceinline__ int helper_split(int n) { return min(n, (n + 4 * kWave - 1) / (4 * kWave) * (2 * kWave)); }

template <int C>
__global__ __launch_bounds__(kPairThreads) void sample_paired(const uint16_t* __restrict__ logits,
                                                             const float* __restrict__ temps,
                                                             const uint64_t* __restrict__ seeds,
                                                             int* __restrict__ out, uint64_t* __restrict__ state,
                                                             int vocab, int batch) {
    constexpr int kQ = kPairQueue, kCap = kPairCap, stride = 2 * kSlotThreads;
    extern __shared__ __align__(16) uint32_t lds[];
    uint32_t* floors = lds + kPairWaves * kQ;
    uint32_t* xfloors = floors + kFloorSteps;                            // [2][kXFloors]
    float* fold_s = reinterpret_cast<float*>(xfloors + 2 * kXFloors);    // [3][kPairWaves]
    int* fold_i = reinterpret_cast<int*>(fold_s + 3 * kPairWaves);       // [3][kPairWaves]
    int* counts = fold_i + 3 * kPairWaves;                               // [kPairWaves]
    float* slot_s0 = reinterpret_cast<float*>(counts + kPairWaves);      // [2]
    int* slot1_row = reinterpret_cast<int*>(slot_s0 + 2);
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int slot = wave / kSlotWaves, sw = wave % kSlotWaves, st = tid % kSlotThreads;
    const int b = blockIdx.x;
    // Slot 1's temperature loads go out before any logit load of the block
    // (the barrier orders the issue only: no memory fence, nothing waits).
    DealTemps deal;
    if (slot == 1) deal = load_deal(temps, batch, b, lane);
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    if (slot == 1) {  // opaque after the barrier: the wait for the loads stays on slot 1's side of it
#pragma unroll
        for (int c = 0; c < kDealLoads; ++c) __asm__ volatile("" : "+v"(deal.t[c]));
        __asm__ volatile("" : "+v"(deal.own));
    }
    const int r = slot == 0 ? b : __builtin_amdgcn_readfirstlane(partner_row(temps, deal, batch, b, lane));
    const int chunks = vocab / 8;
    const int first = slot * kSlotThreads + st;
    const uint16_t* row = logits + int64_t(r) * vocab;
    uint4 w[C];
#pragma unroll
    for (int k = 0; k < C; ++k) w[k] = nvr::load_stream(row + 8 * int64_t(min(k * stride + first, chunks - 1)));
    const float temperature = temps[r];
    const uint64_t seed = seeds[r];
    const bool gumbel = temperature > 0.0f;
    for (int k = tid; k < kFloorSteps; k += kPairThreads) floors[k] = noise_floor(k);
    if (tid == kSlotThreads) *slot1_row = r;

    // Phase 1: lane maxima; each slot's greedy maximum. Phase 2 (Gumbel
    // halves): every lane scores its maximum's token exactly; the best of
    // those real scores is the half's s0 (folded after the same barrier, while
    // an early slot waits for the other).
    const Best lb = lane_best<C>(w, stride, first, chunks);
    {
        const Best wb = wave_argmax(lb);
        if (lane == 0) { fold_s[wave] = wb.score; fold_i[wave] = wb.index; }
        Best own{-__builtin_inff(), nvr::kNoIndex};
        if (gumbel && lb.index != nvr::kNoIndex)
            own = Best{nvr::gumbel_score(lb.score, temperature, seed, uint32_t(lb.index)), lb.index};
        own = wave_argmax(own);
        if (lane == 0) { fold_s[kPairWaves + wave] = own.score; fold_i[kPairWaves + wave] = own.index; }
    }
    __syncthreads();
    const int r1 = *slot1_row;
    const bool whole = r1 == b;  // both halves of row b in this block
    const Best top = whole ? fold_waves(fold_s, fold_i, 0, kPairWaves)
                           : fold_waves(fold_s, fold_i, slot * kSlotWaves, kSlotWaves);
    if (!gumbel && whole) {  // a whole greedy row: done (every wave of the block leaves here)
        if (tid == 0) out[r] = top.index == nvr::kNoIndex ? 0 : top.index;
        return;
    }

    // s0 of the half (or of the row); a split Gumbel row trades its halves'.
    const Best seeded = whole ? fold_waves(fold_s + kPairWaves, fold_i + kPairWaves, 0, kPairWaves)
                              : fold_waves(fold_s + kPairWaves, fold_i + kPairWaves, slot * kSlotWaves, kSlotWaves);
    if (gumbel && !whole && st == 0) slot_s0[slot] = exchange_s0(state, r, slot, seeded.score);
    if (!whole) __syncthreads();  // a whole row exchanges nothing here
    // A greedy half deposits its maximum here, while the Gumbel half compacts.
    // Before the barrier its round trip would hold that compaction back, and
    // so would any vector load in flight there: the memory counter retires in
    // issue order, so the next wait for one waits for all of them.
    if (!gumbel && !whole && st == 0) deposit(state, r, top, out);

    // The Gumbel half whose queues this wave compacts or helps score: its own
    // slot, or (a greedy half split from a Gumbel row's) the other slot.
    const int gslot = gumbel || whole ? slot : 1 - slot;
    const bool helps = !gumbel && !whole && (temps[slot == 0 ? r1 : b] > 0.0f);
    const int grow = gslot == 0 ? b : r1;
    const float gt = gumbel ? temperature : temps[grow];
    const uint64_t gseed = gumbel ? seed : seeds[grow];
    const float s0 = whole ? seeded.score : slot_s0[gslot];
    const float inv_t = 1.0f / gt;
    const bool on = __builtin_fabsf(s0) < __builtin_inff() && inv_t < __builtin_inff();
    const float lx = candidate_floor(s0, inv_t, gt, on);
    const Pruner p{s0, inv_t, gt, gseed, on, floors};
    // Tabulated hash floors over the candidate values [lx, the half's maximum].
    const float hmax = whole ? top.score : fold_waves(fold_s, fold_i, gslot * kSlotWaves, kSlotWaves).score;
    const int lxb = int(__float_as_uint(lx) >> 16);
    const int span = (on & (lx > 0.0f) & (hmax >= lx)) ? int(__float_as_uint(hmax) >> 16) - lxb + 1 : 0;
    const bool tab = span > 0 && span <= kXFloors;
    uint32_t* gxf = xfloors + (whole ? 0 : gslot) * kXFloors;
    if (gumbel && tab) {
        // one table per Gumbel half; a whole row's slots share slot 0's
        if (!whole || slot == 0)
            for (int j = st; j < span; j += kSlotThreads) gxf[j] = hash_floor(p, nvr::bf16_to_f32(uint16_t(lxb + j)));
    }

    // Phase 3: window 0 of each Gumbel wave's compaction.
    uint32_t* queue = lds + wave * kQ;
    const uint32_t lane_code = uint32_t(lane) << 3;
    int n = 0;
    if (gumbel) n = compact_window_dense<C>(w, lx, queue, 0, kCap, lane_code);
    // The helper waves read this queue after the barrier: wait for the
    // compaction's stores, which the compiler's own waits do not count.
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane == 0) counts[wave] = n;
    __syncthreads();

    // Phase 4: scoring. A Gumbel half whose every queue fits scores the front
    // of each queue itself and leaves the back to its helper; otherwise each
    // wave works through its own windows.
    bool fits = true;
#pragma unroll
    for (int i = 0; i < kSlotWaves; ++i) fits &= counts[gslot * kSlotWaves + i] <= kCap;
    Best best = gumbel ? seeded : Best{-__builtin_inff(), nvr::kNoIndex};
    if (gumbel) {
        const int base = slot * kSlotThreads + sw * kWave;
        if (fits) {
            const int end = whole ? n : helper_split(n);
            if (tab) score_queue<true>(queue, 0, end, lane, base, stride, p, gxf, lxb, best);
            else score_queue<false>(queue, 0, end, lane, base, stride, p, gxf, lxb, best);
        } else if (n > 2 * kCap) {
            score_in_place(row, first, stride, chunks, lx, p, best);
        } else {
            for (int window = 0;; window += kCap) {
                const int m = window == 0 ? n : compact_window_dense<C>(w, lx, queue, window, kCap, lane_code);
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (tab) score_queue<true>(queue, 0, min(m, kCap), lane, base, stride, p, gxf, lxb, best);
                else score_queue<false>(queue, 0, min(m, kCap), lane, base, stride, p, gxf, lxb, best);
                if (m <= kCap) break;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
        }
    } else if (helps && fits) {
        const int gw = gslot * kSlotWaves + sw;
        const int gn = counts[gw];
        const int base = gslot * kSlotThreads + sw * kWave;
        if (tab) score_queue<true>(lds + gw * kQ, helper_split(gn), gn, lane, base, stride, p, gxf, lxb, best);
        else score_queue<false>(lds + gw * kQ, helper_split(gn), gn, lane, base, stride, p, gxf, lxb, best);
    }

    // Phase 5: the Gumbel row's best over every wave that scored for it.
    best = wave_argmax(best);
    if (lane == 0) { fold_s[2 * kPairWaves + wave] = best.score; fold_i[2 * kPairWaves + wave] = best.index; }
    __syncthreads();
    if (sw == 0 && gumbel && (!whole || slot == 0)) {
        // The first wave of each Gumbel slot: its slot's row is r (b, or r1)
        // and `gumbel` its kind, both known since the start (no load here, on
        // the launch's last step).
        const Best fin = fold_waves(fold_s + 2 * kPairWaves, fold_i + 2 * kPairWaves, 0, kPairWaves);
        if (st == 0) {
            if (whole) out[b] = fin.index == nvr::kNoIndex ? 0 : fin.index;
            else deposit(state, r, fin, out);
        }
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
    // Two partials of every lane in flight before either is compared: one
    // memory round trip per 128 partials (a 151936-token row has 75). The
    // fold is a maximum under a total order, so its order is free.
    for (int p0 = 0; p0 < parts; p0 += 2 * kWave) {
        const int p = p0 + int(threadIdx.x), q = p + kWave;
        const float s0 = p < parts ? partial_scores[base + p] : -__builtin_inff();
        const int i0 = p < parts ? partial_ids[base + p] : nvr::kNoIndex;
        const float s1 = q < parts ? partial_scores[base + q] : -__builtin_inff();
        const int i1 = q < parts ? partial_ids[base + q] : nvr::kNoIndex;
        consider(b, s0, i0);
        consider(b, s1, i1);
    }
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

template <int TPB>
int launch_resident(nv_context* c, const uint16_t* logits, const float* temps, const uint64_t* seeds, int* out,
                    float* partial_scores, int* partial_ids, int batch, int vocab, int chunks_per_lane) {
    constexpr int parts = 1024 / TPB;
    const dim3 grid(unsigned(batch * parts)), block(TPB);
    const size_t lds = ResGeometry<TPB>::kLdsBytes;
    switch (chunks_per_lane) {
    case 4: hipLaunchKernelGGL((sample_resident<4, TPB>), grid, block, lds, c->stream, logits, temps, seeds, out, partial_scores, partial_ids, vocab, parts, parts); break;
    case 8: hipLaunchKernelGGL((sample_resident<8, TPB>), grid, block, lds, c->stream, logits, temps, seeds, out, partial_scores, partial_ids, vocab, parts, parts); break;
    case 12: hipLaunchKernelGGL((sample_resident<12, TPB>), grid, block, lds, c->stream, logits, temps, seeds, out, partial_scores, partial_ids, vocab, parts, parts); break;
    case 16: hipLaunchKernelGGL((sample_resident<16, TPB>), grid, block, lds, c->stream, logits, temps, seeds, out, partial_scores, partial_ids, vocab, parts, parts); break;
    default: hipLaunchKernelGGL((sample_resident<20, TPB>), grid, block, lds, c->stream, logits, temps, seeds, out, partial_scores, partial_ids, vocab, parts, parts); break;
    }
    if (parts == 1) return nvr::launch_status();
    NVR_HIP(hipGetLastError());
    hipLaunchKernelGGL(sample_combine, dim3(unsigned(batch)), dim3(64), 0, c->stream, partial_scores, partial_ids, out,
                       parts);
    return nvr::launch_status();
}

int launch_paired(nv_context* c, const uint16_t* logits, const float* temps, const uint64_t* seeds, int* out,
                  int batch, int vocab, int chunks_per_lane) {
    const dim3 grid = dim3(unsigned(batch)), block = dim3(unsigned(kPairThreads));
    auto* state = static_cast<uint64_t*>(c->pair_state);
    switch (chunks_per_lane) {
    case 4: hipLaunchKernelGGL(sample_paired<4>, grid, block, kPairLdsBytes, c->stream, logits, temps, seeds, out, state, vocab, batch); break;
    case 8: hipLaunchKernelGGL(sample_paired<8>, grid, block, kPairLdsBytes, c->stream, logits, temps, seeds, out, state, vocab, batch); break;
    case 12: hipLaunchKernelGGL(sample_paired<12>, grid, block, kPairLdsBytes, c->stream, logits, temps, seeds, out, state, vocab, batch); break;
    case 16: hipLaunchKernelGGL(sample_paired<16>, grid, block, kPairLdsBytes, c->stream, logits, temps, seeds, out, state, vocab, batch); break;
    default: hipLaunchKernelGGL(sample_paired<20>, grid, block, kPairLdsBytes, c->stream, logits, temps, seeds, out, state, vocab, batch); break;
    }
    return nvr::launch_status();
}

int launch_parallel(nv_context* c, const void* logits, const void* temps, const void* seeds, void* out,
                    void* partial_scores, void* partial_ids, int batch, int vocab) {
    const int64_t ref_parts = (int64_t(vocab) + kRefPartition - 1) / kRefPartition;
    if (ref_parts <= 1 || int64_t(batch) * ref_parts > 0x7fffffff)
        return launch_serial(c, logits, temps, seeds, out, batch, vocab);
    auto l16 = static_cast<const uint16_t*>(logits);
    auto t = static_cast<const float*>(temps);
    auto s = static_cast<const uint64_t*>(seeds);
    auto ps = static_cast<float*>(partial_scores);
    auto pi = static_cast<int*>(partial_ids);
    // One row per CU: worth it once every CU has a row (measured at 256 rows
    // of 151936 on MI355X: greedy 16 vs 23 us, T = 0.6 39 vs 51 us, half and
    // half 38 vs 40 us, T = 1 76 vs 86 us; with 192 rows the partitions win
    // mixed and T = 1 batches).
    const int min_rows = c->cu_count > 0 ? c->cu_count : 256;
    const int64_t lane_chunks = (int64_t(vocab) / 8 + 1023) / 1024;  // per lane of the row's 1024 threads
    if (batch >= min_rows && vector_rows(logits, vocab) && lane_chunks <= kResMaxChunks) {
        if (batch <= kPairRows && c->pair_state)
            return launch_paired(c, l16, t, s, static_cast<int*>(out), batch, vocab, int((lane_chunks + 3) / 4 * 4));
        return launch_resident<kResThreads>(c, l16, t, s, static_cast<int*>(out), ps, pi, batch, vocab,
                                            int((lane_chunks + 3) / 4 * 4));
    }
    int parts;
    if (vector_rows(logits, vocab) && batch <= kFullScoreRows) {
        parts = int(ref_parts);  // 2048-token partitions: the most blocks the scratch allows
        hipLaunchKernelGGL(sample_partitions_full<1>, dim3(unsigned(batch * parts)), dim3(256), 0, c->stream, l16, t, s,
                           ps, pi, vocab, parts);
    } else if (vector_rows(logits, vocab)) {
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

// Partials of nv_sample_parallel_static, in place of caller scratch: scores
// (f32) in words [0, kStaticPartials), ids (i32) in [kStaticPartials,
// 2 * kStaticPartials). 1 MiB, held by every device the library runs on
// until the process ends. Host code must not pass `scratch` itself to a
// kernel (in host code the name is a stand-in, not a device address): it uses
// the address hipGetSymbolAddress gives for the current device, kept in the
// context by bind_static_partials.
constexpr int kStaticPartials = 1 << 17;
static __device__ __align__(256) uint32_t scratch[2 * kStaticPartials];

}  // namespace

namespace nvr {

int bind_static_partials(nv_context* c) {
    void* ptr = nullptr;
    NVR_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    c->static_partials = ptr;
    return 0;
}

int create_pair_state(nv_context* c) {
    void* ptr = nullptr;
    const size_t bytes = sizeof(uint64_t) * 2 * size_t(kPairRows);
    NVR_HIP(hipMalloc(&ptr, bytes));
    c->pair_state = ptr;
    NVR_HIP(hipMemset(ptr, 0, bytes));
    return 0;
}

}  // namespace nvr

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
    return launch_parallel(c, logits, temps, seeds, out, partial_scores, partial_ids, batch, vocab);
}

int nv_sample_parallel_static(nv_context* c, const void* logits, const void* temps, const void* seeds, void* out,
                              int batch, int vocab) {
    NVR_ACTIVATE(c);
    if (batch <= 0 || vocab <= 0) return nvr::fail(-2, "sample_parallel_static: dimensions must be positive");
    const int64_t partials = int64_t(batch) * ((int64_t(vocab) + kRefPartition - 1) / kRefPartition);
    if (partials > kStaticPartials)
        return nvr::fail(-2,
                         "sample_parallel_static: batch %d x ceil(vocab %d / 2048) = %lld partials exceed the "
                         "static scratch of %d; use nv_sample_parallel with caller scratch",
                         batch, vocab, (long long)partials, kStaticPartials);
    if (!c->static_partials) return nvr::fail(-2, "sample_parallel_static: static scratch not bound");
    auto* words = static_cast<uint32_t*>(c->static_partials);
    return launch_parallel(c, logits, temps, seeds, out, words, words + kStaticPartials, batch, vocab);
}

}  // extern "C"
