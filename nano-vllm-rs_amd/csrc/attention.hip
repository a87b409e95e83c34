// Paged causal GQA attention (nv_attention).
//
// Semantics: kernels/kernels.cu:226-270 (attention_kernel) and :289-346
// (attention_ordered_kernel) of nano-vllm-rs, which the reference keeps
// bit-identical (:286-287). Per (row, q head h), kv head = h / (qh / kvh):
//   - a row whose seq lies outside [0, batch) or whose context = pos + 1 lies
//     outside [1, max_context] or above stride * bs is all zeros;
//   - token t < context reads physical block table[seq * stride + t / bs]; a
//     block outside [0, blocks) scores -inf and adds no V term;
//   - score_t = tree(chain_0 .. chain_31) * (1 / sqrt(dim)): chain c is the
//     fma chain of q[d] * k_t[d] over d = c, c + 32, ... < dim starting from 0,
//     and tree is the 32-lane shuffle-down sum (offsets 16, 8, 4, 2, 1);
//   - m = max_t score_t; p_t = exp(score_t - m) if m is finite, else 0;
//   - den = the reference's 256-thread block sum: thread i adds p_i, p_{i+256},
//     ... in order; each 32-thread warp folds by shuffle-down; the 8 warp
//     sums fold as ((w0+w4)+(w2+w6))+((w1+w5)+(w3+w7));
//   - out[h, d] = bf16(den > 0 ? value_d / den : 0), value_d = the fma chain of
//     p_t * v_t[d] over tokens in increasing order, from 0.
// Every one of those rounding steps is kept, so results equal the host
// oracle's bit for bit; exp is nvr_expf, and 1 / sqrt(dim) is correctly
// rounded (the reference's rsqrtf and expf have no public bit-exact
// definition).
//
// Layout (head dims 32, 64, 128, 256 with 16-byte aligned operands): one
// 256-thread block per (row, group of HPB q heads sharing a kv head), so a
// row's K and V are read once for both heads of a GQA pair. The row's block
// table is copied to LDS first, so cache addresses never wait on global loads.
// Every K/V load instruction reads whole token rows (16 lanes per 256-byte
// row): on MI355X that streams at ~6.6 TB/s, against ~5.2 TB/s when each
// instruction touches half lines of 16 rows.
//   1. Scores: four lanes per token. Lane a of a quad owns chains 8a .. 8a+7
//      (pieces 4j + a of the row, j < dim/32), reached by staging each wave's
//      16 rows in its own LDS rows (no block barrier). The first two tree
//      levels (offsets 16 and 8) pair lanes a ^ 2 and a ^ 1 of the quad (DPP
//      adds); the last three run inside the lane. Three steps of K loads stay
//      in flight behind the one being scored. Scores go to LDS.
//   2. Block max, exp in place, the block sum in the reference's order.
//   3. Values: 16 KB V tiles in LDS, one block barrier per tile. Thread
//      (g, d) runs its fma chain over the tile's tokens in order. Launches of
//      at most one block per CU whose tiles lie in whole blocks (kStreamed)
//      stream each tile from memory straight into one of four LDS slots
//      (global_load_lds), three tiles ahead, and skip a tile of an invalid
//      block. Otherwise tiles alternate between two LDS slots with two more
//      in flight in registers; tokens of an invalid block are staged as -0.0
//      with p = +0, which leaves every chain value (including -0) unchanged,
//      exactly as skipping them does.
// Other head dims, unaligned operands and caches of more than 2^31 token rows
// use a direct kernel with the same arithmetic.
#include "../../include/nano_hip.h"
#include "nvr_device.h"
#include "nvr_internal.h"

namespace {

using nvr::kWave;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxContext = 4096;  // src/gpu.rs:848-852
constexpr uint32_t kNegZeroPair = 0x80008000u;

// 32-lane shuffle-down fold of the reference's warp_sum, valid in lanes 0 and
// 32 of the wave (the reference's warps are the two 32-lane halves).
__device__ __forceinline__ float half_wave_sum(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += nvr::xor_lane(v, o);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, nvr::xor_lane(v, o));
    return v;
}

// The reference's final fold of its 8 warp sums (zeros in lanes 8..31).
__device__ __forceinline__ float fold8(const float* w) {
    return ((w[0] + w[4]) + (w[2] + w[6])) + ((w[1] + w[5]) + (w[3] + w[7]));
}

// Block barrier once this wave's vector memory operations have dropped to N
// outstanding and its LDS operations to none.
template <int N>
__device__ __forceinline__ void stream_barrier() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Byte address in LDS of a pointer into shared memory.
template <typename T>
__device__ __forceinline__ uint32_t lds_address(const T* p) {
    using Lds = __attribute__((address_space(3))) const T*;
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((Lds)p));
}

// Block barrier over LDS only: unlike __syncthreads it does not wait for
// outstanding vector memory operations (the streamed V tiles).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One whole 64-token V tile of the value chain at head dim 128, in inline
// asm: acc = fma(p_t, v_t[d], acc) for the tile's tokens in order. va is the
// LDS address of this lane's dimension in token 0 of the tile (token rows of
// 256 bytes); pa the address of p_{t0 + lane % 16}. V elements are read with
// ds_read_u16_d16_hi into registers whose low halves are zero, so each
// register already holds the element as an f32 (no shift); the
// probabilities are read once per 16 tokens, lane j of each 16-lane row
// holding p_{16k + j}, and reach the fma through DPP row_newbcast:j (no
// broadcast read per token). Groups of 8 tokens alternate between two
// register banks, the next group's reads issued before the current group's
// fmas. z holds the 16 zero-low registers (kept by the caller; only the high
// halves are ever written). Measured alone (one 64-token tile in LDS, 128
// chains per block): 11.2 against 15.5 clock ticks per token for the compiled
// chain (u16 read, shift, fma, broadcast reads).
#define NVR_RD(bank, i, g) "ds_read_u16_d16_hi %[" #bank #i "], %[va] offset:(8*" #g "+" #i ")*256\n\t"
#define NVR_RD8(bank, g)                                                                                          \
    NVR_RD(bank, 0, g) NVR_RD(bank, 1, g) NVR_RD(bank, 2, g) NVR_RD(bank, 3, g) NVR_RD(bank, 4, g)              \
        NVR_RD(bank, 5, g) NVR_RD(bank, 6, g) NVR_RD(bank, 7, g)
#define NVR_P(k) "ds_read_b32 %[p" #k "], %[pa] offset:" #k "*64\n\t"
#define NVR_FMA(bank, i, k, j) \
    "v_fmac_f32_dpp %[acc], %[p" #k "], %[" #bank #i "] row_newbcast:" #j " row_mask:0xf bank_mask:0xf\n\t"
#define NVR_FMA8(bank, k, j0)                                                                                     \
    NVR_FMA(bank, 0, k, j0 + 0) NVR_FMA(bank, 1, k, j0 + 1) NVR_FMA(bank, 2, k, j0 + 2)                          \
        NVR_FMA(bank, 3, k, j0 + 3) NVR_FMA(bank, 4, k, j0 + 4) NVR_FMA(bank, 5, k, j0 + 5)                      \
            NVR_FMA(bank, 6, k, j0 + 6) NVR_FMA(bank, 7, k, j0 + 7)
__device__ __forceinline__ void value_tile_d128(float& acc, uint32_t va, uint32_t pa, uint32_t (&z)[16]) {
    float p0, p1, p2, p3;
    asm volatile(
        NVR_P(0) NVR_RD8(a, 0)
        NVR_RD8(b, 1) "s_waitcnt lgkmcnt(8)\n\t" NVR_FMA8(a, 0, 0)           // tokens 0-7
        NVR_P(1) NVR_RD8(a, 2) "s_waitcnt lgkmcnt(9)\n\t" NVR_FMA8(b, 0, 8)  // 8-15
        NVR_RD8(b, 3) "s_waitcnt lgkmcnt(8)\n\t" NVR_FMA8(a, 1, 0)           // 16-23
        NVR_P(2) NVR_RD8(a, 4) "s_waitcnt lgkmcnt(9)\n\t" NVR_FMA8(b, 1, 8)  // 24-31
        NVR_RD8(b, 5) "s_waitcnt lgkmcnt(8)\n\t" NVR_FMA8(a, 2, 0)           // 32-39
        NVR_P(3) NVR_RD8(a, 6) "s_waitcnt lgkmcnt(9)\n\t" NVR_FMA8(b, 2, 8)  // 40-47
        NVR_RD8(b, 7) "s_waitcnt lgkmcnt(8)\n\t" NVR_FMA8(a, 3, 0)           // 48-55
        "s_waitcnt lgkmcnt(0)\n\t" NVR_FMA8(b, 3, 8)                         // 56-63
        : [acc] "+v"(acc), [a0] "+v"(z[0]), [a1] "+v"(z[1]), [a2] "+v"(z[2]), [a3] "+v"(z[3]), [a4] "+v"(z[4]),
          [a5] "+v"(z[5]), [a6] "+v"(z[6]), [a7] "+v"(z[7]), [b0] "+v"(z[8]), [b1] "+v"(z[9]), [b2] "+v"(z[10]),
          [b3] "+v"(z[11]), [b4] "+v"(z[12]), [b5] "+v"(z[13]), [b6] "+v"(z[14]), [b7] "+v"(z[15]),
          [p0] "=&v"(p0), [p1] "=&v"(p1), [p2] "=&v"(p2), [p3] "=&v"(p3)
        : [va] "v"(va), [pa] "v"(pa)
        : "memory");
}
#undef NVR_RD
#undef NVR_RD8
#undef NVR_P
#undef NVR_FMA
#undef NVR_FMA8

// Physical token index of a table entry and logical token, or -1.
__device__ __forceinline__ int64_t phys_token(int entry, int t, int bs, int blocks) {
    return entry >= 0 && entry < blocks ? int64_t(entry) * bs + t % bs : int64_t(-1);
}

// Compile-time geometry of attention_ordered. OCC trades pipeline depth for
// occupancy (see launch_ordered): 32-token V tiles instead of 64 and three K
// buffers instead of four.
template <int DIM, int HPB, bool OCC>
struct OrderedLayout {
    static_assert(DIM % 32 == 0 && DIM <= 256 && HPB * DIM <= kThreads, "shape");
    static constexpr int P = DIM / 32;                    // elements per dot chain
    static constexpr int kPieces = DIM / 8;               // 16-byte pieces per K/V row
    static constexpr int kRowsPerLoad = kWave / kPieces;  // whole rows per wave load instruction
    static constexpr int kQuads = kWave / 4;              // tokens per wave per phase-1 step
    static constexpr int kStep = kQuads * kWaves;         // tokens per block step
    static constexpr int kKLoads = kQuads / kRowsPerLoad; // load instructions per wave step (= P)
    static constexpr int kKRow = DIM * 2 + 64;            // staged K row bytes; the pad makes quad reads conflict-free
    static constexpr int kVTile = (OCC ? 4096 : 8192) / DIM;  // tokens per V tile (8 or 16 KB)
    static constexpr int kVLoads = kVTile * kPieces / kThreads;  // V loads per thread per tile (2 or 4)
    static constexpr int kKStage = kWaves * kQuads * kKRow;
    static constexpr int kVStage = 2 * kVTile * DIM * 2;
    static constexpr int kStageBytes = kKStage > kVStage ? kKStage : kVStage;
    static constexpr int kSlots = 4;  // kStreamed's V slots (they reuse the K rows' LDS)
    static constexpr int kSlotBytes = kVTile * DIM * 2;
    static constexpr int kStreamStage = kKStage > kSlots * kSlotBytes ? kKStage : kSlots * kSlotBytes;
    static_assert(kKLoads * kRowsPerLoad == kQuads && kVLoads * kThreads == kVTile * kPieces, "tiles");
};

// How a logical token finds its physical row: kAnyBs divides by the block
// size; kPow2 shifts (bs a power of two); kAligned (bs a power of two holding
// whole K steps and V tiles) looks the block entry up once per step or tile.
// kStreamed is kAligned with the V tiles streamed into LDS slots.
constexpr int kAnyBs = 0, kPow2 = 1, kAligned = 2, kStreamed = 3;

// The q/k norm + RoPE + KV-slot write that FUSED blocks run first (the
// decode-batch entry point); unused otherwise.
struct QkvRopeArgs {
    const uint16_t* qkv;   // [rows, qh + 2 kvh, 128]
    const uint16_t* qw;    // q norm weight [128]
    const uint16_t* kw;    // k norm weight [128]
    const int* slots;      // [rows]
    const float* rope;     // [max_positions, 128]: cos | sin
    int max_positions;
    float eps;
};

template <int DIM, int HPB, int TABLE, bool OCC, bool FUSED>
__global__ __launch_bounds__(kThreads) void attention_ordered(
    const uint16_t* __restrict__ q, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
    const int* __restrict__ positions, const int* __restrict__ seqs, const int* __restrict__ tables,
    uint16_t* __restrict__ out, int qh, int kvh, int bs, int bs_shift, int blocks, int stride, int batch,
    int max_context, int score_stride, QkvRopeArgs fa) {
    using L = OrderedLayout<DIM, HPB, OCC>;
    constexpr int P = L::P, kPieces = L::kPieces, kQuads = L::kQuads, kStep = L::kStep;
    constexpr int kRowsPerLoad = L::kRowsPerLoad, kKLoads = L::kKLoads, kKRow = L::kKRow;
    constexpr int kVTile = L::kVTile, kVLoads = L::kVLoads;

    extern __shared__ __align__(16) unsigned char smem[];
    float* probs = reinterpret_cast<float*>(smem);                          // [HPB][score_stride]
    unsigned char* stage = smem + sizeof(float) * HPB * score_stride;       // K rows (phase 1) / V slots (phase 3)
    int* ltable = reinterpret_cast<int*>(stage + L::kStageBytes);           // the row's block-table entries (kAnyBs, kPow2)
    __shared__ float red_max[HPB][kWaves];
    __shared__ float red_sum[HPB][2 * kWaves];

    const int row = blockIdx.x;
    const int h0 = blockIdx.y * HPB;
    const int kvhead = h0 / (qh / kvh);
    const int seq = seqs[row];
    const int64_t context64 = int64_t(positions[row]) + 1;
    uint16_t* orow = out + (int64_t(row) * qh + h0) * DIM;

    // ---- 0. (FUSED) this row's q/k norm + RoPE and its KV-slot write ----
    // Wave 0, one 16-lane group per head in the layout of qkv_rope's d128
    // kernel (lane m holds elements 8m..8m+7) and the same arithmetic
    // (nvr::norm_rotate_d128): groups g < HPB normalise and rotate q head
    // h0 + g into LDS; group HPB does the kv head's K and writes it to the
    // cache slot; group HPB + 1 copies its V. With one q head per block the
    // two blocks of a kv head write the same bytes. The barrier orders those
    // stores before this block's K/V loads. It runs for every row, as the
    // separate q/k-norm + RoPE launch would, also those the attention below
    // then skips.
    __shared__ __align__(16) uint16_t qs[FUSED ? HPB : 1][FUSED ? DIM : 8];
    if constexpr (FUSED) {
        static_assert(DIM == 128, "the fused q/k norm + RoPE runs at head dim 128");
        if (threadIdx.x < kWave) {
            const int grp = (threadIdx.x >> 4) & 3, m = threadIdx.x & 15;
            const int heads = qh + 2 * kvh;
            const bool qgrp = grp < HPB, kgrp = grp == HPB, vgrp = grp == HPB + 1;
            const int hsel = qgrp ? h0 + grp : kgrp ? qh + kvhead : qh + kvh + kvhead;  // idle group: a v head
            const uint4 xw = nvr::load_stream(fa.qkv + (int64_t(row) * heads + hsel) * DIM + 8 * m);
            const uint4 wv = *reinterpret_cast<const uint4*>((qgrp ? fa.qw : fa.kw) + 8 * m);
            const int pos = positions[row];
            const int slot = fa.slots[row];
            const bool valid_slot = slot >= 0 && int64_t(slot) < int64_t(bs) * blocks;
            const int pair0 = 8 * (m & 7);
            float cs[8], sn[8], wf[8];
            if (pos >= 0 && pos < fa.max_positions) {
                const float4* t = reinterpret_cast<const float4*>(fa.rope + int64_t(pos) * DIM + pair0);
                const float4 c0 = t[0], c1 = t[1], s0 = t[DIM / 8], s1 = t[DIM / 8 + 1];
                cs[0] = c0.x; cs[1] = c0.y; cs[2] = c0.z; cs[3] = c0.w;
                cs[4] = c1.x; cs[5] = c1.y; cs[6] = c1.z; cs[7] = c1.w;
                sn[0] = s0.x; sn[1] = s0.y; sn[2] = s0.z; sn[3] = s0.w;
                sn[4] = s1.x; sn[5] = s1.y; sn[6] = s1.z; sn[7] = s1.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) { cs[i] = 1.0f; sn[i] = 0.0f; }
            }
            if (m < 8) {
#pragma unroll
                for (int i = 0; i < 8; ++i) sn[i] = -sn[i];
            }
            nvr::unpack8(wv, wf);
            const uint4 rot = nvr::norm_rotate_d128(xw, wf, cs, sn, fa.eps);
            if (qgrp) *reinterpret_cast<uint4*>(&qs[qgrp ? grp : 0][8 * m]) = rot;
            if (kgrp & valid_slot) nvr::store_stream(kc + (int64_t(slot) * kvh + kvhead) * DIM + 8 * m, rot);
            if (vgrp & valid_slot) nvr::store_stream(vc + (int64_t(slot) * kvh + kvhead) * DIM + 8 * m, xw);
        }
        __syncthreads();
    }

    if (seq < 0 || seq >= batch || context64 < 1 || context64 > max_context ||
        context64 > int64_t(stride) * bs) {
        for (int i = threadIdx.x; i < HPB * DIM; i += kThreads) orow[i] = 0;
        return;
    }
    const int ctx = int(context64);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int64_t token_stride = int64_t(kvh) * DIM;  // elements between consecutive tokens of a block
    // The row's block-table entries: with kAligned (at most 64 entries) lane i
    // of every wave holds entry i, read back with readlane; otherwise they go
    // to LDS once. Either way K/V addresses never wait on a global load.
    const int* table = tables + int64_t(seq) * stride;
    const int nent = (ctx - 1) / bs + 1;
    int lane_entry = -1;
    if constexpr (TABLE >= kAligned) {
        if (lane < nent) lane_entry = table[lane];
    } else {
        for (int i = threadIdx.x; i < nent; i += kThreads) ltable[i] = table[i];
        __syncthreads();
    }
    // Physical token row (block * bs + offset) of logical token t < ctx, or -1
    // for an invalid block. The host guarantees blocks * bs fits in int32.
    constexpr bool kShift = TABLE != kAnyBs;
    auto phys = [&](int t) -> int {
        const int lb = kShift ? t >> bs_shift : t / bs;
        const int off = kShift ? t & (bs - 1) : t - lb * bs;
        const int e = ltable[lb];
        return e >= 0 && e < blocks ? e * bs + off : -1;
    };
    // kAligned: the block entry of the aligned group (a K step or a V tile)
    // that starts at logical token t0 (clamped into the context; uniform),
    // whether it is a valid block, and the address of the group's first token
    // row in `col`. A group past the context or in an invalid block reads the
    // first rows of physical block 0 instead: every load stays inside an
    // allocated block, its data is discarded, and all such reads share the
    // same lines (cache hits rather than HBM traffic).
    auto group_entry = [&](int t0) -> int {
        return __builtin_amdgcn_readlane(lane_entry, min(t0, ctx - 1) >> bs_shift);
    };
    auto entry_ok = [&](int e) { return e >= 0 && e < blocks; };
    auto group_base = [&](const uint16_t* col, int e, int t0) {
        return t0 < ctx && entry_ok(e) ? col + (int64_t(e) * bs + (t0 & (bs - 1))) * token_stride : col;
    };

    // ---- 1. scores ----
    // Loads read whole rows: load instruction k of a wave step gives lane l
    // 16-byte piece l % kPieces of token k * kRowsPerLoad + l / kPieces (full
    // 128-byte lines per instruction, which streams markedly faster than
    // partial lines). The wave stages its kQuads rows in its own LDS rows and
    // reads them back in the quad layout: lane (tq, a) of quad tq owns chains
    // 8a .. 8a+7, i.e. pieces 4j + a (j < P) of token tq.
    const int tq = lane >> 2, a = lane & 3;
    const int lrow = lane / kPieces, lpiece = lane % kPieces;
    // kStreamed: this lane's byte offsets, from a V tile's first row, of its
    // four 16-byte loads (phase 3). Computed here and made opaque so that they
    // stay in registers of their own: computed after the scores, they would
    // reuse the registers of the K loads still in flight past the last step,
    // and the compiler would make the V loads wait for those.
    uint32_t voff[4] = {};
    if constexpr (TABLE == kStreamed) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            voff[u] = uint32_t((((wave * 4 + u) * kRowsPerLoad + lrow) * int(token_stride) + 8 * lpiece) * 2);
            asm volatile("" : "+v"(voff[u]));
        }
    }
    unsigned char* krows = stage + wave * kQuads * kKRow;
    const uint16_t* kcol = kc + int64_t(kvhead) * DIM + 8 * lpiece;
    float qf[HPB][P][8];
#pragma unroll
    for (int g = 0; g < HPB; ++g)
#pragma unroll
        for (int j = 0; j < P; ++j)
            nvr::unpack8(FUSED ? *reinterpret_cast<const uint4*>(&qs[FUSED ? g : 0][FUSED ? 32 * j + 8 * a : 0])
                               : *reinterpret_cast<const uint4*>(q + (int64_t(row) * qh + h0 + g) * DIM + 32 * j + 8 * a),
                         qf[g][j]);
    const float kScale = 1.0f / sqrtf(float(DIM));
    float m[HPB];
#pragma unroll
    for (int g = 0; g < HPB; ++g) m[g] = -__builtin_inff();

    // Step s covers tokens [s * kStep, (s + 1) * kStep); wave w takes
    // s * kStep + w * kQuads + (0 .. kQuads - 1). Four K buffers in fixed roles
    // keep three steps of loads in flight behind the one being scored. Loads
    // are unconditional (a token past the context or in an invalid block reads
    // token 0 of block 0 and its dot is discarded), so no branch makes the
    // compiler drain the load queue.
    // kAligned: lane offsets of a step's rows from the step's first row.
    const int klane = (wave * kQuads + lrow) * int(token_stride);
    auto issue = [&](uint4 (&kb)[kKLoads], int s) {
        if constexpr (TABLE >= kAligned) {
            const uint16_t* base = group_base(kcol, group_entry(s * kStep), s * kStep);
#pragma unroll
            for (int k = 0; k < kKLoads; ++k)
                kb[k] = nvr::load_stream(base + klane + k * kRowsPerLoad * int(token_stride));
        } else {
#pragma unroll
            for (int k = 0; k < kKLoads; ++k) {
                const int t = s * kStep + wave * kQuads + k * kRowsPerLoad + lrow;
                const int ph = phys(min(t, ctx - 1));
                kb[k] = nvr::load_stream(kcol + int64_t(t < ctx && ph >= 0 ? ph : 0) * token_stride);
            }
        }
    };
    auto score = [&](const uint4 (&kb)[kKLoads], int s) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the previous step's reads are done
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int k = 0; k < kKLoads; ++k)
            *reinterpret_cast<uint4*>(krows + (k * kRowsPerLoad + lrow) * kKRow + 16 * lpiece) = kb[k];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float kf[P][8];
#pragma unroll
        for (int j = 0; j < P; ++j)
            nvr::unpack8(*reinterpret_cast<const uint4*>(krows + tq * kKRow + 16 * (4 * j + a)), kf[j]);
        const int t = s * kStep + wave * kQuads + tq;
        const bool live = t < ctx;
        const bool valid = live && (TABLE >= kAligned ? entry_ok(group_entry(s * kStep))
                                                      : phys(min(t, ctx - 1)) >= 0);
#pragma unroll
        for (int g = 0; g < HPB; ++g) {
            float acc[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = __builtin_fmaf(qf[g][0][i], kf[0][i], 0.0f);
#pragma unroll
            for (int j = 1; j < P; ++j)
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[i] = __builtin_fmaf(qf[g][j][i], kf[j][i], acc[i]);
            // Offset 16: chain c + 16 = 8 (a ^ 2) + i. Offset 8: chain c + 8 = 8 (a ^ 1) + i.
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] += nvr::dpp<nvr::kDppQuadXor2>(acc[i]);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] += nvr::dpp<nvr::kDppQuadXor1>(acc[i]);
            float dot = ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
            // Pin the tree before any branch: the compiler would otherwise sink it
            // under `valid`, where the DPP operands cannot be fused into their adds.
            __asm__ volatile("" : "+v"(dot));
            const float sc = valid ? dot * kScale : -__builtin_inff();
            m[g] = fmaxf(m[g], live ? sc : -__builtin_inff());
            if (live && a == 0) probs[g * score_stride + t] = sc;
        }
    };
    const int nsteps = (ctx + kStep - 1) / kStep;
    if constexpr (OCC) {  // three buffers: two steps in flight behind the one being scored
        uint4 kA[kKLoads], kB[kKLoads], kC[kKLoads];
        issue(kA, 0);
        issue(kB, 1);
        for (int s = 0; s < nsteps; s += 3) {
            issue(kC, s + 2);
            score(kA, s);
            issue(kA, s + 3);
            if (s + 1 < nsteps) score(kB, s + 1);
            issue(kB, s + 4);
            if (s + 2 < nsteps) score(kC, s + 2);
        }
    } else {
        uint4 kA[kKLoads], kB[kKLoads], kC[kKLoads], kD[kKLoads];
        issue(kA, 0);
        issue(kB, 1);
        issue(kC, 2);
        for (int s = 0; s < nsteps; s += 4) {
            issue(kD, s + 3);
            score(kA, s);
            issue(kA, s + 4);
            if (s + 1 < nsteps) score(kB, s + 1);
            issue(kB, s + 5);
            if (s + 2 < nsteps) score(kC, s + 2);
            issue(kC, s + 6);
            if (s + 3 < nsteps) score(kD, s + 3);
        }
    }

    // ---- V prefetch (see phase 3) ----
    // A V tile is kVTile whole token rows (8 or 16 KB): load u of thread tid covers
    // piece cc % kPieces of token cc / kPieces, cc = tid + 256 u. Loads are
    // unconditional; invalid tokens become -0.0 when staged, which with p = +0
    // leaves every chain value unchanged, exactly as skipping them does.
    const uint16_t* vcol = vc + int64_t(kvhead) * DIM;
    auto load_vtile = [&](uint4 (&r)[kVLoads], bool (&ok)[kVLoads], int t0) {
        if constexpr (TABLE >= kAligned) {
            const int e = group_entry(t0);
            const uint16_t* base = group_base(vcol, e, t0);
#pragma unroll
            for (int u = 0; u < kVLoads; ++u) {
                const int cc = int(threadIdx.x) + kThreads * u;
                ok[u] = entry_ok(e) && t0 + cc / kPieces < ctx;
                r[u] = nvr::load_stream(base + (cc / kPieces) * int(token_stride) + 8 * (cc % kPieces));
            }
        } else {
#pragma unroll
            for (int u = 0; u < kVLoads; ++u) {
                const int cc = int(threadIdx.x) + kThreads * u;
                const int t = t0 + cc / kPieces;
                const int ph = phys(min(t, ctx - 1));
                ok[u] = t < ctx && ph >= 0;
                r[u] = nvr::load_stream(vcol + int64_t(ok[u] ? ph : 0) * token_stride + 8 * (cc % kPieces));
            }
        }
    };
    bool okW[kVLoads], okX[kVLoads], okY[kVLoads];
    uint4 rW[kVLoads], rX[kVLoads], rY[kVLoads];
    if constexpr (TABLE != kStreamed) {
        load_vtile(rW, okW, 0);
        load_vtile(rX, okX, kVTile);
        load_vtile(rY, okY, 2 * kVTile);
    }
    // kStreamed: a tile goes from memory straight into its LDS slot. Load u
    // of wave w brings kRowsPerLoad whole token rows (1 KB): tokens
    // (4w + u) * kRowsPerLoad onwards, lane l landing at byte 16 l. The loads
    // are inline asm, so the compiler (which would make every later LDS read
    // wait for all of them) never sees them: stream_wait orders them. M0
    // holds the LDS address and is restored after each load. Every address
    // lies in an allocated block (group_base), and a tile is only issued when
    // it starts inside the context.
    const int ntiles = (ctx + kVTile - 1) / kVTile;
    const uint32_t stage_lds = lds_address(stage);
    auto stream_vtile = [&](int t0, int slot) {
        const uint16_t* base = group_base(vcol, group_entry(t0), t0);  // uniform: scalar base
        const uint32_t dst = __builtin_amdgcn_readfirstlane(stage_lds + slot * L::kSlotBytes + wave * 4096);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            uint32_t saved;
            asm volatile(
                "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\t"
                "s_mov_b32 m0, %0"
                : "=&s"(saved)
                : "v"(voff[u]), "s"(base), "s"(dst + u * 1024)
                : "memory");
        }
    };
    static_assert(TABLE != kStreamed || 4 * kWaves * 1024 == L::kSlotBytes, "a tile is four 1 KB loads per wave");
    // Block barrier once every wave's loads of the tile to be consumed have
    // landed, `ahead` tiles (four loads each) having been issued after it.
    auto stream_wait = [&](int ahead) {
        static_assert(L::kSlots == 4, "up to two tiles ahead");
        if (ahead >= 2) stream_barrier<8>();
        else if (ahead == 1) stream_barrier<4>();
        else stream_barrier<0>();
    };

    // ---- 2. max, exp, block sum ----
#pragma unroll
    for (int g = 0; g < HPB; ++g) {
        m[g] = wave_max(m[g]);
        if (lane == 0) red_max[g][wave] = m[g];
    }
    __syncthreads();
    if constexpr (TABLE == kStreamed) {  // every wave is past its scores: the K rows' LDS is free
        for (int i = 0; i < L::kSlots - 1 && i < ntiles; ++i) stream_vtile(i * kVTile, i);
    }
    float den[HPB];
#pragma unroll
    for (int g = 0; g < HPB; ++g) {
        const float mg = fmaxf(fmaxf(red_max[g][0], red_max[g][1]), fmaxf(red_max[g][2], red_max[g][3]));
        const bool finite = __builtin_isfinite(mg);
        float sum = 0.0f;
        for (int t = threadIdx.x; t < ctx; t += kThreads) {
            const float pr = finite ? nvr::nvr_expf(probs[g * score_stride + t] - mg) : 0.0f;
            probs[g * score_stride + t] = pr;
            sum += pr;
        }
        sum = half_wave_sum(sum);
        if ((lane & 31) == 0) red_sum[g][2 * wave + (lane >> 5)] = sum;
    }
    if constexpr (TABLE == kStreamed)
        lds_barrier();  // leaves the V tiles in flight
    else
        __syncthreads();
#pragma unroll
    for (int g = 0; g < HPB; ++g) den[g] = fold8(red_sum[g]);

    // ---- 3. values ----
    // Thread (g, d) runs the fma chain of head g, dimension d. Tiles alternate
    // between two LDS slots; one block barrier per tile both publishes the tile
    // and guarantees the slot written next was consumed by every wave.
    const int g = threadIdx.x / DIM, d = threadIdx.x - g * DIM;
    const bool chain = threadIdx.x < HPB * DIM;
    const float* pg = probs + (chain ? g : 0) * score_stride;
    uint16_t* slots = reinterpret_cast<uint16_t*>(stage);  // [2][kVTile][DIM]
    float acc = 0.0f;
    uint32_t zlo[16] = {};  // kStreamed, head dim 128: value_tile_d128's zero-low registers
    auto put = [&](const uint4 (&r)[kVLoads], const bool (&ok)[kVLoads], int slot) {
#pragma unroll
        for (int u = 0; u < kVLoads; ++u)
            *reinterpret_cast<uint4*>(slots + slot * kVTile * DIM + 8 * (int(threadIdx.x) + kThreads * u)) =
                ok[u] ? r[u] : make_uint4(kNegZeroPair, kNegZeroPair, kNegZeroPair, kNegZeroPair);
        __syncthreads();
    };
    auto consume = [&](int slot, int t0) {
        const int n = min(kVTile, ctx - t0);
        if (!chain || n <= 0) return;
        const uint16_t* vt = slots + slot * kVTile * DIM + d;
        auto eight = [&](int j) {
            const float4 p0 = *reinterpret_cast<const float4*>(pg + t0 + j);
            const float4 p1 = *reinterpret_cast<const float4*>(pg + t0 + j + 4);
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = nvr::bf16_to_f32(vt[(j + k) * DIM]);
            acc = __builtin_fmaf(p0.x, v[0], acc);
            acc = __builtin_fmaf(p0.y, v[1], acc);
            acc = __builtin_fmaf(p0.z, v[2], acc);
            acc = __builtin_fmaf(p0.w, v[3], acc);
            acc = __builtin_fmaf(p1.x, v[4], acc);
            acc = __builtin_fmaf(p1.y, v[5], acc);
            acc = __builtin_fmaf(p1.z, v[6], acc);
            acc = __builtin_fmaf(p1.w, v[7], acc);
        };
        if constexpr (TABLE == kStreamed && DIM == 128) {
            if (n == kVTile) {
                value_tile_d128(acc, lds_address(vt), lds_address(pg + t0 + (lane & 15)), zlo);
                return;
            }
        }
        if (n == kVTile) {
            // A whole tile, software-pipelined: the LDS reads of the next 8
            // tokens are issued before the current 8 are chained, so each
            // group's LDS round trip hides behind the previous group's FMAs.
            float pa[8], pb[8];
            uint32_t va[8], vb[8];
            auto fetch = [&](int j, float (&p)[8], uint32_t (&v)[8]) {
                const float4 p0 = *reinterpret_cast<const float4*>(pg + t0 + j);
                const float4 p1 = *reinterpret_cast<const float4*>(pg + t0 + j + 4);
                p[0] = p0.x; p[1] = p0.y; p[2] = p0.z; p[3] = p0.w;
                p[4] = p1.x; p[5] = p1.y; p[6] = p1.z; p[7] = p1.w;
#pragma unroll
                for (int k = 0; k < 8; ++k) v[k] = vt[(j + k) * DIM];
            };
            auto chain8 = [&](const float (&p)[8], const uint32_t (&v)[8]) {
#pragma unroll
                for (int k = 0; k < 8; ++k) acc = __builtin_fmaf(p[k], __uint_as_float(v[k] << 16), acc);
            };
            fetch(0, pa, va);
#pragma unroll
            for (int j = 0; j < kVTile; j += 16) {
                fetch(j + 8, pb, vb);
                __builtin_amdgcn_sched_barrier(0);
                chain8(pa, va);
                if (j + 16 < kVTile) fetch(j + 16, pa, va);
                __builtin_amdgcn_sched_barrier(0);
                chain8(pb, vb);
            }
            return;
        }
        int j = 0;
        for (; j + 8 <= n; j += 8) eight(j);
        for (; j < n; ++j) acc = __builtin_fmaf(pg[t0 + j], nvr::bf16_to_f32(vt[j * DIM]), acc);
    };
    if constexpr (TABLE == kStreamed) {
        // Tile i is consumed while tiles i + 1 and i + 2 stream in; the
        // barrier before each issue also frees the slot it refills.
        for (int i = 0; i < ntiles; ++i) {
            stream_wait(min(ntiles - 1 - i, L::kSlots - 2));
            const int next = i + L::kSlots - 1;
            if (next < ntiles) stream_vtile(next * kVTile, next % L::kSlots);
            const int t0 = i * kVTile;
            if (entry_ok(group_entry(t0))) consume(i % L::kSlots, t0);  // an invalid block adds no V term
        }
    } else
    // Three register tiles in fixed roles keep two tiles in flight while one
    // is consumed. The loads past the context stay unconditional (they hit
    // token 0 of block 0 in L2; a branch would drain the load queue).
    for (int i = 0, t0 = 0; t0 < ctx; i += 3, t0 += 3 * kVTile) {
        put(rW, okW, i & 1);
        load_vtile(rW, okW, t0 + 3 * kVTile);
        consume(i & 1, t0);
        if (t0 + kVTile >= ctx) break;  // uniform
        put(rX, okX, (i + 1) & 1);
        load_vtile(rX, okX, t0 + 4 * kVTile);
        consume((i + 1) & 1, t0 + kVTile);
        if (t0 + 2 * kVTile >= ctx) break;  // uniform
        put(rY, okY, (i + 2) & 1);
        load_vtile(rY, okY, t0 + 5 * kVTile);
        consume((i + 2) & 1, t0 + 2 * kVTile);
    }
    if (chain) {
        float dg = den[0];
#pragma unroll
        for (int k = 1; k < HPB; ++k) dg = g == k ? den[k] : dg;
        orow[g * DIM + d] = nvr::f32_to_bf16(dg > 0.0f ? acc / dg : 0.0f);
    }
}

// Any even head dim up to 256, element loads. One block per (row, q head);
// each 32-lane half-wave scores one token at a time.
__global__ __launch_bounds__(kThreads) void attention_direct(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    const int* __restrict__ positions, const int* __restrict__ seqs, const int* __restrict__ tables,
    uint16_t* __restrict__ out, int qh, int kvh, int dim, int bs, int blocks, int stride, int batch,
    int max_context) {
    extern __shared__ __align__(16) unsigned char smem[];
    float* probs = reinterpret_cast<float*>(smem);
    __shared__ float red_max[kWaves];
    __shared__ float red_sum[2 * kWaves];
    const int row = blockIdx.x, head = blockIdx.y;
    const int kvhead = head / (qh / kvh);
    const int seq = seqs[row];
    const int64_t context64 = int64_t(positions[row]) + 1;
    const int64_t qbase = (int64_t(row) * qh + head) * dim;
    if (seq < 0 || seq >= batch || context64 < 1 || context64 > max_context ||
        context64 > int64_t(stride) * bs) {
        for (int d = threadIdx.x; d < dim; d += kThreads) out[qbase + d] = 0;
        return;
    }
    const int ctx = int(context64);
    const int* table = tables + int64_t(seq) * stride;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int c = lane & 31, half = threadIdx.x >> 5;
    const float scale = 1.0f / sqrtf(float(dim));
    float m = -__builtin_inff();
    for (int t = half; t < ctx; t += 2 * kWaves) {
        const int64_t ph = phys_token(table[t / bs], t, bs, blocks);
        float dot = 0.0f;
        if (ph >= 0) {
            const uint16_t* k = kc + (ph * kvh + kvhead) * dim;
            for (int d = c; d < dim; d += 32) dot = __builtin_fmaf(nvr::bf16_to_f32(q[qbase + d]),
                                                                  nvr::bf16_to_f32(k[d]), dot);
        }
        dot = half_wave_sum(dot);
        const float score = ph >= 0 ? dot * scale : -__builtin_inff();
        m = fmaxf(m, score);
        if (c == 0) probs[t] = score;
    }
    m = wave_max(m);
    if (lane == 0) red_max[wave] = m;
    __syncthreads();
    const float mg = fmaxf(fmaxf(red_max[0], red_max[1]), fmaxf(red_max[2], red_max[3]));
    const bool finite = __builtin_isfinite(mg);
    float sum = 0.0f;
    for (int t = threadIdx.x; t < ctx; t += kThreads) {
        const float pr = finite ? nvr::nvr_expf(probs[t] - mg) : 0.0f;
        probs[t] = pr;
        sum += pr;
    }
    sum = half_wave_sum(sum);
    if (c == 0) red_sum[half] = sum;
    __syncthreads();
    const float den = fold8(red_sum);
    for (int d = threadIdx.x; d < dim; d += kThreads) {
        float value = 0.0f;
        for (int t = 0; t < ctx; ++t) {
            const int64_t ph = phys_token(table[t / bs], t, bs, blocks);
            if (ph >= 0) value = __builtin_fmaf(probs[t], nvr::bf16_to_f32(vc[(ph * kvh + kvhead) * dim + d]), value);
        }
        out[qbase + d] = nvr::f32_to_bf16(den > 0.0f ? value / den : 0.0f);
    }
}

// Launch geometry of the ordered kernels. FUSED launches (head dim 128 only)
// also run the rows' q/k norm + RoPE + KV-slot write (QkvRopeArgs).
template <int DIM, int HPB, bool OCC, bool FUSED>
void launch_layout(nv_context* c, const uint16_t* q, uint16_t* k, uint16_t* v, const int* p, const int* s,
                   const int* t, uint16_t* o, int rows, int qh, int kvh, int bs, int blocks, int stride, int batch,
                   int max_context, const QkvRopeArgs& fa) {
    const int score_stride = (max_context + 3) & ~3;
    const int table_entries = (max_context - 1) / bs + 1;
    using L = OrderedLayout<DIM, HPB, OCC>;
    const size_t lds = sizeof(float) * HPB * score_stride + L::kStageBytes + sizeof(int) * table_entries;
    const dim3 grid(unsigned(rows), unsigned(qh / HPB));
    const bool pow2 = (bs & (bs - 1)) == 0;
    const int shift = pow2 ? __builtin_ctz(unsigned(bs)) : 0;
    // kAligned also needs the row's table in one wave (at most 64 entries) and
    // in-block offsets that fit in int32.
    const bool aligned = pow2 && bs >= L::kStep && bs >= L::kVTile && (max_context - 1) / bs < kWave &&
                         int64_t(bs) * kvh * DIM < (int64_t(1) << 31);
    // kStreamed's four V slots take the LDS a second block per CU would use:
    // it runs when the launch has at most one block per CU anyway (decode
    // batches up to 32 rows at Qwen3 shapes). Measured on MI355X at 8 rows x
    // 1024 tokens: 27.7 -> 23.7 us; 8-row serving step 1.075 -> 1.035 ms.
    if constexpr (!OCC) {
        const int64_t cus = c->cu_count > 0 ? c->cu_count : 256;
        if (aligned && int64_t(rows) * (qh / HPB) <= cus) {
            hipLaunchKernelGGL((attention_ordered<DIM, HPB, kStreamed, false, FUSED>), grid, dim3(kThreads),
                               sizeof(float) * HPB * score_stride + L::kStreamStage, c->stream, q, k, v, p, s, t, o,
                               qh, kvh, bs, shift, blocks, stride, batch, max_context, score_stride, fa);
            return;
        }
    }
    if (aligned)
        hipLaunchKernelGGL((attention_ordered<DIM, HPB, kAligned, OCC, FUSED>), grid, dim3(kThreads), lds, c->stream,
                           q, k, v, p, s, t, o, qh, kvh, bs, shift, blocks, stride, batch, max_context, score_stride,
                           fa);
    else if (pow2)
        hipLaunchKernelGGL((attention_ordered<DIM, HPB, kPow2, OCC, FUSED>), grid, dim3(kThreads), lds, c->stream,
                           q, k, v, p, s, t, o, qh, kvh, bs, shift, blocks, stride, batch, max_context, score_stride,
                           fa);
    else
        hipLaunchKernelGGL((attention_ordered<DIM, HPB, kAnyBs, OCC, FUSED>), grid, dim3(kThreads), lds, c->stream,
                           q, k, v, p, s, t, o, qh, kvh, bs, 0, blocks, stride, batch, max_context, score_stride,
                           fa);
}

// Blocks are (row, head group) and each walks its context serially, so when
// there are more than two blocks per CU the occupancy layout wins (three
// blocks per CU at 164 VGPRs and 52 KB of LDS for head dim 128 and 4096
// positions): measured on MI355X, 1024 prefill rows 164 -> 108 us (8 x 128
// tokens) and 457 -> 348 us (one 1024-token prompt). With at most two per CU
// the deeper pipelines win (64 x 4096 decode: 200 vs 210 us). FUSED launches
// (decode batches) keep the default layout.
template <int DIM, int HPB, bool FUSED = false>
void launch_ordered(nv_context* c, const uint16_t* q, uint16_t* k, uint16_t* v, const int* p,
                    const int* s, const int* t, uint16_t* o, int rows, int qh, int kvh, int bs, int blocks,
                    int stride, int batch, int max_context, const QkvRopeArgs& fa = {}) {
    if constexpr (DIM == 128 && HPB == 2 && !FUSED) {
        const int64_t groups = int64_t(rows) * (qh / HPB);
        if (groups > 2 * int64_t(c->cu_count > 0 ? c->cu_count : 256)) {
            launch_layout<DIM, HPB, true, false>(c, q, k, v, p, s, t, o, rows, qh, kvh, bs, blocks, stride, batch,
                                                 max_context, fa);
            return;
        }
    }
    launch_layout<DIM, HPB, false, FUSED>(c, q, k, v, p, s, t, o, rows, qh, kvh, bs, blocks, stride, batch,
                                          max_context, fa);
}

template <int DIM, bool FUSED = false>
void launch_dim(nv_context* c, const uint16_t* q, uint16_t* k, uint16_t* v, const int* p, const int* s,
                const int* t, uint16_t* o, int rows, int qh, int kvh, int bs, int blocks, int stride, int batch,
                int max_context, const QkvRopeArgs& fa = {}) {
    // A GQA pair per block reads each K/V row once for two heads. With fewer
    // pairs than CUs (small decode batches) one head per block wins instead:
    // twice the blocks on an otherwise idle GPU (measured on MI355X at 8 rows:
    // 9.0 vs 10.4 us at 130 tokens of context, 30.5 vs 35.2 us at 1024).
    const int64_t cus = c->cu_count > 0 ? c->cu_count : 256;
    if (DIM <= 128 && (qh / kvh) % 2 == 0 && int64_t(rows) * (qh / 2) >= cus)
        launch_ordered<DIM, (DIM <= 128 ? 2 : 1), FUSED>(c, q, k, v, p, s, t, o, rows, qh, kvh, bs, blocks, stride,
                                                         batch, max_context, fa);
    else
        launch_ordered<DIM, 1, FUSED>(c, q, k, v, p, s, t, o, rows, qh, kvh, bs, blocks, stride, batch, max_context,
                                      fa);
}

int check_attention(int rows, int qh, int kvh, int dim, int bs, int blocks, int stride, int batch,
                    int max_context) {
    if (rows <= 0 || qh <= 0 || kvh <= 0 || dim <= 0 || bs <= 0 || blocks <= 0 || stride <= 0 || batch <= 0 ||
        max_context <= 0)
        return nvr::fail(-2, "attention: dimensions must be positive");
    if (qh % kvh != 0 || dim % 2 != 0 || dim > 256 || qh > 65535)
        return nvr::fail(-2, "attention: need qh %% kvh == 0, an even head dim <= 256 and qh <= 65535");
    if (max_context > kMaxContext) return nvr::fail(-2, "attention: max_context above %d", kMaxContext);
    return 0;
}

}  // namespace

extern "C" int nv_attention(nv_context* c, const void* q, const void* kc, const void* vc, const void* positions,
                            const void* seqs, const void* tables, void* out, int rows, int qh, int kvh, int dim,
                            int bs, int blocks, int stride, int batch, int max_context) {
    NVR_ACTIVATE(c);
    if (int e = check_attention(rows, qh, kvh, dim, bs, blocks, stride, batch, max_context)) return e;
    auto q16 = static_cast<const uint16_t*>(q);
    auto k16 = static_cast<uint16_t*>(const_cast<void*>(kc));  // read only: this entry point writes no cache
    auto v16 = static_cast<uint16_t*>(const_cast<void*>(vc));
    auto p32 = static_cast<const int*>(positions);
    auto s32 = static_cast<const int*>(seqs);
    auto t32 = static_cast<const int*>(tables);
    auto o16 = static_cast<uint16_t*>(out);
    // The ordered kernels index cache rows in int32.
    const bool vec = nvr::aligned(q, 16) && nvr::aligned(kc, 16) && nvr::aligned(vc, 16) &&
                     int64_t(blocks) * bs <= 0x7fffffff;
    if (vec && dim == 128)
        launch_dim<128>(c, q16, k16, v16, p32, s32, t32, o16, rows, qh, kvh, bs, blocks, stride, batch, max_context);
    else if (vec && dim == 64)
        launch_dim<64>(c, q16, k16, v16, p32, s32, t32, o16, rows, qh, kvh, bs, blocks, stride, batch, max_context);
    else if (vec && dim == 32)
        launch_dim<32>(c, q16, k16, v16, p32, s32, t32, o16, rows, qh, kvh, bs, blocks, stride, batch, max_context);
    else if (vec && dim == 256)
        launch_ordered<256, 1>(c, q16, k16, v16, p32, s32, t32, o16, rows, qh, kvh, bs, blocks, stride, batch,
                               max_context);
    else
        hipLaunchKernelGGL(attention_direct, dim3(unsigned(rows), unsigned(qh)), dim3(kThreads),
                           sizeof(float) * size_t(max_context), c->stream, q16, k16, v16, p32, s32, t32, o16, qh,
                           kvh, dim, bs, blocks, stride, batch, max_context);
    return nvr::launch_status();
}

// Decode form: nv_qkv_rope_cached's q/k norm + RoPE + KV-slot write run inside
// the attention launch (QkvRopeArgs), so the rotated q never leaves LDS and
// one launch per layer goes away. Each row's prologue finishes before that
// row's blocks read the cache, but rows do not wait for each other: no row may
// read a slot that another row of the call writes (one row per sequence, as in
// a decode batch whose written slots sit in blocks no other row maps).
extern "C" int nv_attention_qkv_rope(nv_context* c, const void* qkv, const void* qw, const void* kw,
                                     const void* positions, const void* slots, void* kc, void* vc,
                                     const void* seqs, const void* tables, void* out, int rows, int qh, int kvh,
                                     int dim, int bs, int blocks, int stride, int batch, int max_context, float eps,
                                     const void* rope_cache, int max_positions) {
    NVR_ACTIVATE(c);
    if (int e = check_attention(rows, qh, kvh, dim, bs, blocks, stride, batch, max_context)) return e;
    if (dim != 128) return nvr::fail(-2, "attention_qkv_rope: head dim %d, the fused form needs 128", dim);
    if (max_positions < 0) return nvr::fail(-2, "attention_qkv_rope: max_positions must be non-negative");
    if (!(nvr::aligned(qkv, 16) && nvr::aligned(qw, 16) && nvr::aligned(kw, 16) && nvr::aligned(kc, 16) &&
          nvr::aligned(vc, 16) && nvr::aligned(rope_cache, 16)) ||
        int64_t(blocks) * bs > 0x7fffffff)
        return nvr::fail(-2, "attention_qkv_rope: needs 16-byte aligned tensors and blocks * bs < 2^31");
    const QkvRopeArgs fa{static_cast<const uint16_t*>(qkv), static_cast<const uint16_t*>(qw),
                         static_cast<const uint16_t*>(kw), static_cast<const int*>(slots),
                         static_cast<const float*>(rope_cache), max_positions, eps};
    launch_dim<128, true>(c, nullptr, static_cast<uint16_t*>(kc), static_cast<uint16_t*>(vc),
                          static_cast<const int*>(positions), static_cast<const int*>(seqs),
                          static_cast<const int*>(tables), static_cast<uint16_t*>(out), rows, qh, kvh, bs, blocks,
                          stride, batch, max_context, fa);
    return nvr::launch_status();
}
