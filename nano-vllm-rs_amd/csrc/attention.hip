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
// row's K and V are read once for both heads of a GQA pair.
//   1. Scores: four lanes per token. Lane a of a quad owns chains 8a .. 8a+7,
//      so it loads k[32j + 8a .. 32j + 8a + 7] (one 16-byte load per j) and q
//      the same way. The first two tree levels (offsets 16 and 8) pair lanes
//      a ^ 2 and a ^ 1 of the quad (DPP adds); the last three run inside the
//      lane. 64 tokens per block step; the next step's K and the step after
//      that's block-table entries are in flight during the current step.
//      Scores go to LDS.
//   2. Block max, exp in place, the block sum in the reference's order.
//   3. Values: V tiles of kVTile tokens are staged in LDS with 16-byte loads
//      (the next tile's loads in flight during the current tile); thread
//      (g, d) runs its fma chain over the tile's tokens in order. Tokens of an
//      invalid block are staged as -0.0 with p = +0, which leaves every chain
//      value (including -0) unchanged, exactly as skipping them does.
// Other head dims use a direct kernel with the same arithmetic.
#include "../../include/nano_hip.h"
#include "nvr_device.h"
#include "nvr_internal.h"

namespace {

using nvr::kWave;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxContext = 4096;  // src/gpu.rs:848-852
constexpr int kVTile = 64;         // tokens per staged V tile
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

// Physical token index of a table entry and logical token, or -1.
__device__ __forceinline__ int64_t phys_token(int entry, int t, int bs, int blocks) {
    return entry >= 0 && entry < blocks ? int64_t(entry) * bs + t % bs : int64_t(-1);
}

template <int DIM, int HPB>
__global__ __launch_bounds__(kThreads) void attention_ordered(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    const int* __restrict__ positions, const int* __restrict__ seqs, const int* __restrict__ tables,
    uint16_t* __restrict__ out, int qh, int kvh, int bs, int blocks, int stride, int batch, int max_context,
    int score_stride) {
    static_assert(DIM % 32 == 0 && DIM <= 256 && HPB * DIM <= kThreads, "shape");
    constexpr int P = DIM / 32;            // elements per chain
    constexpr int kQuads = kWave / 4;      // tokens per wave per step
    constexpr int kStep = kQuads * kWaves;  // tokens per block step
    constexpr int kPieces = DIM / 8;       // 16-byte pieces per K/V row
    constexpr int kTileLoads = kVTile * kPieces / kThreads;  // per thread
    static_assert(kTileLoads * kThreads == kVTile * kPieces, "tile");

    extern __shared__ __align__(16) unsigned char smem[];
    float* probs = reinterpret_cast<float*>(smem);  // [HPB][score_stride]
    uint16_t* vtile = reinterpret_cast<uint16_t*>(smem + sizeof(float) * HPB * score_stride);  // [kVTile][DIM]
    __shared__ float red_max[HPB][kWaves];
    __shared__ float red_sum[HPB][2 * kWaves];

    const int row = blockIdx.x;
    const int h0 = blockIdx.y * HPB;
    const int kvhead = h0 / (qh / kvh);
    const int seq = seqs[row];
    const int64_t context64 = int64_t(positions[row]) + 1;
    uint16_t* orow = out + (int64_t(row) * qh + h0) * DIM;
    if (seq < 0 || seq >= batch || context64 < 1 || context64 > max_context ||
        context64 > int64_t(stride) * bs) {
        for (int i = threadIdx.x; i < HPB * DIM; i += kThreads) orow[i] = 0;
        return;
    }
    const int ctx = int(context64);
    const int* table = tables + int64_t(seq) * stride;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int a = lane & 3;
    const int64_t token_stride = int64_t(kvh) * DIM;  // elements between tokens of a block
    const uint16_t* kcol = kc + int64_t(kvhead) * DIM + 8 * a;

    // ---- 1. scores ----
    float qf[HPB][P][8];
#pragma unroll
    for (int g = 0; g < HPB; ++g)
#pragma unroll
        for (int j = 0; j < P; ++j)
            nvr::unpack8(*reinterpret_cast<const uint4*>(q + (int64_t(row) * qh + h0 + g) * DIM + 32 * j + 8 * a),
                         qf[g][j]);
    const float kScale = 1.0f / sqrtf(float(DIM));

    int tc = wave * kQuads + (lane >> 2);  // this quad's token in the current step
    int64_t pc = tc < ctx ? phys_token(table[tc / bs], tc, bs, blocks) : -1;
    uint4 kcur[P];
#pragma unroll
    for (int j = 0; j < P; ++j)
        kcur[j] = pc >= 0 ? nvr::load_stream(kcol + pc * token_stride + 32 * j) : make_uint4(0, 0, 0, 0);
    int tn = tc + kStep;
    int entry_n = tn < ctx ? table[tn / bs] : -1;
    float m[HPB];
#pragma unroll
    for (int g = 0; g < HPB; ++g) m[g] = -__builtin_inff();

    for (int t0 = 0; t0 < ctx; t0 += kStep) {
        const int64_t pn = tn < ctx ? phys_token(entry_n, tn, bs, blocks) : -1;
        uint4 knext[P];
#pragma unroll
        for (int j = 0; j < P; ++j)
            knext[j] = pn >= 0 ? nvr::load_stream(kcol + pn * token_stride + 32 * j) : make_uint4(0, 0, 0, 0);
        const int tnn = tn + kStep;
        const int entry_nn = tnn < ctx ? table[tnn / bs] : -1;

        float kf[P][8];
#pragma unroll
        for (int j = 0; j < P; ++j) nvr::unpack8(kcur[j], kf[j]);
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
            const float dot = ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
            const float score = pc >= 0 ? dot * kScale : -__builtin_inff();
            if (tc < ctx) {
                m[g] = fmaxf(m[g], score);
                if (a == 0) probs[g * score_stride + tc] = score;
            }
        }
#pragma unroll
        for (int j = 0; j < P; ++j) kcur[j] = knext[j];
        pc = pn;
        tc = tn;
        tn = tnn;
        entry_n = entry_nn;
    }

    // ---- 2. max, exp, block sum ----
#pragma unroll
    for (int g = 0; g < HPB; ++g) {
        m[g] = wave_max(m[g]);
        if (lane == 0) red_max[g][wave] = m[g];
    }
    __syncthreads();
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
    __syncthreads();
#pragma unroll
    for (int g = 0; g < HPB; ++g) den[g] = fold8(red_sum[g]);

    // ---- 3. values ----
    const int g = threadIdx.x / DIM, d = threadIdx.x - g * DIM;
    const bool chain = threadIdx.x < HPB * DIM;
    const float* pg = probs + (chain ? g : 0) * score_stride;
    float acc = 0.0f;
    // Staging: load u of this thread covers token (tid + 256u) / kPieces of the
    // tile, piece (tid + 256u) % kPieces.
    int entry[kTileLoads];
    uint4 vr[kTileLoads];
    auto tile_token = [&](int t0, int u) { return t0 + (int(threadIdx.x) + kThreads * u) / kPieces; };
    auto load_entries = [&](int t0) {
#pragma unroll
        for (int u = 0; u < kTileLoads; ++u) {
            const int t = tile_token(t0, u);
            entry[u] = t < ctx ? table[t / bs] : -1;
        }
    };
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int u = 0; u < kTileLoads; ++u) {
            const int t = tile_token(t0, u);
            const int piece = (int(threadIdx.x) + kThreads * u) % kPieces;
            const int64_t ph = t < ctx ? phys_token(entry[u], t, bs, blocks) : -1;
            vr[u] = ph >= 0 ? nvr::load_stream(vc + (ph * kvh + kvhead) * DIM + 8 * piece)
                            : make_uint4(kNegZeroPair, kNegZeroPair, kNegZeroPair, kNegZeroPair);
        }
    };
    load_entries(0);
    load_tile(0);
    load_entries(kVTile);
    for (int t0 = 0; t0 < ctx; t0 += kVTile) {
        __syncthreads();  // the previous tile is consumed
#pragma unroll
        for (int u = 0; u < kTileLoads; ++u)
            *reinterpret_cast<uint4*>(vtile + 8 * (int(threadIdx.x) + kThreads * u)) = vr[u];
        __syncthreads();
        if (t0 + kVTile < ctx) {
            load_tile(t0 + kVTile);
            load_entries(t0 + 2 * kVTile);
        }
        const int n = min(kVTile, ctx - t0);
        if (chain) {
            int j = 0;
            for (; j + 8 <= n; j += 8) {
                const float4 p0 = *reinterpret_cast<const float4*>(pg + t0 + j);
                const float4 p1 = *reinterpret_cast<const float4*>(pg + t0 + j + 4);
                float v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = nvr::bf16_to_f32(vtile[(j + i) * DIM + d]);
                acc = __builtin_fmaf(p0.x, v[0], acc);
                acc = __builtin_fmaf(p0.y, v[1], acc);
                acc = __builtin_fmaf(p0.z, v[2], acc);
                acc = __builtin_fmaf(p0.w, v[3], acc);
                acc = __builtin_fmaf(p1.x, v[4], acc);
                acc = __builtin_fmaf(p1.y, v[5], acc);
                acc = __builtin_fmaf(p1.z, v[6], acc);
                acc = __builtin_fmaf(p1.w, v[7], acc);
            }
            for (; j < n; ++j) acc = __builtin_fmaf(pg[t0 + j], nvr::bf16_to_f32(vtile[j * DIM + d]), acc);
        }
    }
    if (chain) {
        float dg = den[0];
#pragma unroll
        for (int i = 1; i < HPB; ++i) dg = g == i ? den[i] : dg;
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

template <int DIM, int HPB>
void launch_ordered(nv_context* c, const uint16_t* q, const uint16_t* k, const uint16_t* v, const int* p,
                    const int* s, const int* t, uint16_t* o, int rows, int qh, int kvh, int bs, int blocks,
                    int stride, int batch, int max_context) {
    const int score_stride = (max_context + 3) & ~3;
    const size_t lds = sizeof(float) * HPB * score_stride + sizeof(uint16_t) * kVTile * DIM;
    hipLaunchKernelGGL((attention_ordered<DIM, HPB>), dim3(unsigned(rows), unsigned(qh / HPB)), dim3(kThreads), lds,
                       c->stream, q, k, v, p, s, t, o, qh, kvh, bs, blocks, stride, batch, max_context, score_stride);
}

template <int DIM>
void launch_dim(nv_context* c, const uint16_t* q, const uint16_t* k, const uint16_t* v, const int* p, const int* s,
                const int* t, uint16_t* o, int rows, int qh, int kvh, int bs, int blocks, int stride, int batch,
                int max_context) {
    if (DIM <= 128 && (qh / kvh) % 2 == 0)
        launch_ordered<DIM, (DIM <= 128 ? 2 : 1)>(c, q, k, v, p, s, t, o, rows, qh, kvh, bs, blocks, stride, batch,
                                                  max_context);
    else
        launch_ordered<DIM, 1>(c, q, k, v, p, s, t, o, rows, qh, kvh, bs, blocks, stride, batch, max_context);
}

}  // namespace

extern "C" int nv_attention(nv_context* c, const void* q, const void* kc, const void* vc, const void* positions,
                            const void* seqs, const void* tables, void* out, int rows, int qh, int kvh, int dim,
                            int bs, int blocks, int stride, int batch, int max_context) {
    NVR_ACTIVATE(c);
    if (rows <= 0 || qh <= 0 || kvh <= 0 || dim <= 0 || bs <= 0 || blocks <= 0 || stride <= 0 || batch <= 0 ||
        max_context <= 0)
        return nvr::fail(-2, "attention: dimensions must be positive");
    if (qh % kvh != 0 || dim % 2 != 0 || dim > 256 || qh > 65535)
        return nvr::fail(-2, "attention: need qh %% kvh == 0, an even head dim <= 256 and qh <= 65535");
    if (max_context > kMaxContext) return nvr::fail(-2, "attention: max_context above %d", kMaxContext);
    auto q16 = static_cast<const uint16_t*>(q);
    auto k16 = static_cast<const uint16_t*>(kc);
    auto v16 = static_cast<const uint16_t*>(vc);
    auto p32 = static_cast<const int*>(positions);
    auto s32 = static_cast<const int*>(seqs);
    auto t32 = static_cast<const int*>(tables);
    auto o16 = static_cast<uint16_t*>(out);
    const bool vec = nvr::aligned(q, 16) && nvr::aligned(kc, 16) && nvr::aligned(vc, 16);
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
