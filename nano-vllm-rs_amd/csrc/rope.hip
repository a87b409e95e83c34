// Per-head q/k RMSNorm + NeoX RoPE + paged KV write (nv_qkv_rope,
// nv_qkv_rope_cached) and the RoPE table (nv_rope_cache).
//
// Semantics: kernels/kernels.cu:166-224 of nano-vllm-rs. For packed row r and
// head h of qkv[r, qh + 2*kvh, dim]:
//   q/k head:  inv = 1/sqrt(sum x^2 / dim + eps)  (reference thread order:
//              thread t holds element t; shuffle-down trees per 32-thread warp,
//              then over the warp sums)
//              n_j = f32(bf16((x_j * inv) * w_j))           (bf16 materialised)
//              j <  dim/2: rot = (n_j * c) - (n_{j+dim/2} * s)  (no FMA)
//              j >= dim/2: rot = (n_j * c) + (n_{j-dim/2} * s)
//              c, s = table[pos][j % (dim/2)], table[pos][dim/2 + j % (dim/2)]
//              (cached, pos outside [0, max_positions) -> c = 1, s = 0) or
//              computed inline (uncached)
//              q -> qout[r, h, j] = bf16(rot); k -> kc[slot, h', j] = bf16(rot)
//   v head:    vc[slot, h', :] = qkv[r, qh + kvh + h', :]  (bit copy)
//   K and V are written only when 0 <= slot < bs * blocks.
//
// Fast path (dim = 128, 16-byte aligned): a head occupies a 16-lane DPP row.
// Lane m holds elements 8m..8m+7 (one 16-byte load), i.e. reference threads
// 8m..8m+7. Warp levels 16/8 -> lane m^2 / m^1, levels 4/2/1 in-lane; the warp
// sums sit in lanes 0,4,8,12 and fold as (W0 + W2) + (W1 + W3). The NeoX
// partner of element j lives in lane m^8 of the same 16-lane row.
#include "../../include/nano_hip.h"
#include "nvr_device.h"
#include "nvr_internal.h"

namespace {

using nvr::kWave;

constexpr int kHeadLanes = 16;
// Row count from which the d128 kernel uses four waves per row instead of two.
constexpr int kRopeSplit4Rows = 4096;

// SPLIT waves per token row. The row's heads form quads 4Q..4Q+3; wave part
// hw takes quads hw, hw+SPLIT, hw+2*SPLIT, ... and group g (16 lanes) of the
// wave takes head 4Q + g of each of its quads. Lane m of a group holds
// elements 8m..8m+7 of a head. All head loads of a lane are issued first;
// position, slot, cos/sin and the norm weights are read once per wave. Four
// waves per row (2 quads each, 67 VGPRs, 7 waves per SIMD) measured fastest
// at 8192 rows, two waves per row (4 quads each) at 2048 rows.
template <bool CACHED, int SPLIT>
__global__ __launch_bounds__(256) void qkv_rope_d128(const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ qw,
                                                     const uint16_t* __restrict__ kw, const int* __restrict__ positions,
                                                     const int* __restrict__ slots, uint16_t* __restrict__ qout,
                                                     uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int rows,
                                                     int qh, int kvh, int bs, int blocks, float eps, float theta,
                                                     const float* __restrict__ table, int max_positions) {
    constexpr int D = 128, HALF = 64, GROUPS = kWave / kHeadLanes, DEPTH = 8 / SPLIT;
    const int lane = threadIdx.x & (kWave - 1);
    const int grp = lane / kHeadLanes, m = lane & (kHeadLanes - 1);
    // The wave's row is uniform: make it a scalar so position and slot come
    // from scalar loads (their own counter), not from the vector queue behind
    // the head loads.
    const int wave = __builtin_amdgcn_readfirstlane(int(blockIdx.x) * int(blockDim.x / kWave) +
                                                    int(threadIdx.x / kWave));
    const int row = wave / SPLIT;
    const int hw = wave - row * SPLIT;
    if (row >= rows) return;  // uniform per wave
    const int heads = qh + 2 * kvh;
    const uint16_t* src = qkv + int64_t(row) * heads * D + 8 * m;
    // Head of slot j in pass `pass`: quad hw + SPLIT * (j + DEPTH * pass).
    // Loads are unconditional (a head index past the row is clamped and its
    // data unused): a branch around a load makes the compiler wait for the
    // whole load queue before the first head is processed.
    auto head_of = [&](int pass, int j) { return GROUPS * (hw + SPLIT * (j + DEPTH * pass)) + grp; };
    uint4 xw[DEPTH];
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) xw[j] = nvr::load_stream(src + int64_t(min(head_of(0, j), heads - 1)) * D);
    const int pos = positions[row];
    const int slot = slots[row];
    const bool valid_slot = slot >= 0 && int64_t(slot) < int64_t(bs) * blocks;

    // Norm weights and the position's cos/sin are requested before anything
    // waits on a load, so all of a wave's loads are in flight together.
    const uint4 qwv = *reinterpret_cast<const uint4*>(qw + 8 * m);
    const uint4 kwv = *reinterpret_cast<const uint4*>(kw + 8 * m);
    const int pair0 = 8 * (m & 7);
    float cs[8], sn[8];
    if constexpr (CACHED) {
        if (pos >= 0 && pos < max_positions) {
            const float4* t = reinterpret_cast<const float4*>(table + int64_t(pos) * D + pair0);
            const float4 c0 = t[0], c1 = t[1];
            const float4 s0 = t[HALF / 4], s1 = t[HALF / 4 + 1];
            cs[0] = c0.x; cs[1] = c0.y; cs[2] = c0.z; cs[3] = c0.w;
            cs[4] = c1.x; cs[5] = c1.y; cs[6] = c1.z; cs[7] = c1.w;
            sn[0] = s0.x; sn[1] = s0.y; sn[2] = s0.z; sn[3] = s0.w;
            sn[4] = s1.x; sn[5] = s1.y; sn[6] = s1.z; sn[7] = s1.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) { cs[i] = 1.0f; sn[i] = 0.0f; }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) nvr::rope_cos_sin(pos, pair0 + i, D, theta, &cs[i], &sn[i]);
    }
    if (m < 8) {
#pragma unroll
        for (int i = 0; i < 8; ++i) sn[i] = -sn[i];
    }
    float qwf[8], kwf[8];
    nvr::unpack8(qwv, qwf);
    nvr::unpack8(kwv, kwf);

    // Uniform trip count: a pass runs while its first quad exists.
    for (int pass = 0; GROUPS * (hw + SPLIT * DEPTH * pass) < heads; ++pass) {
        if (pass > 0) {  // rows with more than 32 heads
#pragma unroll
            for (int j = 0; j < DEPTH; ++j)
                xw[j] = nvr::load_stream(src + int64_t(min(head_of(pass, j), heads - 1)) * D);
        }
#pragma unroll
        for (int j = 0; j < DEPTH; ++j) {
            const int h = head_of(pass, j);
            if (h >= heads) continue;
            if (h >= qh + kvh) {  // V head: bit copy into the cache
                if (valid_slot) nvr::store_stream(vc + (int64_t(slot) * kvh + (h - qh - kvh)) * D + 8 * m, xw[j]);
            } else if (h < qh) {
                nvr::store_stream(qout + (int64_t(row) * qh + h) * D + 8 * m,
                                  nvr::norm_rotate_d128(xw[j], qwf, cs, sn, eps));
            } else {
                const uint4 rot = nvr::norm_rotate_d128(xw[j], kwf, cs, sn, eps);
                if (valid_slot) nvr::store_stream(kc + (int64_t(slot) * kvh + (h - qh)) * D + 8 * m, rot);
            }
        }
    }
}

// Any even dim <= 256, 2-byte alignment: one (row, head) per wave, lane l plays
// reference threads 4l..4l+3 (thread t holds element t when t < dim). The
// normalised head is staged in LDS so each element can read its NeoX partner.
template <bool CACHED>
__global__ __launch_bounds__(256) void qkv_rope_generic(const uint16_t* __restrict__ qkv,
                                                        const uint16_t* __restrict__ qw,
                                                        const uint16_t* __restrict__ kw,
                                                        const int* __restrict__ positions,
                                                        const int* __restrict__ slots, uint16_t* __restrict__ qout,
                                                        uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int rows,
                                                        int qh, int kvh, int dim, int bs, int blocks, float eps,
                                                        float theta, const float* __restrict__ table,
                                                        int max_positions) {
    __shared__ float staged[4][256];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int heads = qh + 2 * kvh;
    const int64_t g = int64_t(blockIdx.x) * 4 + wave;
    const int64_t row = g / heads;
    const int head = int(g - row * heads);
    if (row >= rows) return;  // uniform per wave
    const int64_t packed = row * heads * dim;
    const int slot = slots[row];
    const bool valid_slot = slot >= 0 && int64_t(slot) < int64_t(bs) * blocks;
    if (head >= qh + kvh) {
        if (valid_slot) {
            const int local = head - qh - kvh;
            for (int j = lane; j < dim; j += kWave)
                vc[(int64_t(slot) * kvh + local) * dim + j] = qkv[packed + int64_t(head) * dim + j];
        }
        return;
    }
    const bool is_q = head < qh;
    const int local = is_q ? head : head - qh;
    const uint16_t* src = qkv + packed + int64_t(head) * dim;
    float s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = 4 * lane + i;
        const float v = t < dim ? nvr::bf16_to_f32(src[t]) : 0.0f;
        s[i] = v * v;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = s[i] + nvr::xor_lane(s[i], 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = s[i] + nvr::xor_lane(s[i], 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = s[i] + nvr::xor_lane(s[i], 1);
    float total = (s[0] + s[2]) + (s[1] + s[3]);
    total = total + nvr::xor_lane(total, 32);
    total = total + nvr::xor_lane(total, 16);
    total = total + nvr::xor_lane(total, 8);
    const float inv = nvr::inv_sqrt_rn(total / float(dim) + eps);
    const uint16_t* w = is_q ? qw : kw;
    for (int j = lane; j < dim; j += kWave)
        staged[wave][j] = nvr::round_bf16((nvr::bf16_to_f32(src[j]) * inv) * nvr::bf16_to_f32(w[j]));
    // staged[wave] is private to this wave: order its LDS writes before the
    // partner reads with a wave-scope fence instead of a block barrier.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int half = dim / 2;
    const int pos = positions[row];
    for (int j = lane; j < dim; j += kWave) {
        const int pair = j % half;
        float c, sn;
        if constexpr (CACHED) {
            const bool ok = pos >= 0 && pos < max_positions;
            c = ok ? table[int64_t(pos) * dim + pair] : 1.0f;
            sn = ok ? table[int64_t(pos) * dim + half + pair] : 0.0f;
        } else {
            nvr::rope_cos_sin(pos, pair, dim, theta, &c, &sn);
        }
        const float a = staged[wave][j] * c;
        const float b = staged[wave][j < half ? j + half : j - half] * sn;
        const float rot = j < half ? a - b : a + b;
        if (is_q) qout[(row * qh + local) * dim + j] = nvr::f32_to_bf16(rot);
        else if (valid_slot) kc[(int64_t(slot) * kvh + local) * dim + j] = nvr::f32_to_bf16(rot);
    }
}

__global__ __launch_bounds__(256) void rope_table(float* __restrict__ cache, int positions, int dim, float theta) {
    const int half = dim / 2;
    const int64_t total = int64_t(positions) * half;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
        const int pos = int(i / half), pair = int(i % half);
        float c, s;
        nvr::rope_cos_sin(pos, pair, dim, theta, &c, &s);
        cache[int64_t(pos) * dim + pair] = c;
        cache[int64_t(pos) * dim + half + pair] = s;
    }
}

template <bool CACHED>
int launch_qkv_rope(nv_context* c, const void* qkv, const void* qw, const void* kw, const void* positions,
                    const void* slots, void* qout, void* kc, void* vc, int rows, int qh, int kvh, int dim, int bs,
                    int blocks, float eps, float theta, const void* table, int max_positions) {
    NVR_ACTIVATE(c);
    if (rows <= 0 || qh <= 0 || kvh <= 0 || dim <= 0 || bs <= 0 || blocks <= 0)
        return nvr::fail(-2, "qkv_rope: dimensions must be positive");
    if (dim % 2 != 0 || dim > 256) return nvr::fail(-2, "qkv_rope: head dimension must be even and at most 256");
    const int64_t heads = int64_t(qh) + 2 * int64_t(kvh);
    const int64_t pairs = int64_t(rows) * heads;
    auto q16 = static_cast<const uint16_t*>(qkv);
    auto qw16 = static_cast<const uint16_t*>(qw);
    auto kw16 = static_cast<const uint16_t*>(kw);
    auto pos = static_cast<const int*>(positions);
    auto sl = static_cast<const int*>(slots);
    auto qo = static_cast<uint16_t*>(qout);
    auto k16 = static_cast<uint16_t*>(kc);
    auto v16 = static_cast<uint16_t*>(vc);
    auto tab = static_cast<const float*>(table);
    const bool vec = dim == 128 && rows <= (1 << 28) && nvr::aligned(qkv, 16) && nvr::aligned(qw, 16) &&
                     nvr::aligned(kw, 16) &&
                     nvr::aligned(qout, 16) && nvr::aligned(kc, 16) && nvr::aligned(vc, 16) &&
                     (!CACHED || nvr::aligned(table, 16));
    if (vec && rows >= kRopeSplit4Rows) {
        const int64_t nblocks = int64_t(rows);  // four waves per row
        if (nblocks > 0x7fffffff) return nvr::fail(-2, "qkv_rope: too many rows for one launch");
        hipLaunchKernelGGL((qkv_rope_d128<CACHED, 4>), dim3(unsigned(nblocks)), dim3(256), 0, c->stream, q16, qw16,
                           kw16, pos, sl, qo, k16, v16, rows, qh, kvh, bs, blocks, eps, theta, tab, max_positions);
    } else if (vec) {
        const int64_t nblocks = (int64_t(rows) * 2 + 3) / 4;  // two waves per row
        hipLaunchKernelGGL((qkv_rope_d128<CACHED, 2>), dim3(unsigned(nblocks)), dim3(256), 0, c->stream, q16, qw16,
                           kw16, pos, sl, qo, k16, v16, rows, qh, kvh, bs, blocks, eps, theta, tab, max_positions);
    } else {
        const int64_t nblocks = (pairs + 3) / 4;
        if (nblocks > 0x7fffffff) return nvr::fail(-2, "qkv_rope: too many rows for one launch");
        hipLaunchKernelGGL((qkv_rope_generic<CACHED>), dim3(unsigned(nblocks)), dim3(256), 0, c->stream, q16, qw16,
                           kw16, pos, sl, qo, k16, v16, rows, qh, kvh, dim, bs, blocks, eps, theta, tab,
                           max_positions);
    }
    return nvr::launch_status();
}

}  // namespace

extern "C" {

int nv_qkv_rope(nv_context* c, const void* qkv, const void* qw, const void* kw, const void* positions,
                const void* slots, void* qout, void* kc, void* vc, int rows, int qh, int kvh, int dim, int bs,
                int blocks, float eps, float theta) {
    return launch_qkv_rope<false>(c, qkv, qw, kw, positions, slots, qout, kc, vc, rows, qh, kvh, dim, bs, blocks,
                                  eps, theta, nullptr, 0);
}

int nv_qkv_rope_cached(nv_context* c, const void* qkv, const void* qw, const void* kw, const void* positions,
                       const void* slots, void* qout, void* kc, void* vc, int rows, int qh, int kvh, int dim, int bs,
                       int blocks, float eps, const void* rope_cache, int max_positions) {
    return launch_qkv_rope<true>(c, qkv, qw, kw, positions, slots, qout, kc, vc, rows, qh, kvh, dim, bs, blocks,
                                 eps, 1.0f, rope_cache, max_positions);
}

int nv_rope_cache(nv_context* c, void* cache, int positions, int dim, float theta) {
    NVR_ACTIVATE(c);
    if (positions <= 0 || dim <= 0 || dim % 2 != 0) return nvr::fail(-2, "rope_cache: invalid dimensions");
    const int64_t total = int64_t(positions) * (dim / 2);
    const int64_t want = (total + 255) / 256;
    const unsigned grid = unsigned(want > 65535 ? 65535 : want);
    hipLaunchKernelGGL(rope_table, dim3(grid), dim3(256), 0, c->stream, static_cast<float*>(cache), positions, dim,
                       theta);
    return nvr::launch_status();
}

}  // extern "C"
