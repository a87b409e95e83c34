// RMSNorm and residual-add + RMSNorm (nv_rms / nv_add_rms).
//
// Semantics: kernels/kernels.cu:145-164 of nano-vllm-rs.
//   v      = f32(x) (+ f32(residual))
//   s      = sum of v^2 in the reference's order (below)
//   inv    = 1 / sqrt(s / hidden + eps)          (fixed-bits replacement of rsqrtf)
//   out    = bf16((v * inv) * f32(weight))        (one rounding)
//   residual <- bf16(v)                           (ADD only; the norm uses unrounded v)
//
// Summation order. The reference reduces with a 256-thread block: thread t
// accumulates s_t = fma(v, v, s_t) over j = t, t+256, ...; each 32-thread warp
// folds its partials with a shuffle-down tree (offsets 16, 8, 4, 2, 1); the
// eight warp sums are folded by the same tree with zeros above lane 7. The
// kernels below keep exactly that association, so their sums carry the
// reference's bits.
//
// Fast path (hidden = 256*K, 16-byte aligned rows): one row per half-wave.
// Lane m (0..31) of a half owns reference threads 8m..8m+7 and loads the
// 16-byte chunk at 256k + 8m for every k < K, so the whole row stays in VGPRs
// (one HBM pass; the reference reads x and residual twice). In that layout
//   warp level 16 -> lane m^2, level 8 -> lane m^1, levels 4/2/1 -> in-lane,
//   block level 4 -> lane m^16, level 2 -> m^8, level 1 -> m^4.
// (The cross-lane steps use LDS-crossbar shuffles; DPP variants and a
// two-source bf16 pack measured slower for this kernel on MI355X.)
// Generic path (any hidden, any alignment): one row per wave, lane l owns
// reference threads 4l..4l+3 with 2-byte accesses.
//
// GATHER (nv_add_rms_gather): output row r is input row index[r] — the final
// add-RMSNorm and the last-token gather of src/model.rs:781-797 in one
// launch, computed for the gathered rows only. The residual is only read
// (after the final norm nothing reads it), so a row may be gathered any
// number of times. An index outside [0, input_rows) gives a +0 row (the
// gather's rule, kernels/kernels.cu:366-371).
#include "../../include/nano_hip.h"
#include "nvr_device.h"
#include "nvr_internal.h"

namespace {

using nvr::kWave;

template <int K, bool ADD, bool GATHER = false>
__global__ __launch_bounds__(256) void rms_rows_fast(const uint16_t* __restrict__ x, uint16_t* __restrict__ residual,
                                                     const uint16_t* __restrict__ weight, uint16_t* __restrict__ out,
                                                     int rows, int hidden, float eps,
                                                     const int* __restrict__ index = nullptr, int input_rows = 0) {
    const int lane = threadIdx.x & (kWave - 1);
    const int m = lane & 31;
    const int64_t row = (int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave) * 2 + (lane >> 5);
    int64_t src = row;
    bool active = row < rows;
    if constexpr (GATHER) {
        src = active ? index[row] : -1;
        if (active && (src < 0 || src >= input_rows)) {  // the gather's +0 row
#pragma unroll
            for (int k = 0; k < K; ++k) nvr::store_stream(out + row * hidden + 8 * m + 256 * k, make_uint4(0, 0, 0, 0));
            active = false;
        }
    }
    const int64_t base = src * hidden + 8 * m;     // input and residual row
    const int64_t obase = row * hidden + 8 * m;    // output row

    float v[K][8];
    if (active) {
        uint4 xw[K];
#pragma unroll
        for (int k = 0; k < K; ++k) xw[k] = nvr::load_stream(x + base + 256 * k);
        if constexpr (ADD) {
            uint4 rw[K];
#pragma unroll
            for (int k = 0; k < K; ++k) rw[k] = nvr::load_stream(residual + base + 256 * k);
#pragma unroll
            for (int k = 0; k < K; ++k) {
                float a[8], b[8];
                nvr::unpack8(xw[k], a);
                nvr::unpack8(rw[k], b);
#pragma unroll
                for (int i = 0; i < 8; ++i) v[k][i] = a[i] + b[i];
            }
        } else {
#pragma unroll
            for (int k = 0; k < K; ++k) nvr::unpack8(xw[k], v[k]);
        }
    } else {
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int i = 0; i < 8; ++i) v[k][i] = 0.0f;
    }

    // Per reference thread 8m+i: s = fma(v_k, v_k, s) for k = 0..K-1.
    float s[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) acc = __builtin_fmaf(v[k][i], v[k][i], acc);
        s[i] = acc;
    }
    // Warp tree: offsets 16 and 8 cross lanes, 4/2/1 stay in the lane.
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] = s[i] + nvr::xor_lane(s[i], 2);
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] = s[i] + nvr::xor_lane(s[i], 1);
    float total = ((s[0] + s[4]) + (s[2] + s[6])) + ((s[1] + s[5]) + (s[3] + s[7]));
    // Block tree over the 8 warp sums (lanes 0,4,...,28 of the half).
    total = total + nvr::xor_lane(total, 16);
    total = total + nvr::xor_lane(total, 8);
    total = total + nvr::xor_lane(total, 4);

    const float inv = nvr::inv_sqrt_rn(total / float(hidden) + eps);
    if (!active) return;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        float wf[8], o[8];
        nvr::unpack8(*reinterpret_cast<const uint4*>(weight + 256 * k + 8 * m), wf);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (v[k][i] * inv) * wf[i];
        if constexpr (ADD && !GATHER) nvr::store_stream(residual + base + 256 * k, nvr::pack8_split(v[k]));
        nvr::store_stream(out + obase + 256 * k, nvr::pack8_split(o));
    }
}

// Any hidden size, 2-byte alignment. One row per wave; lane l plays reference
// threads 4l..4l+3: warp w = lanes 8w..8w+7, so warp level 16 -> lane ^4,
// 8 -> ^2, 4 -> ^1, 2/1 in-lane; block level 4 -> ^32, 2 -> ^16, 1 -> ^8.
template <bool ADD, bool GATHER = false>
__global__ __launch_bounds__(256) void rms_rows_generic(const uint16_t* __restrict__ x, uint16_t* __restrict__ residual,
                                                        const uint16_t* __restrict__ weight,
                                                        uint16_t* __restrict__ out, int rows, int hidden, float eps,
                                                        const int* __restrict__ index = nullptr, int input_rows = 0) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;  // whole wave exits together
    int64_t src = row;
    if constexpr (GATHER) {
        src = index[row];
        if (src < 0 || src >= input_rows) {  // the gather's +0 row
            for (int j = lane; j < hidden; j += kWave) out[row * hidden + j] = 0;
            return;
        }
    }
    const int64_t base = src * hidden, obase = row * hidden;
    float s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float acc = 0.0f;
        for (int j = 4 * lane + i; j < hidden; j += 256) {
            float v = nvr::bf16_to_f32(x[base + j]);
            if constexpr (ADD) v += nvr::bf16_to_f32(residual[base + j]);
            acc = __builtin_fmaf(v, v, acc);
        }
        s[i] = acc;
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
    const float inv = nvr::inv_sqrt_rn(total / float(hidden) + eps);
    for (int j = lane; j < hidden; j += kWave) {
        float v = nvr::bf16_to_f32(x[base + j]);
        if constexpr (ADD) {
            v += nvr::bf16_to_f32(residual[base + j]);
            if constexpr (!GATHER) residual[base + j] = nvr::f32_to_bf16(v);
        }
        out[obase + j] = nvr::f32_to_bf16((v * inv) * nvr::bf16_to_f32(weight[j]));
    }
}

template <int K, bool ADD, bool GATHER>
void launch_fast(hipStream_t stream, const uint16_t* x, uint16_t* res, const uint16_t* w, uint16_t* out, int rows,
                 int hidden, float eps, const int* index, int input_rows) {
    const int rows_per_block = 8;  // 4 waves x 2 rows
    const unsigned blocks = unsigned((int64_t(rows) + rows_per_block - 1) / rows_per_block);
    hipLaunchKernelGGL((rms_rows_fast<K, ADD, GATHER>), dim3(blocks), dim3(256), 0, stream, x, res, w, out, rows,
                       hidden, eps, index, input_rows);
}

template <bool ADD, bool GATHER = false>
int launch_rms(nv_context* c, const void* xv, void* resv, const void* wv, void* outv, int rows, int hidden,
               float eps, const int* index = nullptr, int input_rows = 0) {
    NVR_ACTIVATE(c);
    if (rows <= 0 || hidden <= 0) return nvr::fail(-2, "rms: rows and hidden must be positive");
    if (GATHER && input_rows <= 0) return nvr::fail(-2, "add_rms_gather: input rows must be positive");
    auto x = static_cast<const uint16_t*>(xv);
    auto res = static_cast<uint16_t*>(resv);
    auto w = static_cast<const uint16_t*>(wv);
    auto out = static_cast<uint16_t*>(outv);
    const bool vec = hidden % 256 == 0 && nvr::aligned(x, 16) && nvr::aligned(w, 16) && nvr::aligned(out, 16) &&
                     (!ADD || nvr::aligned(res, 16));
    const int K = hidden / 256;
    if (vec && (K == 1 || K == 2 || K == 3 || K == 4 || K == 5 || K == 6 || K == 8 || K == 10 || K == 12 ||
                K == 14 || K == 16 || K == 20)) {
        hipStream_t s = c->stream;
        switch (K) {
            case 1: launch_fast<1, ADD, GATHER>(s, x, res, w, out, rows, hidden, eps, index, input_rows); break;
            case 2: launch_fast<2, ADD, GATHER>(s, x, res, w, out, rows, hidden, eps, index, input_rows); break;
            case 3: launch_fast<3, ADD, GATHER>(s, x, res, w, out, rows, hidden, eps, index, input_rows); break;
            case 4: launch_fast<4, ADD, GATHER>(s, x, res, w, out, rows, hidden, eps, index, input_rows); break;
            case 5: launch_fast<5, ADD, GATHER>(s, x, res, w, out, rows, hidden, eps, index, input_rows); break;
            case 6: launch_fast<6, ADD, GATHER>(s, x, res, w, out, rows, hidden, eps, index, input_rows); break;
            case 8: launch_fast<8, ADD, GATHER>(s, x, res, w, out, rows, hidden, eps, index, input_rows); break;
            case 10: launch_fast<10, ADD, GATHER>(s, x, res, w, out, rows, hidden, eps, index, input_rows); break;
            case 12: launch_fast<12, ADD, GATHER>(s, x, res, w, out, rows, hidden, eps, index, input_rows); break;
            case 14: launch_fast<14, ADD, GATHER>(s, x, res, w, out, rows, hidden, eps, index, input_rows); break;
            case 16: launch_fast<16, ADD, GATHER>(s, x, res, w, out, rows, hidden, eps, index, input_rows); break;
            default: launch_fast<20, ADD, GATHER>(s, x, res, w, out, rows, hidden, eps, index, input_rows); break;
        }
    } else {
        const unsigned blocks = unsigned((int64_t(rows) + 3) / 4);
        hipLaunchKernelGGL((rms_rows_generic<ADD, GATHER>), dim3(blocks), dim3(256), 0, c->stream, x, res, w, out,
                           rows, hidden, eps, index, input_rows);
    }
    return nvr::launch_status();
}

}  // namespace

extern "C" {

int nv_rms(nv_context* c, const void* x, const void* weight, void* out, int rows, int hidden, float eps) {
    return launch_rms<false>(c, x, nullptr, weight, out, rows, hidden, eps);
}

int nv_add_rms(nv_context* c, const void* x, void* residual, const void* weight, void* out, int rows, int hidden,
               float eps) {
    return launch_rms<true>(c, x, residual, weight, out, rows, hidden, eps);
}

int nv_add_rms_gather(nv_context* c, const void* x, const void* residual, const void* weight, const void* indices,
                      void* out, int rows, int hidden, int input_rows, float eps) {
    // The gather form never writes the residual (the kernel's pointer is
    // non-const only for the shared template).
    return launch_rms<true, true>(c, x, const_cast<void*>(residual), weight, out, rows, hidden, eps,
                                  static_cast<const int*>(indices), input_rows);
}

}  // extern "C"
