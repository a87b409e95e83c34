// RMSNorm (or residual-add + RMSNorm) fused into the GEMM that consumes it,
// for decode-sized batches (nv_rms_gemm).
//
// Semantics: the norm of kernels/kernels.cu:145-164 (nv_rms / nv_add_rms,
// bit for bit: the same arithmetic and summation order as norm.hip) followed
// by the GEMM of :98-106, Y[m, n] = bf16(sum_k X[m, k] W[n, k]) with fp32
// accumulation, where X is the norm's bf16 output. This is the pair
// src/model.rs:659-678 (input norm, qkv projection) and :753-770
// (post-attention norm, gate_up projection) in one launch.
//
// Why: at 8-32 decode rows a norm is one memory round trip plus a launch
// (~3.5 us) and the GEMM that follows streams its weights in a few us; fusing
// them removes a launch and overlaps the norm with the weight stream.
//
// Layout (W = 4 or 8 waves, column tile of 16 outputs per block, n / 16
// blocks):
//  1. Each half-wave issues the loads of its first input row (x, residual),
//     then every wave its share of the tile's weights: wave w owns the k range
//     [w k/W, (w+1) k/W) and lane l loads, for each 32-wide k step, the 16
//     bytes W[n0 + l % 16][k0 + 8 (l / 16) ..] — the B operand layout of
//     v_mfma_f32_16x16x32_bf16 (B[k][j] with k = 8 (l / 16) + e, j = l % 16).
//     Loads retire in issue order, so the norm waits only for its rows.
//  2. While the weights stream in, the block normalises the m input rows (one
//     row per half-wave per pass of 2W rows, the layout and reduction tree of
//     norm.hip's rms_rows_fast) into an LDS tile X[16 or 32][k] (rows >= m
//     zero). Block 0 also writes residual_out (bf16(x + residual)) and, when
//     asked, the normalised rows.
//  3. Each wave runs its k steps on MFMA: A = X[l % 16 (+16)][k0 + 8 (l / 16) ..]
//     from LDS, one accumulator tile per 16 rows.
//  4. The W waves' partial tiles are summed through LDS in wave order and
//     rounded once to bf16.
// The GEMM's summation order (MFMA's, then the W k slices in order, W fixed
// by n) is fixed, so every launch of a shape gives the same bits; it is not hipBLAS's order, so
// the result matches nv_gemm's to fp32 rounding (checked against the float64
// product's bound), while the norm outputs match the oracle bit for bit.
// The residual is read from one buffer and written to another: a block that
// updated it in place would race with blocks still reading it.
#include "../../include/nano_hip.h"
#include "nvr_device.h"
#include "nvr_internal.h"

namespace {

using nvr::kWave;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTileN = 16;      // output columns per block (MFMA N)
constexpr int kMaxRows = 32;    // two MFMA row tiles
constexpr int kRowPad = 8;      // bf16 elements of padding per LDS row (spreads the A reads over the banks)

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8_t, v); }

// KC = k / 256 (16-byte chunks per lane of a half-wave row); MT = row tiles.
// SILU: w is the gate_up weight with its rows in tile order (tile t = gate
// rows 8t..8t+7, then up rows 8t..8t+7; n = 2 * inter), y (when not null)
// receives gate_up in the reference's [gate | up] column order, and
// act[m, 8t + j] = bf16(silu(gate) * up) of the tile's bf16 outputs.
template <int KC, int MT, bool ADD, bool SILU, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void rms_gemm(const uint16_t* __restrict__ x,
                                                     const uint16_t* __restrict__ residual,
                                                     uint16_t* __restrict__ residual_out,
                                                     const uint16_t* __restrict__ norm_weight,
                                                     const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
                                                     uint16_t* __restrict__ normed, int m, int n, float eps,
                                                     uint16_t* __restrict__ act, int inter) {
    constexpr int K = 256 * KC, KW = K / WAVES, STEPS = KW / 32, LDX = K + kRowPad, ROWS = 2 * WAVES;
    extern __shared__ __align__(16) unsigned char smem[];
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);                          // [MT * 16][LDX]
    float* red = reinterpret_cast<float*>(smem + sizeof(uint16_t) * MT * 16 * LDX);  // [WAVES][MT][256]
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int n0 = blockIdx.x * kTileN;

    // 1. The first pass's input rows, then the tile's weights: all in flight
    // before anything waits, and the norm (which waits only for the rows,
    // issued first) overlaps the weight stream.
    const int half = lane >> 5, hm = lane & 31;
    const bool writer = blockIdx.x == 0;
    const int passes = (m + ROWS - 1) / ROWS;  // uniform; rows of a pass: pass * ROWS + (wave * 2 + half)
    auto row_of = [&](int pass) { return pass * ROWS + wave * 2 + half; };
    auto base_of = [&](int pass) { return int64_t(row_of(pass) < m ? row_of(pass) : 0) * K + 8 * hm; };
    uint4 xw[KC], rw[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) xw[c] = nvr::load_stream(x + base_of(0) + 256 * c);
    if constexpr (ADD) {
#pragma unroll
        for (int c = 0; c < KC; ++c) rw[c] = *reinterpret_cast<const uint4*>(residual + base_of(0) + 256 * c);
    }
    // 4-wave blocks (two share a CU) issue the norm weight here too: loads
    // retire in issue order, so issued after the tile's weights it would hold
    // the norm until the whole stream is in (gate_up at 8 rows: 7.28 -> 6.86
    // us). With one 8-wave block per CU the MFMA waits for the stream anyway,
    // and the extra loads only delay it (qkv at 8 rows: 5.08 -> 5.23 us).
    constexpr bool kEarlyNorm = WAVES == 4;
    uint4 nwv[KC];
    if constexpr (kEarlyNorm) {
#pragma unroll
        for (int c = 0; c < KC; ++c) nwv[c] = *reinterpret_cast<const uint4*>(norm_weight + 256 * c + 8 * hm);
    }
    const int kb = wave * KW;
    uint4 wv[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
        wv[s] = nvr::load_stream(w + int64_t(n0 + lane % 16) * K + kb + 32 * s + 8 * (lane / 16));

    // 2. The norm of every input row into LDS (rms_rows_fast's arithmetic);
    // row tiles past the last pass are zero.
    if (passes * ROWS < MT * 16) {
        for (int i = threadIdx.x; i < (MT * 16 - passes * ROWS) * (K / 8); i += WAVES * 64) {
            const int row = passes * ROWS + i / (K / 8), col = 8 * (i % (K / 8));
            *reinterpret_cast<uint4*>(xs + row * LDX + col) = make_uint4(0, 0, 0, 0);
        }
    }
#pragma unroll
    for (int pass = 0; pass < (MT * 16 + ROWS - 1) / ROWS; ++pass) {
        if (pass >= passes) break;  // uniform
        const int row = row_of(pass);
        const bool active = row < m;
        const int64_t base = base_of(pass);
        if (pass > 0) {
#pragma unroll
            for (int c = 0; c < KC; ++c) xw[c] = nvr::load_stream(x + base + 256 * c);
            if constexpr (ADD) {
#pragma unroll
                for (int c = 0; c < KC; ++c) rw[c] = *reinterpret_cast<const uint4*>(residual + base + 256 * c);
            }
        }
        float v[KC][8];
        if constexpr (ADD) {
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                float a[8], b[8];
                nvr::unpack8(xw[c], a);
                nvr::unpack8(rw[c], b);
#pragma unroll
                for (int i = 0; i < 8; ++i) v[c][i] = active ? a[i] + b[i] : 0.0f;
            }
        } else {
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                nvr::unpack8(xw[c], v[c]);
#pragma unroll
                for (int i = 0; i < 8; ++i) v[c][i] = active ? v[c][i] : 0.0f;
            }
        }
        float s[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float acc = 0.0f;
#pragma unroll
            for (int c = 0; c < KC; ++c) acc = __builtin_fmaf(v[c][i], v[c][i], acc);
            s[i] = acc;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) s[i] = s[i] + nvr::xor_lane(s[i], 2);
#pragma unroll
        for (int i = 0; i < 8; ++i) s[i] = s[i] + nvr::xor_lane(s[i], 1);
        float total = ((s[0] + s[4]) + (s[2] + s[6])) + ((s[1] + s[5]) + (s[3] + s[7]));
        total = total + nvr::xor_lane(total, 16);
        total = total + nvr::xor_lane(total, 8);
        total = total + nvr::xor_lane(total, 4);
        const float inv = nvr::inv_sqrt_rn(total / float(K) + eps);
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            float wf[8], o[8];
            nvr::unpack8(kEarlyNorm ? nwv[c] : *reinterpret_cast<const uint4*>(norm_weight + 256 * c + 8 * hm), wf);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = (v[c][i] * inv) * wf[i];
            const uint4 ob = active ? nvr::pack8_split(o) : make_uint4(0, 0, 0, 0);
            *reinterpret_cast<uint4*>(xs + row * LDX + 256 * c + 8 * hm) = ob;
            if (writer && active) {
                if (ADD && residual_out != nullptr)
                    nvr::store_stream(residual_out + base + 256 * c, nvr::pack8_split(v[c]));
                if (normed != nullptr) nvr::store_stream(normed + base + 256 * c, ob);
            }
        }
    }
    __syncthreads();

    // 3. This wave's k quarter on MFMA.
    f32x4_t acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
        const int kk = kb + 32 * s + 8 * (lane / 16);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const uint4 a = *reinterpret_cast<const uint4*>(xs + (t * 16 + lane % 16) * LDX + kk);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(wv[s]), acc[t], 0, 0, 0);
        }
    }

    // 4. Sum the four quarters in wave order; lane l holds D[4 (l / 16) + r][l % 16].
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wave * MT + t) * 256 + (4 * (lane / 16) + r) * 16 + lane % 16] = acc[t][r];
    __syncthreads();
    // Output (t, e): tile t, element e = 16 i + j; wave-uniform trip count.
    for (int idx = threadIdx.x; idx < MT * 256; idx += WAVES * 64) {
        const int t = idx / 256, e = idx % 256;
        const int i = e / 16, j = e % 16, row = t * 16 + i;
        float sum = red[(0 * MT + t) * 256 + e];
#pragma unroll
        for (int q = 1; q < WAVES; ++q) sum += red[(q * MT + t) * 256 + e];
        const uint16_t yb = nvr::f32_to_bf16(sum);
        if constexpr (SILU) {
            // Column j of tile b = blockIdx.x: gate index 8b + j (j < 8) or
            // up index 8b + j - 8; lane j ^ 8 of the same 16-lane group
            // holds the partner.
            const int idx = 8 * int(blockIdx.x) + (j & 7);
            const float own = nvr::bf16_to_f32(yb), partner = nvr::xor_lane(own, 8);
            if (row < m) {
                if (y != nullptr) y[int64_t(row) * n + (j < 8 ? idx : inter + idx)] = yb;
                if (j < 8) act[int64_t(row) * inter + idx] = nvr::f32_to_bf16(nvr::silu_mul(own, partner));
            }
        } else {
            if (row < m) y[int64_t(row) * n + n0 + j] = yb;
        }
    }
}

// Blocks of 8 waves when the grid is at most one block per CU (n <= 4096 on
// MI355X's 256 CUs: more loads in flight per CU, and for 32 rows two passes
// of the norm instead of four); 4 waves when it is wider, where two smaller
// blocks per CU (LDS permitting) hide each other's norm.
inline int64_t cus_of(const nv_context* c) { return c->cu_count > 0 ? c->cu_count : 256; }

template <int KC, int MT, bool ADD, bool SILU, int WAVES>
void launch_waves(nv_context* c, const uint16_t* x, const uint16_t* res, uint16_t* res_out, const uint16_t* nw,
                  const uint16_t* w, uint16_t* y, uint16_t* normed, int m, int n, float eps, uint16_t* act) {
    constexpr int K = 256 * KC;
    const size_t lds = sizeof(uint16_t) * MT * 16 * (K + kRowPad) + sizeof(float) * WAVES * MT * 256;
    hipLaunchKernelGGL((rms_gemm<KC, MT, ADD, SILU, WAVES>), dim3(unsigned(n / kTileN)), dim3(WAVES * 64), lds,
                       c->stream, x, res, res_out, nw, w, y, normed, m, n, eps, act, n / 2);
}

template <int KC, int MT, bool ADD, bool SILU>
void launch(nv_context* c, const uint16_t* x, const uint16_t* res, uint16_t* res_out, const uint16_t* nw,
            const uint16_t* w, uint16_t* y, uint16_t* normed, int m, int n, float eps, uint16_t* act) {
    if (n / kTileN <= cus_of(c)) launch_waves<KC, MT, ADD, SILU, 8>(c, x, res, res_out, nw, w, y, normed, m, n, eps, act);
    else launch_waves<KC, MT, ADD, SILU, 4>(c, x, res, res_out, nw, w, y, normed, m, n, eps, act);
}

template <int KC, bool SILU>
void launch_rows(nv_context* c, const uint16_t* x, const uint16_t* res, uint16_t* res_out, const uint16_t* nw,
                 const uint16_t* w, uint16_t* y, uint16_t* normed, int m, int n, float eps, uint16_t* act) {
    const bool add = res != nullptr;
    if (m <= 16) {
        add ? launch<KC, 1, true, SILU>(c, x, res, res_out, nw, w, y, normed, m, n, eps, act)
            : launch<KC, 1, false, SILU>(c, x, res, res_out, nw, w, y, normed, m, n, eps, act);
    } else {
        add ? launch<KC, 2, true, SILU>(c, x, res, res_out, nw, w, y, normed, m, n, eps, act)
            : launch<KC, 2, false, SILU>(c, x, res, res_out, nw, w, y, normed, m, n, eps, act);
    }
}

// Plain decode-sized GEMM (nv_gemm_rows): Y[m, n] = bf16(X W^T), m <= 32.
// A block of WAVES waves owns a column tile of 16 and splits k over its
// waves; each wave loads its W and X pieces straight into the MFMA operand
// layouts (rows >= m read row m - 1 and are zeroed), all before the first
// MFMA, and the partial tiles are summed through LDS in wave order. 4-wave
// blocks serve wide outputs; outputs with fewer 16-column tiles than CUs take
// gemm_narrow below 17 rows and 16-wave blocks (each streaming its tile's
// whole k with 16 waves of loads in flight) from 17 rows.
template <int WAVES, int STEPS, int MT>
__global__ __launch_bounds__(WAVES * 64) void gemm_rows(const uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
                                                        int m, int n, int k) {
    __shared__ float red[WAVES][MT][256];
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int n0 = blockIdx.x * kTileN;
    const int kb = wave * (32 * STEPS) + 8 * (lane / 16);
    uint4 wv[STEPS], xv[MT][STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) wv[s] = nvr::load_stream(w + int64_t(n0 + lane % 16) * k + kb + 32 * s);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int row = t * 16 + lane % 16;
        const int64_t base = int64_t(row < m ? row : m - 1) * k + kb;
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
            const uint4 v = *reinterpret_cast<const uint4*>(x + base + 32 * s);
            xv[t][s] = row < m ? v : make_uint4(0, 0, 0, 0);
        }
    }
    f32x4_t acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
#pragma unroll
        for (int t = 0; t < MT; ++t)
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xv[t][s]), as_bf16x8(wv[s]), acc[t], 0, 0, 0);
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][t][(4 * (lane / 16) + r) * 16 + lane % 16] = acc[t][r];
    __syncthreads();
    for (int idx = threadIdx.x; idx < MT * 256; idx += WAVES * 64) {
        const int t = idx / 256, e = idx % 256, row = t * 16 + e / 16;
        float sum = red[0][t][e];
#pragma unroll
        for (int q = 1; q < WAVES; ++q) sum += red[q][t][e];
        if (row < m) y[int64_t(row) * n + n0 + e % 16] = nvr::f32_to_bf16(sum);
    }
}

// Narrow decode GEMM (nv_gemm_rows when n / 16 column tiles leave most CUs
// idle, as n = 1024 does with 64): one block per NC = 32 / MR output columns
// (n = 1024: 256 blocks at m <= 8, 512 at m <= 16) and one thread per
// 16-byte chunk of k (THREADS = k / 8). A thread loads its chunk of the NC
// weight rows and of the MR input rows (rows >= m repeat row m - 1 and are
// never written), forms the MR * NC partial dot products in k order with
// v_dot2_f32_bf16 (four per chunk), and stores them to LDS. Then FIN threads
// per output sum the partials of chunks p, p + FIN, ... in order and fold
// across their FIN lanes with DPP (lane ^ 1, lane ^ 2, then the other half of
// the 8-lane group). The order is fixed, so every launch gives the same bits.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

template <int MR, int THREADS>
__global__ __launch_bounds__(THREADS) void gemm_narrow(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                       uint16_t* __restrict__ y, int m, int n, int k) {
    constexpr int NC = 32 / MR, OUT = 32, FIN = THREADS >= 256 ? 8 : 4, PER = THREADS / FIN;
    constexpr int LDP = THREADS + 8;  // row pitch: the 8 outputs a wave folds start in different banks
    static_assert(OUT * FIN <= THREADS && THREADS % 64 == 0, "gemm_narrow block shape");
    __shared__ float part[OUT * LDP];
    const int t = threadIdx.x;
    const int c0 = blockIdx.x * NC;
    uint4 wv[NC], xv[MR];
#pragma unroll
    for (int c = 0; c < NC; ++c) wv[c] = nvr::load_stream(w + int64_t(c0 + c) * k + 8 * t);
#pragma unroll
    for (int r = 0; r < MR; ++r) xv[r] = *reinterpret_cast<const uint4*>(x + int64_t(r < m ? r : m - 1) * k + 8 * t);
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            float acc = dot2(xv[r].x, wv[c].x, 0.0f);
            acc = dot2(xv[r].y, wv[c].y, acc);
            acc = dot2(xv[r].z, wv[c].z, acc);
            acc = dot2(xv[r].w, wv[c].w, acc);
            part[(r * NC + c) * LDP + t] = acc;
        }
    __syncthreads();
    if (t < OUT * FIN) {
        const int o = t / FIN, p = t % FIN;
        const float* src = part + o * LDP + p;
        float s = src[0];
#pragma unroll
        for (int i = 1; i < PER; ++i) s += src[i * FIN];
        s += nvr::dpp<nvr::kDppQuadXor1>(s);
        s += nvr::dpp<nvr::kDppQuadXor2>(s);
        if constexpr (FIN == 8) s += nvr::dpp<nvr::kDppRowHalfMirror>(s);
        const int r = o / NC;
        if (p == 0 && r < m) y[int64_t(r) * n + c0 + o % NC] = nvr::f32_to_bf16(s);
    }
}

template <int MR>
void launch_narrow(nv_context* c, const uint16_t* x, const uint16_t* w, uint16_t* y, int m, int n, int k) {
    const dim3 grid(unsigned(n / (32 / MR)));
    switch (k) {
        case 1024: hipLaunchKernelGGL((gemm_narrow<MR, 128>), grid, dim3(128), 0, c->stream, x, w, y, m, n, k); break;
        case 2048: hipLaunchKernelGGL((gemm_narrow<MR, 256>), grid, dim3(256), 0, c->stream, x, w, y, m, n, k); break;
        case 3072: hipLaunchKernelGGL((gemm_narrow<MR, 384>), grid, dim3(384), 0, c->stream, x, w, y, m, n, k); break;
        default: hipLaunchKernelGGL((gemm_narrow<MR, 512>), grid, dim3(512), 0, c->stream, x, w, y, m, n, k); break;
    }
}

template <int WAVES, int STEPS>
void launch_rows_plain(nv_context* c, const uint16_t* x, const uint16_t* w, uint16_t* y, int m, int n, int k) {
    const dim3 grid(unsigned(n / kTileN)), block(WAVES * 64);
    if (m <= 16) hipLaunchKernelGGL((gemm_rows<WAVES, STEPS, 1>), grid, block, 0, c->stream, x, w, y, m, n, k);
    else hipLaunchKernelGGL((gemm_rows<WAVES, STEPS, 2>), grid, block, 0, c->stream, x, w, y, m, n, k);
}

template <bool SILU>
int launch_rms_gemm(nv_context* c, const void* x, const void* residual, void* residual_out, const void* norm_weight,
                    const void* w, void* y, void* normed, int m, int n, int k, float eps, void* act) {
    NVR_ACTIVATE(c);
    if (m <= 0 || m > kMaxRows || n <= 0 || n % kTileN != 0)
        return nvr::fail(-2, "rms_gemm: needs 1 <= m <= 32 rows and n a positive multiple of 16 (m %d, n %d)", m, n);
    if (SILU && act == nullptr) return nvr::fail(-2, "rms_gemm_silu: the activation output is required");
    if (!SILU && y == nullptr) return nvr::fail(-2, "rms_gemm: the output y is required");
    if (k != 512 && k != 1024 && k != 2048)
        return nvr::fail(-2, "rms_gemm: k must be 512, 1024 or 2048 (k %d)", k);
    if (residual == nullptr && residual_out != nullptr)
        return nvr::fail(-2, "rms_gemm: residual_out needs a residual to add");
    if (!nvr::aligned(x, 16) || !nvr::aligned(residual, 16) || !nvr::aligned(residual_out, 16) ||
        !nvr::aligned(norm_weight, 16) || !nvr::aligned(w, 16) || !nvr::aligned(normed, 16))
        return nvr::fail(-2, "rms_gemm: x, residual, residual_out, norm_weight, w and normed must be 16-byte aligned");
    auto xb = static_cast<const uint16_t*>(x);
    auto rb = static_cast<const uint16_t*>(residual);
    auto ro = static_cast<uint16_t*>(residual_out);
    auto nw = static_cast<const uint16_t*>(norm_weight);
    auto wb = static_cast<const uint16_t*>(w);
    auto yb = static_cast<uint16_t*>(y);
    auto nb = static_cast<uint16_t*>(normed);
    auto ab = static_cast<uint16_t*>(act);
    switch (k) {
        case 512: launch_rows<2, SILU>(c, xb, rb, ro, nw, wb, yb, nb, m, n, eps, ab); break;
        case 1024: launch_rows<4, SILU>(c, xb, rb, ro, nw, wb, yb, nb, m, n, eps, ab); break;
        default: launch_rows<8, SILU>(c, xb, rb, ro, nw, wb, yb, nb, m, n, eps, ab); break;
    }
    return nvr::launch_status();
}

}  // namespace

extern "C" {

int nv_rms_gemm(nv_context* c, const void* x, const void* residual, void* residual_out, const void* norm_weight,
                const void* w, void* y, void* normed, int m, int n, int k, float eps) {
    return launch_rms_gemm<false>(c, x, residual, residual_out, norm_weight, w, y, normed, m, n, k, eps, nullptr);
}

int nv_gemm_rows(nv_context* c, const void* x, const void* w, void* y, int m, int n, int k) {
    NVR_ACTIVATE(c);
    if (m <= 0 || m > kMaxRows || n <= 0 || n % kTileN != 0)
        return nvr::fail(-2, "gemm_rows: needs 1 <= m <= 32 rows and n a positive multiple of 16 (m %d, n %d)", m, n);
    if (k != 1024 && k != 2048 && k != 3072 && k != 4096)
        return nvr::fail(-2, "gemm_rows: k must be 1024, 2048, 3072 or 4096 (k %d)", k);
    if (!nvr::aligned(x, 16) || !nvr::aligned(w, 16))
        return nvr::fail(-2, "gemm_rows: x and w must be 16-byte aligned");
    auto xb = static_cast<const uint16_t*>(x);
    auto wb = static_cast<const uint16_t*>(w);
    auto yb = static_cast<uint16_t*>(y);
    if (n / kTileN < cus_of(c) && m <= 16) {  // too few 16-column tiles to fill the GPU
        if (m <= 8) launch_narrow<8>(c, xb, wb, yb, m, n, k);
        else launch_narrow<16>(c, xb, wb, yb, m, n, k);
    } else if (n / kTileN >= cus_of(c) && k <= 2048) {  // enough tiles to fill the GPU with 4-wave blocks
        if (k == 1024) launch_rows_plain<4, 8>(c, xb, wb, yb, m, n, k);
        else launch_rows_plain<4, 16>(c, xb, wb, yb, m, n, k);
    } else {
        switch (k) {
            case 1024: launch_rows_plain<16, 2>(c, xb, wb, yb, m, n, k); break;
            case 2048: launch_rows_plain<16, 4>(c, xb, wb, yb, m, n, k); break;
            case 3072: launch_rows_plain<16, 6>(c, xb, wb, yb, m, n, k); break;
            default: launch_rows_plain<16, 8>(c, xb, wb, yb, m, n, k); break;
        }
    }
    return nvr::launch_status();
}

int nv_rms_gemm_silu(nv_context* c, const void* x, const void* residual, void* residual_out,
                     const void* norm_weight, const void* w_tiled, void* gate_up, void* act, void* normed, int m,
                     int intermediate, int k, float eps) {
    if (intermediate <= 0 || intermediate % 8 != 0) {
        NVR_ACTIVATE(c);
        return nvr::fail(-2, "rms_gemm_silu: intermediate must be a positive multiple of 8 (%d)", intermediate);
    }
    return launch_rms_gemm<true>(c, x, residual, residual_out, norm_weight, w_tiled, gate_up, normed, m,
                                 2 * intermediate, k, eps, act);
}

}  // extern "C"
