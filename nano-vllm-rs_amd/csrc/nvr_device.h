// Device-side helpers shared by every nano-vllm-rs fused kernel on gfx950.
//
// Numerics contract (all sources are compiled with -ffp-contract=off, so every
// a*b+c below is two roundings unless written as __builtin_fmaf):
//  * bf16 is the upper half of an IEEE binary32; widening is exact and
//    narrowing is round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
//  * nvr_logf is a deterministic logarithm (range reduction to
//    [sqrt(1/2), sqrt(2)) plus a degree-8 polynomial evaluated with explicit
//    FMAs). It uses only correctly rounded IEEE operations, so the host oracle
//    reproduces it bit for bit; its error is below 1 ulp over all positive
//    normal floats.
//  * The RoPE angle helpers evaluate pow/sin/cos in binary64 with fixed
//    operation sequences, again reproducible on the host.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nvr {

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 ----
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}
// Two floats -> two bf16 in one dword (lo in bits 0..15), round to nearest
// even. pack_bf16x2 is one two-source v_cvt_pk_bf16_f32; pack_bf16x2_split
// converts each half on its own and merges them. Both give the same bits;
// which one schedules better is kernel-specific (measured per kernel).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f32x2_t f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}
__device__ __forceinline__ uint32_t pack_bf16x2_split(float lo, float hi) {
    return uint32_t(f32_to_bf16(lo)) | (uint32_t(f32_to_bf16(hi)) << 16);
}
// Widen 8 packed bf16 (one 16-byte load) into floats.
__device__ __forceinline__ void unpack8(const uint4& w, float* f) {
    f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
    f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
    f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
    f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}
__device__ __forceinline__ uint4 pack8(const float* f) {
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]),
                      pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7]));
}
__device__ __forceinline__ uint4 pack8_split(const float* f) {
    return make_uint4(pack_bf16x2_split(f[0], f[1]), pack_bf16x2_split(f[2], f[3]),
                      pack_bf16x2_split(f[4], f[5]), pack_bf16x2_split(f[6], f[7]));
}

// Streaming 16-byte accesses (non-temporal hint on the global load/store) for
// data each launch touches exactly once; on MI355X they keep the caches for
// the reused operands and raise copy bandwidth by roughly 7-40% per kernel.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load(static_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store_stream(void* p, const uint4& v) {
    const u32x4_t w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, static_cast<u32x4_t*>(p));
}

// SiLU(g) * u for nv_silu and the SiLU epilogue of nv_rms_gemm_silu (one
// definition, so both give the same bits): the hardware base-2 exponential and
// reciprocal, with the IEEE division where 1 + exp(-g) >= 2^126 (there the
// quotient is subnormal and the reciprocal would flush).
__device__ __forceinline__ float silu_mul(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896340736f);
    const float d = 1.0f + e;
    const float act = d < 0x1.0p126f ? g * __builtin_amdgcn_rcpf(d) : g / d;
    return act * u;
}

// Round a float to bf16 precision and widen it back (the value a bf16 store
// followed by a load would produce).
__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// -------------------------------------------------------- cross-lane ops ----
// DPP lane permutations (data-parallel primitives: the operand is read from
// another lane of the same 16-lane row, no LDS traffic, and the compiler folds
// the move into the consuming VALU op when it can).
constexpr int kDppQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppQuadReverse = 0x1B;    // quad_perm [3,2,1,0]: lane ^ 3
constexpr int kDppRowRor8 = 0x128;       // row_ror:8 : lane ^ 8 inside a 16-lane row
constexpr int kDppRowHalfMirror = 0x141; // row_half_mirror: lane i <-> 7-i inside each 8 lanes
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, 0xF, 0xF, false));
}

// Butterfly exchange with lane ^ mask inside a wave64 (every lane active).
// For an IEEE sum the butterfly leaves every lane with the same bits as the
// down-shift tree's lane 0, because each level adds the same two operands
// (a+b == b+a). Masks 1, 2 and 8 are one DPP move, 4 two (the 8-lane mirror
// i <-> 7-i, then the quad reversal j <-> j ^ 3: i ^ 4 in all), 16 a swizzle
// inside each 32-lane half; only 32 goes through the LDS crossbar.
__device__ __forceinline__ uint32_t xor_lane_bits(uint32_t v, int mask) {
    switch (mask) {
        case 1: return dpp<kDppQuadXor1>(v);
        case 2: return dpp<kDppQuadXor2>(v);
        case 4: return dpp<kDppQuadReverse>(dpp<kDppRowHalfMirror>(v));
        case 8: return dpp<kDppRowRor8>(v);
        case 16: return uint32_t(__builtin_amdgcn_ds_swizzle(int(v), 0x401F));  // bitmask mode: and 0x1f, xor 0x10
        default: return uint32_t(__shfl_xor(int(v), mask, kWave));
    }
}
__device__ __forceinline__ float xor_lane(float v, int mask) {
    return __uint_as_float(xor_lane_bits(__float_as_uint(v), mask));
}
__device__ __forceinline__ int xor_lane(int v, int mask) { return int(xor_lane_bits(uint32_t(v), mask)); }

// ------------------------------------------------------------- 1 / sqrt ----
// Correctly rounded sqrt followed by a correctly rounded division: fixed bits
// on host and device. HIP keeps fp32 `/` and sqrtf correctly rounded by
// default (v_sqrt_f32 plus a residual-based fix-up); __fsqrt_rn lowers to the
// bare v_sqrt_f32 and is deliberately not used.
__device__ __forceinline__ float inv_sqrt_rn(float x) { return 1.0f / sqrtf(x); }

// ----------------------------------------------------------- exponential ----
// e^x with fixed bits on host and device (the oracle's ora_expf performs the
// same operations). k = rint(x * log2 e); r = x - k*ln2_hi - k*ln2_lo with a
// 16-bit ln2_hi so k*ln2_hi is exact; e^r by its degree-7 Taylor polynomial on
// |r| <= 0.35; then 2^k by exponent construction. A result below 2^-126 is
// formed by one multiplication into the subnormal range (one rounding).
__device__ __forceinline__ float pow2i(int n) { return __uint_as_float(uint32_t(n + 127) << 23); }  // -126..127
__device__ __forceinline__ float nvr_expf(float x) {
    if (!(x >= -110.0f)) return x != x ? x : 0.0f;  // NaN stays NaN; e^x < 2^-158 rounds to 0
    if (x > 88.75f) return __builtin_inff();
    const float kf = __builtin_rintf(x * 0x1.715476p+0f);
    const int k = int(kf);
    float r = __builtin_fmaf(kf, -0x1.62e400p-1f, x);
    r = __builtin_fmaf(kf, -0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;            // 1/7!
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);  // 1/6!
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);   // 1/5!
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);   // 1/4!
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);   // 1/3!
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    if (k > 127) return (p * pow2i(k - 1)) * 2.0f;
    if (k >= -126) return p * pow2i(k);
    return (p * pow2i(k + 64)) * 0x1.0p-64f;
}

// ------------------------------------------------------------- logarithm ----
// ln(x) for positive normal x. x = 2^e * m with m in [sqrt(1/2), sqrt(2));
// f = m - 1 is exact; ln(1+f) = f + f^2 * Q(f) with Q a degree-8 fit of
// (ln(1+f) - f) / f^2; ln x = e*ln2_hi + (e*ln2_lo + ln(1+f)).
__device__ __forceinline__ float nvr_logf(float x) {
    const uint32_t ix = __float_as_uint(x);
    int32_t e = int32_t(ix >> 23) - 127;
    const uint32_t mb = ix & 0x7fffffu;
    const bool big = mb >= 0x3504f3u;  // m >= sqrt(2): halve m, bump e
    const float m = __uint_as_float(mb | (big ? 0x3f000000u : 0x3f800000u));
    e += big ? 1 : 0;
    const float f = m - 1.0f;
    const float z = f * f;
    float q = -0x1.38dc50p-4f;                   // c8
    q = __builtin_fmaf(q, f, 0x1.087188p-3f);    // c7
    q = __builtin_fmaf(q, f, -0x1.0f27e8p-3f);   // c6
    q = __builtin_fmaf(q, f, 0x1.2269fep-3f);    // c5
    q = __builtin_fmaf(q, f, -0x1.542872p-3f);   // c4
    q = __builtin_fmaf(q, f, 0x1.99a462p-3f);    // c3
    q = __builtin_fmaf(q, f, -0x1.000422p-2f);   // c2
    q = __builtin_fmaf(q, f, 0x1.555550p-2f);    // c1
    q = __builtin_fmaf(q, f, -0x1.fffff8p-2f);   // c0
    const float r = __builtin_fmaf(z, q, f);
    const float ef = float(e);
    return __builtin_fmaf(ef, 0x1.62e430p-1f, __builtin_fmaf(ef, -0x1.05c610p-29f, r));
}

// ------------------------------------------------------------- sampling ----
// SplitMix64 finaliser (Steele, Lea, Flood 2014; constants by Vigna).
__device__ __forceinline__ uint64_t splitmix64(uint64_t v) {
    v += 0x9e3779b97f4a7c15ull;
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}
constexpr uint64_t kTokenMix = 0xd2b74407b1ce6e93ull;

// Uniform in (0,1) from the top 23 hash bits: (k + 0.5) * 2^-23, exact in fp32.
__device__ __forceinline__ float hash_uniform(uint64_t r) {
    return (float(uint32_t(r >> 41)) + 0.5f) * (1.0f / 8388608.0f);
}
// Gumbel-max score of one vocabulary entry: logit / T - ln(-ln(u)).
__device__ __forceinline__ float gumbel_score(float logit, float temperature, uint64_t seed, uint32_t token) {
    const uint64_t r = splitmix64(seed ^ (uint64_t(token) * kTokenMix));
    const float u = hash_uniform(r);
    return logit / temperature - nvr_logf(-nvr_logf(u));
}

// Total order used by every argmax: higher score wins, equal scores go to the
// lower index, NaN never wins (all comparisons with NaN are false).
__device__ __forceinline__ bool better(float s, int i, float best, int best_i) {
    return s > best || (s == best && i < best_i);
}
constexpr int kNoIndex = 0x7fffffff;

// ------------------------------------------------------- RoPE frequencies ----
// Binary64 helpers with fixed operation order; only used to build the cos/sin
// values of one (position, pair), so speed is secondary to reproducibility.
__device__ __forceinline__ double d_log(double x) {
    // x > 0 normal. x = 2^k * m, m in [sqrt(1/2), sqrt(2)); ln m = 2 atanh(s).
    int k;
    double m = frexp(x, &k);  // m in [0.5, 1)
    if (m < 0.70710678118654752440) { m *= 2.0; k -= 1; }
    const double s = (m - 1.0) / (m + 1.0);
    const double s2 = s * s;
    double t = 1.0 / 25.0;
    for (int n = 23; n >= 1; n -= 2) t = t * s2 + 1.0 / double(n);
    const double kd = double(k);
    return kd * 0x1.62e42fee00000p-1 + (kd * 0x1.a39ef35793c76p-33 + 2.0 * s * t);
}
__device__ __forceinline__ double d_exp(double y) {
    const double kd = floor(y * 0x1.71547652b82fep+0 + 0.5);
    const double r = (y - kd * 0x1.62e42fee00000p-1) - kd * 0x1.a39ef35793c76p-33;
    double t = 1.0;
    for (int n = 18; n >= 1; --n) t = 1.0 + t * r / double(n);
    return ldexp(t, int(kd));
}
__device__ __forceinline__ void d_sincos(double a, double* s, double* c) {
    const double kd = floor(a * 0x1.45f306dc9c883p-1 + 0.5);
    const double r = ((a - kd * 0x1.921fb54400000p+0) - kd * 0x1.0b4611a600000p-34) - kd * 0x1.3198a2e037073p-69;
    const double r2 = r * r;
    double ts = 0.0, tc = 0.0;
    // sin r = r * sum (-r^2)^n / (2n+1)!, cos r = sum (-r^2)^n / (2n)!, n <= 11
    double fs = 1.0, fc = 1.0;
    for (int n = 11; n >= 1; --n) {
        fs = 1.0 - fs * r2 / double((2 * n) * (2 * n + 1));
        fc = 1.0 - fc * r2 / double((2 * n - 1) * (2 * n));
    }
    ts = r * fs;
    tc = fc;
    const long long q = (long long)kd & 3;
    if (q == 0) { *s = ts; *c = tc; }
    else if (q == 1) { *s = tc; *c = -ts; }
    else if (q == 2) { *s = -ts; *c = -tc; }
    else { *s = -tc; *c = ts; }
}
// cos/sin of position * theta^(-2*pair/dim), with the exponent, the power and
// the angle each rounded to fp32 as the reference forms them, and cos/sin
// evaluated in binary64 then rounded to fp32.
__device__ __forceinline__ void rope_cos_sin(int position, int pair, int dim, float theta, float* c, float* s) {
    const float expo = -float(2 * pair) / float(dim);
    const float inv_freq = float(d_exp(double(expo) * d_log(double(theta))));
    const float angle = float(position) * inv_freq;
    double sd, cd;
    d_sincos(double(angle), &sd, &cd);
    *c = float(cd);
    *s = float(sd);
}

// q/k head: RMSNorm in the reference's order, bf16 rounding, NeoX rotation.
// Returns the rotated chunk of this lane (elements 8m..8m+7), packed. The
// 16 lanes of a head form one DPP row: warp level 16 is quad lane ^2, level 8
// quad lane ^1; the warp sums (lanes 0,4,8,12) fold as (W0 + W2) + (W1 + W3)
// through row_ror:8 then row_half_mirror (each quad holds one replicated sum).
// sn_signed is -sin for elements j < 64 and +sin above, so that
// rot = n*c + p*sn_signed rounds exactly like (n*c) -/+ (p*sin).
__device__ __forceinline__ uint4 norm_rotate_d128(const uint4& xw, const float* wf, const float* cs,
                                                  const float* sn_signed, float eps) {
    constexpr int D = 128;
    float x[8];
    unpack8(xw, x);
    float s[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] = x[i] * x[i];
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] = s[i] + dpp<kDppQuadXor2>(s[i]);
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] = s[i] + dpp<kDppQuadXor1>(s[i]);
    float total = ((s[0] + s[4]) + (s[2] + s[6])) + ((s[1] + s[5]) + (s[3] + s[7]));
    total = total + dpp<kDppRowRor8>(total);
    total = total + dpp<kDppRowHalfMirror>(total);
    const float inv = inv_sqrt_rn(total / float(D) + eps);
    float n[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) n[i] = (x[i] * inv) * wf[i];
    const uint4 np = pack8(n);  // the bf16-materialised normalised head
    unpack8(np, n);
    uint4 pp;  // NeoX partner chunk (elements j +/- 64) from lane m ^ 8
    pp.x = dpp<kDppRowRor8>(np.x);
    pp.y = dpp<kDppRowRor8>(np.y);
    pp.z = dpp<kDppRowRor8>(np.z);
    pp.w = dpp<kDppRowRor8>(np.w);
    float p[8];
    unpack8(pp, p);
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = n[i] * cs[i] + p[i] * sn_signed[i];
    return pack8(o);
}

}  // namespace nvr
