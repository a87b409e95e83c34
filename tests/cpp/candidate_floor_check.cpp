// The sampler's candidate floor (nano-vllm-rs_amd/csrc/sample.hip,
// candidate_floor): its direct form, from bound * T and a few predicate
// steps, restated here in host fp32 (no contraction), against the binary
// search over every bf16 key that defines it, on random and edge-case
// (s0, T) pairs. Exit status 0 when every pair gives the same bits.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>

namespace {

float from_bits(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
uint32_t to_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

const float kNoiseMax = 0x1.0a2b24p+4f;  // the largest Gumbel noise of a 23-bit hash

// bf16 value of an order-preserving 16-bit key (0x007f = -inf .. 0xff80 = +inf)
float value(int key) { return from_bits(uint32_t(key >= 0x8000 ? key - 0x8000 : 0xffff - key) << 16); }
float bound_of(float s0) { return (s0 - kNoiseMax) - (std::fabs(s0) + 34.0f) * 0x1.0p-17f; }

float search(float s0, float inv_t) {
    const float bound = bound_of(s0);
    int lo = 0x007f, hi = 0xff80;
    if (value(lo) * inv_t >= bound) hi = lo;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (value(mid) * inv_t >= bound) hi = mid;
        else lo = mid;
    }
    return value(hi);
}

long fallbacks = 0;

float direct(float s0, float inv_t, float t) {
    const float bound = bound_of(s0);
    auto pass = [&](int key) { return value(key) * inv_t >= bound; };
    const float v0 = bound * t;
    const uint32_t u = to_bits(v0);
    int key = (u & 0x80000000u) ? 0xffff - int((u >> 16) + ((u & 0xffffu) != 0u)) : int(u >> 16) + 0x8000;
    if (std::fabs(v0) >= 0x1.0p-100f && std::fabs(v0) <= 0x1.0p+100f) {
        key += !pass(key);
        key += !pass(key);
        key -= pass(key - 1);
        key -= pass(key - 1);
        if (pass(key) && !pass(key - 1)) return value(key);
    }
    ++fallbacks;
    return search(s0, inv_t);
}

}  // namespace

int main(int argc, char** argv) {
    const long pairs = argc > 1 ? std::atol(argv[1]) : 4000000;
    std::mt19937_64 gen(20261202);
    long checked = 0, bad = 0;
    auto check = [&](float s0, float t) {
        const float inv_t = 1.0f / t;
        if (!(std::fabs(s0) < INFINITY && inv_t < INFINITY)) return;  // pruning off: no floor
        const float a = search(s0, inv_t), b = direct(s0, inv_t, t);
        ++checked;
        if (to_bits(a) != to_bits(b)) {
            if (bad < 10) std::printf("mismatch s0=%a T=%a search=%a direct=%a\n", s0, t, a, b);
            ++bad;
        }
    };
    std::uniform_real_distribution<double> score(-200.0, 200.0), log_t(-6.0, 6.0), near(-30.0, 30.0);
    for (long i = 0; i < pairs; ++i) check(float(score(gen)), float(std::exp(log_t(gen))));
    for (long i = 0; i < pairs / 10; ++i)  // the bound within a few ulps of zero
        check(kNoiseMax + float(near(gen)) * 1e-5f, float(std::exp(log_t(gen))));
    const float s0s[] = {kNoiseMax, std::nextafter(kNoiseMax, 0.0f), std::nextafter(kNoiseMax, 100.0f), 0.0f, -0.0f,
                         16.0f, 17.0f, 1e-30f, -1e-30f, 1e30f, -1e30f, 3.4e38f, -3.4e38f, 1e-40f};
    const float ts[] = {1e-38f, 1e-30f, 1e-10f, 1e-3f, 0.1f, 0.6f, 1.0f, 2.0f, 1e3f, 1e10f, 1e30f, 3e38f};
    for (float s0 : s0s)
        for (float t : ts) check(s0, t);
    std::printf("candidate floor: %ld pairs, %ld mismatches, %ld by the full search\n", checked, bad, fallbacks);
    return bad == 0 ? 0 : 1;
}
