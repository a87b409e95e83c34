/*
 * oracle.c — CPU restatement of the nano-vllm-rs fused per-layer kernels.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP library,
 * never part of the product path.
 *
 * Compile with -ffp-contract=off: every fp32 expression below rounds exactly
 * where the reference's CUDA source rounds; multiply-adds the reference's nvcc
 * build contracts (the `+= v*v` accumulations) are written as fmaf.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ threads ---- */

typedef void (*range_fn)(void* ctx, int64_t begin, int64_t end);

struct range_job {
    range_fn fn;
    void* ctx;
    int64_t begin, end;
};

static void* range_thread(void* arg) {
    struct range_job* job = (struct range_job*)arg;
    job->fn(job->ctx, job->begin, job->end);
    return NULL;
}

/* Runs fn over [0, n) split into `threads` contiguous ranges. */
static void parallel_for(int64_t n, int threads, range_fn fn, void* ctx) {
    if (threads <= 1 || n < 2) {
        fn(ctx, 0, n);
        return;
    }
    if (threads > 256) threads = 256;
    if (threads > n) threads = (int)n;
    pthread_t tid[256];
    int joined[256];
    struct range_job jobs[256];
    for (int t = 0; t < threads; ++t) {
        jobs[t].fn = fn;
        jobs[t].ctx = ctx;
        jobs[t].begin = n * t / threads;
        jobs[t].end = n * (t + 1) / threads;
        joined[t] = 0;
        if (t == 0) continue;
        if (pthread_create(&tid[t], NULL, range_thread, &jobs[t]) == 0) {
            joined[t] = 1;
        } else {
            range_thread(&jobs[t]); /* no worker: run the range here */
        }
    }
    range_thread(&jobs[0]);
    for (int t = 1; t < threads; ++t)
        if (joined[t]) pthread_join(tid[t], NULL);
}

/* ------------------------------------------------------------ scalars ---- */

static inline uint32_t f2u(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float x;
    memcpy(&x, &u, 4);
    return x;
}

/* __float2bfloat16_rn (cuda_bf16.h, used at kernels/kernels.cu:157,162,185,
 * 205,207,363): round to nearest even; NaN stays NaN (quiet bit set). */
uint16_t ora_bf16_from_f32(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float ora_f32_from_bf16(uint16_t h) { return u2f((uint32_t)h << 16); }

static inline float bf(uint16_t h) { return ora_f32_from_bf16(h); }
static inline float round_bf(float x) { return bf(ora_bf16_from_f32(x)); }

/* kernels/kernels.cu:372-377 (published SplitMix64 finaliser). */
uint64_t ora_splitmix64(uint64_t v) {
    v += 0x9e3779b97f4a7c15ull;
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}

/* src/runtime.rs:780-790. */
uint64_t ora_sampling_seed(uint64_t base, uint64_t request_id, uint64_t generated) {
    return ora_splitmix64(ora_splitmix64(base) ^ ora_splitmix64(request_id) ^ ora_splitmix64(generated));
}

/* Stands in for CUDA logf at kernels/kernels.cu:387,447. x = 2^e * m with
 * m in [sqrt(1/2), sqrt(2)); f = m - 1 (exact); ln(1+f) = f + f^2 * Q(f) with
 * Q a degree-8 least-squares fit of (ln(1+f) - f) / f^2 on that interval;
 * ln x = e*ln2_hi + (e*ln2_lo + ln(1+f)). Positive normal inputs only (the
 * Gumbel path never produces anything else). */
float ora_logf(float x) {
    const uint32_t ix = f2u(x);
    int32_t e = (int32_t)(ix >> 23) - 127;
    const uint32_t mb = ix & 0x7fffffu;
    const int big = mb >= 0x3504f3u;
    const float m = u2f(mb | (big ? 0x3f000000u : 0x3f800000u));
    e += big;
    const float f = m - 1.0f;
    const float z = f * f;
    static const float c[9] = {-0x1.fffff8p-2f, 0x1.555550p-2f, -0x1.000422p-2f, 0x1.99a462p-3f, -0x1.542872p-3f,
                               0x1.2269fep-3f,  -0x1.0f27e8p-3f, 0x1.087188p-3f, -0x1.38dc50p-4f};
    float q = c[8];
    for (int i = 7; i >= 0; --i) q = fmaf(q, f, c[i]);
    const float r = fmaf(z, q, f);
    const float ef = (float)e;
    return fmaf(ef, 0x1.62e430p-1f, fmaf(ef, -0x1.05c610p-29f, r));
}

void ora_logf_n(const float* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = ora_logf(in[i]);
}

/* Stands in for CUDA expf at kernels/kernels.cu:254,320 (attention
 * probabilities). k = rint(x*log2 e); r = x - k*ln2_hi - k*ln2_lo (ln2_hi has
 * 16 significant bits, so k*ln2_hi is exact); e^r = degree-7 Taylor polynomial
 * on |r| <= 0.35; 2^k by exponent construction, with results below 2^-126
 * formed by one multiplication into the subnormal range. */
static inline float pow2i(int n) { return u2f((uint32_t)(n + 127) << 23); }
float ora_expf(float x) {
    if (!(x >= -110.0f)) return x != x ? x : 0.0f;
    if (x > 88.75f) return INFINITY;
    const float kf = rintf(x * 0x1.715476p+0f);
    const int k = (int)kf;
    float r = fmaf(kf, -0x1.62e400p-1f, x);
    r = fmaf(kf, -0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    if (k > 127) return (p * pow2i(k - 1)) * 2.0f;
    if (k >= -126) return p * pow2i(k);
    return (p * pow2i(k + 64)) * 0x1.0p-64f;
}

void ora_expf_n(const float* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = ora_expf(in[i]);
}

/* kernels/kernels.cu:384-388. */
float ora_gumbel_score(float logit, float temperature, uint64_t seed, uint32_t token) {
    const uint64_t r = ora_splitmix64(seed ^ ((uint64_t)token * 0xd2b74407b1ce6e93ull));
    const float u = ((float)(uint32_t)(r >> 41) + 0.5f) * (1.0f / 8388608.0f);
    return logit / temperature - ora_logf(-ora_logf(u));
}

/* ------------------------------------------------------ RoPE angles ---- */
/* kernels/kernels.cu:199-200 and :218-220 form, in fp32,
 *   angle = position * powf(theta, -float(2*pair)/dim)
 * and take sincosf(angle). Here powf is exp(expo*ln theta) and sin/cos are
 * evaluated in binary64 (fixed series, Cody-Waite reduction by pi/2 split in
 * three parts), then rounded to fp32. */
static double d_log(double x) {
    int k;
    double m = frexp(x, &k);
    if (m < 0.70710678118654752440) {
        m *= 2.0;
        k -= 1;
    }
    const double s = (m - 1.0) / (m + 1.0);
    const double s2 = s * s;
    double t = 1.0 / 25.0;
    for (int n = 23; n >= 1; n -= 2) t = t * s2 + 1.0 / (double)n;
    const double kd = (double)k;
    return kd * 0x1.62e42fee00000p-1 + (kd * 0x1.a39ef35793c76p-33 + 2.0 * s * t);
}

static double d_exp(double y) {
    const double kd = floor(y * 0x1.71547652b82fep+0 + 0.5);
    const double r = (y - kd * 0x1.62e42fee00000p-1) - kd * 0x1.a39ef35793c76p-33;
    double t = 1.0;
    for (int n = 18; n >= 1; --n) t = 1.0 + t * r / (double)n;
    return ldexp(t, (int)kd);
}

static void d_sincos(double a, double* s, double* c) {
    const double kd = floor(a * 0x1.45f306dc9c883p-1 + 0.5);
    const double r = ((a - kd * 0x1.921fb54400000p+0) - kd * 0x1.0b4611a600000p-34) - kd * 0x1.3198a2e037073p-69;
    const double r2 = r * r;
    double fs = 1.0, fc = 1.0;
    for (int n = 11; n >= 1; --n) {
        fs = 1.0 - fs * r2 / (double)((2 * n) * (2 * n + 1));
        fc = 1.0 - fc * r2 / (double)((2 * n - 1) * (2 * n));
    }
    const double ts = r * fs, tc = fc;
    const long long q = (long long)kd & 3;
    if (q == 0) {
        *s = ts;
        *c = tc;
    } else if (q == 1) {
        *s = tc;
        *c = -ts;
    } else if (q == 2) {
        *s = -ts;
        *c = -tc;
    } else {
        *s = -tc;
        *c = ts;
    }
}

void ora_rope_cos_sin(int position, int pair, int dim, float theta, float* c, float* s) {
    const float expo = -(float)(2 * pair) / (float)dim;
    const float inv_freq = (float)d_exp((double)expo * d_log((double)theta));
    const float angle = (float)position * inv_freq;
    double sd, cd;
    d_sincos((double)angle, &sd, &cd);
    *c = (float)cd;
    *s = (float)sd;
}

/* ------------------------------------------------- block reductions ---- */
/* kernels/kernels.cu:109-125: warp_sum is a shuffle-down tree over 32 lanes
 * (a lane whose source is out of range reads its own value); block_sum runs
 * it per warp, then once more over the 8 warp results with zeros above. */
static float warp_sum_lane0(float lane[32]) {
    for (int off = 16; off > 0; off >>= 1) {
        float next[32];
        for (int i = 0; i < 32; ++i) next[i] = lane[i] + (i + off < 32 ? lane[i + off] : lane[i]);
        memcpy(lane, next, sizeof(next));
    }
    return lane[0];
}

static float block_sum_256(const float part[256]) {
    float warp[8];
    for (int w = 0; w < 8; ++w) {
        float lane[32];
        memcpy(lane, part + 32 * w, sizeof(lane));
        warp[w] = warp_sum_lane0(lane);
    }
    float lane[32];
    for (int i = 0; i < 32; ++i) lane[i] = i < 8 ? warp[i] : 0.0f;
    return warp_sum_lane0(lane);
}

/* Per-thread partials of kernels/kernels.cu:148-153 / :178-179: thread t
 * accumulates j = t, t+256, ... with `s += v*v` (contracted to an fma). */
float ora_block_sum_sq(const float* v, int n) {
    float part[256];
    for (int t = 0; t < 256; ++t) {
        float s = 0.0f;
        for (int j = t; j < n; j += 256) s = fmaf(v[j], v[j], s);
        part[t] = s;
    }
    return block_sum_256(part);
}

/* ----------------------------------------------------------- copies ---- */

struct gather_ctx {
    const int32_t* index;
    const uint16_t* src;
    uint16_t* out;
    int hidden, src_rows;
};

static void gather_range(void* p, int64_t r0, int64_t r1) {
    const struct gather_ctx* g = (const struct gather_ctx*)p;
    for (int64_t r = r0; r < r1; ++r) {
        const int32_t i = g->index[r];
        uint16_t* dst = g->out + r * g->hidden;
        if (i >= 0 && i < g->src_rows) memcpy(dst, g->src + (int64_t)i * g->hidden, (size_t)g->hidden * 2);
        else memset(dst, 0, (size_t)g->hidden * 2); /* __float2bfloat16(0.0f) = +0 */
    }
}

/* kernels/kernels.cu:139-144. */
void ora_embedding(const int32_t* tokens, const uint16_t* weight, uint16_t* out, int rows, int hidden, int vocab,
                   int threads) {
    struct gather_ctx g = {tokens, weight, out, hidden, vocab};
    parallel_for(rows, threads, gather_range, &g);
}

/* kernels/kernels.cu:366-371. */
void ora_gather(const uint16_t* x, const int32_t* indices, uint16_t* out, int rows, int hidden, int input_rows,
                int threads) {
    struct gather_ctx g = {indices, x, out, hidden, input_rows};
    parallel_for(rows, threads, gather_range, &g);
}

struct kv_ctx {
    const uint16_t *k, *v;
    const int32_t* slots;
    uint16_t *kc, *vc;
    int64_t width, capacity;
};

static void kv_range(void* p, int64_t r0, int64_t r1) {
    const struct kv_ctx* g = (const struct kv_ctx*)p;
    for (int64_t r = r0; r < r1; ++r) {
        const int32_t slot = g->slots[r];
        if (slot < 0 || (int64_t)slot >= g->capacity) continue;
        memcpy(g->kc + (int64_t)slot * g->width, g->k + r * g->width, (size_t)g->width * 2);
        memcpy(g->vc + (int64_t)slot * g->width, g->v + r * g->width, (size_t)g->width * 2);
    }
}

/* The K/V half of kernels/kernels.cu:188-190,206-209 as a plain copy. */
void ora_kv_write(const uint16_t* k, const uint16_t* v, const int32_t* slots, uint16_t* kc, uint16_t* vc, int rows,
                  int kvh, int dim, int bs, int blocks, int threads) {
    struct kv_ctx g = {k, v, slots, kc, vc, (int64_t)kvh * dim, (int64_t)bs * blocks};
    parallel_for(rows, threads, kv_range, &g);
}

/* ---------------------------------------------------------- RMSNorm ---- */

struct rms_ctx {
    const uint16_t* x;
    uint16_t* residual;
    const uint16_t* weight;
    uint16_t* out;
    int hidden, add;
    float eps;
};

/* kernels/kernels.cu:145-164. */
static void rms_range(void* p, int64_t r0, int64_t r1) {
    const struct rms_ctx* g = (const struct rms_ctx*)p;
    const int H = g->hidden;
    float* v = (float*)malloc(sizeof(float) * (size_t)H);
    for (int64_t r = r0; r < r1; ++r) {
        const int64_t base = r * H;
        for (int j = 0; j < H; ++j) {
            float value = bf(g->x[base + j]);
            if (g->add) value += bf(g->residual[base + j]);
            v[j] = value;
        }
        const float inv = 1.0f / sqrtf(ora_block_sum_sq(v, H) / (float)H + g->eps);
        for (int j = 0; j < H; ++j) {
            if (g->add) g->residual[base + j] = ora_bf16_from_f32(v[j]);
            const float normalized = v[j] * inv;
            g->out[base + j] = ora_bf16_from_f32(normalized * bf(g->weight[j]));
        }
    }
    free(v);
}

void ora_rms(const uint16_t* x, const uint16_t* weight, uint16_t* out, int rows, int hidden, float eps, int threads) {
    struct rms_ctx g = {x, NULL, weight, out, hidden, 0, eps};
    parallel_for(rows, threads, rms_range, &g);
}

void ora_add_rms(const uint16_t* x, uint16_t* residual, const uint16_t* weight, uint16_t* out, int rows, int hidden,
                 float eps, int threads) {
    struct rms_ctx g = {x, residual, weight, out, hidden, 1, eps};
    parallel_for(rows, threads, rms_range, &g);
}

/* ------------------------------------------------------------- RoPE ---- */

struct table_ctx {
    float* cache;
    int dim;
    float theta;
};

static void table_range(void* p, int64_t r0, int64_t r1) {
    const struct table_ctx* g = (const struct table_ctx*)p;
    const int half = g->dim / 2;
    for (int64_t pos = r0; pos < r1; ++pos)
        for (int pair = 0; pair < half; ++pair) {
            float c, s;
            ora_rope_cos_sin((int)pos, pair, g->dim, g->theta, &c, &s);
            g->cache[pos * g->dim + pair] = c;
            g->cache[pos * g->dim + half + pair] = s;
        }
}

/* kernels/kernels.cu:213-224. */
void ora_rope_cache(float* cache, int positions, int dim, float theta, int threads) {
    struct table_ctx g = {cache, dim, theta};
    parallel_for(positions, threads, table_range, &g);
}

struct rope_ctx {
    const uint16_t *qkv, *qw, *kw;
    const int32_t *positions, *slots;
    uint16_t *qout, *kc, *vc;
    int qh, kvh, dim, bs, blocks;
    float eps, theta;
    const float* table;
    int max_positions;
};

/* kernels/kernels.cu:166-211, one (row, head) block at a time. */
static void rope_range(void* p, int64_t r0, int64_t r1) {
    const struct rope_ctx* g = (const struct rope_ctx*)p;
    const int dim = g->dim, half = dim / 2;
    const int heads = g->qh + 2 * g->kvh;
    float vals[256], normalized[256];
    for (int64_t row = r0; row < r1; ++row) {
        const int64_t packed = row * heads * dim;
        const int position = g->positions[row], slot = g->slots[row];
        const int valid_slot = slot >= 0 && (int64_t)slot < (int64_t)g->bs * g->blocks;
        for (int head = 0; head < g->qh + g->kvh; ++head) {
            const int is_q = head < g->qh;
            const int local = is_q ? head : head - g->qh;
            const int64_t base = packed + (int64_t)head * dim;
            const uint16_t* weight = is_q ? g->qw : g->kw;
            for (int j = 0; j < dim; ++j) vals[j] = bf(g->qkv[base + j]);
            const float inv = 1.0f / sqrtf(ora_block_sum_sq(vals, dim) / (float)dim + g->eps);
            for (int j = 0; j < dim; ++j) {
                const float norm = vals[j] * inv;
                normalized[j] = round_bf(norm * bf(weight[j]));
            }
            const int64_t cache_base = ((int64_t)slot * g->kvh + local) * dim;
            for (int j = 0; j < dim; ++j) {
                const int pair = j % half;
                float sine, cosine;
                if (g->table) {
                    const int valid_position = position >= 0 && position < g->max_positions;
                    cosine = valid_position ? g->table[(int64_t)position * dim + pair] : 1.0f;
                    sine = valid_position ? g->table[(int64_t)position * dim + half + pair] : 0.0f;
                } else {
                    ora_rope_cos_sin(position, pair, dim, g->theta, &cosine, &sine);
                }
                const float rotated = j < half ? (normalized[j] * cosine) - (normalized[j + half] * sine)
                                               : (normalized[j] * cosine) + (normalized[j - half] * sine);
                if (is_q) {
                    g->qout[(row * g->qh + local) * dim + j] = ora_bf16_from_f32(rotated);
                } else if (valid_slot) {
                    g->kc[cache_base + j] = ora_bf16_from_f32(rotated);
                    g->vc[cache_base + j] = g->qkv[packed + (int64_t)(g->qh + g->kvh + local) * dim + j];
                }
            }
        }
    }
}

void ora_qkv_rope(const uint16_t* qkv, const uint16_t* qw, const uint16_t* kw, const int32_t* positions,
                  const int32_t* slots, uint16_t* qout, uint16_t* kc, uint16_t* vc, int rows, int qh, int kvh, int dim,
                  int bs, int blocks, float eps, float theta, const float* table, int max_positions, int threads) {
    struct rope_ctx g = {qkv, qw, kw, positions, slots, qout, kc, vc, qh, kvh, dim, bs, blocks, eps, theta, table,
                         max_positions};
    parallel_for(rows, threads, rope_range, &g);
}

/* ------------------------------------------------------------- SiLU ---- */

struct silu_ctx {
    const uint16_t* packed;
    uint16_t* out;
    int intermediate;
};

/* kernels/kernels.cu:356-365. */
static void silu_range(void* p, int64_t r0, int64_t r1) {
    const struct silu_ctx* g = (const struct silu_ctx*)p;
    const int I = g->intermediate;
    for (int64_t r = r0; r < r1; ++r)
        for (int i = 0; i < I; ++i) {
            const int64_t base = r * 2 * I + i;
            const float gate = bf(g->packed[base]);
            const float activation = gate / (1.0f + expf(-gate));
            g->out[r * I + i] = ora_bf16_from_f32(activation * bf(g->packed[base + I]));
        }
}

void ora_silu(const uint16_t* packed, uint16_t* out, int rows, int intermediate, int threads) {
    struct silu_ctx g = {packed, out, intermediate};
    parallel_for(rows, threads, silu_range, &g);
}

/* ----------------------------------------------------- paged attention ---- */
/* kernels/kernels.cu:226-270 (attention_kernel) and :289-346
 * (attention_ordered_kernel, documented at :286-287 to keep the first one's
 * fp32 order). Per (row, head), kvhead = head / (qh / kvh):
 *   - rows with seq outside [0, batch) or context = pos + 1 outside
 *     [1, max_context] or above stride * bs produce zeros (:231-234, :295-298);
 *   - token t reads physical block table[seq*stride + t/bs] (:240, :277-284);
 *     a block outside [0, num_blocks) gives score -inf and no V term;
 *   - score = warp_sum(chain_0 .. chain_31) * rsqrt(dim), where lane c's chain
 *     accumulates q[d]*k[d] for d = c, c+32, ... < dim with `dot += q*k`
 *     (contracted to fma) from 0 (:243-245, :306-312); rsqrt -> 1/sqrtf;
 *   - m = max of the scores; p_t = exp(score_t - m) when m is finite, else 0
 *     (:253-254, :319-320); den = block_sum of thread partials, thread i adding
 *     p_i, p_{i+256}, ... in order (:251-258, :318-324);
 *   - value_d = sum over tokens in order of p_t * v_t[d] (contracted to fma)
 *     from 0; out = bf16(den > 0 ? value_d / den : 0) (:260-268, :325-345). */
struct attn_ctx {
    const uint16_t *q, *kc, *vc;
    const int32_t *positions, *seqs, *tables;
    uint16_t* out;
    int qh, kvh, dim, bs, blocks, stride, batch, max_context;
};

static void attention_range(void* p, int64_t i0, int64_t i1) {
    const struct attn_ctx* a = (const struct attn_ctx*)p;
    float* scores = (float*)malloc(sizeof(float) * (size_t)(a->max_context > 0 ? a->max_context : 1));
    const float scale = 1.0f / sqrtf((float)a->dim);
    for (int64_t i = i0; i < i1; ++i) {
        const int64_t row = i / a->qh;
        const int head = (int)(i % a->qh);
        const int kvhead = head / (a->qh / a->kvh);
        const uint16_t* q = a->q + i * a->dim;
        uint16_t* out = a->out + i * a->dim;
        const int seq = a->seqs[row];
        const int64_t context = (int64_t)a->positions[row] + 1;
        if (seq < 0 || seq >= a->batch || context < 1 || context > a->max_context ||
            context > (int64_t)a->stride * a->bs || scores == NULL) {
            for (int d = 0; d < a->dim; ++d) out[d] = 0;
            continue;
        }
        const int32_t* table = a->tables + (int64_t)seq * a->stride;
        float m = -INFINITY;
        for (int t = 0; t < (int)context; ++t) {
            const int block = table[t / a->bs];
            float score = -INFINITY;
            if (block >= 0 && block < a->blocks) {
                const uint16_t* k = a->kc + (((int64_t)block * a->bs + t % a->bs) * a->kvh + kvhead) * a->dim;
                float lane[32];
                for (int c = 0; c < 32; ++c) {
                    float dot = 0.0f;
                    for (int d = c; d < a->dim; d += 32) dot = fmaf(bf(q[d]), bf(k[d]), dot);
                    lane[c] = dot;
                }
                score = warp_sum_lane0(lane) * scale;
            }
            scores[t] = score;
            m = fmaxf(m, score);
        }
        float part[256];
        for (int th = 0; th < 256; ++th) {
            float sum = 0.0f;
            for (int t = th; t < (int)context; t += 256) {
                const float pr = isfinite(m) ? ora_expf(scores[t] - m) : 0.0f;
                scores[t] = pr;
                sum += pr;
            }
            part[th] = sum;
        }
        const float den = block_sum_256(part);
        for (int d = 0; d < a->dim; ++d) {
            float value = 0.0f;
            for (int t = 0; t < (int)context; ++t) {
                const int block = table[t / a->bs];
                if (block < 0 || block >= a->blocks) continue;
                const uint16_t* v = a->vc + (((int64_t)block * a->bs + t % a->bs) * a->kvh + kvhead) * a->dim;
                value = fmaf(scores[t], bf(v[d]), value);
            }
            out[d] = ora_bf16_from_f32(den > 0.0f ? value / den : 0.0f);
        }
    }
    free(scores);
}

void ora_attention(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, const int32_t* positions,
                   const int32_t* seqs, const int32_t* tables, uint16_t* out, int rows, int qh, int kvh, int dim,
                   int bs, int blocks, int stride, int batch, int max_context, int threads) {
    struct attn_ctx a = {q, kc, vc, positions, seqs, tables, out, qh, kvh, dim, bs, blocks, stride, batch, max_context};
    parallel_for((int64_t)rows * qh, threads, attention_range, &a);
}

/* --------------------------------------------------------- sampling ---- */

static inline int better(float s, int i, float best, int best_i) { return s > best || (s == best && i < best_i); }

/* Best (score, index) of tokens [begin, end) of one row. */
static void scan(const uint16_t* row, int64_t begin, int64_t end, float temperature, uint64_t seed, float* best_score,
                 int32_t* best_index) {
    float best = -INFINITY;
    int32_t idx = 0x7fffffff;
    for (int64_t t = begin; t < end; ++t) {
        float score = bf(row[t]);
        if (temperature > 0) score = ora_gumbel_score(score, temperature, seed, (uint32_t)t);
        if (better(score, (int)t, best, idx)) {
            best = score;
            idx = (int32_t)t;
        }
    }
    *best_score = best;
    *best_index = idx;
}

struct sample_ctx {
    const uint16_t* logits;
    const float* temps;
    const uint64_t* seeds;
    int32_t* out;
    int vocab;
};

/* kernels/kernels.cu:378-407. */
static void sample_range(void* p, int64_t r0, int64_t r1) {
    const struct sample_ctx* g = (const struct sample_ctx*)p;
    for (int64_t r = r0; r < r1; ++r) {
        float s;
        int32_t i;
        scan(g->logits + r * g->vocab, 0, g->vocab, g->temps[r], g->seeds[r], &s, &i);
        g->out[r] = i == 0x7fffffff ? 0 : i;
    }
}

void ora_sample(const uint16_t* logits, const float* temps, const uint64_t* seeds, int32_t* out, int batch, int vocab,
                int threads) {
    struct sample_ctx g = {logits, temps, seeds, out, vocab};
    parallel_for(batch, threads, sample_range, &g);
}

/* kernels/kernels.cu:433-466. */
void ora_sample_partitioned(const uint16_t* logits, const float* temps, const uint64_t* seeds, int32_t* out,
                            float* partial_scores, int32_t* partial_ids, int batch, int vocab, int width) {
    const int parts = (int)(((int64_t)vocab + width - 1) / width);
    for (int r = 0; r < batch; ++r) {
        for (int p = 0; p < parts; ++p) {
            const int64_t begin = (int64_t)p * width;
            const int64_t end = begin + width < vocab ? begin + width : vocab;
            scan(logits + (int64_t)r * vocab, begin, end, temps[r], seeds[r], &partial_scores[(int64_t)r * parts + p],
                 &partial_ids[(int64_t)r * parts + p]);
        }
        float best = -INFINITY;
        int32_t idx = 0x7fffffff;
        for (int p = 0; p < parts; ++p) {
            const float s = partial_scores[(int64_t)r * parts + p];
            const int32_t i = partial_ids[(int64_t)r * parts + p];
            if (better(s, i, best, idx)) {
                best = s;
                idx = i;
            }
        }
        out[r] = idx == 0x7fffffff ? 0 : idx;
    }
}

/* ----------------------------------------------------- synthetic data ---- */

struct fill_ctx {
    uint16_t* out;
    size_t n;
    uint64_t seed;
    double mean, stddev;
};

/* Pair p uses draws 2p and 2p+1 of the SplitMix64 sequence started at seed. */
static void fill_range(void* p, int64_t q0, int64_t q1) {
    const struct fill_ctx* g = (const struct fill_ctx*)p;
    const double two_pi = 6.283185307179586476925;
    for (int64_t q = q0; q < q1; ++q) {
        const uint64_t a = ora_splitmix64(g->seed + (uint64_t)(2 * q) * 0x9e3779b97f4a7c15ull);
        const uint64_t b = ora_splitmix64(g->seed + (uint64_t)(2 * q + 1) * 0x9e3779b97f4a7c15ull);
        const double u1 = ((double)(a >> 11) + 0.5) * 0x1.0p-53;
        const double u2 = ((double)(b >> 11) + 0.5) * 0x1.0p-53;
        const double rad = sqrt(-2.0 * log(u1));
        const size_t i = (size_t)(2 * q);
        g->out[i] = ora_bf16_from_f32((float)(g->mean + g->stddev * rad * cos(two_pi * u2)));
        if (i + 1 < g->n) g->out[i + 1] = ora_bf16_from_f32((float)(g->mean + g->stddev * rad * sin(two_pi * u2)));
    }
}

void ora_fill_normal_bf16(uint16_t* out, size_t n, uint64_t seed, double mean, double stddev) {
    struct fill_ctx g = {out, n, seed, mean, stddev};
    parallel_for((int64_t)((n + 1) / 2), 8, fill_range, &g);
}
