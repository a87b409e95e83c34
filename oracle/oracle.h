/*
 * oracle.h — CPU restatement of the nano-vllm-rs fused per-layer kernels.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP kernels in
 * nano-vllm-rs_amd/: tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline leg call it; the product never links, loads or falls back to it.
 *
 * Every function restates kernels/kernels.cu of the reference (file:line in
 * oracle.c) with scalar C and fp32 arithmetic at the reference's rounding
 * points. bf16 values are uint16_t (upper half of an IEEE binary32).
 *
 * Where the reference calls CUDA math with no reproducible definition
 * (rsqrtf, expf, logf, powf, sincosf), the oracle fixes one:
 *   rsqrtf(x)  -> 1.0f / sqrtf(x)                 (two correctly rounded ops)
 *   logf       -> ora_logf (range reduction + degree-8 polynomial, <1 ulp)
 *   powf/sincosf in the RoPE table -> binary64 series, rounded to fp32
 *   expf (SiLU) -> the C library's expf (SiLU is compared within 1 bf16 ulp)
 *   expf (attention) -> ora_expf (range reduction + degree-7 polynomial)
 *
 * Functions taking `threads` split rows over that many POSIX threads
 * (threads <= 1 runs on the caller's thread); results do not depend on it.
 */
#ifndef NVR_ORACLE_H
#define NVR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Scalars. */
uint16_t ora_bf16_from_f32(float x);
float ora_f32_from_bf16(uint16_t h);
uint64_t ora_splitmix64(uint64_t v);
uint64_t ora_sampling_seed(uint64_t base, uint64_t request_id, uint64_t generated);
float ora_logf(float x);
void ora_logf_n(const float* in, float* out, size_t n);
float ora_expf(float x);
void ora_expf_n(const float* in, float* out, size_t n);
float ora_gumbel_score(float logit, float temperature, uint64_t seed, uint32_t token);
void ora_rope_cos_sin(int position, int pair, int dim, float theta, float* c, float* s);
/* Sum of squares of v[0..n) in the reference's 256-thread block order. */
float ora_block_sum_sq(const float* v, int n);

/* Kernels. */
void ora_embedding(const int32_t* tokens, const uint16_t* weight, uint16_t* out, int rows, int hidden, int vocab,
                   int threads);
void ora_gather(const uint16_t* x, const int32_t* indices, uint16_t* out, int rows, int hidden, int input_rows,
                int threads);
void ora_rms(const uint16_t* x, const uint16_t* weight, uint16_t* out, int rows, int hidden, float eps, int threads);
void ora_add_rms(const uint16_t* x, uint16_t* residual, const uint16_t* weight, uint16_t* out, int rows, int hidden,
                 float eps, int threads);
void ora_rope_cache(float* cache, int positions, int dim, float theta, int threads);
/* table == NULL selects the inline angle (nv_qkv_rope); otherwise the cached
 * path (nv_qkv_rope_cached) with max_positions rows of table. */
void ora_qkv_rope(const uint16_t* qkv, const uint16_t* qw, const uint16_t* kw, const int32_t* positions,
                  const int32_t* slots, uint16_t* qout, uint16_t* kc, uint16_t* vc, int rows, int qh, int kvh, int dim,
                  int bs, int blocks, float eps, float theta, const float* table, int max_positions, int threads);
void ora_kv_write(const uint16_t* k, const uint16_t* v, const int32_t* slots, uint16_t* kc, uint16_t* vc, int rows,
                  int kvh, int dim, int bs, int blocks, int threads);
void ora_silu(const uint16_t* packed, uint16_t* out, int rows, int intermediate, int threads);
/* Serial per-row scan (nv_sample). */
void ora_sample(const uint16_t* logits, const float* temps, const uint64_t* seeds, int32_t* out, int batch, int vocab,
                int threads);
/* The reference's two-stage reduction with `width`-token partitions
 * (nv_sample_parallel uses 2048), partials included. */
void ora_sample_partitioned(const uint16_t* logits, const float* temps, const uint64_t* seeds, int32_t* out,
                            float* partial_scores, int32_t* partial_ids, int batch, int vocab, int width);

/* Paged causal GQA attention (nv_attention); q, out [rows, qh, dim];
 * caches [blocks, bs, kvh, dim]; tables [batch, stride]. */
void ora_attention(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, const int32_t* positions,
                   const int32_t* seqs, const int32_t* tables, uint16_t* out, int rows, int qh, int kvh, int dim,
                   int bs, int blocks, int stride, int batch, int max_context, int threads);

/* Deterministic synthetic data: SplitMix64 stream `seed`, Box-Muller in
 * binary64, rounded to bf16. */
void ora_fill_normal_bf16(uint16_t* out, size_t n, uint64_t seed, double mean, double stddev);

#ifdef __cplusplus
}
#endif

#endif /* NVR_ORACLE_H */
