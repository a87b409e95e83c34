/*
 * nano_hip.h — C ABI of the nano-vllm-rs fused per-layer kernels for AMD
 * Instinct MI355X (gfx950).
 *
 * Every `nv_*` entry point keeps the name, argument order and meaning of the
 * CUDA library that the nano-vllm-rs Rust host links against, so the Rust
 * declarations in src/gpu.rs:17-178 bind to this library unchanged. Each
 * declaration cites the reference definition it replaces
 * (kernels/kernels.cu:<line>) and the Rust wrapper that calls it.
 *
 * Conventions (as in the reference):
 *  - Every function returning int returns 0 on success, a HIP error code on a
 *    runtime failure, hipBLAS status + 10000 on a BLAS failure, -1 when a host
 *    allocation fails, and -2 when arguments are rejected. The message is in a
 *    thread-local buffer returned by nv_last_error().
 *  - One context = one device, one non-blocking stream, one hipBLAS handle.
 *    Kernels are asynchronous launches on that stream; they never allocate or
 *    synchronise, so every kernel entry point is safe under graph capture.
 *  - Tensor arguments are device pointers. bf16 tensors are arrays of IEEE
 *    binary32 upper halves (uint16_t); int tensors are int32; seeds are uint64.
 *  - Row-major layouts; extents and aliasing are validated by the caller
 *    (src/gpu.rs:482-509 in the reference). The kernels still guard device
 *    metadata: token ids, gather indices, KV slots and RoPE positions.
 */
#ifndef NANO_HIP_H
#define NANO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct nv_context nv_context;

/* ------------------------------------------------------------ runtime ---- */

/* kernels/kernels.cu:28 — thread-local text of the last failure. */
const char* nv_last_error(void);
/* kernels/kernels.cu:29-33 — the context's hipStream_t (src/gpu.rs:18). */
int nv_stream(nv_context* c, void** output);
/* kernels/kernels.cu:34-38 — compute-unit count (src/gpu.rs:19, sm_count). */
int nv_sm_count(nv_context* c, int* output);
/* kernels/kernels.cu:39-51 — device, non-blocking stream, hipBLAS handle. */
int nv_create(int device, nv_context** output);
/* kernels/kernels.cu:52-59 — synchronises the stream, then frees. */
void nv_destroy(nv_context* c);
/* kernels/kernels.cu:60-66 — device allocation, zero-filled on the stream.
 * Refused while the stream is being captured. */
int nv_alloc(nv_context* c, size_t bytes, void** output);
/* kernels/kernels.cu:67 */
void nv_free(nv_context* c, void* buffer);
/* kernels/kernels.cu:68-72 — host -> device, synchronous on return. */
int nv_upload(nv_context* c, void* dst, const void* src, size_t bytes);
/* kernels/kernels.cu:73-77 — device -> host, synchronous on return. */
int nv_download(nv_context* c, const void* src, void* dst, size_t bytes);
/* kernels/kernels.cu:78 */
int nv_sync(nv_context* c);
/* kernels/kernels.cu:79 */
int nv_mem_info(nv_context* c, size_t* free_bytes, size_t* total_bytes);
/* kernels/kernels.cu:80 — thread-local stream capture. */
int nv_capture_begin(nv_context* c);
/* kernels/kernels.cu:81-89 — ends capture and instantiates (hipGraphExec_t). */
int nv_capture_end(nv_context* c, void** graph);
/* kernels/kernels.cu:90-95 */
void nv_capture_abort(nv_context* c);
/* kernels/kernels.cu:96 */
int nv_graph_replay(nv_context* c, void* graph);
/* kernels/kernels.cu:97 */
void nv_graph_destroy(nv_context* c, void* graph);

/* ---------------------------------------------------------------- GEMM ---- */

/* kernels/kernels.cu:98-106 — row-major Y[m,n] = X[m,k] * W[n,k]^T, bf16 in and
 * out, fp32 accumulation, through hipBLAS (src/gpu.rs:535-560). */
int nv_gemm(nv_context* c, const void* x, const void* w, void* y, int m, int n, int k);

/* ------------------------------------------------ fused per-layer kernels ---- */

/* kernels/kernels.cu:139-144,469 — out[r,:] = weight[tokens[r],:], or +0 when
 * the token is outside [0, vocab) (src/gpu.rs:561-585). */
int nv_embedding(nv_context* c, const void* tokens, const void* weight, void* out,
                 int rows, int hidden, int vocab);

/* kernels/kernels.cu:145-164,470 — out = RMSNorm(x) * weight (src/gpu.rs:586-611). */
int nv_rms(nv_context* c, const void* x, const void* weight, void* out,
           int rows, int hidden, float eps);

/* kernels/kernels.cu:145-164,471 — v = x + residual (fp32); residual <- bf16(v);
 * out = RMSNorm(v) * weight, normalising the unrounded v (src/gpu.rs:612-642). */
int nv_add_rms(nv_context* c, const void* x, void* residual, const void* weight, void* out,
               int rows, int hidden, float eps);

/* The final add-RMSNorm and the last-token gather of src/model.rs:781-797 in
 * one launch (no single reference entry point: nv_add_rms, kernels/kernels.cu:471,
 * followed by nv_gather, :487). For output row r with i = indices[r] in
 * [0, input_rows): out[r] = nv_add_rms's output row i; other indices give a
 * +0 row. Only gathered rows are computed, and the residual is read, not
 * updated (nothing reads it after the final norm), so rows may repeat.
 * x and residual are [input_rows, hidden], out is [rows, hidden]. */
int nv_add_rms_gather(nv_context* c, const void* x, const void* residual, const void* weight,
                      const void* indices, void* out, int rows, int hidden, int input_rows,
                      float eps);

/* No single counterpart in the reference: nv_rms / nv_add_rms
 * (kernels/kernels.cu:145-164,470-471) followed by nv_gemm (:98-106) on the
 * normalised rows, in one launch for decode-sized batches
 * (src/model.rs:659-678 and :753-770). With residual == NULL, X = RMSNorm(x);
 * otherwise v = x + residual, residual_out <- bf16(v) (a different buffer from
 * residual; may be NULL) and X = RMSNorm(v), both exactly as nv_add_rms.
 * Then y[m, n] = bf16(X W^T) with fp32 accumulation in a fixed order (not
 * hipBLAS's: equal to nv_gemm to fp32 rounding). normed (may be NULL) receives
 * X. Limits (else -2): 1 <= m <= 32, n a multiple of 16, k in {512, 1024, 2048},
 * 16-byte aligned tensors. x, residual, residual_out, normed: [m, k];
 * w: [n, k]; y: [m, n]. */
int nv_rms_gemm(nv_context* c, const void* x, const void* residual, void* residual_out,
                const void* norm_weight, const void* w, void* y, void* normed, int m, int n, int k,
                float eps);

/* nv_gemm for decode-sized batches without hipBLAS (kernels/kernels.cu:98-106's
 * Y[m, n] = X[m, k] W[n, k]^T, bf16 in and out, fp32 accumulation in a fixed
 * order — on MFMA, or with dot2 instructions for outputs narrower than one
 * 16-column tile per CU at m <= 16: equal to nv_gemm to fp32 rounding, the
 * same bits on every launch of a shape). Limits (else -2): 1 <= m <= 32, n a multiple of 16,
 * k in {1024, 2048, 3072, 4096}, 16-byte aligned x and w. */
int nv_gemm_rows(nv_context* c, const void* x, const void* w, void* y, int m, int n, int k);

/* nv_rms_gemm for the gate_up projection with SiLU·up (kernels/kernels.cu:356-365,
 * nv_silu) as its epilogue: no single counterpart in the reference
 * (src/model.rs:753-770). w_tiled is the [2 * intermediate, k] gate_up weight
 * with its rows in tile order — tile t holds gate rows 8t..8t+7, then up rows
 * 8t..8t+7 — and act[m, i] = bf16(silu(gate) * up) of the bf16-rounded GEMM
 * outputs, with nv_silu's arithmetic (the same bits). gate_up (may be NULL)
 * receives the GEMM output in the reference's [m, gate | up] layout.
 * Limits as nv_rms_gemm, and intermediate a multiple of 8. */
int nv_rms_gemm_silu(nv_context* c, const void* x, const void* residual, void* residual_out,
                     const void* norm_weight, const void* w_tiled, void* gate_up, void* act, void* normed,
                     int m, int intermediate, int k, float eps);

/* kernels/kernels.cu:166-211,472 — per-head q/k RMSNorm, NeoX RoPE with the
 * angle computed inline, q -> qout, k/v -> paged caches at slots[r]
 * (src/gpu.rs:661-706). qkv is [rows, qh + 2*kvh, dim]; caches are
 * [blocks, bs, kvh, dim]. */
int nv_qkv_rope(nv_context* c, const void* qkv, const void* qw, const void* kw,
                const void* positions, const void* slots, void* qout, void* kc, void* vc,
                int rows, int qh, int kvh, int dim, int bs, int blocks, float eps, float theta);

/* kernels/kernels.cu:213-224,473 — fp32 table [positions, cos(dim/2) | sin(dim/2)]
 * (src/gpu.rs:753-773). */
int nv_rope_cache(nv_context* c, void* cache, int positions, int dim, float theta);

/* kernels/kernels.cu:166-211,474 — as nv_qkv_rope with cos/sin read from the
 * table; positions outside [0, max_positions) rotate by angle 0
 * (src/gpu.rs:774-825). */
int nv_qkv_rope_cached(nv_context* c, const void* qkv, const void* qw, const void* kw,
                       const void* positions, const void* slots, void* qout, void* kc, void* vc,
                       int rows, int qh, int kvh, int dim, int bs, int blocks, float eps,
                       const void* rope_cache, int max_positions);

/* kernels/kernels.cu:475-485 — causal paged GQA attention over flattened
 * ragged prefill and decode rows (src/gpu.rs:826-887). q, out: [rows, qh, dim]
 * bf16; kc, vc: [blocks, bs, kvh, dim] bf16; positions, seqs: [rows] i32;
 * tables: [batch, stride] i32. Row r attends to positions[r] + 1 keys of
 * sequence seqs[r] in the fp32 order of kernels/kernels.cu:226-346. Returns -2
 * for qh % kvh != 0, an odd head dim or one above 256, or max_context outside
 * [1, 4096]. */
int nv_attention(nv_context* c, const void* q, const void* kc, const void* vc,
                 const void* positions, const void* seqs, const void* tables, void* out,
                 int rows, int qh, int kvh, int dim, int bs, int blocks, int stride, int batch,
                 int max_context);

/* No single counterpart in the reference: nv_qkv_rope_cached followed by
 * nv_attention (kernels/kernels.cu:166-211,474 then 475-485) in one launch for
 * decode batches, with the same outputs (out; K and V at slots[r]) bit for bit
 * and without writing the rotated q to memory. Head dim 128 and 16-byte
 * aligned tensors only (else -2). No row may read a KV slot that another row
 * of the call writes: rows do not wait for each other's cache writes. */
int nv_attention_qkv_rope(nv_context* c, const void* qkv, const void* qw, const void* kw,
                          const void* positions, const void* slots, void* kc, void* vc,
                          const void* seqs, const void* tables, void* out, int rows, int qh, int kvh,
                          int dim, int bs, int blocks, int stride, int batch, int max_context, float eps,
                          const void* rope_cache, int max_positions);

/* kernels/kernels.cu:356-365,486 — out[r,i] = bf16(silu(gate) * up) with
 * packed = [rows, 2, intermediate] (src/gpu.rs:996-1019). */
int nv_silu(nv_context* c, const void* packed, void* out, int rows, int intermediate);

/* kernels/kernels.cu:366-371,487 — out[r,:] = x[indices[r],:], or +0 when the
 * index is outside [0, input_rows) (src/gpu.rs:1020-1043). */
int nv_gather(nv_context* c, const void* x, const void* indices, void* out,
              int rows, int hidden, int input_rows);

/* kernels/kernels.cu:372-407,488 — one token per row: greedy argmax when
 * temps[r] <= 0, else Gumbel-max with SplitMix64 noise keyed by seeds[r]
 * (src/gpu.rs:1045-1072). */
int nv_sample(nv_context* c, const void* logits, const void* temps, const void* seeds, void* out,
              int batch, int vocab);

/* kernels/kernels.cu:409-466,489-501 — same result as nv_sample through a
 * vocabulary-partitioned reduction. partial_scores (f32) and partial_ids (i32)
 * are caller scratch of batch * ceil(vocab / 2048) entries each
 * (src/gpu.rs:1073-1111). */
int nv_sample_parallel(nv_context* c, const void* logits, const void* temps, const void* seeds,
                       void* out, void* partial_scores, void* partial_ids, int batch, int vocab);

/* ------------------------------------------------- additions (no Rust caller) ---- */

/* Standalone paged KV-cache slot write: the K/V half of
 * kernels/kernels.cu:188-190,206-209 without the norm and rotation.
 * k, v are [rows, kvh, dim]; for each row with 0 <= slots[r] < bs*blocks,
 * kc[slots[r]] = k[r] and vc[slots[r]] = v[r] (bit-exact copies); other rows
 * are skipped. Slot derivation follows src/runtime.rs:747-755. */
int nv_kv_write(nv_context* c, const void* k, const void* v, const void* slots, void* kc, void* vc,
                int rows, int kvh, int dim, int bs, int blocks);

/* No counterpart in the reference: nv_sample_parallel without the caller's
 * scratch, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The partials
 * live in a static 1 MiB device array per GPU (131072 entries of f32 score +
 * i32 id), bound at nv_create; it calls no allocator. Returns -2 when
 * batch * ceil(vocab / 2048) exceeds 131072. Every call on one GPU shares that
 * array: calls that overlap on one GPU (two streams or contexts at once) race. */
int nv_sample_parallel_static(nv_context* c, const void* logits, const void* temps, const void* seeds,
                              void* out, int batch, int vocab);

/* Per-row Gumbel seed of src/runtime.rs:780-790 (host function, no device
 * work): mix(mix(base) ^ mix(request_id) ^ mix(generated)). */
uint64_t nv_sampling_seed(uint64_t base, uint64_t request_id, uint64_t generated);

#ifdef __cplusplus
}
#endif

#endif /* NANO_HIP_H */
