// C++ host API over the nv_* C ABI: the object model and argument checks of
// nano-vllm-rs's src/gpu.rs (Gpu, Buffer, Graph; src/gpu.rs:214-1146).
//
// Ownership follows the reference: a Gpu owns one context (device, stream,
// BLAS handle); every Buffer keeps its allocation and the context alive, and
// views (Buffer::slice) share the allocation; a Graph keeps every buffer its
// capture touched alive. Failures throw nvr::Error with the reference's
// messages. Objects are not thread-safe (one context = one stream; the
// reference's Rc types are !Send as well).
//
// Link with libnano_hip.so; this file needs no HIP headers.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <initializer_list>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "../../include/nano_hip.h"

namespace nvr {

class Error : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};

// Argument checks of src/gpu.rs:214-241.
void check(int status);                                                 // non-zero -> Error with nv_last_error()
int dimension(std::size_t value);                                       // 0 < value <= INT_MAX
std::size_t extent(std::initializer_list<std::size_t> dims, std::size_t element_size);
void positive(float value, const char* name);                           // finite and > 0
void heads(std::size_t qheads, std::size_t kvheads, std::size_t head_dim);  // src/gpu.rs:643-660

namespace detail {
struct Context;
struct Allocation;
}  // namespace detail

class Buffer {
public:
    Buffer() = default;  // empty; holds no allocation
    std::size_t len() const { return bytes_; }
    bool empty() const { return bytes_ == 0; }
    // A checked view of `bytes` bytes at `offset`; it keeps the allocation alive.
    Buffer slice(std::size_t offset, std::size_t bytes) const;
    bool overlaps(const Buffer& other) const;

    void upload_bytes(const std::vector<uint8_t>& values) const { upload(values.data(), values.size()); }
    void upload_i32(const std::vector<int32_t>& values) const { upload(values.data(), values.size() * 4); }
    void upload_u64(const std::vector<uint64_t>& values) const { upload(values.data(), values.size() * 8); }
    void upload_f32(const std::vector<float>& values) const { upload(values.data(), values.size() * 4); }
    void upload_u16(const std::vector<uint16_t>& values) const { upload(values.data(), values.size() * 2); }
    std::vector<uint8_t> download_bytes(std::size_t count) const { return download<uint8_t>(count); }
    std::vector<int32_t> download_i32(std::size_t count) const { return download<int32_t>(count); }
    std::vector<uint64_t> download_u64(std::size_t count) const { return download<uint64_t>(count); }
    std::vector<float> download_f32(std::size_t count) const { return download<float>(count); }
    std::vector<uint16_t> download_u16(std::size_t count) const { return download<uint16_t>(count); }

private:
    friend class Gpu;
    Buffer(std::shared_ptr<detail::Allocation> allocation, std::size_t offset, std::size_t bytes)
        : allocation_(std::move(allocation)), offset_(offset), bytes_(bytes) {}
    void* ptr() const;
    void bounds(std::size_t bytes) const;
    void upload(const void* data, std::size_t bytes) const;
    void download_into(void* data, std::size_t bytes) const;
    template <class T>
    std::vector<T> download(std::size_t count) const {
        if (count > SIZE_MAX / sizeof(T)) throw Error("download byte count overflow");
        std::vector<T> out(count);
        download_into(out.data(), count * sizeof(T));
        return out;
    }

    std::shared_ptr<detail::Allocation> allocation_;
    std::size_t offset_ = 0;
    std::size_t bytes_ = 0;
};

class Graph {
public:
    Graph(const Graph&) = delete;
    Graph& operator=(const Graph&) = delete;
    Graph(Graph&&) noexcept;
    Graph& operator=(Graph&&) noexcept;
    ~Graph();
    void replay() const;

private:
    friend class Gpu;
    Graph(std::shared_ptr<detail::Context> context, void* handle, std::vector<Buffer> buffers);
    std::shared_ptr<detail::Context> context_;
    void* handle_ = nullptr;
    std::vector<Buffer> buffers_;  // captured allocations stay alive with the graph
};

class Gpu {
public:
    explicit Gpu(int device);

    Buffer alloc(std::size_t bytes) const;  // zero-filled
    void sync() const;
    std::pair<std::size_t, std::size_t> mem_info() const;  // (free, total) bytes
    std::size_t sm_count() const;                          // compute units
    // Captures the device work `forward` enqueues; allocation, transfers and
    // synchronisation inside it throw.
    Graph capture(const std::function<void()>& forward) const;

    // Y[m, n] = X[m, k] * W[n, k]^T, bf16 in/out, fp32 accumulation.
    void gemm(const Buffer& x, const Buffer& w, const Buffer& y, std::size_t m, std::size_t n, std::size_t k) const;
    void embedding(const Buffer& tokens, const Buffer& weight, const Buffer& out, std::size_t rows,
                   std::size_t hidden, std::size_t vocab) const;
    void rms_norm(const Buffer& x, const Buffer& weight, const Buffer& out, std::size_t rows, std::size_t hidden,
                  float eps) const;
    // residual <- bf16(x + residual); out <- RMSNorm(f32(x) + f32(residual)).
    void add_rms_norm(const Buffer& x, const Buffer& residual, const Buffer& weight, const Buffer& out,
                      std::size_t rows, std::size_t hidden, float eps) const;
    void qkv_rope(const Buffer& qkv, const Buffer& qweight, const Buffer& kweight, const Buffer& positions,
                  const Buffer& slots, const Buffer& qout, const Buffer& kcache, const Buffer& vcache,
                  std::size_t rows, std::size_t qheads, std::size_t kvheads, std::size_t head_dim,
                  std::size_t block_size, std::size_t num_blocks, float eps, float theta) const;
    // f32 [max_positions, head_dim]: cos of the head_dim/2 pairs, then sin.
    void rope_cache(const Buffer& cache, std::size_t max_positions, std::size_t head_dim, float theta) const;
    void qkv_rope_cached(const Buffer& qkv, const Buffer& qweight, const Buffer& kweight, const Buffer& positions,
                         const Buffer& slots, const Buffer& qout, const Buffer& kcache, const Buffer& vcache,
                         std::size_t rows, std::size_t qheads, std::size_t kvheads, std::size_t head_dim,
                         std::size_t block_size, std::size_t num_blocks, float eps, const Buffer& rope_cache,
                         std::size_t max_positions) const;
    // Causal paged GQA over flattened ragged prefill and decode rows; KV layout
    // [blocks, block_size, kvheads, head_dim]; row r reads positions[r] + 1 keys.
    void paged_attention(const Buffer& q, const Buffer& kcache, const Buffer& vcache, const Buffer& positions,
                         const Buffer& seq_indices, const Buffer& block_tables, const Buffer& out, std::size_t rows,
                         std::size_t qheads, std::size_t kvheads, std::size_t head_dim, std::size_t block_size,
                         std::size_t num_blocks, std::size_t table_stride, std::size_t batch_size,
                         std::size_t max_context) const;
    // Decode form of qkv_rope_cached followed by paged_attention (head dim 128):
    // one launch, and the rotated q stays on chip. No row may read a KV slot
    // that another row writes.
    void attention_qkv_rope(const Buffer& qkv, const Buffer& qweight, const Buffer& kweight, const Buffer& positions,
                            const Buffer& slots, const Buffer& kcache, const Buffer& vcache,
                            const Buffer& seq_indices, const Buffer& block_tables, const Buffer& out,
                            std::size_t rows, std::size_t qheads, std::size_t kvheads, std::size_t head_dim,
                            std::size_t block_size, std::size_t num_blocks, std::size_t table_stride,
                            std::size_t batch_size, std::size_t max_context, float eps, const Buffer& rope_cache,
                            std::size_t max_positions) const;
    void silu_mul(const Buffer& gateup, const Buffer& out, std::size_t rows, std::size_t intermediate) const;
    void gather(const Buffer& x, const Buffer& indices, const Buffer& out, std::size_t rows, std::size_t hidden,
                std::size_t input_rows) const;
    // bf16 logits; f32 temperatures (<= 0: greedy); u64 seeds; i32 out.
    void sample(const Buffer& logits, const Buffer& temperatures, const Buffer& seeds, const Buffer& out,
                std::size_t batch, std::size_t vocab) const;
    // Scratch: [batch, ceil(vocab / 2048)] f32 scores and i32 ids.
    void sample_parallel(const Buffer& logits, const Buffer& temperatures, const Buffer& seeds, const Buffer& out,
                         const Buffer& partial_scores, const Buffer& partial_ids, std::size_t batch,
                         std::size_t vocab) const;
    // Standalone paged KV slot write (no Rust caller in the reference).
    void kv_write(const Buffer& k, const Buffer& v, const Buffer& slots, const Buffer& kcache, const Buffer& vcache,
                  std::size_t rows, std::size_t kvheads, std::size_t head_dim, std::size_t block_size,
                  std::size_t num_blocks) const;

    // Extent, alignment and context checks of one tensor argument (and, during
    // capture, retention of its allocation by the graph).
    void tensor(const Buffer& buffer, std::initializer_list<std::size_t> dims, std::size_t element_size) const;
    // Throws when `output` overlaps any of `inputs`.
    static void distinct(const Buffer& output, std::initializer_list<const Buffer*> inputs);

private:
    nv_context* handle() const;
    void check_qkv_rope(const Buffer& qkv, const Buffer& qweight, const Buffer& kweight, const Buffer& positions,
                        const Buffer& slots, const Buffer& qout, const Buffer& kcache, const Buffer& vcache,
                        std::size_t rows, std::size_t qheads, std::size_t kvheads, std::size_t head_dim,
                        std::size_t block_size, std::size_t num_blocks, float eps) const;
    std::shared_ptr<detail::Context> context_;
};

// Host-side seed of src/runtime.rs:780-790.
inline uint64_t sampling_seed(uint64_t base, uint64_t request_id, uint64_t generated) {
    return nv_sampling_seed(base, request_id, generated);
}

}  // namespace nvr
