// C++ host API over the nv_* C ABI of libnano_hip.so, used by the Qwen3 runner
// (model.hpp), decode_bench and the C++ tests.
//
// The class and method names follow the Rust host of nano-vllm-rs
// (src/gpu.rs: Gpu, Buffer, Graph, one method per kernel) so that callers read
// the same in either language. The checks are this library's own contract:
//
//  Tensor arguments. A kernel call lists its tensor arguments, each with a
//  name, whether the kernel writes it, an element width and a shape, and one
//  routine (Gpu::admit) checks them all before the C call:
//    - every dimension is in [1, INT_MAX] and the byte count fits size_t
//      (Fault::Dimension, Fault::Extent);
//    - the view holds at least that many bytes (Fault::Extent);
//    - the view starts at a multiple of the element width (Fault::Alignment);
//    - the buffer was allocated by this Gpu (Fault::Foreign);
//    - the bytes a written argument covers overlap no byte that another
//      argument covers (Fault::Overlap): outputs alias nothing.
//  Scalars. eps and theta must be finite and positive; q heads a multiple of
//  KV heads, head_dim even and at most 256, q + KV heads at most 65535
//  (Fault::Value).
//  Capture. The library itself refuses allocation, transfers and
//  synchronisation while its stream is being captured (status -2, surfaced
//  as Fault::Backend). A capture here only records the allocations its
//  kernels use, and the Graph keeps them alive.
//
// Memory ownership: a Buffer is a view (offset, length) of a reference-counted
// device allocation, which in turn holds the device context; the context is
// destroyed (after a stream synchronisation) when its last user goes. Objects
// are single-threaded: one context is one stream.
//
// This header needs no HIP headers; link libnvr_host.a and libnano_hip.so.
#pragma once

#include <array>
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

// What a failure was about; tests assert on it rather than on message text.
enum class Fault { Backend, Dimension, Extent, Alignment, Foreign, Overlap, Value, Batch };
const char* fault_name(Fault fault);

class Error : public std::runtime_error {
public:
    Error(Fault fault, const std::string& what) : std::runtime_error(what), fault_(fault) {}
    Fault fault() const { return fault_; }

private:
    Fault fault_;
};

// Throws Fault::Backend carrying nv_last_error() when status != 0.
void require_status(int status);
// value as a kernel dimension: 1 <= value <= INT_MAX, else Fault::Dimension.
int as_dim(std::size_t value);
// width * prod(dims), every dimension checked by as_dim; Fault::Extent on overflow.
std::size_t byte_count(std::initializer_list<std::size_t> dims, std::size_t width);
// Fault::Value unless value is finite and > 0.
void require_positive(float value, const char* what);
// Fault::Value unless the head layout is one the kernels take (see above).
void require_head_layout(std::size_t qheads, std::size_t kvheads, std::size_t head_dim);

// The [2 * intermediate, k] gate_up weight (gate rows, then up rows) in the
// tile row order rms_gemm_silu reads.
std::vector<uint16_t> tile_gate_up_rows(const std::vector<uint16_t>& gate_up, std::size_t intermediate,
                                        std::size_t k);

namespace detail {
struct Device;
struct Allocation;
}  // namespace detail

class Buffer {
public:
    Buffer() = default;  // empty: no allocation
    std::size_t len() const { return length_; }
    bool empty() const { return length_ == 0; }
    // A view of `bytes` bytes starting `offset` bytes into this view; it
    // shares (and keeps alive) the allocation.
    Buffer slice(std::size_t offset, std::size_t bytes) const;
    // True when both views have bytes in one allocation in common.
    bool overlaps(const Buffer& other) const;

    // Synchronous copies (the library waits for its stream before returning).
    void upload_bytes(const std::vector<uint8_t>& values) const { write(values.data(), values.size()); }
    void upload_i32(const std::vector<int32_t>& values) const { write(values.data(), values.size() * 4); }
    void upload_u64(const std::vector<uint64_t>& values) const { write(values.data(), values.size() * 8); }
    void upload_f32(const std::vector<float>& values) const { write(values.data(), values.size() * 4); }
    void upload_u16(const std::vector<uint16_t>& values) const { write(values.data(), values.size() * 2); }
    std::vector<uint8_t> download_bytes(std::size_t count) const { return fetch<uint8_t>(count); }
    std::vector<int32_t> download_i32(std::size_t count) const { return fetch<int32_t>(count); }
    std::vector<uint64_t> download_u64(std::size_t count) const { return fetch<uint64_t>(count); }
    std::vector<float> download_f32(std::size_t count) const { return fetch<float>(count); }
    std::vector<uint16_t> download_u16(std::size_t count) const { return fetch<uint16_t>(count); }

private:
    friend class Gpu;
    Buffer(std::shared_ptr<detail::Allocation> allocation, std::size_t offset, std::size_t length)
        : allocation_(std::move(allocation)), offset_(offset), length_(length) {}
    void* address() const;
    void write(const void* data, std::size_t bytes) const;
    void read(void* data, std::size_t bytes) const;
    template <class T>
    std::vector<T> fetch(std::size_t count) const {
        if (count > length_ / sizeof(T))
            throw Error(Fault::Extent, "download of " + std::to_string(count) + " elements of " +
                                           std::to_string(sizeof(T)) + " bytes from a " + std::to_string(length_) +
                                           "-byte view");
        std::vector<T> out(count);
        read(out.data(), count * sizeof(T));
        return out;
    }

    std::shared_ptr<detail::Allocation> allocation_;
    std::size_t offset_ = 0;
    std::size_t length_ = 0;
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
    Graph(std::shared_ptr<detail::Device> device, void* exec, std::vector<std::shared_ptr<detail::Allocation>> held);
    void release() noexcept;
    std::shared_ptr<detail::Device> device_;
    void* exec_ = nullptr;
    std::vector<std::shared_ptr<detail::Allocation>> held_;  // allocations the captured kernels use
};

// One tensor argument of a kernel call, for Gpu::admit.
struct TensorArg {
    const char* name;
    const Buffer* buffer;
    std::size_t width;  // bytes per element
    std::array<std::size_t, 4> dims;
    int rank;
    bool written;
};
TensorArg read_arg(const char* name, const Buffer& b, std::size_t width, std::initializer_list<std::size_t> dims);
TensorArg write_arg(const char* name, const Buffer& b, std::size_t width, std::initializer_list<std::size_t> dims);

class Gpu {
public:
    explicit Gpu(int device);

    Buffer alloc(std::size_t bytes) const;  // zero-filled
    void sync() const;
    std::pair<std::size_t, std::size_t> mem_info() const;  // (free, total) bytes
    std::size_t sm_count() const;                          // compute units
    // Records the device work `forward` enqueues into a graph.
    Graph capture(const std::function<void()>& forward) const;

    // Checks every tensor argument of kernel `op` (the contract above) and,
    // during a capture, records their allocations.
    void admit(const char* op, std::initializer_list<TensorArg> args) const;
    void admit(const char* op, const std::vector<TensorArg>& args) const;

    // Y[m, n] = X[m, k] * W[n, k]^T, bf16 in/out, fp32 accumulation.
    void gemm(const Buffer& x, const Buffer& w, const Buffer& y, std::size_t m, std::size_t n, std::size_t k) const;
    void embedding(const Buffer& tokens, const Buffer& weight, const Buffer& out, std::size_t rows,
                   std::size_t hidden, std::size_t vocab) const;
    void rms_norm(const Buffer& x, const Buffer& weight, const Buffer& out, std::size_t rows, std::size_t hidden,
                  float eps) const;
    // residual <- bf16(x + residual); out <- RMSNorm(f32(x) + f32(residual)).
    void add_rms_norm(const Buffer& x, const Buffer& residual, const Buffer& weight, const Buffer& out,
                      std::size_t rows, std::size_t hidden, float eps) const;
    // Y[m, n] = X[m, k] * W[n, k]^T for 1 <= m <= 32 rows on this library's
    // MFMA kernel (n % 16 == 0, k in {1024, 2048, 3072, 4096}).
    void gemm_rows(const Buffer& x, const Buffer& w, const Buffer& y, std::size_t m, std::size_t n,
                   std::size_t k) const;
    // y = bf16(RMSNorm(x [+ residual]) W^T) for 1 <= m <= 32 rows (n % 16 == 0,
    // k in {512, 1024, 2048}); residual_out <- bf16(x + residual) in another
    // buffer and normed <- the normalised rows, each when not empty.
    void rms_gemm(const Buffer& x, const Buffer& residual, const Buffer& residual_out, const Buffer& norm_weight,
                  const Buffer& w, const Buffer& y, const Buffer& normed, std::size_t m, std::size_t n,
                  std::size_t k, float eps) const;
    // rms_gemm on the gate_up weight in tile row order (tile t: gate rows
    // 8t..8t+7, then up rows 8t..8t+7; see tile_gate_up_rows) with SiLU·up as
    // the epilogue: act <- silu(gate) * up; gate_up (when not empty) <- the
    // GEMM output in [gate | up] order.
    void rms_gemm_silu(const Buffer& x, const Buffer& residual, const Buffer& residual_out,
                       const Buffer& norm_weight, const Buffer& w_tiled, const Buffer& gate_up, const Buffer& act,
                       const Buffer& normed, std::size_t m, std::size_t intermediate, std::size_t k, float eps) const;
    // add_rms_norm's output for input rows indices[r] in output row r (+0
    // rows for indices outside [0, input_rows)); residual is only read.
    void add_rms_norm_gather(const Buffer& x, const Buffer& residual, const Buffer& weight, const Buffer& indices,
                             const Buffer& out, std::size_t rows, std::size_t hidden, std::size_t input_rows,
                             float eps) const;
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
    // The same without caller scratch (the library's static partials).
    void sample_parallel_static(const Buffer& logits, const Buffer& temperatures, const Buffer& seeds,
                                const Buffer& out, std::size_t batch, std::size_t vocab) const;
    // Standalone paged KV slot write (no Rust caller in the reference).
    void kv_write(const Buffer& k, const Buffer& v, const Buffer& slots, const Buffer& kcache, const Buffer& vcache,
                  std::size_t rows, std::size_t kvheads, std::size_t head_dim, std::size_t block_size,
                  std::size_t num_blocks) const;

private:
    nv_context* context() const;
    std::shared_ptr<detail::Device> device_;
};

// Host-side seed of src/runtime.rs:780-790.
inline uint64_t sampling_seed(uint64_t base, uint64_t request_id, uint64_t generated) {
    return nv_sampling_seed(base, request_id, generated);
}

}  // namespace nvr
