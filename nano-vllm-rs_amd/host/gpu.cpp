// C++ host API over the nv_* C ABI (see gpu.hpp); the checks restate
// src/gpu.rs:214-1146 of nano-vllm-rs.
#include "gpu.hpp"

#include <climits>
#include <cmath>
#include <sstream>

namespace nvr {

namespace detail {

struct Context {
    nv_context* handle = nullptr;
    bool capturing = false;
    std::vector<Buffer> captured;  // allocations touched by the capture in progress

    ~Context() {
        if (handle) nv_destroy(handle);  // synchronises first
    }
    void outside_capture() const {
        if (capturing) throw Error("allocation, transfer and synchronization are forbidden during graph capture");
    }
};

struct Allocation {
    std::shared_ptr<Context> context;
    void* ptr = nullptr;
    std::size_t bytes = 0;

    ~Allocation() { nv_free(context->handle, ptr); }
};

}  // namespace detail

namespace {

template <class... Args>
std::string format(const Args&... args) {
    std::ostringstream s;
    (s << ... << args);
    return s.str();
}

}  // namespace

// ------------------------------------------------------------------ checks --
void check(int status) {
    if (status == 0) return;
    const char* message = nv_last_error();
    throw Error(format("HIP backend: ", message ? message : "", " (status ", status, ")"));
}

int dimension(std::size_t value) {
    if (value == 0) throw Error("tensor dimensions must be positive");
    if (value > std::size_t(INT_MAX)) throw Error(format("dimension ", value, " exceeds i32"));
    return int(value);
}

std::size_t extent(std::initializer_list<std::size_t> dims, std::size_t element_size) {
    std::size_t n = element_size;
    for (std::size_t d : dims) {
        dimension(d);
        if (n > SIZE_MAX / d) throw Error("tensor byte count overflow");
        n *= d;
    }
    return n;
}

void positive(float value, const char* name) {
    if (!(std::isfinite(value) && value > 0.0f)) throw Error(format(name, " must be positive and finite"));
}

void heads(std::size_t qheads, std::size_t kvheads, std::size_t head_dim) {
    dimension(qheads);
    dimension(kvheads);
    dimension(head_dim);
    if (qheads % kvheads != 0) throw Error("query heads must be a multiple of KV heads");
    if (head_dim % 2 != 0 || head_dim > 256) throw Error("head dimension must be even and at most 256");
    if (qheads + kvheads > 65535) throw Error("too many heads for one launch");
}

// ------------------------------------------------------------------ Buffer --
void* Buffer::ptr() const { return static_cast<char*>(allocation_->ptr) + offset_; }

void Buffer::bounds(std::size_t bytes) const {
    if (bytes > bytes_) throw Error(format("buffer needs ", bytes, " bytes, allocation has ", bytes_));
}

Buffer Buffer::slice(std::size_t offset, std::size_t bytes) const {
    if (offset > SIZE_MAX - bytes) throw Error("buffer view extent overflow");
    bounds(offset + bytes);
    if (offset_ > SIZE_MAX - offset) throw Error("buffer view offset overflow");
    const std::size_t start = offset_ + offset;
    if (start > allocation_->bytes || bytes > allocation_->bytes - start) throw Error("buffer view exceeds allocation");
    return Buffer(allocation_, start, bytes);
}

bool Buffer::overlaps(const Buffer& other) const {
    return bytes_ > 0 && other.bytes_ > 0 && allocation_ == other.allocation_ &&
           offset_ < other.offset_ + other.bytes_ && other.offset_ < offset_ + bytes_;
}

void Buffer::upload(const void* data, std::size_t bytes) const {
    allocation_->context->outside_capture();
    bounds(bytes);
    if (bytes == 0) return;
    check(nv_upload(allocation_->context->handle, ptr(), data, bytes));  // synchronises
}

void Buffer::download_into(void* data, std::size_t bytes) const {
    allocation_->context->outside_capture();
    bounds(bytes);
    if (bytes == 0) return;
    check(nv_download(allocation_->context->handle, ptr(), data, bytes));  // synchronises
}

// ------------------------------------------------------------------- Graph --
Graph::Graph(std::shared_ptr<detail::Context> context, void* handle, std::vector<Buffer> buffers)
    : context_(std::move(context)), handle_(handle), buffers_(std::move(buffers)) {}

Graph::Graph(Graph&& other) noexcept
    : context_(std::move(other.context_)), handle_(other.handle_), buffers_(std::move(other.buffers_)) {
    other.handle_ = nullptr;
}

Graph& Graph::operator=(Graph&& other) noexcept {
    if (this != &other) {
        if (handle_) nv_graph_destroy(context_->handle, handle_);
        context_ = std::move(other.context_);
        handle_ = other.handle_;
        buffers_ = std::move(other.buffers_);
        other.handle_ = nullptr;
    }
    return *this;
}

Graph::~Graph() {
    if (handle_) nv_graph_destroy(context_->handle, handle_);
}

void Graph::replay() const {
    context_->outside_capture();
    check(nv_graph_replay(context_->handle, handle_));
}

// --------------------------------------------------------------------- Gpu --
Gpu::Gpu(int device) {
    if (device < 0) throw Error("device index must be nonnegative");
    nv_context* ctx = nullptr;
    check(nv_create(device, &ctx));
    if (!ctx) throw Error("the backend returned a null context");
    context_ = std::make_shared<detail::Context>();
    context_->handle = ctx;
}

nv_context* Gpu::handle() const { return context_->handle; }

Buffer Gpu::alloc(std::size_t bytes) const {
    context_->outside_capture();
    if (bytes == 0 || bytes > std::size_t(PTRDIFF_MAX)) throw Error(format("invalid allocation size ", bytes));
    void* ptr = nullptr;
    check(nv_alloc(handle(), bytes, &ptr));
    if (!ptr) throw Error("the backend returned a null allocation");
    auto allocation = std::make_shared<detail::Allocation>();
    allocation->context = context_;
    allocation->ptr = ptr;
    allocation->bytes = bytes;
    return Buffer(std::move(allocation), 0, bytes);
}

void Gpu::sync() const {
    context_->outside_capture();
    check(nv_sync(handle()));
}

std::pair<std::size_t, std::size_t> Gpu::mem_info() const {
    context_->outside_capture();
    std::size_t free_bytes = 0, total = 0;
    check(nv_mem_info(handle(), &free_bytes, &total));
    return {free_bytes, total};
}

std::size_t Gpu::sm_count() const {
    int n = 0;
    check(nv_sm_count(handle(), &n));
    if (n <= 0) throw Error("invalid compute unit count");
    return std::size_t(n);
}

void Gpu::tensor(const Buffer& buffer, std::initializer_list<std::size_t> dims, std::size_t element_size) const {
    if (buffer.allocation_->context != context_) throw Error("buffer belongs to a different context");
    buffer.bounds(extent(dims, element_size));
    if (buffer.offset_ % element_size != 0) throw Error("tensor view is not aligned to its element size");
    if (context_->capturing) {
        for (const Buffer& b : context_->captured)
            if (b.allocation_ == buffer.allocation_) return;
        context_->captured.push_back(buffer);
    }
}

void Gpu::distinct(const Buffer& output, std::initializer_list<const Buffer*> inputs) {
    for (const Buffer* input : inputs)
        if (output.overlaps(*input)) throw Error("kernel output aliases an input or another output");
}

Graph Gpu::capture(const std::function<void()>& forward) const {
    context_->outside_capture();
    check(nv_capture_begin(handle()));
    context_->capturing = true;
    struct Guard {  // ends an interrupted capture exactly once
        detail::Context* context;
        bool active = true;
        ~Guard() {
            if (!active) return;
            nv_capture_abort(context->handle);
            context->capturing = false;
            context->captured.clear();
        }
    } guard{context_.get()};
    forward();
    void* graph = nullptr;
    const int status = nv_capture_end(handle(), &graph);  // consumes the capture, also on failure
    guard.active = false;
    context_->capturing = false;
    std::vector<Buffer> buffers = std::move(context_->captured);
    context_->captured.clear();
    check(status);
    if (!graph) throw Error("the backend returned a null graph");
    return Graph(context_, graph, std::move(buffers));
}

// ----------------------------------------------------------------- kernels --
void Gpu::gemm(const Buffer& x, const Buffer& w, const Buffer& y, std::size_t m, std::size_t n,
               std::size_t k) const {
    tensor(x, {m, k}, 2);
    tensor(w, {n, k}, 2);
    tensor(y, {m, n}, 2);
    distinct(y, {&x, &w});
    check(nv_gemm(handle(), x.ptr(), w.ptr(), y.ptr(), dimension(m), dimension(n), dimension(k)));
}

void Gpu::embedding(const Buffer& tokens, const Buffer& weight, const Buffer& out, std::size_t rows,
                    std::size_t hidden, std::size_t vocab) const {
    tensor(tokens, {rows}, 4);
    tensor(weight, {vocab, hidden}, 2);
    tensor(out, {rows, hidden}, 2);
    distinct(out, {&tokens, &weight});
    check(nv_embedding(handle(), tokens.ptr(), weight.ptr(), out.ptr(), dimension(rows), dimension(hidden),
                       dimension(vocab)));
}

void Gpu::rms_norm(const Buffer& x, const Buffer& weight, const Buffer& out, std::size_t rows, std::size_t hidden,
                   float eps) const {
    positive(eps, "RMS epsilon");
    tensor(x, {rows, hidden}, 2);
    tensor(weight, {hidden}, 2);
    tensor(out, {rows, hidden}, 2);
    distinct(out, {&x, &weight});
    check(nv_rms(handle(), x.ptr(), weight.ptr(), out.ptr(), dimension(rows), dimension(hidden), eps));
}

void Gpu::add_rms_norm(const Buffer& x, const Buffer& residual, const Buffer& weight, const Buffer& out,
                       std::size_t rows, std::size_t hidden, float eps) const {
    positive(eps, "RMS epsilon");
    tensor(x, {rows, hidden}, 2);
    tensor(residual, {rows, hidden}, 2);
    tensor(weight, {hidden}, 2);
    tensor(out, {rows, hidden}, 2);
    distinct(out, {&x, &residual, &weight});
    distinct(residual, {&x, &weight});
    check(nv_add_rms(handle(), x.ptr(), residual.ptr(), weight.ptr(), out.ptr(), dimension(rows), dimension(hidden),
                     eps));
}

void Gpu::check_qkv_rope(const Buffer& qkv, const Buffer& qweight, const Buffer& kweight, const Buffer& positions,
                         const Buffer& slots, const Buffer& qout, const Buffer& kcache, const Buffer& vcache,
                         std::size_t rows, std::size_t qheads, std::size_t kvheads, std::size_t head_dim,
                         std::size_t block_size, std::size_t num_blocks, float eps) const {
    heads(qheads, kvheads, head_dim);
    positive(eps, "RMS epsilon");
    if (kvheads > SIZE_MAX / 2 || qheads > SIZE_MAX - 2 * kvheads) throw Error("head count overflow");
    tensor(qkv, {rows, qheads + 2 * kvheads, head_dim}, 2);
    tensor(qweight, {head_dim}, 2);
    tensor(kweight, {head_dim}, 2);
    tensor(positions, {rows}, 4);
    tensor(slots, {rows}, 4);
    tensor(qout, {rows, qheads, head_dim}, 2);
    tensor(kcache, {num_blocks, block_size, kvheads, head_dim}, 2);
    tensor(vcache, {num_blocks, block_size, kvheads, head_dim}, 2);
    for (const Buffer* out : {&qout, &kcache, &vcache}) distinct(*out, {&qkv, &qweight, &kweight, &positions, &slots});
    distinct(qout, {&kcache, &vcache});
    distinct(kcache, {&vcache});
}

void Gpu::qkv_rope(const Buffer& qkv, const Buffer& qweight, const Buffer& kweight, const Buffer& positions,
                   const Buffer& slots, const Buffer& qout, const Buffer& kcache, const Buffer& vcache,
                   std::size_t rows, std::size_t qheads, std::size_t kvheads, std::size_t head_dim,
                   std::size_t block_size, std::size_t num_blocks, float eps, float theta) const {
    positive(theta, "RoPE theta");
    check_qkv_rope(qkv, qweight, kweight, positions, slots, qout, kcache, vcache, rows, qheads, kvheads, head_dim,
                   block_size, num_blocks, eps);
    check(nv_qkv_rope(handle(), qkv.ptr(), qweight.ptr(), kweight.ptr(), positions.ptr(), slots.ptr(), qout.ptr(),
                      kcache.ptr(), vcache.ptr(), dimension(rows), dimension(qheads), dimension(kvheads),
                      dimension(head_dim), dimension(block_size), dimension(num_blocks), eps, theta));
}

void Gpu::rope_cache(const Buffer& cache, std::size_t max_positions, std::size_t head_dim, float theta) const {
    heads(1, 1, head_dim);
    positive(theta, "RoPE theta");
    tensor(cache, {max_positions, head_dim}, 4);
    check(nv_rope_cache(handle(), cache.ptr(), dimension(max_positions), dimension(head_dim), theta));
}

void Gpu::qkv_rope_cached(const Buffer& qkv, const Buffer& qweight, const Buffer& kweight, const Buffer& positions,
                          const Buffer& slots, const Buffer& qout, const Buffer& kcache, const Buffer& vcache,
                          std::size_t rows, std::size_t qheads, std::size_t kvheads, std::size_t head_dim,
                          std::size_t block_size, std::size_t num_blocks, float eps, const Buffer& rope_cache,
                          std::size_t max_positions) const {
    check_qkv_rope(qkv, qweight, kweight, positions, slots, qout, kcache, vcache, rows, qheads, kvheads, head_dim,
                   block_size, num_blocks, eps);
    tensor(rope_cache, {max_positions, head_dim}, 4);
    for (const Buffer* out : {&qout, &kcache, &vcache}) distinct(*out, {&rope_cache});
    check(nv_qkv_rope_cached(handle(), qkv.ptr(), qweight.ptr(), kweight.ptr(), positions.ptr(), slots.ptr(),
                             qout.ptr(), kcache.ptr(), vcache.ptr(), dimension(rows), dimension(qheads),
                             dimension(kvheads), dimension(head_dim), dimension(block_size), dimension(num_blocks),
                             eps, rope_cache.ptr(), dimension(max_positions)));
}

void Gpu::paged_attention(const Buffer& q, const Buffer& kcache, const Buffer& vcache, const Buffer& positions,
                          const Buffer& seq_indices, const Buffer& block_tables, const Buffer& out, std::size_t rows,
                          std::size_t qheads, std::size_t kvheads, std::size_t head_dim, std::size_t block_size,
                          std::size_t num_blocks, std::size_t table_stride, std::size_t batch_size,
                          std::size_t max_context) const {
    heads(qheads, kvheads, head_dim);
    if (max_context == 0 || max_context > 4096) throw Error("paged attention supports at most 4096 context tokens");
    tensor(q, {rows, qheads, head_dim}, 2);
    tensor(out, {rows, qheads, head_dim}, 2);
    tensor(kcache, {num_blocks, block_size, kvheads, head_dim}, 2);
    tensor(vcache, {num_blocks, block_size, kvheads, head_dim}, 2);
    tensor(positions, {rows}, 4);
    tensor(seq_indices, {rows}, 4);
    tensor(block_tables, {batch_size, table_stride}, 4);
    distinct(out, {&q, &kcache, &vcache, &positions, &seq_indices, &block_tables});
    check(nv_attention(handle(), q.ptr(), kcache.ptr(), vcache.ptr(), positions.ptr(), seq_indices.ptr(),
                       block_tables.ptr(), out.ptr(), dimension(rows), dimension(qheads), dimension(kvheads),
                       dimension(head_dim), dimension(block_size), dimension(num_blocks), dimension(table_stride),
                       dimension(batch_size), dimension(max_context)));
}

void Gpu::attention_qkv_rope(const Buffer& qkv, const Buffer& qweight, const Buffer& kweight,
                             const Buffer& positions, const Buffer& slots, const Buffer& kcache,
                             const Buffer& vcache, const Buffer& seq_indices, const Buffer& block_tables,
                             const Buffer& out, std::size_t rows, std::size_t qheads, std::size_t kvheads,
                             std::size_t head_dim, std::size_t block_size, std::size_t num_blocks,
                             std::size_t table_stride, std::size_t batch_size, std::size_t max_context, float eps,
                             const Buffer& rope_cache, std::size_t max_positions) const {
    if (head_dim != 128) throw Error("fused attention needs head_dim 128");
    if (max_context == 0 || max_context > 4096) throw Error("paged attention supports at most 4096 context tokens");
    tensor(out, {rows, qheads, head_dim}, 2);
    tensor(seq_indices, {rows}, 4);
    tensor(block_tables, {batch_size, table_stride}, 4);
    tensor(rope_cache, {max_positions, head_dim}, 4);
    // The q/k norm + RoPE prologue reads and writes what qkv_rope_cached does
    // (qout is not written: q stays on chip).
    check_qkv_rope(qkv, qweight, kweight, positions, slots, out, kcache, vcache, rows, qheads, kvheads, head_dim,
                   block_size, num_blocks, eps);
    distinct(out, {&qkv, &kcache, &vcache, &positions, &seq_indices, &block_tables, &rope_cache});
    for (const Buffer* cache : {&kcache, &vcache}) distinct(*cache, {&rope_cache, &seq_indices, &block_tables});
    check(nv_attention_qkv_rope(handle(), qkv.ptr(), qweight.ptr(), kweight.ptr(), positions.ptr(), slots.ptr(),
                                kcache.ptr(), vcache.ptr(), seq_indices.ptr(), block_tables.ptr(), out.ptr(),
                                dimension(rows), dimension(qheads), dimension(kvheads), dimension(head_dim),
                                dimension(block_size), dimension(num_blocks), dimension(table_stride),
                                dimension(batch_size), dimension(max_context), eps, rope_cache.ptr(),
                                dimension(max_positions)));
}

void Gpu::silu_mul(const Buffer& gateup, const Buffer& out, std::size_t rows, std::size_t intermediate) const {
    tensor(gateup, {rows, 2, intermediate}, 2);
    tensor(out, {rows, intermediate}, 2);
    if (intermediate > std::size_t(INT_MAX) / 2) throw Error("intermediate size too large");
    distinct(out, {&gateup});
    check(nv_silu(handle(), gateup.ptr(), out.ptr(), dimension(rows), dimension(intermediate)));
}

void Gpu::gather(const Buffer& x, const Buffer& indices, const Buffer& out, std::size_t rows, std::size_t hidden,
                 std::size_t input_rows) const {
    tensor(x, {input_rows, hidden}, 2);
    tensor(indices, {rows}, 4);
    tensor(out, {rows, hidden}, 2);
    distinct(out, {&x, &indices});
    check(nv_gather(handle(), x.ptr(), indices.ptr(), out.ptr(), dimension(rows), dimension(hidden),
                    dimension(input_rows)));
}

void Gpu::sample(const Buffer& logits, const Buffer& temperatures, const Buffer& seeds, const Buffer& out,
                 std::size_t batch, std::size_t vocab) const {
    tensor(logits, {batch, vocab}, 2);
    tensor(temperatures, {batch}, 4);
    tensor(seeds, {batch}, 8);
    tensor(out, {batch}, 4);
    distinct(out, {&logits, &temperatures, &seeds});
    check(nv_sample(handle(), logits.ptr(), temperatures.ptr(), seeds.ptr(), out.ptr(), dimension(batch),
                    dimension(vocab)));
}

void Gpu::sample_parallel(const Buffer& logits, const Buffer& temperatures, const Buffer& seeds, const Buffer& out,
                          const Buffer& partial_scores, const Buffer& partial_ids, std::size_t batch,
                          std::size_t vocab) const {
    tensor(logits, {batch, vocab}, 2);
    tensor(temperatures, {batch}, 4);
    tensor(seeds, {batch}, 8);
    tensor(out, {batch}, 4);
    const std::size_t parts = (vocab + 2047) / 2048;
    tensor(partial_scores, {batch, parts}, 4);
    tensor(partial_ids, {batch, parts}, 4);
    for (const Buffer* output : {&out, &partial_scores, &partial_ids})
        distinct(*output, {&logits, &temperatures, &seeds});
    distinct(out, {&partial_scores, &partial_ids});
    distinct(partial_scores, {&partial_ids});
    check(nv_sample_parallel(handle(), logits.ptr(), temperatures.ptr(), seeds.ptr(), out.ptr(),
                             partial_scores.ptr(), partial_ids.ptr(), dimension(batch), dimension(vocab)));
}

void Gpu::kv_write(const Buffer& k, const Buffer& v, const Buffer& slots, const Buffer& kcache, const Buffer& vcache,
                   std::size_t rows, std::size_t kvheads, std::size_t head_dim, std::size_t block_size,
                   std::size_t num_blocks) const {
    heads(kvheads, kvheads, head_dim);
    tensor(k, {rows, kvheads, head_dim}, 2);
    tensor(v, {rows, kvheads, head_dim}, 2);
    tensor(slots, {rows}, 4);
    tensor(kcache, {num_blocks, block_size, kvheads, head_dim}, 2);
    tensor(vcache, {num_blocks, block_size, kvheads, head_dim}, 2);
    for (const Buffer* out : {&kcache, &vcache}) distinct(*out, {&k, &v, &slots});
    distinct(kcache, {&vcache});
    check(nv_kv_write(handle(), k.ptr(), v.ptr(), slots.ptr(), kcache.ptr(), vcache.ptr(), dimension(rows),
                      dimension(kvheads), dimension(head_dim), dimension(block_size), dimension(num_blocks)));
}

}  // namespace nvr
