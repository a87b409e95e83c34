// C++ host API over the nv_* C ABI (contract in gpu.hpp): argument admission,
// buffer views, graph capture and one checked method per kernel.
#include "gpu.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdint>
#include <unordered_set>

namespace nvr {

namespace detail {

// Allocations used by the kernels of the capture in progress.
struct Recorder {
    std::vector<std::shared_ptr<Allocation>> held;
    std::unordered_set<const Allocation*> known;
    void hold(const std::shared_ptr<Allocation>& a) {
        if (known.insert(a.get()).second) held.push_back(a);
    }
};

struct Device {
    nv_context* ctx = nullptr;
    std::unique_ptr<Recorder> recorder;  // non-null while a capture runs
    ~Device() {
        if (ctx) nv_destroy(ctx);  // waits for the stream first
    }
};

struct Allocation {
    std::shared_ptr<Device> device;
    void* base = nullptr;
    std::size_t size = 0;
    ~Allocation() {
        if (base) nv_free(device->ctx, base);
    }
};

}  // namespace detail

namespace {

std::string str(std::size_t v) { return std::to_string(v); }

// width * dims[0] * ... * dims[rank - 1], each dimension in [1, INT_MAX].
std::size_t span_bytes(const std::size_t* dims, int rank, std::size_t width) {
    std::size_t bytes = width;
    for (int i = 0; i < rank; ++i) {
        as_dim(dims[i]);
        if (bytes > SIZE_MAX / dims[i]) throw Error(Fault::Extent, "tensor byte count overflows size_t");
        bytes *= dims[i];
    }
    return bytes;
}

TensorArg make_arg(const char* name, const Buffer& b, std::size_t width, std::initializer_list<std::size_t> dims,
                   bool written) {
    TensorArg a{name, &b, width, {0, 0, 0, 0}, 0, written};
    if (dims.size() > a.dims.size()) throw Error(Fault::Dimension, std::string(name) + ": more than 4 dimensions");
    for (std::size_t d : dims) a.dims[std::size_t(a.rank++)] = d;
    return a;
}

}  // namespace

const char* fault_name(Fault fault) {
    switch (fault) {
    case Fault::Backend: return "backend";
    case Fault::Dimension: return "dimension";
    case Fault::Extent: return "extent";
    case Fault::Alignment: return "alignment";
    case Fault::Foreign: return "foreign";
    case Fault::Overlap: return "overlap";
    case Fault::Value: return "value";
    case Fault::Batch: return "batch";
    }
    return "?";
}

void require_status(int status) {
    if (status == 0) return;
    const char* text = nv_last_error();
    throw Error(Fault::Backend, "libnano_hip status " + std::to_string(status) + ": " + (text ? text : ""));
}

int as_dim(std::size_t value) {
    if (value == 0 || value > std::size_t(INT_MAX))
        throw Error(Fault::Dimension, "dimension " + str(value) + " outside [1, 2^31 - 1]");
    return int(value);
}

std::size_t byte_count(std::initializer_list<std::size_t> dims, std::size_t width) {
    if (dims.size() > 8) throw Error(Fault::Dimension, "more than 8 dimensions");
    std::size_t d[8];
    int rank = 0;
    for (std::size_t v : dims) d[rank++] = v;
    return span_bytes(d, rank, width);
}

void require_positive(float value, const char* what) {
    if (!(value > 0.0f) || !std::isfinite(value))
        throw Error(Fault::Value, std::string(what) + " = " + std::to_string(value) + ", not a positive finite number");
}

void require_head_layout(std::size_t qheads, std::size_t kvheads, std::size_t head_dim) {
    as_dim(qheads);
    as_dim(kvheads);
    as_dim(head_dim);
    if (qheads % kvheads != 0)
        throw Error(Fault::Value, str(qheads) + " query heads do not group evenly over " + str(kvheads) + " KV heads");
    if (head_dim % 2 != 0 || head_dim > 256)
        throw Error(Fault::Value, "head_dim " + str(head_dim) + " is not an even number up to 256");
    if (qheads + kvheads > 65535)
        throw Error(Fault::Value, str(qheads + kvheads) + " q + KV heads exceed one launch's 65535 grid rows");
}

TensorArg read_arg(const char* name, const Buffer& b, std::size_t width, std::initializer_list<std::size_t> dims) {
    return make_arg(name, b, width, dims, false);
}
TensorArg write_arg(const char* name, const Buffer& b, std::size_t width, std::initializer_list<std::size_t> dims) {
    return make_arg(name, b, width, dims, true);
}

// ------------------------------------------------------------------ Buffer --
void* Buffer::address() const { return static_cast<char*>(allocation_->base) + offset_; }

Buffer Buffer::slice(std::size_t offset, std::size_t bytes) const {
    // This view lies inside its allocation, so a sub-range of it does too.
    if (offset > length_ || bytes > length_ - offset)
        throw Error(Fault::Extent, "sub-view [" + str(offset) + ", +" + str(bytes) + ") of a " + str(length_) +
                                       "-byte view");
    return Buffer(allocation_, offset_ + offset, bytes);
}

bool Buffer::overlaps(const Buffer& other) const {
    if (!allocation_ || allocation_ != other.allocation_ || length_ == 0 || other.length_ == 0) return false;
    return std::max(offset_, other.offset_) < std::min(offset_ + length_, other.offset_ + other.length_);
}

void Buffer::write(const void* data, std::size_t bytes) const {
    if (bytes > length_) throw Error(Fault::Extent, "upload of " + str(bytes) + " bytes into a " + str(length_) + "-byte view");
    if (bytes != 0) require_status(nv_upload(allocation_->device->ctx, address(), data, bytes));
}

void Buffer::read(void* data, std::size_t bytes) const {
    if (bytes != 0) require_status(nv_download(allocation_->device->ctx, address(), data, bytes));
}

// ------------------------------------------------------------------- Graph --
Graph::Graph(std::shared_ptr<detail::Device> device, void* exec, std::vector<std::shared_ptr<detail::Allocation>> held)
    : device_(std::move(device)), exec_(exec), held_(std::move(held)) {}

void Graph::release() noexcept {
    if (exec_) nv_graph_destroy(device_->ctx, exec_);
    exec_ = nullptr;
}

Graph::Graph(Graph&& other) noexcept
    : device_(std::move(other.device_)), exec_(std::exchange(other.exec_, nullptr)), held_(std::move(other.held_)) {}

Graph& Graph::operator=(Graph&& other) noexcept {
    if (this != &other) {
        release();
        device_ = std::move(other.device_);
        exec_ = std::exchange(other.exec_, nullptr);
        held_ = std::move(other.held_);
    }
    return *this;
}

Graph::~Graph() { release(); }

void Graph::replay() const {
    if (!exec_) throw Error(Fault::Value, "replay of an empty graph");
    require_status(nv_graph_replay(device_->ctx, exec_));
}

// --------------------------------------------------------------------- Gpu --
Gpu::Gpu(int device) {
    if (device < 0) throw Error(Fault::Value, "device index " + std::to_string(device) + " is negative");
    nv_context* ctx = nullptr;
    require_status(nv_create(device, &ctx));
    device_ = std::make_shared<detail::Device>();
    device_->ctx = ctx;
}

nv_context* Gpu::context() const { return device_->ctx; }

Buffer Gpu::alloc(std::size_t bytes) const {
    if (bytes == 0 || bytes > std::size_t(PTRDIFF_MAX)) throw Error(Fault::Extent, "allocation of " + str(bytes) + " bytes");
    void* base = nullptr;
    require_status(nv_alloc(context(), bytes, &base));
    auto a = std::make_shared<detail::Allocation>();
    a->device = device_;
    a->base = base;
    a->size = bytes;
    return Buffer(std::move(a), 0, bytes);
}

void Gpu::sync() const { require_status(nv_sync(context())); }

std::pair<std::size_t, std::size_t> Gpu::mem_info() const {
    std::size_t free_bytes = 0, total = 0;
    require_status(nv_mem_info(context(), &free_bytes, &total));
    return {free_bytes, total};
}

std::size_t Gpu::sm_count() const {
    int n = 0;
    require_status(nv_sm_count(context(), &n));
    return std::size_t(as_dim(std::size_t(std::max(n, 0))));
}

Graph Gpu::capture(const std::function<void()>& forward) const {
    detail::Device& d = *device_;
    if (d.recorder) throw Error(Fault::Value, "a capture is already running on this Gpu");
    require_status(nv_capture_begin(d.ctx));
    d.recorder = std::make_unique<detail::Recorder>();
    try {
        forward();
    } catch (...) {
        nv_capture_abort(d.ctx);
        d.recorder.reset();
        throw;
    }
    void* exec = nullptr;
    const int status = nv_capture_end(d.ctx, &exec);  // the capture is over whatever the status
    std::unique_ptr<detail::Recorder> rec = std::move(d.recorder);
    require_status(status);
    return Graph(device_, exec, std::move(rec->held));
}

void Gpu::admit(const char* op, std::initializer_list<TensorArg> args) const {
    admit(op, std::vector<TensorArg>(args));
}

void Gpu::admit(const char* op, const std::vector<TensorArg>& args) const {
    struct Span {
        const detail::Allocation* allocation;
        std::size_t begin, end;
    };
    std::vector<Span> spans;
    spans.reserve(args.size());
    for (const TensorArg& a : args) {
        const Buffer& b = *a.buffer;
        const std::string who = std::string(op) + ": argument '" + a.name + "'";
        if (!b.allocation_ || b.allocation_->device != device_)
            throw Error(Fault::Foreign, who + " was not allocated by this Gpu");
        const std::size_t need = span_bytes(a.dims.data(), a.rank, a.width);
        if (need > b.length_)
            throw Error(Fault::Extent, who + " needs " + str(need) + " bytes; its view holds " + str(b.length_));
        if (b.offset_ % a.width != 0)
            throw Error(Fault::Alignment, who + " starts at byte " + str(b.offset_) + ", not a multiple of " +
                                              str(a.width));
        spans.push_back({b.allocation_.get(), b.offset_, b.offset_ + need});
    }
    std::size_t i = 0;
    for (const TensorArg& a : args) {
        if (a.written) {
            std::size_t j = 0;
            for (const TensorArg& other : args) {
                const Span& x = spans[i];
                const Span& y = spans[j];
                if (j != i && x.allocation == y.allocation && std::max(x.begin, y.begin) < std::min(x.end, y.end))
                    throw Error(Fault::Overlap, std::string(op) + ": written argument '" + a.name +
                                                    "' shares bytes with argument '" + other.name + "'");
                ++j;
            }
        }
        ++i;
    }
    if (device_->recorder)
        for (const TensorArg& a : args) device_->recorder->hold(a.buffer->allocation_);
}

// ----------------------------------------------------------------- kernels --
void Gpu::gemm(const Buffer& x, const Buffer& w, const Buffer& y, std::size_t m, std::size_t n,
               std::size_t k) const {
    admit("gemm", {read_arg("x", x, 2, {m, k}), read_arg("w", w, 2, {n, k}), write_arg("y", y, 2, {m, n})});
    require_status(nv_gemm(context(), x.address(), w.address(), y.address(), as_dim(m), as_dim(n), as_dim(k)));
}

void Gpu::embedding(const Buffer& tokens, const Buffer& weight, const Buffer& out, std::size_t rows,
                    std::size_t hidden, std::size_t vocab) const {
    admit("embedding", {read_arg("tokens", tokens, 4, {rows}), read_arg("weight", weight, 2, {vocab, hidden}),
                        write_arg("out", out, 2, {rows, hidden})});
    require_status(nv_embedding(context(), tokens.address(), weight.address(), out.address(), as_dim(rows),
                                as_dim(hidden), as_dim(vocab)));
}

void Gpu::rms_norm(const Buffer& x, const Buffer& weight, const Buffer& out, std::size_t rows, std::size_t hidden,
                   float eps) const {
    require_positive(eps, "rms_norm eps");
    admit("rms_norm", {read_arg("x", x, 2, {rows, hidden}), read_arg("weight", weight, 2, {hidden}),
                       write_arg("out", out, 2, {rows, hidden})});
    require_status(nv_rms(context(), x.address(), weight.address(), out.address(), as_dim(rows), as_dim(hidden), eps));
}

void Gpu::add_rms_norm(const Buffer& x, const Buffer& residual, const Buffer& weight, const Buffer& out,
                       std::size_t rows, std::size_t hidden, float eps) const {
    require_positive(eps, "add_rms_norm eps");
    admit("add_rms_norm", {read_arg("x", x, 2, {rows, hidden}), write_arg("residual", residual, 2, {rows, hidden}),
                           read_arg("weight", weight, 2, {hidden}), write_arg("out", out, 2, {rows, hidden})});
    require_status(nv_add_rms(context(), x.address(), residual.address(), weight.address(), out.address(),
                              as_dim(rows), as_dim(hidden), eps));
}

void Gpu::gemm_rows(const Buffer& x, const Buffer& w, const Buffer& y, std::size_t m, std::size_t n,
                    std::size_t k) const {
    if (m < 1 || m > 32 || n % 16 != 0 || (k != 1024 && k != 2048 && k != 3072 && k != 4096))
        throw Error(Fault::Value, "gemm_rows: unsupported shape m " + std::to_string(m) + ", n " + std::to_string(n) +
                                      ", k " + std::to_string(k));
    admit("gemm_rows", {read_arg("x", x, 2, {m, k}), read_arg("w", w, 2, {n, k}), write_arg("y", y, 2, {m, n})});
    require_status(nv_gemm_rows(context(), x.address(), w.address(), y.address(), as_dim(m), as_dim(n), as_dim(k)));
}

void Gpu::rms_gemm(const Buffer& x, const Buffer& residual, const Buffer& residual_out, const Buffer& norm_weight,
                   const Buffer& w, const Buffer& y, const Buffer& normed, std::size_t m, std::size_t n,
                   std::size_t k, float eps) const {
    require_positive(eps, "rms_gemm eps");
    if (residual.empty() && !residual_out.empty())
        throw Error(Fault::Value, "rms_gemm: residual_out needs a residual to add");
    if (m < 1 || m > 32 || n % 16 != 0 || (k != 512 && k != 1024 && k != 2048))
        throw Error(Fault::Value, "rms_gemm: unsupported shape m " + std::to_string(m) + ", n " + std::to_string(n) +
                                      ", k " + std::to_string(k));
    std::vector<TensorArg> args = {read_arg("x", x, 2, {m, k}), read_arg("norm_weight", norm_weight, 2, {k}),
                                   read_arg("w", w, 2, {n, k}), write_arg("y", y, 2, {m, n})};
    if (!residual.empty()) args.push_back(read_arg("residual", residual, 2, {m, k}));
    if (!residual_out.empty()) args.push_back(write_arg("residual_out", residual_out, 2, {m, k}));
    if (!normed.empty()) args.push_back(write_arg("normed", normed, 2, {m, k}));
    admit("rms_gemm", args);
    auto ptr = [](const Buffer& b) { return b.empty() ? nullptr : b.address(); };
    require_status(nv_rms_gemm(context(), x.address(), ptr(residual), ptr(residual_out), norm_weight.address(),
                               w.address(), y.address(), ptr(normed), as_dim(m), as_dim(n), as_dim(k), eps));
}

void Gpu::rms_gemm_silu(const Buffer& x, const Buffer& residual, const Buffer& residual_out,
                        const Buffer& norm_weight, const Buffer& w_tiled, const Buffer& gate_up, const Buffer& act,
                        const Buffer& normed, std::size_t m, std::size_t intermediate, std::size_t k,
                        float eps) const {
    require_positive(eps, "rms_gemm_silu eps");
    if (residual.empty() && !residual_out.empty())
        throw Error(Fault::Value, "rms_gemm_silu: residual_out needs a residual to add");
    if (m < 1 || m > 32 || intermediate % 8 != 0 || (k != 512 && k != 1024 && k != 2048))
        throw Error(Fault::Value, "rms_gemm_silu: unsupported shape m " + std::to_string(m) + ", intermediate " +
                                      std::to_string(intermediate) + ", k " + std::to_string(k));
    std::vector<TensorArg> args = {read_arg("x", x, 2, {m, k}), read_arg("norm_weight", norm_weight, 2, {k}),
                                   read_arg("w_tiled", w_tiled, 2, {2 * intermediate, k}),
                                   write_arg("act", act, 2, {m, intermediate})};
    if (!residual.empty()) args.push_back(read_arg("residual", residual, 2, {m, k}));
    if (!residual_out.empty()) args.push_back(write_arg("residual_out", residual_out, 2, {m, k}));
    if (!gate_up.empty()) args.push_back(write_arg("gate_up", gate_up, 2, {m, 2 * intermediate}));
    if (!normed.empty()) args.push_back(write_arg("normed", normed, 2, {m, k}));
    admit("rms_gemm_silu", args);
    auto ptr = [](const Buffer& b) { return b.empty() ? nullptr : b.address(); };
    require_status(nv_rms_gemm_silu(context(), x.address(), ptr(residual), ptr(residual_out), norm_weight.address(),
                                    w_tiled.address(), ptr(gate_up), act.address(), ptr(normed), as_dim(m),
                                    as_dim(intermediate), as_dim(k), eps));
}

std::vector<uint16_t> tile_gate_up_rows(const std::vector<uint16_t>& gate_up, std::size_t intermediate,
                                        std::size_t k) {
    if (intermediate % 8 != 0 || gate_up.size() != 2 * intermediate * k)
        throw Error(Fault::Value, "tile_gate_up_rows: needs a [2 * intermediate, k] weight, intermediate % 8 == 0");
    std::vector<uint16_t> out(gate_up.size());
    for (std::size_t t = 0; t < intermediate / 8; ++t)
        for (std::size_t half = 0; half < 2; ++half)
            for (std::size_t e = 0; e < 8; ++e)
                std::copy_n(gate_up.begin() + std::ptrdiff_t((half * intermediate + 8 * t + e) * k), k,
                            out.begin() + std::ptrdiff_t((16 * t + 8 * half + e) * k));
    return out;
}

void Gpu::add_rms_norm_gather(const Buffer& x, const Buffer& residual, const Buffer& weight, const Buffer& indices,
                              const Buffer& out, std::size_t rows, std::size_t hidden, std::size_t input_rows,
                              float eps) const {
    require_positive(eps, "add_rms_norm_gather eps");
    admit("add_rms_norm_gather",
          {read_arg("x", x, 2, {input_rows, hidden}), read_arg("residual", residual, 2, {input_rows, hidden}),
           read_arg("weight", weight, 2, {hidden}), read_arg("indices", indices, 4, {rows}),
           write_arg("out", out, 2, {rows, hidden})});
    require_status(nv_add_rms_gather(context(), x.address(), residual.address(), weight.address(),
                                     indices.address(), out.address(), as_dim(rows), as_dim(hidden),
                                     as_dim(input_rows), eps));
}

namespace {
// The arguments shared by the q/k norm + RoPE + KV write kernels.
struct RopeShape {
    std::size_t rows, qheads, kvheads, head_dim, block_size, num_blocks;
    std::size_t heads() const { return qheads + 2 * kvheads; }
};
}  // namespace

void Gpu::qkv_rope(const Buffer& qkv, const Buffer& qweight, const Buffer& kweight, const Buffer& positions,
                   const Buffer& slots, const Buffer& qout, const Buffer& kcache, const Buffer& vcache,
                   std::size_t rows, std::size_t qheads, std::size_t kvheads, std::size_t head_dim,
                   std::size_t block_size, std::size_t num_blocks, float eps, float theta) const {
    require_positive(eps, "qkv_rope eps");
    require_positive(theta, "qkv_rope theta");
    require_head_layout(qheads, kvheads, head_dim);
    const RopeShape s{rows, qheads, kvheads, head_dim, block_size, num_blocks};
    admit("qkv_rope", {read_arg("qkv", qkv, 2, {rows, s.heads(), head_dim}), read_arg("qweight", qweight, 2, {head_dim}),
                       read_arg("kweight", kweight, 2, {head_dim}), read_arg("positions", positions, 4, {rows}),
                       read_arg("slots", slots, 4, {rows}), write_arg("qout", qout, 2, {rows, qheads, head_dim}),
                       write_arg("kcache", kcache, 2, {num_blocks, block_size, kvheads, head_dim}),
                       write_arg("vcache", vcache, 2, {num_blocks, block_size, kvheads, head_dim})});
    require_status(nv_qkv_rope(context(), qkv.address(), qweight.address(), kweight.address(), positions.address(),
                               slots.address(), qout.address(), kcache.address(), vcache.address(), as_dim(rows),
                               as_dim(qheads), as_dim(kvheads), as_dim(head_dim), as_dim(block_size),
                               as_dim(num_blocks), eps, theta));
}

void Gpu::rope_cache(const Buffer& cache, std::size_t max_positions, std::size_t head_dim, float theta) const {
    require_positive(theta, "rope_cache theta");
    require_head_layout(1, 1, head_dim);
    admit("rope_cache", {write_arg("cache", cache, 4, {max_positions, head_dim})});
    require_status(nv_rope_cache(context(), cache.address(), as_dim(max_positions), as_dim(head_dim), theta));
}

void Gpu::qkv_rope_cached(const Buffer& qkv, const Buffer& qweight, const Buffer& kweight, const Buffer& positions,
                          const Buffer& slots, const Buffer& qout, const Buffer& kcache, const Buffer& vcache,
                          std::size_t rows, std::size_t qheads, std::size_t kvheads, std::size_t head_dim,
                          std::size_t block_size, std::size_t num_blocks, float eps, const Buffer& rope_cache,
                          std::size_t max_positions) const {
    require_positive(eps, "qkv_rope_cached eps");
    require_head_layout(qheads, kvheads, head_dim);
    const RopeShape s{rows, qheads, kvheads, head_dim, block_size, num_blocks};
    admit("qkv_rope_cached",
          {read_arg("qkv", qkv, 2, {rows, s.heads(), head_dim}), read_arg("qweight", qweight, 2, {head_dim}),
           read_arg("kweight", kweight, 2, {head_dim}), read_arg("positions", positions, 4, {rows}),
           read_arg("slots", slots, 4, {rows}), read_arg("rope_cache", rope_cache, 4, {max_positions, head_dim}),
           write_arg("qout", qout, 2, {rows, qheads, head_dim}),
           write_arg("kcache", kcache, 2, {num_blocks, block_size, kvheads, head_dim}),
           write_arg("vcache", vcache, 2, {num_blocks, block_size, kvheads, head_dim})});
    require_status(nv_qkv_rope_cached(context(), qkv.address(), qweight.address(), kweight.address(),
                                      positions.address(), slots.address(), qout.address(), kcache.address(),
                                      vcache.address(), as_dim(rows), as_dim(qheads), as_dim(kvheads),
                                      as_dim(head_dim), as_dim(block_size), as_dim(num_blocks), eps,
                                      rope_cache.address(), as_dim(max_positions)));
}

namespace {
void require_context_limit(std::size_t max_context) {
    if (max_context == 0 || max_context > 4096)
        throw Error(Fault::Value, "max_context " + std::to_string(max_context) + " outside [1, 4096]");
}
}  // namespace

void Gpu::paged_attention(const Buffer& q, const Buffer& kcache, const Buffer& vcache, const Buffer& positions,
                          const Buffer& seq_indices, const Buffer& block_tables, const Buffer& out, std::size_t rows,
                          std::size_t qheads, std::size_t kvheads, std::size_t head_dim, std::size_t block_size,
                          std::size_t num_blocks, std::size_t table_stride, std::size_t batch_size,
                          std::size_t max_context) const {
    require_head_layout(qheads, kvheads, head_dim);
    require_context_limit(max_context);
    admit("paged_attention",
          {read_arg("q", q, 2, {rows, qheads, head_dim}),
           read_arg("kcache", kcache, 2, {num_blocks, block_size, kvheads, head_dim}),
           read_arg("vcache", vcache, 2, {num_blocks, block_size, kvheads, head_dim}),
           read_arg("positions", positions, 4, {rows}), read_arg("seq_indices", seq_indices, 4, {rows}),
           read_arg("block_tables", block_tables, 4, {batch_size, table_stride}),
           write_arg("out", out, 2, {rows, qheads, head_dim})});
    require_status(nv_attention(context(), q.address(), kcache.address(), vcache.address(), positions.address(),
                                seq_indices.address(), block_tables.address(), out.address(), as_dim(rows),
                                as_dim(qheads), as_dim(kvheads), as_dim(head_dim), as_dim(block_size),
                                as_dim(num_blocks), as_dim(table_stride), as_dim(batch_size), as_dim(max_context)));
}

void Gpu::attention_qkv_rope(const Buffer& qkv, const Buffer& qweight, const Buffer& kweight,
                             const Buffer& positions, const Buffer& slots, const Buffer& kcache,
                             const Buffer& vcache, const Buffer& seq_indices, const Buffer& block_tables,
                             const Buffer& out, std::size_t rows, std::size_t qheads, std::size_t kvheads,
                             std::size_t head_dim, std::size_t block_size, std::size_t num_blocks,
                             std::size_t table_stride, std::size_t batch_size, std::size_t max_context, float eps,
                             const Buffer& rope_cache, std::size_t max_positions) const {
    require_positive(eps, "attention_qkv_rope eps");
    require_head_layout(qheads, kvheads, head_dim);
    if (head_dim != 128) throw Error(Fault::Value, "attention_qkv_rope takes head_dim 128 only");
    require_context_limit(max_context);
    const RopeShape s{rows, qheads, kvheads, head_dim, block_size, num_blocks};
    admit("attention_qkv_rope",
          {read_arg("qkv", qkv, 2, {rows, s.heads(), head_dim}), read_arg("qweight", qweight, 2, {head_dim}),
           read_arg("kweight", kweight, 2, {head_dim}), read_arg("positions", positions, 4, {rows}),
           read_arg("slots", slots, 4, {rows}), read_arg("seq_indices", seq_indices, 4, {rows}),
           read_arg("block_tables", block_tables, 4, {batch_size, table_stride}),
           read_arg("rope_cache", rope_cache, 4, {max_positions, head_dim}),
           write_arg("kcache", kcache, 2, {num_blocks, block_size, kvheads, head_dim}),
           write_arg("vcache", vcache, 2, {num_blocks, block_size, kvheads, head_dim}),
           write_arg("out", out, 2, {rows, qheads, head_dim})});
    require_status(nv_attention_qkv_rope(context(), qkv.address(), qweight.address(), kweight.address(),
                                         positions.address(), slots.address(), kcache.address(), vcache.address(),
                                         seq_indices.address(), block_tables.address(), out.address(), as_dim(rows),
                                         as_dim(qheads), as_dim(kvheads), as_dim(head_dim), as_dim(block_size),
                                         as_dim(num_blocks), as_dim(table_stride), as_dim(batch_size),
                                         as_dim(max_context), eps, rope_cache.address(), as_dim(max_positions)));
}

void Gpu::silu_mul(const Buffer& gateup, const Buffer& out, std::size_t rows, std::size_t intermediate) const {
    if (intermediate > std::size_t(INT_MAX) / 2)
        throw Error(Fault::Dimension, "silu_mul: 2 * intermediate exceeds 2^31 - 1");
    admit("silu_mul", {read_arg("gateup", gateup, 2, {rows, 2, intermediate}),
                       write_arg("out", out, 2, {rows, intermediate})});
    require_status(nv_silu(context(), gateup.address(), out.address(), as_dim(rows), as_dim(intermediate)));
}

void Gpu::gather(const Buffer& x, const Buffer& indices, const Buffer& out, std::size_t rows, std::size_t hidden,
                 std::size_t input_rows) const {
    admit("gather", {read_arg("x", x, 2, {input_rows, hidden}), read_arg("indices", indices, 4, {rows}),
                     write_arg("out", out, 2, {rows, hidden})});
    require_status(nv_gather(context(), x.address(), indices.address(), out.address(), as_dim(rows), as_dim(hidden),
                             as_dim(input_rows)));
}

void Gpu::sample(const Buffer& logits, const Buffer& temperatures, const Buffer& seeds, const Buffer& out,
                 std::size_t batch, std::size_t vocab) const {
    admit("sample", {read_arg("logits", logits, 2, {batch, vocab}), read_arg("temperatures", temperatures, 4, {batch}),
                     read_arg("seeds", seeds, 8, {batch}), write_arg("out", out, 4, {batch})});
    require_status(nv_sample(context(), logits.address(), temperatures.address(), seeds.address(), out.address(),
                             as_dim(batch), as_dim(vocab)));
}

void Gpu::sample_parallel(const Buffer& logits, const Buffer& temperatures, const Buffer& seeds, const Buffer& out,
                          const Buffer& partial_scores, const Buffer& partial_ids, std::size_t batch,
                          std::size_t vocab) const {
    const std::size_t parts = (vocab + 2047) / 2048;
    admit("sample_parallel",
          {read_arg("logits", logits, 2, {batch, vocab}), read_arg("temperatures", temperatures, 4, {batch}),
           read_arg("seeds", seeds, 8, {batch}), write_arg("out", out, 4, {batch}),
           write_arg("partial_scores", partial_scores, 4, {batch, parts}),
           write_arg("partial_ids", partial_ids, 4, {batch, parts})});
    require_status(nv_sample_parallel(context(), logits.address(), temperatures.address(), seeds.address(),
                                      out.address(), partial_scores.address(), partial_ids.address(), as_dim(batch),
                                      as_dim(vocab)));
}

void Gpu::sample_parallel_static(const Buffer& logits, const Buffer& temperatures, const Buffer& seeds,
                                 const Buffer& out, std::size_t batch, std::size_t vocab) const {
    admit("sample_parallel_static",
          {read_arg("logits", logits, 2, {batch, vocab}), read_arg("temperatures", temperatures, 4, {batch}),
           read_arg("seeds", seeds, 8, {batch}), write_arg("out", out, 4, {batch})});
    require_status(nv_sample_parallel_static(context(), logits.address(), temperatures.address(), seeds.address(),
                                             out.address(), as_dim(batch), as_dim(vocab)));
}

void Gpu::kv_write(const Buffer& k, const Buffer& v, const Buffer& slots, const Buffer& kcache, const Buffer& vcache,
                   std::size_t rows, std::size_t kvheads, std::size_t head_dim, std::size_t block_size,
                   std::size_t num_blocks) const {
    as_dim(kvheads);
    as_dim(head_dim);
    if (kvheads > std::size_t(INT_MAX) / head_dim)
        throw Error(Fault::Dimension, "kv_write: kvheads * head_dim exceeds 2^31 - 1");
    admit("kv_write", {read_arg("k", k, 2, {rows, kvheads, head_dim}), read_arg("v", v, 2, {rows, kvheads, head_dim}),
                       read_arg("slots", slots, 4, {rows}),
                       write_arg("kcache", kcache, 2, {num_blocks, block_size, kvheads, head_dim}),
                       write_arg("vcache", vcache, 2, {num_blocks, block_size, kvheads, head_dim})});
    require_status(nv_kv_write(context(), k.address(), v.address(), slots.address(), kcache.address(),
                               vcache.address(), as_dim(rows), as_dim(kvheads), as_dim(head_dim), as_dim(block_size),
                               as_dim(num_blocks)));
}

}  // namespace nvr
