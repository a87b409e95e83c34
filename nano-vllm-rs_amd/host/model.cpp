// Qwen3 forward runner (see model.hpp); restates src/model.rs of nano-vllm-rs.
#include "model.hpp"

#include <climits>
#include <cmath>
#include <cstring>
#include <set>
#include <sstream>

namespace nvr {

namespace {

template <class... Args>
std::string format(const Args&... args) {
    std::ostringstream s;
    (s << ... << args);
    return s.str();
}

void ensure(bool ok, const char* message) {
    if (!ok) throw Error(message);
}

// src/model.rs:1000-1004.
std::size_t byte_size(std::initializer_list<std::size_t> dims, std::size_t width) {
    std::size_t n = width;
    for (std::size_t d : dims) {
        if (d != 0 && n > SIZE_MAX / d) throw Error("tensor byte size overflow");
        n *= d;
    }
    return n;
}

std::size_t add(std::size_t a, std::size_t b, const char* what) {
    if (a > SIZE_MAX - b) throw Error(what);
    return a + b;
}

}  // namespace

// ------------------------------------------------------------- config ------
void ModelConfig::validate() const {
    ensure(num_hidden_layers > 0 && hidden_size > 0 && intermediate_size > 0 && vocab_size > 0,
           "model dimensions must be positive");
    ensure(num_attention_heads > 0 && num_key_value_heads > 0 && num_attention_heads % num_key_value_heads == 0,
           "query heads must be a positive multiple of KV heads");
    ensure(head_dim > 0 && head_dim <= 256 && head_dim % 2 == 0, "head_dim must be even and at most 256");
    ensure(std::isfinite(rms_norm_eps) && rms_norm_eps > 0.0f && std::isfinite(rope_theta) && rope_theta > 0.0f,
           "RMS epsilon and RoPE theta must be positive finite values");
    ensure(max_position_embeddings > 0 && vocab_size <= std::size_t(INT_MAX), "invalid model context or vocabulary size");
    for (std::size_t n : {hidden_size, intermediate_size, num_hidden_layers, num_attention_heads, num_key_value_heads,
                          max_position_embeddings})
        ensure(n <= std::size_t(INT_MAX), "model dimensions exceed 32-bit indexing");
    byte_size({num_attention_heads, head_dim}, 2);
}

// --------------------------------------------------------- metadata --------
MetadataLayout MetadataLayout::make(std::size_t tokens, std::size_t sequences, std::size_t table_stride) {
    MetadataLayout m;
    std::size_t cursor = 0;
    auto segment = [&](std::size_t count, std::size_t width) {
        Range r;
        r.start = add(cursor, 7, "metadata alignment overflow") & ~std::size_t(7);
        r.end = add(r.start, byte_size({count}, width), "metadata extent overflow");
        cursor = r.end;
        return r;
    };
    if (table_stride != 0 && sequences > SIZE_MAX / table_stride) throw Error("block table size overflow");
    m.tokens = segment(tokens, 4);
    m.positions = segment(tokens, 4);
    m.sequences = segment(tokens, 4);
    m.slots = segment(tokens, 4);
    m.tables = segment(sequences * table_stride, 4);
    m.last_indices = segment(sequences, 4);
    m.temperatures = segment(sequences, 4);
    m.seeds = segment(sequences, 8);
    m.bytes = cursor;
    return m;
}

void MetadataLayout::pack(std::vector<uint8_t>& staging, const Batch& batch, std::size_t sequences,
                          std::size_t table_stride) const {
    auto put = [&](const Range& r, std::size_t offset, const void* data, std::size_t bytes) {
        std::memcpy(staging.data() + r.start + offset, data, bytes);
    };
    put(tokens, 0, batch.token_ids.data(), batch.token_ids.size() * 4);
    put(positions, 0, batch.positions.data(), batch.positions.size() * 4);
    put(this->sequences, 0, batch.sequence_ids.data(), batch.sequence_ids.size() * 4);
    put(slots, 0, batch.slot_mapping.data(), batch.slot_mapping.size() * 4);
    std::memset(staging.data() + tables.start, 0xff, sequences * table_stride * 4);
    for (std::size_t s = 0; s < sequences; ++s)
        put(tables, s * table_stride * 4, batch.block_tables.data() + s * batch.table_stride, batch.table_stride * 4);
    put(last_indices, 0, batch.last_token_indices.data(), batch.last_token_indices.size() * 4);
    put(temperatures, 0, batch.temperatures.data(), batch.temperatures.size() * 4);
    put(seeds, 0, batch.seeds.data(), batch.seeds.size() * 8);
}

// ------------------------------------------------------------- model -------
QwenModel::QwenModel(const ModelConfig& config, const ModelOptions& options, const WeightSource& weights)
    : config_(config), options_(options), gpu_(options.device) {
    config_.validate();
    const ModelOptions& o = options_;
    ensure(o.block_size > 0 && o.num_blocks > 0 && o.max_batch_tokens > 0 && o.max_sequences > 0 &&
               o.max_model_len > 0,
           "all model capacities must be positive");
    ensure(o.max_model_len <= config_.max_position_embeddings,
           "max_model_len exceeds checkpoint max_position_embeddings");
    ensure(o.max_model_len <= 4096, "this attention implementation supports max_model_len up to 4096");
    ensure(o.max_sequences <= o.max_batch_tokens, "max_sequences must not exceed max_batch_tokens");
    if (o.num_blocks > SIZE_MAX / o.block_size) throw Error("KV slot count overflow");
    const std::size_t cache_slots = o.num_blocks * o.block_size;
    ensure(cache_slots <= std::size_t(INT_MAX) && o.max_batch_tokens <= std::size_t(INT_MAX),
           "configured capacity exceeds 32-bit indexing");
    table_stride_ = (o.max_model_len + o.block_size - 1) / o.block_size;

    const ModelConfig& c = config_;
    auto load = [&](const std::string& name, const std::vector<std::vector<std::size_t>>& parts,
                    const std::vector<std::string>& names) {
        std::vector<uint16_t> all;
        for (std::size_t i = 0; i < parts.size(); ++i) {
            std::size_t n = 1;
            for (std::size_t d : parts[i]) n = byte_size({d}, n);
            std::vector<uint16_t> bits = weights(names[i], parts[i]);
            if (bits.size() != n)
                throw Error(format("weight ", names[i], " has ", bits.size(), " elements; expected ", n));
            all.insert(all.end(), bits.begin(), bits.end());
        }
        if (all.empty()) throw Error(format("weight ", name, " is empty"));
        Buffer b = gpu_.alloc(all.size() * 2);
        b.upload_u16(all);
        memory_.weights_bytes += all.size() * 2;
        return b;
    };
    auto one = [&](const std::string& name, std::vector<std::size_t> shape) { return load(name, {shape}, {name}); };

    embedding_ = one("model.embed_tokens.weight", {c.vocab_size, c.hidden_size});
    final_norm_ = one("model.norm.weight", {c.hidden_size});
    lm_head_ = c.tie_word_embeddings ? embedding_ : one("lm_head.weight", {c.vocab_size, c.hidden_size});
    const std::size_t q_size = c.num_attention_heads * c.head_dim, kv_size = c.num_key_value_heads * c.head_dim;
    const std::size_t cache_bytes = byte_size({cache_slots, kv_size}, 2);
    for (std::size_t i = 0; i < c.num_hidden_layers; ++i) {
        const std::string p = format("model.layers.", i, ".");
        Layer l;
        l.input_norm = one(p + "input_layernorm.weight", {c.hidden_size});
        l.qkv = load(p + "self_attn.qkv", {{q_size, c.hidden_size}, {kv_size, c.hidden_size}, {kv_size, c.hidden_size}},
                     {p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight", p + "self_attn.v_proj.weight"});
        l.q_norm = one(p + "self_attn.q_norm.weight", {c.head_dim});
        l.k_norm = one(p + "self_attn.k_norm.weight", {c.head_dim});
        l.attention_out = one(p + "self_attn.o_proj.weight", {c.hidden_size, q_size});
        l.post_norm = one(p + "post_attention_layernorm.weight", {c.hidden_size});
        l.gate_up = load(p + "mlp.gate_up", {{c.intermediate_size, c.hidden_size}, {c.intermediate_size, c.hidden_size}},
                         {p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight"});
        l.down = one(p + "mlp.down_proj.weight", {c.hidden_size, c.intermediate_size});
        l.k_cache = gpu_.alloc(cache_bytes);
        l.v_cache = gpu_.alloc(cache_bytes);
        layers_.push_back(std::move(l));
    }

    auto alloc = [&](std::initializer_list<std::size_t> dims, std::size_t width) {
        const std::size_t bytes = byte_size(dims, width);
        memory_.workspace_bytes += bytes;
        return gpu_.alloc(bytes);
    };
    const std::size_t t = o.max_batch_tokens, s = o.max_sequences, h = c.hidden_size;
    layout_ = MetadataLayout::make(t, s, table_stride_);
    Workspace& w = work_;
    w.metadata = alloc({layout_.bytes}, 1);
    auto view = [&](const MetadataLayout::Range& r) { return w.metadata.slice(r.start, r.size()); };
    w.tokens = view(layout_.tokens);
    w.positions = view(layout_.positions);
    w.seq_indices = view(layout_.sequences);
    w.slots = view(layout_.slots);
    w.block_tables = view(layout_.tables);
    w.last_indices = view(layout_.last_indices);
    w.temperatures = view(layout_.temperatures);
    w.seeds = view(layout_.seeds);
    const std::size_t parts = (c.vocab_size + 2047) / 2048;
    w.samples = alloc({s}, 4);
    w.sample_scores = alloc({s, parts}, 4);
    w.sample_ids = alloc({s, parts}, 4);
    w.rope_cache = alloc({o.max_model_len, c.head_dim}, 4);
    w.residual = alloc({t, h}, 2);
    w.hidden = alloc({t, h}, 2);
    w.normed = alloc({t, h}, 2);
    w.qkv = alloc({t, q_size + 2 * kv_size}, 2);
    w.query = alloc({t, q_size}, 2);
    w.attention = alloc({t, q_size}, 2);
    w.gate_up = alloc({t, 2 * c.intermediate_size}, 2);
    w.activated = alloc({t, c.intermediate_size}, 2);
    w.gathered = alloc({s, h}, 2);
    w.logits = alloc({s, c.vocab_size}, 2);
    host_metadata_.assign(layout_.bytes, 0);
    gpu_.rope_cache(w.rope_cache, o.max_model_len, c.head_dim, c.rope_theta);
    gpu_.sync();
    memory_.kv_cache_bytes = byte_size({cache_bytes, 2, c.num_hidden_layers}, 1);
}

// src/model.rs:635-818, without the FlashAttention branch.
void QwenModel::forward(std::size_t rows, std::size_t sequences, std::size_t samples, bool fused) const {
    const ModelConfig& c = config_;
    const ModelOptions& o = options_;
    const Workspace& w = work_;
    const Gpu& g = gpu_;
    const std::size_t q_size = c.num_attention_heads * c.head_dim;
    const std::size_t qkv_size = q_size + 2 * c.num_key_value_heads * c.head_dim;
    g.embedding(w.tokens, embedding_, w.residual, rows, c.hidden_size, c.vocab_size);
    for (std::size_t i = 0; i < layers_.size(); ++i) {
        const Layer& l = layers_[i];
        if (i == 0)
            g.rms_norm(w.residual, l.input_norm, w.normed, rows, c.hidden_size, c.rms_norm_eps);
        else
            g.add_rms_norm(w.hidden, w.residual, l.input_norm, w.normed, rows, c.hidden_size, c.rms_norm_eps);
        g.gemm(w.normed, l.qkv, w.qkv, rows, qkv_size, c.hidden_size);
        if (fused) {
            g.attention_qkv_rope(w.qkv, l.q_norm, l.k_norm, w.positions, w.slots, l.k_cache, l.v_cache,
                                 w.seq_indices, w.block_tables, w.attention, rows, c.num_attention_heads,
                                 c.num_key_value_heads, c.head_dim, o.block_size, o.num_blocks, table_stride_,
                                 sequences, o.max_model_len, c.rms_norm_eps, w.rope_cache, o.max_model_len);
        } else {
            g.qkv_rope_cached(w.qkv, l.q_norm, l.k_norm, w.positions, w.slots, w.query, l.k_cache, l.v_cache, rows,
                              c.num_attention_heads, c.num_key_value_heads, c.head_dim, o.block_size, o.num_blocks,
                              c.rms_norm_eps, w.rope_cache, o.max_model_len);
            g.paged_attention(w.query, l.k_cache, l.v_cache, w.positions, w.seq_indices, w.block_tables, w.attention,
                              rows, c.num_attention_heads, c.num_key_value_heads, c.head_dim, o.block_size,
                              o.num_blocks, table_stride_, sequences, o.max_model_len);
        }
        g.gemm(w.attention, l.attention_out, w.hidden, rows, c.hidden_size, q_size);
        g.add_rms_norm(w.hidden, w.residual, l.post_norm, w.normed, rows, c.hidden_size, c.rms_norm_eps);
        g.gemm(w.normed, l.gate_up, w.gate_up, rows, 2 * c.intermediate_size, c.hidden_size);
        g.silu_mul(w.gate_up, w.activated, rows, c.intermediate_size);
        g.gemm(w.activated, l.down, w.hidden, rows, c.hidden_size, c.intermediate_size);
    }
    if (samples > 0) {
        g.add_rms_norm(w.hidden, w.residual, final_norm_, w.normed, rows, c.hidden_size, c.rms_norm_eps);
        g.gather(w.normed, w.last_indices, w.gathered, samples, c.hidden_size, rows);
        g.gemm(w.gathered, lm_head_, w.logits, samples, c.vocab_size, c.hidden_size);
        g.sample_parallel(w.logits, w.temperatures, w.seeds, w.samples, w.sample_scores, w.sample_ids, samples,
                          c.vocab_size);
    }
}

// src/model.rs:820-923.
std::array<std::size_t, 4> QwenModel::validate_batch(const Batch& b) const {
    const ModelOptions& o = options_;
    const std::size_t rows = b.token_ids.size(), samples = b.last_token_indices.size();
    ensure(rows > 0 && rows <= o.max_batch_tokens, "batch token count is outside model capacity");
    ensure(b.positions.size() == rows && b.sequence_ids.size() == rows && b.slot_mapping.size() == rows,
           "token metadata lengths differ");
    ensure(b.table_stride > 0 && b.table_stride <= table_stride_ && b.block_tables.size() % b.table_stride == 0,
           "invalid block table shape");
    const std::size_t sequences = b.block_tables.size() / b.table_stride;
    ensure(sequences > 0 && sequences <= o.max_sequences, "batch sequence count exceeds capacity");
    ensure(samples <= sequences && samples == b.temperatures.size() && samples == b.seeds.size(),
           "invalid sampling metadata lengths");
    for (int32_t token : b.token_ids)
        ensure(token >= 0 && std::size_t(token) < config_.vocab_size, "token id outside model vocabulary");
    for (int32_t index : b.last_token_indices)
        ensure(index >= 0 && std::size_t(index) < rows, "sample row outside batch");
    for (float t : b.temperatures) ensure(std::isfinite(t) && t >= 0.0f, "temperature must be finite and nonnegative");
    std::set<std::size_t> seen;
    std::vector<long long> max_position(sequences, -1);
    for (std::size_t r = 0; r < rows; ++r) {
        const int32_t position = b.positions[r], sequence = b.sequence_ids[r];
        ensure(position >= 0 && std::size_t(position) < o.max_model_len, "token position exceeds max_model_len");
        ensure(sequence >= 0 && std::size_t(sequence) < sequences, "token sequence index outside block tables");
        const std::size_t column = std::size_t(position) / o.block_size;
        ensure(column < b.table_stride, "block table does not cover token position");
        const int32_t block = b.block_tables[std::size_t(sequence) * b.table_stride + column];
        ensure(block >= 0 && std::size_t(block) < o.num_blocks, "invalid physical KV block");
        const std::size_t expected = std::size_t(block) * o.block_size + std::size_t(position) % o.block_size;
        ensure(b.slot_mapping[r] >= 0 && std::size_t(b.slot_mapping[r]) == expected,
               "KV slot mapping disagrees with block table");
        ensure(seen.insert(expected).second, "two input tokens write the same KV slot");
        max_position[sequence] = std::max<long long>(max_position[sequence], position);
    }
    for (std::size_t s = 0; s < sequences; ++s) {
        if (max_position[s] < 0) continue;
        for (std::size_t column = 0; column <= std::size_t(max_position[s]) / o.block_size; ++column) {
            const int32_t block = b.block_tables[s * b.table_stride + column];
            ensure(block >= 0 && std::size_t(block) < o.num_blocks, "missing KV block in causal context");
        }
    }
    bool fused = config_.head_dim == 128 && rows == sequences;
    std::map<int32_t, std::size_t> writer;  // block -> the row writing into it
    for (std::size_t r = 0; fused && r < rows; ++r) {
        fused = max_position[std::size_t(b.sequence_ids[r])] == b.positions[r];  // its sequence's only row
        writer.emplace(int32_t(std::size_t(b.slot_mapping[r]) / o.block_size), r);
    }
    for (std::size_t r = 0; fused && r < rows; ++r) {
        const int32_t* table = &b.block_tables[std::size_t(b.sequence_ids[r]) * b.table_stride];
        for (std::size_t column = 0; fused && column <= std::size_t(b.positions[r]) / o.block_size; ++column) {
            const auto it = writer.find(table[column]);
            fused = it == writer.end() || it->second == r;
        }
    }
    return {rows, sequences, samples, fused ? 1u : 0u};
}

// src/model.rs:925-987, without the FlashAttention metadata.
std::vector<uint32_t> QwenModel::run(const Batch& batch) {
    const auto [rows, sequences, samples, fused] = validate_batch(batch);
    last_sample_count_ = 0;
    layout_.pack(host_metadata_, batch, sequences, table_stride_);
    // Upload synchronises before returning, so both eager launches and graph
    // replays see complete input and the staging vector may be reused.
    work_.metadata.upload_bytes(host_metadata_);
    if (options_.graphs && batch.is_decode && rows == sequences && samples == sequences) {
        auto it = graphs_.find(2 * rows + fused);
        if (it == graphs_.end()) {
            // hipBLAS may initialise state on first use of a shape: warm up
            // before capture; the replay then rewrites the same KV slots.
            forward(rows, sequences, samples, fused);
            gpu_.sync();
            Graph graph = gpu_.capture([&] { forward(rows, sequences, samples, fused); });
            it = graphs_.emplace(2 * rows + fused, std::move(graph)).first;
        }
        it->second.replay();
    } else {
        forward(rows, sequences, samples, fused);
    }
    last_sample_count_ = samples;
    if (samples == 0) {
        gpu_.sync();
        return {};
    }
    std::vector<uint32_t> out;
    for (int32_t id : work_.samples.download_i32(samples)) {
        ensure(id >= 0 && std::size_t(id) < config_.vocab_size, "GPU sampler returned an invalid token id");
        out.push_back(uint32_t(id));
    }
    return out;
}

std::vector<std::vector<float>> QwenModel::last_logits() const {
    const std::size_t v = config_.vocab_size;
    const std::vector<uint16_t> bits = work_.logits.download_u16(last_sample_count_ * v);
    std::vector<std::vector<float>> rows(last_sample_count_, std::vector<float>(v));
    for (std::size_t r = 0; r < last_sample_count_; ++r)
        for (std::size_t i = 0; i < v; ++i) {
            const uint32_t u = uint32_t(bits[r * v + i]) << 16;
            std::memcpy(&rows[r][i], &u, 4);
        }
    return rows;
}

}  // namespace nvr
