// Qwen3 forward runner (contract in model.hpp). The layer order and the math
// are Qwen3's, as nano-vllm-rs runs it (src/model.rs:635-818); batch checks,
// step records, graph keys and the observer are this library's own.
#include "model.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>
#include <unordered_map>
#include <unordered_set>

namespace nvr {

namespace {

// Rows up to which the norms run inside the qkv / gate_up GEMMs (nv_rms_gemm):
// measured on MI355X at hidden 1024, 8 rows save ~2.5 us per norm + GEMM
// pair, 16 rows ~0.5 us, 32 rows lose ~3 us (each block normalises every row).
constexpr std::size_t kFusedNormRows = 16;

std::string str(std::size_t v) { return std::to_string(v); }

// Whether the model's shapes suit nv_rms_gemm / nv_rms_gemm_silu and the
// options ask for them.
bool norm_gemm_fits(const ModelConfig& c, const ModelOptions& o) {
    const std::size_t h = c.hidden_size;
    const std::size_t qkv_cols = (c.num_attention_heads + 2 * c.num_key_value_heads) * c.head_dim;
    return o.fuse_norm_gemm && (h == 512 || h == 1024 || h == 2048) && qkv_cols % 16 == 0 &&
           c.intermediate_size % 8 == 0;
}

[[noreturn]] void reject(Reject reason, const std::string& detail) {
    throw BatchError(reason, std::string("batch rejected (") + reject_name(reason) + "): " + detail);
}

std::size_t round_up(std::size_t v, std::size_t to) {
    if (v > SIZE_MAX - (to - 1)) throw Error(Fault::Extent, "step record size overflows size_t");
    return (v + to - 1) / to * to;
}

}  // namespace

const char* reject_name(Reject reason) {
    switch (reason) {
    case Reject::Rows: return "row count";
    case Reject::Lengths: return "per-row lengths";
    case Reject::TableShape: return "table shape";
    case Reject::Sequences: return "sequence count";
    case Reject::Sampling: return "sampling lengths";
    case Reject::Token: return "token id";
    case Reject::SampleRow: return "sampled row";
    case Reject::Temperature: return "temperature";
    case Reject::Position: return "position";
    case Reject::Sequence: return "sequence id";
    case Reject::TableColumn: return "table column";
    case Reject::Block: return "block";
    case Reject::Slot: return "slot";
    case Reject::SlotReuse: return "slot reuse";
    case Reject::Context: return "context block";
    }
    return "?";
}

// ------------------------------------------------------------- config ------
void ModelConfig::validate() const {
    auto fail = [](const std::string& what) { throw Error(Fault::Value, "model config: " + what); };
    for (std::size_t v : {hidden_size, intermediate_size, num_hidden_layers, num_attention_heads,
                          num_key_value_heads, head_dim, vocab_size, max_position_embeddings})
        if (v == 0 || v > std::size_t(INT_MAX)) fail("a dimension is 0 or above 2^31 - 1");
    require_head_layout(num_attention_heads, num_key_value_heads, head_dim);
    if (!(rms_norm_eps > 0.0f) || !std::isfinite(rms_norm_eps)) fail("rms_norm_eps is not a positive finite number");
    if (!(rope_theta > 0.0f) || !std::isfinite(rope_theta)) fail("rope_theta is not a positive finite number");
    byte_count({num_attention_heads + 2 * num_key_value_heads, head_dim, hidden_size}, 2);
}

// --------------------------------------------------------- step record -----
StepRecord StepRecord::for_capacity(std::size_t rows, std::size_t sequences, std::size_t table_stride) {
    StepRecord r;
    std::size_t at = 0;
    auto place = [&](Field& f, std::size_t count, std::size_t width) {
        f.offset = at;
        f.bytes = byte_count({std::max<std::size_t>(count, 1)}, width);
        at = round_up(f.offset + f.bytes, 256);
    };
    place(r.seeds, sequences, 8);
    place(r.tokens, rows, 4);
    place(r.positions, rows, 4);
    place(r.sequence_ids, rows, 4);
    place(r.slots, rows, 4);
    place(r.last_rows, sequences, 4);
    if (table_stride != 0 && sequences > SIZE_MAX / table_stride)
        throw Error(Fault::Extent, "block table entries overflow size_t");
    place(r.tables, sequences * table_stride, 4);
    place(r.temperatures, sequences, 4);
    r.size = at;
    return r;
}

void StepRecord::fill(std::vector<uint8_t>& host, const Batch& b, std::size_t sequences,
                      std::size_t table_stride) const {
    auto copy = [&](const Field& f, const void* data, std::size_t bytes) {
        if (bytes > f.bytes) throw Error(Fault::Extent, "step record field overflow");
        if (bytes != 0) std::memcpy(host.data() + f.offset, data, bytes);
    };
    copy(seeds, b.seeds.data(), b.seeds.size() * 8);
    copy(tokens, b.token_ids.data(), b.token_ids.size() * 4);
    copy(positions, b.positions.data(), b.positions.size() * 4);
    copy(sequence_ids, b.sequence_ids.data(), b.sequence_ids.size() * 4);
    copy(slots, b.slot_mapping.data(), b.slot_mapping.size() * 4);
    copy(last_rows, b.last_token_indices.data(), b.last_token_indices.size() * 4);
    copy(temperatures, b.temperatures.data(), b.temperatures.size() * 4);
    // Tables: each sequence's row widened to the model's stride with -1 (the
    // attention kernels treat a negative entry as no block).
    int32_t* table = reinterpret_cast<int32_t*>(host.data() + tables.offset);
    std::fill(table, table + tables.bytes / 4, -1);
    for (std::size_t s = 0; s < sequences; ++s)
        std::copy_n(b.block_tables.begin() + std::ptrdiff_t(s * b.table_stride), b.table_stride, table + s * table_stride);
}

// ------------------------------------------------------------------ model --
QwenModel::QwenModel(const ModelConfig& config, const ModelOptions& options, const WeightSource& weights)
    : config_(config), options_(options), gpu_(options.device) {
    config_.validate();
    const ModelOptions& o = options_;
    auto fail = [](const std::string& what) { throw Error(Fault::Value, "model options: " + what); };
    for (std::size_t v : {o.block_size, o.num_blocks, o.max_batch_tokens, o.max_sequences, o.max_model_len})
        if (v == 0) fail("every capacity must be at least 1");
    if (o.max_model_len > config_.max_position_embeddings) fail("max_model_len exceeds max_position_embeddings");
    if (o.max_model_len > 4096) fail("the attention kernels hold at most 4096 context tokens");
    if (o.max_sequences > o.max_batch_tokens) fail("max_sequences exceeds max_batch_tokens");
    if (o.num_blocks > std::size_t(INT_MAX) / o.block_size || o.max_batch_tokens > std::size_t(INT_MAX))
        fail("KV slots or batch rows exceed 2^31 - 1");
    table_stride_ = (o.max_model_len + o.block_size - 1) / o.block_size;

    const ModelConfig& c = config_;
    // Uploads the concatenation of the named tensors (fused projections
    // keep the reference's row order: q, k, v and gate, up).
    auto read = [&](const std::vector<std::pair<std::string, std::vector<std::size_t>>>& parts) {
        std::vector<uint16_t> bits;
        for (const auto& [name, shape] : parts) {
            std::size_t n = 1;
            for (std::size_t d : shape) n *= d;
            std::vector<uint16_t> t = weights(name, shape);
            if (t.size() != n)
                throw Error(Fault::Extent, "weight " + name + ": " + str(t.size()) + " elements, shape holds " + str(n));
            bits.insert(bits.end(), t.begin(), t.end());
        }
        return bits;
    };
    auto put = [&](const std::vector<uint16_t>& bits) {
        Buffer b = gpu_.alloc(bits.size() * 2);
        b.upload_u16(bits);
        memory_.weights_bytes += bits.size() * 2;
        return b;
    };
    auto upload = [&](const std::vector<std::pair<std::string, std::vector<std::size_t>>>& parts) {
        return put(read(parts));
    };
    const std::size_t h = c.hidden_size, q = c.num_attention_heads * c.head_dim, kv = c.num_key_value_heads * c.head_dim;
    embedding_ = upload({{"model.embed_tokens.weight", {c.vocab_size, h}}});
    final_norm_ = upload({{"model.norm.weight", {h}}});
    lm_head_ = c.tie_word_embeddings ? embedding_ : upload({{"lm_head.weight", {c.vocab_size, h}}});
    const std::size_t slots = o.num_blocks * o.block_size;
    const std::size_t cache_bytes = byte_count({slots, kv}, 2);
    for (std::size_t i = 0; i < c.num_hidden_layers; ++i) {
        const std::string p = "model.layers." + str(i) + ".";
        LayerWeights l;
        l.input_norm = upload({{p + "input_layernorm.weight", {h}}});
        l.qkv = upload({{p + "self_attn.q_proj.weight", {q, h}},
                        {p + "self_attn.k_proj.weight", {kv, h}},
                        {p + "self_attn.v_proj.weight", {kv, h}}});
        l.q_norm = upload({{p + "self_attn.q_norm.weight", {c.head_dim}}});
        l.k_norm = upload({{p + "self_attn.k_norm.weight", {c.head_dim}}});
        l.o_proj = upload({{p + "self_attn.o_proj.weight", {h, q}}});
        l.post_norm = upload({{p + "post_attention_layernorm.weight", {h}}});
        const std::vector<uint16_t> gate_up = read({{p + "mlp.gate_proj.weight", {c.intermediate_size, h}},
                                                    {p + "mlp.up_proj.weight", {c.intermediate_size, h}}});
        l.gate_up = put(gate_up);
        // The same weight in the tile row order of the fused gate_up + SiLU
        // kernel (decode-sized steps).
        if (norm_gemm_fits(c, o)) l.gate_up_tiled = put(tile_gate_up_rows(gate_up, c.intermediate_size, h));
        l.down = upload({{p + "mlp.down_proj.weight", {h, c.intermediate_size}}});
        l.k_cache = gpu_.alloc(cache_bytes);
        l.v_cache = gpu_.alloc(cache_bytes);
        memory_.kv_cache_bytes += 2 * cache_bytes;
        layers_.push_back(std::move(l));
    }

    const std::size_t t = o.max_batch_tokens, s = o.max_sequences;
    auto scratch = [&](std::initializer_list<std::size_t> dims, std::size_t width) {
        const std::size_t bytes = byte_count(dims, width);
        memory_.workspace_bytes += bytes;
        return gpu_.alloc(bytes);
    };
    record_ = StepRecord::for_capacity(t, s, table_stride_);
    Workspace& w = work_;
    w.record = scratch({record_.size}, 1);
    auto field = [&](const StepRecord::Field& f) { return w.record.slice(f.offset, f.bytes); };
    w.seeds = field(record_.seeds);
    w.tokens = field(record_.tokens);
    w.positions = field(record_.positions);
    w.sequence_ids = field(record_.sequence_ids);
    w.slots = field(record_.slots);
    w.last_rows = field(record_.last_rows);
    w.tables = field(record_.tables);
    w.temperatures = field(record_.temperatures);
    const std::size_t partials = (c.vocab_size + 2047) / 2048;
    w.samples = scratch({s}, 4);
    w.partial_scores = scratch({s, partials}, 4);
    w.partial_ids = scratch({s, partials}, 4);
    w.rope_cache = scratch({o.max_model_len, c.head_dim}, 4);
    w.residual = scratch({t, h}, 2);
    w.residual_alt = scratch({t, h}, 2);
    residual_ = &w.residual;
    w.hidden = scratch({t, h}, 2);
    w.normed = scratch({t, h}, 2);
    w.qkv = scratch({t, q + 2 * kv}, 2);
    w.query = scratch({t, q}, 2);
    w.attention = scratch({t, q}, 2);
    w.gate_up = scratch({t, 2 * c.intermediate_size}, 2);
    w.activated = scratch({t, c.intermediate_size}, 2);
    w.gathered = scratch({s, h}, 2);
    w.logits = scratch({s, c.vocab_size}, 2);
    host_record_.assign(record_.size, 0);
    gpu_.rope_cache(w.rope_cache, o.max_model_len, c.head_dim, c.rope_theta);
    gpu_.sync();
}

StepPlan QwenModel::plan(const Batch& b) const {
    const ModelOptions& o = options_;
    StepPlan p;
    // Shapes.
    p.rows = b.token_ids.size();
    if (p.rows == 0 || p.rows > o.max_batch_tokens)
        reject(Reject::Rows, str(p.rows) + " rows for a capacity of " + str(o.max_batch_tokens));
    if (b.positions.size() != p.rows || b.sequence_ids.size() != p.rows || b.slot_mapping.size() != p.rows)
        reject(Reject::Lengths, "positions, sequence ids and slots must each hold " + str(p.rows) + " entries");
    if (b.table_stride == 0 || b.table_stride > table_stride_ || b.block_tables.size() % b.table_stride != 0)
        reject(Reject::TableShape, str(b.block_tables.size()) + " entries in rows of " + str(b.table_stride) +
                                       " (model stride " + str(table_stride_) + ")");
    p.sequences = b.block_tables.size() / b.table_stride;
    if (p.sequences == 0 || p.sequences > o.max_sequences)
        reject(Reject::Sequences, str(p.sequences) + " table rows for a capacity of " + str(o.max_sequences));
    p.samples = b.last_token_indices.size();
    if (p.samples > p.sequences || b.temperatures.size() != p.samples || b.seeds.size() != p.samples)
        reject(Reject::Sampling, str(p.samples) + " sampled rows, " + str(b.temperatures.size()) + " temperatures, " +
                                     str(b.seeds.size()) + " seeds, " + str(p.sequences) + " sequences");
    // Values.
    for (int32_t token : b.token_ids)
        if (token < 0 || std::size_t(token) >= config_.vocab_size) reject(Reject::Token, "token " + std::to_string(token));
    for (int32_t row : b.last_token_indices)
        if (row < 0 || std::size_t(row) >= p.rows) reject(Reject::SampleRow, "row " + std::to_string(row));
    for (float temperature : b.temperatures)
        if (!(temperature >= 0.0f) || !std::isfinite(temperature))
            reject(Reject::Temperature, std::to_string(temperature));
    // Rows against their tables: the slot a row writes is the one its table
    // gives for its position, and no two rows write the same slot.
    auto block_at = [&](std::size_t sequence, std::size_t column) {
        return b.block_tables[sequence * b.table_stride + column];
    };
    auto is_block = [&](int32_t block) { return block >= 0 && std::size_t(block) < o.num_blocks; };
    std::vector<long long> last_position(p.sequences, -1);
    std::vector<std::size_t> rows_of(p.sequences, 0);
    std::unordered_set<int64_t> written;
    written.reserve(p.rows * 2);
    for (std::size_t r = 0; r < p.rows; ++r) {
        const int32_t position = b.positions[r], sequence = b.sequence_ids[r];
        if (position < 0 || std::size_t(position) >= o.max_model_len)
            reject(Reject::Position, "row " + str(r) + " at position " + std::to_string(position));
        if (sequence < 0 || std::size_t(sequence) >= p.sequences)
            reject(Reject::Sequence, "row " + str(r) + " in sequence " + std::to_string(sequence));
        const std::size_t column = std::size_t(position) / o.block_size;
        if (column >= b.table_stride)
            reject(Reject::TableColumn, "row " + str(r) + " needs table column " + str(column));
        const int32_t block = block_at(std::size_t(sequence), column);
        if (!is_block(block)) reject(Reject::Block, "row " + str(r) + " writes through block " + std::to_string(block));
        const int64_t slot = int64_t(block) * int64_t(o.block_size) + position % int64_t(o.block_size);
        if (b.slot_mapping[r] != slot)
            reject(Reject::Slot, "row " + str(r) + " has slot " + std::to_string(b.slot_mapping[r]) + ", its table gives " +
                                     std::to_string(slot));
        if (!written.insert(slot).second) reject(Reject::SlotReuse, "slot " + std::to_string(slot));
        last_position[std::size_t(sequence)] = std::max<long long>(last_position[std::size_t(sequence)], position);
        ++rows_of[std::size_t(sequence)];
    }
    // Every block a sequence's attention reads exists.
    for (std::size_t s = 0; s < p.sequences; ++s)
        for (long long column = 0; last_position[s] >= 0 && column <= last_position[s] / static_cast<long long>(o.block_size); ++column)
            if (!is_block(block_at(s, std::size_t(column))))
                reject(Reject::Context, "sequence " + str(s) + " column " + std::to_string(column));

    // Launch choices. The fused decode attention lets rows run without waiting
    // for each other's K/V writes, so it needs every row alone in its
    // sequence and no row reading a block another row writes.
    p.fused_attention = o.fuse_decode_attention && config_.head_dim == 128;
    for (std::size_t s = 0; p.fused_attention && s < p.sequences; ++s) p.fused_attention = rows_of[s] <= 1;
    if (p.fused_attention) {
        std::unordered_map<int32_t, std::size_t> writer;  // block -> the row writing into it
        for (std::size_t r = 0; r < p.rows; ++r)
            writer.emplace(int32_t(b.slot_mapping[r] / int32_t(o.block_size)), r);
        for (std::size_t r = 0; p.fused_attention && r < p.rows; ++r) {
            const std::size_t s = std::size_t(b.sequence_ids[r]);
            for (std::size_t column = 0; column <= std::size_t(b.positions[r]) / o.block_size; ++column) {
                const auto it = writer.find(block_at(s, column));
                if (it != writer.end() && it->second != r) {
                    p.fused_attention = false;
                    break;
                }
            }
        }
    }
    // The fused norm + GEMM kernels serve up to 16 rows (beyond that every
    // block's copy of the norm costs more than the launch it saves).
    p.fused_norms = norm_gemm_fits(config_, o) && p.rows <= kFusedNormRows;
    p.replayable = o.graphs && b.is_decode && p.rows == p.sequences && p.samples == p.sequences;
    return p;
}

void QwenModel::observe(Stage stage, std::size_t layer) const {
    if (observer_ && !capturing_) {
        gpu_.sync();
        observer_(stage, layer);
    }
}

void QwenModel::embed(const StepPlan& p) const {
    residual_ = &work_.residual;
    gpu_.embedding(work_.tokens, embedding_, work_.residual, p.rows, config_.hidden_size, config_.vocab_size);
    observe(Stage::Embedded);
}

// One decoder layer in Qwen3's order (src/model.rs:659-789): input norm (layer
// 0 normalises the embedding; later layers first add the previous MLP output
// into the residual), QKV projection, q/k norm + RoPE + KV write, paged
// attention, output projection, post-attention add-norm, gate/up projection,
// SiLU·up, down projection.
void QwenModel::decoder_layer(const StepPlan& p, std::size_t i) const {
    const ModelConfig& c = config_;
    const ModelOptions& o = options_;
    const Workspace& w = work_;
    const LayerWeights& l = layers_[i];
    const std::size_t h = c.hidden_size, q = c.num_attention_heads * c.head_dim;
    const std::size_t qkv = q + 2 * c.num_key_value_heads * c.head_dim;
    // With fused norms the residual alternates between its two buffers: each
    // add-norm reads one and writes the other.
    auto other = [&](const Buffer* b) { return b == &w.residual ? &w.residual_alt : &w.residual; };
    if (p.fused_norms) {
        if (i == 0) {
            gpu_.rms_gemm(*residual_, Buffer(), Buffer(), l.input_norm, l.qkv, w.qkv, w.normed, p.rows, qkv, h,
                          c.rms_norm_eps);
        } else {
            const Buffer* next = other(residual_);
            gpu_.rms_gemm(w.hidden, *residual_, *next, l.input_norm, l.qkv, w.qkv, w.normed, p.rows, qkv, h,
                          c.rms_norm_eps);
            residual_ = next;
        }
        observe(Stage::InputNorm, i);
    } else {
        if (i == 0)
            gpu_.rms_norm(*residual_, l.input_norm, w.normed, p.rows, h, c.rms_norm_eps);
        else
            gpu_.add_rms_norm(w.hidden, *residual_, l.input_norm, w.normed, p.rows, h, c.rms_norm_eps);
        observe(Stage::InputNorm, i);
        gpu_.gemm(w.normed, l.qkv, w.qkv, p.rows, qkv, h);
    }
    observe(Stage::Qkv, i);
    if (p.fused_attention) {
        gpu_.attention_qkv_rope(w.qkv, l.q_norm, l.k_norm, w.positions, w.slots, l.k_cache, l.v_cache, w.sequence_ids,
                                w.tables, w.attention, p.rows, c.num_attention_heads, c.num_key_value_heads,
                                c.head_dim, o.block_size, o.num_blocks, table_stride_, p.sequences, o.max_model_len,
                                c.rms_norm_eps, w.rope_cache, o.max_model_len);
    } else {
        gpu_.qkv_rope_cached(w.qkv, l.q_norm, l.k_norm, w.positions, w.slots, w.query, l.k_cache, l.v_cache, p.rows,
                             c.num_attention_heads, c.num_key_value_heads, c.head_dim, o.block_size, o.num_blocks,
                             c.rms_norm_eps, w.rope_cache, o.max_model_len);
        observe(Stage::QkvRope, i);
        gpu_.paged_attention(w.query, l.k_cache, l.v_cache, w.positions, w.sequence_ids, w.tables, w.attention, p.rows,
                             c.num_attention_heads, c.num_key_value_heads, c.head_dim, o.block_size, o.num_blocks,
                             table_stride_, p.sequences, o.max_model_len);
    }
    observe(Stage::Attention, i);
    // Decode-sized batches take nv_gemm_rows for the output and down
    // projections (hidden 1024 at 8 rows: 3.4 vs 5.5 us for o_proj, 4.2 vs
    // 7.2 us for down against hipBLAS).
    auto rows_gemm = [&](std::size_t k) {
        return p.fused_norms && (k == 1024 || k == 2048 || k == 3072 || k == 4096) && h % 16 == 0;
    };
    if (rows_gemm(q))
        gpu_.gemm_rows(w.attention, l.o_proj, w.hidden, p.rows, h, q);
    else
        gpu_.gemm(w.attention, l.o_proj, w.hidden, p.rows, h, q);
    observe(Stage::OutProj, i);
    if (p.fused_norms) {
        // Post-attention add-norm, gate_up projection and SiLU·up in one launch.
        const Buffer* next = other(residual_);
        gpu_.rms_gemm_silu(w.hidden, *residual_, *next, l.post_norm, l.gate_up_tiled, w.gate_up, w.activated,
                           w.normed, p.rows, c.intermediate_size, h, c.rms_norm_eps);
        residual_ = next;
        observe(Stage::PostNorm, i);
        observe(Stage::GateUp, i);
    } else {
        gpu_.add_rms_norm(w.hidden, *residual_, l.post_norm, w.normed, p.rows, h, c.rms_norm_eps);
        observe(Stage::PostNorm, i);
        gpu_.gemm(w.normed, l.gate_up, w.gate_up, p.rows, 2 * c.intermediate_size, h);
        observe(Stage::GateUp, i);
        gpu_.silu_mul(w.gate_up, w.activated, p.rows, c.intermediate_size);
    }
    observe(Stage::Activated, i);
    if (rows_gemm(c.intermediate_size))
        gpu_.gemm_rows(w.activated, l.down, w.hidden, p.rows, h, c.intermediate_size);
    else
        gpu_.gemm(w.activated, l.down, w.hidden, p.rows, h, c.intermediate_size);
    observe(Stage::Down, i);
}

// Final norm, the sampled rows, tied lm_head and the sampler
// (src/model.rs:781-815).
void QwenModel::head(const StepPlan& p) const {
    const ModelConfig& c = config_;
    const Workspace& w = work_;
    // The final add-RMSNorm computed for the sampled rows only, straight
    // into the gathered buffer (one launch instead of a norm over every row
    // and a gather).
    gpu_.add_rms_norm_gather(w.hidden, *residual_, final_norm_, w.last_rows, w.gathered, p.samples, c.hidden_size,
                             p.rows, c.rms_norm_eps);
    observe(Stage::FinalNorm);
    gpu_.gemm(w.gathered, lm_head_, w.logits, p.samples, c.vocab_size, c.hidden_size);
    observe(Stage::Logits);
    gpu_.sample_parallel(w.logits, w.temperatures, w.seeds, w.samples, w.partial_scores, w.partial_ids, p.samples,
                         c.vocab_size);
    observe(Stage::Sampled);
}

void QwenModel::forward(const StepPlan& p) const {
    embed(p);
    for (std::size_t i = 0; i < layers_.size(); ++i) decoder_layer(p, i);
    if (p.samples > 0) head(p);
}

std::vector<uint32_t> QwenModel::run(const Batch& batch) {
    const StepPlan p = plan(batch);
    last_samples_ = 0;
    record_.fill(host_record_, batch, p.sequences, table_stride_);
    work_.record.upload_bytes(host_record_);  // synchronous: the host copy may be refilled next step
    if (p.replayable) {
        const auto key = std::make_pair(p.rows, p.fused_attention);
        auto found = graphs_.find(key);
        if (found == graphs_.end()) {
            forward(p);  // warm-up: first use of each GEMM shape stays outside the capture
            gpu_.sync();
            capturing_ = true;
            try {
                Graph g = gpu_.capture([&] { forward(p); });
                capturing_ = false;
                found = graphs_.emplace(key, std::move(g)).first;
            } catch (...) {
                capturing_ = false;
                throw;
            }
        }
        found->second.replay();  // the replay rewrites the warm-up's KV slots with the same values
    } else {
        forward(p);
    }
    last_samples_ = p.samples;
    if (p.samples == 0) {
        gpu_.sync();
        return {};
    }
    std::vector<uint32_t> tokens;
    tokens.reserve(p.samples);
    for (int32_t id : work_.samples.download_i32(p.samples)) {
        if (id < 0 || std::size_t(id) >= config_.vocab_size)
            throw Error(Fault::Backend, "sampler returned token " + std::to_string(id));
        tokens.push_back(uint32_t(id));
    }
    return tokens;
}

std::vector<std::vector<float>> QwenModel::last_logits() const {
    const std::size_t v = config_.vocab_size;
    const std::vector<uint16_t> bits = work_.logits.download_u16(last_samples_ * v);
    std::vector<std::vector<float>> rows(last_samples_, std::vector<float>(v));
    for (std::size_t r = 0; r < last_samples_; ++r)
        for (std::size_t i = 0; i < v; ++i) {
            const uint32_t u = uint32_t(bits[r * v + i]) << 16;
            std::memcpy(&rows[r][i], &u, 4);
        }
    return rows;
}

}  // namespace nvr
