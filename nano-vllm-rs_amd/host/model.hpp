// Qwen3 forward over the nv_* kernels: the runner of nano-vllm-rs's
// src/model.rs (QwenModel, Workspace, MetadataLayout, validate_batch, run) on
// the C++ host API of gpu.hpp.
//
// Persistent bf16 workspaces sized for the configured capacities, a paged KV
// cache per layer, every per-batch input packed into one staging buffer with
// fixed, 8-byte aligned ranges (one upload per step, and kernel pointers that
// stay identical across graph replays), and one HIP graph per decode batch
// size, captured on first use after a warm-up forward.
//
// Weights come from a WeightSource: the reference reads them from safetensors
// files by tensor name and shape (src/model.rs:425-517); any loader with that
// contract plugs in here.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <map>
#include <string>
#include <vector>

#include "gpu.hpp"

namespace nvr {

// The Qwen3 fields the forward uses (src/model.rs:18-48).
struct ModelConfig {
    std::size_t hidden_size = 1024;
    std::size_t intermediate_size = 3072;
    std::size_t num_hidden_layers = 28;
    std::size_t num_attention_heads = 16;
    std::size_t num_key_value_heads = 8;
    std::size_t head_dim = 128;
    std::size_t vocab_size = 151936;
    std::size_t max_position_embeddings = 40960;
    float rms_norm_eps = 1e-6f;
    float rope_theta = 1e6f;
    bool tie_word_embeddings = true;

    void validate() const;  // src/model.rs:63-140 (dimension and value checks)
};

// src/model.rs:150-173; cuda_graphs is `graphs`.
struct ModelOptions {
    int device = 0;
    std::size_t block_size = 256;
    std::size_t num_blocks = 128;
    std::size_t max_batch_tokens = 1024;
    std::size_t max_sequences = 32;
    std::size_t max_model_len = 4096;
    bool graphs = true;
};

// One scheduler step (src/runtime.rs:18-29): flattened rows, paged block
// tables of `table_stride` entries per sequence, and the rows to sample.
struct Batch {
    std::vector<int32_t> token_ids, positions, sequence_ids, slot_mapping, block_tables;
    std::size_t table_stride = 0;
    std::vector<int32_t> last_token_indices;
    std::vector<float> temperatures;
    std::vector<uint64_t> seeds;
    bool is_decode = false;
};

// Byte ranges of the packed per-step metadata (src/model.rs:269-359): each
// segment starts 8-byte aligned; block tables are padded with -1 up to the
// model's table stride.
struct MetadataLayout {
    struct Range {
        std::size_t start = 0, end = 0;
        std::size_t size() const { return end - start; }
    };
    Range tokens, positions, sequences, slots, tables, last_indices, temperatures, seeds;
    std::size_t bytes = 0;

    static MetadataLayout make(std::size_t tokens, std::size_t sequences, std::size_t table_stride);
    void pack(std::vector<uint8_t>& staging, const Batch& batch, std::size_t sequences,
              std::size_t table_stride) const;
};

struct ModelMemoryInfo {
    std::size_t weights_bytes = 0, kv_cache_bytes = 0, workspace_bytes = 0;
};

// bf16 bits of the named tensor, row-major in `shape` (the element count must
// match; src/model.rs:425-437).
using WeightSource = std::function<std::vector<uint16_t>(const std::string& name, const std::vector<std::size_t>& shape)>;

class QwenModel {
public:
    QwenModel(const ModelConfig& config, const ModelOptions& options, const WeightSource& weights);

    // Validates, uploads the packed metadata (one synchronous copy), runs the
    // forward (as a graph replay for decode batches that sample every row),
    // and returns the sampled token of each sampled row (src/model.rs:925-987).
    std::vector<uint32_t> run(const Batch& batch);
    // bf16 logits of the last run's sampled rows, as f32 (src/model.rs:617-633).
    std::vector<std::vector<float>> last_logits() const;

    std::size_t graph_count() const { return graphs_.size(); }
    const ModelMemoryInfo& memory_usage() const { return memory_; }
    const ModelConfig& config() const { return config_; }
    const ModelOptions& options() const { return options_; }
    const Gpu& gpu() const { return gpu_; }

    // rows, sequences, samples of a valid batch (src/model.rs:820-923).
    // {rows, sequences, samples, fused}: fused = 1 when the q/k norm + RoPE +
    // KV write may run inside the attention launch (head dim 128, one row per
    // sequence, and no row's context holds a block another row writes).
    std::array<std::size_t, 4> validate_batch(const Batch& batch) const;

private:
    struct Layer {
        Buffer input_norm, qkv, q_norm, k_norm, attention_out, post_norm, gate_up, down, k_cache, v_cache;
    };
    struct Workspace {
        Buffer metadata, tokens, positions, seq_indices, slots, block_tables, last_indices, temperatures, seeds;
        Buffer samples, sample_scores, sample_ids, rope_cache;
        Buffer residual, hidden, normed, qkv, query, attention, gate_up, activated, gathered, logits;
    };

    void forward(std::size_t rows, std::size_t sequences, std::size_t samples, bool fused) const;

    ModelConfig config_;
    ModelOptions options_;
    Gpu gpu_;
    std::size_t table_stride_ = 0;
    MetadataLayout layout_;
    std::vector<uint8_t> host_metadata_;
    std::vector<Layer> layers_;
    Buffer embedding_, final_norm_, lm_head_;
    Workspace work_;
    ModelMemoryInfo memory_;
    std::map<std::size_t, Graph> graphs_;  // 2 * decode row count + fused -> captured forward
    std::size_t last_sample_count_ = 0;
};

}  // namespace nvr
