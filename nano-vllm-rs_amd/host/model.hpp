// Qwen3 forward runner over the nv_* kernels: the C++ counterpart of
// nano-vllm-rs's QwenModel (src/model.rs), with the same outward interface
// (model config, runtime options, run a scheduler Batch, read the last
// logits). Internals are this library's own:
//
//  - StepPlan. A batch is checked once against the contract of plan() (see
//    Reject) and reduced to its row, sequence and sample counts and to two
//    launch choices: whether the attention of each layer may run in its fused
//    decode form, and whether the step may replay a captured graph.
//  - StepRecord. All per-step host data goes to the device in one synchronous
//    copy: one record whose arrays sit at fixed 256-byte aligned offsets
//    (widest elements first), sized for the configured capacities, so the
//    kernels' pointers are the same in every step and every graph replay.
//  - Graphs. A decode step that samples every row replays the HIP graph of
//    its (row count, attention form), captured on first use after one eager
//    warm-up forward: hipBLAS may set up state on a shape's first use, which a
//    capture cannot contain.
//  - Observer. Tests may watch every stage of an eager forward and read the
//    workspace and weights at that point (used to check the forward against
//    the CPU oracle stage by stage).
//
// Weights come from a WeightSource: the reference reads them from safetensors
// files by tensor name and shape (src/model.rs:425-517); any loader with that
// contract plugs in.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <map>
#include <string>
#include <utility>
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

    // Throws Fault::Value for a configuration the kernels cannot run.
    void validate() const;
};

// Runtime capacities (src/model.rs:150-173; `graphs` is the reference's
// cuda_graphs). fuse_decode_attention = false keeps every step on the
// separate q/k norm + RoPE and attention launches; fuse_norm_gemm = false
// keeps the norms apart from the GEMMs that follow them.
struct ModelOptions {
    int device = 0;
    std::size_t block_size = 256;
    std::size_t num_blocks = 128;
    std::size_t max_batch_tokens = 1024;
    std::size_t max_sequences = 32;
    std::size_t max_model_len = 4096;
    bool graphs = true;
    bool fuse_decode_attention = true;
    bool fuse_norm_gemm = true;
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

// Why plan() refused a batch (BatchError::reason()).
enum class Reject {
    Rows,         // no rows, or more than max_batch_tokens
    Lengths,      // positions, sequence ids or slots not one per row
    TableShape,   // table_stride 0 or wider than the model's, or tables not whole rows
    Sequences,    // no table row, or more than max_sequences
    Sampling,     // more sampled rows than sequences, or temperatures / seeds not one per sampled row
    Token,        // token id outside [0, vocab_size)
    SampleRow,    // sampled row index outside the batch
    Temperature,  // temperature negative, NaN or infinite
    Position,     // position outside [0, max_model_len)
    Sequence,     // sequence id outside the table rows
    TableColumn,  // position / block_size beyond table_stride
    Block,        // the table entry a row writes through is not a block of the cache
    Slot,         // slot_mapping differs from block * block_size + position % block_size
    SlotReuse,    // two rows write the same slot
    Context,      // a table entry before a sequence's last position is not a block of the cache
};
const char* reject_name(Reject reason);

class BatchError : public Error {
public:
    BatchError(Reject reason, const std::string& what) : Error(Fault::Batch, what), reason_(reason) {}
    Reject reason() const { return reason_; }

private:
    Reject reason_;
};

struct StepPlan {
    std::size_t rows = 0, sequences = 0, samples = 0;
    bool fused_attention = false;  // q/k norm + RoPE + KV write inside the attention launch
    bool fused_norms = false;      // input / post-attention norms inside the qkv / gate_up GEMM launches
    bool replayable = false;       // served by a captured graph
};

// Byte offsets of the arrays of one step's record in device memory.
struct StepRecord {
    struct Field {
        std::size_t offset = 0, bytes = 0;
    };
    Field seeds, tokens, positions, sequence_ids, slots, last_rows, tables, temperatures;
    std::size_t size = 0;

    // Layout for up to `rows` rows and `sequences` table rows of `table_stride`.
    static StepRecord for_capacity(std::size_t rows, std::size_t sequences, std::size_t table_stride);
    // Writes `batch` into `host` (size bytes); table rows are widened to
    // `table_stride` with -1 and unused table rows are -1.
    void fill(std::vector<uint8_t>& host, const Batch& batch, std::size_t sequences, std::size_t table_stride) const;
};

struct ModelMemoryInfo {
    std::size_t weights_bytes = 0, kv_cache_bytes = 0, workspace_bytes = 0;
};

// bf16 bits of the named tensor, row-major in `shape` (the element count must
// match; src/model.rs:425-437).
using WeightSource = std::function<std::vector<uint16_t>(const std::string& name, const std::vector<std::size_t>& shape)>;

// Points of an eager forward an observer sees, in order; `layer` is the layer
// index for the per-layer stages and 0 otherwise.
enum class Stage {
    Embedded,    // residual = embedding rows
    InputNorm,   // normed (and residual, from layer 1) after the input (add-)RMSNorm
    Qkv,         // qkv GEMM output
    QkvRope,     // query and this layer's K/V caches (separate launches only)
    Attention,   // attention output (and the caches, in the fused form)
    OutProj,     // hidden = o-proj GEMM output
    PostNorm,    // residual and normed after the post-attention add-RMSNorm
    GateUp,      // gate_up GEMM output (with fused norms, seen after the SiLU too)
    Activated,   // SiLU(gate) * up
    Down,        // hidden = down GEMM output
    FinalNorm,   // gathered = the final add-RMSNorm of the sampled rows (residual not updated)
    Logits,      // lm_head GEMM output
    Sampled,     // sampled token ids
};
using StageObserver = std::function<void(Stage stage, std::size_t layer)>;

// Device buffers a test may read (Workspace::*) at an observed stage.
struct Workspace {
    Buffer record, tokens, positions, sequence_ids, slots, tables, last_rows, temperatures, seeds;
    Buffer samples, partial_scores, partial_ids, rope_cache;
    // residual and residual_alt alternate as the residual stream when the
    // norms run inside the GEMMs (QwenModel::residual() names the current one).
    Buffer residual, residual_alt, hidden, normed, qkv, query, attention, gate_up, activated, gathered, logits;
};
struct LayerWeights {
    Buffer input_norm, qkv, q_norm, k_norm, o_proj, post_norm, gate_up, down, k_cache, v_cache;
    Buffer gate_up_tiled;  // gate_up in the fused SiLU kernel's tile row order (when fuse_norm_gemm)
};

class QwenModel {
public:
    QwenModel(const ModelConfig& config, const ModelOptions& options, const WeightSource& weights);

    // plan(), one record upload, the forward (a graph replay when the plan
    // allows), and the sampled token of each sampled row.
    std::vector<uint32_t> run(const Batch& batch);
    // bf16 logits of the last run's sampled rows, as f32.
    std::vector<std::vector<float>> last_logits() const;

    // Checks `batch` and chooses its launches; throws BatchError.
    StepPlan plan(const Batch& batch) const;

    void set_observer(StageObserver observer) { observer_ = std::move(observer); }
    const Workspace& workspace() const { return work_; }
    const LayerWeights& layer(std::size_t i) const { return layers_.at(i); }
    const Buffer& embedding_weight() const { return embedding_; }
    const Buffer& final_norm_weight() const { return final_norm_; }
    std::size_t table_stride() const { return table_stride_; }
    // The buffer holding the residual stream at the current point of the
    // forward (for observers).
    const Buffer& residual() const { return *residual_; }

    std::size_t graph_count() const { return graphs_.size(); }
    const ModelMemoryInfo& memory_usage() const { return memory_; }
    const ModelConfig& config() const { return config_; }
    const ModelOptions& options() const { return options_; }
    const Gpu& gpu() const { return gpu_; }

private:
    void forward(const StepPlan& plan) const;
    void embed(const StepPlan& plan) const;
    void decoder_layer(const StepPlan& plan, std::size_t i) const;
    void head(const StepPlan& plan) const;
    void observe(Stage stage, std::size_t layer = 0) const;

    ModelConfig config_;
    ModelOptions options_;
    Gpu gpu_;
    std::size_t table_stride_ = 0;
    StepRecord record_;
    std::vector<uint8_t> host_record_;
    std::vector<LayerWeights> layers_;
    Buffer embedding_, final_norm_, lm_head_;
    Workspace work_;
    ModelMemoryInfo memory_;
    std::map<std::pair<std::size_t, bool>, Graph> graphs_;  // (decode rows, fused attention) -> captured forward
    StageObserver observer_;
    bool capturing_ = false;
    mutable const Buffer* residual_ = nullptr;
    std::size_t last_samples_ = 0;
};

}  // namespace nvr
