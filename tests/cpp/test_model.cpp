// The Qwen3 runner (nano-vllm-rs_amd/host/model.hpp):
//  cpu: the step record layout, config checks;
//  gpu: batch checks (each rejection by its reason), the fused-attention
//       choice, the forward against the CPU oracle stage by stage (prefill
//       of 1024 rows, then a decode step of 8 rows), fused against split
//       attention, graph replay against the eager forward, decode against
//       prefill, memory accounting.
//
// Usage: test_model cpu|gpu
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "../../oracle/oracle.h"
#include "gpu.hpp"
#include "harness.hpp"
#include "model.hpp"

namespace {

using nvr::Batch;
using nvr::Reject;
using nvr::Stage;
using nvr::StepRecord;

void expect_reject(const std::function<void()>& fn, Reject reason, const char* what) {
    try {
        fn();
    } catch (const nvr::BatchError& e) {
        if (e.reason() != reason)
            throw harness::Failure{std::string(what) + ": rejected for " + nvr::reject_name(e.reason()) + " (" +
                                   e.what() + "), expected " + nvr::reject_name(reason)};
        return;
    }
    throw harness::Failure{std::string(what) + ": accepted; expected a rejection for " + nvr::reject_name(reason)};
}

// -------------------------------------------------------------- CPU suite --
TEST(step_record_layout_fill_and_table_padding, "cpu") {
    const StepRecord r = StepRecord::for_capacity(3, 2, 3);
    const StepRecord::Field fields[] = {r.seeds, r.tokens, r.positions, r.sequence_ids,
                                        r.slots, r.last_rows, r.tables, r.temperatures};
    for (const auto& f : fields) {
        CHECK(f.offset % 256 == 0);
        CHECK(f.offset + f.bytes <= r.size);
    }
    for (std::size_t i = 1; i < sizeof(fields) / sizeof(fields[0]); ++i)
        CHECK(fields[i - 1].offset + fields[i - 1].bytes <= fields[i].offset);
    CHECK(r.tables.bytes == 2 * 3 * 4 && r.seeds.bytes == 2 * 8 && r.tokens.bytes == 3 * 4);
    Batch batch;
    batch.token_ids = {5, 8, 13};
    batch.positions = {0, 1, 0};
    batch.sequence_ids = {0, 0, 1};
    batch.slot_mapping = {20, 21, 40};
    batch.block_tables = {2, 4};
    batch.table_stride = 1;
    batch.last_token_indices = {1, 2};
    batch.temperatures = {0.0f, 0.6f};
    batch.seeds = {0x0102030405060708ull, UINT64_MAX};
    std::vector<uint8_t> host(r.size, 0x55);
    r.fill(host, batch, 2, 3);
    auto ints = [&](const StepRecord::Field& f) {
        std::vector<int32_t> out(f.bytes / 4);
        std::memcpy(out.data(), host.data() + f.offset, f.bytes);
        return out;
    };
    CHECK(ints(r.tokens) == batch.token_ids);
    CHECK(ints(r.positions) == batch.positions);
    CHECK(ints(r.sequence_ids) == batch.sequence_ids);
    CHECK(ints(r.slots) == batch.slot_mapping);
    CHECK(ints(r.last_rows) == batch.last_token_indices);
    CHECK((ints(r.tables) == std::vector<int32_t>{2, -1, -1, 4, -1, -1}));  // rows widened with -1
    CHECK(std::memcmp(host.data() + r.seeds.offset + 8, &batch.seeds[1], 8) == 0);
    const float t = 0.6f;
    CHECK(std::memcmp(host.data() + r.temperatures.offset + 4, &t, 4) == 0);
    // A smaller batch leaves no stale table entry behind.
    Batch smaller;
    smaller.token_ids = {21};
    smaller.positions = {0};
    smaller.sequence_ids = {0};
    smaller.slot_mapping = {70};
    smaller.block_tables = {7};
    smaller.table_stride = 1;
    r.fill(host, smaller, 1, 3);
    CHECK((ints(r.tables) == std::vector<int32_t>{7, -1, -1, -1, -1, -1}));
}

TEST(model_config_rejects_unsupported_shapes, "cpu") {
    nvr::ModelConfig c;
    c.validate();
    auto bad = [&](const std::function<void(nvr::ModelConfig&)>& edit) {
        nvr::ModelConfig b = c;
        edit(b);
        CHECK_FAULT(b.validate(), nvr::Fault::Value);
    };
    bad([](nvr::ModelConfig& b) { b.num_key_value_heads = 6; });
    bad([](nvr::ModelConfig& b) { b.head_dim = 131; });
    bad([](nvr::ModelConfig& b) { b.head_dim = 258; });
    bad([](nvr::ModelConfig& b) { b.rms_norm_eps = 0.0f; });
    bad([](nvr::ModelConfig& b) { b.rope_theta = INFINITY; });
    bad([](nvr::ModelConfig& b) { b.num_hidden_layers = 0; });
}

// ---------------------------------------------------------- test models ----
uint64_t mix(uint64_t v) {
    v += 0x9e3779b97f4a7c15ull;
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}
uint16_t bf16_bits(float x) {
    uint32_t b;
    std::memcpy(&b, &x, 4);
    return uint16_t((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
float f32(uint16_t h) {
    const uint32_t u = uint32_t(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
// Normal(mean, std) by Box-Muller over a stream keyed by the tensor name
// (norm weights ~N(1, 0.02), the rest ~N(0, std)).
nvr::WeightSource random_weights(uint64_t seed, double std = 0.05) {
    return [seed, std](const std::string& name, const std::vector<std::size_t>& shape) {
        std::size_t n = 1;
        for (std::size_t d : shape) n *= d;
        uint64_t state = seed;
        for (char ch : name) state = mix(state ^ uint8_t(ch));
        const bool norm = name.find("norm") != std::string::npos;
        const double mean = norm ? 1.0 : 0.0, sd = norm ? 0.02 : std;
        std::vector<uint16_t> out(n);
        for (std::size_t i = 0; i < n; ++i) {
            const double u1 = (double(mix(state + 2 * i) >> 11) + 0.5) * 0x1.0p-53;
            const double u2 = double(mix(state + 2 * i + 1) >> 11) * 0x1.0p-53;
            const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
            out[i] = bf16_bits(float(mean + sd * z));
        }
        return out;
    };
}

// Qwen3's structure at small sizes (head_dim 128, GQA 4:2, vocabulary a
// multiple of 8).
nvr::ModelConfig tiny_config() {
    nvr::ModelConfig c;
    c.hidden_size = 256;
    c.intermediate_size = 512;
    c.num_hidden_layers = 2;
    c.num_attention_heads = 4;
    c.num_key_value_heads = 2;
    c.head_dim = 128;
    c.vocab_size = 1024;
    c.max_position_embeddings = 4096;
    return c;
}
nvr::ModelOptions tiny_options(bool graphs, bool fuse = true) {
    nvr::ModelOptions o;
    o.block_size = 16;
    o.num_blocks = 64;
    o.max_batch_tokens = 64;
    o.max_sequences = 8;
    o.max_model_len = 256;
    o.graphs = graphs;
    o.fuse_decode_attention = fuse;
    return o;
}

// Sequence s owns physical blocks s*8 .. s*8+7 (the first entries of its table).
struct Tables {
    std::size_t stride = 16, block_size = 16;
    std::vector<int32_t> table(std::size_t sequences) const {
        std::vector<int32_t> t(sequences * stride, -1);
        for (std::size_t s = 0; s < sequences; ++s)
            for (std::size_t c = 0; c < 8 && c < stride; ++c) t[s * stride + c] = int32_t(s * 8 + c);
        return t;
    }
    int32_t slot(std::size_t s, int32_t position) const {
        return int32_t((s * 8 + std::size_t(position) / block_size) * block_size + std::size_t(position) % block_size);
    }
};

// Rows for groups of tokens (group g: sequence seq_of_group[g], positions
// first_position[g] onward); the last row of each of the first temps.size()
// groups is sampled with that temperature and seed.
Batch make_batch(const std::vector<std::vector<int32_t>>& tokens, const std::vector<int32_t>& first_position,
                 const std::vector<std::size_t>& seq_of_group, std::size_t sequences, bool decode,
                 const std::vector<float>& temps, const std::vector<uint64_t>& seeds, const Tables& t = Tables()) {
    Batch b;
    for (std::size_t g = 0; g < tokens.size(); ++g) {
        for (std::size_t i = 0; i < tokens[g].size(); ++i) {
            const int32_t pos = first_position[g] + int32_t(i);
            b.token_ids.push_back(tokens[g][i]);
            b.positions.push_back(pos);
            b.sequence_ids.push_back(int32_t(seq_of_group[g]));
            b.slot_mapping.push_back(t.slot(seq_of_group[g], pos));
        }
        if (g < temps.size()) b.last_token_indices.push_back(int32_t(b.token_ids.size()) - 1);
    }
    b.block_tables = t.table(sequences);
    b.table_stride = t.stride;
    b.temperatures = temps;
    b.seeds = seeds;
    b.is_decode = decode;
    return b;
}

// ------------------------------------------------------ batch contract ----
TEST(plan_rejects_invalid_batches, "gpu") {
    nvr::QwenModel model(tiny_config(), tiny_options(true), random_weights(1));
    const Batch good = make_batch({{1, 2, 3}, {4}}, {0, 0}, {0, 1}, 2, false, {0.0f, 0.5f}, {1, 2});
    const nvr::StepPlan p = model.plan(good);
    CHECK(p.rows == 4 && p.sequences == 2 && p.samples == 2 && !p.replayable);
    auto bad = [&](const char* what, Reject reason, const std::function<void(Batch&)>& edit) {
        Batch b = good;
        edit(b);
        expect_reject([&] { model.plan(b); }, reason, what);
    };
    bad("empty", Reject::Rows, [](Batch& b) { b = Batch(); });
    bad("too many rows", Reject::Rows, [](Batch& b) { b.token_ids.resize(65, 1); });
    bad("short positions", Reject::Lengths, [](Batch& b) { b.positions.pop_back(); });
    bad("stride 0", Reject::TableShape, [](Batch& b) { b.table_stride = 0; });
    bad("stride above the model's", Reject::TableShape, [](Batch& b) { b.table_stride = 17; });
    bad("ragged tables", Reject::TableShape, [](Batch& b) { b.block_tables.push_back(0); });
    bad("too many sequences", Reject::Sequences, [](Batch& b) { b.block_tables.resize(16 * 9, 0); });
    bad("temperatures short", Reject::Sampling, [](Batch& b) { b.temperatures.pop_back(); });
    bad("more samples than sequences", Reject::Sampling, [](Batch& b) {
        b.last_token_indices.push_back(0);
        b.temperatures.push_back(0.0f);
        b.seeds.push_back(0);
    });
    bad("token past the vocabulary", Reject::Token, [](Batch& b) { b.token_ids[0] = 1024; });
    bad("negative token", Reject::Token, [](Batch& b) { b.token_ids[0] = -1; });
    bad("sampled row past the batch", Reject::SampleRow, [](Batch& b) { b.last_token_indices[0] = 4; });
    bad("NaN temperature", Reject::Temperature, [](Batch& b) { b.temperatures[1] = NAN; });
    bad("negative temperature", Reject::Temperature, [](Batch& b) { b.temperatures[1] = -1.0f; });
    bad("position past max_model_len", Reject::Position, [](Batch& b) { b.positions[0] = 256; });
    bad("sequence past the tables", Reject::Sequence, [](Batch& b) { b.sequence_ids[3] = 2; });
    bad("row's block missing", Reject::Block, [](Batch& b) { b.positions[3] = 200; });
    bad("row's block past the cache", Reject::Block, [](Batch& b) { b.block_tables[16] = 64; });
    bad("slot disagrees with the table", Reject::Slot, [](Batch& b) { b.slot_mapping[1] = 5; });
    bad("two rows, one slot", Reject::SlotReuse, [](Batch& b) {
        b.positions[1] = 0;
        b.slot_mapping[1] = b.slot_mapping[0];
    });
    bad("hole before the last position", Reject::Context, [](Batch& b) {
        b.block_tables[0] = -1;  // sequence 0's rows sit in column 1; column 0 is missing
        for (int r = 0; r < 3; ++r) {
            b.positions[r] = 20 + r;
            b.slot_mapping[r] = 1 * 16 + 4 + r;
        }
    });
    Batch narrow = good;  // a table narrower than the token position
    narrow.table_stride = 1;
    narrow.block_tables = {0, 8};
    narrow.positions[2] = 16;
    narrow.slot_mapping[2] = 16;
    expect_reject([&] { model.plan(narrow); }, Reject::TableColumn, "table narrower than the position");
}

TEST(plan_fuses_attention_only_for_independent_rows, "gpu") {
    nvr::QwenModel model(tiny_config(), tiny_options(true), random_weights(1));
    // A plain decode batch: one row per sequence, each in its own blocks.
    const Batch decode = make_batch({{1}, {2}, {3}}, {20, 7, 40}, {0, 1, 2}, 3, true, {0, 0, 0}, {0, 0, 0});
    nvr::StepPlan p = model.plan(decode);
    CHECK(p.fused_attention && p.replayable);
    // A sequence with two rows.
    const Batch two_rows = make_batch({{1, 2}, {3}}, {20, 7}, {0, 1}, 2, false, {0}, {0});
    CHECK(!model.plan(two_rows).fused_attention);
    // A prefix-shared block: sequence 1 (its row at position 20, in its own
    // column-1 block) maps sequence 0's first block in column 0, and sequence
    // 0's row (position 3) writes that block.
    Batch shared = make_batch({{1}, {2}, {3}}, {3, 20, 40}, {0, 1, 2}, 3, true, {0, 0, 0}, {0, 0, 0});
    CHECK(model.plan(shared).fused_attention);  // before the sharing: independent rows
    shared.block_tables[1 * 16 + 0] = shared.block_tables[0];
    p = model.plan(shared);
    CHECK(!p.fused_attention && p.replayable);
    // head_dim 64 has no fused kernel; the option turns fusion off.
    nvr::ModelConfig c64 = tiny_config();
    c64.head_dim = 64;
    nvr::QwenModel small_heads(c64, tiny_options(true), random_weights(1));
    CHECK(!small_heads.plan(decode).fused_attention);
    nvr::QwenModel unfused(tiny_config(), tiny_options(true, false), random_weights(1));
    CHECK(!unfused.plan(decode).fused_attention);
}

// ------------------------------------------------- the forward vs oracle ---
std::vector<uint16_t> down16(const nvr::Buffer& b, std::size_t n) { return b.download_u16(n); }

struct Mismatch {
    std::size_t count = 0, first = 0;
};
Mismatch compare(const std::vector<uint16_t>& got, const std::vector<uint16_t>& want, int ulps = 0) {
    Mismatch m;
    for (std::size_t i = 0; i < got.size(); ++i) {
        const auto key = [](uint16_t h) { return (h & 0x8000) ? -int(h & 0x7fff) : int(h & 0x7fff); };
        if (std::abs(key(got[i]) - key(want[i])) > ulps) {
            if (m.count++ == 0) m.first = i;
        }
    }
    return m;
}
#define CHECK_SAME(got, want, ulps, what)                                                                        \
    do {                                                                                                         \
        const Mismatch m_ = compare(got, want, ulps);                                                            \
        if (m_.count)                                                                                            \
            throw harness::Failure{std::string(what) + ": " + std::to_string(m_.count) + " of " +                \
                                   std::to_string((got).size()) + " differ, first at " + std::to_string(m_.first)}; \
    } while (0)

// A GEMM output against the float64 product of its own inputs: within
// 2^-8 |y| + 2^-20 k sum|x w| (fp32 accumulation and one bf16 rounding).
void check_gemm(const std::vector<uint16_t>& x, const std::vector<uint16_t>& w, const std::vector<uint16_t>& y,
                std::size_t rows, std::size_t n, std::size_t k, const std::string& what) {
    std::size_t outside = 0;
    for (std::size_t r = 0; r < rows; ++r)
        for (std::size_t j = 0; j < n; ++j) {
            double acc = 0.0, mag = 0.0;
            for (std::size_t i = 0; i < k; ++i) {
                const double p = double(f32(x[r * k + i])) * double(f32(w[j * k + i]));
                acc += p;
                mag += std::fabs(p);
            }
            const double bound = 0x1.0p-8 * std::fabs(acc) + 0x1.0p-20 * double(k) * mag;
            if (std::fabs(double(f32(y[r * n + j])) - acc) > bound) ++outside;
        }
    if (outside) throw harness::Failure{what + ": " + std::to_string(outside) + " outputs outside the GEMM bound"};
}

// Every stage of an eager forward against the oracle fed the GPU's own GEMM
// outputs: the non-GEMM kernels must give the oracle's bits (SiLU within 1
// bf16 ulp), the K/V caches must equal the oracle's, the lm_head GEMM must
// lie within the fp32-accumulation bound of the float64 product, and the
// sampled tokens must be the oracle sampler's on those logits.
struct OracleShadow {
    const nvr::QwenModel& m;
    const Batch* batch = nullptr;
    std::size_t rows = 0, threads = 16, stages = 0;
    std::vector<uint16_t> table, final_norm, residual, hidden, qkv, query, normed, act, gathered, logits;
    std::vector<std::vector<uint16_t>> in_norm, post_norm, q_norm, k_norm, kc, vc;
    std::vector<float> rope;

    explicit OracleShadow(const nvr::QwenModel& model) : m(model) {
        const nvr::ModelConfig& c = m.config();
        const nvr::ModelOptions& o = m.options();
        table = down16(m.embedding_weight(), c.vocab_size * c.hidden_size);
        final_norm = down16(m.final_norm_weight(), c.hidden_size);
        const std::size_t cache = o.num_blocks * o.block_size * c.num_key_value_heads * c.head_dim;
        for (std::size_t l = 0; l < c.num_hidden_layers; ++l) {
            in_norm.push_back(down16(m.layer(l).input_norm, c.hidden_size));
            post_norm.push_back(down16(m.layer(l).post_norm, c.hidden_size));
            q_norm.push_back(down16(m.layer(l).q_norm, c.head_dim));
            k_norm.push_back(down16(m.layer(l).k_norm, c.head_dim));
            kc.emplace_back(cache, 0);  // a fresh model's caches are zero
            vc.emplace_back(cache, 0);
        }
        rope.resize(o.max_model_len * c.head_dim);
        ora_rope_cache(rope.data(), int(o.max_model_len), int(c.head_dim), c.rope_theta, int(threads));
        const std::vector<float> gpu_rope = m.workspace().rope_cache.download_f32(rope.size());
        CHECK(std::memcmp(gpu_rope.data(), rope.data(), rope.size() * 4) == 0);
    }

    void operator()(Stage stage, std::size_t l) {
        const nvr::ModelConfig& c = m.config();
        const nvr::ModelOptions& o = m.options();
        const nvr::Workspace& w = m.workspace();
        const Batch& b = *batch;
        const int R = int(rows), H = int(c.hidden_size), I = int(c.intermediate_size);
        const int QH = int(c.num_attention_heads), KVH = int(c.num_key_value_heads), D = int(c.head_dim);
        const int S = int(b.block_tables.size() / b.table_stride);
        const std::string at = "layer " + std::to_string(l) + " ";
        ++stages;
        switch (stage) {
        case Stage::Embedded:
            residual.resize(rows * c.hidden_size);
            ora_embedding(b.token_ids.data(), table.data(), residual.data(), R, H, int(c.vocab_size), int(threads));
            CHECK_SAME(down16(m.residual(), residual.size()), residual, 0, "embedding");
            break;
        case Stage::InputNorm:
            normed.resize(residual.size());
            if (l == 0)
                ora_rms(residual.data(), in_norm[l].data(), normed.data(), R, H, c.rms_norm_eps, int(threads));
            else
                ora_add_rms(hidden.data(), residual.data(), in_norm[l].data(), normed.data(), R, H, c.rms_norm_eps,
                            int(threads));
            CHECK_SAME(down16(m.residual(), residual.size()), residual, 0, at + "input norm residual");
            CHECK_SAME(down16(w.normed, normed.size()), normed, 0, at + "input norm");
            break;
        case Stage::Qkv:
            qkv = down16(w.qkv, rows * std::size_t(QH + 2 * KVH) * c.head_dim);
            if (rows <= 16)  // decode-sized: the GEMM runs inside nv_rms_gemm
                check_gemm(normed, down16(m.layer(l).qkv, std::size_t(QH + 2 * KVH) * D * c.hidden_size), qkv, rows,
                           std::size_t(QH + 2 * KVH) * D, c.hidden_size, at + "qkv GEMM");
            break;
        case Stage::QkvRope:
        case Stage::Attention: {
            // The oracle's tables: the batch's rows widened to the model's
            // stride with -1, as the runner stages them.
            const std::size_t stride = m.table_stride();
            std::vector<int32_t> tables(std::size_t(S) * stride, -1);
            for (int s = 0; s < S; ++s)
                std::copy_n(b.block_tables.begin() + std::ptrdiff_t(std::size_t(s) * b.table_stride), b.table_stride,
                            tables.begin() + std::ptrdiff_t(std::size_t(s) * stride));
            const bool rotate = stage == Stage::QkvRope || query.empty();
            if (rotate) {  // q/k norm + RoPE + KV write (in the fused form, inside the attention stage)
                query.assign(rows * std::size_t(QH) * c.head_dim, 0);
                ora_qkv_rope(qkv.data(), q_norm[l].data(), k_norm[l].data(), b.positions.data(),
                             b.slot_mapping.data(), query.data(), kc[l].data(), vc[l].data(), R, QH, KVH, D,
                             int(o.block_size), int(o.num_blocks), c.rms_norm_eps, 1.0f, rope.data(),
                             int(o.max_model_len), int(threads));
            }
            if (stage == Stage::QkvRope) {
                CHECK_SAME(down16(w.query, query.size()), query, 0, at + "rotated q");
            } else {
                std::vector<uint16_t> out(query.size());
                ora_attention(query.data(), kc[l].data(), vc[l].data(), b.positions.data(), b.sequence_ids.data(),
                              tables.data(), out.data(), R, QH, KVH, D, int(o.block_size), int(o.num_blocks),
                              int(stride), S, int(o.max_model_len), int(threads));
                CHECK_SAME(down16(w.attention, out.size()), out, 0, at + "attention");
                query.clear();
            }
            CHECK_SAME(down16(m.layer(l).k_cache, kc[l].size()), kc[l], 0, at + "K cache");
            CHECK_SAME(down16(m.layer(l).v_cache, vc[l].size()), vc[l], 0, at + "V cache");
            break;
        }
        case Stage::OutProj:
        case Stage::Down: {
            const std::vector<uint16_t> in = stage == Stage::OutProj
                                                 ? down16(w.attention, rows * std::size_t(QH) * D)
                                                 : down16(w.activated, rows * c.intermediate_size);
            hidden = down16(w.hidden, rows * c.hidden_size);
            if (rows <= 16) {
                const std::size_t k = stage == Stage::OutProj ? std::size_t(QH) * D : c.intermediate_size;
                check_gemm(in, down16(stage == Stage::OutProj ? m.layer(l).o_proj : m.layer(l).down, c.hidden_size * k),
                           hidden, rows, c.hidden_size, k, at + (stage == Stage::OutProj ? "o_proj GEMM" : "down GEMM"));
            }
            break;
        }
        case Stage::PostNorm:
            ora_add_rms(hidden.data(), residual.data(), post_norm[l].data(), normed.data(), R, H, c.rms_norm_eps,
                        int(threads));
            CHECK_SAME(down16(m.residual(), residual.size()), residual, 0, at + "add-norm residual");
            CHECK_SAME(down16(w.normed, normed.size()), normed, 0, at + "add-norm");
            break;
        case Stage::FinalNorm: {
            // The runner computes the final add-RMSNorm for the sampled rows
            // only, straight into the gathered rows: those must equal the
            // oracle's norm over every row followed by the gather, and the
            // residual is left as it was.
            const std::vector<uint16_t> before = residual;
            ora_add_rms(hidden.data(), residual.data(), final_norm.data(), normed.data(), R, H, c.rms_norm_eps,
                        int(threads));
            const std::size_t n = b.last_token_indices.size();
            gathered.resize(n * c.hidden_size);
            ora_gather(normed.data(), b.last_token_indices.data(), gathered.data(), int(n), H, R, int(threads));
            CHECK_SAME(down16(w.gathered, gathered.size()), gathered, 0, "final norm of the sampled rows");
            CHECK_SAME(down16(m.residual(), before.size()), before, 0, "final norm residual");
            break;
        }
        case Stage::GateUp: {
            const std::vector<uint16_t> gate_up = down16(w.gate_up, rows * 2 * c.intermediate_size);
            if (rows <= 16)
                check_gemm(normed, down16(m.layer(l).gate_up, 2 * c.intermediate_size * c.hidden_size), gate_up,
                           rows, 2 * c.intermediate_size, c.hidden_size, at + "gate_up GEMM");
            act.resize(rows * c.intermediate_size);
            ora_silu(gate_up.data(), act.data(), R, I, int(threads));
            break;
        }
        case Stage::Activated:
            CHECK_SAME(down16(w.activated, act.size()), act, 1, at + "SiLU");
            break;
        case Stage::Logits: {
            const std::size_t n = b.last_token_indices.size(), V = c.vocab_size, K = c.hidden_size;
            logits = down16(w.logits, n * V);
            std::size_t outside = 0;
            for (std::size_t r = 0; r < n; ++r)
                for (std::size_t v = 0; v < V; ++v) {
                    double y = 0.0, mag = 0.0;
                    for (std::size_t k = 0; k < K; ++k) {
                        const double p = double(f32(gathered[r * K + k])) * double(f32(table[v * K + k]));
                        y += p;
                        mag += std::fabs(p);
                    }
                    const double bound = 0x1.0p-8 * std::fabs(y) + 0x1.0p-20 * double(K) * mag;
                    if (std::fabs(double(f32(logits[r * V + v])) - y) > bound) ++outside;
                }
            if (outside) throw harness::Failure{"lm_head: " + std::to_string(outside) + " logits outside the bound"};
            break;
        }
        case Stage::Sampled: {
            const std::size_t n = b.last_token_indices.size();
            std::vector<int32_t> want(n);
            ora_sample(logits.data(), b.temperatures.data(), b.seeds.data(), want.data(), int(n), int(c.vocab_size),
                       int(threads));
            CHECK(w.samples.download_i32(n) == want);
            break;
        }
        }
    }
};

// Qwen3-0.6B widths (hidden 1024, intermediate 3072, 16/8 heads of 128,
// vocabulary 151936) with three layers, run eagerly so that every stage is
// observed: a prefill of S sequences x P tokens sampling every sequence, then
// a decode step of those S sequences.
void stage_by_stage(std::size_t S, std::size_t P) {
    nvr::ModelConfig c;
    c.num_hidden_layers = 3;
    nvr::ModelOptions o;
    o.block_size = 256;
    o.num_blocks = 2 * S;
    o.max_batch_tokens = S * P;
    o.max_sequences = S;
    o.max_model_len = 512;
    o.graphs = false;
    nvr::QwenModel model(c, o, random_weights(11, 0.03));
    OracleShadow shadow(model);
    model.set_observer([&](Stage st, std::size_t l) { shadow(st, l); });
    Tables t;
    t.block_size = 256;
    t.stride = 2;
    std::vector<std::vector<int32_t>> prompts(S);
    std::vector<int32_t> starts(S, 0);
    std::vector<std::size_t> seqs(S);
    std::vector<float> temps(S);
    std::vector<uint64_t> seeds(S);
    for (std::size_t s = 0; s < S; ++s) {
        for (std::size_t i = 0; i < P; ++i) prompts[s].push_back(int32_t(mix(s * 1000 + i) % c.vocab_size));
        seqs[s] = s;
        temps[s] = s % 2 ? 0.6f : 0.0f;
        seeds[s] = nvr::sampling_seed(9, s, 0);
    }
    // Sequence s owns blocks 2s and 2s + 1.
    auto batch_of = [&](const std::vector<std::vector<int32_t>>& toks, const std::vector<int32_t>& first, bool decode,
                        const std::vector<uint64_t>& sd) {
        Batch b = make_batch(toks, first, seqs, S, decode, temps, sd, t);
        for (std::size_t s = 0; s < S; ++s) {
            b.block_tables[s * 2] = int32_t(2 * s);
            b.block_tables[s * 2 + 1] = int32_t(2 * s + 1);
        }
        for (std::size_t r = 0; r < b.token_ids.size(); ++r)
            b.slot_mapping[r] = int32_t(2 * std::size_t(b.sequence_ids[r]) * 256 + std::size_t(b.positions[r]));
        return b;
    };
    const Batch prefill = batch_of(prompts, starts, false, seeds);
    shadow.batch = &prefill;
    shadow.rows = prefill.token_ids.size();
    const std::vector<uint32_t> first = model.run(prefill);
    std::printf("[prefill: %zu stages] ", shadow.stages);
    CHECK(shadow.stages == 1 + 3 * 9 + 3);  // split attention (a QkvRope stage) in the prefill
    std::vector<std::vector<int32_t>> next(S);
    std::vector<int32_t> at(S, int32_t(P));
    for (std::size_t s = 0; s < S; ++s) {
        next[s] = {int32_t(first[s])};
        seeds[s] = nvr::sampling_seed(9, s, 1);
    }
    const Batch decode = batch_of(next, at, true, seeds);
    CHECK(model.plan(decode).fused_attention);
    shadow.batch = &decode;
    shadow.rows = decode.token_ids.size();
    shadow.stages = 0;
    model.run(decode);
    std::printf("[decode: %zu stages] ", shadow.stages);
    CHECK(shadow.stages == 1 + 3 * 8 + 3);  // fused attention: no QkvRope stage
}

TEST(forward_matches_the_oracle_stage_by_stage, "gpu") { stage_by_stage(8, 128); }

// 16 decode rows: the widest fused-norm step (one norm pass in 8-wave blocks
// for qkv, two in 4-wave blocks for gate_up, the 16-row narrow GEMMs).
TEST(forward_matches_the_oracle_stage_by_stage_16_rows, "gpu") { stage_by_stage(16, 64); }

// ------------------------------------------------------ runner behaviour ---
bool same_bits(const std::vector<std::vector<float>>& a, const std::vector<std::vector<float>>& b) {
    if (a.size() != b.size()) return false;
    for (std::size_t r = 0; r < a.size(); ++r)
        if (a[r].size() != b[r].size() || std::memcmp(a[r].data(), b[r].data(), a[r].size() * 4) != 0) return false;
    return true;
}

// Runs a prefill of three prompts, then six decode steps whose positions,
// slots and seeds change every step (steps 4-5 decode two sequences), on two
// runners with the same weights; samples and logits must match bit for bit.
void lockstep(nvr::QwenModel& a_model, nvr::QwenModel& b_model) {
    const std::vector<std::vector<int32_t>> prompts = {{11, 12, 13, 14, 15}, {200, 201, 202, 203, 204, 205, 206, 207, 208}};
    const std::vector<float> temps = {0.0f, 0.8f, 0.0f};
    Batch prefill = make_batch({prompts[0], prompts[1], {300, 301}}, {0, 0, 0}, {0, 1, 2}, 3, false, temps, {7, 8, 9});
    std::vector<uint32_t> a = a_model.run(prefill), b = b_model.run(prefill);
    CHECK(a == b);
    CHECK(same_bits(a_model.last_logits(), b_model.last_logits()));
    std::vector<int32_t> next = {int32_t(a[0]), int32_t(a[1]), int32_t(a[2])};
    std::vector<int32_t> length = {5, 9, 2};
    for (int step = 0; step < 6; ++step) {
        const std::size_t live = step < 4 ? 3 : 2;
        std::vector<std::vector<int32_t>> toks;
        std::vector<int32_t> pos;
        std::vector<std::size_t> seqs;
        std::vector<float> t;
        std::vector<uint64_t> seeds;
        for (std::size_t s = 0; s < live; ++s) {
            toks.push_back({next[s]});
            pos.push_back(length[s]);
            seqs.push_back(s);
            t.push_back(temps[s]);
            seeds.push_back(nvr::sampling_seed(3, s, std::size_t(step)));
        }
        const Batch decode = make_batch(toks, pos, seqs, live, true, t, seeds);
        a = a_model.run(decode);
        b = b_model.run(decode);
        CHECK(a == b);
        CHECK(same_bits(a_model.last_logits(), b_model.last_logits()));
        for (std::size_t s = 0; s < live; ++s) {
            next[s] = int32_t(a[s]);
            ++length[s];
        }
    }
}

TEST(decode_graphs_replay_the_eager_forward, "gpu") {
    nvr::QwenModel graphs(tiny_config(), tiny_options(true), random_weights(2));
    nvr::QwenModel eager(tiny_config(), tiny_options(false), random_weights(2));
    lockstep(graphs, eager);
    CHECK(graphs.graph_count() == 2);  // 3-row and 2-row decode batches
    CHECK(eager.graph_count() == 0);
}

TEST(fused_and_split_attention_give_identical_steps, "gpu") {
    nvr::QwenModel fused(tiny_config(), tiny_options(true, true), random_weights(5));
    nvr::QwenModel split(tiny_config(), tiny_options(true, false), random_weights(5));
    lockstep(fused, split);
}

TEST(decode_step_matches_prefill_of_the_longer_prompt, "gpu") {
    // Decoding token x at position L after a prefill of L tokens must agree
    // with a prefill of the L + 1 tokens (KV write, cached RoPE, paged
    // attention over the cache, last-row gather): the same greedy token, and
    // logits equal within the GEMMs' row-count-dependent rounding.
    nvr::QwenModel model(tiny_config(), tiny_options(true), random_weights(3));
    std::vector<int32_t> prompt;
    for (int i = 0; i < 21; ++i) prompt.push_back(int32_t((i * 37 + 5) % 1024));
    const int32_t x = 777;
    model.run(make_batch({prompt}, {0}, {0}, 1, false, {0.0f}, {0}));
    const std::vector<uint32_t> dec = model.run(make_batch({{x}}, {21}, {0}, 1, true, {0.0f}, {0}));
    const std::vector<float> dec_logits = model.last_logits()[0];
    std::vector<int32_t> longer = prompt;
    longer.push_back(x);
    // Sequence 1 (its own blocks) gets the whole prompt at once.
    const std::vector<uint32_t> pre = model.run(make_batch({{1}, longer}, {0, 0}, {0, 1}, 2, false, {0.0f, 0.0f}, {0, 0}));
    const std::vector<float> pre_logits = model.last_logits()[1];
    double worst = 0.0, scale = 0.0;
    for (std::size_t i = 0; i < dec_logits.size(); ++i) {
        worst = std::fmax(worst, std::fabs(double(dec_logits[i]) - pre_logits[i]));
        scale = std::fmax(scale, std::fabs(double(pre_logits[i])));
    }
    std::printf("[max |logit| %.4f, max diff %.5f] ", scale, worst);
    CHECK(scale > 0.05);
    CHECK(worst <= 0.02 * scale + 1e-3);
    CHECK(dec[0] == pre[1]);
}

TEST(model_reports_memory_and_keeps_graphs_per_batch_size, "gpu") {
    nvr::QwenModel model(tiny_config(), tiny_options(true), random_weights(4));
    const nvr::ModelMemoryInfo& m = model.memory_usage();
    const nvr::ModelConfig c = tiny_config();
    const std::size_t per_layer = c.hidden_size * 2 + (512 + 2 * 256) * c.hidden_size + 2 * c.head_dim +
                                  c.hidden_size * 512 + 2 * c.intermediate_size * c.hidden_size +
                                  c.hidden_size * c.intermediate_size;
    CHECK(m.weights_bytes == 2 * (c.vocab_size * c.hidden_size + c.hidden_size + 2 * per_layer));
    CHECK(m.kv_cache_bytes == 2 * 2 * 64 * 16 * 256 * 2);
    CHECK(m.workspace_bytes > 0);
    // A decode batch that does not sample every row runs eagerly.
    Batch partial = make_batch({{1}, {2}}, {0, 0}, {0, 1}, 2, true, {0.0f}, {0});
    model.run(partial);
    CHECK(model.graph_count() == 0);
    model.run(make_batch({{3}, {4}}, {1, 1}, {0, 1}, 2, true, {0.0f, 0.0f}, {0, 0}));
    CHECK(model.graph_count() == 1);
    model.run(make_batch({{5}, {6}}, {2, 2}, {0, 1}, 2, true, {0.0f, 0.0f}, {0, 0}));
    CHECK(model.graph_count() == 1);
    // Prefill without samples synchronises and returns nothing.
    CHECK(model.run(make_batch({{7, 8}}, {3}, {0}, 1, false, {}, {})).empty());
}

}  // namespace
