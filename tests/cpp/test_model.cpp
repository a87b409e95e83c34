// The Qwen3 runner (nano-vllm-rs_amd/host/model.hpp): the reference's own
// model tests that apply (packed metadata, src/model.rs:1232-1297), its batch
// validation (src/model.rs:820-923), and whole-forward checks on the GPU:
// graph replay against the eager forward, and decode against prefill.
//
// Usage: test_model cpu|gpu
#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "gpu.hpp"
#include "harness.hpp"
#include "model.hpp"

namespace {

using nvr::Batch;
using nvr::MetadataLayout;

void expect_error(const std::function<void()>& fn, const std::string& message) {
    try {
        fn();
    } catch (const nvr::Error& e) {
        if (message != e.what()) throw harness::Failure{"expected \"" + message + "\", got \"" + e.what() + "\""};
        return;
    }
    throw harness::Failure{"no error; expected \"" + message + "\""};
}

// -------------------------------------------------------------- CPU suite --
TEST(packed_metadata_preserves_values_alignment_and_clears_table_padding, "cpu") {  // src/model.rs:1232-1297
    const MetadataLayout layout = MetadataLayout::make(3, 2, 3);
    const MetadataLayout::Range ranges[] = {layout.tokens,       layout.positions,    layout.sequences,
                                            layout.slots,        layout.tables,       layout.last_indices,
                                            layout.temperatures, layout.seeds};
    for (const auto& r : ranges) {
        CHECK(r.start % 8 == 0);
        CHECK(r.end <= layout.bytes);
    }
    for (std::size_t i = 1; i < sizeof(ranges) / sizeof(ranges[0]); ++i) CHECK(ranges[i - 1].end <= ranges[i].start);
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
    std::vector<uint8_t> staging(layout.bytes, 0x55);
    layout.pack(staging, batch, 2, 3);
    auto i32s = [&](const MetadataLayout::Range& r) {
        std::vector<int32_t> out(r.size() / 4);
        std::memcpy(out.data(), staging.data() + r.start, r.size());
        return out;
    };
    CHECK(i32s(layout.tokens) == batch.token_ids);
    CHECK(i32s(layout.positions) == batch.positions);
    CHECK((i32s(layout.tables) == std::vector<int32_t>{2, -1, -1, 4, -1, -1}));
    CHECK(std::memcmp(staging.data() + layout.seeds.start, &batch.seeds[0], 8) == 0);
    const float t = 0.6f;
    CHECK(std::memcmp(staging.data() + layout.temperatures.start + 4, &t, 4) == 0);
    Batch smaller;
    smaller.token_ids = {21};
    smaller.positions = {0};
    smaller.sequence_ids = {0};
    smaller.slot_mapping = {70};
    smaller.block_tables = {7};
    smaller.table_stride = 1;
    layout.pack(staging, smaller, 1, 3);
    for (std::size_t i = 4; i < 12; ++i) CHECK(staging[layout.tables.start + i] == 0xff);
}

TEST(model_config_rejects_unsupported_shapes, "cpu") {  // src/model.rs:63-140
    nvr::ModelConfig c;
    c.validate();
    nvr::ModelConfig bad = c;
    bad.num_key_value_heads = 6;
    expect_error([&] { bad.validate(); }, "query heads must be a positive multiple of KV heads");
    bad = c;
    bad.head_dim = 131;
    expect_error([&] { bad.validate(); }, "head_dim must be even and at most 256");
    bad = c;
    bad.head_dim = 258;
    expect_error([&] { bad.validate(); }, "head_dim must be even and at most 256");
    bad = c;
    bad.rms_norm_eps = 0.0f;
    expect_error([&] { bad.validate(); }, "RMS epsilon and RoPE theta must be positive finite values");
    bad = c;
    bad.rope_theta = INFINITY;
    expect_error([&] { bad.validate(); }, "RMS epsilon and RoPE theta must be positive finite values");
    bad = c;
    bad.num_hidden_layers = 0;
    expect_error([&] { bad.validate(); }, "model dimensions must be positive");
}

// ---------------------------------------------------------- tiny model -----
// Qwen3's structure at small sizes (head_dim 128, GQA 4:2, vocabulary a
// multiple of 8), weights from a fixed SplitMix64 stream.
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
nvr::ModelOptions tiny_options(bool graphs) {
    nvr::ModelOptions o;
    o.block_size = 16;
    o.num_blocks = 64;
    o.max_batch_tokens = 64;
    o.max_sequences = 8;
    o.max_model_len = 256;
    o.graphs = graphs;
    return o;
}

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
// Normal(mean, std) by Box-Muller over a stream keyed by the tensor name.
nvr::WeightSource random_weights(uint64_t seed) {
    return [seed](const std::string& name, const std::vector<std::size_t>& shape) {
        std::size_t n = 1;
        for (std::size_t d : shape) n *= d;
        uint64_t state = seed;
        for (char ch : name) state = mix(state ^ uint8_t(ch));
        const bool norm = name.find("norm") != std::string::npos;
        const float mean = norm ? 1.0f : 0.0f, std = norm ? 0.02f : 0.05f;
        std::vector<uint16_t> out(n);
        for (std::size_t i = 0; i < n; ++i) {
            const double u1 = (double(mix(state + 2 * i) >> 11) + 0.5) * 0x1.0p-53;
            const double u2 = double(mix(state + 2 * i + 1) >> 11) * 0x1.0p-53;
            const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
            out[i] = bf16_bits(float(mean + std * z));
        }
        return out;
    };
}

// Sequence s owns physical blocks s*8 .. s*8+7 (the first rows of its table).
struct Tables {
    std::size_t stride = 16, block_size = 16;
    std::vector<int32_t> table(std::size_t sequences) const {
        std::vector<int32_t> t(sequences * stride, -1);
        for (std::size_t s = 0; s < sequences; ++s)
            for (std::size_t c = 0; c < 8; ++c) t[s * stride + c] = int32_t(s * 8 + c);
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
                 const std::vector<float>& temps, const std::vector<uint64_t>& seeds) {
    const Tables t;
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

TEST(model_rejects_invalid_batches_like_the_reference, "gpu") {  // src/model.rs:820-923
    nvr::QwenModel model(tiny_config(), tiny_options(true), random_weights(1));
    const Batch good = make_batch({{1, 2, 3}, {4}}, {0, 0}, {0, 1}, 2, false, {0.0f, 0.5f}, {1, 2});
    model.validate_batch(good);
    auto bad = [&](const std::function<void(Batch&)>& edit, const std::string& message) {
        Batch b = good;
        edit(b);
        expect_error([&] { model.validate_batch(b); }, message);
    };
    bad([](Batch& b) { b = Batch(); }, "batch token count is outside model capacity");
    bad([](Batch& b) { b.positions.pop_back(); }, "token metadata lengths differ");
    bad([](Batch& b) { b.table_stride = 0; }, "invalid block table shape");
    bad([](Batch& b) { b.table_stride = 17; }, "invalid block table shape");
    bad([](Batch& b) { b.block_tables.resize(16 * 9, 0); }, "batch sequence count exceeds capacity");
    bad([](Batch& b) { b.temperatures.pop_back(); }, "invalid sampling metadata lengths");
    bad([](Batch& b) { b.token_ids[0] = 1024; }, "token id outside model vocabulary");
    bad([](Batch& b) { b.last_token_indices[0] = 4; }, "sample row outside batch");
    bad([](Batch& b) { b.temperatures[1] = NAN; }, "temperature must be finite and nonnegative");
    bad([](Batch& b) { b.temperatures[1] = -1.0f; }, "temperature must be finite and nonnegative");
    bad([](Batch& b) { b.positions[0] = 256; }, "token position exceeds max_model_len");
    bad([](Batch& b) { b.sequence_ids[3] = 2; }, "token sequence index outside block tables");
    bad([](Batch& b) { b.positions[3] = 200; }, "invalid physical KV block");
    bad([](Batch& b) { b.block_tables[16] = 64; }, "invalid physical KV block");
    bad([](Batch& b) { b.slot_mapping[1] = 5; }, "KV slot mapping disagrees with block table");
    bad([](Batch& b) {
        b.positions[1] = 0;
        b.slot_mapping[1] = b.slot_mapping[0];
    }, "two input tokens write the same KV slot");
    bad([](Batch& b) {  // sequence 0's rows sit in column 1; column 0 is missing
        b.block_tables[0] = -1;
        for (int r = 0; r < 3; ++r) {
            b.positions[r] = 20 + r;
            b.slot_mapping[r] = 1 * 16 + 4 + r;
        }
    }, "missing KV block in causal context");
    Batch narrow = good;  // a table narrower than the token position
    narrow.table_stride = 1;
    narrow.block_tables = {0, 8};
    narrow.positions[2] = 16;
    narrow.slot_mapping[2] = 16;
    expect_error([&] { model.validate_batch(narrow); }, "block table does not cover token position");
}

bool same_bits(const std::vector<std::vector<float>>& a, const std::vector<std::vector<float>>& b) {
    if (a.size() != b.size()) return false;
    for (std::size_t r = 0; r < a.size(); ++r)
        if (a[r].size() != b[r].size() || std::memcmp(a[r].data(), b[r].data(), a[r].size() * 4) != 0) return false;
    return true;
}

TEST(decode_graphs_replay_the_eager_forward, "gpu") {
    // Two runners with the same weights, one replaying captured decode graphs
    // and one launching eagerly, fed the same prefill then decode steps whose
    // positions, slots and seeds change every step: samples and logits must be
    // identical bit for bit, with one graph per decode batch size.
    nvr::QwenModel graphs(tiny_config(), tiny_options(true), random_weights(2));
    nvr::QwenModel eager(tiny_config(), tiny_options(false), random_weights(2));
    const std::vector<std::vector<int32_t>> prompts = {{11, 12, 13, 14, 15}, {200, 201, 202, 203, 204, 205, 206, 207, 208}};
    const std::vector<float> temps = {0.0f, 0.8f, 0.0f};
    Batch prefill = make_batch({prompts[0], prompts[1], {300, 301}}, {0, 0, 0}, {0, 1, 2}, 3, false, temps, {7, 8, 9});
    std::vector<uint32_t> a = graphs.run(prefill), b = eager.run(prefill);
    CHECK(a == b);
    CHECK(same_bits(graphs.last_logits(), eager.last_logits()));
    std::vector<int32_t> next = {int32_t(a[0]), int32_t(a[1]), int32_t(a[2])};
    std::vector<int32_t> length = {5, 9, 2};
    for (int step = 0; step < 6; ++step) {
        // Steps 0-3 decode all three sequences; steps 4-5 only the first two.
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
        a = graphs.run(decode);
        b = eager.run(decode);
        CHECK(a == b);
        CHECK(same_bits(graphs.last_logits(), eager.last_logits()));
        for (std::size_t s = 0; s < live; ++s) {
            next[s] = int32_t(a[s]);
            ++length[s];
        }
    }
    CHECK(graphs.graph_count() == 2);  // 3-row and 2-row decode batches
    CHECK(eager.graph_count() == 0);
}

TEST(decode_step_matches_prefill_of_the_longer_prompt, "gpu") {
    // Decoding token x at position L after a prefill of L tokens must agree
    // with a prefill of the L + 1 tokens (KV write, cached RoPE, paged
    // attention over the cache, last-row gather): same greedy token, logits
    // equal up to the GEMMs' different row counts.
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
