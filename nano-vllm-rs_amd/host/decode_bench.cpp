// Serving-step benchmark of the Qwen3 runner (model.hpp) at Qwen3-0.6B shapes
// with random bf16 weights, in the shape of nano-vllm-rs's throughput-b8
// workload: S sequences whose prompts total 1024 tokens prefill in one
// forward, then D decode steps of S rows at T = 0.6, each one HIP graph
// replay. The eager forward of the same decode steps is timed too.
//
// Usage: decode_bench [S=8] [D=127] [eager]   -> one JSON line on stdout.
// With "eager" no graph is captured (both timed loops launch eagerly), for
// profilers that do not follow graph launches.
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "model.hpp"

namespace {

uint64_t mix(uint64_t v) {
    v += 0x9e3779b97f4a7c15ull;
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
    return v ^ (v >> 31);
}

// One pool of N(0,1) bf16-ready floats, sliced per tensor at a name-keyed offset
// (weights: std 0.02; norm weights: 1 + 0.02 z).
nvr::WeightSource pooled_weights() {
    constexpr std::size_t kPool = std::size_t(1) << 24;
    auto pool = std::make_shared<std::vector<float>>(kPool);
    for (std::size_t i = 0; i < kPool; ++i) {
        const double u1 = (double(mix(2 * i) >> 11) + 0.5) * 0x1.0p-53;
        const double u2 = double(mix(2 * i + 1) >> 11) * 0x1.0p-53;
        (*pool)[i] = float(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
    }
    return [pool](const std::string& name, const std::vector<std::size_t>& shape) {
        std::size_t n = 1;
        for (std::size_t d : shape) n *= d;
        uint64_t h = 0;
        for (char c : name) h = mix(h ^ uint8_t(c));
        const bool norm = name.find("norm") != std::string::npos;
        std::vector<uint16_t> out(n);
        std::size_t at = h % kPool;
        for (std::size_t i = 0; i < n; ++i, at = at + 1 == kPool ? 0 : at + 1) {
            const float x = norm ? 1.0f + 0.02f * (*pool)[at] : 0.02f * (*pool)[at];
            uint32_t b;
            std::memcpy(&b, &x, 4);
            out[i] = uint16_t((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
        }
        return out;
    };
}

double now_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

}  // namespace

int main(int argc, char** argv) {
    const std::size_t S = argc > 1 ? std::strtoul(argv[1], nullptr, 10) : 8;
    const std::size_t D = argc > 2 ? std::strtoul(argv[2], nullptr, 10) : 127;
    nvr::ModelConfig config;     // Qwen3-0.6B
    nvr::ModelOptions options;   // block 256, 128 blocks, 1024 batch tokens, 32 sequences, 4096 context
    options.graphs = !(argc > 3 && std::strcmp(argv[3], "eager") == 0);
    if (S == 0 || S > options.max_sequences || 1024 % S != 0) {
        std::fprintf(stderr, "S must divide 1024 and be at most %zu\n", options.max_sequences);
        return 2;
    }
    try {
        nvr::QwenModel model(config, options, pooled_weights());
        const std::size_t prompt = 1024 / S, bs = options.block_size;
        const std::size_t stride = (options.max_model_len + bs - 1) / bs;
        const std::size_t per_seq = (prompt + D + 1 + bs - 1) / bs;  // blocks per sequence
        if (per_seq * S > options.num_blocks) {
            std::fprintf(stderr, "KV cache too small for %zu sequences of %zu tokens\n", S, prompt + D + 1);
            return 2;
        }
        std::vector<int32_t> tables(S * stride, -1);
        for (std::size_t s = 0; s < S; ++s)
            for (std::size_t c = 0; c < per_seq; ++c) tables[s * stride + c] = int32_t(s * per_seq + c);
        auto slot = [&](std::size_t s, std::size_t pos) { return int32_t((s * per_seq + pos / bs) * bs + pos % bs); };

        nvr::Batch prefill;
        for (std::size_t s = 0; s < S; ++s) {
            for (std::size_t i = 0; i < prompt; ++i) {
                prefill.token_ids.push_back(int32_t(mix(s * 4096 + i) % config.vocab_size));
                prefill.positions.push_back(int32_t(i));
                prefill.sequence_ids.push_back(int32_t(s));
                prefill.slot_mapping.push_back(slot(s, i));
            }
            prefill.last_token_indices.push_back(int32_t(prefill.token_ids.size() - 1));
            prefill.temperatures.push_back(0.6f);
            prefill.seeds.push_back(nvr::sampling_seed(0, s, 0));
        }
        prefill.block_tables = tables;
        prefill.table_stride = stride;
        model.run(prefill);  // warm-up (hipBLAS shapes, code objects)
        const double p0 = now_ms();
        std::vector<uint32_t> next = model.run(prefill);
        const double prefill_ms = now_ms() - p0;

        auto step = [&](std::size_t d, bool decode) {
            nvr::Batch b;
            for (std::size_t s = 0; s < S; ++s) {
                b.token_ids.push_back(int32_t(next[s]));
                b.positions.push_back(int32_t(prompt + d));
                b.sequence_ids.push_back(int32_t(s));
                b.slot_mapping.push_back(slot(s, prompt + d));
                b.last_token_indices.push_back(int32_t(s));
                b.temperatures.push_back(0.6f);
                b.seeds.push_back(nvr::sampling_seed(0, s, d + 1));
            }
            b.block_tables = tables;
            b.table_stride = stride;
            b.is_decode = decode;
            next = model.run(b);
        };
        step(0, true);  // captures this batch size's graph
        const double g0 = now_ms();
        for (std::size_t d = 1; d <= D; ++d) step(d, true);
        const double graph_ms = (now_ms() - g0) / double(D);
        const double e0 = now_ms();
        for (std::size_t d = 1; d <= D; ++d) step(d, false);  // same steps, eager launches
        const double eager_ms = (now_ms() - e0) / double(D);
        const double total_ms = prefill_ms + graph_ms * double(D);
        std::printf("{\"workload\": \"Qwen3-0.6B shapes, random bf16 weights: %zu prompts of %zu tokens in one prefill "
                    "forward, then %zu decode steps of %zu rows at T=0.6\", \"sequences\": %zu, \"prefill_tokens\": %zu, "
                    "\"prefill_ms\": %.3f, \"decode_step_ms_graph\": %.4f, \"decode_step_ms_eager\": %.4f, "
                    "\"decode_tokens_per_s\": %.1f, \"output_tokens_per_s\": %.1f, \"graphs\": %zu}\n",
                    S, prompt, D, S, S, S * prompt, prefill_ms, graph_ms, eager_ms, double(S) / (graph_ms / 1e3),
                    double(S * (D + 1)) / (total_ms / 1e3), model.graph_count());
    } catch (const std::exception& e) {
        std::fprintf(stderr, "decode_bench: %s\n", e.what());
        return 1;
    }
    return 0;
}
