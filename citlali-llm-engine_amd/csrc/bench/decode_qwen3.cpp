// decode_qwen3.cpp -- synthetic Qwen3 greedy decode through QwenModel.
//
// BASELINE config 5 by default: Qwen3-8B shapes (36 layers, hidden 4096,
// FFN 12288, 32/8 heads, head_dim 128, vocab 151936, rope_theta 1e6,
// rms_eps 1e-6), Q4_K for most matrices, Q6_K for attn_v, ffn_down, the
// output and the token embedding; a prompt of 512 random token ids fed as
// the reference's session does (session.cpp:71-74: one forward_token per
// prompt token, logits only for the last), then 256 greedy steps
// (session.cpp:92).  Weights are the random quant blocks of
// synth_qwen3.hpp (d keeps every matrix at rms ~ gain/sqrt(in)); every layer
// has its own weights (36 distinct sets for Qwen3-8B, ~4.4 GB of layer
// weights read from HBM per token); `--distinct N` reuses N byte sets
// cyclically instead (each layer still gets its own device copy when loaded
// from handles; a GGUF file then stores each set once).  The greedy steps
// run twice: as the reference's loop of
// forward_token calls, then through QwenModel::decode_greedy (each step
// replayed from a captured HIP graph); both must give the same tokens.
// With `--gguf PATH` the same weights are first written to a GGUF file at
// PATH (layers of one byte set share their data in the file; the norms are
// F32 ones) and the model is loaded from it by QwenModel::load(GgufFile)
// with KeepQuantized, the reference's load path (qwen_model.cpp:45-186); the
// file is removed after loading and the load time is reported.  `--fp16`
// (with --gguf) loads it with DequantizeToFp16 instead, the reference's
// default policy: every matrix becomes fp16 in device memory and the fp16
// GEMVs run.
// `--model` picks another Qwen3 size's shapes (layers, hidden, FFN, query /
// kv heads; head_dim 128, the same vocab and quant types): 0.6b (28, 1024,
// 3072, 16/8), 1.7b (28, 2048, 6144, 16/8), 4b (36, 2560, 9728, 32/8), 8b
// (the default), 14b (40, 5120, 17408, 40/8), 32b (64, 5120, 25600, 64/8).
// Prints one JSON line.
//
// usage: decode_qwen3 [--model 0.6b|1.7b|4b|8b|14b|32b] [--layers N] [--prompt 512] [--steps 256]
//                     [--distinct N] [--seed 1] [--no-graph] [--gguf PATH [--fp16]]
#include "citlali/common.h"
#include "citlali/compute/hip/kernels.h"
#include "citlali/io/gguf_reader.h"
#include "citlali/model/qwen_model.h"
#include "citlali_hip.h"
#include "gguf_out.hpp"
#include "synth_qwen3.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

using namespace citlali;
using compute::GgufTensorType;

namespace {

model::WeightHandle quant_handle(const std::vector<uint8_t>& bytes, GgufTensorType t, int rows, int cols,
                                 const std::string& name) {
    model::WeightHandle w;
    w.name = name;
    w.gguf_type = t;
    w.storage_kind = compute::WeightStorageKind::QuantizedDevice;
    w.dims = {(uint64_t)cols, (uint64_t)rows};
    w.element_count = (uint64_t)rows * cols;
    w.buffer = compute::make_device_buffer(bytes.size());
    w.buffer->copy_from_host(bytes.data(), bytes.size());
    return w;
}

model::WeightHandle norm_handle(int n, const std::string& name) {
    std::vector<uint16_t> v(n, compute::float_to_half_bits(1.0f));
    model::WeightHandle w;
    w.name = name;
    w.gguf_type = GgufTensorType::F16;
    w.storage_kind = compute::WeightStorageKind::Fp16Device;
    w.dims = {(uint64_t)n, 1};
    w.element_count = n;
    w.buffer = compute::make_device_half_buffer(n);
    w.buffer->copy_from_host(v.data(), v.size() * 2);
    return w;
}

const char* str_arg(int argc, char** argv, const char* key) {
    for (int i = 1; i + 1 < argc; ++i)
        if (std::strcmp(argv[i], key) == 0) return argv[i + 1];
    return nullptr;
}

int arg(int argc, char** argv, const char* key, int def) {
    for (int i = 1; i + 1 < argc; ++i)
        if (std::strcmp(argv[i], key) == 0) return std::atoi(argv[i + 1]);
    return def;
}

}  // namespace

int main(int argc, char** argv) {
    const char* model_arg = str_arg(argc, argv, "--model");
    const bench::Qwen3Shape* shape = &bench::kConfig5;
    if (model_arg != nullptr) {
        shape = nullptr;
        for (const bench::Qwen3Shape& m : bench::kQwen3Shapes)
            if (std::strcmp(model_arg, m.name) == 0) shape = &m;
        if (shape == nullptr) {
            std::fprintf(stderr, "decode_qwen3: --model is one of 0.6b 1.7b 4b 8b 14b 32b\n");
            return 2;
        }
    }
    const int layers = arg(argc, argv, "--layers", shape->layers);
    const int prompt = arg(argc, argv, "--prompt", 512);
    const int steps = arg(argc, argv, "--steps", 256);
    const int distinct = std::max(1, std::min(layers, arg(argc, argv, "--distinct", layers)));
    const uint64_t seed = (uint64_t)arg(argc, argv, "--seed", 1);
    bool graph_pass = true;   // --no-graph: forward_token loop only (for tracing tools)
    bool fp16_weights = false;
    for (int i = 1; i < argc; ++i) {
        if (std::strcmp(argv[i], "--no-graph") == 0) graph_pass = false;
        if (std::strcmp(argv[i], "--fp16") == 0) fp16_weights = true;
    }
    try {
        if (citlali_hip_init(0) != CITLALI_OK) throw Error(citlali_hip_last_error());
        model::QwenConfig cfg;
        cfg.architecture = "qwen3";
        cfg.vocab_size = 151936;
        cfg.context_length = 40960;
        const int H = shape->hidden, F = shape->ffn, HEADS = shape->heads, KVH = 8;
        const int NQ = HEADS * 128, NKV = KVH * 128, V = 151936;
        cfg.embedding_length = (uint32_t)H;
        cfg.block_count = layers;
        cfg.feed_forward_length = (uint32_t)F;
        cfg.head_count = (uint32_t)HEADS;
        cfg.head_count_kv = (uint32_t)KVH;
        cfg.head_dim = 128;
        cfg.rms_norm_eps = 1e-6f;
        cfg.rope_theta = 1e6f;

        const auto t0 = std::chrono::steady_clock::now();
        using bench::LayerBytes;
        std::vector<LayerBytes> sets;
        for (int i = 0; i < distinct; ++i) sets.push_back(bench::layer_bytes(seed, i, *shape));
        const std::vector<uint8_t> embd = bench::embedding_bytes(seed, *shape);
        const std::vector<uint8_t> outw = bench::output_bytes(seed, *shape);
        const int ctx = prompt + steps;
        model::QwenModel m;
        const char* gguf_path = str_arg(argc, argv, "--gguf");
        double gguf_write_s = 0, load_s = 0, file_bytes = 0, loaded_bytes = 0;
        if (gguf_path != nullptr) {
            // the weights as a GGUF file, then the reference's load path
            bench::GgufOut o;
            o.str("general.architecture", "qwen3");
            o.strings("tokenizer.ggml.tokens", V);
            o.u32("qwen3.context_length", cfg.context_length);
            o.u32("qwen3.embedding_length", H);
            o.u32("qwen3.block_count", (uint32_t)layers);
            o.u32("qwen3.feed_forward_length", F);
            o.u32("qwen3.attention.head_count", (uint32_t)HEADS);
            o.u32("qwen3.attention.head_count_kv", (uint32_t)KVH);
            o.u32("qwen3.attention.key_length", 128);
            o.u32("qwen3.attention.value_length", 128);
            o.f32("qwen3.attention.layer_norm_rms_epsilon", cfg.rms_norm_eps);
            o.f32("qwen3.rope.freq_base", cfg.rope_theta);
            const std::vector<float> ones(H, 1.0f);
            const auto Q4 = GgufTensorType::Q4_K, Q6 = GgufTensorType::Q6_K, F32T = GgufTensorType::F32;
            const uint64_t h = (uint64_t)H, f = (uint64_t)F, nq = (uint64_t)NQ, nkv = (uint64_t)NKV;
            o.tensor("token_embd.weight", {h, (uint64_t)V}, Q6, embd.data(), embd.size());
            o.tensor("output_norm.weight", {h}, F32T, ones.data(), (size_t)H * 4);
            o.tensor("output.weight", {h, (uint64_t)V}, Q6, outw.data(), outw.size());
            std::vector<size_t> first(distinct * 7);
            for (int l = 0; l < layers; ++l) {
                const LayerBytes& b = sets[l % distinct];
                const std::string n = "blk." + std::to_string(l) + ".";
                o.tensor(n + "attn_norm.weight", {h}, F32T, ones.data(), (size_t)H * 4);
                o.tensor(n + "attn_q_norm.weight", {128}, F32T, ones.data(), 128 * 4);
                o.tensor(n + "attn_k_norm.weight", {128}, F32T, ones.data(), 128 * 4);
                o.tensor(n + "ffn_norm.weight", {h}, F32T, ones.data(), (size_t)H * 4);
                const struct {
                    const char* name;
                    const std::vector<uint8_t>* bytes;
                    GgufTensorType t;
                    uint64_t in, out;
                } mats[7] = {{"attn_q.weight", &b.q, Q4, h, nq},       {"attn_k.weight", &b.k, Q4, h, nkv},
                             {"attn_v.weight", &b.v, Q6, h, nkv},      {"attn_output.weight", &b.o, Q4, nq, h},
                             {"ffn_gate.weight", &b.gate, Q4, h, f},   {"ffn_up.weight", &b.up, Q4, h, f},
                             {"ffn_down.weight", &b.down, Q6, f, h}};
                for (int j = 0; j < 7; ++j) {
                    size_t& slot = first[(l % distinct) * 7 + j];
                    if (l < distinct) {
                        slot = o.tensor(n + mats[j].name, {mats[j].in, mats[j].out}, mats[j].t, mats[j].bytes->data(),
                                        mats[j].bytes->size());
                    } else {
                        o.alias(n + mats[j].name, {mats[j].in, mats[j].out}, mats[j].t, slot);
                    }
                }
            }
            const auto w0 = std::chrono::steady_clock::now();
            file_bytes = (double)o.write(gguf_path);
            const auto w1 = std::chrono::steady_clock::now();
            gguf_write_s = std::chrono::duration<double>(w1 - w0).count();
            io::GgufFile g;
            g.load(gguf_path);
            m.load(g, (uint32_t)ctx, /*quantized=*/!fp16_weights);
            m.synchronize();
            load_s = std::chrono::duration<double>(std::chrono::steady_clock::now() - w1).count();
            for (const auto& t : g.tensors()) loaded_bytes += (double)t.nbytes;
            std::remove(gguf_path);
        } else {
            model::QwenWeights w;
            w.token_embedding = quant_handle(embd, GgufTensorType::Q6_K, V, H, "token_embd.weight");
            w.output_norm = norm_handle(H, "output_norm.weight");
            w.output_weight = quant_handle(outw, GgufTensorType::Q6_K, V, H, "output.weight");
            for (int l = 0; l < layers; ++l) {
                const LayerBytes& b = sets[l % distinct];
                const std::string n = "blk." + std::to_string(l) + ".";
                model::QwenLayerWeights L;
                L.attn_norm = norm_handle(H, n + "attn_norm.weight");
                L.attn_q = quant_handle(b.q, GgufTensorType::Q4_K, NQ, H, n + "attn_q.weight");
                L.attn_k = quant_handle(b.k, GgufTensorType::Q4_K, NKV, H, n + "attn_k.weight");
                L.attn_v = quant_handle(b.v, GgufTensorType::Q6_K, NKV, H, n + "attn_v.weight");
                L.attn_o = quant_handle(b.o, GgufTensorType::Q4_K, H, NQ, n + "attn_output.weight");
                L.attn_q_norm = norm_handle(128, n + "attn_q_norm.weight");
                L.attn_k_norm = norm_handle(128, n + "attn_k_norm.weight");
                L.ffn_norm = norm_handle(H, n + "ffn_norm.weight");
                L.ffn_gate = quant_handle(b.gate, GgufTensorType::Q4_K, F, H, n + "ffn_gate.weight");
                L.ffn_up = quant_handle(b.up, GgufTensorType::Q4_K, F, H, n + "ffn_up.weight");
                L.ffn_down = quant_handle(b.down, GgufTensorType::Q6_K, H, F, n + "ffn_down.weight");
                w.layers.push_back(std::move(L));
            }
            m.load(cfg, std::move(w), (uint32_t)ctx);
            m.synchronize();
        }
        sets.clear();
        const double setup_s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();

        // prompt, one token at a time (logits only for the last one)
        const std::vector<int32_t> ids = bench::prompt_ids(seed, prompt, V);
        void *e0 = nullptr, *e1 = nullptr, *e2 = nullptr;
        citlali_hip_event_create(&e0);
        citlali_hip_event_create(&e1);
        citlali_hip_event_create(&e2);
        uint32_t pos = 0;
        int32_t next = 0;
        const auto p0 = std::chrono::steady_clock::now();
        citlali_hip_event_record(e0);
        for (int i = 0; i < prompt; ++i) next = m.forward_token(ids[i], pos++, i == prompt - 1);
        citlali_hip_event_record(e1);
        const auto p1 = std::chrono::steady_clock::now();
        // greedy decode, one forward_token per step (the reference's loop)
        const int32_t first = next;
        const uint32_t first_pos = pos;
        std::vector<int32_t> eager;
        for (int i = 0; i < steps; ++i) {
            next = m.forward_token(next, pos++);
            eager.push_back(next);
        }
        citlali_hip_event_record(e2);
        citlali_hip_event_synchronize(e2);
        const auto p2 = std::chrono::steady_clock::now();
        float prompt_ms = 0, eager_ms = 0;
        citlali_hip_event_elapsed_ms(e0, e1, &prompt_ms);
        citlali_hip_event_elapsed_ms(e1, e2, &eager_ms);
        const double eager_wall = std::chrono::duration<double>(p2 - p1).count();
        const double prompt_wall = std::chrono::duration<double>(p1 - p0).count();
        // the same steps again through decode_greedy (each step replayed from
        // a captured graph, no host synchronisation between steps): the first
        // call captures the graphs, the second is timed, wall clock around
        // the whole call including the copy of the tokens
        std::vector<int32_t> warm = eager, graph = eager;
        double graph_wall = eager_wall;
        if (graph_pass) {
            warm = m.decode_greedy(first, first_pos, (uint32_t)steps);
            const auto g0 = std::chrono::steady_clock::now();
            graph = m.decode_greedy(first, first_pos, (uint32_t)steps);
            const auto g1 = std::chrono::steady_clock::now();
            graph_wall = std::chrono::duration<double>(g1 - g0).count();
        }
        const bool match = graph == eager && warm == eager;
        uint64_t checksum = 0;
        for (int32_t t : graph) checksum = checksum * 1000003ull + (uint64_t)t;
        const double decode_ms = graph_wall * 1e3;
        // bytes one decode step must read: every weight once, the KV cache
        // up to the position, the embedding row and the logits
        // (fp16 weights: every matrix as 2-byte values)
        // (K-quants: 144 / 210 bytes per 256 values; fp16 weights 2 bytes each)
        const auto q4 = [](double rows, double cols) { return rows * cols / 256 * 144; };
        const auto q6 = [](double rows, double cols) { return rows * cols / 256 * 210; };
        const double layer_bytes = fp16_weights ? 2.0 * ((double)NQ * H * 2 + (double)NKV * H * 2 + 3.0 * F * H)
                                                : q4(NQ, H) * 2 + q4(NKV, H) + q6(NKV, H) + q4(F, H) * 2 + q6(H, F);
        const double mean_len = prompt + (steps + 1) / 2.0;
        const double out_bytes = fp16_weights ? 2.0 * V * H : q6(V, H);
        const double step_bytes = layer_bytes * layers + out_bytes + q6(1, H) + V * 4.0 +
                                  (double)layers * 2 * 2 * NKV * mean_len;
        std::printf("{\"workload\": \"%s\", \"layers\": %d, "
                    "\"distinct_layer_weight_sets\": %d, \"prompt\": %d, \"steps\": %d, \"decode_tok_per_s\": %.2f, "
                    "\"decode_ms_per_token\": %.4f, \"decode_mode\": \"%s\", "
                    "\"decode_GBps\": %.1f, \"decode_tok_per_s_forward_token\": %.2f, "
                    "\"decode_ms_per_token_forward_token\": %.4f, \"decode_ms_per_token_forward_token_wall\": %.4f, "
                    "\"graph_tokens_equal_forward_token\": %s, \"prompt_tok_per_s\": %.2f, "
                    "\"prompt_ms_per_token_wall\": %.4f, \"setup_s\": %.1f, \"token_checksum\": %llu, "
                    "\"weights_from\": \"%s\", \"gguf_file_bytes\": %.0f, \"gguf_write_s\": %.2f, "
                    "\"gguf_load_s\": %.3f, \"gguf_load_GBps\": %.2f}\n",
                    shape->workload,
                    layers, distinct, prompt, steps, steps / (decode_ms * 1e-3), decode_ms / steps,
                    graph_pass ? "QwenModel::decode_greedy (graph replay), wall clock"
                               : "forward_token loop, wall clock (--no-graph)",
                    step_bytes / (decode_ms * 1e-3 / steps) / 1e9, steps / (eager_ms * 1e-3), eager_ms / steps,
                    eager_wall * 1e3 / steps, match ? "true" : "false", prompt / (prompt_ms * 1e-3),
                    prompt_wall * 1e3 / prompt, setup_s, (unsigned long long)checksum,
                    gguf_path ? (fp16_weights ? "GGUF file, QwenModel::load(GgufFile) DequantizeToFp16"
                                              : "GGUF file, QwenModel::load(GgufFile) KeepQuantized")
                              : "WeightHandles",
                    file_bytes, gguf_write_s, load_s, load_s > 0 ? loaded_bytes / load_s / 1e9 : 0.0);
        if (!match) {
            std::fprintf(stderr, "decode_qwen3: decode_greedy tokens differ from the forward_token loop\n");
            return 1;
        }
        citlali_hip_event_destroy(e0);
        citlali_hip_event_destroy(e1);
        citlali_hip_event_destroy(e2);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "decode_qwen3: %s\n", e.what());
        return 1;
    }
    return 0;
}
