// make_cfg5_greedy.cpp -- writes the config-5 greedy fixtures
// (tests/golden/cfg5_greedy*.txt): the oracle's greedy decode of BASELINE
// config 5's synthetic Qwen3-8B (36 layers, each with its own weights,
// hidden 4096, FFN 12288, 32/8 heads, vocab 151936, Q4_K_M types; the recipe
// of csrc/bench/synth_qwen3.hpp, model seed 1): a prompt of seeded random
// ids, then greedy steps, with each step's top-2 logits.  The GPU test
// (tests/cpp/test_host_layer cfg5) builds the same model in QwenModel and
// must reproduce every token id.
//
// The oracle (oracle/citlali_oracle.c, orc_forward_token) follows
// qwen_model.cpp:239-419 with its fp16 store points, accumulating in double;
// prompt positions before the last run orc_prefill_token (no logits), as
// the session's prompt loop asks forward_token for no logits there.
//
// usage:
//   make_cfg5_greedy write PATH [PROMPT_SEED [PROMPT_LEN [STEPS]]]
//       the fixture (defaults: seed 1, 8 prompt tokens, 64 steps; BASELINE
//       config 5 itself is 512 and 256, the benchmark's prompt is seed 1)
//   make_cfg5_greedy probe GAIN STEPS [LAYERS]  sensitivity of the recipe with
//       attn_output / ffn_down gain GAIN: the oracle against itself with half
//       of the embedding values moved by one fp16 ulp, teacher-forced, per
//       step max |logit diff| and the top-2 margin, both / rms(logits)
#include "citlali_oracle.h"
#include "synth_qwen3.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

constexpr uint64_t kModelSeed = 1;
constexpr int kPrompt = 8;   // the probe's prompt

struct Model {
    const citlali::bench::Qwen3Shape& shape = citlali::bench::kConfig5;
    std::vector<citlali::bench::LayerBytes> sets;
    std::vector<uint8_t> embd, outw;
    std::vector<uint16_t> ones;
    std::vector<OrcLayer> layers;
    OrcModel m{};
    Model(double gain, int n_layers, int max_ctx) {
        const int H = shape.hidden;
        ones.assign(H, 0x3c00);   // fp16 1.0: every norm weight
        for (int l = 0; l < n_layers; ++l) sets.push_back(citlali::bench::layer_bytes(kModelSeed, l, shape, gain));
        embd = citlali::bench::embedding_bytes(kModelSeed, shape);
        outw = citlali::bench::output_bytes(kModelSeed, shape);
        for (int l = 0; l < n_layers; ++l) {
            const citlali::bench::LayerBytes& b = sets[l];
            OrcLayer o{};
            o.attn_norm = ones.data();
            o.q = {ORC_Q4K, b.q.data()};
            o.k = {ORC_Q4K, b.k.data()};
            o.v = {ORC_Q6K, b.v.data()};
            o.o = {ORC_Q4K, b.o.data()};
            o.q_norm = ones.data();
            o.k_norm = ones.data();
            o.ffn_norm = ones.data();
            o.gate = {ORC_Q4K, b.gate.data()};
            o.up = {ORC_Q4K, b.up.data()};
            o.down = {ORC_Q6K, b.down.data()};
            layers.push_back(o);
        }
        m.hidden = H;
        m.heads = shape.heads;
        m.kv_heads = shape.kv_heads;
        m.head_dim = shape.head_dim;
        m.ff = shape.ffn;
        m.n_layers = n_layers;
        m.vocab = shape.vocab;
        m.max_ctx = max_ctx;
        m.eps = 1e-6f;
        m.theta = 1e6f;
        m.token_embd = {ORC_Q6K, embd.data()};
        m.output_norm = ones.data();
        m.output = {ORC_Q6K, outw.data()};
        m.layers = layers.data();
    }
};

struct Caches {
    std::vector<std::vector<uint16_t>> c;
    std::vector<uint16_t*> p;
    Caches(const OrcModel& m) {
        for (int i = 0; i < 2 * m.n_layers; ++i) c.emplace_back((size_t)m.max_ctx * m.kv_heads * m.head_dim, 0);
        for (auto& v : c) p.push_back(v.data());
    }
};

struct Top2 {
    int32_t a, b;
    float va, vb;
    double rms;
};

Top2 top2(const std::vector<float>& lg) {
    Top2 t{0, 0, -INFINITY, -INFINITY, 0};
    double ss = 0;
    for (size_t i = 0; i < lg.size(); ++i) {
        ss += (double)lg[i] * lg[i];
        if (!std::isfinite(lg[i])) continue;
        if (lg[i] > t.va) {
            t.b = t.a;
            t.vb = t.va;
            t.a = (int32_t)i;
            t.va = lg[i];
        } else if (lg[i] > t.vb) {
            t.b = (int32_t)i;
            t.vb = lg[i];
        }
    }
    t.rms = std::sqrt(ss / lg.size());
    return t;
}

int write_fixture(const char* path, uint64_t prompt_seed, int n_prompt, int n_steps) {
    if (n_prompt < 1 || n_steps < 1) {
        std::fprintf(stderr, "prompt length and steps must be positive\n");
        return 2;
    }
    Model model(citlali::bench::kLayerOutGain, citlali::bench::kConfig5.layers, n_prompt + n_steps);
    Caches caches(model.m);
    const std::vector<int32_t> prompt = citlali::bench::prompt_ids(prompt_seed, n_prompt, model.shape.vocab);
    std::vector<float> lg(model.shape.vocab);
    std::FILE* f = std::fopen(path, "w");
    if (!f) {
        std::perror(path);
        return 1;
    }
    std::fprintf(f, "# oracle greedy decode, BASELINE config 5 synthetic Qwen3-8B (model seed %llu, "
                    "attn_output/ffn_down gain %.3g), written by tests/golden/make_cfg5_greedy\n",
                 (unsigned long long)kModelSeed, citlali::bench::kLayerOutGain);
    std::fprintf(f, "prompt_seed %llu\nprompt %d", (unsigned long long)prompt_seed, n_prompt);
    for (int32_t t : prompt) std::fprintf(f, " %d", t);
    std::fprintf(f, "\nsteps %d\n# step id logit second_id second_logit rms_logits\n", n_steps);
    int32_t tok = 0;
    double min_margin = 1e30;
    int min_step = 0;
    const auto t0 = std::chrono::steady_clock::now();
    const auto secs = [&] { return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count(); };
    for (int p = 0; p < n_prompt + n_steps - 1; ++p) {
        const int32_t in = p < n_prompt ? prompt[p] : tok;
        if (p < n_prompt - 1) {
            orc_prefill_token(&model.m, caches.p.data(), in, p);
            if ((p + 1) % 64 == 0) {
                std::printf("prompt position %d (%.0f s)\n", p, secs());
                std::fflush(stdout);
            }
            continue;
        }
        tok = orc_forward_token(&model.m, caches.p.data(), in, p, lg.data());
        const Top2 t = top2(lg);
        if (t.a != tok) {
            std::fprintf(stderr, "top-2 scan disagrees with orc_argmax at position %d\n", p);
            return 1;
        }
        const int step = p - (n_prompt - 1);   // the token this position picks is greedy step `step`
        std::fprintf(f, "%d %d %.9g %d %.9g %.9g\n", step, t.a, t.va, t.b, t.vb, t.rms);
        std::fflush(f);
        if ((t.va - t.vb) / t.rms < min_margin) {
            min_margin = (t.va - t.vb) / t.rms;
            min_step = step;
        }
        std::printf("step %3d: id %6d margin / rms %.3e (%.0f s)\n", step, t.a, (t.va - t.vb) / t.rms, secs());
        std::fflush(stdout);
    }
    std::fclose(f);
    std::printf("wrote %s: min top-2 margin / rms = %.3e (step %d)\n", path, min_margin, min_step);
    return 0;
}

int probe(double gain, int steps, int n_layers) {
    Model model(gain, n_layers, kPrompt + steps);
    Caches a(model.m), b(model.m);
    // the twin: the embedding as fp16 rows with half of the values moved by one ulp
    const int H = model.shape.hidden, V = model.shape.vocab;
    std::vector<uint16_t> e16((size_t)V * H);
    for (int t = 0; t < V; ++t) orc_embed_q6k(model.embd.data(), t, e16.data() + (size_t)t * H, H);
    citlali::bench::SplitMix flip{77};
    for (auto& h : e16)
        if ((h & 0x7fff) && (flip.next() & 1)) h ^= 1;
    OrcModel twin = model.m;
    twin.token_embd = {ORC_F16, e16.data()};
    const std::vector<int32_t> prompt = citlali::bench::prompt_ids(1, kPrompt, V);
    std::vector<float> la(V), lb(V);
    int32_t tok = 0;
    for (int p = 0; p < kPrompt + steps; ++p) {
        const int32_t in = p < kPrompt ? prompt[p] : tok;
        tok = orc_forward_token(&model.m, a.p.data(), in, p, la.data());
        const int32_t tb = orc_forward_token(&twin, b.p.data(), in, p, lb.data());
        const Top2 t = top2(la);
        double d = 0;
        for (int i = 0; i < V; ++i) d = std::max(d, std::fabs((double)la[i] - lb[i]));
        std::printf("gain %.3g layers %d pos %2d: rms %.3f  max|diff|/rms %.3e  top-2 margin/rms %.3e  %s\n", gain,
                    n_layers, p, t.rms, d / t.rms, (t.va - t.vb) / t.rms, tok == tb ? "same pick" : "PICK DIFFERS");
        std::fflush(stdout);
    }
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "";
    if (mode == "write" && argc >= 3)
        return write_fixture(argv[2], argc > 3 ? std::strtoull(argv[3], nullptr, 10) : 1,
                             argc > 4 ? std::atoi(argv[4]) : 8, argc > 5 ? std::atoi(argv[5]) : 64);
    if (mode == "probe" && argc >= 4)
        return probe(std::atof(argv[2]), std::atoi(argv[3]), argc > 4 ? std::atoi(argv[4]) : citlali::bench::kConfig5.layers);
    std::fprintf(stderr, "usage: %s write PATH [PROMPT_SEED [PROMPT_LEN [STEPS]]] | probe GAIN STEPS [LAYERS]\n", argv[0]);
    return 2;
}
