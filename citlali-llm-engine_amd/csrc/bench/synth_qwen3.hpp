// synth_qwen3.hpp -- the synthetic Qwen3 models of the decode benchmark
// (BASELINE config 5 and the other Qwen3 sizes), shared by
// bin/decode_qwen3, the greedy-parity fixture generator and its GPU test so
// that all three build the same bytes.
//
// Shapes follow the Qwen3 family (head_dim 128, 8 kv heads, vocab 151936,
// rope_theta 1e6, rms_eps 1e-6).  Quant types are Q4_K_M's: Q4_K for
// attn_q / attn_k / attn_output / ffn_gate / ffn_up, Q6_K for attn_v,
// ffn_down, the output and the token embedding.  Every block's bytes are
// splitmix64 output (random 4- / 6-bit codes and scale codes); the fp16
// scale d (and Q4_K's dmin, equal to d) is one value per matrix chosen so
// the matrix has rms(w) ~ gain / sqrt(in_features): random Q4_K codes give
// rms ~ 300 d, random Q6_K codes ~ 1366 d.  Norm weights are 1.0.
//
// Gains: q/k/v 1.0, gate/up 1.0, attn_output and ffn_down kLayerOutGain,
// the embedding sqrt(hidden) (rows of rms ~1) and the output 3.0.  With
// these the Qwen3-8B model does not amplify rounding differences through its
// 36 layers: moving half of the embedding values by one fp16 ulp moves the
// logits by 3-4e-3 of their rms (the oracle against itself,
// tests/golden/make_cfg5_greedy probe), about what the embedding change
// alone gives, so greedy tokens are decided by the arithmetic and not by
// one implementation's summation order (a layer gain of 0.1 measured
// 6-8e-3 and smaller top-2 margins).
#pragma once

#include "citlali/compute/common/dtype.h"

#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

namespace citlali::bench {

constexpr double kLayerOutGain = 0.5;

struct SplitMix {
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
};

// Raw GGUF blocks of a rows x cols matrix of type t (Q4_K or Q6_K).
inline std::vector<uint8_t> quant_bytes(uint64_t seed, citlali::compute::GgufTensorType t, int rows, int cols,
                                        double gain) {
    using citlali::compute::GgufTensorType;
    const size_t bb = citlali::compute::gguf_type_block_bytes(t);
    const size_t blocks = (size_t)rows * cols / 256;
    std::vector<uint8_t> b(blocks * bb);
    SplitMix r{seed};
    for (size_t i = 0; i + 8 <= b.size(); i += 8) {
        const uint64_t v = r.next();
        std::memcpy(b.data() + i, &v, 8);
    }
    const double d = gain / std::sqrt((double)cols) / (t == GgufTensorType::Q4_K ? 300.0 : 1366.0);
    const uint16_t dh = citlali::compute::float_to_half_bits((float)d);
    for (size_t i = 0; i < blocks; ++i) {
        uint8_t* p = b.data() + i * bb;
        if (t == GgufTensorType::Q4_K) {
            std::memcpy(p, &dh, 2);
            std::memcpy(p + 2, &dh, 2);
        } else {
            std::memcpy(p + 208, &dh, 2);
        }
    }
    return b;
}

struct Qwen3Shape {
    const char* name;
    int layers, hidden, ffn, heads;
    const char* workload;
    static constexpr int kv_heads = 8, head_dim = 128, vocab = 151936;
};

constexpr Qwen3Shape kQwen3Shapes[] = {
    {"0.6b", 28, 1024, 3072, 16, "Qwen3-0.6B shapes, synthetic Q4_K_M greedy decode"},
    {"1.7b", 28, 2048, 6144, 16, "Qwen3-1.7B shapes, synthetic Q4_K_M greedy decode"},
    {"4b", 36, 2560, 9728, 32, "Qwen3-4B shapes, synthetic Q4_K_M greedy decode"},
    {"8b", 36, 4096, 12288, 32, "BASELINE config 5: Qwen3-8B synthetic Q4_K_M greedy decode"},
    {"14b", 40, 5120, 17408, 40, "Qwen3-14B shapes, synthetic Q4_K_M greedy decode"},
    {"32b", 64, 5120, 25600, 64, "Qwen3-32B shapes, synthetic Q4_K_M greedy decode"},
};
constexpr const Qwen3Shape& kConfig5 = kQwen3Shapes[3];

// One layer's seven matrices; byte set i of model seed s.
struct LayerBytes {
    std::vector<uint8_t> q, k, v, o, gate, up, down;
};

inline LayerBytes layer_bytes(uint64_t seed, int set, const Qwen3Shape& m, double out_gain = kLayerOutGain) {
    using citlali::compute::GgufTensorType;
    const int H = m.hidden, F = m.ffn, NQ = m.heads * m.head_dim, NKV = m.kv_heads * m.head_dim;
    const uint64_t s = seed * 1000 + (uint64_t)set * 10;
    LayerBytes b;
    b.q = quant_bytes(s + 1, GgufTensorType::Q4_K, NQ, H, 1.0);
    b.k = quant_bytes(s + 2, GgufTensorType::Q4_K, NKV, H, 1.0);
    b.v = quant_bytes(s + 3, GgufTensorType::Q6_K, NKV, H, 1.0);
    b.o = quant_bytes(s + 4, GgufTensorType::Q4_K, H, NQ, out_gain);
    b.gate = quant_bytes(s + 5, GgufTensorType::Q4_K, F, H, 1.0);
    b.up = quant_bytes(s + 6, GgufTensorType::Q4_K, F, H, 1.0);
    b.down = quant_bytes(s + 7, GgufTensorType::Q6_K, H, F, out_gain);
    return b;
}

inline std::vector<uint8_t> embedding_bytes(uint64_t seed, const Qwen3Shape& m) {
    return quant_bytes(seed * 7 + 11, citlali::compute::GgufTensorType::Q6_K, m.vocab, m.hidden,
                       std::sqrt((double)m.hidden));
}

inline std::vector<uint8_t> output_bytes(uint64_t seed, const Qwen3Shape& m) {
    return quant_bytes(seed * 7 + 13, citlali::compute::GgufTensorType::Q6_K, m.vocab, m.hidden, 3.0);
}

// `n` prompt token ids of model seed s.
inline std::vector<int32_t> prompt_ids(uint64_t seed, int n, int vocab) {
    SplitMix r{seed * 31 + 7};
    std::vector<int32_t> ids(n);
    for (auto& t : ids) t = (int32_t)(r.next() % (uint64_t)vocab);
    return ids;
}

}  // namespace citlali::bench
