// test_host_layer.cpp -- tests of the C++ host API (libcitlali.so) against
// the CPU oracle (liboracle.so, test infrastructure).
//
//   test_host_layer cpu   dtype tables, host fp16 rules (exhaustive), the
//                         LinearBackend dispatch and its errors; no GPU.
//   test_host_layer gpu   DeviceBuffer, LinearBackend::forward (Q4_K, Q6_K,
//                         fp16), launch_attention, launch_embed_q6k on the
//                         GPU, compared with the oracle.
//   test_host_layer greedy / greedy2   QwenModel greedy decode against the
//                         oracle's forward (two halves of the model forms).
//   test_host_layer graph  decode_greedy (graph replay) = the forward_token
//                         loop.
//   test_host_layer gguf  QwenModel loaded from a GGUF file of the model.
//   test_host_layer cfg5 FIXTURE   BASELINE config 5's full Qwen3-8B shape:
//                         the fixture's greedy tokens equal the oracle's.
// Prints one line per check and exits non-zero on the first failure.
#include "citlali/common.h"
#include "citlali/compute/common/dtype.h"
#include "citlali/compute/hip/kernels.h"
#include "citlali/compute/hip/tensor.h"
#include "citlali/io/gguf_reader.h"
#include "citlali/model/linear_backend.h"
#include "citlali/model/qwen_model.h"
#include "citlali/runtime/session.h"
#include "citlali/tokenizer/tokenizer.h"
#include "citlali_hip.h"
#include "citlali_oracle.h"
#include "gguf_out.hpp"
#include "synth_qwen3.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include <unistd.h>

using namespace citlali;
using compute::GgufTensorType;
using compute::WeightStorageKind;

namespace {

int g_checks = 0;

void check(bool ok, const std::string& what) {
    ++g_checks;
    if (!ok) {
        std::printf("FAIL: %s\n", what.c_str());
        std::fflush(stdout);
        std::exit(1);
    }
}

// Runs f, expects citlali::Error whose message contains `needle`.
void expect_error(const std::function<void()>& f, const std::string& needle, const std::string& what) {
    try {
        f();
    } catch (const Error& e) {
        check(std::string(e.what()).find(needle) != std::string::npos,
              what + ": message '" + e.what() + "' lacks '" + needle + "'");
        return;
    }
    check(false, what + ": no citlali::Error thrown");
}

struct Rng {   // splitmix64
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    double uniform() { return (next() >> 11) * (1.0 / 9007199254740992.0); }
    double normal() {
        const double u1 = 1.0 - uniform(), u2 = uniform();
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    }
};

std::vector<uint16_t> normal_f16(Rng& r, size_t n) {
    std::vector<uint16_t> v(n);
    for (auto& h : v) h = orc_f2h_rne((float)r.normal());
    return v;
}

// Random quant bytes; d (and dmin) = fp16 of U[d_lo, d_hi].
std::vector<uint8_t> quant_blocks(Rng& r, GgufTensorType t, size_t blocks, double d_lo = 1e-3, double d_hi = 1e-2) {
    const size_t bb = compute::gguf_type_block_bytes(t);
    std::vector<uint8_t> b(blocks * bb);
    for (auto& x : b) x = (uint8_t)r.next();
    for (size_t i = 0; i < blocks; ++i) {
        uint8_t* p = b.data() + i * bb;
        auto put = [&](size_t off) {
            const uint16_t h = orc_f2h_rne((float)(d_lo + (d_hi - d_lo) * r.uniform()));
            std::memcpy(p + off, &h, 2);
        };
        if (t == GgufTensorType::Q4_K) {
            put(0);
            put(2);
        } else {
            put(208);
        }
    }
    return b;
}

bool close(double got, double ref) { return std::fabs(got - ref) <= 2e-3 + 1e-2 * std::fabs(ref); }

// ------------------------------------------------------------------ CPU
void test_dtype() {
    check(compute::to_string(GgufTensorType::Q4_K) == "Q4_K", "to_string Q4_K");
    check(compute::to_string(GgufTensorType::BF16) == "BF16", "to_string BF16");
    check(compute::to_string(static_cast<GgufTensorType>(99)) == "Unknown", "to_string unknown code");
    check(compute::gguf_type_block_size(GgufTensorType::Q6_K) == 256 &&
              compute::gguf_type_block_bytes(GgufTensorType::Q6_K) == 210,
          "Q6_K geometry");
    check(compute::gguf_type_block_bytes(GgufTensorType::Q4_K) == 144, "Q4_K bytes");
    check(compute::gguf_type_block_bytes(GgufTensorType::Q8_0) == 34, "Q8_0 bytes");
    check(compute::gguf_type_block_size(GgufTensorType::Q5_K) == 0, "Q5_K not storable");
    check(compute::gguf_tensor_nbytes(GgufTensorType::Q4_K, 4096ull * 4096) == 9437184, "attn_q bytes");
    check(compute::gguf_tensor_nbytes(GgufTensorType::Q6_K, 12288ull * 4096) == 41287680, "ffn_down bytes");
    check(compute::gguf_tensor_nbytes(GgufTensorType::Q4_K, 257) == 288, "partial block rounds up");
    check(compute::gguf_tensor_nbytes(GgufTensorType::F16, 3) == 6, "F16 bytes");
    check(compute::gguf_tensor_nbytes(GgufTensorType::Q2_K, 256) == 0, "unknown type has no size");
    std::printf("dtype tables ok\n");
}

void test_fp16_rules() {
    // every float: the product rule equals the oracle's (pinned against the
    // compiled reference over the same 2^32 inputs)
    long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long hi = 0; hi < 65536; ++hi) {
        for (uint32_t lo = 0; lo < 65536; ++lo) {
            const uint32_t u = (uint32_t)hi << 16 | lo;
            float f;
            std::memcpy(&f, &u, 4);
            bad += compute::float_to_half_bits(f) != orc_f2h(f);
        }
    }
    check(bad == 0, "float_to_half_bits over all 2^32 floats (" + std::to_string(bad) + " differ)");
    for (uint32_t h = 0; h < 65536; ++h) {
        const float a = compute::half_bits_to_float((uint16_t)h), b = orc_h2f((uint16_t)h);
        check(std::memcmp(&a, &b, 4) == 0, "half_bits_to_float " + std::to_string(h));
        const uint32_t u = h << 16;
        float bf;
        std::memcpy(&bf, &u, 4);
        check(compute::bfloat16_to_half_bits((uint16_t)h) == orc_f2h(bf), "bfloat16_to_half_bits " + std::to_string(h));
    }
    check(compute::float_to_half_bits(1.0f + std::ldexp(1.0f, -11)) == 0x3C01, "tie rounds away from zero");
    check(compute::float_to_half_bits(NAN) == 0x7C00, "NaN -> Inf");
    std::printf("fp16 rules ok (all 2^32 floats, all 2^16 halves)\n");
}

void test_dispatch_errors() {
    auto backend = model::make_fp16_linear_backend();
    auto empty = std::make_shared<compute::DeviceBuffer>();
    model::WeightHandle w;
    w.name = "blk.0.attn_q.weight";
    w.gguf_type = GgufTensorType::Q4_K;
    w.storage_kind = WeightStorageKind::QuantizedDevice;
    w.dims = {4096, 4096};
    w.buffer = empty;
    expect_error([&] { backend->forward(w, nullptr, empty); }, "linear backend received a null buffer",
                 "null input");
    w.gguf_type = GgufTensorType::Q8_0;
    expect_error([&] { backend->forward(w, empty, empty); }, "unsupported weight storage kind for: blk.0.attn_q.weight",
                 "quantised Q8_0");
    w.gguf_type = GgufTensorType::Q4_K;
    w.dims = {4096, 1ull << 32};
    expect_error([&] { backend->forward(w, empty, empty); }, "blk.0.attn_q.weight rows is too large", "rows > INT_MAX");
    w.dims = {4096, 4096};
    expect_error([&] { backend->forward(w, empty, empty); }, "weight buffer holds 0 bytes, 9437184 needed",
                 "empty weight buffer");
    w.storage_kind = static_cast<WeightStorageKind>(7);
    expect_error([&] { backend->forward(w, empty, empty); }, "unknown storage_kind", "bad storage kind");
    // launchers validate before touching the GPU
    expect_error([] { compute::launch_matvec_q4k(nullptr, nullptr, nullptr, 4096, 4096); }, "null buffer",
                 "launch_matvec_q4k null");
    expect_error([] { compute::launch_attention(nullptr, nullptr, nullptr, nullptr, nullptr, 0, 1, 32, 8, 128); },
                 "null buffer", "launch_attention null");
    // move-only buffer semantics without allocation
    compute::DeviceBuffer a;
    compute::DeviceBuffer b(std::move(a));
    check(b.data() == nullptr && b.bytes() == 0, "empty move");
    expect_error([&] { b.copy_from_host("x", 1); }, "1 bytes into a buffer of 0", "copy past the end");
    std::printf("dispatch errors ok\n");
}

// ------------------------------------------------------------------ GPU
template <class T>
compute::DeviceBufferPtr upload(const std::vector<T>& v) {
    auto b = compute::make_device_buffer(v.size() * sizeof(T));
    b->copy_from_host(v.data(), v.size() * sizeof(T));
    return b;
}

std::vector<uint16_t> download_half(const compute::DeviceBufferPtr& b, size_t n) {
    std::vector<uint16_t> v(n);
    b->copy_to_host(v.data(), n * 2);
    return v;
}

void test_buffers() {
    std::vector<uint16_t> h(1000);
    for (size_t i = 0; i < h.size(); ++i) h[i] = (uint16_t)(i * 37);
    auto b = upload(h);
    compute::DeviceBuffer moved(std::move(*b));
    check(b->data() == nullptr && moved.bytes() == 2000, "move transfers ownership");
    std::vector<uint16_t> back(1000);
    moved.copy_to_host(back.data(), 2000);
    check(back == h, "host -> device -> host round trip");
    expect_error([&] { moved.copy_to_host(back.data(), 2002); }, "2002 bytes from a buffer of 2000", "read past end");
    // cuda_zero under its reference name (kernels.h:8): bytes [6, 1006)
    compute::cuda_zero(static_cast<uint8_t*>(moved.data()) + 6, 1000);
    moved.copy_to_host(back.data(), 2000);
    bool zeroed = true;
    for (size_t i = 0; i < h.size(); ++i) zeroed = zeroed && back[i] == ((i >= 3 && i < 503) ? 0 : h[i]);
    check(zeroed, "cuda_zero clears exactly its range");
    moved.allocate(0);
    check(moved.data() == nullptr, "allocate(0) empties");
    std::printf("device buffers ok\n");
}

void test_linear(GgufTensorType t, WeightStorageKind kind, int in_f, int out_f, uint64_t seed) {
    Rng r{seed};
    const size_t nb = (size_t)in_f / 256;
    model::WeightHandle w;
    w.name = "blk.3.test." + compute::to_string(t);
    w.gguf_type = t;
    w.storage_kind = kind;
    w.dims = {(uint64_t)in_f, (uint64_t)out_f};
    w.element_count = (uint64_t)in_f * out_f;
    const std::vector<uint16_t> x = normal_f16(r, in_f);
    std::vector<double> ref(out_f);
    if (kind == WeightStorageKind::QuantizedDevice) {
        const std::vector<uint8_t> q = quant_blocks(r, t, nb * out_f);
        w.buffer = upload(q);
        if (t == GgufTensorType::Q4_K)
            orc_matvec_q4k(q.data(), x.data(), ref.data(), in_f, out_f, 0);
        else
            orc_matvec_q6k(q.data(), x.data(), ref.data(), in_f, out_f, 0);
    } else {
        std::vector<uint16_t> wf(w.element_count);
        for (auto& v : wf) v = orc_f2h_rne((float)(r.normal() / std::sqrt((double)in_f)));
        w.buffer = upload(wf);
        for (int o = 0; o < out_f; ++o) {
            double acc = 0;
            for (int i = 0; i < in_f; ++i) acc += (double)orc_h2f(wf[(size_t)o * in_f + i]) * orc_h2f(x[i]);
            ref[o] = acc;
        }
    }
    auto xb = upload(x);
    auto yb = compute::make_device_half_buffer(out_f);
    auto backend = model::make_fp16_linear_backend();
    backend->forward(w, xb, yb);
    const std::vector<uint16_t> y = download_half(yb, out_f);
    // same bits as the C ABI called directly
    auto yd = compute::make_device_half_buffer(out_f);
    if (kind == WeightStorageKind::Fp16Device)
        check(citlali_hip_matvec_fp16(w.device_half_data(), xb->half_data(), yd->half_data(), in_f, out_f) == 0, "abi");
    else if (t == GgufTensorType::Q4_K)
        check(citlali_hip_matvec_q4k(w.device_quantized_data(), xb->half_data(), yd->half_data(), in_f, out_f) == 0,
              "abi");
    else
        check(citlali_hip_matvec_q6k(w.device_quantized_data(), xb->half_data(), yd->half_data(), in_f, out_f) == 0,
              "abi");
    check(download_half(yd, out_f) == y, w.name + ": backend and C ABI agree bit for bit");
    int bad = 0;
    for (int o = 0; o < out_f; ++o) bad += !close(orc_h2f(y[o]), ref[o]);
    check(bad == 0, w.name + " " + std::to_string(out_f) + "x" + std::to_string(in_f) + ": " + std::to_string(bad) +
                        " rows outside tolerance");
    std::printf("linear %s %dx%d ok\n", w.name.c_str(), out_f, in_f);
}

void test_linear_errors() {
    auto backend = model::make_fp16_linear_backend();
    model::WeightHandle w;
    w.name = "blk.0.ffn_down.weight";
    w.gguf_type = GgufTensorType::Q6_K;
    w.storage_kind = WeightStorageKind::QuantizedDevice;
    w.dims = {300, 8};   // in_features not a multiple of 256
    w.buffer = compute::make_device_buffer(2 * 8 * 210);
    auto x = compute::make_device_half_buffer(300), y = compute::make_device_half_buffer(8);
    expect_error([&] { backend->forward(w, x, y); }, "not a multiple of the 256-value super-block", "K % 256");
    w.dims = {512, 8};
    expect_error([&] { backend->forward(w, x, y); }, "input buffer holds 600 bytes, 1024 needed", "short input");
    std::printf("linear errors ok\n");
}

void test_attention() {
    const int heads = 16, kv = 8, hd = 128, max_ctx = 1024, position = 1023;   // config 2
    Rng r{5};
    const std::vector<uint16_t> q = normal_f16(r, heads * hd);
    const std::vector<uint16_t> k = normal_f16(r, (size_t)max_ctx * kv * hd);
    const std::vector<uint16_t> v = normal_f16(r, (size_t)max_ctx * kv * hd);
    std::vector<double> ref(heads * hd);
    orc_attention(q.data(), k.data(), v.data(), position, heads, kv, hd, ref.data());
    auto qb = upload(q), kb = upload(k), vb = upload(v);
    auto scores = compute::make_device_buffer((size_t)heads * max_ctx * 4);
    auto out = compute::make_device_half_buffer(heads * hd);
    compute::launch_attention(qb->half_data(), kb->half_data(), vb->half_data(), static_cast<float*>(scores->data()),
                              out->half_data(), position, max_ctx, heads, kv, hd);
    const std::vector<uint16_t> o = download_half(out, heads * hd);
    int bad = 0;
    for (int i = 0; i < heads * hd; ++i) bad += !close(orc_h2f(o[i]), ref[i]);
    check(bad == 0, "launch_attention 16/8/128 L=1024: " + std::to_string(bad) + " outside tolerance");
    expect_error([&] {
        compute::launch_attention(qb->half_data(), kb->half_data(), vb->half_data(), nullptr, out->half_data(),
                                  max_ctx, max_ctx, heads, kv, hd);
    }, "position exceeds max_context", "position == max_context");
    std::printf("attention ok\n");
}

void test_embed() {
    const int hidden = 4096, vocab = 64;
    Rng r{11};
    const std::vector<uint8_t> table = quant_blocks(r, GgufTensorType::Q6_K, (size_t)vocab * hidden / 256);
    auto tb = upload(table);
    auto out = compute::make_device_half_buffer(hidden);
    for (int token : {0, 17, vocab - 1}) {
        compute::launch_embed_q6k(static_cast<const uint8_t*>(tb->data()), token, out->half_data(), hidden);
        std::vector<uint16_t> ref(hidden);
        orc_embed_q6k(table.data(), token, ref.data(), hidden);
        check(download_half(out, hidden) == ref, "embed_q6k token " + std::to_string(token) + " bit-exact");
    }
    std::printf("embed_q6k ok\n");
}

// ------------------------------------------------------------ the model
// A synthetic Qwen3-style model: host bytes for the oracle, WeightHandles for
// QwenModel.  d is chosen so every matrix has rms ~ gain / sqrt(in), which
// keeps the fp16 activations in range (random Q4_K codes give rms(w) ~ 300 d,
// random Q6_K codes ~ 1366 d).
struct HostMatrix {
    GgufTensorType type;
    int rows, cols;
    std::vector<uint8_t> bytes;
};

struct SynthModel {
    model::QwenConfig cfg;
    HostMatrix embd, output;
    std::vector<uint16_t> output_norm;
    struct Layer {
        std::vector<uint16_t> attn_norm, q_norm, k_norm, ffn_norm;   // q_norm / k_norm empty: absent
        std::vector<uint16_t> q_bias, k_bias, v_bias, o_bias, gate_bias, up_bias, down_bias;   // empty: absent
        HostMatrix q, k, v, o, gate, up, down;
    };
    std::vector<Layer> layers;
};

HostMatrix make_matrix(Rng& r, GgufTensorType t, int rows, int cols, double gain) {
    const double per = t == GgufTensorType::Q4_K ? 300.0 : 1366.0;
    const double d = gain / std::sqrt((double)cols) / per;
    HostMatrix m{t, rows, cols, quant_blocks(r, t, (size_t)rows * cols / 256, 0.8 * d, 1.2 * d)};
    return m;
}

std::vector<uint16_t> make_norm(Rng& r, int n) {
    std::vector<uint16_t> v(n);
    for (auto& h : v) h = orc_f2h_rne((float)(1.0 + 0.1 * r.normal()));
    return v;
}

SynthModel make_model(uint64_t seed, int hidden, int heads, int kv_heads, int ff, int layers, int vocab) {
    Rng r{seed};
    SynthModel m;
    m.cfg.vocab_size = vocab;
    m.cfg.context_length = 4096;
    m.cfg.embedding_length = hidden;
    m.cfg.block_count = layers;
    m.cfg.feed_forward_length = ff;
    m.cfg.head_count = heads;
    m.cfg.head_count_kv = kv_heads;
    m.cfg.head_dim = 128;
    m.cfg.architecture = "qwen3";
    m.embd = make_matrix(r, GgufTensorType::Q6_K, vocab, hidden, std::sqrt((double)hidden));   // rows of rms ~1
    m.output = make_matrix(r, GgufTensorType::Q6_K, vocab, hidden, 3.0);
    m.output_norm = make_norm(r, hidden);
    const int nq = heads * 128, nkv = kv_heads * 128;
    for (int l = 0; l < layers; ++l) {
        SynthModel::Layer L;
        L.attn_norm = make_norm(r, hidden);
        L.q_norm = make_norm(r, 128);
        L.k_norm = make_norm(r, 128);
        L.ffn_norm = make_norm(r, hidden);
        L.q = make_matrix(r, GgufTensorType::Q4_K, nq, hidden, 1.0);
        L.k = make_matrix(r, GgufTensorType::Q4_K, nkv, hidden, 1.0);
        L.v = make_matrix(r, GgufTensorType::Q6_K, nkv, hidden, 1.0);
        L.o = make_matrix(r, GgufTensorType::Q4_K, hidden, nq, 0.5);
        L.gate = make_matrix(r, GgufTensorType::Q4_K, ff, hidden, 1.0);
        L.up = make_matrix(r, GgufTensorType::Q4_K, ff, hidden, 1.0);
        L.down = make_matrix(r, GgufTensorType::Q6_K, hidden, ff, 0.5);
        m.layers.push_back(std::move(L));
    }
    return m;
}

std::vector<uint16_t> make_bias(Rng& r, int n, double scale) {
    std::vector<uint16_t> v(n);
    for (auto& h : v) h = orc_f2h_rne((float)(scale * r.normal()));
    return v;
}

// Qwen2-style: biases on q/k/v (the Qwen2 checkpoints), and here on o and
// the FFN matrices too (so every bias add and the unfused gate/up path run);
// no q/k head norms.
SynthModel make_model_biased(uint64_t seed, int hidden, int heads, int kv_heads, int ff, int layers, int vocab) {
    SynthModel m = make_model(seed, hidden, heads, kv_heads, ff, layers, vocab);
    m.cfg.architecture = "qwen2";
    Rng r{seed * 7 + 5};
    const int nq = heads * 128, nkv = kv_heads * 128;
    for (auto& L : m.layers) {
        L.q_norm.clear();
        L.k_norm.clear();
        L.q_bias = make_bias(r, nq, 0.5);
        L.k_bias = make_bias(r, nkv, 0.5);
        L.v_bias = make_bias(r, nkv, 0.5);
        L.o_bias = make_bias(r, hidden, 0.1);
        L.gate_bias = make_bias(r, ff, 0.2);
        L.up_bias = make_bias(r, ff, 0.2);
        L.down_bias = make_bias(r, hidden, 0.1);
    }
    return m;
}

const uint16_t* opt(const std::vector<uint16_t>& v) { return v.empty() ? nullptr : v.data(); }

OrcMatrix orc_of(const HostMatrix& m) { return {m.type == GgufTensorType::Q4_K ? ORC_Q4K : ORC_Q6K, m.bytes.data()}; }

// The oracle's model view; `drop` zeroes nothing, it only selects layers.
struct OracleModel {
    std::vector<OrcLayer> layers;
    OrcModel m{};
    std::vector<std::vector<uint16_t>> caches;
    std::vector<uint16_t*> cache_ptrs;
    OracleModel(const SynthModel& s, int max_ctx, int n_layers) {
        for (int l = 0; l < n_layers; ++l) {
            const auto& L = s.layers[l];
            OrcLayer o{};
            o.attn_norm = L.attn_norm.data();
            o.q = orc_of(L.q); o.k = orc_of(L.k); o.v = orc_of(L.v); o.o = orc_of(L.o);
            o.q_norm = opt(L.q_norm); o.k_norm = opt(L.k_norm);
            o.q_bias = opt(L.q_bias); o.k_bias = opt(L.k_bias); o.v_bias = opt(L.v_bias); o.o_bias = opt(L.o_bias);
            o.gate_bias = opt(L.gate_bias); o.up_bias = opt(L.up_bias); o.down_bias = opt(L.down_bias);
            o.ffn_norm = L.ffn_norm.data();
            o.gate = orc_of(L.gate); o.up = orc_of(L.up); o.down = orc_of(L.down);
            layers.push_back(o);
        }
        m.hidden = (int)s.cfg.embedding_length; m.heads = (int)s.cfg.head_count; m.kv_heads = (int)s.cfg.head_count_kv;
        m.head_dim = 128; m.ff = (int)s.cfg.feed_forward_length; m.n_layers = n_layers;
        m.vocab = (int)s.cfg.vocab_size; m.max_ctx = max_ctx; m.eps = s.cfg.rms_norm_eps; m.theta = s.cfg.rope_theta;
        m.token_embd = orc_of(s.embd); m.output_norm = s.output_norm.data(); m.output = orc_of(s.output);
        m.layers = layers.data();
        for (int i = 0; i < 2 * n_layers; ++i) caches.emplace_back((size_t)max_ctx * m.kv_heads * 128, 0);
        for (auto& c : caches) cache_ptrs.push_back(c.data());
    }
    int32_t step(int32_t tok, int pos, float* logits) { return orc_forward_token(&m, cache_ptrs.data(), tok, pos, logits); }
};

// The host loader's fp16 values of a quantised matrix (DequantizeToFp16).
std::vector<uint16_t> dequant_f16(const HostMatrix& m) {
    std::vector<uint16_t> out((size_t)m.rows * m.cols);
    if (m.type == GgufTensorType::Q4_K) {
        orc_dequant_q4k_f16(m.bytes.data(), out.size(), out.data());
    } else {
        orc_dequant_q6k_f16(m.bytes.data(), out.size(), out.data());
    }
    return out;
}

// The oracle's matrices replaced by their fp16 dequantisation (`keep` owns
// the values), as QwenModel sees them under DequantizeToFp16.
void oracle_over_f16(OracleModel& o, const SynthModel& s, std::vector<std::vector<uint16_t>>& keep) {
    auto f16 = [&](const HostMatrix& m) {
        keep.push_back(dequant_f16(m));
        return OrcMatrix{ORC_F16, keep.back().data()};
    };
    keep.reserve(keep.size() + 2 + 7 * o.layers.size());
    o.m.token_embd = f16(s.embd);
    o.m.output = f16(s.output);
    for (size_t l = 0; l < o.layers.size(); ++l) {
        const auto& L = s.layers[l];
        OrcLayer& d = o.layers[l];
        d.q = f16(L.q); d.k = f16(L.k); d.v = f16(L.v); d.o = f16(L.o);
        d.gate = f16(L.gate); d.up = f16(L.up); d.down = f16(L.down);
    }
    o.m.layers = o.layers.data();
}

// A matrix as QwenModel holds it: raw blocks (KeepQuantized) or, with fp16,
// the host loader's fp16 values (DequantizeToFp16).
model::WeightHandle handle_of(const HostMatrix& m, const std::string& name, bool fp16 = false) {
    model::WeightHandle w;
    w.name = name;
    w.gguf_type = m.type;
    w.storage_kind = fp16 ? WeightStorageKind::Fp16Device : WeightStorageKind::QuantizedDevice;
    w.dims = {(uint64_t)m.cols, (uint64_t)m.rows};
    w.element_count = (uint64_t)m.rows * m.cols;
    w.buffer = fp16 ? upload(dequant_f16(m)) : upload(m.bytes);
    return w;
}

model::WeightHandle handle_of_norm(const std::vector<uint16_t>& v, const std::string& name) {
    model::WeightHandle w;
    w.name = name;
    w.gguf_type = GgufTensorType::F16;
    w.storage_kind = WeightStorageKind::Fp16Device;
    w.dims = {(uint64_t)v.size(), 1};
    w.element_count = v.size();
    w.buffer = upload(v);
    return w;
}

model::QwenWeights device_weights(const SynthModel& s, bool fp16 = false) {
    model::QwenWeights w;
    w.token_embedding = handle_of(s.embd, "token_embd.weight", fp16);
    w.output_norm = handle_of_norm(s.output_norm, "output_norm.weight");
    w.output_weight = handle_of(s.output, "output.weight", fp16);
    for (size_t l = 0; l < s.layers.size(); ++l) {
        const auto& L = s.layers[l];
        const std::string b = "blk." + std::to_string(l) + ".";
        model::QwenLayerWeights d;
        d.attn_norm = handle_of_norm(L.attn_norm, b + "attn_norm.weight");
        d.attn_q = handle_of(L.q, b + "attn_q.weight", fp16);
        d.attn_k = handle_of(L.k, b + "attn_k.weight", fp16);
        d.attn_v = handle_of(L.v, b + "attn_v.weight", fp16);
        d.attn_o = handle_of(L.o, b + "attn_output.weight", fp16);
        const auto vec = [&](const std::vector<uint16_t>& v, const std::string& name) {
            return v.empty() ? model::WeightHandle{} : handle_of_norm(v, b + name);
        };
        d.attn_q_norm = vec(L.q_norm, "attn_q_norm.weight");
        d.attn_k_norm = vec(L.k_norm, "attn_k_norm.weight");
        d.attn_q_bias = vec(L.q_bias, "attn_q.bias");
        d.attn_k_bias = vec(L.k_bias, "attn_k.bias");
        d.attn_v_bias = vec(L.v_bias, "attn_v.bias");
        d.attn_o_bias = vec(L.o_bias, "attn_output.bias");
        d.ffn_gate_bias = vec(L.gate_bias, "ffn_gate.bias");
        d.ffn_up_bias = vec(L.up_bias, "ffn_up.bias");
        d.ffn_down_bias = vec(L.down_bias, "ffn_down.bias");
        d.ffn_norm = handle_of_norm(L.ffn_norm, b + "ffn_norm.weight");
        d.ffn_gate = handle_of(L.gate, b + "ffn_gate.weight", fp16);
        d.ffn_up = handle_of(L.up, b + "ffn_up.weight", fp16);
        d.ffn_down = handle_of(L.down, b + "ffn_down.weight", fp16);
        w.layers.push_back(std::move(d));
    }
    return w;
}

// CPU: pins of the oracle's forward composition.
void test_oracle_forward_pins() {
    SynthModel s = make_model(21, 1024, 8, 4, 2048, 2, 512);
    const int ctx = 8;
    // (1) attn_o and ffn_down zero: every layer adds nothing, so the logits
    // are output(rms_norm(embed(token))) -- residual stream and final norm wiring
    SynthModel z = s;
    for (auto& L : z.layers) {
        std::fill(L.o.bytes.begin(), L.o.bytes.end(), 0);
        std::fill(L.down.bytes.begin(), L.down.bytes.end(), 0);
    }
    OracleModel oz(z, ctx, 2);
    std::vector<float> lg(512);
    oz.step(5, 0, lg.data());
    oz.step(77, 1, lg.data());
    std::vector<uint16_t> e(1024), n(1024);
    orc_embed_q6k(z.embd.bytes.data(), 77, e.data(), 1024);
    orc_rms_norm(e.data(), z.output_norm.data(), n.data(), 1024, z.cfg.rms_norm_eps);
    std::vector<double> ref(512);
    orc_matvec_q6k(z.output.bytes.data(), n.data(), ref.data(), 1024, 512, 0);
    for (int i = 0; i < 512; ++i) check(lg[i] == (float)ref[i], "zero residual branches: logit " + std::to_string(i));
    // (2) a second layer whose attn_o and ffn_down are zero changes nothing:
    // the two-layer model equals the one-layer model, step by step
    SynthModel t = s;
    std::fill(t.layers[1].o.bytes.begin(), t.layers[1].o.bytes.end(), 0);
    std::fill(t.layers[1].down.bytes.begin(), t.layers[1].down.bytes.end(), 0);
    OracleModel two(t, ctx, 2), one(s, ctx, 1);
    std::vector<float> a(512), b(512);
    for (int p = 0; p < 4; ++p) {
        two.step(3 + 11 * p, p, a.data());
        one.step(3 + 11 * p, p, b.data());
        check(a == b, "inert second layer, position " + std::to_string(p));
    }
    // (3) history matters: the same token at position 1 after different
    // first tokens gives different logits (attention reads the cache)
    OracleModel h1(s, ctx, 2), h2(s, ctx, 2);
    h1.step(1, 0, a.data());
    h2.step(2, 0, b.data());
    h1.step(9, 1, a.data());
    h2.step(9, 1, b.data());
    check(a != b, "the cache feeds attention");

    // The closed forms below recompute one layer from the separately pinned
    // routines (embed, rms_norm, the GEMVs, swiglu, add) with one branch made
    // trivial, so a wiring slip in the composition fails them: the residual
    // added to the wrong buffer, a norm taking the other norm's weight,
    // gate/up exchanged, the attention range off by one, RoPE before the
    // q/k norm.  fp16 roundings here go by way of float, so values are
    // compared to a bound (1 ulp for cache rows, 5e-3 of the logit rms).
    const int H = 1024, V = 512, NQ = 8 * 128, NKV = 4 * 128, F = 2048, group = 2;
    const float eps = s.cfg.rms_norm_eps;
    const auto f16 = [](const std::vector<double>& v) {
        std::vector<uint16_t> h(v.size());
        for (size_t i = 0; i < v.size(); ++i) h[i] = orc_f2h_rne((float)v[i]);
        return h;
    };
    const auto embed = [&](int tok) {
        std::vector<uint16_t> e(H);
        orc_embed_q6k(s.embd.bytes.data(), tok, e.data(), H);
        return e;
    };
    const auto gemv = [](const HostMatrix& w, const std::vector<uint16_t>& x) {
        std::vector<double> y(w.rows);
        if (w.type == GgufTensorType::Q4_K) {
            orc_matvec_q4k(w.bytes.data(), x.data(), y.data(), w.cols, w.rows, 0);
        } else {
            orc_matvec_q6k(w.bytes.data(), x.data(), y.data(), w.cols, w.rows, 0);
        }
        return y;
    };
    const auto norm = [&](const std::vector<uint16_t>& x, const std::vector<uint16_t>& w) {
        std::vector<uint16_t> n(x.size());
        orc_rms_norm(x.data(), w.data(), n.data(), (int)x.size(), eps);
        return n;
    };
    const auto logit_err = [&](const std::vector<float>& got, const std::vector<uint16_t>& x) {
        const std::vector<double> want = gemv(s.output, norm(x, s.output_norm));
        double e = 0, ss = 0;
        for (int i = 0; i < V; ++i) {
            e = std::max(e, std::fabs(got[i] - want[i]));
            ss += want[i] * want[i];
        }
        return e / std::sqrt(ss / V);
    };
    const auto within_ulp = [](uint16_t got, double want) {
        return std::fabs(orc_h2f(got) - want) <= std::ldexp(std::fabs(want), -10) + 1e-7;
    };
    const std::vector<int> seq = {4, 9, 100, 33, 250, 71};

    // (4) attn_q zero: q = 0 after its norm and RoPE, every score is 0 and
    // attention is the mean of V over positions 0..pos inclusive; with
    // ffn_down zero the layer adds o(mean V) to the residual stream only.
    SynthModel qz = s;
    std::fill(qz.layers[0].q.bytes.begin(), qz.layers[0].q.bytes.end(), 0);
    std::fill(qz.layers[0].down.bytes.begin(), qz.layers[0].down.bytes.end(), 0);
    OracleModel oq(qz, ctx, 1);
    std::vector<std::vector<uint16_t>> vrows;
    for (int p = 0; p < (int)seq.size(); ++p) {
        oq.step(seq[p], p, a.data());
        const std::vector<uint16_t> x0 = embed(seq[p]);
        const std::vector<double> v = gemv(s.layers[0].v, norm(x0, s.layers[0].attn_norm));
        const uint16_t* vc = oq.caches[1].data() + (size_t)p * NKV;
        bool row_ok = true;
        for (int i = 0; i < NKV; ++i) row_ok = row_ok && within_ulp(vc[i], v[i]);
        check(row_ok, "V cache row " + std::to_string(p) + " = v(attn_norm(embed))");
        vrows.push_back(f16(v));
        std::vector<double> att(NQ, 0.0);
        for (int h = 0; h < 8; ++h)
            for (int d = 0; d < 128; ++d) {
                double sum = 0;
                for (int t = 0; t <= p; ++t) sum += orc_h2f(vrows[t][(h / group) * 128 + d]);
                att[h * 128 + d] = sum / (p + 1);
            }
        const std::vector<uint16_t> proj = f16(gemv(s.layers[0].o, f16(att)));
        std::vector<uint16_t> x1 = x0;
        orc_add_inplace(x1.data(), proj.data(), H);
        const double e = logit_err(a, x1);
        check(e < 5e-3, "attn_q zero, position " + std::to_string(p) +
                            ": logits = output(norm(embed + o(mean of V[0..pos]))), error / rms " + std::to_string(e));
    }

    // (5) attn_o zero: the layer adds down(silu(gate(n)) * up(n)) with
    // n = rms_norm(x, ffn_norm) -- the FFN's norm weight and operand order.
    SynthModel oz2 = s;
    std::fill(oz2.layers[0].o.bytes.begin(), oz2.layers[0].o.bytes.end(), 0);
    OracleModel of(oz2, ctx, 1);
    for (int p = 0; p < 3; ++p) {
        of.step(seq[p], p, a.data());
        const std::vector<uint16_t> x0 = embed(seq[p]);
        const std::vector<uint16_t> n = norm(x0, s.layers[0].ffn_norm);
        const std::vector<uint16_t> g = f16(gemv(s.layers[0].gate, n)), u = f16(gemv(s.layers[0].up, n));
        std::vector<uint16_t> act(F);
        orc_swiglu(g.data(), u.data(), act.data(), F);
        const std::vector<uint16_t> dn = f16(gemv(s.layers[0].down, act));
        std::vector<uint16_t> x1 = x0;
        orc_add_inplace(x1.data(), dn.data(), H);
        const double e = logit_err(a, x1);
        check(e < 5e-3, "attn_o zero, position " + std::to_string(p) +
                            ": logits = output(norm(embed + down(swiglu(gate, up)(ffn_norm)))), error / rms " +
                            std::to_string(e));
    }

    // (6) RoPE acts after the k norm, V is not rotated: layer 0's k and v of
    // a token depend only on the token, so its cache rows at position P are
    // its rows at position 0 with each pair (i, i + 64) of K rotated by
    // P * theta^(-2i/128).  The other order -- RoPE on the raw k, then the
    // norm with this model's uneven k_norm weights -- misses by far more.
    const int P = 5, tok = 71;
    OracleModel o0(s, ctx, 1), oP(s, ctx, 1);
    o0.step(tok, 0, a.data());
    for (int p = 0; p <= P; ++p) oP.step(p < P ? seq[p] : tok, p, b.data());
    const uint16_t* k0 = o0.caches[0].data();
    const uint16_t* kP = oP.caches[0].data() + (size_t)P * NKV;
    check(std::memcmp(o0.caches[1].data(), oP.caches[1].data() + (size_t)P * NKV, NKV * 2) == 0,
          "V cache row of a token is the same at positions 0 and 5");
    const std::vector<double> kraw = gemv(s.layers[0].k, norm(embed(tok), s.layers[0].attn_norm));
    const std::vector<uint16_t> kraw16 = f16(kraw);
    bool rot_ok = true;
    double other = 0;
    for (int h = 0; h < 4; ++h) {
        // the other order: rotate the raw k, then rms-normalise with k_norm
        std::vector<double> r(128);
        for (int i = 0; i < 64; ++i) {
            const double ang = P * std::pow((double)s.cfg.rope_theta, -2.0 * i / 128.0);
            const double x0 = orc_h2f(k0[h * 128 + i]), x1 = orc_h2f(k0[h * 128 + 64 + i]);
            rot_ok = rot_ok && within_ulp(kP[h * 128 + i], x0 * std::cos(ang) - x1 * std::sin(ang)) &&
                     within_ulp(kP[h * 128 + 64 + i], x0 * std::sin(ang) + x1 * std::cos(ang));
            const double y0 = orc_h2f(kraw16[h * 128 + i]), y1 = orc_h2f(kraw16[h * 128 + 64 + i]);
            r[i] = y0 * std::cos(ang) - y1 * std::sin(ang);
            r[64 + i] = y0 * std::sin(ang) + y1 * std::cos(ang);
        }
        double ss = 0;
        for (double v : r) ss += v * v;
        const double inv = 1.0 / std::sqrt(ss / 128 + eps);
        for (int i = 0; i < 128; ++i)
            other = std::max(other, std::fabs(r[i] * inv * orc_h2f(s.layers[0].k_norm[i]) - orc_h2f(kP[h * 128 + i])));
    }
    check(rot_ok, "K cache row at position 5 = its position-0 row rotated by RoPE (norm, then RoPE)");
    check(other > 0.05, "RoPE-then-norm would differ from the oracle's K row by " + std::to_string(other));
    std::printf("oracle forward pins ok\n");
}

void test_model_load_errors() {
    SynthModel s = make_model(22, 1024, 8, 4, 2048, 1, 512);
    model::QwenModel m;
    expect_error([&] { m.forward_token(0, 0); }, "model is not loaded", "forward before load");
    // shapes are checked before anything is allocated on the device
    model::QwenWeights w;
    w.token_embedding.name = "token_embd.weight";
    w.token_embedding.dims = {1024, 500};
    w.layers.resize(1);
    expect_error([&] { m.load(s.cfg, w); },
                 "unexpected tensor shape for token_embd.weight: got [1024, 500], expected [1024, 512]",
                 "embedding shape");
    model::QwenConfig bad = s.cfg;
    bad.head_count_kv = 3;
    expect_error([&] { m.load(bad, model::QwenWeights{}); }, "head_count must be divisible by head_count_kv",
                 "GQA divisibility");
    std::printf("model load errors ok\n");
}

// GPU: greedy decode through QwenModel against the oracle's forward.  Both
// are fed the oracle's token at every step (teacher forcing), so each step
// compares the two models on identical inputs.  Every pick must be identical;
// the smallest top-2 margin of the oracle's logits is logged beside the
// logit error, so a seed whose margin fell inside the error would show why.
//
// How far the logits may move: the model itself amplifies fp16 rounding
// differences, so the bound is measured, not assumed.  A third model -- the
// oracle with half of its embedding values moved by one fp16 ulp -- runs in
// lockstep, and the GPU must stay within the spread that this 1-ulp input
// noise produces in the oracle.
void greedy_run(uint64_t seed, int prompt, int steps, int* identical, int* differ, int hidden = 2048,
                int heads = 16, bool biased = false, bool fp16 = false) {
    SynthModel s = biased ? make_model_biased(seed, hidden, heads, 8, 4096, 2, 8192)
                          : make_model(seed, hidden, heads, 8, 4096, 2, 8192);
    const int ctx = 128;
    model::QwenModel gpu;
    gpu.load(s.cfg, device_weights(s, fp16), ctx);
    OracleModel orc(s, ctx, 2), ctl(s, ctx, 2);
    std::vector<std::vector<uint16_t>> keep;
    std::vector<uint16_t> e16((size_t)8192 * hidden);
    if (fp16) {   // DequantizeToFp16: the oracle over the same fp16 values
        oracle_over_f16(orc, s, keep);
        oracle_over_f16(ctl, s, keep);
        e16 = keep.front();   // the embedding table
    } else {
        for (int t = 0; t < 8192; ++t) orc_embed_q6k(s.embd.bytes.data(), t, e16.data() + (size_t)t * hidden, hidden);
    }
    Rng flip{seed + 100};
    for (auto& h : e16)
        if ((h & 0x7fff) && (flip.next() & 1)) h ^= 1;
    ctl.m.token_embd = {ORC_F16, e16.data()};
    Rng r{seed * 31 + 1};
    std::vector<float> lo(8192), lg(8192), lc(8192);
    int32_t to = 0;
    double worst = 0, ctl_worst = 0, min_margin = 1e30, rms_sum = 0;
    std::string profile;
    *identical = 0;
    *differ = 0;
    for (int p = 0; p < prompt + steps; ++p) {
        const int32_t tok = p < prompt ? (int32_t)(r.next() % 8192) : to;
        const int32_t tg = gpu.forward_token(tok, (uint32_t)p);
        to = orc.step(tok, p, lo.data());
        ctl.step(tok, p, lc.data());
        gpu.logits()->copy_to_host(lg.data(), lg.size() * 4);
        double step_err = 0, ctl_err = 0;
        double ss = 0;
        for (int i = 0; i < 8192; ++i) {
            const double d = std::fabs((double)lg[i] - lo[i]);
            step_err = std::max(step_err, d);
            ctl_err = std::max(ctl_err, std::fabs((double)lc[i] - lo[i]));
            ss += (double)lo[i] * lo[i];
        }
        const double rms = std::sqrt(ss / 8192);
        rms_sum += rms;
        worst = std::max(worst, step_err / rms);
        ctl_worst = std::max(ctl_worst, ctl_err / rms);
        if (p == 0 || p == 1 || p == 4 || p == 16 || p == 40 || p == prompt + steps - 1) {
            char b[64];
            std::snprintf(b, sizeof b, " p%d:%.1e", p, step_err / rms);
            profile += b;
        }
        // device argmax = host rule on the device's own logits
        int32_t host_pick = 0;
        float hb = -INFINITY;
        for (int i = 0; i < 8192; ++i)
            if (std::isfinite(lg[i]) && lg[i] > hb) { hb = lg[i]; host_pick = i; }
        check(tg == host_pick, "device argmax = host rule at position " + std::to_string(p));
        if (p < prompt) continue;
        float best = -INFINITY, second = -INFINITY;
        for (float v : lo) {
            if (v > best) { second = best; best = v; } else if (v > second) second = v;
        }
        min_margin = std::min(min_margin, (double)(best - second));
        if (tg == to) {
            ++*identical;
        } else {
            ++*differ;
            check(false, "greedy step " + std::to_string(p - prompt) + ": gpu " + std::to_string(tg) + " oracle " +
                             std::to_string(to) + ", oracle gap " + std::to_string((double)lo[to] - lo[tg]) +
                             ", logit error " + std::to_string(step_err));
        }
    }
    std::printf("greedy decode seed %llu (hidden %d%s%s): %d prompt tokens, %d greedy steps: %d identical, %d differ; "
                "max |logit diff| / rms(logits) = %.2e (rms %.2f; by position%s); oracle under 1-ulp embedding "
                "noise: %.2e; min oracle top-2 margin %.2e\n",
                (unsigned long long)seed, hidden, biased ? ", Qwen2-style biases, no q/k norm" : "",
                fp16 ? ", fp16 weights" : "", prompt, steps, *identical, *differ, worst, rms_sum / (prompt + steps),
                profile.c_str(), ctl_worst, min_margin);
    check(worst <= ctl_worst, "GPU logits within the oracle's own 1-ulp sensitivity");
}

// part 0: hidden 2048 (three seeds) and 4096; part 1: the other model forms
void test_forward_greedy(int part) {
    int identical = 0, differ = 0, all_differ = 0;
    if (part == 0) {
        for (uint64_t seed : {7ull, 8ull, 9ull}) {
            greedy_run(seed, 8, 64, &identical, &differ);
            all_differ += differ;
        }
        // hidden 4096, 32/8 heads
        greedy_run(10, 8, 64, &identical, &differ, 4096, 32);
        all_differ += differ;
        check(all_differ == 0, "every greedy pick identical");
        return;
    }
    // biases on every matrix, no q/k head norms (the unfused gate/up path and
    // the attention prologue without norm weights)
    greedy_run(12, 8, 64, &identical, &differ, 2048, 16, /*biased=*/true);
    all_differ += differ;
    // DequantizeToFp16 weights at hidden 4096: the fp16 GEMVs in the grouped,
    // gate/up and norm-prologue launches
    greedy_run(13, 8, 64, &identical, &differ, 4096, 32, /*biased=*/false, /*fp16=*/true);
    all_differ += differ;
    // rows ending in a partial wave step: hidden 1024 with 16/8 heads (q/k/v,
    // gate/up at K = 1024, attn_o at 2048: Qwen3-0.6B-like) and hidden 5120
    // with 40/8 heads (K = 5120, GQA group 5: Qwen3-14B-like)
    greedy_run(14, 8, 64, &identical, &differ, 1024, 16);
    all_differ += differ;
    greedy_run(15, 8, 64, &identical, &differ, 5120, 40);
    all_differ += differ;
    check(all_differ == 0, "every greedy pick identical");
}

// QwenModel::decode_greedy (captured steps replayed per token) against the
// forward_token loop: the same tokens exactly, across attention plan lengths
// 256, 512 and the max_context cap (600), replayed several times with eager
// work and synchronisations in between, and split over two calls.
void test_decode_greedy_graph(int hidden, int heads, bool fp16 = false) {
    SynthModel s = make_model(11, hidden, heads, 8, 4096, 2, 8192);
    const int ctx = 600, first = 240, steps = ctx - first;
    model::QwenModel gpu;
    gpu.load(s.cfg, device_weights(s, fp16), ctx);
    Rng r{77};
    for (int p = 0; p < first; ++p) gpu.forward_token((int32_t)(r.next() % 8192), (uint32_t)p, false);
    const int32_t start = (int32_t)(r.next() % 8192);
    std::vector<int32_t> eager;
    int32_t tok = start;
    for (int i = 0; i < steps; ++i) {
        tok = gpu.forward_token(tok, (uint32_t)(first + i));
        eager.push_back(tok);
    }
    for (int rep = 0; rep < 3; ++rep) {
        const std::vector<int32_t> got = gpu.decode_greedy(start, first, steps);
        check(got == eager, "decode_greedy replay " + std::to_string(rep) + " equals the forward_token loop");
        // eager work between replays: a forward_token whose cache write lies
        // past every position the replays read
        const int32_t t = gpu.forward_token(got.back(), ctx - 1);
        check(t >= 0 && t < 8192, "eager step between replays");
    }
    const std::vector<int32_t> a = gpu.decode_greedy(start, first, 17);
    const std::vector<int32_t> b = gpu.decode_greedy(a.back(), first + 17, steps - 17);
    std::vector<int32_t> ab = a;
    ab.insert(ab.end(), b.begin(), b.end());
    check(ab == eager, "decode_greedy split over two calls equals one call");
    check(gpu.decode_greedy(start, first, 0).empty(), "zero steps");
    expect_error([&] { gpu.decode_greedy(start, first, steps + 1); }, "position + steps exceeds max_context",
                 "steps past max_context");
    expect_error([&] { gpu.decode_greedy(8192, first, 1); }, "token id out of vocab range", "bad token");
    // forward_token after decode_greedy still runs on the library stream
    check(gpu.forward_token(start, first) == eager[0], "forward_token after decode_greedy");
    std::printf("decode_greedy (hidden %d): %d graph-replayed steps x 3 equal the forward_token loop\n", hidden,
                steps);
}

// max_context 3000 at 32/8 heads: the 2048-position bucket plans more
// attention chunks (32 of 64 positions) than max_context itself (24 of 128),
// so the model's split workspace must cover every bucket, not only the
// longest plan.  forward_token and the graph-replayed decode run from
// position 1000 through 1024 into that bucket and must agree.
void test_long_context_buckets() {
    SynthModel s = make_model(21, 4096, 32, 8, 4096, 1, 2048);
    const int ctx = 3000, first = 1000, steps = 90;
    model::QwenModel gpu;
    gpu.load(s.cfg, device_weights(s, false), ctx);
    Rng r{5};
    for (int p = 0; p < first; ++p) gpu.forward_token((int32_t)(r.next() % 2048), (uint32_t)p, false);
    const int32_t start = (int32_t)(r.next() % 2048);
    std::vector<int32_t> eager;
    int32_t tok = start;
    for (int i = 0; i < steps; ++i) {
        tok = gpu.forward_token(tok, (uint32_t)(first + i));
        eager.push_back(tok);
    }
    check(gpu.decode_greedy(start, first, steps) == eager,
          "max_context 3000: decode_greedy across the 1024 -> 2048 bucket equals the forward_token loop");
    std::printf("max_context 3000: %d steps from position %d through the 2048 bucket, graph = eager\n", steps, first);
}

// BASELINE config 5 at its full shape: the benchmark's synthetic Qwen3-8B
// (csrc/bench/synth_qwen3.hpp, model seed 1: 36 layers with their own
// weights, hidden 4096, FFN 12288, 32/8 heads, vocab 151936, Q4_K_M types)
// decodes the fixture's prompt (forward_token without logits but at its last
// position, as the session's prompt loop does), then its greedy steps
// free-running; every token must equal the oracle's
// (tests/golden/cfg5_greedy*.txt, written by tests/golden/make_cfg5_greedy),
// through the forward_token loop and through the graph-replayed
// decode_greedy.  The GPU's logits at the oracle's top-2 tokens are logged
// against the oracle's; a differing pick reports that step's GPU logit error
// beside the oracle's top-2 margin, so a near-tie resolved the other way
// reads differently from a wrong result.
void test_config5_greedy(const std::string& fixture) {
    std::FILE* f = std::fopen(fixture.c_str(), "r");
    check(f != nullptr, "open " + fixture);
    std::vector<int32_t> prompt, ids, second;
    std::vector<double> top, top2, rms;
    int want_steps = -1;
    std::vector<char> buf(1 << 16);
    while (std::fgets(buf.data(), (int)buf.size(), f)) {
        const char* line = buf.data();
        if (line[0] == '#' || line[0] == '\n') continue;
        if (std::strncmp(line, "prompt_seed", 11) == 0) continue;
        if (std::strncmp(line, "steps", 5) == 0) {
            want_steps = std::atoi(line + 5);
            continue;
        }
        if (std::strncmp(line, "prompt", 6) == 0) {
            int n = 0, used = 0;
            std::sscanf(line + 6, "%d%n", &n, &used);
            int off = 6 + used;
            for (int i = 0; i < n; ++i) {
                int32_t t = 0;
                check(std::sscanf(line + off, "%d%n", &t, &used) == 1, "fixture prompt id " + std::to_string(i));
                off += used;
                prompt.push_back(t);
            }
            continue;
        }
        int step = 0, id = 0, id2 = 0;
        double a = 0, b = 0, r = 0;
        if (std::sscanf(line, "%d %d %lf %d %lf %lf", &step, &id, &a, &id2, &b, &r) == 6) {
            check(step == (int)ids.size(), "fixture steps in order");
            ids.push_back(id);
            top.push_back(a);
            second.push_back(id2);
            top2.push_back(b);
            rms.push_back(r);
        }
    }
    std::fclose(f);
    const int P = (int)prompt.size(), S = (int)ids.size();
    check(P > 0 && S > 1 && S == want_steps, "fixture holds a prompt and all of its steps");

    namespace bq = citlali::bench;
    const bq::Qwen3Shape& shape = bq::kConfig5;
    SynthModel s;
    s.cfg.architecture = "qwen3";
    s.cfg.vocab_size = shape.vocab;
    s.cfg.context_length = 40960;
    s.cfg.embedding_length = shape.hidden;
    s.cfg.block_count = shape.layers;
    s.cfg.feed_forward_length = shape.ffn;
    s.cfg.head_count = shape.heads;
    s.cfg.head_count_kv = shape.kv_heads;
    s.cfg.head_dim = shape.head_dim;
    s.cfg.rms_norm_eps = 1e-6f;
    s.cfg.rope_theta = 1e6f;
    const int H = shape.hidden, F = shape.ffn, NQ = shape.heads * 128, NKV = shape.kv_heads * 128, V = shape.vocab;
    const std::vector<uint16_t> ones(H, 0x3c00), ones_hd(128, 0x3c00);
    const auto Q4 = GgufTensorType::Q4_K, Q6 = GgufTensorType::Q6_K;
    s.embd = {Q6, V, H, bq::embedding_bytes(1, shape)};
    s.output = {Q6, V, H, bq::output_bytes(1, shape)};
    s.output_norm = ones;
    for (int l = 0; l < shape.layers; ++l) {
        bq::LayerBytes b = bq::layer_bytes(1, l, shape);
        SynthModel::Layer L;
        L.attn_norm = ones;
        L.q_norm = ones_hd;
        L.k_norm = ones_hd;
        L.ffn_norm = ones;
        L.q = {Q4, NQ, H, std::move(b.q)};
        L.k = {Q4, NKV, H, std::move(b.k)};
        L.v = {Q6, NKV, H, std::move(b.v)};
        L.o = {Q4, H, NQ, std::move(b.o)};
        L.gate = {Q4, F, H, std::move(b.gate)};
        L.up = {Q4, F, H, std::move(b.up)};
        L.down = {Q6, H, F, std::move(b.down)};
        s.layers.push_back(std::move(L));
    }
    const int ctx = P + S;
    model::QwenModel gpu;
    gpu.load(s.cfg, device_weights(s), ctx);
    s.layers.clear();

    std::vector<float> lg(V);
    int32_t tok = 0;
    std::vector<int32_t> got;
    double worst = 0, min_margin = 1e30, worst_gap = 0, gap_at_min = 0, min_ratio = 1e30;
    int worst_step = 0, min_step = 0, worst_gap_step = 0, ratio_step = 0;
    for (int p = 0; p < P + S - 1; ++p) {
        tok = gpu.forward_token(p < P ? prompt[p] : tok, (uint32_t)p, p >= P - 1);
        if (p < P - 1) continue;
        const int step = p - (P - 1);
        gpu.logits()->copy_to_host(lg.data(), lg.size() * 4);
        got.push_back(tok);
        // the GPU's logits of the oracle's two best tokens against the oracle's
        const double e = std::max(std::fabs(lg[ids[step]] - top[step]), std::fabs(lg[second[step]] - top2[step]));
        const double margin = (top[step] - top2[step]) / rms[step];
        // what decides the pick: the error of the top-2 gap, not of each logit
        const double gap_err =
            std::fabs(((double)lg[ids[step]] - lg[second[step]]) - (top[step] - top2[step])) / rms[step];
        if (e / rms[step] > worst) {
            worst = e / rms[step];
            worst_step = step;
        }
        if (gap_err > worst_gap) {
            worst_gap = gap_err;
            worst_gap_step = step;
        }
        if (margin < min_margin) {
            min_margin = margin;
            min_step = step;
            gap_at_min = gap_err;
        }
        // headroom of the pick: oracle margin over the GPU's gap error
        if (margin / std::max(gap_err, 1e-12) < min_ratio) {
            min_ratio = margin / std::max(gap_err, 1e-12);
            ratio_step = step;
        }
        char why[320];
        std::snprintf(why, sizeof why,
                      "config 5 greedy step %d: gpu %d oracle %d (oracle top-2 margin / rms %.3e; gpu error of the "
                      "top-2 gap / rms %.3e, of each logit %.3e; largest gap error so far %.3e at step %d)",
                      step, tok, ids[step], margin, gap_err, e / rms[step], worst_gap, worst_gap_step);
        check(tok == ids[step], why);
        std::printf("  step %3d: id %6d ok; top-2 logits gpu %.6f %.6f oracle %.6f %.6f\n", step, tok, lg[ids[step]],
                    lg[second[step]], top[step], top2[step]);
        std::fflush(stdout);
    }
    // the last step through the graph-replayed decode: all steps again
    const std::vector<int32_t> g = gpu.decode_greedy(got[0], (uint32_t)P, (uint32_t)(S - 1));
    std::vector<int32_t> all = {got[0]};
    all.insert(all.end(), g.begin(), g.end());
    check(all == ids, "config 5: decode_greedy (graph replay) reproduces all " + std::to_string(S) + " oracle tokens");
    std::printf("config 5 (36 layers, hidden 4096, vocab 151936, %d-token prompt): %d of %d greedy tokens equal the "
                "oracle's, forward_token loop and decode_greedy; max |logit error| / rms at the top-2 tokens %.2e "
                "(step %d); max error of the top-2 gap / rms %.2e (step %d); min oracle top-2 margin / rms %.2e "
                "(step %d, gap error there %.2e); smallest margin / gap error %.2f (step %d)\n",
                P, S, S, worst, worst_step, worst_gap, worst_gap_step, min_margin, min_step, gap_at_min, min_ratio,
                ratio_step);
}

// ---- the synthetic model as a GGUF file ----------------------------------
// Matrices keep their Q4_K / Q6_K blocks with dims [in, out]; the norm
// vectors are stored as F32, as Qwen GGUF files store them.
// With `tokenizer`, its tokens, merges, ids and add_bos_token go into the
// file (the vocabulary size must be the model's); eos >= 0 replaces its EOS id.
void write_synth_gguf(const SynthModel& s, const std::string& path, const io::GgufFile* tokenizer = nullptr,
                      int64_t eos = -1) {
    bench::GgufOut o;
    std::vector<std::vector<float>> norms;   // borrowed by `o` until write()
    norms.reserve(1 + 11 * s.layers.size());
    const auto matrix = [&](const std::string& name, const HostMatrix& m) {
        o.tensor(name, {(uint64_t)m.cols, (uint64_t)m.rows}, m.type, m.bytes.data(), m.bytes.size());
    };
    const auto norm = [&](const std::string& name, const std::vector<uint16_t>& h) {
        norms.emplace_back(h.size());
        for (size_t i = 0; i < h.size(); ++i) norms.back()[i] = orc_h2f(h[i]);
        o.tensor(name, {(uint64_t)h.size()}, GgufTensorType::F32, norms.back().data(), h.size() * 4);
    };
    const model::QwenConfig& c = s.cfg;
    const std::string a = c.architecture;
    o.str("general.architecture", a);
    if (tokenizer) {
        const std::vector<std::string> tokens = tokenizer->get_string_array("tokenizer.ggml.tokens");
        check(tokens.size() == c.vocab_size, "tokenizer vocabulary size equals the model's");
        o.strings("tokenizer.ggml.tokens", tokens);
        o.strings("tokenizer.ggml.merges", tokenizer->get_string_array("tokenizer.ggml.merges"));
        o.u32("tokenizer.ggml.bos_token_id", (uint32_t)tokenizer->get_u64("tokenizer.ggml.bos_token_id", 151643));
        o.u32("tokenizer.ggml.eos_token_id",
              eos >= 0 ? (uint32_t)eos : (uint32_t)tokenizer->get_u64("tokenizer.ggml.eos_token_id", 151645));
        o.u32("tokenizer.ggml.padding_token_id", (uint32_t)tokenizer->get_u64("tokenizer.ggml.padding_token_id", 151643));
        o.boolean("tokenizer.ggml.add_bos_token", tokenizer->get_bool("tokenizer.ggml.add_bos_token", false));
    } else {
        o.strings("tokenizer.ggml.tokens", (int)c.vocab_size);
    }
    o.u32(a + ".context_length", c.context_length);
    o.u32(a + ".embedding_length", c.embedding_length);
    o.u32(a + ".block_count", c.block_count);
    o.u32(a + ".feed_forward_length", c.feed_forward_length);
    o.u32(a + ".attention.head_count", c.head_count);
    o.u32(a + ".attention.head_count_kv", c.head_count_kv);
    o.u32(a + ".attention.key_length", c.head_dim);
    o.u32(a + ".attention.value_length", c.head_dim);
    o.f32(a + ".attention.layer_norm_rms_epsilon", c.rms_norm_eps);
    o.f32(a + ".rope.freq_base", c.rope_theta);
    matrix("token_embd.weight", s.embd);
    norm("output_norm.weight", s.output_norm);
    matrix("output.weight", s.output);
    for (size_t l = 0; l < s.layers.size(); ++l) {
        const auto& L = s.layers[l];
        const std::string b = "blk." + std::to_string(l) + ".";
        norm(b + "attn_norm.weight", L.attn_norm);
        matrix(b + "attn_q.weight", L.q);
        matrix(b + "attn_k.weight", L.k);
        matrix(b + "attn_v.weight", L.v);
        matrix(b + "attn_output.weight", L.o);
        const auto opt_vec = [&](const std::string& name, const std::vector<uint16_t>& v) {
            if (!v.empty()) norm(b + name, v);
        };
        opt_vec("attn_q_norm.weight", L.q_norm);
        opt_vec("attn_k_norm.weight", L.k_norm);
        opt_vec("attn_q.bias", L.q_bias);
        opt_vec("attn_k.bias", L.k_bias);
        opt_vec("attn_v.bias", L.v_bias);
        opt_vec("attn_output.bias", L.o_bias);
        opt_vec("ffn_gate.bias", L.gate_bias);
        opt_vec("ffn_up.bias", L.up_bias);
        opt_vec("ffn_down.bias", L.down_bias);
        norm(b + "ffn_norm.weight", L.ffn_norm);
        matrix(b + "ffn_gate.weight", L.gate);
        matrix(b + "ffn_up.weight", L.up);
        matrix(b + "ffn_down.weight", L.down);
    }
    o.write(path);
}

std::string temp_path(const std::string& name) {
    const char* d = std::getenv("TMPDIR");
    return std::string(d && *d ? d : "/tmp") + "/citlali_" + std::to_string((long long)getpid()) + "_" + name;
}

// QwenModel::load from a GGUF file of the synthetic model.  KeepQuantized:
// the same device bytes as the model built from WeightHandles, so the same
// logits bit for bit and the same tokens.  DequantizeToFp16: fp16 weights and
// the fp16 GEMVs, against the oracle run over the same fp16 dequantisation
// (bound as greedy_run: within the oracle's own spread under 1-ulp input
// noise, every greedy token identical).
void test_load_from_gguf(bool biased) {
    SynthModel s = biased ? make_model_biased(24, 1024, 8, 4, 2048, 2, 512) : make_model(23, 1024, 8, 4, 2048, 2, 512);
    const int ctx = 64, vocab = 512, prompt = 8, steps = 40;
    const std::string path = temp_path(biased ? "synth_qwen2.gguf" : "synth_qwen3.gguf");
    write_synth_gguf(s, path);
    io::GgufFile g;
    g.load(path);
    const model::QwenConfig c = model::QwenConfig::from_gguf(g);
    check(c.architecture == s.cfg.architecture && c.vocab_size == 512 && c.embedding_length == 1024 && c.block_count == 2 &&
              c.feed_forward_length == 2048 && c.head_count == 8 && c.head_count_kv == 4 && c.head_dim == 128 &&
              c.value_dim == 128 && c.context_length == s.cfg.context_length && c.rms_norm_eps == s.cfg.rms_norm_eps &&
              c.rope_theta == s.cfg.rope_theta,
          "QwenConfig::from_gguf of the written model");

    model::QwenModel a, b, f;
    a.load(s.cfg, device_weights(s), ctx);
    b.load(g, ctx, /*quantized=*/true);
    f.load(g, ctx, /*quantized=*/false);
    std::remove(path.c_str());   // the loaded weights live in device memory

    // the oracle over fp16 weights, and a twin with 1-ulp embedding noise
    std::vector<std::vector<uint16_t>> keep;
    OracleModel orc(s, ctx, 2), ctl(s, ctx, 2);
    oracle_over_f16(orc, s, keep);
    oracle_over_f16(ctl, s, keep);
    std::vector<uint16_t> noisy(static_cast<const uint16_t*>(ctl.m.token_embd.data),
                                static_cast<const uint16_t*>(ctl.m.token_embd.data) + (size_t)vocab * 1024);
    Rng flip{5};
    for (auto& h : noisy)
        if ((h & 0x7fff) && (flip.next() & 1)) h ^= 1;
    ctl.m.token_embd = {ORC_F16, noisy.data()};

    Rng r{99};
    std::vector<float> la(vocab), lb(vocab), lf(vocab), lo(vocab), lc(vocab);
    int32_t tok = 0, mismatched = 0;
    double worst = 0, ctl_worst = 0;
    for (int p = 0; p < prompt + steps; ++p) {
        const int32_t in = p < prompt ? (int32_t)(r.next() % vocab) : tok;
        const int32_t ta = a.forward_token(in, (uint32_t)p);
        const int32_t tb = b.forward_token(in, (uint32_t)p);
        const int32_t tf = f.forward_token(in, (uint32_t)p);
        const int32_t to = orc.step(in, p, lo.data());
        ctl.step(in, p, lc.data());
        a.logits()->copy_to_host(la.data(), la.size() * 4);
        b.logits()->copy_to_host(lb.data(), lb.size() * 4);
        f.logits()->copy_to_host(lf.data(), lf.size() * 4);
        check(ta == tb && std::memcmp(la.data(), lb.data(), la.size() * 4) == 0,
              "GGUF KeepQuantized load = WeightHandle load, logits bit for bit at position " + std::to_string(p));
        double err = 0, cerr = 0, ss = 0;
        for (int i = 0; i < vocab; ++i) {
            err = std::max(err, std::fabs((double)lf[i] - lo[i]));
            cerr = std::max(cerr, std::fabs((double)lc[i] - lo[i]));
            ss += (double)lo[i] * lo[i];
        }
        const double rms = std::sqrt(ss / vocab);
        worst = std::max(worst, err / rms);
        ctl_worst = std::max(ctl_worst, cerr / rms);
        if (p >= prompt && tf != to) {
            ++mismatched;
            check(false, "fp16-path token at step " + std::to_string(p - prompt) + ": gpu " + std::to_string(tf) +
                             " oracle " + std::to_string(to) + ", oracle gap " +
                             std::to_string((double)lo[to] - lo[tf]) + ", logit error " + std::to_string(err));
        }
        tok = ta;
    }
    std::printf("GGUF load (%s): KeepQuantized = WeightHandles over %d positions; DequantizeToFp16 vs fp16 oracle: "
                "max |logit diff| / rms = %.2e (oracle under 1-ulp embedding noise %.2e), %d/%d greedy tokens differ\n",
                biased ? "qwen2, biases, no q/k norm" : "qwen3", prompt + steps, worst, ctl_worst, mismatched, steps);
    check(worst <= std::max(ctl_worst, 1e-3), "fp16-path logits within the oracle's own 1-ulp sensitivity");
    check(mismatched == 0, "fp16-path greedy tokens identical");
}

// ---- InferenceSession over the synthetic model ----------------------------
// The reference's generation loop (session.cpp:61-104) restated over
// forward_token, one token at a time: what the session must reproduce with
// its chunked decode_greedy.
struct Manual {
    runtime::GenerationResult r;
    std::vector<std::string> pieces;
    std::vector<int32_t> ids;   // every greedy token computed, emitted or not
};
Manual manual_generate(model::QwenModel& m, const tokenizer::Tokenizer& t, const std::string& prompt,
                       uint32_t max_new) {
    Manual out;
    const std::vector<int32_t> toks = t.encode(prompt, true);
    check(!toks.empty() && toks.size() + max_new < m.max_context(), "manual loop: prompt fits");
    uint32_t pos = 0;
    int32_t next = 0;
    for (size_t i = 0; i < toks.size(); ++i) next = m.forward_token(toks[i], pos++, i + 1 == toks.size());
    for (uint32_t i = 0; i < max_new; ++i) {
        out.ids.push_back(next);
        if (next == t.eos_id()) {
            out.r.stop_reason = runtime::StopReason::Eos;
            break;
        }
        out.pieces.push_back(t.decode_token(next));
        out.r.text += out.pieces.back();
        ++out.r.generated_tokens;
        next = m.forward_token(next, pos++);
        if (pos >= m.max_context()) {
            out.r.stop_reason = runtime::StopReason::ContextLimit;
            break;
        }
    }
    return out;
}

const char* stop_name(runtime::StopReason r) {
    return r == runtime::StopReason::Eos ? "eos" : r == runtime::StopReason::MaxNewTokens ? "max_new" : "context";
}

void check_same(const runtime::GenerationResult& got, const std::vector<std::string>& got_pieces, const Manual& want,
                const std::string& what) {
    check(got.text == want.r.text && got.generated_tokens == want.r.generated_tokens &&
              got.stop_reason == want.r.stop_reason && got_pieces == want.pieces,
          what + ": session = forward_token loop (" + std::to_string(got.generated_tokens) + " vs " +
              std::to_string(want.r.generated_tokens) + " tokens, stop " + stop_name(got.stop_reason) + " vs " +
              stop_name(want.r.stop_reason) + ")");
}

void test_session(const std::string& tok_path, bool quantized) {
    io::GgufFile tg;
    tg.load(tok_path);
    tokenizer::Tokenizer tok;
    tok.load_from_gguf(tg);
    const int vocab = tok.vocab_size(), ctx = 256;
    SynthModel s = make_model(41, 1024, 8, 4, 2048, 2, vocab);
    const std::string path = temp_path("session.gguf");
    write_synth_gguf(s, path, &tg);

    runtime::InferenceSession sess;
    sess.load_model(path, ctx, quantized);
    io::GgufFile g;
    g.load(path);
    model::QwenModel ref;
    ref.load(g, ctx, quantized);
    check(sess.tokenizer().vocab_size() == vocab && sess.tokenizer().eos_id() == tok.eos_id() &&
              sess.config().vocab_size == (uint32_t)vocab,
          "session: tokenizer and config from the GGUF file");

    const std::vector<std::string> prompts = {"The quick brown fox", "人工智能正在改变世界。",
                                              "<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n", "a"};
    runtime::GenerationOptions opt;
    opt.max_new_tokens = 40;
    const auto distinct = [](std::vector<int32_t> v) {
        std::sort(v.begin(), v.end());
        return (size_t)(std::unique(v.begin(), v.end()) - v.begin());
    };
    std::vector<int32_t> seen;   // greedy ids of the most varied prompt, for the EOS case
    std::string eos_prompt;
    for (const std::string& p : prompts) {
        const Manual want = manual_generate(ref, tok, p, opt.max_new_tokens);
        if (distinct(want.ids) > distinct(seen)) {
            seen = want.ids;
            eos_prompt = p;
        }
        for (uint32_t chunk : {1u, 5u, 16u, 64u}) {
            sess.set_decode_chunk(chunk);
            std::vector<std::string> pieces;
            const runtime::GenerationResult r =
                sess.generate_once_result(p, opt, [&](const std::string& x) { pieces.push_back(x); });
            check_same(r, pieces, want, "generate, prompt of " + std::to_string(p.size()) + " bytes, chunk " +
                                            std::to_string(chunk));
        }
        std::printf("  prompt %zu bytes -> %u tokens, stop %s, text %zu bytes: same for chunks 1/5/16/64\n", p.size(),
                    want.r.generated_tokens, stop_name(want.r.stop_reason), want.r.text.size());
    }
    check(sess.generate_once("The quick brown fox", opt) == manual_generate(ref, tok, "The quick brown fox", 40).r.text,
          "generate_once returns the result's text");

    // EOS: a greedy token of the most varied prompt made the EOS id, the one
    // whose first appearance is latest (so that the stop falls inside a
    // chunk when the model varies enough)
    check(seen.size() >= 8, "the prompt ran 8 steps");
    int32_t eos = seen[0];
    size_t first = 0;
    for (size_t k = 0; k < seen.size(); ++k)
        if (std::find(seen.begin(), seen.begin() + k, seen[k]) == seen.begin() + k && seen[k] != tok.eos_id()) {
            eos = seen[k];
            first = k;
        }
    const std::string path_eos = temp_path("session_eos.gguf");
    write_synth_gguf(s, path_eos, &tg, eos);
    runtime::InferenceSession se;
    se.load_model(path_eos, ctx, quantized);
    // chunks that end just before, at and after the EOS step, and a long one
    const uint32_t at = (uint32_t)std::max<size_t>(first, 1);
    for (uint32_t chunk : {1u, at, at + 1, 16u}) {
        se.set_decode_chunk(chunk);
        std::vector<std::string> pieces;
        const runtime::GenerationResult r =
            se.generate_once_result(eos_prompt, opt, [&](const std::string& x) { pieces.push_back(x); });
        check(r.stop_reason == runtime::StopReason::Eos && r.generated_tokens == first &&
                  pieces.size() == first,
              "EOS id " + std::to_string(eos) + " stops generation before it, after " + std::to_string(first) +
                  " tokens (chunk " + std::to_string(chunk) + ")");
        std::string text;
        for (size_t i = 0; i < first; ++i) text += tok.decode_token(seen[i]);
        check(r.text == text, "EOS: text of the tokens before it");
    }
    std::printf("  EOS id %d: stops after %zu tokens for chunks 1/%u/%u/16 (%zu distinct ids among %zu)\n", eos,
                first, at, at + 1, distinct(seen), seen.size());
    std::remove(path_eos.c_str());

    // chat: the history grows by the user message and the reply
    sess.set_decode_chunk(16);
    sess.reset_conversation();
    std::vector<std::pair<std::string, std::string>> hist;
    for (const std::string& msg : {std::string("Hello there"), std::string("And again?")}) {
        hist.emplace_back("user", msg);
        const Manual want = manual_generate(ref, tok, tok.apply_chat_template(hist, true), 24);
        opt.max_new_tokens = 24;
        std::vector<std::string> pieces;
        const runtime::GenerationResult r =
            sess.chat_once_result(msg, opt, [&](const std::string& x) { pieces.push_back(x); });
        check_same(r, pieces, want, "chat turn " + std::to_string(hist.size() / 2 + 1));
        hist.emplace_back("assistant", want.r.text);
        check(sess.history() == hist, "chat history holds the user messages and replies");
    }
    sess.reset_conversation();
    check(sess.history().empty(), "reset_conversation clears the history");
    const std::string fresh = tok.apply_chat_template({{"user", "Hello there"}}, true);
    check(sess.chat_once("Hello there", opt) == manual_generate(ref, tok, fresh, 24).r.text,
          "after reset, chat starts from the new message alone");

    // the prompt-length rule: prompt + max_new must stay below max_context
    const size_t n_prompt = tok.encode(prompts[0], true).size();
    opt.max_new_tokens = (uint32_t)(ctx - n_prompt);
    bool threw = false;
    try {
        sess.generate_once_result(prompts[0], opt);
    } catch (const Error& e) {
        threw = std::string(e.what()).find("prompt plus generation exceeds max_context") != std::string::npos;
    }
    check(threw, "prompt + max_new == max_context is refused");
    opt.max_new_tokens = (uint32_t)(ctx - n_prompt - 1);
    const Manual want = manual_generate(ref, tok, prompts[0], opt.max_new_tokens);
    std::vector<std::string> pieces;
    const runtime::GenerationResult r =
        sess.generate_once_result(prompts[0], opt, [&](const std::string& x) { pieces.push_back(x); });
    check_same(r, pieces, want, "generation to the last position");
    std::printf("  %zu-token prompt + %u new tokens in a %d-position context: same, stop %s\n", n_prompt,
                opt.max_new_tokens, ctx, stop_name(r.stop_reason));

    // wall time of that generation per decode chunk (not a check)
    for (uint32_t chunk : {1u, 4u, 16u, 64u}) {
        sess.set_decode_chunk(chunk);
        sess.generate_once_result(prompts[0], opt);   // graphs captured
        const auto t0 = std::chrono::steady_clock::now();
        const runtime::GenerationResult g = sess.generate_once_result(prompts[0], opt);
        const double s_ = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        std::printf("  chunk %2u: %u tokens in %.2f ms, %.0f tok/s (prompt included)\n", chunk, g.generated_tokens,
                    s_ * 1e3, g.generated_tokens / s_);
    }
    std::remove(path.c_str());
}

// The session test's model (2 layers, hidden 1024, the tokenizer of
// `tok_path`) written to `path`, for the command-line tests.
void write_session_model(const std::string& tok_path, const std::string& path) {
    io::GgufFile tg;
    tg.load(tok_path);
    const int vocab = (int)tg.get_string_array("tokenizer.ggml.tokens").size();
    write_synth_gguf(make_model(41, 1024, 8, 4, 2048, 2, vocab), path, &tg);
    std::printf("wrote %s (vocab %d)\n", path.c_str(), vocab);
}

// CPU: the reference's load signatures with a RemoteOptions argument
// (include/citlali/model/qwen_model.h:38-40, include/citlali/runtime/
// session.h:39-42), called as the reference's session.cpp:15 and cli/main.cpp
// call them.  Options that offload layers are refused before any weight
// reaches the device; an out-of-range layer gets the reference's message.
void test_remote_options() {
    char exe[4096];
    const ssize_t n = readlink("/proc/self/exe", exe, sizeof exe - 1);
    check(n > 0, "locate the test program");
    exe[n] = 0;
    std::string dir(exe);
    dir = dir.substr(0, dir.rfind('/'));
    const std::string tok = dir + "/../golden/tokenizer/qwen_like.gguf";
    const std::string path = "/tmp/citlali_remote_" + std::to_string(getpid()) + ".gguf";
    write_session_model(tok, path);
    io::GgufFile g;
    g.load(path);

    remote::RemoteOptions r;
    r.endpoint = "127.0.0.1:9000";
    r.transport = remote::Transport::Wifi6;
    r.backend = remote::Backend::Hybrid;
    r.layers = {1};
    check(r.enabled() && r.offloads_layer(1) && !r.offloads_layer(0), "RemoteOptions::enabled / offloads_layer");
    model::QwenModel m;
    expect_error([&] { m.load(g, 0, true, r); }, "remote layer offload is not supported by this build",
                 "QwenModel::load with a remote layer");
    r.layers = {0, 7};
    expect_error([&] { m.load(g, 0, true, r); }, "remote layer index is out of range: 7",
                 "QwenModel::load with an out-of-range remote layer");
    remote::RemoteOptions no_endpoint;
    no_endpoint.layers = {0};
    check(!no_endpoint.enabled(), "layers without an endpoint: not enabled");
    expect_error([&] { m.load(g, 0, false, no_endpoint); }, "remote layer offload is not supported",
                 "QwenModel::load with layers and no endpoint");
    expect_error([&] { m.forward_token(0, 0); }, "model is not loaded", "a refused load loads nothing");

    runtime::InferenceSession session;
    r.layers = {0};
    expect_error([&] { session.load_model(path, 2048, true, r); }, "remote layer offload is not supported",
                 "InferenceSession::load_model with a remote layer");
    std::remove(path.c_str());
    std::printf("remote options ok\n");
}

// One InferenceSession generation, printed as "tokens N stop S text HEX".
void session_text(const std::string& model, const std::string& prompt, uint32_t max_new, bool chat, bool quantized) {
    runtime::InferenceSession sess;
    sess.load_model(model, 256, quantized);
    runtime::GenerationOptions opt;
    opt.max_new_tokens = max_new;
    const runtime::GenerationResult r =
        chat ? sess.chat_once_result(prompt, opt) : sess.generate_once_result(prompt, opt);
    std::string hex;
    for (unsigned char c : r.text) {
        char b[4];
        std::snprintf(b, sizeof b, "%02x", c);
        hex += b;
    }
    std::printf("tokens %u stop %s text %s\n", r.generated_tokens, stop_name(r.stop_reason), hex.c_str());
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    try {
        if (mode == "cpu") {
            test_dtype();
            test_fp16_rules();
            test_dispatch_errors();
            test_oracle_forward_pins();
            test_model_load_errors();
            test_remote_options();
        } else if (mode == "write_session_model") {
            check(argc > 3, "write_session_model TOKENIZER_GGUF OUT");
            write_session_model(argv[2], argv[3]);
        } else if (mode == "session_text") {
            check(argc > 6, "session_text MODEL PROMPT MAX_NEW CHAT QUANTIZED");
            if (citlali_hip_init(0) != CITLALI_OK) {
                std::printf("FAIL: no GPU: %s\n", citlali_hip_last_error());
                return 1;
            }
            session_text(argv[2], argv[3], (uint32_t)std::atoi(argv[4]), std::atoi(argv[5]) != 0,
                         std::atoi(argv[6]) != 0);
        } else if (mode == "gpu" || mode == "greedy" || mode == "greedy2" || mode == "graph" || mode == "gguf" ||
                   mode == "cfg5" || mode == "session") {
            // GPU modes, each a part of a length that one test run prints
            // progress within
            if (citlali_hip_init(0) != CITLALI_OK) {
                std::printf("FAIL: no GPU: %s\n", citlali_hip_last_error());
                return 1;
            }
            if (mode == "gpu") {
                test_buffers();
                test_linear(GgufTensorType::Q4_K, WeightStorageKind::QuantizedDevice, 4096, 1024, 1);
                test_linear(GgufTensorType::Q6_K, WeightStorageKind::QuantizedDevice, 12288, 512, 2);
                test_linear(GgufTensorType::Q4_K, WeightStorageKind::QuantizedDevice, 1024, 3072, 3);   // config 1
                test_linear(GgufTensorType::F16, WeightStorageKind::Fp16Device, 1024, 256, 4);
                test_linear_errors();
                test_attention();
                test_embed();
            } else if (mode == "greedy") {
                test_forward_greedy(0);
            } else if (mode == "greedy2") {
                test_forward_greedy(1);
            } else if (mode == "graph") {
                test_decode_greedy_graph(2048, 16);
                test_decode_greedy_graph(4096, 32);
                test_decode_greedy_graph(4096, 32, /*fp16=*/true);
                test_long_context_buckets();
            } else if (mode == "session") {
                check(argc > 2, "session needs a tokenizer GGUF file");
                std::printf("KeepQuantized weights:\n");
                test_session(argv[2], true);
                std::printf("DequantizeToFp16 weights:\n");
                test_session(argv[2], false);
            } else if (mode == "cfg5") {
                check(argc > 2, "cfg5 needs the fixture path");
                test_config5_greedy(argv[2]);
            } else {
                test_load_from_gguf(false);
                test_load_from_gguf(true);
            }
            compute::synchronize();
        } else {
            std::printf("usage: %s cpu|gpu|greedy|greedy2|graph|gguf|cfg5 FIXTURE|session TOKENIZER_GGUF|\n"
                        "       write_session_model TOKENIZER_GGUF OUT|session_text MODEL PROMPT MAX_NEW CHAT QUANTIZED\n",
                        argv[0]);
            return 2;
        }
    } catch (const std::exception& e) {
        std::printf("FAIL: uncaught %s\n", e.what());
        return 1;
    }
    std::printf("%s: %d checks passed\n", mode.c_str(), g_checks);
    return 0;
}
