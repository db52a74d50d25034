// test_host_layer.cpp -- tests of the C++ host API (libcitlali.so) against
// the CPU oracle (liboracle.so, test infrastructure).
//
//   test_host_layer cpu   dtype tables, host fp16 rules (exhaustive), the
//                         LinearBackend dispatch and its errors; no GPU.
//   test_host_layer gpu   DeviceBuffer, LinearBackend::forward (Q4_K, Q6_K,
//                         fp16), launch_attention, launch_embed_q6k on the
//                         GPU, compared with the oracle.
// Prints one line per check and exits non-zero on the first failure.
#include "citlali/common.h"
#include "citlali/compute/common/dtype.h"
#include "citlali/compute/hip/kernels.h"
#include "citlali/compute/hip/tensor.h"
#include "citlali/model/linear_backend.h"
#include "citlali_hip.h"
#include "citlali_oracle.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

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

// Random quant bytes; d (and dmin) = fp16 of U[1e-3, 1e-2].
std::vector<uint8_t> quant_blocks(Rng& r, GgufTensorType t, size_t blocks) {
    const size_t bb = compute::gguf_type_block_bytes(t);
    std::vector<uint8_t> b(blocks * bb);
    for (auto& x : b) x = (uint8_t)r.next();
    for (size_t i = 0; i < blocks; ++i) {
        uint8_t* p = b.data() + i * bb;
        auto put = [&](size_t off) {
            const uint16_t h = orc_f2h_rne((float)(1e-3 + 9e-3 * r.uniform()));
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

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    try {
        if (mode == "cpu") {
            test_dtype();
            test_fp16_rules();
            test_dispatch_errors();
        } else if (mode == "gpu") {
            if (citlali_hip_init(0) != CITLALI_OK) {
                std::printf("FAIL: no GPU: %s\n", citlali_hip_last_error());
                return 1;
            }
            test_buffers();
            test_linear(GgufTensorType::Q4_K, WeightStorageKind::QuantizedDevice, 4096, 1024, 1);
            test_linear(GgufTensorType::Q6_K, WeightStorageKind::QuantizedDevice, 12288, 512, 2);
            test_linear(GgufTensorType::Q4_K, WeightStorageKind::QuantizedDevice, 1024, 3072, 3);   // config 1
            test_linear(GgufTensorType::F16, WeightStorageKind::Fp16Device, 1024, 256, 4);
            test_linear_errors();
            test_attention();
            test_embed();
            compute::synchronize();
        } else {
            std::printf("usage: %s cpu|gpu\n", argv[0]);
            return 2;
        }
    } catch (const std::exception& e) {
        std::printf("FAIL: uncaught %s\n", e.what());
        return 1;
    }
    std::printf("%s: %d checks passed\n", mode.c_str(), g_checks);
    return 0;
}
