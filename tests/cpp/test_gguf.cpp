// test_gguf.cpp -- the engine's GGUF reader, QwenConfig::from_gguf and
// WeightLoader through their C++ API.
//   test_gguf dump FILE...   canonical dumps (oracle/gguf_dump.hpp), each
//                            followed by a NUL line; no GPU
//   test_gguf gpu DIR        WeightLoader on the fixtures in DIR under both
//                            policies: device bytes against the file bytes
//                            (KeepQuantized) or the oracle's fp16 rules
#include "citlali/common.h"
#include "citlali/io/gguf_reader.h"
#include "citlali/model/qwen_config.h"
#include "citlali/model/weight_loader.h"
#include "citlali_oracle.h"
#include "gguf_dump.hpp"

#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

namespace {

using citlali::compute::GgufTensorType;
using citlali::compute::WeightStorageKind;
using citlali::model::WeightLoadPolicy;

int g_checks = 0, g_failed = 0;

void check(bool ok, const std::string& what) {
    ++g_checks;
    if (!ok) {
        ++g_failed;
        std::printf("FAIL: %s\n", what.c_str());
    }
}

void expect_error(const std::function<void()>& f, const std::string& needle, const std::string& what) {
    try {
        f();
        check(false, what + ": no error");
    } catch (const citlali::Error& e) {
        check(std::string(e.what()).find(needle) != std::string::npos, what + ": message '" + e.what() + "'");
    }
}

// What DequantizeToFp16 must produce, from the oracle's pinned rules.
std::vector<uint16_t> expected_fp16(const citlali::io::GgufTensorInfo& t, const std::vector<uint8_t>& b) {
    const uint64_t n = t.element_count();
    std::vector<uint16_t> out(n);
    switch (t.type) {
        case GgufTensorType::F16: std::memcpy(out.data(), b.data(), n * 2); break;
        case GgufTensorType::F32:
            for (uint64_t i = 0; i < n; ++i) {
                float f;
                std::memcpy(&f, b.data() + 4 * i, 4);
                out[i] = orc_f2h(f);
            }
            break;
        case GgufTensorType::BF16:   // bf16 -> fp32 exactly, then the host rule
            for (uint64_t i = 0; i < n; ++i) {
                uint16_t h;
                std::memcpy(&h, b.data() + 2 * i, 2);
                const uint32_t u = (uint32_t)h << 16;
                float f;
                std::memcpy(&f, &u, 4);
                out[i] = orc_f2h(f);
            }
            break;
        case GgufTensorType::Q8_0:
            for (uint64_t i = 0; i < n; ++i) {
                const uint8_t* blk = b.data() + (i / 32) * 34;
                uint16_t d;
                std::memcpy(&d, blk, 2);
                out[i] = orc_f2h(orc_h2f(d) * (float)(int8_t)blk[2 + i % 32]);
            }
            break;
        case GgufTensorType::Q4_K: orc_dequant_q4k_f16(b.data(), n, out.data()); break;
        case GgufTensorType::Q6_K: orc_dequant_q6k_f16(b.data(), n, out.data()); break;
        default: break;
    }
    return out;
}

bool is_quantized(GgufTensorType t) {
    return t == GgufTensorType::Q8_0 || t == GgufTensorType::Q4_K || t == GgufTensorType::Q6_K;
}

void check_file(const std::string& path, WeightLoadPolicy policy) {
    citlali::io::GgufFile g;
    g.load(path);
    const citlali::model::WeightLoader loader(g, policy);
    const bool keep = policy == WeightLoadPolicy::KeepQuantized;
    for (const auto& t : g.tensors()) {
        if (g.find_tensor(t.name) != &t) continue;   // a repeated name loads the last entry
        const std::string what = path.substr(path.rfind('/') + 1) + ":" + t.name + (keep ? " keep" : " fp16");
        const citlali::model::WeightHandle h = loader.load_required(t.name);
        check(h.name == t.name && h.gguf_type == t.type && h.dims == t.dims &&
                  h.element_count == t.element_count(), what + ": handle fields");
        const std::vector<uint8_t> file = g.read_tensor_bytes(t);
        if (keep && is_quantized(t.type)) {
            check(h.storage_kind == WeightStorageKind::QuantizedDevice && h.buffer && h.buffer->bytes() == t.nbytes,
                  what + ": raw blocks");
            std::vector<uint8_t> dev(t.nbytes);
            h.buffer->copy_to_host(dev.data(), dev.size());
            check(dev == file, what + ": device bytes = file bytes");
        } else {
            check(h.storage_kind == WeightStorageKind::Fp16Device && h.buffer &&
                      h.buffer->bytes() == t.element_count() * 2, what + ": fp16 buffer");
            std::vector<uint16_t> dev(t.element_count());
            h.buffer->copy_to_host(dev.data(), dev.size() * 2);
            check(dev == expected_fp16(t, file), what + ": fp16 values");
        }
    }
}

int gpu(const std::string& dir) {
    for (const char* f : {"qwen3_basic.gguf", "all_types.gguf", "alignment_48.gguf", "version_2.gguf"}) {
        for (WeightLoadPolicy p : {WeightLoadPolicy::KeepQuantized, WeightLoadPolicy::DequantizeToFp16}) {
            check_file(dir + "/" + f, p);
        }
    }
    citlali::io::GgufFile g;
    g.load(dir + "/qwen3_basic.gguf");
    const citlali::model::WeightLoader loader(g);
    check(loader.policy() == WeightLoadPolicy::DequantizeToFp16, "default policy");
    check(!loader.load_optional("blk.9.missing").buffer, "load_optional of an absent tensor");
    expect_error([&] { loader.load_required("blk.9.missing"); }, "missing required tensor: blk.9.missing",
                 "load_required of an absent tensor");
    const citlali::model::WeightHandle r = loader.load_remote_required("blk.0.attn_q.weight");
    check(!r.buffer && r.dims == std::vector<uint64_t>({256, 256}) && r.gguf_type == GgufTensorType::Q4_K,
          "load_remote_required: metadata only");
    citlali::io::GgufFile far;
    far.load(dir + "/tensor_past_end.gguf");
    const citlali::model::WeightLoader fl(far, WeightLoadPolicy::KeepQuantized);
    expect_error([&] { fl.load_required("far"); }, "failed to read GGUF tensor: far", "tensor past the end");
    citlali::io::GgufFile cut;
    cut.load(dir + "/truncated_data.gguf");
    expect_error([&] { citlali::model::WeightLoader(cut).load_required("partial.q4k"); },
                 "failed to read GGUF tensor: partial.q4k", "tensor cut short");
    std::printf("gpu: %d checks passed, %d failed\n", g_checks - g_failed, g_failed);
    return g_failed == 0 ? 0 : 1;
}

int dump(int argc, char** argv) {
    for (int i = 2; i < argc; ++i) {
        const std::string d = gguf_dump::dump_path<citlali::io::GgufFile, citlali::model::QwenConfig>(
            argv[i], [](const citlali::io::GgufValue& v) { return citlali::io::metadata_value_to_string(v); });
        std::fwrite(d.data(), 1, d.size(), stdout);
        std::fputc('\0', stdout);
        std::fputc('\n', stdout);
    }
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc >= 2 && std::strcmp(argv[1], "dump") == 0) return dump(argc, argv);
    if (argc == 3 && std::strcmp(argv[1], "gpu") == 0) {
        try {
            return gpu(argv[2]);
        } catch (const std::exception& e) {
            std::printf("FAIL: unexpected error: %s\n", e.what());
            return 1;
        }
    }
    std::fprintf(stderr, "usage: test_gguf dump FILE... | test_gguf gpu FIXTURE_DIR\n");
    return 2;
}
