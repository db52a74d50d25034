// gguf_dump.hpp -- canonical text of what a GgufFile exposes.
//
// TEST INFRASTRUCTURE ONLY.  Compiled twice: against the reference's reader
// (oracle/ref_gguf_dump.cpp -> oracle/_ref/ref_gguf_dump, from the reference
// sources where they lie) and against the engine's (tests/cpp/test_gguf.cpp).
// oracle/gguf_oracle.py prints the same bytes for its restatement, so the
// three can be compared byte for byte.  Only the public interface of
// include/citlali/io/gguf_reader.h and QwenConfig::from_gguf is used.
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <string>
#include <vector>
#include <algorithm>

namespace gguf_dump {

inline std::string esc(const std::string& s) {
    static const char* kSpecial = "\\;,[]=";
    std::string out;
    for (unsigned char c : s) {
        if (c >= 0x21 && c <= 0x7e && !std::strchr(kSpecial, c)) {
            out += static_cast<char>(c);
        } else {
            char b[8];
            std::snprintf(b, sizeof b, "\\x%02x", c);
            out += b;
        }
    }
    return out;
}

inline std::string f64bits(double v) {
    uint64_t u;
    std::memcpy(&u, &v, 8);
    char b[32];
    std::snprintf(b, sizeof b, "%016llx", static_cast<unsigned long long>(u));
    return b;
}

inline std::string f32bits(float v) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    char b[16];
    std::snprintf(b, sizeof b, "%08x", u);
    return b;
}

constexpr uint64_t kFallbackU64 = 0xDEADBEEFDEADBEEFull;
constexpr int64_t kFallbackI64 = -0x123456789ll;
constexpr double kFallbackF64 = 0.5;
constexpr float kFallbackF32 = 0.25f;
inline const std::string kFallbackStr = "\x01" "fallback";
inline const std::string kAbsentKey = "no.such.key";

template <class File>
std::string getters(const File& g, const std::string& key) {
    std::string o;
    o += "u64=" + std::to_string(g.get_u64(key, kFallbackU64));
    o += " i64=" + std::to_string(g.get_i64(key, kFallbackI64));
    o += " f64=" + f64bits(g.get_f64(key, kFallbackF64));
    o += " f32=" + f32bits(g.get_f32(key, kFallbackF32));
    o += " b=" + std::to_string((int)g.get_bool(key, false)) + std::to_string((int)g.get_bool(key, true));
    o += " str=" + esc(g.get_string(key, kFallbackStr));
    const auto sa = g.get_string_array(key);
    o += " sarr=" + std::to_string(sa.size()) + "[";
    for (size_t i = 0; i < sa.size(); ++i) o += (i ? ";" : "") + esc(sa[i]);
    const auto fa = g.get_f32_array(key);
    o += "] farr=" + std::to_string(fa.size()) + "[";
    for (size_t i = 0; i < fa.size(); ++i) o += (i ? "," : "") + f32bits(fa[i]);
    const auto ua = g.get_u32_array(key);
    o += "] uarr=" + std::to_string(ua.size()) + "[";
    for (size_t i = 0; i < ua.size(); ++i) o += (i ? "," : "") + std::to_string(ua[i]);
    return o + "]";
}

template <class File, class ValueToString>
std::string dump_file(const File& g, ValueToString to_string) {
    std::string o;
    o += "version " + std::to_string(g.version()) + "\n";
    o += "alignment " + std::to_string(g.alignment()) + "\n";
    const auto& ts = g.tensors();
    o += "tensors " + std::to_string(ts.size()) + "\n";
    for (size_t i = 0; i < ts.size(); ++i) {
        const auto& t = ts[i];
        std::string dims;
        for (size_t d = 0; d < t.dims.size(); ++d) dims += (d ? "," : "") + std::to_string(t.dims[d]);
        const auto* found = g.find_tensor(t.name);
        o += "T " + std::to_string(i) + " " + esc(t.name) + " dims=" + dims +
             " type=" + std::to_string(static_cast<uint32_t>(t.type)) + " rel=" + std::to_string(t.relative_offset) +
             " abs=" + std::to_string(t.absolute_offset) + " nbytes=" + std::to_string(t.nbytes) +
             " find=" + std::to_string(found ? (long long)(found - ts.data()) : -1ll) + "\n";
    }
    std::vector<std::string> keys;
    for (const auto& kv : g.metadata()) keys.push_back(kv.first);
    std::sort(keys.begin(), keys.end());
    o += "metadata " + std::to_string(keys.size()) + "\n";
    for (const auto& k : keys) {
        const auto& v = g.metadata().at(k);
        const bool is_array = v.index() == 1;
        const size_t alt = is_array ? std::get<1>(v).index() : std::get<0>(v).index();
        o += "M " + esc(k) + " kind=" + (is_array ? "a" : "s") + std::to_string(alt) + " text=" + esc(to_string(v)) +
             " " + getters(g, k) + "\n";
    }
    o += "A has=" + std::to_string((int)g.has_key(kAbsentKey)) + " " + getters(g, kAbsentKey) + "\n";
    return o;
}

template <class Config, class File>
std::string dump_config(const File& g) {
    try {
        const Config c = Config::from_gguf(g);
        return "config arch=" + esc(c.architecture) + " vocab=" + std::to_string(c.vocab_size) +
               " ctx=" + std::to_string(c.context_length) + " emb=" + std::to_string(c.embedding_length) +
               " blocks=" + std::to_string(c.block_count) + " ff=" + std::to_string(c.feed_forward_length) +
               " heads=" + std::to_string(c.head_count) + " kv=" + std::to_string(c.head_count_kv) +
               " hd=" + std::to_string(c.head_dim) + " vd=" + std::to_string(c.value_dim) +
               " eps=" + f32bits(c.rms_norm_eps) + " theta=" + f32bits(c.rope_theta) + "\n";
    } catch (const std::exception& e) {
        return "config error: " + esc(e.what()) + "\n";
    }
}

// read_tensor_bytes of every tensor: FNV-1a 64 of the bytes, or "error".
template <class File>
std::string dump_reads(const File& g) {
    std::string o;
    const auto& ts = g.tensors();
    for (size_t i = 0; i < ts.size(); ++i) {
        o += "R " + std::to_string(i) + " ";
        try {
            const std::vector<uint8_t> b = g.read_tensor_bytes(ts[i]);
            uint64_t h = 0xcbf29ce484222325ull;
            for (uint8_t c : b) h = (h ^ c) * 0x100000001b3ull;
            char buf[40];
            std::snprintf(buf, sizeof buf, "n=%zu fnv=%016llx", b.size(), static_cast<unsigned long long>(h));
            o += buf;
        } catch (const std::exception&) {
            o += "error";
        }
        o += "\n";
    }
    return o;
}

// The whole dump of `path`: file, config and reads, or "error: ..." when
// load fails.
template <class File, class Config, class ValueToString>
std::string dump_path(const std::string& path, ValueToString to_string) {
    File g;
    try {
        g.load(path);
    } catch (const std::exception& e) {
        return "error: " + esc(e.what()) + "\n";
    }
    return dump_file(g, to_string) + dump_config<Config>(g) + dump_reads(g);
}

}  // namespace gguf_dump
