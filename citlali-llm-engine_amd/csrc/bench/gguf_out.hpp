// gguf_out.hpp -- a small GGUF v3 writer for synthetic model files (the
// decode benchmark and the host-API tests).
//
// Layout read by GgufFile (the reference's gguf_reader.cpp:160-241): "GGUF",
// u32 version 3, u64 tensor count, u64 metadata count; metadata as string
// key + u32 type + value; the tensor directory (string name, u32 rank, u64
// dims, u32 type, u64 offset relative to the data section); zero padding to
// a 32-byte boundary, then the tensor bytes, each at a 32-byte aligned
// offset.  Tensor bytes are borrowed until write(); an entry may point at the
// bytes of an earlier one (alias), which the format allows and which keeps a
// file of repeated layer weights small.
#pragma once

#include "citlali/common.h"
#include "citlali/compute/common/dtype.h"

#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

namespace citlali::bench {

class GgufOut {
public:
    static constexpr uint64_t kAlign = 32;

    void u32(const std::string& k, uint32_t v) {
        key(k, 4);
        put(kv_, v);
    }
    void f32(const std::string& k, float v) {
        key(k, 6);
        put(kv_, v);
    }
    void str(const std::string& k, const std::string& v) {
        key(k, 8);
        text(kv_, v);
    }
    void boolean(const std::string& k, bool v) {
        key(k, 7);
        put<uint8_t>(kv_, v ? 1 : 0);
    }
    // tokenizer.ggml.tokens-style array of n placeholder strings
    void strings(const std::string& k, int n) {
        key(k, 9);
        put<uint32_t>(kv_, 8);
        put<uint64_t>(kv_, (uint64_t)n);
        for (int i = 0; i < n; ++i) text(kv_, "t" + std::to_string(i));
    }
    void strings(const std::string& k, const std::vector<std::string>& v) {
        key(k, 9);
        put<uint32_t>(kv_, 8);
        put<uint64_t>(kv_, (uint64_t)v.size());
        for (const std::string& s : v) text(kv_, s);
    }

    // Adds a tensor with its own bytes; returns its index.
    size_t tensor(const std::string& name, std::vector<uint64_t> dims, compute::GgufTensorType t, const void* p,
                  size_t n) {
        entries_.push_back({name, std::move(dims), t, static_cast<const uint8_t*>(p), n, align(end_), false});
        end_ = entries_.back().offset + n;
        return entries_.size() - 1;
    }
    // Adds a tensor that reads the bytes of entry `of`.
    void alias(const std::string& name, std::vector<uint64_t> dims, compute::GgufTensorType t, size_t of) {
        const Entry& e = entries_.at(of);
        entries_.push_back({name, std::move(dims), t, e.data, e.bytes, e.offset, true});
    }

    // Returns the file size.
    uint64_t write(const std::string& path) const {
        std::vector<uint8_t> head = {'G', 'G', 'U', 'F'};
        put<uint32_t>(head, 3);
        put<uint64_t>(head, entries_.size());
        put<uint64_t>(head, n_kv_);
        head.insert(head.end(), kv_.begin(), kv_.end());
        for (const Entry& e : entries_) {
            text(head, e.name);
            put<uint32_t>(head, (uint32_t)e.dims.size());
            for (uint64_t d : e.dims) put(head, d);
            put<uint32_t>(head, (uint32_t)e.type);
            put<uint64_t>(head, e.offset);
        }
        while (head.size() % kAlign) head.push_back(0);
        FILE* f = std::fopen(path.c_str(), "wb");
        require(f != nullptr, "cannot create " + path);
        bool ok = std::fwrite(head.data(), 1, head.size(), f) == head.size();
        uint64_t pos = 0;
        static const uint8_t zeros[kAlign] = {};
        for (const Entry& e : entries_) {
            if (!ok || e.alias) continue;
            ok = std::fwrite(zeros, 1, e.offset - pos, f) == e.offset - pos &&
                 std::fwrite(e.data, 1, e.bytes, f) == e.bytes;
            pos = e.offset + e.bytes;
        }
        ok = std::fclose(f) == 0 && ok;
        require(ok, "short write to " + path);
        return head.size() + pos;
    }

private:
    struct Entry {
        std::string name;
        std::vector<uint64_t> dims;
        compute::GgufTensorType type;
        const uint8_t* data;
        size_t bytes;
        uint64_t offset;
        bool alias;
    };
    static uint64_t align(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
    template <typename T>
    static void put(std::vector<uint8_t>& b, T v) {
        const uint8_t* p = reinterpret_cast<const uint8_t*>(&v);
        b.insert(b.end(), p, p + sizeof v);
    }
    static void text(std::vector<uint8_t>& b, const std::string& s) {
        put<uint64_t>(b, s.size());
        b.insert(b.end(), s.begin(), s.end());
    }
    void key(const std::string& k, uint32_t type) {
        text(kv_, k);
        put(kv_, type);
        ++n_kv_;
    }
    std::vector<uint8_t> kv_;
    uint64_t n_kv_ = 0;
    std::vector<Entry> entries_;
    uint64_t end_ = 0;
};

}  // namespace citlali::bench
