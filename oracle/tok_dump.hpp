// tok_dump.hpp -- canonical text of what a Tokenizer does with a GGUF file's
// tokenizer metadata and a list of texts.
//
// TEST INFRASTRUCTURE ONLY.  Compiled twice: against the reference's
// tokenizer (oracle/ref_tok_dump.cpp -> oracle/_ref/ref_tok_dump, from the
// reference sources where they lie) and against the engine's
// (tests/cpp/test_tokenizer.cpp).  Only the public interface of
// include/citlali/tokenizer/tokenizer.h (tokenizer.h:12-35 in the reference)
// and GgufFile::load is used, so the two dumps can be compared byte for byte.
//
// TEXTS holds one text per line, hex-encoded (an empty line is the empty
// text).  The dump:
//   load error            when load_from_gguf throws (then nothing else)
//   vocab N bos B eos E pad P
//   piece ID HEX(token_piece) HEX(decode_token)     for every id in [-2, N+2)
//                                                   and 151643, 151645
//   text K HEX(text)
//   enc K ids of encode(text, false)
//   bos K ids of encode(text, true)
//   dec K HEX(decode(encode(text, false)))
//   chat K HEX(apply_chat_template({("system", text), ("user", text)}, true))
//   chat0 K HEX(apply_chat_template({("user", text)}, false))
// reload() is the state left by loading two files into one object;
// dump_fresh() the same dump for a tokenizer that never loaded one.
#pragma once

#include <cstdint>
#include <cstdio>
#include <exception>
#include <fstream>
#include <string>
#include <utility>
#include <vector>

namespace tok_dump {

inline std::string hex(const std::string& s) {
    static const char* d = "0123456789abcdef";
    std::string out;
    out.reserve(2 * s.size());
    for (unsigned char c : s) {
        out += d[c >> 4];
        out += d[c & 15];
    }
    return out;
}

inline std::string unhex(const std::string& h) {
    const auto v = [](char c) { return c <= '9' ? c - '0' : (c | 0x20) - 'a' + 10; };
    std::string out;
    for (size_t i = 0; i + 1 < h.size(); i += 2) out += static_cast<char>((v(h[i]) << 4) | v(h[i + 1]));
    return out;
}

inline std::vector<std::string> read_texts(const std::string& path) {
    std::ifstream in(path, std::ios::binary);
    std::vector<std::string> texts;
    std::string line;
    while (std::getline(in, line)) {
        if (!line.empty() && line.back() == '\r') line.pop_back();
        texts.push_back(unhex(line));
    }
    return texts;
}

inline std::string ids(const std::vector<int32_t>& v) {
    std::string out;
    for (int32_t t : v) out += " " + std::to_string(t);
    return out;
}

template <class Tokenizer>
std::string dump_state(const Tokenizer& t, const std::vector<std::string>& texts);

template <class GgufFile, class Tokenizer>
std::string dump(const std::string& gguf_path, const std::vector<std::string>& texts) {
    GgufFile g;
    Tokenizer t;
    try {
        g.load(gguf_path);
        t.load_from_gguf(g);
    } catch (const std::exception&) {
        return "load error\n";
    }
    return dump_state(t, texts);
}

// A tokenizer that never loaded a file (its defaults, no vocabulary).
template <class Tokenizer>
std::string dump_fresh(const std::vector<std::string>& texts) {
    const Tokenizer t;
    return dump_state(t, texts);
}

template <class Tokenizer>
std::string dump_state(const Tokenizer& t, const std::vector<std::string>& texts) {
    std::string out;
    const int32_t n = t.vocab_size();
    out += "vocab " + std::to_string(n) + " bos " + std::to_string(t.bos_id()) + " eos " +
           std::to_string(t.eos_id()) + " pad " + std::to_string(t.pad_id()) + "\n";
    std::vector<int32_t> probe;
    for (int32_t i = -2; i < n + 2; ++i) probe.push_back(i);
    probe.push_back(151643);
    probe.push_back(151645);
    for (int32_t i : probe)
        out += "piece " + std::to_string(i) + " " + hex(t.token_piece(i)) + " " + hex(t.decode_token(i)) + "\n";
    for (size_t k = 0; k < texts.size(); ++k) {
        const std::string K = std::to_string(k);
        const std::string& s = texts[k];
        const std::vector<int32_t> e = t.encode(s, false);
        out += "text " + K + " " + hex(s) + "\n";
        out += "enc " + K + ids(e) + "\n";
        out += "bos " + K + ids(t.encode(s, true)) + "\n";
        out += "dec " + K + " " + hex(t.decode(e)) + "\n";
        out += "chat " + K + " " + hex(t.apply_chat_template({{"system", s}, {"user", s}}, true)) + "\n";
        out += "chat0 " + K + " " + hex(t.apply_chat_template({{"user", s}}, false)) + "\n";
    }
    return out;
}

// load_from_gguf of A, then of B, on one object: "vocab N bos B eos E pad P"
// (ids that B does not set keep A's values), "load error" when either throws.
template <class GgufFile, class Tokenizer>
std::string reload(const std::string& a, const std::string& b) {
    GgufFile ga, gb;
    Tokenizer t;
    std::string out;
    for (const std::string* path : {&a, &b}) {
        try {
            GgufFile& g = path == &a ? ga : gb;
            g.load(*path);
            t.load_from_gguf(g);
            out += "vocab " + std::to_string(t.vocab_size()) + " bos " + std::to_string(t.bos_id()) + " eos " +
                   std::to_string(t.eos_id()) + " pad " + std::to_string(t.pad_id()) + "\n";
        } catch (const std::exception&) {
            out += "load error\n";
        }
    }
    return out;
}

}  // namespace tok_dump
