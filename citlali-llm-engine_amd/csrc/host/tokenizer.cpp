// Byte-level BPE tokenizer (the reference's src/tokenizer/tokenizer.cpp).
//
//   load_from_gguf       tokenizer.cpp:130-170
//   initial pieces       tokenizer.cpp:107-121 (control tokens), 172-210
//   encode               tokenizer.cpp:226-292 (merge order: lowest rank,
//                        then leftmost; pieces starting with '<' never merge)
//   decode_token/decode  tokenizer.cpp:307-383
//   apply_chat_template  tokenizer.cpp:385-400
//
// The byte-level alphabet is GPT-2's: the bytes 0x21-0x7E, 0xA1-0xAC and
// 0xAE-0xFF stand for themselves as code points, every other byte for
// 256 + (its index among those others), written as UTF-8 (tokenizer.cpp:64-95).
#include "citlali/tokenizer/tokenizer.h"

#include "citlali/common.h"

#include <array>
#include <queue>
#include <functional>

namespace citlali::tokenizer {
namespace {

// The Qwen control tokens matched in raw text, in the order they are tried
// (tokenizer.cpp:108-112).
const std::array<const char*, 14> kControlTokens = {
    "<|endoftext|>",   "<|im_start|>",    "<|im_end|>",     "<|object_ref_start|>", "<|object_ref_end|>",
    "<|box_start|>",   "<|box_end|>",     "<|quad_start|>", "<|quad_end|>",         "<|vision_start|>",
    "<|vision_end|>",  "<|vision_pad|>",  "<|image_pad|>",  "<|video_pad|>"};

bool stands_for_itself(int b) {
    return (b >= 0x21 && b <= 0x7e) || (b >= 0xa1 && b <= 0xac) || (b >= 0xae && b <= 0xff);
}

// Byte <-> byte-level character.  Every code point is below 0x200, so a
// character is one UTF-8 byte (0x21-0x7E) or two; `one` and `two` map those
// exact byte strings back to byte + 1 (0: not a byte-level character).
struct ByteLevel {
    std::array<std::string, 256> chars;
    std::array<uint16_t, 256> one{};
    std::vector<uint16_t> two = std::vector<uint16_t>(65536, 0);

    ByteLevel() {
        int shifted = 0;
        for (int b = 0; b < 256; ++b) {
            const uint32_t cp = stands_for_itself(b) ? static_cast<uint32_t>(b) : 256u + shifted++;
            std::string& s = chars[b];
            if (cp < 0x80) {
                s.push_back(static_cast<char>(cp));
                one[cp] = static_cast<uint16_t>(b + 1);
            } else {
                s.push_back(static_cast<char>(0xc0 | (cp >> 6)));
                s.push_back(static_cast<char>(0x80 | (cp & 0x3f)));
                two[(static_cast<uint8_t>(s[0]) << 8) | static_cast<uint8_t>(s[1])] = static_cast<uint16_t>(b + 1);
            }
        }
    }
};

const ByteLevel& byte_level() {
    static const ByteLevel t;
    return t;
}

// Bytes of the UTF-8 character that starts with `lead`; 1 for a byte that
// cannot start one (tokenizer.cpp:98-104).
size_t utf8_length(uint8_t lead) {
    if (lead < 0x80) return 1;
    if ((lead & 0xe0) == 0xc0) return 2;
    if ((lead & 0xf0) == 0xe0) return 3;
    if ((lead & 0xf8) == 0xf0) return 4;
    return 1;
}

int hex_digit(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    return 0;
}

}  // namespace

void Tokenizer::load_from_gguf(const io::GgufFile& gguf) {
    std::vector<std::string> vocab = gguf.get_string_array("tokenizer.ggml.tokens");
    require(!vocab.empty(), "GGUF tokenizer.ggml.tokens is missing");
    std::unordered_map<std::string, int32_t> ids;
    ids.reserve(vocab.size());
    for (size_t i = 0; i < vocab.size(); ++i) ids[vocab[i]] = static_cast<int32_t>(i);

    // A missing id keeps the value this object holds (the constructor's
    // defaults on a first load), as the reference does.
    const auto id_or = [&](const char* key, int32_t current) {
        return static_cast<int32_t>(gguf.get_u64(key, static_cast<uint64_t>(static_cast<int64_t>(current))));
    };
    const int32_t bos = id_or("tokenizer.ggml.bos_token_id", bos_id_);
    const int32_t eos = id_or("tokenizer.ggml.eos_token_id", eos_id_);
    const int32_t pad = id_or("tokenizer.ggml.padding_token_id", pad_id_);
    const int32_t unk = id_or("tokenizer.ggml.unknown_token_id", unk_id_);

    std::unordered_map<std::string, Rule> rules;
    const std::vector<std::string> merges = gguf.get_string_array("tokenizer.ggml.merges");
    rules.reserve(merges.size());
    int rank = 0;
    for (const std::string& line : merges) {
        const size_t space = line.find(' ');
        if (space == std::string::npos) continue;
        std::string key = line;
        key[space] = '\n';
        Rule& r = rules[std::move(key)];
        r.merged = line.substr(0, space) + line.substr(space + 1);
        r.rank = rank++;
    }

    const ByteLevel& bl = byte_level();
    std::vector<std::string> byte_pieces(256);
    for (int b = 0; b < 256; ++b) {
        static const char* kHex = "0123456789ABCDEF";
        const std::string escaped = std::string("<0x") + kHex[b >> 4] + kHex[b & 15] + ">";
        if (ids.count(bl.chars[b]))
            byte_pieces[b] = bl.chars[b];
        else if (ids.count(escaped))
            byte_pieces[b] = escaped;
        else
            byte_pieces[b] = std::string(1, static_cast<char>(b));
    }

    vocab_ = std::move(vocab);
    ids_ = std::move(ids);
    rules_ = std::move(rules);
    byte_pieces_ = std::move(byte_pieces);
    bos_id_ = bos;
    eos_id_ = eos;
    pad_id_ = pad;
    unk_id_ = unk;
    add_bos_token_ = gguf.get_bool("tokenizer.ggml.add_bos_token", false);
    chat_template_ = gguf.get_string("tokenizer.chat_template", "");
}

std::vector<std::string> Tokenizer::raw_byte_pieces() {
    std::vector<std::string> pieces(256);
    for (int b = 0; b < 256; ++b) pieces[b] = std::string(1, static_cast<char>(b));
    return pieces;
}

const std::string& Tokenizer::byte_piece(uint8_t byte) const {
    return byte_pieces_[byte];
}

std::vector<std::string> Tokenizer::initial_pieces(const std::string& text) const {
    std::vector<std::string> pieces;
    pieces.reserve(text.size());
    for (size_t i = 0; i < text.size();) {
        if (text[i] == '<') {
            // the first control token written at i, used when the vocabulary has it
            const char* hit = nullptr;
            for (const char* c : kControlTokens)
                if (text.compare(i, std::char_traits<char>::length(c), c) == 0) {
                    hit = c;
                    break;
                }
            if (hit && ids_.count(hit)) {
                pieces.emplace_back(hit);
                i += pieces.back().size();
                continue;
            }
        }
        pieces.push_back(byte_piece(static_cast<uint8_t>(text[i])));
        ++i;
    }
    return pieces;
}

const Tokenizer::Rule* Tokenizer::rule_for(const std::string& left, const std::string& right, std::string& key) const {
    if ((!left.empty() && left[0] == '<') || (!right.empty() && right[0] == '<')) return nullptr;
    key.assign(left);
    key.push_back('\n');
    key.append(right);
    const auto it = rules_.find(key);
    return it == rules_.end() ? nullptr : &it->second;
}

std::vector<int32_t> Tokenizer::encode(const std::string& text, bool add_bos) const {
    std::vector<int32_t> out;
    if (add_bos && add_bos_token_ && bos_id_ >= 0) out.push_back(bos_id_);

    // The pieces as a doubly linked list; a node that absorbs its right
    // neighbour bumps its version, so heap entries naming an older content
    // are skipped when they surface.
    struct Node {
        std::string piece;
        int prev, next;
        uint32_t version = 0;
        bool alive = true;
    };
    struct Candidate {
        int rank, left, right;
        uint32_t left_version, right_version;
        const Rule* rule;
        bool operator>(const Candidate& o) const { return rank != o.rank ? rank > o.rank : left > o.left; }
    };

    std::vector<std::string> init = initial_pieces(text);
    const int n = static_cast<int>(init.size());
    std::vector<Node> nodes(n);
    for (int i = 0; i < n; ++i) nodes[i] = Node{std::move(init[i]), i - 1, i + 1 < n ? i + 1 : -1};

    std::priority_queue<Candidate, std::vector<Candidate>, std::greater<Candidate>> heap;
    std::string key;
    const auto offer = [&](int l, int r) {
        if (l < 0 || r < 0) return;
        if (const Rule* rule = rule_for(nodes[l].piece, nodes[r].piece, key))
            heap.push({rule->rank, l, r, nodes[l].version, nodes[r].version, rule});
    };
    for (int i = 0; i + 1 < n; ++i) offer(i, i + 1);

    while (!heap.empty()) {
        const Candidate c = heap.top();
        heap.pop();
        Node& l = nodes[c.left];
        Node& r = nodes[c.right];
        if (!l.alive || !r.alive || l.next != c.right || l.version != c.left_version || r.version != c.right_version)
            continue;
        l.piece = c.rule->merged;
        ++l.version;
        r.alive = false;
        l.next = r.next;
        if (r.next >= 0) nodes[r.next].prev = c.left;
        offer(l.prev, c.left);
        offer(c.left, l.next);
    }

    for (int i = n > 0 ? 0 : -1; i >= 0; i = nodes[i].next) {
        const auto it = ids_.find(nodes[i].piece);
        out.push_back(it == ids_.end() ? unk_id_ : it->second);
    }
    return out;
}

std::string Tokenizer::byte_level_to_bytes(const std::string& token) const {
    if (token.size() == 6 && token.compare(0, 3, "<0x") == 0 && token[5] == '>')
        return std::string(1, static_cast<char>((hex_digit(token[3]) << 4) | hex_digit(token[4])));
    const ByteLevel& bl = byte_level();
    std::string bytes;
    bytes.reserve(token.size());
    for (size_t i = 0; i < token.size();) {
        const uint8_t lead = static_cast<uint8_t>(token[i]);
        const size_t len = utf8_length(lead);
        if (i + len > token.size()) return token;
        uint16_t b = 0;
        if (len == 1)
            b = bl.one[lead];
        else if (len == 2)
            b = bl.two[(lead << 8) | static_cast<uint8_t>(token[i + 1])];
        if (b == 0) return token;
        bytes.push_back(static_cast<char>(b - 1));
        i += len;
    }
    return bytes;
}

std::string Tokenizer::token_piece(int32_t token_id) const {
    if (token_id < 0 || token_id >= vocab_size()) return "";
    return vocab_[static_cast<size_t>(token_id)];
}

std::string Tokenizer::decode_token(int32_t token_id) const {
    if (token_id < 0 || token_id >= vocab_size()) return "";
    const std::string& t = vocab_[static_cast<size_t>(token_id)];
    if (t.empty()) return "";
    if (t.size() >= 3 && t.compare(0, 2, "<|") == 0 && t.compare(t.size() - 2, 2, "|>") == 0) return "";
    return byte_level_to_bytes(t);
}

std::string Tokenizer::decode(const std::vector<int32_t>& tokens) const {
    std::string text;
    for (int32_t t : tokens) text += decode_token(t);
    return text;
}

std::string Tokenizer::apply_chat_template(const std::vector<std::pair<std::string, std::string>>& messages,
                                           bool add_generation_prompt) const {
    std::string out;
    for (const auto& [role, content] : messages) {
        out += "<|im_start|>";
        out += role;
        out += '\n';
        out += content;
        out += "<|im_end|>\n";
    }
    if (add_generation_prompt) out += "<|im_start|>assistant\n";
    return out;
}

}  // namespace citlali::tokenizer
