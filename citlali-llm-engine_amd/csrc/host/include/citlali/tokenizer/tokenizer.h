// citlali/tokenizer/tokenizer.h -- byte-level BPE tokenizer read from GGUF
// metadata, with the reference's public interface
// (include/citlali/tokenizer/tokenizer.h:12-35) and its results byte for byte
// (src/tokenizer/tokenizer.cpp:130-400).
//
// Vocabulary: tokenizer.ggml.tokens (required); a token string listed twice
// maps to its last id.  Ids: tokenizer.ggml.{bos,eos,padding,unknown}_token_id
// with defaults 151643 / 151645 / 151643 / 0, tokenizer.ggml.add_bos_token
// (default false).  Merges: tokenizer.ggml.merges, "left right" split at the
// first space; lines without a space are skipped without using a rank, and a
// pair listed twice keeps the later rank.
//
// Encoding: the text is cut into initial pieces -- one of the 14 Qwen control
// tokens where it starts at this byte and is in the vocabulary, else one byte
// as its GPT-2 byte-level character (or "<0xXX>", or the raw byte, whichever
// the vocabulary has first) -- then the adjacent pair of lowest merge rank is
// merged, leftmost first, until no pair has a rule.  Pieces that begin with
// '<' never merge.  A piece outside the vocabulary becomes the unknown id.
// The merge order is kept in a heap over a linked list of pieces, so a text
// of n bytes costs O(n log n) rule lookups instead of one scan per merge.
#pragma once

#include "citlali/io/gguf_reader.h"

#include <cstdint>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace citlali::tokenizer {

class Tokenizer {
public:
    void load_from_gguf(const io::GgufFile& gguf);
    // ids of `text`; with add_bos, the BOS id first when the file asks for it
    // (add_bos_token) and the id is not negative.
    std::vector<int32_t> encode(const std::string& text, bool add_bos) const;
    // the vocabulary string of an id; "" out of range
    std::string token_piece(int32_t token_id) const;
    // the bytes an id stands for: "" for control tokens "<|...|>", the byte
    // of "<0xXX>", else the byte-level characters mapped back to bytes (the
    // piece unchanged when one is not a byte-level character)
    std::string decode_token(int32_t token_id) const;
    std::string decode(const std::vector<int32_t>& tokens) const;

    int32_t bos_id() const { return bos_id_; }
    int32_t eos_id() const { return eos_id_; }
    int32_t pad_id() const { return pad_id_; }
    int32_t vocab_size() const { return static_cast<int32_t>(vocab_.size()); }

    // ChatML: "<|im_start|>role\ncontent<|im_end|>\n" per message, then
    // "<|im_start|>assistant\n" with add_generation_prompt.  The file's
    // tokenizer.chat_template is kept but not interpreted (as the reference).
    std::string apply_chat_template(const std::vector<std::pair<std::string, std::string>>& messages,
                                    bool add_generation_prompt) const;

private:
    struct Rule {
        std::string merged;
        int rank = 0;
    };

    // the pieces of a tokenizer that has no vocabulary: every byte as itself
    static std::vector<std::string> raw_byte_pieces();
    // initial piece for one byte of text
    const std::string& byte_piece(uint8_t byte) const;
    std::vector<std::string> initial_pieces(const std::string& text) const;
    const Rule* rule_for(const std::string& left, const std::string& right, std::string& key) const;
    std::string byte_level_to_bytes(const std::string& token) const;

    std::vector<std::string> vocab_;
    std::unordered_map<std::string, int32_t> ids_;
    // keyed "left\nright", the form the reference looks pairs up in
    std::unordered_map<std::string, Rule> rules_;
    std::vector<std::string> byte_pieces_ = raw_byte_pieces();   // [256], chosen at load

    int32_t bos_id_ = 151643;
    int32_t eos_id_ = 151645;
    int32_t pad_id_ = 151643;
    int32_t unk_id_ = 0;
    bool add_bos_token_ = false;
    std::string chat_template_;
};

}  // namespace citlali::tokenizer
