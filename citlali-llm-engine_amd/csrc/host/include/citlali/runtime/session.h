// citlali/runtime/session.h -- prompt in, text out: the reference's
// InferenceSession (include/citlali/runtime/session.h:16-59,
// src/runtime/session.cpp) over the gfx950 QwenModel.
//
// generate_*: encode(prompt, true); the whole prompt plus max_new_tokens must
// stay below the model's max_context; the prompt runs token by token from
// position 0 (logits on its last token only); then up to max_new_tokens
// greedy tokens are emitted, stopping before an EOS id (StopReason::Eos) or
// when the next position reaches max_context (ContextLimit).  Each emitted
// token's decode_token text is appended to the result and passed to
// on_token.  chat_*: the user message joins the history, the ChatML prompt
// of the whole history is generated from, and the reply joins the history.
//
// Unlike the reference's loop (session.cpp:77-96), which waits for every
// token, the greedy tokens are produced `decode_chunk()` at a time by
// QwenModel::decode_greedy (graph replays, no host wait between steps); the
// tokens, text, callbacks and stop reasons are the same.  A chunk may run up
// to chunk - 1 steps past an EOS; those cache positions are rewritten by the
// next prompt, which always starts at position 0.  Remote layers are not
// part of this build: load_model passes its RemoteOptions to
// QwenModel::load, which refuses any that offload layers.
#pragma once

#include "citlali/io/gguf_reader.h"
#include "citlali/model/qwen_model.h"
#include "citlali/tokenizer/tokenizer.h"

#include <cstdint>
#include <functional>
#include <string>
#include <utility>
#include <vector>

namespace citlali::runtime {

struct GenerationOptions {
    uint32_t max_new_tokens = 256;
    uint32_t max_context = 2048;   // not read by generation: the model's max_context binds (as the reference)
    bool chat_template = true;     // read by callers that choose chat_* or generate_*
};

enum class StopReason {
    Eos,
    MaxNewTokens,
    ContextLimit,
};

struct GenerationResult {
    std::string text;
    uint32_t generated_tokens = 0;
    StopReason stop_reason = StopReason::MaxNewTokens;
};

using TokenCallback = std::function<void(const std::string&)>;

class InferenceSession {
public:
    // GGUF file -> tokenizer + model (KeepQuantized when `quantized`), history
    // cleared; a summary line goes to stderr (session.cpp:9-25).  The
    // signature is the reference's (include/citlali/runtime/session.h:39-42).
    void load_model(const std::string& model_path, uint32_t max_context = 2048, bool quantized = false,
                    const remote::RemoteOptions& remote_options = {});

    std::string generate_once(const std::string& prompt, const GenerationOptions& options,
                              const TokenCallback& on_token = {});
    std::string chat_once(const std::string& user_message, const GenerationOptions& options,
                          const TokenCallback& on_token = {});
    GenerationResult generate_once_result(const std::string& prompt, const GenerationOptions& options,
                                          const TokenCallback& on_token = {});
    GenerationResult chat_once_result(const std::string& user_message, const GenerationOptions& options,
                                      const TokenCallback& on_token = {});
    void reset_conversation();

    const model::QwenConfig& config() const { return model_.config(); }
    const tokenizer::Tokenizer& tokenizer() const { return tokenizer_; }
    const std::vector<std::pair<std::string, std::string>>& history() const { return history_; }

    // Greedy tokens per decode_greedy call (>= 1; 1 waits for every token).
    void set_decode_chunk(uint32_t chunk);
    uint32_t decode_chunk() const { return decode_chunk_; }

private:
    GenerationResult generate_from_prompt_text(const std::string& prompt_text, const GenerationOptions& options,
                                               const TokenCallback& on_token);

    io::GgufFile gguf_;
    tokenizer::Tokenizer tokenizer_;
    model::QwenModel model_;
    std::vector<std::pair<std::string, std::string>> history_;
    uint32_t decode_chunk_ = 16;
};

}  // namespace citlali::runtime
