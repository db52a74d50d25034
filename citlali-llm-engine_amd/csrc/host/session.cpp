// InferenceSession (the reference's src/runtime/session.cpp).
//
//   load_model                 session.cpp:9-25 (remote layers refused by QwenModel::load)
//   generate_* / chat_*        session.cpp:27-59
//   generate_from_prompt_text  session.cpp:61-104
#include "citlali/runtime/session.h"

#include "citlali/common.h"

#include <algorithm>
#include <iostream>

namespace citlali::runtime {

void InferenceSession::load_model(const std::string& model_path, uint32_t max_context, bool quantized,
                                  const remote::RemoteOptions& remote_options) {
    std::cerr << "Reading GGUF: " << model_path << std::endl;
    gguf_.load(model_path);
    tokenizer_.load_from_gguf(gguf_);
    model_.load(gguf_, max_context, quantized, remote_options);
    history_.clear();
    const model::QwenConfig& c = config();
    std::cerr << "Model loaded. vocab=" << c.vocab_size << " layers=" << c.block_count
              << " hidden=" << c.embedding_length << " heads=" << c.head_count << " kv_heads=" << c.head_count_kv
              << " head_dim=" << c.head_dim << " ctx=" << model_.max_context() << "\n";
}

std::string InferenceSession::generate_once(const std::string& prompt, const GenerationOptions& options,
                                            const TokenCallback& on_token) {
    return generate_once_result(prompt, options, on_token).text;
}

std::string InferenceSession::chat_once(const std::string& user_message, const GenerationOptions& options,
                                        const TokenCallback& on_token) {
    return chat_once_result(user_message, options, on_token).text;
}

GenerationResult InferenceSession::generate_once_result(const std::string& prompt, const GenerationOptions& options,
                                                        const TokenCallback& on_token) {
    return generate_from_prompt_text(prompt, options, on_token);
}

GenerationResult InferenceSession::chat_once_result(const std::string& user_message, const GenerationOptions& options,
                                                    const TokenCallback& on_token) {
    history_.emplace_back("user", user_message);
    const std::string prompt = tokenizer_.apply_chat_template(history_, true);
    GenerationResult result = generate_from_prompt_text(prompt, options, on_token);
    history_.emplace_back("assistant", result.text);
    return result;
}

void InferenceSession::reset_conversation() {
    history_.clear();
}

void InferenceSession::set_decode_chunk(uint32_t chunk) {
    require(chunk >= 1, "decode chunk must be at least 1");
    decode_chunk_ = chunk;
}

GenerationResult InferenceSession::generate_from_prompt_text(const std::string& prompt_text,
                                                             const GenerationOptions& options,
                                                             const TokenCallback& on_token) {
    const std::vector<int32_t> prompt = tokenizer_.encode(prompt_text, true);
    require(!prompt.empty(), "prompt produced no tokens");
    const uint32_t max_context = model_.max_context();
    require(prompt.size() + options.max_new_tokens < max_context, "prompt plus generation exceeds max_context");

    uint32_t position = 0;
    int32_t next = 0;
    for (size_t i = 0; i < prompt.size(); ++i) next = model_.forward_token(prompt[i], position++, i + 1 == prompt.size());

    // `ahead` holds greedy tokens already computed on the device for the
    // positions after `position`, oldest first.
    GenerationResult result;
    std::vector<int32_t> ahead;
    size_t used = 0;
    for (uint32_t i = 0; i < options.max_new_tokens; ++i) {
        if (next == tokenizer_.eos_id()) {
            result.stop_reason = StopReason::Eos;
            break;
        }
        const std::string piece = tokenizer_.decode_token(next);
        result.text += piece;
        ++result.generated_tokens;
        if (on_token) on_token(piece);

        if (used == ahead.size()) {
            // as many steps as the remaining budget may still ask for
            const uint32_t steps = std::min({decode_chunk_, options.max_new_tokens - i, max_context - position});
            ahead = model_.decode_greedy(next, position, steps);
            used = 0;
        }
        next = ahead[used++];
        ++position;
        if (position >= max_context) {
            result.stop_reason = StopReason::ContextLimit;
            break;
        }
    }
    model_.synchronize();
    return result;
}

}  // namespace citlali::runtime
