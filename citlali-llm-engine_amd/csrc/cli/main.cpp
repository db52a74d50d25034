// citlali_cli -- text in, text out over InferenceSession: the reference's
// command line (src/cli/main.cpp:192-355) with its flags and output lines.
//
//   citlali_cli --model M.gguf --prompt TEXT [--max-new-tokens N] [--ctx N]
//               [--no-chat-template] [--quantized] [--decode-chunk N]
//   citlali_cli --model M.gguf --interactive [--quantized]
//   citlali_cli --model M.gguf --info                     (no weights loaded)
//   citlali_cli --model M.gguf --prompt TEXT --tokens [--no-chat-template]
//
// Generated text streams to stdout piece by piece, then
// "[stats] tokens=N time=S.SSSs speed=X.XX tok/s stop=REASON".  The
// remote-offload flags of the reference (--remote, --remote-transport,
// --remote-backend, --offload) are refused: remote layers are not part of
// this build.  --decode-chunk sets InferenceSession::set_decode_chunk.
#include "citlali/common.h"
#include "citlali/compute/common/dtype.h"
#include "citlali/io/gguf_reader.h"
#include "citlali/model/qwen_config.h"
#include "citlali/runtime/session.h"
#include "citlali/tokenizer/tokenizer.h"

#include <chrono>
#include <cstdio>
#include <exception>
#include <iostream>
#include <map>
#include <string>
#include <vector>

namespace {

struct Args {
    std::string model, prompt;
    uint32_t max_new_tokens = 256, max_context = 2048, decode_chunk = 16;
    bool chat = true, interactive = false, info = false, tokens = false, quantized = false, help = false;
};

const char* kUsage =
    "Citlali-LLM-Engine (MI355X)\n"
    "\n"
    "Usage:\n"
    "  citlali_cli --model <path.gguf> --prompt <text> [--max-new-tokens N] [--ctx N]\n"
    "  citlali_cli --model <path.gguf> --interactive\n"
    "  citlali_cli --model <path.gguf> --info\n"
    "  citlali_cli --model <path.gguf> --prompt <text> --tokens [--no-chat-template]\n"
    "\n"
    "Options:\n"
    "  --model <path>          GGUF model path\n"
    "  --prompt <text>         Prompt or user message\n"
    "  --max-new-tokens <N>    Tokens to generate, default 256\n"
    "  --ctx <N>               Max context, default 2048\n"
    "  --no-chat-template      Treat --prompt as raw text\n"
    "  --interactive           Multi-turn chat (/reset clears the history, /exit quits)\n"
    "  --info                  Print GGUF/config summary without loading weights\n"
    "  --tokens                Print prompt tokenization without loading weights\n"
    "  --quantized             Keep Q4_K/Q6_K weights quantized on the device\n"
    "  --decode-chunk <N>      Greedy tokens per device round trip, default 16\n";

uint32_t to_u32(const std::string& flag, const std::string& v) {
    size_t used = 0;
    unsigned long x = 0;
    try {
        x = std::stoul(v, &used);
    } catch (const std::exception&) {
        used = 0;
    }
    if (used != v.size() || v.empty() || x > 0xffffffffUL) throw citlali::Error(flag + " needs a number, got '" + v + "'");
    return static_cast<uint32_t>(x);
}

Args parse(int argc, char** argv) {
    Args a;
    for (int i = 1; i < argc; ++i) {
        const std::string f = argv[i];
        const auto value = [&]() -> std::string {
            if (i + 1 >= argc) throw citlali::Error("missing value for " + f);
            return argv[++i];
        };
        if (f == "--model") a.model = value();
        else if (f == "--prompt") a.prompt = value();
        else if (f == "--max-new-tokens") a.max_new_tokens = to_u32(f, value());
        else if (f == "--ctx" || f == "--context") a.max_context = to_u32(f, value());
        else if (f == "--decode-chunk") {
            a.decode_chunk = to_u32(f, value());
            if (a.decode_chunk < 1) throw citlali::Error("--decode-chunk must be at least 1");   // before any load
        }
        else if (f == "--no-chat-template") a.chat = false;
        else if (f == "--interactive") a.interactive = true;
        else if (f == "--info") a.info = true;
        else if (f == "--tokens") a.tokens = true;
        else if (f == "--quantized") a.quantized = true;
        else if (f == "--help" || f == "-h") a.help = true;
        else if (f == "--remote" || f == "--remote-transport" || f == "--remote-backend" || f == "--offload")
            throw citlali::Error(f + ": remote layer offload is not part of this build");
        else throw citlali::Error("unknown argument: " + f);
    }
    return a;
}

// Control bytes, quotes and backslashes as C escapes, so a token listing
// stays on one line.
std::string escaped(const std::string& s) {
    std::string out;
    for (unsigned char c : s) {
        switch (c) {
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            default:
                if (c < 0x20 || c == 0x7f) {
                    char b[8];
                    std::snprintf(b, sizeof b, "\\x%02X", c);
                    out += b;
                } else {
                    out += static_cast<char>(c);
                }
        }
    }
    return out;
}

const char* stop_name(citlali::runtime::StopReason r) {
    switch (r) {
        case citlali::runtime::StopReason::Eos: return "eos";
        case citlali::runtime::StopReason::MaxNewTokens: return "max_new_tokens";
        case citlali::runtime::StopReason::ContextLimit: return "context_limit";
    }
    return "unknown";
}

void print_stats(const citlali::runtime::GenerationResult& r, double seconds) {
    const double speed = seconds > 0 ? r.generated_tokens / seconds : 0.0;
    std::printf("\n[stats] tokens=%u time=%.3fs speed=%.2f tok/s stop=%s\n", r.generated_tokens, seconds, speed,
                stop_name(r.stop_reason));
    std::fflush(stdout);
}

void print_info(const std::string& path) {
    citlali::io::GgufFile g;
    g.load(path);
    const auto c = citlali::model::QwenConfig::from_gguf(g);
    std::map<citlali::compute::GgufTensorType, size_t> types;
    uint64_t bytes = 0;
    for (const auto& t : g.tensors()) {
        ++types[t.type];
        bytes += t.nbytes;
    }
    std::cout << "model: " << path << "\n"
              << "architecture: " << c.architecture << "\n"
              << "vocab: " << c.vocab_size << "\n"
              << "layers: " << c.block_count << "\n"
              << "hidden: " << c.embedding_length << "\n"
              << "ffn: " << c.feed_forward_length << "\n"
              << "heads: " << c.head_count << "\n"
              << "kv_heads: " << c.head_count_kv << "\n"
              << "head_dim: " << c.head_dim << "\n"
              << "value_dim: " << c.value_dim << "\n"
              << "context: " << c.context_length << "\n"
              << "rope_theta: " << c.rope_theta << "\n"
              << "rms_norm_eps: " << c.rms_norm_eps << "\n"
              << "tensors: " << g.tensors().size() << "\n"
              << "raw tensor bytes: " << bytes << "\n"
              << "tensor types:\n";
    for (const auto& [type, n] : types) std::cout << "  " << citlali::compute::to_string(type) << ": " << n << "\n";
}

void print_tokens(const std::string& path, const std::string& prompt, bool chat) {
    citlali::io::GgufFile g;
    g.load(path);
    citlali::tokenizer::Tokenizer t;
    t.load_from_gguf(g);
    const std::string text = chat ? t.apply_chat_template({{"user", prompt}}, true) : prompt;
    const std::vector<int32_t> ids = t.encode(text, true);
    std::cout << "prompt_text: " << text << "\n"
              << "token_count: " << ids.size() << "\n";
    for (size_t i = 0; i < ids.size(); ++i)
        std::cout << i << "\t" << ids[i] << "\tpiece=\"" << escaped(t.token_piece(ids[i])) << "\"\tdecoded=\""
                  << escaped(t.decode_token(ids[i])) << "\"\n";
}

int run(int argc, char** argv) {
    const Args a = parse(argc, argv);
    if (a.help) {
        std::cout << kUsage;
        return 0;
    }
    if (a.model.empty()) {
        std::cout << kUsage;
        return 1;
    }
    if (a.info) {
        print_info(a.model);
        return 0;
    }
    if (a.tokens) {
        if (a.prompt.empty()) {
            std::cout << kUsage;
            return 1;
        }
        print_tokens(a.model, a.prompt, a.chat);
        return 0;
    }
    if (!a.interactive && a.prompt.empty()) {
        std::cout << kUsage;
        return 1;
    }

    citlali::runtime::GenerationOptions opt;
    opt.max_new_tokens = a.max_new_tokens;
    opt.max_context = a.max_context;
    opt.chat_template = a.chat;
    citlali::runtime::InferenceSession session;
    session.load_model(a.model, a.max_context, a.quantized);
    session.set_decode_chunk(a.decode_chunk);
    const auto emit = [](const std::string& piece) {
        std::fwrite(piece.data(), 1, piece.size(), stdout);
        std::fflush(stdout);
    };
    const auto timed = [&](auto&& generate) {
        const auto t0 = std::chrono::steady_clock::now();
        const citlali::runtime::GenerationResult r = generate();
        print_stats(r, std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
    };

    if (a.interactive) {
        std::cout << "Citlali chat. Type /exit to quit, /reset to clear history.\n";
        std::string line;
        for (;;) {
            std::cout << "\n<user> " << std::flush;
            if (!std::getline(std::cin, line) || line == "/exit" || line == "/quit") break;
            if (line == "/reset") {
                session.reset_conversation();
                std::cout << "history cleared\n";
                continue;
            }
            std::cout << "<assistant> " << std::flush;
            timed([&] { return session.chat_once_result(line, opt, emit); });
        }
        return 0;
    }
    if (a.chat)
        timed([&] { return session.chat_once_result(a.prompt, opt, emit); });
    else
        timed([&] { return session.generate_once_result(a.prompt, opt, emit); });
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception& e) {
        std::cerr << "error: " << e.what() << "\n";
        return 1;
    }
}
