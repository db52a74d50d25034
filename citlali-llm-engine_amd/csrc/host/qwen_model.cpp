// qwen_model.cpp -- QwenModel::forward_token over the gfx950 launchers
// (reference: src/model/qwen_model.cpp:15-33, 39-213, 239-465).
#include "citlali/model/qwen_model.h"

#include "citlali/common.h"
#include "citlali/compute/hip/kernels.h"

#include <algorithm>
#include <limits>
#include <string>

namespace citlali::model {
namespace {

// Decode steps per graph replay in decode_greedy.  A replay boundary costs
// about 5 us on MI355X: config 5 decoded 622.2 tok/s with one step per
// replay, 623.2-623.4 with 2, 624.2 with 4, 624.4-624.5 with 16 (the same
// tokens each time); 8 keeps each graph at a few thousand nodes.
constexpr uint32_t kGraphSteps = 8;

int as_int(uint64_t value, const std::string& label) {
    require(value <= static_cast<uint64_t>(std::numeric_limits<int>::max()),
            label + " is too large for this minimal kernel path");
    return static_cast<int>(value);
}

void require_shape(const WeightHandle& weight, uint64_t cols, uint64_t rows) {
    require(weight.cols() == cols && weight.rows() == rows,
            "unexpected tensor shape for " + weight.name + ": got [" + std::to_string(weight.cols()) + ", " +
                std::to_string(weight.rows()) + "], expected [" + std::to_string(cols) + ", " +
                std::to_string(rows) + "]");
}

void add_bias_if_present(const WeightHandle& bias, const compute::DeviceBufferPtr& target, uint64_t elements) {
    if (!bias.buffer) return;
    require_shape(bias, elements, 1);
    compute::launch_add_bias_inplace(target->half_data(), bias.device_half_data(),
                                     as_int(elements, bias.name + " elements"));
}

}  // namespace

void QwenModel::load(const io::GgufFile& gguf, uint32_t max_context, bool quantized,
                     const remote::RemoteOptions& remote_options) {
    const QwenConfig config = QwenConfig::from_gguf(gguf);
    if (remote_options.enabled()) {
        for (const uint32_t layer_index : remote_options.layers)
            require(layer_index < config.block_count,
                    "remote layer index is out of range: " + std::to_string(layer_index));
    }
    require(remote_options.layers.empty(),
            "remote layer offload is not supported by this build (" + std::to_string(remote_options.layers.size()) +
                " layer(s) requested" + (remote_options.endpoint.empty() ? ", no endpoint" : " at " + remote_options.endpoint) +
                "): load with no remote layers");
    const WeightLoader loader(gguf, quantized ? WeightLoadPolicy::KeepQuantized : WeightLoadPolicy::DequantizeToFp16);
    const auto blk = [](uint32_t i, const char* suffix) { return "blk." + std::to_string(i) + "." + suffix; };
    QwenWeights w;
    w.token_embedding = loader.load_required("token_embd.weight");
    w.output_norm = loader.load_required("output_norm.weight");
    w.output_weight = loader.load_optional("output.weight");   // absent: tied to token_embd
    w.layers.resize(config.block_count);
    for (uint32_t i = 0; i < config.block_count; ++i) {
        QwenLayerWeights& l = w.layers[i];
        l.attn_norm = loader.load_required(blk(i, "attn_norm.weight"));
        l.attn_q = loader.load_required(blk(i, "attn_q.weight"));
        l.attn_q_bias = loader.load_optional(blk(i, "attn_q.bias"));
        l.attn_k = loader.load_required(blk(i, "attn_k.weight"));
        l.attn_k_bias = loader.load_optional(blk(i, "attn_k.bias"));
        l.attn_v = loader.load_required(blk(i, "attn_v.weight"));
        l.attn_v_bias = loader.load_optional(blk(i, "attn_v.bias"));
        l.attn_o = loader.load_required(blk(i, "attn_output.weight"));
        l.attn_o_bias = loader.load_optional(blk(i, "attn_output.bias"));
        l.attn_q_norm = loader.load_optional(blk(i, "attn_q_norm.weight"));
        l.attn_k_norm = loader.load_optional(blk(i, "attn_k_norm.weight"));
        l.ffn_norm = loader.load_required(blk(i, "ffn_norm.weight"));
        l.ffn_gate = loader.load_required(blk(i, "ffn_gate.weight"));
        l.ffn_gate_bias = loader.load_optional(blk(i, "ffn_gate.bias"));
        l.ffn_up = loader.load_required(blk(i, "ffn_up.weight"));
        l.ffn_up_bias = loader.load_optional(blk(i, "ffn_up.bias"));
        l.ffn_down = loader.load_required(blk(i, "ffn_down.weight"));
        l.ffn_down_bias = loader.load_optional(blk(i, "ffn_down.bias"));
    }
    load(config, std::move(w), max_context);
}

void QwenModel::load(const QwenConfig& config, QwenWeights weights, uint32_t max_context) {
    config_ = config;
    max_context_ = max_context == 0 ? std::min<uint32_t>(config_.context_length, 2048)
                                    : std::min(max_context, config_.context_length);
    require(max_context_ > 0, "max_context must be positive");
    require(config_.head_count_kv > 0 && config_.head_count % config_.head_count_kv == 0,
            "attention head_count must be divisible by head_count_kv");
    linear_backend_.reset();   // set again only once everything below succeeded
    release_graphs();          // they hold the previous buffers

    token_embedding_ = std::move(weights.token_embedding);
    output_norm_ = std::move(weights.output_norm);
    output_weight_ = std::move(weights.output_weight);
    if (!output_weight_.buffer) output_weight_ = token_embedding_;
    layers_ = std::move(weights.layers);

    const uint64_t hidden = config_.embedding_length;
    const uint64_t q_size = static_cast<uint64_t>(config_.head_count) * config_.head_dim;
    const uint64_t kv_size = static_cast<uint64_t>(config_.head_count_kv) * config_.head_dim;
    const uint64_t ff = config_.feed_forward_length;
    require(layers_.size() == config_.block_count, "expected " + std::to_string(config_.block_count) +
                                                       " layers, got " + std::to_string(layers_.size()));
    require_shape(token_embedding_, hidden, config_.vocab_size);
    require_shape(output_norm_, hidden, 1);
    require_shape(output_weight_, hidden, config_.vocab_size);
    for (QwenLayerWeights& layer : layers_) {
        require_shape(layer.attn_norm, hidden, 1);
        require_shape(layer.attn_q, hidden, q_size);
        if (layer.attn_q_bias.buffer) require_shape(layer.attn_q_bias, q_size, 1);
        require_shape(layer.attn_k, hidden, kv_size);
        if (layer.attn_k_bias.buffer) require_shape(layer.attn_k_bias, kv_size, 1);
        require_shape(layer.attn_v, hidden, kv_size);
        if (layer.attn_v_bias.buffer) require_shape(layer.attn_v_bias, kv_size, 1);
        require_shape(layer.attn_o, q_size, hidden);
        if (layer.attn_o_bias.buffer) require_shape(layer.attn_o_bias, hidden, 1);
        if (layer.attn_q_norm.buffer) require_shape(layer.attn_q_norm, config_.head_dim, 1);
        if (layer.attn_k_norm.buffer) require_shape(layer.attn_k_norm, config_.head_dim, 1);
        require_shape(layer.ffn_norm, hidden, 1);
        require_shape(layer.ffn_gate, hidden, ff);
        if (layer.ffn_gate_bias.buffer) require_shape(layer.ffn_gate_bias, ff, 1);
        require_shape(layer.ffn_up, hidden, ff);
        if (layer.ffn_up_bias.buffer) require_shape(layer.ffn_up_bias, ff, 1);
        require_shape(layer.ffn_down, ff, hidden);
        if (layer.ffn_down_bias.buffer) require_shape(layer.ffn_down_bias, hidden, 1);
        layer.k_cache = compute::make_device_half_buffer(static_cast<size_t>(max_context_) * kv_size);
        layer.v_cache = compute::make_device_half_buffer(static_cast<size_t>(max_context_) * kv_size);
    }
    allocate_runtime_buffers();
    linear_backend_ = make_fp16_linear_backend();
}

void QwenModel::allocate_runtime_buffers() {
    const size_t hidden = config_.embedding_length;
    const size_t q = static_cast<size_t>(config_.head_count) * config_.head_dim;
    const size_t kv = static_cast<size_t>(config_.head_count_kv) * config_.head_dim;
    const size_t ff = config_.feed_forward_length;
    x_ = compute::make_device_half_buffer(hidden);
    x_alt_ = compute::make_device_half_buffer(hidden);   // the residual stream alternates between the two
    norm_ = compute::make_device_half_buffer(hidden);
    q_ = compute::make_device_half_buffer(q);
    k_ = compute::make_device_half_buffer(kv);
    v_ = compute::make_device_half_buffer(kv);
    attn_out_ = compute::make_device_half_buffer(q);
    attn_proj_ = compute::make_device_half_buffer(hidden);
    gate_ = compute::make_device_half_buffer(ff);
    up_ = compute::make_device_half_buffer(ff);
    ff_act_ = compute::make_device_half_buffer(ff);
    ff_out_ = compute::make_device_half_buffer(hidden);
    logits_ = compute::make_device_buffer(static_cast<size_t>(config_.vocab_size) * sizeof(float));
    // the reference's heads x max_context floats, or more: the attention
    // split partials of every plan up to max_context (each bucket's plan and
    // max_context's own), so no step -- a captured one included -- needs the
    // library's own workspace
    const size_t reference_scores = static_cast<size_t>(config_.head_count) * max_context_ * sizeof(float);
    scores_ = compute::make_device_buffer(std::max(
        reference_scores,
        compute::attention_workspace_bytes(static_cast<int>(max_context_), static_cast<int>(config_.head_count),
                                           static_cast<int>(config_.head_count_kv),
                                           static_cast<int>(config_.head_dim))));
    next_token_ = compute::make_device_buffer(sizeof(int32_t));
    state_ = compute::make_device_buffer(4 * sizeof(int32_t));
    tokens_ = compute::make_device_buffer(static_cast<size_t>(max_context_) * sizeof(int32_t));
}

namespace {
// A weight as an operand of the grouped / fused GEMV launches: a Q4_K / Q6_K
// device tensor as its raw blocks, an fp16 device tensor as GGUF type F16
// over its rows.  False for anything else or a buffer shorter than the
// tensor (the separate launch then reports it).
bool fused_operand(const WeightHandle& w, compute::GgufTensorType* type, const uint8_t** data) {
    if (!w.buffer) return false;
    const uint64_t n = w.cols() * w.rows();
    if (w.storage_kind == compute::WeightStorageKind::QuantizedDevice) {
        if (w.buffer->bytes() < compute::gguf_tensor_nbytes(w.gguf_type, n)) return false;
        *type = w.gguf_type;
        *data = w.device_quantized_data();
        return true;
    }
    if (w.storage_kind == compute::WeightStorageKind::Fp16Device) {
        if (w.buffer->bytes() < n * 2) return false;
        *type = compute::GgufTensorType::F16;
        *data = reinterpret_cast<const uint8_t*>(w.device_half_data());
        return true;
    }
    return false;
}
}  // namespace

// attn_q, attn_k and attn_v in one launch when all three are Q4_K/Q6_K
// device tensors or all three fp16 ones (the separate GEMVs' results bit for
// bit), reading `input` or, with `norm`, the residual add + RMSNorm of it;
// false, nothing launched, otherwise -- then LinearBackend::forward runs
// (and reports what it rejects).  The bias adds that follow are independent
// of order.
bool QwenModel::launch_qkv_grouped(const QwenLayerWeights& layer, int hidden, const uint16_t* input,
                                   const compute::NormInput* norm) {
    const WeightHandle* w[3] = {&layer.attn_q, &layer.attn_k, &layer.attn_v};
    const compute::DeviceBufferPtr* out[3] = {&q_, &k_, &v_};
    compute::GgufTensorType types[3];
    const uint8_t* weights[3];
    uint16_t* outputs[3];
    int rows[3];
    for (int i = 0; i < 3; ++i) {
        if (!fused_operand(*w[i], &types[i], &weights[i])) return false;
        if ((types[i] == compute::GgufTensorType::F16) != (types[0] == compute::GgufTensorType::F16)) return false;
        outputs[i] = (*out[i])->half_data();
        rows[i] = as_int(w[i]->rows(), w[i]->name + " rows");
    }
    if (norm) return compute::launch_matvec_group_norm(3, types, weights, input, *norm, outputs, rows, hidden);
    return compute::launch_matvec_group(3, types, weights, input, outputs, rows, hidden);
}

int32_t QwenModel::forward_token(int32_t token_id, uint32_t position, bool compute_logits) {
    require(linear_backend_ != nullptr, "model is not loaded");
    require(position < max_context_, "position exceeds max_context");
    require(token_id >= 0 && token_id < static_cast<int32_t>(config_.vocab_size), "token id out of vocab range");
    enqueue_token(token_id, static_cast<int>(position), nullptr, 0, compute_logits);
    if (!compute_logits) return -1;
    return sample_greedy_from_logits();
}

// The launches of one token.  With `state` (device {token, position, step,
// 0}) the token and position are read from there, attention is planned for
// `plan_length`, and the greedy pick advances the state instead of being
// copied back -- the same kernels and arguments otherwise, so a captured
// step replays what forward_token computes at every position whose plan
// length is plan_length.
void QwenModel::enqueue_token(int32_t token_id, int pos, int32_t* state, int plan_length, bool compute_logits) {
    const int hidden = as_int(config_.embedding_length, "hidden size");
    const int head_dim = as_int(config_.head_dim, "head_dim");
    const int heads = as_int(config_.head_count, "head_count");
    const int kv_heads = as_int(config_.head_count_kv, "head_count_kv");
    const int ff = as_int(config_.feed_forward_length, "feed_forward_length");
    const int vocab = as_int(config_.vocab_size, "vocab_size");
    const int32_t* state_position = state ? state + 1 : nullptr;

    if (token_embedding_.storage_kind == compute::WeightStorageKind::QuantizedDevice) {
        if (token_embedding_.gguf_type != compute::GgufTensorType::Q6_K)
            throw Error("unsupported quantized embedding type");
        if (state)
            compute::launch_embed_q6k_at(token_embedding_.device_quantized_data(), state, vocab, x_->half_data(),
                                         hidden);
        else
            compute::launch_embed_q6k(token_embedding_.device_quantized_data(), token_id, x_->half_data(), hidden);
    } else {
        if (state)
            compute::launch_embed_at(token_embedding_.device_half_data(), state, vocab, x_->half_data(), hidden);
        else
            compute::launch_embed(token_embedding_.device_half_data(), token_id, x_->half_data(), hidden);
    }

    // The reference's per-layer sequence.  Its launches are grouped or fused
    // where a kernel gives the same results bit for bit: attn_q/k/v in one
    // launch; each residual add + RMSNorm inside the GEMV launch that reads
    // the normed vector (its workgroups form the input themselves, and the
    // sum goes to the other residual buffer); the q/k head norms with RoPE
    // and the KV store; gate/up with SwiGLU.  Where no such kernel covers a
    // shape, the add + norm runs as its own launch into norm_.
    const float eps = config_.rms_norm_eps;
    uint16_t* xr[2] = {x_->half_data(), x_alt_->half_data()};
    int cur = 0;                          // xr[cur] is the residual stream
    const uint16_t* pending = nullptr;    // ffn_down output not yet added to it
    auto prologue = [&](const WeightHandle& w, const uint16_t* delta) {
        return compute::NormInput{delta, w.device_half_data(), delta ? xr[1 - cur] : nullptr, eps};
    };
    auto norm_into_buffer = [&](const WeightHandle& w, const uint16_t* delta) {
        if (delta)
            compute::launch_add_rms_norm(xr[cur], delta, w.device_half_data(), norm_->half_data(), hidden, eps);
        else
            compute::launch_rms_norm(xr[cur], w.device_half_data(), norm_->half_data(), hidden, eps);
    };

    for (size_t li = 0; li < layers_.size(); ++li) {
        QwenLayerWeights& layer = layers_[li];
        const compute::NormInput attn_in = prologue(layer.attn_norm, pending);
        if (launch_qkv_grouped(layer, hidden, xr[cur], &attn_in)) {
            if (pending) cur ^= 1;
        } else {
            norm_into_buffer(layer.attn_norm, pending);
            if (!launch_qkv_grouped(layer, hidden, norm_->half_data(), nullptr)) {
                linear_backend_->forward(layer.attn_q, norm_, q_);
                linear_backend_->forward(layer.attn_k, norm_, k_);
                linear_backend_->forward(layer.attn_v, norm_, v_);
            }
        }
        pending = nullptr;
        add_bias_if_present(layer.attn_q_bias, q_, static_cast<uint64_t>(heads) * head_dim);
        add_bias_if_present(layer.attn_k_bias, k_, static_cast<uint64_t>(kv_heads) * head_dim);
        add_bias_if_present(layer.attn_v_bias, v_, static_cast<uint64_t>(kv_heads) * head_dim);
        const uint16_t* q_norm = layer.attn_q_norm.buffer ? layer.attn_q_norm.device_half_data() : nullptr;
        const uint16_t* k_norm = layer.attn_k_norm.buffer ? layer.attn_k_norm.device_half_data() : nullptr;
        // q/k norm + RoPE + KV store inside the attention launch where a
        // fused kernel covers the shape (the same bits as the two launches)
        if (compute::launch_qk_norm_rope_store_attention(
                q_->half_data(), k_->half_data(), v_->half_data(), q_norm, k_norm, heads, kv_heads, head_dim,
                state ? 0 : pos, state ? state_position : nullptr, state ? plan_length : 0,
                static_cast<int>(max_context_), config_.rope_theta, eps, layer.k_cache->half_data(),
                layer.v_cache->half_data(), static_cast<float*>(scores_->data()), scores_->bytes(),
                attn_out_->half_data())) {
        } else if (state) {
            compute::launch_qk_norm_rope_store_at(q_->half_data(), k_->half_data(), v_->half_data(), q_norm, k_norm,
                                                  heads, kv_heads, head_dim, state_position,
                                                  static_cast<int>(max_context_), config_.rope_theta, eps,
                                                  layer.k_cache->half_data(), layer.v_cache->half_data());
            compute::launch_attention_at(q_->half_data(), layer.k_cache->half_data(), layer.v_cache->half_data(),
                                         state_position, plan_length, static_cast<float*>(scores_->data()),
                                         scores_->bytes(), attn_out_->half_data(), heads, kv_heads, head_dim);
        } else {
            compute::launch_qk_norm_rope_store(q_->half_data(), k_->half_data(), v_->half_data(), q_norm, k_norm,
                                               heads, kv_heads, head_dim, pos, config_.rope_theta, eps,
                                               layer.k_cache->half_data(), layer.v_cache->half_data());
            compute::launch_attention(q_->half_data(), layer.k_cache->half_data(), layer.v_cache->half_data(),
                                      static_cast<float*>(scores_->data()), attn_out_->half_data(), pos,
                                      static_cast<int>(max_context_), heads, kv_heads, head_dim);
        }
        linear_backend_->forward(layer.attn_o, attn_out_, attn_proj_);
        add_bias_if_present(layer.attn_o_bias, attn_proj_, hidden);

        compute::GgufTensorType gate_type{}, up_type{};
        const uint8_t *gate_w = nullptr, *up_w = nullptr;
        const bool fuse_ffn = fused_operand(layer.ffn_gate, &gate_type, &gate_w) &&
                              fused_operand(layer.ffn_up, &up_type, &up_w) && gate_type == up_type &&
                              !layer.ffn_gate_bias.buffer && !layer.ffn_up_bias.buffer;
        const compute::NormInput ffn_in = prologue(layer.ffn_norm, attn_proj_->half_data());
        if (fuse_ffn && compute::launch_matvec_gate_up_swiglu_norm(gate_type, gate_w, up_w, xr[cur], ffn_in,
                                                                   ff_act_->half_data(), hidden, ff)) {
            cur ^= 1;
        } else {
            norm_into_buffer(layer.ffn_norm, attn_proj_->half_data());
            if (!fuse_ffn || !compute::launch_matvec_gate_up_swiglu(gate_type, gate_w, up_w, norm_->half_data(),
                                                                    ff_act_->half_data(), hidden, ff)) {
                linear_backend_->forward(layer.ffn_gate, norm_, gate_);
                add_bias_if_present(layer.ffn_gate_bias, gate_, ff);
                linear_backend_->forward(layer.ffn_up, norm_, up_);
                add_bias_if_present(layer.ffn_up_bias, up_, ff);
                compute::launch_swiglu(gate_->half_data(), up_->half_data(), ff_act_->half_data(), ff);
            }
        }
        linear_backend_->forward(layer.ffn_down, ff_act_, ff_out_);
        add_bias_if_present(layer.ffn_down_bias, ff_out_, hidden);
        pending = ff_out_->half_data();
    }
    // without logits nothing reads the last residual add
    if (!compute_logits) return;

    float* logits = static_cast<float*>(logits_->data());
    const compute::NormInput out_in = prologue(output_norm_, pending);
    if (output_weight_.storage_kind == compute::WeightStorageKind::QuantizedDevice) {
        if (output_weight_.gguf_type != compute::GgufTensorType::Q6_K)
            throw Error("unsupported quantized output weight type: " + compute::to_string(output_weight_.gguf_type));
        if (!compute::launch_matvec_norm(output_weight_.gguf_type, output_weight_.device_quantized_data(), xr[cur],
                                         out_in, logits, true, hidden, vocab)) {
            norm_into_buffer(output_norm_, pending);
            compute::launch_matvec_q6k_to_float(output_weight_.device_quantized_data(), norm_->half_data(), logits,
                                                hidden, vocab);
        }
    } else {
        compute::GgufTensorType type{};
        const uint8_t* w = nullptr;
        if (!fused_operand(output_weight_, &type, &w) ||
            !compute::launch_matvec_norm(type, w, xr[cur], out_in, logits, true, hidden, vocab)) {
            norm_into_buffer(output_norm_, pending);
            compute::launch_matvec_fp16_to_float(output_weight_.device_half_data(), norm_->half_data(), logits,
                                                 hidden, vocab);
        }
    }
    if (state)
        compute::launch_argmax_advance(static_cast<const float*>(logits_->data()), vocab, state,
                                       static_cast<int32_t*>(tokens_->data()), static_cast<int>(max_context_));
}

namespace {

// Runs the library on `stream` for its lifetime: the work queued on the
// previous stream is finished first, and that stream is restored (after the
// new one has drained) at the end.
class StreamSwitch {
public:
    explicit StreamSwitch(void* stream) : previous_(compute::current_stream()) {
        compute::synchronize();
        compute::set_stream(stream);
    }
    ~StreamSwitch() {
        try {
            compute::synchronize();
        } catch (...) {
        }
        try {
            compute::set_stream(previous_);
        } catch (...) {
        }
    }
    StreamSwitch(const StreamSwitch&) = delete;
    StreamSwitch& operator=(const StreamSwitch&) = delete;

private:
    void* previous_;
};

}  // namespace

std::vector<int32_t> QwenModel::decode_greedy(int32_t token_id, uint32_t position, uint32_t steps) {
    require(linear_backend_ != nullptr, "model is not loaded");
    require(token_id >= 0 && token_id < static_cast<int32_t>(config_.vocab_size), "token id out of vocab range");
    require(position < max_context_ && steps <= max_context_ - position, "position + steps exceeds max_context");
    std::vector<int32_t> out(steps);
    if (steps == 0) return out;
    if (!stream_) stream_ = compute::create_stream();
    StreamSwitch on_model_stream(stream_);

    const int32_t init[4] = {token_id, static_cast<int32_t>(position), 0, 0};
    state_->copy_from_host(init, sizeof(init));
    uint32_t pos = position, left = steps;
    while (left > 0) {
        // positions pos .. plan - 1 share one attention plan, hence one
        // graph: kGraphSteps steps per replay, the rest one step per replay
        const int plan = compute::attention_plan_length(static_cast<int>(pos) + 1, static_cast<int>(max_context_));
        const uint32_t n = std::min<uint32_t>(left, static_cast<uint32_t>(plan) - pos);
        uint32_t i = 0;
        if (n >= kGraphSteps) {
            void* graph = step_graph(plan, static_cast<int>(kGraphSteps));
            for (; i + kGraphSteps <= n; i += kGraphSteps) compute::graph_launch(graph);
        }
        if (i < n) {
            void* graph = step_graph(plan, 1);
            for (; i < n; ++i) compute::graph_launch(graph);
        }
        pos += n;
        left -= n;
    }
    tokens_->copy_to_host(out.data(), out.size() * sizeof(int32_t));   // waits for the stream
    return out;
}

// `steps` captured decode steps for one attention plan length (made on
// first use): each step reads its token and position from the device state
// and advances it, so one replay decodes `steps` tokens.
void* QwenModel::step_graph(int plan_length, int steps) {
    for (const auto& g : graphs_)
        if (g.plan_length == plan_length && g.steps == steps) return g.graph;
    compute::graph_begin();
    try {
        for (int s = 0; s < steps; ++s)
            enqueue_token(0, 0, static_cast<int32_t*>(state_->data()), plan_length, true);
    } catch (...) {
        try {
            compute::graph_destroy(compute::graph_end());
        } catch (...) {
        }
        throw;
    }
    void* graph = compute::graph_end();
    graphs_.push_back({plan_length, steps, graph});
    return graph;
}

void QwenModel::release_graphs() noexcept {
    for (const auto& g : graphs_) compute::graph_destroy(g.graph);
    graphs_.clear();
}

QwenModel::~QwenModel() {
    release_graphs();
    compute::destroy_stream(stream_);
}

void QwenModel::synchronize() const { compute::synchronize(); }

int32_t QwenModel::sample_greedy_from_logits() {
    compute::launch_argmax(static_cast<const float*>(logits_->data()), static_cast<int>(config_.vocab_size),
                           static_cast<int32_t*>(next_token_->data()));
    int32_t next = 0;
    next_token_->copy_to_host(&next, sizeof(next));   // waits for the stream
    return next;
}

}  // namespace citlali::model
