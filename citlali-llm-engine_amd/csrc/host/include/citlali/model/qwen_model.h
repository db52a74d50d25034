// citlali/model/qwen_model.h -- single-token decode of a Qwen-family model.
//
// forward_token follows the reference's QwenModel::forward_token
// (src/model/qwen_model.cpp:239-419) operation by operation, with its fp16
// store points and output-weight rule, over the gfx950 compute:: launchers.
// The weights arrive from a GGUF file (the reference's load()) or as
// WeightHandles (QwenWeights); remote layer ranges are not part of this
// build (a load that asks for them is refused).  Greedy sampling picks the first largest finite logit
// (qwen_model.cpp:448-465) on the device and copies back one index.
#pragma once

#include "citlali/compute/hip/kernels.h"
#include "citlali/compute/hip/tensor.h"
#include "citlali/model/linear_backend.h"
#include "citlali/model/qwen_config.h"
#include "citlali/model/weight_handle.h"
#include "citlali/model/weight_loader.h"
#include "citlali/remote/remote_client.h"

#include <cstdint>
#include <memory>
#include <utility>
#include <vector>

namespace citlali::model {

// Same fields as the reference (include/citlali/model/qwen_model.h:16-33).
struct QwenLayerWeights {
    WeightHandle attn_norm;
    WeightHandle attn_q, attn_q_bias;
    WeightHandle attn_k, attn_k_bias;
    WeightHandle attn_v, attn_v_bias;
    WeightHandle attn_o, attn_o_bias;
    WeightHandle attn_q_norm, attn_k_norm;
    WeightHandle ffn_norm;
    WeightHandle ffn_gate, ffn_gate_bias;
    WeightHandle ffn_up, ffn_up_bias;
    WeightHandle ffn_down, ffn_down_bias;
    compute::DeviceBufferPtr k_cache;   // allocated by load()
    compute::DeviceBufferPtr v_cache;
};

// What the reference's load() reads from GGUF.  An output_weight without a
// buffer falls back to token_embedding (qwen_model.cpp:73-75).
struct QwenWeights {
    WeightHandle token_embedding;
    WeightHandle output_norm;
    WeightHandle output_weight;
    std::vector<QwenLayerWeights> layers;
};

class QwenModel {
public:
    QwenModel() = default;
    ~QwenModel();
    QwenModel(const QwenModel&) = delete;
    QwenModel& operator=(const QwenModel&) = delete;

    // From a GGUF file, as the reference's load (qwen_model.cpp:45-186):
    // config by QwenConfig::from_gguf, tensors by their GGUF names through a
    // WeightLoader (KeepQuantized when `quantized`, else DequantizeToFp16),
    // then the load below.  remote_options keeps the reference's signature
    // (include/citlali/model/qwen_model.h:38-40): options that offload
    // layers (enabled(): an endpoint and a layer list) get the reference's
    // range check ("remote layer index is out of range: N"), then
    // citlali::Error, before any weight is read; a layer list without an
    // endpoint is refused too (the reference would dereference a missing
    // client).  Otherwise every layer runs on the GPU.
    void load(const io::GgufFile& gguf, uint32_t max_context = 0, bool quantized = false,
              const remote::RemoteOptions& remote_options = {});
    // max_context 0 -> min(context_length, 2048), as the reference.
    void load(const QwenConfig& config, QwenWeights weights, uint32_t max_context = 0);
    // Runs one token at `position`; returns the greedy next token, or -1
    // when compute_logits is false.
    int32_t forward_token(int32_t token_id, uint32_t position, bool compute_logits = true);
    // `steps` greedy tokens after token_id at `position`: the tokens that
    // forward_token would return one call at a time, bit for bit, but with
    // each step replayed from a HIP graph (one per attention plan length) on
    // a stream of the model's own and no host synchronisation between steps.
    // Needs position + steps <= max_context.  No reference counterpart (the
    // reference's caller loops over forward_token).
    std::vector<int32_t> decode_greedy(int32_t token_id, uint32_t position, uint32_t steps);
    void synchronize() const;

    const QwenConfig& config() const { return config_; }
    uint32_t max_context() const { return max_context_; }
    // fp32 logits [vocab] of the last forward_token that computed them.
    const compute::DeviceBufferPtr& logits() const { return logits_; }

private:
    void allocate_runtime_buffers();
    bool launch_qkv_grouped(const QwenLayerWeights& layer, int hidden, const uint16_t* input,
                            const compute::NormInput* norm);
    void enqueue_token(int32_t token_id, int position, int32_t* state, int plan_length, bool compute_logits);
    void* step_graph(int plan_length, int steps);
    void release_graphs() noexcept;
    int32_t sample_greedy_from_logits();

    QwenConfig config_;
    uint32_t max_context_ = 0;
    WeightHandle token_embedding_;
    WeightHandle output_norm_;
    WeightHandle output_weight_;
    std::vector<QwenLayerWeights> layers_;

    compute::DeviceBufferPtr x_, x_alt_, norm_, q_, k_, v_, attn_out_, attn_proj_;
    compute::DeviceBufferPtr gate_, up_, ff_act_, ff_out_, logits_, scores_, next_token_;
    compute::DeviceBufferPtr state_, tokens_;   // decode_greedy: {token, position, step, 0}, picks
    std::unique_ptr<LinearBackend> linear_backend_;
    void* stream_ = nullptr;                                  // decode_greedy's stream
    struct StepGraph {
        int plan_length, steps;
        void* graph;
    };
    std::vector<StepGraph> graphs_;   // captured decode steps, by plan length and step count
};

}  // namespace citlali::model
