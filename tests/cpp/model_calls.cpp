// model_calls.cpp - every firefly::kernels call shape of the reference model's forward pass and engine, compiled
// against this repository's include/firefly (tests/test_hal.py compiles it; nothing here runs).
//
// forward_shapes() follows QwenModel::forward (src/model/qwen_model.cu:98-191): the tensors it builds, the
// off-path operators it calls around the KV-cache path (embedding_lookup, rms_norm, matmul, add_inplace, swiglu),
// apply_rope, the append (the private kernel launch at :139-143 becomes kernels::append_kv_cache) and both
// branches of kernels::attention (:147-156).  engine_shapes() follows the engine's graph capture and prefill
// (src/engine.cc:136-148, :258-267): set_default_stream, argmax.  The off-path operators are declared by
// include/firefly/kernels.h and defined by the caller's own kernel files, so this unit is compiled, not linked.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <vector>

#include "firefly/kernels.h"
#include "firefly/tensor.h"

using namespace firefly;

namespace call_shapes
{

struct Layer
{
    Tensor input_layernorm, post_attention_layernorm;
    Tensor q_proj, k_proj, v_proj, o_proj, q_norm, k_norm;
    Tensor gate_proj, up_proj, down_proj;
};

struct Config
{
    int    hidden_size = 4096, num_attention_heads = 32, num_key_value_heads = 8, head_dim = 128;
    int    intermediate_size = 12288, vocab_size = 151936, num_hidden_layers = 36;
    double rms_norm_eps = 1e-6;
    float  rope_theta = 1000000.0f;
};

Tensor forward_shapes(const Config& config, const std::vector<Layer>& layers, const Tensor& token_embeddings,
                      const Tensor& norm, const Tensor& lm_head, const Tensor& input_ids, const Tensor& context_lens,
                      std::vector<Tensor>& k_caches, std::vector<Tensor>& v_caches, int* block_table, int max_blocks)
{
    int batch_size = input_ids.shape()[0];
    int seq_len = input_ids.shape()[1];

    Tensor hidden_states({(long)batch_size, seq_len, (long)config.hidden_size}, DType::F16, Device::CUDA);
    kernels::embedding_lookup(input_ids, token_embeddings, hidden_states);

    for (int i = 0; i < config.num_hidden_layers; ++i)
    {
        const auto& layer = layers[i];
        Tensor norm_out({(long)batch_size, seq_len, (long)config.hidden_size}, DType::F16, Device::CUDA);
        kernels::rms_norm(hidden_states, layer.input_layernorm, norm_out, config.rms_norm_eps);

        Tensor q({(long)batch_size, seq_len, (long)config.num_attention_heads, (long)config.head_dim}, DType::F16,
                 Device::CUDA);
        Tensor k({(long)batch_size, seq_len, (long)config.num_key_value_heads, (long)config.head_dim}, DType::F16,
                 Device::CUDA);
        Tensor v({(long)batch_size, seq_len, (long)config.num_key_value_heads, (long)config.head_dim}, DType::F16,
                 Device::CUDA);
        kernels::matmul(norm_out, layer.q_proj, q);
        kernels::matmul(norm_out, layer.k_proj, k);
        kernels::matmul(norm_out, layer.v_proj, v);
        if (layer.q_norm.data() != nullptr && layer.k_norm.data() != nullptr)
        {
            kernels::rms_norm(q, layer.q_norm, q, config.rms_norm_eps);
            kernels::rms_norm(k, layer.k_norm, k, config.rms_norm_eps);
        }

        const int* context_lens_ptr = nullptr;
        if (context_lens.data() != nullptr) context_lens_ptr = static_cast<const int*>(context_lens.data());

        kernels::apply_rope(q, k, config.head_dim, seq_len, config.rope_theta, context_lens_ptr);
        // the reference's private append_kv_cache<<<grid, 128, 0, get_default_stream()>>> launch, exported
        kernels::append_kv_cache(k, v, k_caches[i], v_caches[i], block_table, context_lens_ptr, max_blocks);

        Tensor attn_out({(long)batch_size, seq_len, (long)(config.num_attention_heads * config.head_dim)}, DType::F16,
                        Device::CUDA);
        if (context_lens_ptr == nullptr || (batch_size == 1 && seq_len > 1))
            kernels::attention(q, k, v, attn_out, nullptr, config.num_key_value_heads, seq_len, max_blocks, nullptr);
        else
            kernels::attention(q, k_caches[i], v_caches[i], attn_out, block_table, config.num_key_value_heads, seq_len,
                               max_blocks, context_lens_ptr);

        Tensor o_out({(long)batch_size, seq_len, (long)config.hidden_size}, DType::F16, Device::CUDA);
        kernels::matmul(attn_out, layer.o_proj, o_out);
        kernels::add_inplace(hidden_states, o_out);
        kernels::rms_norm(hidden_states, layer.post_attention_layernorm, norm_out, config.rms_norm_eps);

        Tensor gate({(long)batch_size, seq_len, (long)config.intermediate_size}, DType::F16, Device::CUDA);
        Tensor up({(long)batch_size, seq_len, (long)config.intermediate_size}, DType::F16, Device::CUDA);
        Tensor mlp_intermediate({(long)batch_size, seq_len, (long)config.intermediate_size}, DType::F16, Device::CUDA);
        kernels::matmul(norm_out, layer.gate_proj, gate);
        kernels::matmul(norm_out, layer.up_proj, up);
        kernels::swiglu(gate, up, mlp_intermediate);
        Tensor mlp_out({(long)batch_size, seq_len, (long)config.hidden_size}, DType::F16, Device::CUDA);
        kernels::matmul(mlp_intermediate, layer.down_proj, mlp_out);
        kernels::add_inplace(hidden_states, mlp_out);
    }

    Tensor final_norm_out({(long)batch_size, 1, (long)config.hidden_size}, DType::F16, Device::CUDA);
    half*  last_token_hidden = (half*)hidden_states.data() + (seq_len - 1) * config.hidden_size;
    Tensor last_hidden =
        Tensor::from_external(last_token_hidden, {batch_size, 1, (long)config.hidden_size}, DType::F16, Device::CUDA);
    kernels::rms_norm(last_hidden, norm, final_norm_out, config.rms_norm_eps);
    Tensor logits({(long)batch_size, 1, (long)config.vocab_size}, DType::F16, Device::CUDA);
    kernels::matmul(final_norm_out, lm_head, logits);
    return logits;
}

void engine_shapes(hipStream_t capture_stream, Tensor& logits, Tensor& next_tokens, Tensor& next_token)
{
    firefly::kernels::set_default_stream(capture_stream);
    kernels::argmax(logits, next_tokens);  // inside the decode graph's capture lambda (src/engine.cc:145)
    firefly::kernels::set_default_stream(nullptr);
    kernels::argmax(logits, next_token);   // after a prefill forward (src/engine.cc:267)
    hipStream_t s = firefly::kernels::get_default_stream();
    (void)s;
}

}  // namespace call_shapes
