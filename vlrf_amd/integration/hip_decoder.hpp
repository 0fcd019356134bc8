// hip_decoder.hpp - device-resident greedy decode for a VLRF TransformerModel.
//
// Drop-in location in the engine tree: include/model/hip_decoder.hpp, used by
// the C API / CLI when the HIP backend is active.  It builds a
// vlrf_hip_model from the engine's ModelConfig and WeightMap (reference
// include/model/config.hpp, weights.hpp) and reproduces the greedy path of
// TransformerModel::generate (transformer.hpp:439-547): reset the KV cache,
// run the prompt, then decode starting from the last prompt id, with only
// token ids crossing PCIe.  Supported: pre-norm Llama-style models
// (use_rms_norm, SiLU with `ffn.gate.weight`, ROTARY, untied LM head or tied
// embeddings), no biases, default MuP multipliers, Q8_0 KV cache.
#pragma once

#include "transformer.hpp"
#include "vlrf_hip.h"

#include <stdexcept>
#include <string>
#include <vector>

namespace vlrf {

class HipDecoder {
public:
    // weight_dtype: VLRF_DT_Q8_0 / VLRF_DT_Q4_0 quantize the engine's f32
    // projection weights with this backend's block encoder; VLRF_DT_F32 keeps them.
    HipDecoder(vlrf_hip_ctx_t ctx, ModelConfig const& c, WeightMap& wm, int weight_dtype = VLRF_DT_Q8_0)
        : ctx_(ctx), vocab_(c.vocab_size) {
        if (!c.use_rms_norm || c.activation != Activation::SILU ||
            c.pos_embedding != PosEmbedding::ROTARY || !c.pre_norm || c.embedding_multiplier != 1.f ||
            c.attention_multiplier != 0.f || c.residual_multiplier != 1.f || c.logits_scaling != 1.f ||
            (c.kv_cache_dtype != static_cast<int>(KVCacheDType::F32) &&
             c.kv_cache_dtype != static_cast<int>(KVCacheDType::F16) &&
             c.kv_cache_dtype != static_cast<int>(KVCacheDType::Q8_0)))
            throw std::runtime_error("HipDecoder: unsupported model family");
        for (int l = 0; l < c.n_layers; ++l) {
            const std::string p = "layers." + std::to_string(l) + ".";
            if (!wm.has(p + "ffn.gate.weight"))
                throw std::runtime_error("HipDecoder: SwiGLU gate weight missing in layer " + std::to_string(l));
            for (const char* b : {"attn.q_proj.bias", "attn.k_proj.bias", "attn.v_proj.bias", "attn.o_proj.bias",
                                  "ffn.fc1.bias", "ffn.fc2.bias", "ffn.gate.bias"})
                if (wm.has(p + b)) throw std::runtime_error(std::string("HipDecoder: biases unsupported: ") + p + b);
        }
        vlrf_hip_model_config mc{};
        mc.vocab_size = c.vocab_size;
        mc.d_model = c.d_model;
        mc.d_ff = c.d_ff;
        mc.n_heads = c.n_heads;
        mc.n_kv_heads = c.n_kv_heads;
        mc.n_layers = c.n_layers;
        mc.max_seq_len = c.max_seq_len;
        mc.norm_eps = c.layer_norm_eps;
        mc.rope_theta = c.rope_theta;
        mc.weight_dtype = weight_dtype;
        mc.kv_dtype = c.kv_cache_dtype;          // KVCacheDType values are the ABI's VLRF_KV_*
        check(vlrf_hip_model_create(ctx_, &mc, &m_));
        auto put_f32 = [&](const std::string& name, const std::string& key) {
            Tensor& t = wm.get(key);
            const int rows = t.ndim() == 2 ? t.dim(0) : 1;
            const int cols = t.ndim() == 2 ? t.dim(1) : t.dim(0);
            check(vlrf_hip_model_set_weight(m_, name.c_str(), t.data_ptr(), VLRF_DT_F32, rows, cols));
        };
        auto put_proj = [&](const std::string& name, const std::string& key) {
            Tensor& t = wm.get(key);
            const int rows = t.dim(0), cols = t.dim(1);
            if (weight_dtype == VLRF_DT_F32) {
                check(vlrf_hip_model_set_weight(m_, name.c_str(), t.data_ptr(), VLRF_DT_F32, rows, cols));
                return;
            }
            const size_t bb = weight_dtype == VLRF_DT_Q8_0 ? 34 : 18;
            std::vector<unsigned char> blocks((size_t)rows * cols / 32 * bb);
            const int rc = weight_dtype == VLRF_DT_Q8_0
                               ? vlrf_quantize_q8_0(t.data_ptr(), blocks.data(), (int64_t)rows * cols)
                               : vlrf_quantize_q4_0(t.data_ptr(), blocks.data(), (int64_t)rows * cols);
            check(rc);
            check(vlrf_hip_model_set_weight(m_, name.c_str(), blocks.data(), weight_dtype, rows, cols));
        };
        put_f32("embed.weight", "embed.weight");
        put_f32("ln_final.weight", "ln_final.weight");
        put_proj("lm_head.weight", c.tie_embeddings ? "embed.weight" : "lm_head.weight");
        for (int l = 0; l < c.n_layers; ++l) {
            const std::string p = "layers." + std::to_string(l) + ".";
            for (const char* k : {"ln1.weight", "ln2.weight"}) put_f32(p + k, p + k);
            for (const char* k : {"attn.q_proj.weight", "attn.k_proj.weight", "attn.v_proj.weight",
                                  "attn.o_proj.weight", "ffn.gate.weight", "ffn.fc1.weight",
                                  "ffn.fc2.weight"})
                put_proj(p + k, p + k);
        }
    }
    HipDecoder(const HipDecoder&) = delete;
    HipDecoder& operator=(const HipDecoder&) = delete;
    ~HipDecoder() { vlrf_hip_model_destroy(m_); }

    // Greedy TransformerModel::generate with default penalties; returns the
    // prompt followed by the generated ids (GenerationResult::token_ids).
    std::vector<int> generate(std::vector<int> const& prompt, int max_new_tokens) {
        if (prompt.empty()) throw std::runtime_error("HipDecoder: empty prompt");
        check(vlrf_hip_model_reset(m_));
        int32_t next = 0;
        std::vector<int32_t> ids(prompt.begin(), prompt.end());
        check(vlrf_hip_model_prefill(m_, ids.data(), (int)ids.size(), &next));
        std::vector<int32_t> gen(max_new_tokens);
        if (max_new_tokens > 0)
            check(vlrf_hip_model_generate(m_, prompt.back(), max_new_tokens, gen.data()));
        std::vector<int> out(prompt);
        out.insert(out.end(), gen.begin(), gen.end());
        return out;
    }

    // One decode step of `token` with the logits copied to host (vocab floats).
    int step(int token, float* logits) {
        int32_t next = 0;
        check(vlrf_hip_model_step(m_, token, &next, logits));
        return next;
    }

private:
    static void check(int rc) {
        if (rc != VLRF_HIP_OK) throw std::runtime_error(std::string("vlrf_hip: ") + vlrf_hip_last_error());
    }
    vlrf_hip_ctx_t ctx_;
    vlrf_hip_model_t m_ = nullptr;
    int vocab_;
};

}  // namespace vlrf
