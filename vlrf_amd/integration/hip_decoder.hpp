// hip_decoder.hpp - device-resident greedy decode for a VLRF TransformerModel.
//
// Drop-in location in the engine tree: include/model/hip_decoder.hpp, used by
// the C API / CLI when the HIP backend is active.  It builds a
// vlrf_hip_model from the engine's ModelConfig and WeightMap (reference
// include/model/config.hpp, weights.hpp) and reproduces the greedy path of
// TransformerModel::generate (transformer.hpp:439-547): reset the KV cache,
// run the prompt, then decode starting from the last prompt id (bos_token_id
// for an empty prompt), stopping at max_seq_len, at the first generated
// eos_token_id (hit_eos) or when on_token returns false, with only token ids
// crossing PCIe.  Supported: pre-norm Llama-style models (use_rms_norm, SiLU
// with `ffn.gate.weight`, ROTARY, untied LM head or tied embeddings), no
// biases (all-zero ones, as converted checkpoints carry, are accepted),
// default MuP multipliers, F32/F16/Q8_0 KV cache.
//
// Weights: the device runs exactly the engine's weights.  A projection is
// uploaded as Q4_0 or Q8_0 blocks only when encoding and decoding the tensor
// reproduces it bit for bit (weights that came from GGUF blocks,
// convert_gguf.py:233-263); otherwise the layers run on f32 weights.
//
// Prompt ingestion.  By default the prompt runs through the decode step one
// token at a time: f32 activations and the f32 GEMV, so the KV rows and the
// greedy stream match the reference bit for bit where its arithmetic allows
// (the parity class of the decode tests).  Opt-in (set_prefill_mfma, or the
// environment variable VLRF_HIP_PREFILL_MFMA=<min prompt tokens>): prompts of
// at least that many tokens run as one batched pass on the matrix cores
// (vlrf_hip_model_prefill_mfma: bf16 operands, f32 accumulation, the
// reference's batched forward(prompt), transformer.hpp:444-448), block-dtype
// weights only.  Its parity class is the bf16 one: logits after the prompt
// within 1e-2 of the reference's; the greedy stream may part from the
// reference's where two logits lie closer than that.
#pragma once

#include "transformer.hpp"
#include "vlrf_hip.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

namespace vlrf {

class HipDecoder {
public:
    // weight_dtype kAuto: per the weights (the smallest of Q4_0, Q8_0 whose
    // blocks hold every layer projection exactly, else F32; the LM head is
    // chosen on its own).  VLRF_HIP_DT_Q8_0 / VLRF_HIP_DT_Q4_0 / VLRF_HIP_DT_F32 force a
    // dtype; a block dtype that would change a tensor is refused (naming it)
    // unless allow_lossy.
    static constexpr int kAuto = -1;

    HipDecoder(vlrf_hip_ctx_t ctx, ModelConfig const& c, WeightMap& wm, int weight_dtype = kAuto,
               bool allow_lossy = false)
        : ctx_(ctx), vocab_(c.vocab_size), max_seq_(c.max_seq_len), eos_(c.eos_token_id), bos_(c.bos_token_id),
          kv_dtype_(c.kv_cache_dtype) {
        if (!c.use_rms_norm || c.activation != Activation::SILU ||
            c.pos_embedding != PosEmbedding::ROTARY || !c.pre_norm || c.embedding_multiplier != 1.f ||
            c.attention_multiplier != 0.f || c.residual_multiplier != 1.f || c.logits_scaling != 1.f ||
            (c.kv_cache_dtype != static_cast<int>(KVCacheDType::F32) &&
             c.kv_cache_dtype != static_cast<int>(KVCacheDType::F16) &&
             c.kv_cache_dtype != static_cast<int>(KVCacheDType::Q8_0)))
            throw std::runtime_error("HipDecoder: unsupported model family");
        if (weight_dtype != kAuto && weight_dtype != VLRF_HIP_DT_F32 && weight_dtype != VLRF_HIP_DT_Q8_0 &&
            weight_dtype != VLRF_HIP_DT_Q4_0)
            throw std::runtime_error("HipDecoder: weight dtype " + std::to_string(weight_dtype) + " unsupported");
        std::vector<std::string> proj;
        for (int l = 0; l < c.n_layers; ++l) {
            const std::string p = "layers." + std::to_string(l) + ".";
            if (!wm.has(p + "ffn.gate.weight"))
                throw std::runtime_error("HipDecoder: SwiGLU gate weight missing in layer " + std::to_string(l));
            // Converted checkpoints carry zero biases (convert_gguf.py); those add
            // nothing, any other bias is refused.
            for (const char* b : {"attn.q_proj.bias", "attn.k_proj.bias", "attn.v_proj.bias", "attn.o_proj.bias",
                                  "ffn.fc1.bias", "ffn.fc2.bias", "ffn.gate.bias"})
                if (wm.has(p + b) && !all_zero(wm.get(p + b)))
                    throw std::runtime_error(std::string("HipDecoder: non-zero bias unsupported: ") + p + b);
            for (const char* k : {"attn.q_proj.weight", "attn.k_proj.weight", "attn.v_proj.weight",
                                  "attn.o_proj.weight", "ffn.gate.weight", "ffn.fc1.weight", "ffn.fc2.weight"})
                proj.push_back(p + k);
        }
        const std::string lm_key = c.tie_embeddings ? "embed.weight" : "lm_head.weight";
        layer_dtype_ = pick_dtype(wm, proj, weight_dtype, allow_lossy);
        lm_dtype_ = pick_dtype(wm, {lm_key}, weight_dtype, allow_lossy);

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
        mc.weight_dtype = layer_dtype_;
        mc.kv_dtype = c.kv_cache_dtype;          // KVCacheDType values are the ABI's VLRF_HIP_KV_*
        check(vlrf_hip_model_create(ctx_, &mc, &m_));
        mfma_ok_ = (layer_dtype_ == VLRF_HIP_DT_Q8_0 || layer_dtype_ == VLRF_HIP_DT_Q4_0) && c.d_model % 64 == 0 &&
                   c.d_ff % 64 == 0;
        if (const char* e = std::getenv("VLRF_HIP_PREFILL_MFMA")) set_prefill_mfma(std::atoi(e));
        try {
            auto put_f32 = [&](const std::string& name, const std::string& key) {
                Tensor& t = wm.get(key);
                const int rows = t.ndim() == 2 ? t.dim(0) : 1;
                const int cols = t.ndim() == 2 ? t.dim(1) : t.dim(0);
                check(vlrf_hip_model_set_weight(m_, name.c_str(), t.data_ptr(), VLRF_HIP_DT_F32, rows, cols));
            };
            auto put_proj = [&](const std::string& name, const std::string& key, int dt) {
                Tensor& t = wm.get(key);
                const int rows = t.dim(0), cols = t.dim(1);
                if (dt == VLRF_HIP_DT_F32) {
                    check(vlrf_hip_model_set_weight(m_, name.c_str(), t.data_ptr(), VLRF_HIP_DT_F32, rows, cols));
                    return;
                }
                std::vector<unsigned char> blocks;
                encode(t, dt, blocks);
                check(vlrf_hip_model_set_weight(m_, name.c_str(), blocks.data(), dt, rows, cols));
            };
            put_f32("embed.weight", "embed.weight");
            put_f32("ln_final.weight", "ln_final.weight");
            put_proj("lm_head.weight", lm_key, lm_dtype_);
            for (int l = 0; l < c.n_layers; ++l) {
                const std::string p = "layers." + std::to_string(l) + ".";
                for (const char* k : {"ln1.weight", "ln2.weight"}) put_f32(p + k, p + k);
            }
            for (auto const& k : proj) put_proj(k, k, layer_dtype_);
        } catch (...) {
            vlrf_hip_model_destroy(m_);
            throw;
        }
    }
    HipDecoder(const HipDecoder&) = delete;
    HipDecoder& operator=(const HipDecoder&) = delete;
    ~HipDecoder() { vlrf_hip_model_destroy(m_); }

    // Greedy TransformerModel::generate with default penalties
    // (transformer.hpp:439-547): at most max_new_tokens ids and never past
    // max_seq_len, ending after the first generated eos_token_id (hit_eos) or
    // after a token for which on_token returns false.  The device runs the
    // steps in batches; ids past a stop are computed and dropped.
    TransformerModel::GenerationResult generate(std::vector<int> const& prompt, int max_new_tokens,
                                                std::function<bool(int)> const& on_token = nullptr) {
        TransformerModel::GenerationResult r;
        r.token_ids = prompt;
        prefill(prompt);
        int32_t last = prompt.empty() ? bos_ : prompt.back();
        int left = std::min(max_new_tokens, max_seq_ - (int)prompt.size());
        std::vector<int32_t> buf;
        for (int batch = 16; left > 0; batch = std::min(batch * 2, 256)) {
            const int n = std::min(batch, left);
            buf.resize(n);
            check(vlrf_hip_model_generate(m_, last, n, buf.data()));
            for (int i = 0; i < n; ++i) {
                const int id = buf[i];
                r.token_ids.push_back(id);
                r.tokens_generated++;
                if (on_token && !on_token(id)) return r;
                if (id == eos_) {
                    r.hit_eos = true;
                    return r;
                }
            }
            last = buf[n - 1];
            left -= n;
        }
        return r;
    }

    // Whether this decoder still fits the engine's config: the KV cache dtype
    // and length (vlrf_set_kv_cache_type / vlrf_set_ctx change them in place)
    // and the token ids generate() stops or starts at.
    bool matches(ModelConfig const& c) const {
        return c.kv_cache_dtype == kv_dtype_ && c.max_seq_len == max_seq_ && c.eos_token_id == eos_ &&
               c.bos_token_id == bos_ && c.vocab_size == vocab_;
    }

    // The dtypes chosen for the layer projections and the LM head.
    int layer_dtype() const { return layer_dtype_; }
    int lm_head_dtype() const { return lm_dtype_; }

    // Prompts of at least min_tokens (> 0) run as one matrix-core pass (see
    // the file comment); 0 switches it off.  No effect where the layers run
    // on f32 weights.
    void set_prefill_mfma(int min_tokens) { prefill_mfma_min_ = min_tokens > 0 ? min_tokens : 0; }
    bool prefill_uses_mfma(size_t n) const { return mfma_ok_ && prefill_mfma_min_ > 0 && (int)n >= prefill_mfma_min_; }

    // Resets the device cache and runs the prompt (the reference's
    // forward(prompt) with the cache, transformer.hpp:444-448).
    void prefill(std::vector<int> const& prompt) {
        check(vlrf_hip_model_reset(m_));
        if (prompt.empty()) return;
        int32_t next = 0;
        std::vector<int32_t> ids(prompt.begin(), prompt.end());
        if (prefill_uses_mfma(ids.size()))
            check(vlrf_hip_model_prefill_mfma(m_, ids.data(), (int)ids.size(), &next));
        else
            check(vlrf_hip_model_prefill(m_, ids.data(), (int)ids.size(), &next));
    }

    // Tokens in the device cache.
    int used() const { return vlrf_hip_model_used(m_); }

    // Copies the device cache's first `used` rows of every layer into the
    // engine's caches (the reference's token-major KVCache storage,
    // kv_cache.hpp:132-148) and sets their `used`, so that a CPU forward
    // with the cache continues where the device stopped.
    void read_cache(std::vector<KVCache>& caches, int used) {
        if (used < 0 || used > max_seq_) throw std::runtime_error("HipDecoder::read_cache: bad row count");
        for (size_t l = 0; l < caches.size(); ++l) {
            KVCache& c = caches[l];
            int8_t *k = nullptr, *v = nullptr;
            float *ks = nullptr, *vs = nullptr;
            switch (c.dtype) {
                case KVCacheDType::Q8_0:
                    k = c.K_q8.data(); v = c.V_q8.data(); ks = c.K_scale.data(); vs = c.V_scale.data();
                    break;
                case KVCacheDType::F16:
                    k = reinterpret_cast<int8_t*>(c.K_f16.data()); v = reinterpret_cast<int8_t*>(c.V_f16.data());
                    break;
                default:
                    k = reinterpret_cast<int8_t*>(c.K.data_ptr()); v = reinterpret_cast<int8_t*>(c.V.data_ptr());
                    break;
            }
            if (used) check(vlrf_hip_model_kv_read(m_, (int)l, 0, used, k, v, ks, vs));
            c.used = used;
        }
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
    static bool all_zero(Tensor& t) {
        const float* v = t.data_ptr();
        for (int64_t i = 0; i < t.numel(); ++i)
            if (v[i] != 0.f) return false;
        return true;
    }
    static size_t block_bytes(int dt) { return dt == VLRF_HIP_DT_Q8_0 ? 34 : 18; }
    static void encode(Tensor& t, int dt, std::vector<unsigned char>& blocks) {
        if (t.numel() % 32 != 0)
            throw std::runtime_error("HipDecoder: a block dtype needs 32 | numel");
        blocks.resize((size_t)t.numel() / 32 * block_bytes(dt));
        check(dt == VLRF_HIP_DT_Q8_0 ? vlrf_quantize_q8_0(t.data_ptr(), blocks.data(), t.numel())
                                 : vlrf_quantize_q4_0(t.data_ptr(), blocks.data(), t.numel()));
    }
    // Whether dtype dt's blocks reproduce the tensor bit for bit.
    static bool exact(Tensor& t, int dt) {
        if (t.numel() % 32 != 0) return false;
        std::vector<unsigned char> blocks;
        encode(t, dt, blocks);
        std::vector<float> back((size_t)t.numel());
        check(vlrf_dequantize(blocks.data(), dt, back.data(), t.numel()));
        return std::memcmp(back.data(), t.data_ptr(), sizeof(float) * back.size()) == 0;
    }
    static int pick_dtype(WeightMap& wm, std::vector<std::string> const& keys, int want, bool allow_lossy) {
        if (want == VLRF_HIP_DT_F32) return VLRF_HIP_DT_F32;
        if (want != kAuto) {
            if (!allow_lossy)
                for (auto const& k : keys)
                    if (!exact(wm.get(k), want))
                        throw std::runtime_error("HipDecoder: " + k + " is not exactly representable in " +
                                                 (want == VLRF_HIP_DT_Q8_0 ? "Q8_0" : "Q4_0") +
                                                 " blocks; pass VLRF_HIP_DT_F32 or kAuto, or allow_lossy");
            return want;
        }
        for (int dt : {VLRF_HIP_DT_Q4_0, VLRF_HIP_DT_Q8_0}) {
            bool all = true;
            for (auto const& k : keys)
                if (!(all = exact(wm.get(k), dt))) break;
            if (all) return dt;
        }
        return VLRF_HIP_DT_F32;
    }
    vlrf_hip_ctx_t ctx_;
    vlrf_hip_model_t m_ = nullptr;
    int vocab_;
    int max_seq_, eos_, bos_, kv_dtype_;
    int layer_dtype_ = VLRF_HIP_DT_F32, lm_dtype_ = VLRF_HIP_DT_F32;
    bool mfma_ok_ = false;
    int prefill_mfma_min_ = 0;
};

}  // namespace vlrf
