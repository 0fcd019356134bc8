// ref_shim.cpp - C entry points onto the reference implementation, compiled
// from the reference's own headers where they lie under /root/reference.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile builds this file into
// oracle/_ref/libvlrf_ref.so when /root/reference is present.  It is used to
// pin the C restatement in oracle/vlrf_oracle.c (tests/test_oracle.py), to
// write golden fixtures (tests/golden/gen_golden.py), and, optionally, as the
// CPU baseline in bench.py.  No reference source is copied: this file only
// calls the reference's functions.
#include "transformer.hpp"

#include <cstdint>
#include <cstring>
#include <memory>
#include <string>

using vlrf::Tensor;
using vlrf::Shape;

namespace {
Tensor wrap(const float* p, std::initializer_list<int32_t> dims) {
    return Tensor::from_ptr(const_cast<float*>(p), Shape(dims));
}
}  // namespace

extern "C" {

// kv_cache.hpp:102-117
float ref_quantize_row_q8_0(const float* src, int8_t* dst, int n) {
    return vlrf::detail::quantize_row_q8_0(src, dst, n);
}

// attention.hpp:207-309
void ref_flash_attn_head(const float* Q, const float* K, const float* V, float* O,
                         int T, int ctx_len, int d_h, float scale, int causal) {
    vlrf::AttentionBlock::flash_attn_head(Q, K, V, O, T, ctx_len, d_h, scale, causal != 0);
}

// ops.hpp:478-499
void ref_rms_norm(const float* x, const float* w, float* out, int rows, int D, float eps) {
    Tensor X = wrap(x, {rows, D}), W = wrap(w, {D}), O = wrap(out, {rows, D});
    vlrf::ops::rms_norm(X, W, O, eps);
}

// rope.hpp:49-99 (a private RopeCache instance, same tables as the global one)
void ref_rope(float* x, int T, int n_heads, int d_head, int pos_offset, int max_seq,
              float theta) {
    static vlrf::RopeCache rc;
    rc.init(max_seq, d_head, theta);
    rc.apply(x, T, n_heads, pos_offset);
}

// compute::linear -> ops::gemm(x, W, y, 1, 0, false, true)  (compute.hpp:64-68)
void ref_linear(const float* x, const float* W, float* y, int M, int K, int N) {
    Tensor X = wrap(x, {M, K}), Wt = wrap(W, {N, K}), Y = wrap(y, {M, N});
    vlrf::ops::gemm(X, Wt, Y, 1.f, 0.f, false, true);
}

// feedforward.hpp:60-62
void ref_silu_mul(float* h, float* g, int64_t n) {
    Tensor Hh = wrap(h, {(int32_t)n}), Gg = wrap(g, {(int32_t)n});
    vlrf::ops::silu_inplace(Gg);
    vlrf::ops::multiply_inplace(Hh, Gg);
}

int ref_hw_threads(void) { return vlrf::ops::hw_threads(); }

// ops.hpp:443-476
void ref_layer_norm(const float* x, const float* w, const float* b, float* out, int rows, int D, float eps) {
    Tensor X = wrap(x, {rows, D}), W = wrap(w, {D}), Bb = wrap(b, {D}), O = wrap(out, {rows, D});
    vlrf::ops::layer_norm(X, W, Bb, O, eps);
}

// ops.hpp:501-540
void ref_softmax(float* x, int rows, int D) {
    Tensor X = wrap(x, {rows, D});
    vlrf::ops::softmax_inplace(X);
}

// ops.hpp:390-404
void ref_gelu(float* x, int64_t n) {
    Tensor X = wrap(x, {(int32_t)n});
    vlrf::ops::gelu_inplace(X);
}

// ops.hpp:170-310 with the operands' stored shapes: A [rA, cA], B [rB, cB].
void ref_gemm(const float* A, int rA, int cA, const float* B, int rB, int cB, float* C, int M, int N,
              float alpha, float beta, int transA, int transB) {
    Tensor At = wrap(A, {rA, cA}), Bt = wrap(B, {rB, cB}), Ct = wrap(C, {M, N});
    vlrf::ops::gemm(At, Bt, Ct, alpha, beta, transA != 0, transB != 0);
}

// ---- whole model: TransformerModel (transformer.hpp) -------------------------
struct RefModel {
    vlrf::TransformerModel m;
};

// kv_cache.hpp:68-97
uint16_t ref_f32_to_f16(float f) { return vlrf::detail::f32_to_f16(f); }

void* ref_model_create_kv(int vocab, int d_model, int d_ff, int n_heads, int n_kv_heads,
                          int n_layers, int max_seq, float eps, float theta, int kv_dtype) {
    auto* r = new RefModel();
    vlrf::ModelConfig c;
    c.vocab_size = vocab;
    c.d_model = d_model;
    c.d_ff = d_ff;
    c.n_heads = n_heads;
    c.n_kv_heads = n_kv_heads;
    c.n_layers = n_layers;
    c.max_seq_len = max_seq;
    c.layer_norm_eps = eps;
    c.rope_theta = theta;
    c.use_rms_norm = true;
    c.pre_norm = true;
    c.activation = vlrf::Activation::SILU;
    c.pos_embedding = vlrf::PosEmbedding::ROTARY;
    c.tie_embeddings = false;
    c.kv_cache_dtype = kv_dtype;  // KVCacheDType: 0 F32, 1 F16, 2 Q8_0
    c.eos_token_id = -1;   // never stop early in fixture runs
    c.do_sample = false;
    r->m.init(c);
    return r;
}

void* ref_model_create(int vocab, int d_model, int d_ff, int n_heads, int n_kv_heads,
                       int n_layers, int max_seq, float eps, float theta) {
    return ref_model_create_kv(vocab, d_model, d_ff, n_heads, n_kv_heads, n_layers, max_seq, eps, theta, 2);
}

// Borrowed pointer (no copy): the caller keeps `data` alive.
void ref_model_set_tensor(void* h, const char* name, const float* data, int rows, int cols) {
    auto* r = static_cast<RefModel*>(h);
    if (rows > 0)
        r->m.wm.tensors[name] = wrap(data, {rows, cols});
    else
        r->m.wm.tensors[name] = wrap(data, {cols});
}

void ref_model_bind(void* h) { static_cast<RefModel*>(h)->m.bind_weights(); }
void ref_model_reset(void* h) { static_cast<RefModel*>(h)->m.reset_kv_cache(); }
int ref_model_used(void* h) { return static_cast<RefModel*>(h)->m.context_used(); }

int ref_model_forward(void* h, const int* ids, int T, float* logits) {
    auto* r = static_cast<RefModel*>(h);
    std::vector<int> v(ids, ids + T);
    Tensor lg = r->m.forward(v, true);
    if (logits) std::memcpy(logits, lg.data_ptr(), sizeof(float) * lg.numel());
    return vlrf::sampler::argmax(lg);
}

void ref_model_kv(void* h, int l, int8_t** kq, int8_t** vq, float** ks, float** vs) {
    auto& c = static_cast<RefModel*>(h)->m.kv_caches[l];
    *kq = c.K_q8.data();
    *vq = c.V_q8.data();
    *ks = c.K_scale.data();
    *vs = c.V_scale.data();
}

// Layer l's K/V storage in the cache's own element type (kv_cache.hpp:141-150).
void ref_model_kv_raw(void* h, int l, void** k, void** v) {
    auto& c = static_cast<RefModel*>(h)->m.kv_caches[l];
    switch (c.dtype) {
        case vlrf::KVCacheDType::F32: *k = c.K.data_ptr(); *v = c.V.data_ptr(); break;
        case vlrf::KVCacheDType::F16: *k = c.K_f16.data(); *v = c.V_f16.data(); break;
        default: *k = c.K_q8.data(); *v = c.V_q8.data(); break;
    }
}

// Fills rows [0, used) of every layer's Q8_0 cache with the same seeded codes
// and scales as the C restatement's orc_model_fill_kv, and sets the caches'
// fill length (kv_cache.hpp:138 `used`), so a decode step can be timed at a
// long context without a CPU prefill.  No-op for other cache types.
void ref_model_fill_kv(void* h, int used, uint64_t seed) {
    auto& m = static_cast<RefModel*>(h)->m;
    uint64_t z = seed * 0x9E3779B97F4A7C15ull + 1;
    for (auto& c : m.kv_caches) {
        if (c.dtype != vlrf::KVCacheDType::Q8_0) return;
        int n = used < c.max_seq_len ? used : c.max_seq_len;
        size_t row = (size_t)c.row_dim;
        for (int r = 0; r < n; ++r) {
            for (size_t i = 0; i < row; ++i) {
                z ^= z << 13; z ^= z >> 7; z ^= z << 17;
                c.K_q8[(size_t)r * row + i] = (int8_t)((int)(z & 0xFF) % 255 - 127);
                c.V_q8[(size_t)r * row + i] = (int8_t)((int)((z >> 8) & 0xFF) % 255 - 127);
            }
            c.K_scale[r] = 0.02f;
            c.V_scale[r] = 0.02f;
        }
        c.used = n;
    }
}

void ref_model_destroy(void* h) { delete static_cast<RefModel*>(h); }

}  // extern "C"
