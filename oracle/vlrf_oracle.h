/*
 * vlrf_oracle.h - CPU restatement of the VLRF reference decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP backend
 * (tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg).  The
 * product (vlrf_amd/) never links, loads or calls it.
 *
 * Every function restates one reference function; the citation is given at
 * the definition in vlrf_oracle.c.  All arithmetic follows the reference's
 * operation order so that results can be compared bit for bit against the
 * reference built from its own sources (oracle/_ref).
 */
#ifndef VLRF_ORACLE_H
#define VLRF_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- KV cache Q8_0 (per token row) ---------------------------------- */
float orc_quantize_row_q8_0(const float* src, int8_t* dst, int n);
void  orc_dequantize_row_q8_0(const int8_t* src, float scale, float* dst, int n);

/* ---- attention -------------------------------------------------------- */
/* Q: [T, d_h] (row stride q_stride), K/V: [ctx, d_h] (row stride kv_stride),
 * O: [T, d_h] (row stride o_stride). */
void orc_flash_attn_head(const float* Q, int q_stride,
                         const float* K, const float* V, int kv_stride,
                         float* O, int o_stride,
                         int T, int ctx_len, int d_h, float scale, int causal);
/* Batched [n_h, T, d_h] / [n_h, ctx, d_h] layout, as IBackend::sdp_attention. */
void orc_sdp_attention(const float* Q, const float* K, const float* V, float* O,
                       int n_h, int T, int ctx_len, int d_h, float scale, int causal);

/* ---- norms / rope / activations ----------------------------------------- */
void orc_rms_norm(const float* x, const float* w, float* out, int rows, int D, float eps);
void orc_rope_tables(int max_seq, int d_head, float theta, float* cos_t, float* sin_t);
void orc_rope_apply(float* x, int T, int n_heads, int d_head, int pos_offset,
                    const float* cos_t, const float* sin_t, int max_seq);
void orc_silu_mul(float* h, float* g, int64_t n);
int  orc_argmax(const float* p, int n);

/* ---- linear: y[M,N] = x[M,K] . W[N,K]^T ------------------------------- */
void orc_linear(const float* x, const float* W, float* y, int M, int K, int N, int n_threads);

/* ---- GGUF block formats (decode = convert_gguf.py; encode = this build's) */
void orc_dequant_q8_0(const uint8_t* blocks, float* out, int64_t numel);
void orc_dequant_q4_0(const uint8_t* blocks, float* out, int64_t numel);
float orc_f16_to_f32(uint16_t h);
/* The engine's remaining per-op backend calls (ops.hpp:170-191, 390-404,
 * 443-476, 501-520). */
void orc_layer_norm(const float* x, const float* w, const float* b, float* out, int rows, int D, float eps);
void orc_softmax(float* x, int rows, int D);
void orc_gelu(float* x, int64_t n);
void orc_gemm(const float* A, const float* B, float* C, int M, int N, int K, int lda, int ldb, int ldc,
              float alpha, float beta, int transA, int transB);
/* KVCache F16 element conversion (kv_cache.hpp:68-97). */
uint16_t orc_f32_to_f16_kv(float f);

/* ---- whole model (Llama-style, RMSNorm / RoPE / SwiGLU / GQA, Q8_0 KV) --- */
/* KV cache dtypes, the reference's KVCacheDType values (kv_cache.hpp:37-41). */
#define ORC_KV_F32  0
#define ORC_KV_F16  1
#define ORC_KV_Q8_0 2

typedef struct orc_config {
    int vocab_size, d_model, d_ff, n_heads, n_kv_heads, n_layers, max_seq_len;
    float norm_eps, rope_theta;
    int n_threads;
    int kv_dtype;          /* ORC_KV_* */
} orc_config;

typedef struct orc_model orc_model;

orc_model* orc_model_create(const orc_config* cfg);
void orc_model_destroy(orc_model* m);
/* Pointers are borrowed (caller keeps the f32 arrays alive). */
void orc_model_set_globals(orc_model* m, const float* embed, const float* ln_final,
                           const float* lm_head);
void orc_model_set_layer(orc_model* m, int l, const float* ln1, const float* ln2,
                         const float* wq, const float* wk, const float* wv, const float* wo,
                         const float* wg, const float* w1, const float* w2);
void orc_model_reset(orc_model* m);
int  orc_model_used(const orc_model* m);
/* Runs T tokens (T=1: decode, T>1: prefill) through the model, appending to the
 * KV cache; writes logits of the last row (may be NULL) and returns the greedy
 * argmax, or -1 on error (cache overflow / bad id). */
int  orc_model_forward(orc_model* m, const int* ids, int T, float* logits);
/* The layers only: x [T][d_model] embedded rows in, residual stream after the
 * last layer out (in place); appends T cache rows.  0, or -1 on overflow. */
int  orc_model_forward_hidden(orc_model* m, float* x, int T);
/* Token-major reference layout of layer l's cache: K/V int8 [max_seq, row_dim],
 * scales [max_seq]. */
void orc_model_kv(orc_model* m, int l, int8_t** kq, int8_t** vq, float** ks, float** vs);
/* Layer l's K/V storage of any dtype: f32, f16 bits or int8 codes [max_seq, row_dim]. */
void orc_model_kv_raw(orc_model* m, int l, void** k, void** v);
/* Timing support for the CPU baseline: marks `used` rows of every layer as
 * filled with seeded pseudo-random codes and scales, so decode steps can be
 * timed at a long context without a CPU prefill. */
void orc_model_fill_kv(orc_model* m, int used, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif
