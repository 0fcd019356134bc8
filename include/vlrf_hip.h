/*
 * vlrf_hip.h - C ABI of the MI355X (gfx950) HIP decode backend for VLRF.
 *
 * Plain C: opaque handles, device pointers, sizes and int status codes.  No
 * exception crosses this boundary; every entry point returns VLRF_HIP_OK (0)
 * or a negative status, and vlrf_hip_last_error() gives the message of the
 * calling thread's last failure.  On a nonzero status a caller keeps the
 * reference's behaviour of running the CPU op instead
 * (reference include/backend/backend.hpp:128-176: "falls back to CPU").
 *
 * Device work is queued on the context's own HIP stream and is asynchronous
 * unless stated otherwise; vlrf_hip_sync() waits for it.  A context, and
 * every handle made from it, is used by one host thread at a time (the
 * reference serialises per model: src/api/vlrf_api.cpp:84,370).
 *
 * Each declaration names the reference interface it replaces or serves.
 */
#ifndef VLRF_HIP_H
#define VLRF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------------- */
#define VLRF_HIP_OK            0
#define VLRF_HIP_ERR_ARG      -1   /* bad argument / unsupported shape          */
#define VLRF_HIP_ERR_RUNTIME  -2   /* HIP runtime error (message has the detail) */
#define VLRF_HIP_ERR_NOMEM    -3   /* device allocation failed                  */
#define VLRF_HIP_ERR_OVERFLOW -4   /* KV cache capacity exceeded                */
#define VLRF_HIP_ERR_NODEV    -5   /* no usable gfx950 device                    */

/* ---- data types: GGML type ids, as the reference's GGUF reader uses them
 * (tools/converter/convert_gguf.py GGMLType) -------------------------------- */
#define VLRF_HIP_DT_F32   0
#define VLRF_HIP_DT_Q4_0  2
#define VLRF_HIP_DT_Q8_0  8

/* KV cache dtypes: reference include/model/kv_cache.hpp:36-40 (KVCacheDType). */
#define VLRF_HIP_KV_F32   0
#define VLRF_HIP_KV_F16   1   /* the reference's f32_to_f16 (kv_cache.hpp:68-97), bit-exact */
#define VLRF_HIP_KV_Q8_0  2

typedef struct vlrf_hip_ctx*    vlrf_hip_ctx_t;
typedef struct vlrf_hip_weight* vlrf_hip_weight_t;
typedef struct vlrf_hip_kv*     vlrf_hip_kv_t;
typedef struct vlrf_hip_model*  vlrf_hip_model_t;

/* ============================================================================
 * Context, device memory, streams
 * Replaces: IBackend::{type,device_info,is_available,synchronize,to_device,
 * to_host} (reference include/backend/ibackend.hpp:48-58) and
 * BackendRegistry::try_opencl/try_sycl (backend.hpp:556-570).
 * ========================================================================== */
const char* vlrf_hip_last_error(void);
int   vlrf_hip_device_count(void);
/* Fails with VLRF_HIP_ERR_NODEV when `device` is not a gfx950 GPU. */
int   vlrf_hip_init(int device, vlrf_hip_ctx_t* out);
void  vlrf_hip_shutdown(vlrf_hip_ctx_t ctx);
int   vlrf_hip_device_info(vlrf_hip_ctx_t ctx, char* buf, size_t len);
int   vlrf_hip_sync(vlrf_hip_ctx_t ctx);
void* vlrf_hip_stream(vlrf_hip_ctx_t ctx);            /* the context's hipStream_t */
int   vlrf_hip_malloc(vlrf_hip_ctx_t ctx, size_t bytes, void** dptr);
int   vlrf_hip_free(vlrf_hip_ctx_t ctx, void* dptr);
/* Copies are ordered on the context stream and return when complete. */
int   vlrf_hip_h2d(vlrf_hip_ctx_t ctx, void* dst, const void* src, size_t bytes);
int   vlrf_hip_d2h(vlrf_hip_ctx_t ctx, void* dst, const void* src, size_t bytes);
int   vlrf_hip_memset(vlrf_hip_ctx_t ctx, void* dst, int value, size_t bytes);
/* Device-to-device copy, queued on the context stream (does not wait). */
int   vlrf_hip_d2d(vlrf_hip_ctx_t ctx, void* dst, const void* src, size_t bytes);
/* Event timing on the context stream: records start/stop around queued work. */
int   vlrf_hip_timer_start(vlrf_hip_ctx_t ctx);
int   vlrf_hip_timer_stop(vlrf_hip_ctx_t ctx, float* ms);  /* waits for the stop event */

/* ============================================================================
 * Attention
 * ========================================================================== */
/* Fused scaled-dot-product attention over f32 K/V, batched per head:
 * Q [n_h,T,d_h], K/V [n_h,ctx_len,d_h], O [n_h,T,d_h]; d_h <= 128.
 * Causal rule: key j is masked for query i when j > i + (ctx_len - T).
 * Replaces: IBackend::sdp_attention (ibackend.hpp:79-82) and the CPU
 * AttentionBlock::flash_attn_head per head (attention.hpp:207-309, 431-442). */
int vlrf_hip_attn_f32(vlrf_hip_ctx_t ctx, const float* Q, const float* K, const float* V,
                      float* O, int n_h, int T, int ctx_len, int d_h, float scale, int causal);

/* ============================================================================
 * KV cache (reference kv_cache.hpp:14-17,132-293), dtype VLRF_HIP_KV_F32, _F16 or
 * _Q8_0 (per token row).  Device layout: per layer, K and V elements
 * [n_kv_heads][max_seq][d_head] (head-major, so one head's history is one
 * contiguous stream): f32, f16 bits, or int8 codes with one f32 scale per
 * token row for K and for V.
 * ========================================================================== */
/* Replaces: KVCache::KVCache (kv_cache.hpp:152-177), per layer. */
int vlrf_hip_kv_create(vlrf_hip_ctx_t ctx, int n_layers, int max_seq, int n_kv_heads,
                       int d_head, int dtype, vlrf_hip_kv_t* out);
void vlrf_hip_kv_destroy(vlrf_hip_kv_t kv);
/* Replaces: KVCache::reset (kv_cache.hpp:179-196): zero data, used = 0. */
int vlrf_hip_kv_reset(vlrf_hip_kv_t kv);
/* Tokens stored so far in `layer` (KVCache::used). */
int vlrf_hip_kv_used(vlrf_hip_kv_t kv, int layer);
/* Replaces: KVCache::append (kv_cache.hpp:215-251): stores T rows of device
 * f32 k/v [T, n_kv_heads*d_head] at positions [used, used+T), then used += T,
 * bit-exactly as the reference: Q8_0 quantize_row_q8_0 (kv_cache.hpp:102-117),
 * F16 its f32_to_f16 (:68-97, half-up rounding, flush to zero), F32 a copy.
 * VLRF_HIP_ERR_OVERFLOW when used+T > max_seq (the reference throws). */
int vlrf_hip_kv_append(vlrf_hip_kv_t kv, int layer, const float* k, const float* v, int T);
/* Copies rows [row0,row0+n) of `layer` to host in the reference's token-major
 * layout: k_q/v_q [n, n_kv_heads*d_head] elements of the cache's dtype (int8
 * codes, f16 bits or f32; the pointers address bytes), k_s/v_s f32 [n] row
 * scales for Q8_0 (ignored otherwise; any pointer may be NULL). Synchronous. */
int vlrf_hip_kv_read(vlrf_hip_kv_t kv, int layer, int row0, int n, int8_t* k_q, int8_t* v_q,
                     float* k_s, float* v_s);
/* Replaces: KVCache::dequant_into (kv_cache.hpp:259-286): device f32
 * K_out/V_out [ctx_len, n_kv_heads*d_head], token-major like the reference. */
int vlrf_hip_kv_dequant(vlrf_hip_kv_t kv, int layer, int ctx_len, float* K_out, float* V_out);
/* Decode attention of one token over the cache (any dtype), GQA-aware:
 * q [n_heads*d_head] (already rotated), out [n_heads*d_head]; query head h
 * reads kv head h/(n_heads/n_kv_heads); non-causal over [0, ctx_len).  At
 * d_head 64 and ctx_len <= 8192 one launch (each head's context in at most 16
 * chunks, merged by the head's last workgroup), else split-K + a combine.
 * Replaces the decode branch of AttentionBlock::forward: dequant_into +
 * reshape/expand_kv_heads + sdp_heads (attention.hpp:127-176). */
int vlrf_hip_attn_decode(vlrf_hip_kv_t kv, int layer, const float* q, float* out,
                         int n_heads, int ctx_len, float scale);
/* vlrf_hip_attn_decode that allocates nothing: no counterpart in the
 * reference; for callers that cannot allocate device memory (HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results; the chunk / split-K partials go to one
 * fixed 2 MiB device array per GPU (resolved at vlrf_hip_init), so n_heads *
 * splits * (d_head + 2) floats must fit in 2^19 (splits = ceil(ctx_len / 64)),
 * otherwise VLRF_HIP_ERR_ARG; the per-head merge counters are the context's
 * (allocated at vlrf_hip_init).  Calls that overlap on one GPU race. */
int vlrf_hip_attn_decode_noalloc(vlrf_hip_kv_t kv, int layer, const float* q, float* out,
                                 int n_heads, int ctx_len, float scale);

/* ============================================================================
 * Quantized linear: y[M,N] = x[M,K] . W[N,K]^T with W in a GGUF block format.
 * Replaces: compute::linear -> IBackend::gemm(x, W, y, 1, 0, false, true)
 * (compute.hpp:58-68, ibackend.hpp:61-63) for weights that the converter
 * would otherwise dequantize offline (convert_gguf.py:233-263).
 * ========================================================================== */
/* Host blocks in the GGUF row layout: row n holds K/32 blocks of
 * Q8_0 [f16 d][32 x int8] (34 B) or Q4_0 [f16 d][16 B: byte j = elements 2j
 * (low nibble) and 2j+1 (high nibble)] (18 B); F32 is plain [N][K].
 * Weights stay resident on the device until vlrf_hip_weight_free. K % 32 == 0
 * for block types. Synchronous. */
int vlrf_hip_weight_upload(vlrf_hip_ctx_t ctx, const void* host, int dtype, int N, int K,
                           vlrf_hip_weight_t* out);
void vlrf_hip_weight_free(vlrf_hip_weight_t w);
size_t vlrf_hip_weight_bytes(vlrf_hip_weight_t w);   /* device bytes of the packed weight, plus its bf16
                                                       expansion once a GEMM of > 128 rows made it */
/* x, y device f32, M >= 1.  norm_w (nullable, device f32 [K]): x rows
 * are first RMS-normalised with weight norm_w and `eps` (ops.hpp:478-499).
 * residual (nullable, device f32 [M,N], may alias y): added after the product
 * (the residual adds of transformer_block.hpp:149-159).
 * M <= 16 (decode, ops.hpp:238-310 for M = 1..16) computes in f32.  M > 16
 * (prefill, ops.hpp:254-305) runs on the matrix cores: x (normalised) and the
 * decoded weights are rounded to bf16, accumulation is f32; it takes Q8_0 or
 * Q4_0 weights with K % 64 == 0 and uses the context's scratch buffer.
 * Graph capture of the stream: the scratch buffer cannot grow while the
 * stream is captured (VLRF_HIP_ERR_ARG: make the same call once first), and a
 * weight's bf16 expansion is not made then (the GEMM decodes the blocks in its
 * tiles instead, same 1e-2 class). */
int vlrf_hip_qlinear(vlrf_hip_ctx_t ctx, vlrf_hip_weight_t w, const float* x, float* y, int M,
                     const float* norm_w, float eps, const float* residual);

/* FFN gate/up half of FeedForward::forward with the SwiGLU epilogue:
 * h[M,F] = silu(rmsnorm(x).Wg^T) * (rmsnorm(x).Wu^T), silu(g) = g/(1+exp(-g)).
 * Replaces: linear(x, fc1), linear(x, gate), silu_inplace, multiply_inplace
 * (feedforward.hpp:54-62, ops.hpp:409-441).  norm_w nullable as above;
 * wg and wu have the same shape and dtype.  M ranges as vlrf_hip_qlinear. */
int vlrf_hip_qlinear_swiglu(vlrf_hip_ctx_t ctx, vlrf_hip_weight_t wg, vlrf_hip_weight_t wu,
                            const float* x, float* h, int M, const float* norm_w, float eps);

/* ============================================================================
 * Edge ops
 * ========================================================================== */
/* Replaces: ops::rms_norm (ops.hpp:478-499). x/out device [rows, D]. */
int vlrf_hip_rmsnorm(vlrf_hip_ctx_t ctx, const float* x, const float* w, float* out,
                     int rows, int D, float eps);
/* Replaces: RopeCache::apply (rope.hpp:75-99) with tables built on the host
 * exactly as RopeCache::init (rope.hpp:49-71): x device [T, n_heads*d_head]
 * rotated in place (half-split pairs) for positions pos_offset+t < max_seq. */
int vlrf_hip_rope(vlrf_hip_ctx_t ctx, float* x, int T, int n_heads, int d_head,
                  int pos_offset, int max_seq, float theta);

/* ============================================================================
 * The engine's remaining per-op backend calls (IBackend, ibackend.hpp:61-70),
 * on device f32 buffers, for GPT-2-family models.  Asynchronous on the
 * context's stream.
 * ========================================================================== */
/* Replaces: IBackend::gemm -> ops::gemm (ops.hpp:170-310): C[M,N] =
 * beta*C + alpha*op(A).op(B), op(A) [M,K] = transA ? A^T : A (A row-major with
 * leading dimension lda), op(B) [K,N] likewise; beta == 0 writes C without
 * reading it.  f32 FMA accumulation. */
int vlrf_hip_gemm_f32(vlrf_hip_ctx_t ctx, const float* A, const float* B, float* C, int M, int N, int K,
                      int lda, int ldb, int ldc, float alpha, float beta, int transA, int transB);
/* Replaces: IBackend::layer_norm -> ops::layer_norm (ops.hpp:443-476) over rows
 * of D: (x - mean) * (1/sqrt(var + eps)) * w + b. */
int vlrf_hip_layer_norm(vlrf_hip_ctx_t ctx, const float* x, const float* w, const float* b, float* out,
                        int rows, int D, float eps);
/* Replaces: IBackend::softmax_inplace -> ops::softmax_inplace (ops.hpp:501-540)
 * over rows of D: exp(x - max) * (1/(sum + 1e-9)). */
int vlrf_hip_softmax(vlrf_hip_ctx_t ctx, float* x, int rows, int D);
/* Replaces: IBackend::gelu_inplace -> ops::gelu_inplace (ops.hpp:390-404), the
 * tanh approximation. */
int vlrf_hip_gelu(vlrf_hip_ctx_t ctx, float* x, int64_t n);
/* Replaces: IBackend::add_inplace -> ops::add_inplace (ops.hpp:344-356). */
int vlrf_hip_add(vlrf_hip_ctx_t ctx, float* dst, const float* src, int64_t n);

/* ============================================================================
 * Host-side format helpers (no device needed)
 * ========================================================================== */
/* This build's block encoders (the reference ships decoders only):
 * Q8_0: d = amax/127 stored as f16, q = round-half-away(x / f32(d16)) in [-127,127];
 * Q4_0: d = (signed max-magnitude element)/-8 stored as f16,
 *       nibble = min(15, (int)(x / f32(d16) + 8.5)).
 * n % 32 == 0. dst holds n/32 blocks. */
int vlrf_quantize_q8_0(const float* src, void* dst, int64_t n);
int vlrf_quantize_q4_0(const float* src, void* dst, int64_t n);
/* Block decode, convert_gguf.py:233-263 semantics. */
int vlrf_dequantize(const void* src, int dtype, float* dst, int64_t n);
/* Synthetic seeded data: counter-based (splitmix64 + Box-Muller in double),
 * identical on any host.  out[i] = std * N(0,1) sample i of stream `stream`. */
int vlrf_synth_normal(uint64_t seed, uint64_t stream, float std_dev, float* out, int64_t n);
/* Uniform token ids in [0, vocab). */
int vlrf_synth_tokens(uint64_t seed, uint64_t stream, int vocab, int32_t* out, int64_t n);

/* ============================================================================
 * Decoder model (Llama-style: RMSNorm, RoPE half-split, SwiGLU, GQA; F32, F16
 * or Q8_0 KV cache).
 * Replaces the decode hot loop of TransformerModel::forward/generate
 * (transformer.hpp:335-424, 439-547) with a device-resident step: only token
 * ids cross PCIe.
 * ========================================================================== */
typedef struct vlrf_hip_model_config {
    int32_t vocab_size, d_model, d_ff, n_heads, n_kv_heads, n_layers, max_seq_len;
    float   norm_eps, rope_theta;
    int32_t weight_dtype;   /* VLRF_HIP_DT_Q8_0 / VLRF_HIP_DT_Q4_0 / VLRF_HIP_DT_F32 for the projections */
    int32_t kv_dtype;       /* VLRF_HIP_KV_F32 / _F16 / _Q8_0: ModelConfig::kv_cache_dtype (config.hpp),
                               the reference's KVCacheDType numbering, whose default F32 is 0 */
} vlrf_hip_model_config;

int  vlrf_hip_model_create(vlrf_hip_ctx_t ctx, const vlrf_hip_model_config* cfg,
                           vlrf_hip_model_t* out);
void vlrf_hip_model_destroy(vlrf_hip_model_t m);
/* Sets one tensor by its reference WeightMap name (transformer.hpp:566-629 plus
 * "layers.{l}.ffn.gate.weight"): embed.weight / lm_head.weight /
 * ln_final.weight, layers.{l}.{ln1,ln2}.weight,
 * layers.{l}.attn.{q,k,v,o}_proj.weight, layers.{l}.ffn.{gate,fc1,fc2}.weight.
 * Norm weights and the embedding are f32 (dtype VLRF_HIP_DT_F32); projection and
 * LM-head weights are in `dtype` host blocks.  Synchronous. */
int  vlrf_hip_model_set_weight(vlrf_hip_model_t m, const char* name, const void* host,
                               int dtype, int rows, int cols);
/* The configuration the model was created with. */
int  vlrf_hip_model_get_config(vlrf_hip_model_t m, vlrf_hip_model_config* out);
/* TransformerModel::reset_kv_cache (transformer.hpp:311-315). */
int  vlrf_hip_model_reset(vlrf_hip_model_t m);
int  vlrf_hip_model_used(vlrf_hip_model_t m);
/* One decode step of token `token` (= forward({token}, true) + argmax,
 * transformer.hpp:472-482): returns the greedy next id in *next and, when
 * logits is non-NULL, copies the logits [vocab] to host. Synchronous. */
int  vlrf_hip_model_step(vlrf_hip_model_t m, int32_t token, int32_t* next, float* logits);
/* Feeds `n` tokens one step at a time (the prompt), without reading logits
 * back; *next receives the greedy id after the last one.  The f32 decode
 * path: the KV cache it leaves matches the reference's prefill to f32
 * rounding, so generation after it reproduces the reference's streams. */
int  vlrf_hip_model_prefill(vlrf_hip_model_t m, const int32_t* ids, int n, int32_t* next);
/* Batched prefill on the matrix cores: TransformerModel::forward over the
 * whole prompt (transformer.hpp:335-424; AttentionBlock::forward with T = n,
 * attention.hpp:89-186: causal attention over the Q8_0 cache, K/V appended
 * before attending).  GEMMs and attention take bf16 operands with f32
 * accumulation (the 1e-2 class), norms / RoPE / KV quantization are f32.
 * Needs Q8_0/Q4_0 weights and d_model, d_ff multiples of 64.  *next receives
 * the greedy id of the last row.  Synchronous. */
int  vlrf_hip_model_prefill_mfma(vlrf_hip_model_t m, const int32_t* ids, int n, int32_t* next);
/* The same layers over T embedded rows: x (device f32 [T][d_model], the first
 * layer's input) is not modified; out (device f32 [T][d_model], may alias x)
 * receives the residual stream after the last layer.  Appends T positions to
 * the KV cache.  Synchronous. */
int  vlrf_hip_model_forward_hidden(vlrf_hip_model_t m, const float* x, int T, float* out);
/* Greedy generation of n_steps tokens starting from `first` entirely on the
 * device (token feedback on the GPU, replayed HIP graph); out_ids (host,
 * n_steps) receives the generated ids.  Synchronous. */
int  vlrf_hip_model_generate(vlrf_hip_model_t m, int32_t first, int n_steps, int32_t* out_ids);
/* Queues n_steps greedy steps without waiting (for timing); the ids stay on
 * the device and are fetched by vlrf_hip_model_read_generated. */
int  vlrf_hip_model_generate_async(vlrf_hip_model_t m, int32_t first, int n_steps);
int  vlrf_hip_model_read_generated(vlrf_hip_model_t m, int32_t* out_ids, int n);
/* Rows [row0,row0+n) of layer `layer` of the model's KV cache, as
 * vlrf_hip_kv_read (token-major elements of the cache dtype, Q8_0 row scales).  Synchronous. */
int  vlrf_hip_model_kv_read(vlrf_hip_model_t m, int layer, int row0, int n, int8_t* k_q,
                            int8_t* v_q, float* k_s, float* v_s);
/* Measurement, no reference counterpart (the reference times whole calls,
 * vlrf_cli's tok/s): n_steps greedy decode steps from token `first`, as
 * vlrf_hip_model_generate_async, with the step's kernels queued one by one and
 * every launch timed by its own start/stop events (hipExtLaunchKernel stamps
 * them with the kernel's begin and end).  Per launch kind: us[k] = summed
 * kernel time in microseconds, calls[k] = launches.  Advances the position
 * by n_steps (1..256); synchronous. */
enum {
    VLRF_HIP_LK_QKV = 0,      /* RMSNorm + QKV projection (fused with RoPE, the KV append and attention) */
    VLRF_HIP_LK_ATTN = 1,     /* stand-alone decode attention (when not fused) */
    VLRF_HIP_LK_O = 2,        /* O projection (+ merge of the attention partials) + residual */
    VLRF_HIP_LK_GATE_UP = 3,  /* RMSNorm + gate/up + SwiGLU */
    VLRF_HIP_LK_DOWN = 4,     /* down projection + residual */
    VLRF_HIP_LK_LM_HEAD = 5,  /* final RMSNorm + LM head */
    VLRF_HIP_LK_ARGMAX = 6,   /* greedy argmax + step state */
    VLRF_HIP_LK_OTHER = 7,    /* embedding gather, attention combine */
    VLRF_HIP_LK_KINDS = 8
};
int  vlrf_hip_model_time_launches(vlrf_hip_model_t m, int32_t first, int n_steps, double us[8], int calls[8]);
/* Device bytes read per decode step at context length ctx_len, by stream:
 * [0] projection + LM-head weights, [1] KV cache, [2] everything else
 * (norm weights, embedding row, activations).  For roofline accounting. */
int  vlrf_hip_model_step_bytes(vlrf_hip_model_t m, int ctx_len, double out[3]);

/* ============================================================================
 * NFW weight files (host side, no device needed) and loading them.
 * Replaces: WeightMap's NFW reader (weights.hpp:58-62 constants, parse_header
 * :289-339, f16 widening :76-96) for versions 1 (f32) and 2 (dtype byte, F32 /
 * F16), extended by version 3: the same layout with block dtypes whose payload
 * is the GGUF blocks (numel/32 blocks, row-major element order), so GGUF
 * Q8_0/Q4_0 tensors are stored as they are instead of being decoded to f32
 * (convert_gguf.py:193-263).  dtype numbers are GGML's.
 * ========================================================================== */
#define VLRF_NFW_F32   0
#define VLRF_NFW_F16   1
#define VLRF_NFW_Q4_0  2   /* 18 B per 32 elements */
#define VLRF_NFW_Q8_0  8   /* 34 B per 32 elements */
typedef struct vlrf_nfw* vlrf_nfw_t;
/* Parses the header and every tensor descriptor; bad magic, unknown version
 * or dtype, inconsistent sizes and truncation are VLRF_HIP_ERR_ARG. */
int  vlrf_nfw_open(const char* path, vlrf_nfw_t* out);
void vlrf_nfw_close(vlrf_nfw_t f);
int  vlrf_nfw_version(vlrf_nfw_t f);
int  vlrf_nfw_count(vlrf_nfw_t f);
/* Index of the tensor called `name`, or -1. */
int  vlrf_nfw_find(vlrf_nfw_t f, const char* name);
/* name (valid until close), dtype, ndim, dims[ndim] (up to 8), numel, payload bytes. */
int  vlrf_nfw_tensor_info(vlrf_nfw_t f, int i, const char** name, int* dtype, int* ndim,
                          int32_t* dims, int64_t* numel, int64_t* bytes);
/* Raw payload of tensor i into dst (cap bytes). */
int  vlrf_nfw_read(vlrf_nfw_t f, int i, void* dst, int64_t cap);
/* Tensor i as f32 (F16 widened as weights.hpp:76-96, blocks decoded as
 * convert_gguf.py:233-263) into dst (n floats). */
int  vlrf_nfw_read_f32(vlrf_nfw_t f, int i, float* dst, int64_t n);
/* Sets every tensor of an NFW file that the model uses, by the engine's names
 * (vlrf_hip_model_set_weight): norms and the embedding as f32, projections in
 * the model's weight dtype (blocks uploaded unchanged), the LM head as blocks
 * or f32.  All-zero bias tensors are accepted and dropped; a non-zero bias or
 * an f32 projection for a block-typed model is VLRF_HIP_ERR_ARG.  *n_loaded
 * receives the number of tensors set.  Synchronous. */
int  vlrf_hip_model_load_nfw(vlrf_hip_model_t m, const char* path, int* n_loaded);

#ifdef __cplusplus
}
#endif
#endif /* VLRF_HIP_H */
