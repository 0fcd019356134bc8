// internal.hpp - shared declarations of the gfx950 decode backend.
//
// Device code here targets CDNA4 wave64 only.  Host-side launchers check every
// operand shape against what their kernel and grid assume before launching.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/vlrf_hip.h"

namespace vlrf_hip {

// ---- error handling ---------------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

#define VH_CHECK(expr)                                                            \
    do {                                                                          \
        hipError_t e_ = (expr);                                                   \
        if (e_ != hipSuccess) {                                                   \
            ::vlrf_hip::set_error("%s failed: %s (%s:%d)", #expr,                 \
                                  hipGetErrorString(e_), __FILE__, __LINE__);     \
            return VLRF_HIP_ERR_RUNTIME;                                          \
        }                                                                         \
    } while (0)

#define VH_ARG(cond, ...)                                                         \
    do {                                                                          \
        if (!(cond)) {                                                            \
            ::vlrf_hip::set_error(__VA_ARGS__);                                   \
            return VLRF_HIP_ERR_ARG;                                              \
        }                                                                         \
    } while (0)

// Checks the launch that was just queued.
#define VH_LAUNCHED()                                                             \
    do {                                                                          \
        hipError_t e_ = hipGetLastError();                                        \
        if (e_ != hipSuccess) {                                                   \
            ::vlrf_hip::set_error("kernel launch failed: %s (%s:%d)",             \
                                  hipGetErrorString(e_), __FILE__, __LINE__);     \
            return VLRF_HIP_ERR_RUNTIME;                                          \
        }                                                                         \
    } while (0)

// ---- per-launch kernel timing ------------------------------------------------
// While a LaunchTimer is installed on the calling thread, launches made with
// VH_LAUNCH take its next start/stop event pair: hipExtLaunchKernel stamps them
// with the kernel's own begin and end, so each launch's duration is measured
// without a marker between launches.  `cur_kind` labels the launches that
// follow (the decode step sets it per phase).  With no timer, a plain launch.
struct LaunchTimer {
    hipEvent_t* start = nullptr;
    hipEvent_t* stop = nullptr;
    int* kind = nullptr;
    int n = 0, cap = 0, cur_kind = 0;
};
LaunchTimer*& launch_timer();   // the calling thread's timer (null: none)

#define VH_LAUNCH(K, GRID, BLOCK, SHM, S, ...)                                                      \
    do {                                                                                            \
        ::vlrf_hip::LaunchTimer* lt_ = ::vlrf_hip::launch_timer();                                  \
        if (lt_ && lt_->n < lt_->cap) {                                                             \
            lt_->kind[lt_->n] = lt_->cur_kind;                                                      \
            hipExtLaunchKernelGGL(K, GRID, BLOCK, SHM, S, lt_->start[lt_->n], lt_->stop[lt_->n], 0, \
                                  __VA_ARGS__);                                                     \
            ++lt_->n;                                                                               \
        } else {                                                                                    \
            hipLaunchKernelGGL(K, GRID, BLOCK, SHM, S, __VA_ARGS__);                                \
        }                                                                                           \
    } while (0)

// ---- device-resident quantized weight ---------------------------------------
// Q8_0: q = int8 [N][K] (the block's 32 codes, rows contiguous),
//       d = f16 [N][K/32] (block scales).
// Q4_0: q = uint8 [N][K/2], byte j of a row's block b holds elements
//       32b+2j (low nibble) and 32b+2j+1 (high nibble), as the GGUF block;
//       d = f16 [N][K/32].
// F32:  f = float [N][K].
struct DevWeight {
    int dtype = VLRF_HIP_DT_F32;
    int N = 0, K = 0;
    uint8_t* q = nullptr;
    __half* d = nullptr;
    float* f = nullptr;
    // bf16(code * scale) of every element, [N][K]: made by the first GEMM with
    // more than 128 rows of A (weight_expand_bf16), dropped when rows are
    // uploaded or the weight is released.  A cache of q / d, hence mutable.
    mutable uint16_t* bf = nullptr;
};

size_t weight_device_bytes(int dtype, int N, int K);
// Splits host GGUF blocks of rows [row0,row0+nrows) into the device arrays.
int weight_upload_rows(hipStream_t s, DevWeight& w, const void* host, int row0, int nrows);
int weight_alloc(DevWeight& w, int dtype, int N, int K);
void weight_release(DevWeight& w);
// Makes w.bf on stream s unless it exists or VLRF_HIP_PREFILL_BF16=0; false
// (the GEMM then decodes codes in registers) when disabled or out of memory.
bool weight_expand_bf16(hipStream_t s, const DevWeight& w);

// ---- KV cache ------------------------------------------------------------------
// k and v address [n_kv][max_seq][d_head] elements of the layer's dtype: int8
// codes (Q8_0, with one f32 scale per token row in ks/vs), f16 bits or f32.
struct KVLayer {
    int8_t* k = nullptr;
    int8_t* v = nullptr;
    float* ks = nullptr;   // [max_seq], Q8_0 only
    float* vs = nullptr;
    int dtype = VLRF_HIP_KV_Q8_0;
};

__host__ __device__ inline int kv_elem_bytes(int dtype) {
    return dtype == VLRF_HIP_KV_F32 ? 4 : dtype == VLRF_HIP_KV_F16 ? 2 : 1;
}

// KVCache's f32 -> f16 element conversion (kv_cache.hpp:68-97): the mantissa is
// rounded half up (+0x1000 then >> 13), exponents <= 0 flush to signed zero,
// overflow gives inf, NaN keeps one quiet bit.  Not IEEE round-to-nearest-even.
__device__ __forceinline__ uint16_t f32_to_f16_kv(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000u, mant = x & 0x7FFFFFu;
    int e = (int)((x >> 23) & 0xFFu) - 112;
    if (((x >> 23) & 0xFFu) == 0xFFu) return (uint16_t)(sign | 0x7C00u | (mant ? 0x0200u : 0u));
    if (e <= 0) return (uint16_t)sign;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    uint32_t r = (mant + 0x1000u) >> 13;
    if (r & 0x400u) {
        r = 0;
        if (++e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | r);
}

// f16 -> f32 widening: exact (v_cvt_f32_f16); the cache never holds the
// subnormals where the reference's loop and the hardware could differ.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)h));
}

// Rows [row0, row0+n) of a head-major cache layer to host in the reference's
// token-major layout (synchronous).
int kv_rows_to_host(hipStream_t s, const KVLayer& L, int G, int D, int max_seq, int row0, int n,
                    int8_t* k_q, int8_t* v_q, float* k_s, float* v_s);

// ---- launchers (all queue on `s`) -----------------------------------------------
// y[M,N] = (norm_w ? rmsnorm(x) : x) . W^T (+ residual)
int launch_qlinear(hipStream_t s, const DevWeight& w, const float* x, float* y, int M,
                   const float* norm_w, float eps, const float* residual);
// y = rmsnorm(table[*row]) . W^T (M = 1, Q8_0/Q4_0): the embedding gather fused
// into the first projection; the raw row is also copied to x_copy.
// y = W . x + residual (M = 1) where x is the decode attention output in its
// chunked form (DecodeFuse::chunks, nch chunks per head), merged in the GEMV's
// prologue.
int launch_qlinear_merge(hipStream_t s, const DevWeight& w, const float* chunks, int nch, const float* residual,
                         float* y, int head_dim = 64);
// Most chunks launch_qlinear_merge takes for w (0: not on that path).
int qlinear_merge_max_chunks(const DevWeight& w);
int launch_qlinear_gather(hipStream_t s, const DevWeight& w, const float* table, const int* row,
                          float* x_copy, float* y, const float* norm_w, float eps);
bool qlinear_gather_supported(const DevWeight& w);
// h[M,N] = silu(rmsnorm(x).Wg^T) * (rmsnorm(x).Wu^T)
int launch_qlinear_swiglu(hipStream_t s, const DevWeight& wg, const DevWeight& wu,
                          const float* x, float* h, int M, const float* norm_w, float eps);

int launch_rmsnorm(hipStream_t s, const float* x, const float* w, float* out, int rows, int D,
                   float eps);

// ---- the engine's remaining per-op backend calls (kernels/ops.hip) ---------------
int launch_gemm_f32(hipStream_t s, const float* A, const float* B, float* C, int M, int N, int K, int lda,
                    int ldb, int ldc, float alpha, float beta, bool transA, bool transB);
int launch_layer_norm(hipStream_t s, const float* x, const float* w, const float* b, float* out, int rows, int D,
                      float eps);
int launch_softmax(hipStream_t s, float* x, int rows, int D);
int launch_gelu(hipStream_t s, float* x, int64_t n);
int launch_add(hipStream_t s, float* dst, const float* src, int64_t n);

// ---- prefill (MFMA) path: bf16 operands, f32 accumulate -------------------------
// out[r] = bf16(w ? rmsnorm(x[r]) * w : x[r]) for rows x D
int launch_rows_to_bf16(hipStream_t s, const float* x, const float* w, uint16_t* out, int rows, int D,
                        float eps);
// y[M,N] = a[M,K] . W^T (+ residual), a in bf16, W Q8_0/Q4_0 with K % 64 == 0.
// `part`: device memory of qgemm_part_bytes(w, M, false) bytes for the K-split
// partial sums of 17 <= M <= 128 (without it such a call takes the unsplit
// register-staged kernel).
int launch_qgemm(hipStream_t s, const DevWeight& w, const uint16_t* a, int M, const float* residual,
                 float* y, float* part = nullptr);
// h[M,N] = silu(a.Wg^T) * (a.Wu^T), stored as bf16 (h_bf16) or f32
int launch_qgemm_swiglu(hipStream_t s, const DevWeight& wg, const DevWeight& wu, const uint16_t* a,
                        int M, void* h, bool h_bf16, float* part = nullptr);
size_t qgemm_part_bytes(const DevWeight& w, int M, bool swiglu);
// Small M (2..16) on the matrix cores with f32-class accuracy (x split into
// bf16 hi + lo): y = x.W0^T (+ residual), or silu(x.W0^T) * (x.W1^T) when w1
// is given, in one launch.  Per-slice partial sums go to scratch
// (qlinear_small_scratch bytes); tile_ctr holds kSmallTileCtrStride ints per
// row tile for at least qlinear_small_tiles(N) tiles, zero between calls.
constexpr int kSmallTileCtrStride = 32;   // ints per row-tile counter (its own 128-byte line)
constexpr int kSmallMaxTiles = 4096;      // row tiles a context's counters cover (N <= 262144 at 64 rows a tile)
bool qlinear_small_supported(const DevWeight& w);
size_t qlinear_small_scratch(int N, int K, bool two);
int qlinear_small_tiles(int N);
int launch_qlinear_small(hipStream_t s, const DevWeight& w0, const DevWeight* w1, const float* x,
                         int M, const float* norm_w, float eps, const float* residual, float* scratch,
                         int* tile_ctr, int tile_ctr_tiles, float* y);
int launch_rope(hipStream_t s, float* x, int T, int n_heads, int d_head, int pos_offset,
                int max_seq, const float* cos_t, const float* sin_t);

// Quantize T rows into the cache at positions pos(+t); pos comes from *pos_dev
// when non-null.  Optionally applies RoPE to q (n_q_heads) and k first (decode
// fusion: q rotated in place, k rotated before quantization).
int launch_kv_append(hipStream_t s, const KVLayer& L, int n_kv, int d_head, int max_seq,
                     const float* k, const float* v, int T, int pos, const int* pos_dev);
int launch_rope_append(hipStream_t s, const KVLayer& L, float* q, const float* k,
                       const float* v, int n_heads, int n_kv, int d_head, int max_seq,
                       const int* pos_dev, const float* cos_t, const float* sin_t);
int launch_kv_dequant(hipStream_t s, const KVLayer& L, int n_kv, int d_head, int max_seq,
                      int ctx_len, float* K_out, float* V_out);
// Prefill: RoPE on k of T tokens of a [T][ld] QKV buffer at positions
// pos0.., then the cache append of their K/V rows (q is left as it is: the
// prefill attention rotates it as it loads it).
int launch_prefill_rope_append(hipStream_t s, const KVLayer& L, const float* qkv, int ld, int T, int n_heads,
                               int n_kv, int d_head, int max_seq, int pos0, const float* cos_t,
                               const float* sin_t);
// x[t] = table[ids[t]] for T device ids
int launch_embed_rows(hipStream_t s, const float* table, const int* ids, float* x, int T, int D);
// Causal attention of T new tokens (positions pos0..) over the cache on the
// matrix cores: q (f32, not yet rotated) read from the [T][ld] QKV buffer and
// rotated by the RoPE tables on load; the cache rows [0, pos0+T) dequantized
// to bf16, out bf16 [T][n_heads*d_head].
int launch_attn_prefill(hipStream_t s, const float* qkv, int ld, const KVLayer& L, int T, int pos0,
                        int n_heads, int n_kv, int d_head, int max_seq, float scale, const float* cos_t,
                        const float* sin_t, uint16_t* out);

// Decode fusion of the attention kernel (model step): RoPE of q and of the
// token's k at the device position, and the append of its K/V row.
struct DecodeFuse {
    const float* k_new = nullptr;   // [n_kv*d_head] unrotated k of the token
    const float* v_new = nullptr;
    const float* cos_t = nullptr;   // [max_seq][d_head/2]
    const float* sin_t = nullptr;
    int8_t* kq_w = nullptr;         // the layer's cache elements, as bytes (same as kc/vc)
    int8_t* vq_w = nullptr;
    float* ks_w = nullptr;          // Q8_0 row scales
    float* vs_w = nullptr;
    int n_kv = 0, max_seq = 0;
    // Chunked form (nch > 0, see attn_decode_chunks): per query head and chunk
    // of the cache, the partial (acc[0..d-1] unnormalised, m, l) at
    // chunks[(h*nch + s)*kAttnChunkStride], merged by the next GEMV's prologue
    // (launch_qlinear_merge) instead of a combine launch.
    float* chunks = nullptr;
    int nch = 0;
};
constexpr int kAttnChunkStride = 68, kAttnMaxChunks = 16;
constexpr int kAttnChunkRows = 512;   // cache rows per chunk of the chunked form
// Chunks of the decode attention's chunked form for a cache of cap rows, or 0
// where it does not apply (d_head != 64, more than 8 KV heads, caches the
// single-pass kernel covers, or more than kAttnMaxChunks chunks).
int attn_decode_chunks(int cap, int d_head, int n_kv);
// The d_head 128 chunked form (Q8_0 cache): nch chunks of 512 rows, whose
// partials (acc[0..127], m, l; d_head + 4 floats) are followed by the new
// key's, nch + 1 per head.  0 where it does not apply.
int attn_decode_chunks128(int cap, int n_heads, int n_kv, int kv_dtype);

// Split-K decode attention over K/V elements of kv_dtype (VLRF_HIP_KV_Q8_0 codes
// with row scales ks/vs, VLRF_HIP_KV_F16 bits, VLRF_HIP_KV_F32) laid out
// [n_kv][head_stride/d][d]: a cache layer (head_stride = max_seq*d) or plain
// f32 K/V.  ctx from *ctx_dev (+1 when fused) when non-null.  part must hold
// n_heads*n_splits*(d+2) floats.  ctr (unfused, host context length, d 64): a
// context's counter array (kSmallTileCtrStride ints per query head, zero
// between calls); with it the attention and the chunk merge run in one launch.
int attn_decode_splits(int max_ctx);
int launch_attn_decode(hipStream_t s, const float* q, const void* kc, const void* vc, const float* ks,
                       const float* vs, int kv_dtype, long head_stride, int n_heads, int n_kv, int d_head,
                       int ctx_len, const int* ctx_dev, int n_splits, float scale, float* part, float* out,
                       const DecodeFuse* fuse = nullptr, int* ctr = nullptr);
int launch_attn_f32_tiled(hipStream_t s, const float* Q, const float* K, const float* V,
                          float* O, int n_h, int T, int ctx_len, int d_h, float scale,
                          int causal);

// A layer's QKV projection and its chunked decode attention in one launch
// (kernels/qkv_attn.hip): the projection's rows are published as tagged words
// (value | epoch << 32, epoch = state[3]) in `tags`, which the attention's
// workgroups wait for.  Per query head, fz.chunks holds fz.nch + 1 partials:
// the cache chunks (the token's row left out) and then the token's own key.
constexpr int kQkvAttnMaxD = 2048;   // d_model of the fused form (the new-row workgroup stages q)
struct QkvAttnParams {
    const uint8_t* qa = nullptr;      // Wqkv codes / scales
    const __half* da = nullptr;
    int N = 0, K = 0;                 // d_model + 2*n_kv*64 rows, d_model columns
    const float* x = nullptr;         // the residual stream, or (gather) the embedding table
    float* x_copy = nullptr;          // gather: the token's row is copied here
    const float* norm_w = nullptr;    // ln1
    float eps = 0.f;
    int nq = 0;                       // projection workgroups (a multiple of 8)
    int na = 0;                       // attention workgroups (then one for the token's K/V row)
    uint64_t* tags = nullptr;         // [N] this layer's tagged projection outputs
    long head_stride = 0;             // cache elements per KV head (max_seq * 64)
    int rep = 1;                      // query heads per KV head
    DecodeFuse fz;                    // RoPE tables, the cache (written at the token's row), chunks
    float scale = 0.f;
    int* state = nullptr;             // [0] token, [1] position, [3] epoch
    int* status = nullptr;            // [4] failure flag, workgroup, phase, layer
    long long limit = 0;              // wall-clock ticks a wait may last
    int layer = 0;
};
bool qkv_attn_supported(int w_dtype, int N, int K, int nch, int n_kv);
int qkv_attn_blocks(int rep, int n_kv, int nch);
int launch_qkv_attn(hipStream_t s, const QkvAttnParams& p, int w_dtype, int kv_dtype, bool gather);

// The LM head's GEMV (RMSNorm fused, the row loop: N > 8 * 768 rows) writing
// besides the logits one (max, first row) pair per workgroup to pairs[*npairs]
// (*npairs <= 512), reduced by launch_argmax_pairs_step.
bool qlinear_argmax_supported(const DevWeight& w);
int launch_qlinear_argmax(hipStream_t s, const DevWeight& w, const float* x, float* y, const float* norm_w,
                          float eps, float2* pairs, int* npairs);
int launch_argmax_pairs_step(hipStream_t s, const float2* pairs, int np, int* state, int* gen_ids, int gen_cap);

int launch_embed(hipStream_t s, const float* table, const int* tok_dev, float* x, int D);
// argmax over logits[n] (first maximum) -> state[0] (token), appends to
// gen_ids[state[2]++], state[1] (position) += 1.
int launch_argmax_step(hipStream_t s, const float* logits, int n, int* state, int* gen_ids,
                       int gen_cap);

// ---- wave64 reductions (DPP within rows of 16, then cross-row shuffles) -------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// f32 -> bf16 bits, round to nearest even (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two f32 -> packed bf16 (lo in bits 0-15), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
    const bf16x2_v v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// Row exchanges in VALU (no LDS round trip): v_permlane16_swap(a, b) returns
// ([a row0, b row0, a row2, b row2], [a row1, b row1, a row3, b row3]) over the
// wave's four 16-lane rows, v_permlane32_swap(a, b) ([a lo, b lo], [a hi, b hi])
// over its 32-lane halves.  Swapping a value with itself puts the partner
// row's (half's) value beside the lane's own.
__device__ __forceinline__ float2 swap_rows16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float2 swap_halves32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum / max over the wave; every lane gets the result (the pairwise order is
// the same in all lanes: row 0 + row 1, then half 0 + half 1).
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);   // row_half_mirror
    v += dpp_f<0x140>(v);   // row_mirror
    float2 t = swap_rows16(v, v);
    v = t.x + t.y;
    t = swap_halves32(v, v);
    return t.x + t.y;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    float2 t = swap_rows16(v, v);
    v = fmaxf(t.x, t.y);
    t = swap_halves32(v, v);
    return fmaxf(t.x, t.y);
}

}  // namespace vlrf_hip
