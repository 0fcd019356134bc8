/*
 * vlrf_oracle.c - CPU restatement of the VLRF reference decode path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP backend.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library;
 * the product under vlrf_amd/ never does.
 *
 * Each function follows one reference function (file:line under
 * /root/reference) in operation order, so that with the same thread count it
 * reproduces the reference's f32 results bit for bit:
 *   - scalar code is compiled with -ffp-contract=off, as the reference's
 *     default GCC build (-mavx -mno-fma) never fuses multiply-adds;
 *   - the reference's AVX2 streaming GEMV, which does use FMA, is restated
 *     with explicit FMA intrinsics in the same accumulation order.
 * Pinning: tests/test_oracle.py checks every function here against the
 * reference compiled from its own sources (oracle/_ref, when present), the
 * reference's own test shapes and tolerances, closed forms and brute force.
 */
#include "vlrf_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>

#define ORC_AVX2 __attribute__((target("avx2,fma")))

/* ------------------------------------------------------------------------ */
/* KV cache F16 element conversion: reference kv_cache.hpp:68-97 (f32_to_f16: */
/* mantissa rounded half up by +0x1000, exponent <= 0 flushed to signed zero, */
/* overflow to inf, NaN keeps only a quiet bit).  The read side widens with   */
/* weights.hpp:76-96 (orc_f16_to_f32 below).                                   */
/* ------------------------------------------------------------------------ */
uint16_t orc_f32_to_f16_kv(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    int32_t e = (int32_t)((x >> 23) & 0xFF) - 127 + 15;
    uint32_t mant = x & 0x7FFFFFu;
    if (((x >> 23) & 0xFF) == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x0200u : 0u));
    if (e <= 0) return (uint16_t)sign;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    uint32_t r = (mant + 0x00001000u) >> 13;
    if (r & 0x0400u) {
        r = 0;
        e += 1;
        if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | r);
}

/* ------------------------------------------------------------------------ */
/* KV cache Q8_0: reference kv_cache.hpp:102-117 (quantize), :119-121 (dequant) */
/* ------------------------------------------------------------------------ */
float orc_quantize_row_q8_0(const float* src, int8_t* dst, int n)
{
    float amax = 0.f;
    for (int i = 0; i < n; ++i) {
        float a = fabsf(src[i]);
        if (amax < a) amax = a;              /* std::max(amax, a) */
    }
    if (amax == 0.f) {
        memset(dst, 0, (size_t)n);
        return 0.f;
    }
    float scale = amax / 127.f;
    float inv = 1.f / scale;
    for (int i = 0; i < n; ++i) {
        long q = lroundf(src[i] * inv);      /* round half away from zero */
        if (q > 127) q = 127;
        if (q < -127) q = -127;
        dst[i] = (int8_t)q;
    }
    return scale;
}

void orc_dequantize_row_q8_0(const int8_t* src, float scale, float* dst, int n)
{
    for (int i = 0; i < n; ++i) dst[i] = (float)src[i] * scale;
}

/* ------------------------------------------------------------------------ */
/* Flash attention, one head: reference attention.hpp:207-309                */
/* 64x64 tiles, online softmax; strides let callers index GQA heads in place  */
/* of the reference's reshape/expand copies (attention.hpp:313-342), which    */
/* move values without changing them.                                         */
/* ------------------------------------------------------------------------ */
void orc_flash_attn_head(const float* Q, int q_stride,
                         const float* K, const float* V, int kv_stride,
                         float* O, int o_stride,
                         int T, int ctx_len, int d_h, float scale, int causal)
{
    enum { BR = 64, BC = 64 };
    float m[BR], l[BR];
    float* acc = (float*)malloc(sizeof(float) * BR * (size_t)d_h);
    float s[BR * BC];
    const float NEG_INF = -INFINITY;

    for (int q0 = 0; q0 < T; q0 += BR) {
        int br = T - q0 < BR ? T - q0 : BR;
        for (int i = 0; i < br; ++i) { m[i] = NEG_INF; l[i] = 0.f; }
        memset(acc, 0, sizeof(float) * (size_t)br * d_h);

        int past = ctx_len - T;
        int k_limit = ctx_len;
        if (causal) {
            int lim = q0 + br + past;
            k_limit = lim < ctx_len ? lim : ctx_len;
        }
        for (int k0 = 0; k0 < k_limit; k0 += BC) {
            int bc = k_limit - k0 < BC ? k_limit - k0 : BC;
            for (int qi = 0; qi < br; ++qi) {
                const float* qrow = Q + (size_t)(q0 + qi) * q_stride;
                for (int kj = 0; kj < bc; ++kj) {
                    const float* krow = K + (size_t)(k0 + kj) * kv_stride;
                    float dot = 0.f;
                    for (int d = 0; d < d_h; ++d) dot += qrow[d] * krow[d];
                    s[qi * BC + kj] = dot * scale;
                }
            }
            if (causal) {
                for (int qi = 0; qi < br; ++qi) {
                    int qpos = q0 + qi + past;
                    for (int kj = 0; kj < bc; ++kj)
                        if (k0 + kj > qpos) s[qi * BC + kj] = NEG_INF;
                }
            }
            for (int qi = 0; qi < br; ++qi) {
                float* srow = &s[qi * BC];
                float blk_max = NEG_INF;
                for (int kj = 0; kj < bc; ++kj)
                    if (blk_max < srow[kj]) blk_max = srow[kj];
                if (blk_max == NEG_INF) continue;            /* fully masked */
                float m_prev = m[qi];
                float m_new = m_prev < blk_max ? blk_max : m_prev;
                float blk_sum = 0.f;
                for (int kj = 0; kj < bc; ++kj) {
                    float p = expf(srow[kj] - m_new);
                    srow[kj] = p;
                    blk_sum += p;
                }
                float corr = (m_prev == NEG_INF) ? 0.f : expf(m_prev - m_new);
                l[qi] = l[qi] * corr + blk_sum;
                float* arow = acc + (size_t)qi * d_h;
                if (corr != 1.f)
                    for (int d = 0; d < d_h; ++d) arow[d] *= corr;
                for (int kj = 0; kj < bc; ++kj) {
                    float w = srow[kj];
                    const float* vrow = V + (size_t)(k0 + kj) * kv_stride;
                    for (int d = 0; d < d_h; ++d) arow[d] += w * vrow[d];
                }
                m[qi] = m_new;
            }
        }
        for (int qi = 0; qi < br; ++qi) {
            float inv_l = (l[qi] > 0.f) ? (1.f / l[qi]) : 0.f;
            const float* arow = acc + (size_t)qi * d_h;
            float* orow = O + (size_t)(q0 + qi) * o_stride;
            for (int d = 0; d < d_h; ++d) orow[d] = arow[d] * inv_l;
        }
    }
    free(acc);
}

/* AttentionBlock::sdp_heads CPU branch: reference attention.hpp:431-442
 * (per head, parallel over heads; each head independent). */
void orc_sdp_attention(const float* Q, const float* K, const float* V, float* O,
                       int n_h, int T, int ctx_len, int d_h, float scale, int causal)
{
#pragma omp parallel for schedule(static)
    for (int h = 0; h < n_h; ++h)
        orc_flash_attn_head(Q + (size_t)h * T * d_h, d_h,
                            K + (size_t)h * ctx_len * d_h,
                            V + (size_t)h * ctx_len * d_h, d_h,
                            O + (size_t)h * T * d_h, d_h,
                            T, ctx_len, d_h, scale, causal);
}

/* ------------------------------------------------------------------------ */
/* RMSNorm: reference ops.hpp:478-499                                         */
/* ------------------------------------------------------------------------ */
void orc_rms_norm(const float* x, const float* w, float* out, int rows, int D, float eps)
{
    for (int r = 0; r < rows; ++r) {
        const float* row = x + (size_t)r * D;
        float* dst = out + (size_t)r * D;
        float ss = 0.f;
        for (int j = 0; j < D; ++j) ss += row[j] * row[j];
        float rms = sqrtf(ss / (float)D + eps);
        float inv = 1.f / rms;
        for (int j = 0; j < D; ++j) dst[j] = row[j] * inv * w[j];
    }
}

/* ------------------------------------------------------------------------ */
/* RoPE: tables reference rope.hpp:49-71, apply rope.hpp:75-99 (half split)   */
/* ------------------------------------------------------------------------ */
void orc_rope_tables(int max_seq, int d_head, float theta, float* cos_t, float* sin_t)
{
    int half = d_head / 2;
    for (int pos = 0; pos < max_seq; ++pos)
        for (int i = 0; i < half; ++i) {
            float freq = 1.f / powf(theta, (float)(2 * i) / (float)d_head);
            float angle = (float)pos * freq;
            cos_t[pos * half + i] = cosf(angle);
            sin_t[pos * half + i] = sinf(angle);
        }
}

void orc_rope_apply(float* x, int T, int n_heads, int d_head, int pos_offset,
                    const float* cos_t, const float* sin_t, int max_seq)
{
    int half = d_head / 2;
    int stride = n_heads * d_head;
    for (int t = 0; t < T; ++t) {
        int pos = pos_offset + t;
        if (pos >= max_seq) break;
        const float* c = cos_t + (size_t)pos * half;
        const float* s = sin_t + (size_t)pos * half;
        for (int h = 0; h < n_heads; ++h) {
            float* v = x + (size_t)t * stride + (size_t)h * d_head;
            for (int i = 0; i < half; ++i) {
                float x0 = v[i], x1 = v[i + half];
                v[i] = x0 * c[i] - x1 * s[i];
                v[i + half] = x1 * c[i] + x0 * s[i];
            }
        }
    }
}

/* SwiGLU elementwise: silu_inplace(g) ops.hpp:409-419, then multiply_inplace(h, g)
 * ops.hpp:431-441 (feedforward.hpp:60-62). */
void orc_silu_mul(float* h, float* g, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) g[i] = g[i] / (1.f + expf(-g[i]));
    for (int64_t i = 0; i < n; ++i) h[i] *= g[i];
}

/* sampler::argmax: reference transformer.hpp:43-47 (first maximum). */
int orc_argmax(const float* p, int n)
{
    int best = 0;
    for (int i = 1; i < n; ++i)
        if (p[best] < p[i]) best = i;
    return best;
}

/* ------------------------------------------------------------------------ */
/* Linear y = x.W^T: reference compute.hpp:64-68 -> ops::gemm ops.hpp:170-310 */
/* ------------------------------------------------------------------------ */

/* M=1 streaming GEMV over a slice of rows: reference stream_gemv_kernel.inc:37-175
 * (AVX2+FMA instantiation, stream_gemv.hpp:52-58).  Groups of 4 rows with two
 * 8-lane FMA chains each over K&~15, one optional 8-wide step, the
 * hadd/hadd/hadd + low/high-half reduction, an FMA scalar tail; leftover rows
 * use four 8-lane chains over K&~31.  y is zero on entry (beta = 0), alpha = 1. */
ORC_AVX2 static void orc_gemv_slice(const float* x, const float* W, float* y,
                                    int K, int N, size_t ldw)
{
    const int K16 = K & ~15;
    int n = 0;
    for (; n + 4 <= N; n += 4) {
        const float* w[4];
        for (int r = 0; r < 4; ++r) w[r] = W + (size_t)(n + r) * ldw;
        __m256 ca[4], cb[4];
        for (int r = 0; r < 4; ++r) { ca[r] = _mm256_setzero_ps(); cb[r] = _mm256_setzero_ps(); }
        int k = 0;
        for (; k < K16; k += 16) {
            __m256 x0 = _mm256_loadu_ps(x + k), x1 = _mm256_loadu_ps(x + k + 8);
            for (int r = 0; r < 4; ++r) {
                ca[r] = _mm256_fmadd_ps(x0, _mm256_loadu_ps(w[r] + k), ca[r]);
                cb[r] = _mm256_fmadd_ps(x1, _mm256_loadu_ps(w[r] + k + 8), cb[r]);
            }
        }
        __m256 s[4];
        for (int r = 0; r < 4; ++r) s[r] = _mm256_add_ps(ca[r], cb[r]);
        if (k + 8 <= K) {
            __m256 x0 = _mm256_loadu_ps(x + k);
            for (int r = 0; r < 4; ++r) s[r] = _mm256_fmadd_ps(x0, _mm256_loadu_ps(w[r] + k), s[r]);
            k += 8;
        }
        __m256 t0 = _mm256_hadd_ps(s[0], s[1]);
        __m256 t1 = _mm256_hadd_ps(s[2], s[3]);
        __m256 t2 = _mm256_hadd_ps(t0, t1);
        __m128 rr = _mm_add_ps(_mm256_castps256_ps128(t2), _mm256_extractf128_ps(t2, 1));
        float out[4];
        _mm_storeu_ps(out, rr);
        for (; k < K; ++k)
            for (int r = 0; r < 4; ++r) out[r] = fmaf(x[k], w[r][k], out[r]);
        for (int r = 0; r < 4; ++r) y[n + r] += out[r];
    }
    for (; n < N; ++n) {
        const float* w = W + (size_t)n * ldw;
        __m256 c0 = _mm256_setzero_ps(), c1 = _mm256_setzero_ps();
        __m256 c2 = _mm256_setzero_ps(), c3 = _mm256_setzero_ps();
        int k = 0;
        const int K32 = K & ~31;
        for (; k < K32; k += 32) {
            c0 = _mm256_fmadd_ps(_mm256_loadu_ps(x + k), _mm256_loadu_ps(w + k), c0);
            c1 = _mm256_fmadd_ps(_mm256_loadu_ps(x + k + 8), _mm256_loadu_ps(w + k + 8), c1);
            c2 = _mm256_fmadd_ps(_mm256_loadu_ps(x + k + 16), _mm256_loadu_ps(w + k + 16), c2);
            c3 = _mm256_fmadd_ps(_mm256_loadu_ps(x + k + 24), _mm256_loadu_ps(w + k + 24), c3);
        }
        for (; k + 8 <= K; k += 8)
            c0 = _mm256_fmadd_ps(_mm256_loadu_ps(x + k), _mm256_loadu_ps(w + k), c0);
        __m256 sum8 = _mm256_add_ps(_mm256_add_ps(c0, c1), _mm256_add_ps(c2, c3));
        __m128 h = _mm_add_ps(_mm256_castps256_ps128(sum8), _mm256_extractf128_ps(sum8, 1));
        h = _mm_hadd_ps(h, h);
        h = _mm_hadd_ps(h, h);
        float sum = _mm_cvtss_f32(h);
        for (; k < K; ++k) sum = fmaf(x[k], w[k], sum);
        y[n] = fmaf(1.f, sum, y[n]);
    }
}

/* M>=4: reference ops.hpp:254-305 with the packed 1x8 micro-kernel
 * simd_gemm.hpp:159-178.  Packing only reorders B, so each output column is an
 * FMA chain over k in order; a partial last panel uses mul+add (ops.hpp:291-297). */
ORC_AVX2 static void orc_gemm_row_packed(const float* a, const float* W, float* c,
                                         int K, int N)
{
    const int NR = 8;
    int full = N / NR * NR;
    for (int j = 0; j < full; ++j) {
        const float* wr = W + (size_t)j * K;
        float acc = 0.f;
        for (int k = 0; k < K; ++k) acc = fmaf(a[k], wr[k], acc);
        c[j] = 0.f + acc * 1.f;
    }
    for (int j = full; j < N; ++j) {
        const float* wr = W + (size_t)j * K;
        float acc = 0.f;
        for (int k = 0; k < K; ++k) acc += a[k] * wr[k];
        c[j] = 0.f + 1.f * acc;
    }
}

/* Scalar tiled fallback: reference ops.hpp:142-168 (M in {2,3}, or K<8, N<8). */
static void orc_gemm_row_scalar(const float* a, const float* W, float* c, int K, int N)
{
    for (int j = 0; j < N; ++j) {
        const float* wr = W + (size_t)j * K;
        float acc = 0.f;
        for (int k = 0; k < K; ++k) acc += a[k] * wr[k];
        c[j] = 0.f + 1.f * acc;
    }
}

void orc_linear(const float* x, const float* W, float* y, int M, int K, int N, int n_threads)
{
    if (n_threads < 1) n_threads = 1;
    if (M == 1 && K >= 8 && N >= 8) {
        memset(y, 0, sizeof(float) * (size_t)N);
        if (N >= 256) {
            /* parallel_for(N): ThreadPool::run splits [0,N) into
             * min(threads,N) contiguous chunks of ceil(N/jobs) (thread_pool.hpp:80-91). */
            int jobs = n_threads < N ? n_threads : N;
            int chunk = (N + jobs - 1) / jobs;
#pragma omp parallel for num_threads(jobs) schedule(static, 1)
            for (int j = 0; j < jobs; ++j) {
                int lo = j * chunk, hi = lo + chunk < N ? lo + chunk : N;
                if (lo < hi) orc_gemv_slice(x, W + (size_t)lo * K, y + lo, K, hi - lo, (size_t)K);
            }
        } else {
            orc_gemv_slice(x, W, y, K, N, (size_t)K);
        }
        return;
    }
    if (M >= 4 && K >= 8 && N >= 8) {
#pragma omp parallel for num_threads(n_threads) schedule(static)
        for (int i = 0; i < M; ++i)
            orc_gemm_row_packed(x + (size_t)i * K, W, y + (size_t)i * N, K, N);
        return;
    }
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int i = 0; i < M; ++i)
        orc_gemm_row_scalar(x + (size_t)i * K, W, y + (size_t)i * N, K, N);
}

/* ------------------------------------------------------------------------ */
/* The engine's remaining per-op backend calls (ops.hpp), sequential order.   */
/* ------------------------------------------------------------------------ */
/* ops::layer_norm ops.hpp:443-476, per row. */
void orc_layer_norm(const float* x, const float* w, const float* b, float* out, int rows, int D, float eps)
{
    for (int r = 0; r < rows; ++r) {
        const float* row = x + (size_t)r * D;
        float* dst = out + (size_t)r * D;
        float mean = 0.f;
        for (int j = 0; j < D; ++j) mean += row[j];
        mean /= D;
        float var = 0.f;
        for (int j = 0; j < D; ++j) {
            float diff = row[j] - mean;
            var += diff * diff;
        }
        var = var / D + eps;
        float inv_std = 1.f / sqrtf(var);
        for (int j = 0; j < D; ++j) dst[j] = (row[j] - mean) * inv_std * w[j] + b[j];
    }
}

/* ops::softmax_inplace ops.hpp:501-520 (the serial branch, D < 4096). */
void orc_softmax(float* x, int rows, int D)
{
    for (int r = 0; r < rows; ++r) {
        float* row = x + (size_t)r * D;
        float mx = row[0];
        for (int j = 1; j < D; ++j)
            if (mx < row[j]) mx = row[j];        /* std::max_element: first maximum */
        float sum = 0.f;
        for (int j = 0; j < D; ++j) { row[j] = expf(row[j] - mx); sum += row[j]; }
        float inv = 1.f / (sum + 1e-9f);
        for (int j = 0; j < D; ++j) row[j] *= inv;
    }
}

/* ops::gelu_inplace ops.hpp:390-404. */
void orc_gelu(float* x, int64_t n)
{
    const float c1 = 0.7978845608028654f, c2 = 0.044715f;
    for (int64_t i = 0; i < n; ++i) {
        float v = x[i];
        float inner = c1 * (v + c2 * v * v * v);
        x[i] = 0.5f * v * (1.f + tanhf(inner));
    }
}

/* ops::gemm semantics ops.hpp:170-191: C = beta*C (0 when beta == 0) then
 * + alpha*op(A)*op(B); a plain f32 triple loop, k ascending. */
void orc_gemm(const float* A, const float* B, float* C, int M, int N, int K, int lda, int ldb, int ldc,
              float alpha, float beta, int transA, int transB)
{
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float acc = 0.f;
            for (int k = 0; k < K; ++k) {
                float a = transA ? A[(size_t)k * lda + m] : A[(size_t)m * lda + k];
                float b = transB ? B[(size_t)n * ldb + k] : B[(size_t)k * ldb + n];
                acc += a * b;
            }
            float* c = C + (size_t)m * ldc + n;
            float prev = beta == 0.f ? 0.f : (beta == 1.f ? *c : *c * beta);
            *c = prev + alpha * acc;
        }
}

/* ------------------------------------------------------------------------ */
/* GGUF block decode: reference tools/converter/convert_gguf.py:233-263        */
/* ------------------------------------------------------------------------ */
float orc_f16_to_f32(uint16_t h)
{
    /* IEEE binary16 -> binary32, exact (weights.hpp:76-96 semantics). */
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, mant = h & 0x3FFu, bits;
    if (e == 0) {
        if (mant == 0) bits = sign;
        else {
            int ee = 1;
            while (!(mant & 0x400u)) { mant <<= 1; --ee; }
            mant &= 0x3FFu;
            bits = sign | ((uint32_t)(ee + 112) << 23) | (mant << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void orc_dequant_q8_0(const uint8_t* blocks, float* out, int64_t numel)
{
    int64_t nb = numel / 32;
    for (int64_t b = 0; b < nb; ++b) {
        const uint8_t* blk = blocks + b * 34;
        uint16_t d16;
        memcpy(&d16, blk, 2);
        float d = orc_f16_to_f32(d16);
        for (int i = 0; i < 32; ++i) out[b * 32 + i] = (float)(int8_t)blk[2 + i] * d;
    }
}

void orc_dequant_q4_0(const uint8_t* blocks, float* out, int64_t numel)
{
    int64_t nb = numel / 32;
    for (int64_t b = 0; b < nb; ++b) {
        const uint8_t* blk = blocks + b * 18;
        uint16_t d16;
        memcpy(&d16, blk, 2);
        float d = orc_f16_to_f32(d16);
        for (int j = 0; j < 16; ++j) {
            uint8_t byte = blk[2 + j];
            out[b * 32 + 2 * j] = (float)((int)(byte & 0x0F) - 8) * d;      /* low nibble -> even */
            out[b * 32 + 2 * j + 1] = (float)((int)(byte >> 4) - 8) * d;    /* high nibble -> odd */
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Whole model: TransformerModel::forward transformer.hpp:335-424,            */
/* TransformerBlock::forward_v2 (pre-norm) transformer_block.hpp:141-159,     */
/* AttentionBlock::forward attention.hpp:89-186, FeedForward::forward        */
/* feedforward.hpp:50-77, KVCache F32 / F16 / Q8_0 kv_cache.hpp:152-286.     */
/* ------------------------------------------------------------------------ */
struct orc_layer {
    const float *ln1, *ln2, *wq, *wk, *wv, *wo, *wg, *w1, *w2;
    int8_t *kq, *vq;          /* Q8_0 codes [max_seq][row] */
    float *ks, *vs;           /* Q8_0 row scales [max_seq] */
    uint16_t *kh, *vh;        /* F16 [max_seq][row] */
    float *kf, *vf;           /* F32 [max_seq][row] */
};

struct orc_model {
    orc_config c;
    const float *embed, *ln_final, *lm_head;
    struct orc_layer* L;
    int used;
    float *cos_t, *sin_t;
};

orc_model* orc_model_create(const orc_config* cfg)
{
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    m->c = *cfg;
    if (m->c.n_threads < 1) m->c.n_threads = 1;
    int d_head = cfg->d_model / cfg->n_heads;
    int row = cfg->n_kv_heads * d_head;
    m->L = (struct orc_layer*)calloc((size_t)cfg->n_layers, sizeof(struct orc_layer));
    size_t n = (size_t)cfg->max_seq_len * row;
    for (int l = 0; l < cfg->n_layers; ++l) {      /* KVCache::KVCache kv_cache.hpp:152-177 */
        struct orc_layer* L = &m->L[l];
        if (cfg->kv_dtype == ORC_KV_F32) {
            L->kf = (float*)calloc(n, sizeof(float));
            L->vf = (float*)calloc(n, sizeof(float));
        } else if (cfg->kv_dtype == ORC_KV_F16) {
            L->kh = (uint16_t*)calloc(n, sizeof(uint16_t));
            L->vh = (uint16_t*)calloc(n, sizeof(uint16_t));
        } else {
            L->kq = (int8_t*)calloc(n, 1);
            L->vq = (int8_t*)calloc(n, 1);
            L->ks = (float*)calloc((size_t)cfg->max_seq_len, sizeof(float));
            L->vs = (float*)calloc((size_t)cfg->max_seq_len, sizeof(float));
        }
    }
    size_t nt = (size_t)cfg->max_seq_len * (d_head / 2);
    m->cos_t = (float*)malloc(nt * sizeof(float));
    m->sin_t = (float*)malloc(nt * sizeof(float));
    orc_rope_tables(cfg->max_seq_len, d_head, cfg->rope_theta, m->cos_t, m->sin_t);
    return m;
}

void orc_model_destroy(orc_model* m)
{
    if (!m) return;
    for (int l = 0; l < m->c.n_layers; ++l) {
        struct orc_layer* L = &m->L[l];
        free(L->kq); free(L->vq); free(L->ks); free(L->vs);
        free(L->kh); free(L->vh); free(L->kf); free(L->vf);
    }
    free(m->L); free(m->cos_t); free(m->sin_t); free(m);
}

void orc_model_set_globals(orc_model* m, const float* embed, const float* ln_final,
                           const float* lm_head)
{
    m->embed = embed; m->ln_final = ln_final; m->lm_head = lm_head;
}

void orc_model_set_layer(orc_model* m, int l, const float* ln1, const float* ln2,
                         const float* wq, const float* wk, const float* wv, const float* wo,
                         const float* wg, const float* w1, const float* w2)
{
    struct orc_layer* L = &m->L[l];
    L->ln1 = ln1; L->ln2 = ln2; L->wq = wq; L->wk = wk; L->wv = wv; L->wo = wo;
    L->wg = wg; L->w1 = w1; L->w2 = w2;
}

/* KVCache::reset kv_cache.hpp:179-196 (all layers). */
void orc_model_reset(orc_model* m)
{
    int d_head = m->c.d_model / m->c.n_heads;
    size_t row = (size_t)m->c.n_kv_heads * d_head;
    size_t n = (size_t)m->c.max_seq_len * row;
    for (int l = 0; l < m->c.n_layers; ++l) {
        struct orc_layer* L = &m->L[l];
        if (L->kq) { memset(L->kq, 0, n); memset(L->vq, 0, n); }
        if (L->ks) { memset(L->ks, 0, (size_t)m->c.max_seq_len * sizeof(float));
                     memset(L->vs, 0, (size_t)m->c.max_seq_len * sizeof(float)); }
        if (L->kh) { memset(L->kh, 0, n * sizeof(uint16_t)); memset(L->vh, 0, n * sizeof(uint16_t)); }
        if (L->kf) { memset(L->kf, 0, n * sizeof(float)); memset(L->vf, 0, n * sizeof(float)); }
    }
    m->used = 0;
}

int orc_model_used(const orc_model* m) { return m->used; }

void orc_model_kv(orc_model* m, int l, int8_t** kq, int8_t** vq, float** ks, float** vs)
{
    *kq = m->L[l].kq; *vq = m->L[l].vq; *ks = m->L[l].ks; *vs = m->L[l].vs;
}

void orc_model_kv_raw(orc_model* m, int l, void** k, void** v)
{
    struct orc_layer* L = &m->L[l];
    if (L->kf) { *k = L->kf; *v = L->vf; }
    else if (L->kh) { *k = L->kh; *v = L->vh; }
    else { *k = L->kq; *v = L->vq; }
}

void orc_model_fill_kv(orc_model* m, int used, uint64_t seed)
{
    int d_head = m->c.d_model / m->c.n_heads;
    size_t row = (size_t)m->c.n_kv_heads * d_head;
    if (used > m->c.max_seq_len) used = m->c.max_seq_len;
    if (m->c.kv_dtype != ORC_KV_Q8_0) {      /* only the Q8_0 baseline fills codes */
        m->used = 0;
        return;
    }
    uint64_t z = seed * 0x9E3779B97F4A7C15ull + 1;
    for (int l = 0; l < m->c.n_layers; ++l)
        for (int r = 0; r < used; ++r) {
            for (size_t i = 0; i < row; ++i) {
                z ^= z << 13; z ^= z >> 7; z ^= z << 17;
                m->L[l].kq[(size_t)r * row + i] = (int8_t)((int)(z & 0xFF) % 255 - 127);
                m->L[l].vq[(size_t)r * row + i] = (int8_t)((int)((z >> 8) & 0xFF) % 255 - 127);
            }
            m->L[l].ks[r] = 0.02f;
            m->L[l].vs[r] = 0.02f;
        }
    m->used = used;
}

/* The layers over T embedded rows x [T][D] (in place), appending T cache rows:
 * the body of TransformerModel::forward between the embedding and the final
 * norm (transformer.hpp:335-398). */
int orc_model_forward_hidden(orc_model* m, float* x, int T)
{
    const orc_config* c = &m->c;
    const int D = c->d_model, F = c->d_ff, H = c->n_heads, G = c->n_kv_heads;
    const int dh = D / H, dkv = G * dh, rep = H / G, nt = c->n_threads;
    if (T <= 0 || m->used + T > c->max_seq_len) return -1;

    size_t TD = (size_t)T * D;
    float* hn = (float*)malloc(TD * sizeof(float));
    float* q = (float*)malloc(TD * sizeof(float));
    float* k = (float*)malloc((size_t)T * dkv * sizeof(float));
    float* v = (float*)malloc((size_t)T * dkv * sizeof(float));
    float* att = (float*)malloc(TD * sizeof(float));
    float* a = (float*)malloc(TD * sizeof(float));
    float* u = (float*)malloc((size_t)T * F * sizeof(float));
    float* g = (float*)malloc((size_t)T * F * sizeof(float));
    float* kd = (float*)malloc((size_t)c->max_seq_len * dkv * sizeof(float));
    float* vd = (float*)malloc((size_t)c->max_seq_len * dkv * sizeof(float));
    const float scale = 1.f / sqrtf((float)dh);        /* attention.hpp:373-374 */
    const int pos_offset = m->used;                      /* attention.hpp:110 */
    const int causal = (T == 1) ? 0 : 1;                 /* attention.hpp:166-174 */
    const int ctx = m->used + T;

    for (int l = 0; l < c->n_layers; ++l) {
        struct orc_layer* L = &m->L[l];
        orc_rms_norm(x, L->ln1, hn, T, D, c->norm_eps);
        orc_linear(hn, L->wq, q, T, D, D, nt);
        orc_linear(hn, L->wk, k, T, D, dkv, nt);
        orc_linear(hn, L->wv, v, T, D, dkv, nt);
        orc_rope_apply(q, T, H, dh, pos_offset, m->cos_t, m->sin_t, c->max_seq_len);
        orc_rope_apply(k, T, G, dh, pos_offset, m->cos_t, m->sin_t, c->max_seq_len);
        size_t r0 = (size_t)m->used * dkv, nr = (size_t)T * dkv, nc = (size_t)ctx * dkv;
        if (c->kv_dtype == ORC_KV_F32) {                 /* KVCache::append / raw f32 view */
            memcpy(L->kf + r0, k, nr * sizeof(float));
            memcpy(L->vf + r0, v, nr * sizeof(float));
            memcpy(kd, L->kf, nc * sizeof(float));
            memcpy(vd, L->vf, nc * sizeof(float));
        } else if (c->kv_dtype == ORC_KV_F16) {          /* append f32_to_f16, dequant_into f16_to_f32 */
            for (size_t i = 0; i < nr; ++i) {
                L->kh[r0 + i] = orc_f32_to_f16_kv(k[i]);
                L->vh[r0 + i] = orc_f32_to_f16_kv(v[i]);
            }
            for (size_t i = 0; i < nc; ++i) {
                kd[i] = orc_f16_to_f32(L->kh[i]);
                vd[i] = orc_f16_to_f32(L->vh[i]);
            }
        } else {
            for (int t = 0; t < T; ++t) {                /* KVCache::append */
                int r = m->used + t;
                L->ks[r] = orc_quantize_row_q8_0(k + (size_t)t * dkv, L->kq + (size_t)r * dkv, dkv);
                L->vs[r] = orc_quantize_row_q8_0(v + (size_t)t * dkv, L->vq + (size_t)r * dkv, dkv);
            }
            for (int r = 0; r < ctx; ++r) {              /* KVCache::dequant_into */
                orc_dequantize_row_q8_0(L->kq + (size_t)r * dkv, L->ks[r], kd + (size_t)r * dkv, dkv);
                orc_dequantize_row_q8_0(L->vq + (size_t)r * dkv, L->vs[r], vd + (size_t)r * dkv, dkv);
            }
        }
#pragma omp parallel for num_threads(nt) schedule(static)
        for (int h = 0; h < H; ++h) {                    /* sdp_heads, head h -> kv head h/rep */
            int gk = h / rep;
            orc_flash_attn_head(q + (size_t)h * dh, D, kd + (size_t)gk * dh, vd + (size_t)gk * dh, dkv,
                                att + (size_t)h * dh, D, T, ctx, dh, scale, causal);
        }
        orc_linear(att, L->wo, a, T, D, D, nt);
        for (size_t i = 0; i < TD; ++i) a[i] += x[i];   /* add_inplace(a, x) */
        orc_rms_norm(a, L->ln2, hn, T, D, c->norm_eps);
        orc_linear(hn, L->w1, u, T, D, F, nt);
        orc_linear(hn, L->wg, g, T, D, F, nt);
        orc_silu_mul(u, g, (int64_t)T * F);
        orc_linear(u, L->w2, x, T, F, D, nt);
        for (size_t i = 0; i < TD; ++i) x[i] += a[i];   /* add_inplace(f, a) */
    }
    m->used += T;
    free(hn); free(q); free(k); free(v); free(att); free(a);
    free(u); free(g); free(kd); free(vd);
    return 0;
}

int orc_model_forward(orc_model* m, const int* ids, int T, float* logits)
{
    const orc_config* c = &m->c;
    const int D = c->d_model, nt = c->n_threads;
    if (T <= 0 || m->used + T > c->max_seq_len) return -1;
    for (int t = 0; t < T; ++t)
        if (ids[t] < 0 || ids[t] >= c->vocab_size) return -1;

    float* x = (float*)malloc((size_t)T * D * sizeof(float));
    float* hn = (float*)malloc((size_t)D * sizeof(float));
    for (int t = 0; t < T; ++t)                          /* ops.hpp:615-626 */
        memcpy(x + (size_t)t * D, m->embed + (size_t)ids[t] * D, sizeof(float) * D);
    orc_model_forward_hidden(m, x, T);

    orc_rms_norm(x + (size_t)(T - 1) * D, m->ln_final, hn, 1, D, c->norm_eps);
    float* lg = logits ? logits : (float*)malloc(sizeof(float) * (size_t)c->vocab_size);
    orc_linear(hn, m->lm_head, lg, 1, D, c->vocab_size, nt);
    int best = orc_argmax(lg, c->vocab_size);
    if (!logits) free(lg);
    free(x); free(hn);
    return best;
}
