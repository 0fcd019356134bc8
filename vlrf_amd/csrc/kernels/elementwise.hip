// elementwise.hip - edge ops of the decode step: RMSNorm, RoPE, the KV append
// (Q8_0 quantize, F16 convert, F32 copy) and dequant, embedding gather and
// greedy argmax.
#include "../internal.hpp"

#include <cstdlib>

#include <cmath>

namespace vlrf_hip {
namespace {

// Block-wide reductions for 256-thread blocks.
__device__ __forceinline__ float block_max256(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_max(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return v;
}

__device__ __forceinline__ float block_sum256(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    v = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return v;
}

// One RoPE pair, rope.hpp:90-96.  Contraction off: the reference's scalar
// build rounds each product separately, so this matches it bit for bit given
// the same cos/sin tables.
__device__ __forceinline__ void rope_pair(float* v, int i, int half, float c, float s) {
#pragma clang fp contract(off)
    const float x0 = v[i], x1 = v[i + half];
    const float a = x0 * c;
    const float b = x1 * s;
    const float e = x1 * c;
    const float f = x0 * s;
    v[i] = a - b;
    v[i + half] = e + f;
}

// rope_pair on values in registers: (x0, x1) -> (x0 c - x1 s, x1 c + x0 s).
__device__ __forceinline__ void rope2v(float x0, float x1, float c, float s, float* y0, float* y1) {
#pragma clang fp contract(off)
    const float a = x0 * c;
    const float b = x1 * s;
    const float e = x1 * c;
    const float f = x0 * s;
    *y0 = a - b;
    *y1 = e + f;
}

// quantize_row_q8_0 (kv_cache.hpp:102-117) of one row of n_kv*D floats into
// the head-major cache at token position p.  Bit-exact: max is
// order-independent, amax/127 and 1/scale are correctly rounded (HIP default,
// also forced by the build), roundf rounds half away from zero as lround.
__device__ void quantize_row_to_cache(const float* __restrict__ src, int8_t* __restrict__ dst,
                                      float* __restrict__ sc, int p, int n_kv, int D,
                                      int max_seq, float* red) {
    const int row = n_kv * D;
    float amax = 0.f;
    for (int i = threadIdx.x; i < row; i += 256) amax = fmaxf(amax, fabsf(src[i]));
    amax = block_max256(amax, red);
    float inv = 0.f;
    if (amax != 0.f) {
        const float scale = amax / 127.f;
        inv = 1.f / scale;
        if (threadIdx.x == 0) sc[p] = scale;
    } else if (threadIdx.x == 0) {
        sc[p] = 0.f;
    }
    for (int i = threadIdx.x; i < row; i += 256) {
        int q = 0;
        if (amax != 0.f) {
            q = (int)roundf(src[i] * inv);
            q = min(127, max(-127, q));
        }
        const int h = i / D, d = i - h * D;
        dst[((size_t)h * max_seq + p) * D + d] = (int8_t)q;
    }
}

// KVCache::append of one row (kv_cache.hpp:215-251) for any cache dtype:
// Q8_0 quantize_row_q8_0, F16 the reference's f32_to_f16 per element, F32 copy.
__device__ void store_row_to_cache(const float* __restrict__ src, int8_t* dst, float* sc, int dtype,
                                   int p, int n_kv, int D, int max_seq, float* red) {
    if (dtype == VLRF_HIP_KV_Q8_0) {
        quantize_row_to_cache(src, dst, sc, p, n_kv, D, max_seq, red);
        return;
    }
    for (int i = threadIdx.x; i < n_kv * D; i += 256) {
        const int h = i / D, d = i - h * D;
        const size_t o = ((size_t)h * max_seq + p) * D + d;
        if (dtype == VLRF_HIP_KV_F16) reinterpret_cast<uint16_t*>(dst)[o] = f32_to_f16_kv(src[i]);
        else reinterpret_cast<float*>(dst)[o] = src[i];
    }
}

__global__ __launch_bounds__(256) void kv_append_kernel(int8_t* kq, int8_t* vq, float* ks, float* vs, int dtype,
                                                        const float* __restrict__ k,
                                                        const float* __restrict__ v, int n_kv, int D,
                                                        int max_seq, int pos, const int* pos_dev) {
    __shared__ float red[4];
    const int t = blockIdx.x;
    const int p = (pos_dev ? *pos_dev : pos) + t;
    if (p < 0 || p >= max_seq) return;   // host checks capacity; never write past the cache
    const size_t row = (size_t)n_kv * D;
    store_row_to_cache(k + t * row, kq, ks, dtype, p, n_kv, D, max_seq, red);
    store_row_to_cache(v + t * row, vq, vs, dtype, p, n_kv, D, max_seq, red);
}

// Decode fusion: rotate q (n_heads) in place and k (n_kv) at position *pos_dev,
// then append k and v to the cache (attention.hpp:109-128 order).
__global__ __launch_bounds__(256) void rope_append_kernel(int8_t* kq, int8_t* vq, float* ks,
                                                          float* vs, int dtype, float* q, const float* __restrict__ k,
                                                          const float* __restrict__ v, int n_heads,
                                                          int n_kv, int D, int max_seq,
                                                          const int* __restrict__ pos_dev,
                                                          const float* __restrict__ cos_t,
                                                          const float* __restrict__ sin_t) {
    __shared__ float red[4];
    __shared__ float kr[1024];
    const int p = *pos_dev;
    if (p < 0 || p >= max_seq) return;   // host checks capacity; never write past the cache
    const int half = D / 2;
    const int row = n_kv * D;
    const float* c = cos_t + (size_t)p * half;
    const float* s = sin_t + (size_t)p * half;
    for (int i = threadIdx.x; i < row; i += 256) kr[i] = k[i];
    __syncthreads();
    if (half % 4 == 0) {
        // four pairs per thread: float4 loads and stores of x0 and x1, the same
        // separately rounded products per element as rope_pair
        for (int i4 = threadIdx.x; i4 < n_heads * half / 4; i4 += 256) {
            const int h = 4 * i4 / half, j = 4 * i4 - h * half;
            float4* x0p = reinterpret_cast<float4*>(q + (size_t)h * D + j);
            float4* x1p = reinterpret_cast<float4*>(q + (size_t)h * D + half + j);
            const float4 x0 = *x0p, x1 = *x1p;
            const float4 c4 = *reinterpret_cast<const float4*>(c + j), s4 = *reinterpret_cast<const float4*>(s + j);
            float4 y0, y1;
            rope2v(x0.x, x1.x, c4.x, s4.x, &y0.x, &y1.x);
            rope2v(x0.y, x1.y, c4.y, s4.y, &y0.y, &y1.y);
            rope2v(x0.z, x1.z, c4.z, s4.z, &y0.z, &y1.z);
            rope2v(x0.w, x1.w, c4.w, s4.w, &y0.w, &y1.w);
            *x0p = y0;
            *x1p = y1;
        }
    } else {
        for (int i = threadIdx.x; i < n_heads * half; i += 256) {
            const int h = i / half, j = i - h * half;
            rope_pair(q + (size_t)h * D, j, half, c[j], s[j]);
        }
    }
    for (int i = threadIdx.x; i < n_kv * half; i += 256) {
        const int h = i / half, j = i - h * half;
        rope_pair(kr + h * D, j, half, c[j], s[j]);
    }
    __syncthreads();
    store_row_to_cache(kr, kq, ks, dtype, p, n_kv, D, max_seq, red);
    store_row_to_cache(v, vq, vs, dtype, p, n_kv, D, max_seq, red);
}

// Prefill: token t of a [T][ld] QKV buffer (q: n_heads*D at column 0, k and v:
// n_kv*D each after it) at position pos0 + t: k rotated, then the K and V rows
// appended to the cache (attention.hpp:109-128 order; q is rotated by the
// prefill attention as it loads it).  One workgroup a token, for the rows
// prefill_kv_rows_kernel's lane layout does not fit.
__global__ __launch_bounds__(256) void prefill_rope_append_kernel(
    int8_t* kq, int8_t* vq, float* ks, float* vs, int dtype, const float* qkv, int ld, int n_heads, int n_kv,
    int D, int max_seq, int pos0, const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
    __shared__ float red[4];
    __shared__ float kr[1024];
    const int t = blockIdx.x, p = pos0 + t;
    if (p < 0 || p >= max_seq) return;   // host checks capacity; never write past the cache
    const int half = D / 2, row = n_kv * D;
    const float* k = qkv + (size_t)t * ld + (size_t)n_heads * D;
    const float* v = k + row;
    const float* c = cos_t + (size_t)p * half;
    const float* s = sin_t + (size_t)p * half;
    for (int i = threadIdx.x; i < row; i += 256) kr[i] = k[i];
    __syncthreads();
    for (int i = threadIdx.x; i < n_kv * half; i += 256) {
        const int h = i / half, j = i - h * half;
        rope_pair(kr + h * D, j, half, c[j], s[j]);
    }
    __syncthreads();
    store_row_to_cache(kr, kq, ks, dtype, p, n_kv, D, max_seq, red);
    store_row_to_cache(v, vq, vs, dtype, p, n_kv, D, max_seq, red);
}

// N consecutive floats (16-byte aligned when VEC).
template <int N, bool VEC>
__device__ __forceinline__ void load_run(const float* __restrict__ p, float (&o)[N]) {
    if constexpr (VEC) {
        static_assert(N % 4 == 0, "whole float4s");
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            const float4 a = reinterpret_cast<const float4*>(p)[i];
            o[4 * i] = a.x; o[4 * i + 1] = a.y; o[4 * i + 2] = a.z; o[4 * i + 3] = a.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) o[i] = p[i];
    }
}

// N consecutive elements of type E stored from e (as whole 4-, 8- or 16-byte
// words when VEC: the run starts at a multiple of its own size, at most 16).
template <int N, bool VEC, typename E>
__device__ __forceinline__ void store_run(E* __restrict__ p, const E (&e)[N]) {
    constexpr int B = N * (int)sizeof(E);
    if constexpr (VEC && B % 4 == 0) {
        uint32_t w[B / 4];
        __builtin_memcpy(w, e, B);
        if constexpr (B % 16 == 0) {
#pragma unroll
            for (int i = 0; i < B / 16; ++i)
                reinterpret_cast<uint4*>(p)[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
        } else if constexpr (B % 8 == 0) {
#pragma unroll
            for (int i = 0; i < B / 8; ++i) reinterpret_cast<uint2*>(p)[i] = make_uint2(w[2 * i], w[2 * i + 1]);
        } else {
#pragma unroll
            for (int i = 0; i < B / 4; ++i) reinterpret_cast<uint32_t*>(p)[i] = w[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) p[i] = e[i];
    }
}

// The prefill's K/V rows with q left to its consumer: one wave per token (four
// a workgroup), no LDS and no barrier.  Lane l holds PPL consecutive RoPE pairs
// of one head (elements j and j + D/2, j = j0 .. j0 + PPL - 1) of the K row
// and 2 PPL consecutive elements of the V row, read straight from the QKV
// buffer; RoPE as rope_pair, then per row the cache dtype's store as
// store_row_to_cache (Q8_0: the row's amax by a wave max, the same scale,
// reciprocal and rounding), as contiguous runs of PPL (K) and 2 PPL (V)
// elements.  n_kv * D / 2 == 64 * PPL and (D / 2) % PPL == 0.  VEC (PPL a
// multiple of 4, every row and table 16-byte aligned, D % 16 == 0): the runs
// are read as float4 and written as whole words; the same values either way.
template <int PPL, bool VEC>
__global__ __launch_bounds__(256) void prefill_kv_rows_kernel(
    int8_t* kq, int8_t* vq, float* ks, float* vs, int dtype, const float* __restrict__ qkv, int ld, int n_heads,
    int D, int max_seq, int pos0, int T, const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
    const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int p = pos0 + t;
    if (t >= T || p < 0 || p >= max_seq) return;   // host checks capacity; never write past the cache
    const int half = D / 2, pr = lane * PPL, h = pr / half, j0 = pr - h * half;
    const float* k = qkv + (size_t)t * ld + (size_t)n_heads * D;
    const float* v = k + (size_t)(64 * PPL * 2);          // the V row follows the K row (n_kv * D = 128 PPL)
    float x0[PPL], x1[PPL], cr[PPL], sr[PPL], y0[PPL], y1[PPL], vv[2 * PPL];
    load_run<PPL, VEC>(k + h * D + j0, x0);
    load_run<PPL, VEC>(k + h * D + half + j0, x1);
    load_run<PPL, VEC>(cos_t + (size_t)p * half + j0, cr);
    load_run<PPL, VEC>(sin_t + (size_t)p * half + j0, sr);
    load_run<2 * PPL, VEC>(v + 2 * PPL * lane, vv);
#pragma unroll
    for (int i = 0; i < PPL; ++i) rope2v(x0[i], x1[i], cr[i], sr[i], &y0[i], &y1[i]);
    const int vh = (2 * PPL * lane) / D, vd = 2 * PPL * lane - vh * D;
    if (dtype == VLRF_HIP_KV_Q8_0) {
        auto quant = [](float x, float amax, float inv) -> int8_t {
            int q = 0;
            if (amax != 0.f) {
                q = (int)roundf(x * inv);
                q = min(127, max(-127, q));
            }
            return (int8_t)q;
        };
        float ak = 0.f, av = 0.f;
#pragma unroll
        for (int i = 0; i < PPL; ++i) ak = fmaxf(ak, fmaxf(fabsf(y0[i]), fabsf(y1[i])));
#pragma unroll
        for (int i = 0; i < 2 * PPL; ++i) av = fmaxf(av, fabsf(vv[i]));
        ak = wave_max(ak);
        av = wave_max(av);
        const float sk = ak != 0.f ? ak / 127.f : 0.f, sv = av != 0.f ? av / 127.f : 0.f;
        const float ik = ak != 0.f ? 1.f / sk : 0.f, iv = av != 0.f ? 1.f / sv : 0.f;
        int8_t* kr = kq + ((size_t)h * max_seq + p) * D;
        int8_t* vr = vq + ((size_t)vh * max_seq + p) * D;
        int8_t c0[PPL], c1[PPL], cv[2 * PPL];
#pragma unroll
        for (int i = 0; i < PPL; ++i) {
            c0[i] = quant(y0[i], ak, ik);
            c1[i] = quant(y1[i], ak, ik);
        }
#pragma unroll
        for (int i = 0; i < 2 * PPL; ++i) cv[i] = quant(vv[i], av, iv);
        store_run<PPL, VEC>(kr + j0, c0);
        store_run<PPL, VEC>(kr + half + j0, c1);
        store_run<2 * PPL, VEC>(vr + vd, cv);
        if (lane == 0) { ks[p] = sk; vs[p] = sv; }
    } else if (dtype == VLRF_HIP_KV_F16) {
        uint16_t* kr = reinterpret_cast<uint16_t*>(kq) + ((size_t)h * max_seq + p) * D;
        uint16_t* vr = reinterpret_cast<uint16_t*>(vq) + ((size_t)vh * max_seq + p) * D;
        uint16_t c0[PPL], c1[PPL], cv[2 * PPL];
#pragma unroll
        for (int i = 0; i < PPL; ++i) {
            c0[i] = f32_to_f16_kv(y0[i]);
            c1[i] = f32_to_f16_kv(y1[i]);
        }
#pragma unroll
        for (int i = 0; i < 2 * PPL; ++i) cv[i] = f32_to_f16_kv(vv[i]);
        store_run<PPL, VEC>(kr + j0, c0);
        store_run<PPL, VEC>(kr + half + j0, c1);
        store_run<2 * PPL, VEC>(vr + vd, cv);
    } else {
        float* kr = reinterpret_cast<float*>(kq) + ((size_t)h * max_seq + p) * D;
        float* vr = reinterpret_cast<float*>(vq) + ((size_t)vh * max_seq + p) * D;
        store_run<PPL, VEC>(kr + j0, y0);
        store_run<PPL, VEC>(kr + half + j0, y1);
        store_run<2 * PPL, VEC>(vr + vd, vv);
    }
}

// x[t] = table[ids[t]] (ops.hpp:615-626), one workgroup per token.
__global__ __launch_bounds__(256) void embed_rows_kernel(const float* __restrict__ table,
                                                         const int* __restrict__ ids, float* __restrict__ x,
                                                         int D) {
    const int t = blockIdx.x;
    const float4* src = reinterpret_cast<const float4*>(table + (size_t)ids[t] * D);
    float4* dst = reinterpret_cast<float4*>(x + (size_t)t * D);
    for (int i = threadIdx.x; i < D / 4; i += 256) dst[i] = src[i];
}

// KVCache::dequant_into (kv_cache.hpp:259-286) for any cache dtype.
__global__ __launch_bounds__(256) void kv_dequant_kernel(const int8_t* __restrict__ kq,
                                                         const int8_t* __restrict__ vq,
                                                         const float* __restrict__ ks,
                                                         const float* __restrict__ vs, int dtype, int n_kv,
                                                         int D, int max_seq, float* K_out, float* V_out) {
    const int t = blockIdx.x;
    const int row = n_kv * D;
    for (int i = threadIdx.x; i < row; i += 256) {
        const int h = i / D, d = i - h * D;
        const size_t src = ((size_t)h * max_seq + t) * D + d;
        float kv, vv;
        if (dtype == VLRF_HIP_KV_Q8_0) {
            kv = (float)kq[src] * ks[t];
            vv = (float)vq[src] * vs[t];
        } else if (dtype == VLRF_HIP_KV_F16) {
            kv = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(kq)[src]);
            vv = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(vq)[src]);
        } else {
            kv = reinterpret_cast<const float*>(kq)[src];
            vv = reinterpret_cast<const float*>(vq)[src];
        }
        K_out[(size_t)t * row + i] = kv;
        V_out[(size_t)t * row + i] = vv;
    }
}

// ops::rms_norm (ops.hpp:478-499) per row: y = x * (1/sqrt(sum(x^2)/D + eps)) * w.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ w, float* out, int D,
                                                      float eps) {
    __shared__ float red[4];
    const float* xr = x + (size_t)blockIdx.x * D;
    float ss = 0.f;
    for (int i = threadIdx.x; i < D; i += 256) ss += xr[i] * xr[i];
    ss = block_sum256(ss, red);
    const float inv = 1.f / sqrtf(ss / (float)D + eps);
    float* o = out + (size_t)blockIdx.x * D;
    for (int i = threadIdx.x; i < D; i += 256) o[i] = xr[i] * inv * w[i];
}

__global__ __launch_bounds__(256) void rope_kernel(float* x, int n_heads, int D, int pos_offset,
                                                   int max_seq, const float* __restrict__ cos_t,
                                                   const float* __restrict__ sin_t) {
    const int t = blockIdx.x, pos = pos_offset + t;
    if (pos >= max_seq) return;
    const int half = D / 2;
    float* row = x + (size_t)t * n_heads * D;
    const float* c = cos_t + (size_t)pos * half;
    const float* s = sin_t + (size_t)pos * half;
    for (int i = threadIdx.x; i < n_heads * half; i += 256) {
        const int h = i / half, j = i - h * half;
        rope_pair(row + (size_t)h * D, j, half, c[j], s[j]);
    }
}

__global__ __launch_bounds__(256) void embed_kernel(const float* __restrict__ table,
                                                    const int* __restrict__ tok, float* x, int D) {
    const float* r = table + (size_t)(*tok) * D;
    for (int i = threadIdx.x; i < D; i += 256) x[i] = r[i];
}

// sampler::argmax (transformer.hpp:43-47): first index of the maximum.  Each
// thread issues all of its float4 loads before comparing (one memory round
// trip); ties keep the lower index at every level.
// The step's state after its token: state[0] = token, appended to
// gen_ids[state[2]++], state[1] (position) += 1, state[3] (the epoch of the
// next step's tagged words: every launch of this step has finished reading
// them) += 1.
__device__ __forceinline__ void step_state_advance(int tok, int* state, int* gen_ids, int gen_cap) {
    state[0] = tok;
    const int g = state[2];
    if (g < gen_cap) gen_ids[g] = tok;
    state[2] = g + 1;
    state[1] = state[1] + 1;
    state[3] = state[3] + 1;
}

constexpr int kArgmaxPer = 16;   // float4 per thread: n <= 1024*4*16 = 65536
__global__ __launch_bounds__(1024) void argmax_step_kernel(const float* __restrict__ logits, int n,
                                                           int* state, int* gen_ids, int gen_cap) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    const int tid = threadIdx.x;
    const int n4 = n / 4;
    float4 v[kArgmaxPer];
#pragma unroll
    for (int k = 0; k < kArgmaxPer; ++k) {
        const int f = tid + k * 1024;
        v[k] = f < n4 ? reinterpret_cast<const float4*>(logits)[f] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float best = -INFINITY;
    int idx = -1;
#pragma unroll
    for (int k = 0; k < kArgmaxPer; ++k) {
        const int f = tid + k * 1024;
        if (f < n4) {
            const float e[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (idx < 0 || best < e[j]) { best = e[j]; idx = 4 * f + j; }
        }
    }
    for (int i = 4 * n4 + tid; i < n; i += 1024) {   // tail when n % 4 != 0
        const float e = logits[i];
        if (idx < 0 || best < e || (best == e && i < idx)) { best = e; idx = i; }
    }
    // Wave butterfly, then wave 0 over the 16 wave results: one barrier.  The
    // rule (larger value; the lower index on equal values) gives the same
    // winner in any combining order.
    auto take = [&](float ov, int oi) {
        if (oi >= 0 && (idx < 0 || best < ov || (best == ov && oi < idx))) { best = ov; idx = oi; }
    };
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const int oi = __shfl_xor(idx, o);
        take(ov, oi);
    }
    if ((tid & 63) == 0) { bv[tid >> 6] = best; bi[tid >> 6] = idx; }
    __syncthreads();
    if (tid < 64) {
        best = tid < 16 ? bv[tid] : -INFINITY;
        idx = tid < 16 ? bi[tid] : -1;
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) {
            const float ov = __shfl_xor(best, o);
            const int oi = __shfl_xor(idx, o);
            take(ov, oi);
        }
    }
    if (tid == 0) step_state_advance(idx < 0 ? 0 : idx, state, gen_ids, gen_cap);
}

// The same step over the LM head's per-workgroup (max, first index) pairs
// (gemv_kernel's argmax form): one pair per thread, the rule of
// argmax_step_kernel (larger value; the lower index on equal values).
__global__ __launch_bounds__(512) void argmax_pairs_step_kernel(const float2* __restrict__ pairs, int np, int* state,
                                                                int* gen_ids, int gen_cap) {
    __shared__ float bv[8];
    __shared__ int bi[8];
    const int tid = threadIdx.x;
    float best = -INFINITY;
    int idx = -1;
    if (tid < np) {
        const float2 p = pairs[tid];
        best = p.x;
        idx = __float_as_int(p.y);
    }
    auto take = [&](float ov, int oi) {
        if (oi >= 0 && (idx < 0 || best < ov || (best == ov && oi < idx))) { best = ov; idx = oi; }
    };
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o);
        const int oi = __shfl_xor(idx, o);
        take(ov, oi);
    }
    if ((tid & 63) == 0) { bv[tid >> 6] = best; bi[tid >> 6] = idx; }
    __syncthreads();
    if (tid < 64) {
        best = tid < 8 ? bv[tid] : -INFINITY;
        idx = tid < 8 ? bi[tid] : -1;
#pragma unroll
        for (int o = 4; o > 0; o >>= 1) {
            const float ov = __shfl_xor(best, o);
            const int oi = __shfl_xor(idx, o);
            take(ov, oi);
        }
    }
    if (tid == 0) step_state_advance(idx < 0 ? 0 : idx, state, gen_ids, gen_cap);
}

}  // namespace

int launch_kv_append(hipStream_t s, const KVLayer& L, int n_kv, int d_head, int max_seq,
                     const float* k, const float* v, int T, int pos, const int* pos_dev) {
    VH_ARG(T >= 1 && n_kv >= 1 && d_head >= 1, "kv_append: empty shape");
    if (!pos_dev) VH_ARG(pos >= 0 && pos + T <= max_seq, "kv_append: rows [%d,%d) beyond max_seq %d",
                         pos, pos + T, max_seq);
    hipLaunchKernelGGL(kv_append_kernel, dim3(T), dim3(256), 0, s, L.k, L.v, L.ks, L.vs, L.dtype, k, v, n_kv,
                       d_head, max_seq, pos, pos_dev);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_rope_append(hipStream_t s, const KVLayer& L, float* q, const float* k, const float* v,
                       int n_heads, int n_kv, int d_head, int max_seq, const int* pos_dev,
                       const float* cos_t, const float* sin_t) {
    VH_ARG(n_kv * d_head <= 1024, "rope_append: kv row %d exceeds 1024", n_kv * d_head);
    VH_ARG(d_head % 2 == 0, "rope_append: odd d_head");
    hipLaunchKernelGGL(rope_append_kernel, dim3(1), dim3(256), 0, s, L.k, L.v, L.ks, L.vs, L.dtype, q, k, v,
                       n_heads, n_kv, d_head, max_seq, pos_dev, cos_t, sin_t);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_prefill_rope_append(hipStream_t s, const KVLayer& L, const float* qkv, int ld, int T, int n_heads,
                               int n_kv, int d_head, int max_seq, int pos0, const float* cos_t,
                               const float* sin_t) {
    VH_ARG(n_kv * d_head <= 1024, "prefill_rope_append: kv row %d exceeds 1024", n_kv * d_head);
    VH_ARG(d_head % 2 == 0 && T >= 1, "prefill_rope_append: bad shape");
    VH_ARG(pos0 >= 0 && pos0 + T <= max_seq, "prefill_rope_append: positions [%d,%d) outside the cache",
           pos0, pos0 + T);
    const int pairs = n_kv * d_head / 2, ppl = pairs / 64;
    if (pairs % 64 == 0 && (ppl == 1 || ppl == 2 || ppl == 4 || ppl == 8) && (d_head / 2) % ppl == 0) {
        const dim3 grid((T + 3) / 4);
        auto a16 = [](const void* ptr) { return ((uintptr_t)ptr & 15) == 0; };
        const char* e = std::getenv("VLRF_HIP_KV_VEC");   // "0": element-wise loads and stores (same values)
        const bool vec = !(e && e[0] == '0') && ppl % 4 == 0 && ld % 4 == 0 && (n_heads * d_head) % 4 == 0 &&
                         d_head % 16 == 0 && a16(qkv) && a16(cos_t) && a16(sin_t) && a16(L.k) && a16(L.v);
#define VH_KVR(P, VEC)                                                                                          \
    hipLaunchKernelGGL((prefill_kv_rows_kernel<P, VEC>), grid, dim3(256), 0, s, L.k, L.v, L.ks, L.vs, L.dtype,   \
                       qkv, ld, n_heads, d_head, max_seq, pos0, T, cos_t, sin_t)
        switch (ppl) {
            case 1: VH_KVR(1, false); break;
            case 2: VH_KVR(2, false); break;
            case 4: if (vec) VH_KVR(4, true); else VH_KVR(4, false); break;
            default: if (vec) VH_KVR(8, true); else VH_KVR(8, false); break;
        }
#undef VH_KVR
        VH_LAUNCHED();
        return VLRF_HIP_OK;
    }
    hipLaunchKernelGGL(prefill_rope_append_kernel, dim3(T), dim3(256), 0, s, L.k, L.v, L.ks, L.vs, L.dtype, qkv, ld,
                       n_heads, n_kv, d_head, max_seq, pos0, cos_t, sin_t);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_embed_rows(hipStream_t s, const float* table, const int* ids, float* x, int T, int D) {
    VH_ARG(T >= 1 && D % 4 == 0, "embed_rows: bad shape");
    hipLaunchKernelGGL(embed_rows_kernel, dim3(T), dim3(256), 0, s, table, ids, x, D);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_kv_dequant(hipStream_t s, const KVLayer& L, int n_kv, int d_head, int max_seq,
                      int ctx_len, float* K_out, float* V_out) {
    VH_ARG(ctx_len >= 0 && ctx_len <= max_seq, "kv_dequant: ctx_len %d outside [0,%d]", ctx_len, max_seq);
    if (ctx_len == 0) return VLRF_HIP_OK;
    hipLaunchKernelGGL(kv_dequant_kernel, dim3(ctx_len), dim3(256), 0, s, L.k, L.v, L.ks, L.vs, L.dtype, n_kv,
                       d_head, max_seq, K_out, V_out);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_rmsnorm(hipStream_t s, const float* x, const float* w, float* out, int rows, int D,
                   float eps) {
    VH_ARG(rows >= 1 && D >= 1, "rmsnorm: empty shape");
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, s, x, w, out, D, eps);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_rope(hipStream_t s, float* x, int T, int n_heads, int d_head, int pos_offset, int max_seq,
                const float* cos_t, const float* sin_t) {
    VH_ARG(T >= 1 && n_heads >= 1 && d_head >= 2 && d_head % 2 == 0, "rope: bad shape");
    VH_ARG(pos_offset >= 0, "rope: negative position");
    hipLaunchKernelGGL(rope_kernel, dim3(T), dim3(256), 0, s, x, n_heads, d_head, pos_offset, max_seq,
                       cos_t, sin_t);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_embed(hipStream_t s, const float* table, const int* tok_dev, float* x, int D) {
    VH_LAUNCH(embed_kernel, dim3(1), dim3(256), 0, s, table, tok_dev, x, D);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_argmax_pairs_step(hipStream_t s, const float2* pairs, int np, int* state, int* gen_ids, int gen_cap) {
    VH_ARG(np >= 1 && np <= 512, "argmax_pairs: %d pairs outside [1,512]", np);
    VH_LAUNCH(argmax_pairs_step_kernel, dim3(1), dim3(512), 0, s, pairs, np, state, gen_ids, gen_cap);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_argmax_step(hipStream_t s, const float* logits, int n, int* state, int* gen_ids,
                       int gen_cap) {
    VH_ARG(n >= 1 && n <= 1024 * 4 * kArgmaxPer, "argmax: %d logits outside [1,%d]", n, 1024 * 4 * kArgmaxPer);
    VH_LAUNCH(argmax_step_kernel, dim3(1), dim3(1024), 0, s, logits, n, state, gen_ids, gen_cap);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

}  // namespace vlrf_hip
