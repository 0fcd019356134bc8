// attention.hip - flash-attention decode over the Q8_0 KV cache and the
// general f32 scaled-dot-product attention.
//
// Reference semantics: AttentionBlock::flash_attn_head (attention.hpp:207-309)
// -- 1/sqrt(d_h) scale (attention.hpp:373-374), online softmax, output
// acc * (1/l) or 0 when l == 0, causal rule kpos > qpos with
// qpos = q + (ctx - T); decode (T == 1 with a cache) is non-causal
// (attention.hpp:171) and attends over the dequantized cache including the
// token just appended (attention.hpp:127-145).
//
// Decode design (gfx950): split-K over the context.  A workgroup owns one KV
// head and a 256-token chunk, so each K/V byte is loaded and dequantized once
// and reused by all REP query heads of the GQA group.  Phase 1: thread t
// scores token c0+t against the REP queries (LDS broadcast reads of q).
// Phase 2: per-head chunk max / sum with DPP + shuffle wave reductions.
// Phase 3: P.V with lanes along d_head (coalesced 64 B rows per token),
// reduced across waves in LDS.  Partials (m, l, acc[d]) per (head, chunk) are
// merged by a small combine kernel with the log-sum-exp rescale.
#include "../internal.hpp"

#include <cmath>

namespace vlrf_hip {
namespace {

constexpr int kChunk = 256;
constexpr float kNegInf = -INFINITY;

template <int D, int REP, bool Q8>
__global__ __launch_bounds__(256) void attn_decode_partial_kernel(
    const float* __restrict__ q, const int8_t* __restrict__ kq, const int8_t* __restrict__ vq,
    const float* __restrict__ ks, const float* __restrict__ vs, const float* __restrict__ kf,
    const float* __restrict__ vf, long head_stride, int ctx_len, const int* __restrict__ ctx_dev,
    int n_splits, float scale, float* __restrict__ part) {
    __shared__ __align__(16) float qs[REP][D];
    __shared__ float sp[REP][kChunk];
    __shared__ float red[4][REP][D];
    __shared__ float mstat[REP], lstat[REP];

    const int split = blockIdx.x, g = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Rows past the cache capacity are never read, even if the device-side
    // position were corrupt (the host checks capacity before queuing).
    const int ctx = min(ctx_dev ? (*ctx_dev + ctx_len) : ctx_len, (int)(head_stride / D));
    const int c0 = split * kChunk;
    const size_t hb = (size_t)g * head_stride;

    for (int i = tid; i < REP * D; i += 256) qs[i / D][i % D] = q[(size_t)(g * REP) * D + i];
    __syncthreads();

    float* pout = part + (size_t)(g * REP) * n_splits * (D + 2) + (size_t)split * (D + 2);
    if (c0 >= ctx) {   // chunk past the context: empty partial
        for (int i = tid; i < REP * (D + 2); i += 256) {
            const int h = i / (D + 2), dd = i % (D + 2);
            pout[(size_t)h * n_splits * (D + 2) + dd] = dd == D ? kNegInf : 0.f;
        }
        return;
    }

    // ---- phase 1: scores --------------------------------------------------
    const int j = c0 + tid;
    float dot[REP];
#pragma unroll
    for (int h = 0; h < REP; ++h) dot[h] = 0.f;
    if (j < ctx) {
        float kscale = Q8 ? ks[j] : 1.f;
#pragma unroll
        for (int d0 = 0; d0 < D; d0 += 16) {
            float kv[16];
            if constexpr (Q8) {
                const uint4 u = *reinterpret_cast<const uint4*>(kq + hb + (size_t)j * D + d0);
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    kv[i] = (float)(int8_t)(w[i >> 2] >> (8 * (i & 3))) * kscale;  // dequantize_row_q8_0
            } else {
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    const float4 v = *reinterpret_cast<const float4*>(kf + hb + (size_t)j * D + d0 + i);
                    kv[i] = v.x; kv[i + 1] = v.y; kv[i + 2] = v.z; kv[i + 3] = v.w;
                }
            }
#pragma unroll
            for (int h = 0; h < REP; ++h) {
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    const float4 qv = *reinterpret_cast<const float4*>(&qs[h][d0 + i]);
                    dot[h] += qv.x * kv[i] + qv.y * kv[i + 1] + qv.z * kv[i + 2] + qv.w * kv[i + 3];
                }
            }
        }
    }
#pragma unroll
    for (int h = 0; h < REP; ++h) sp[h][tid] = (j < ctx) ? dot[h] * scale : kNegInf;
    __syncthreads();

    // ---- phase 2: chunk max and sum per head ---------------------------------
    for (int h = wave; h < REP; h += 4) {
        float v[4], mx = kNegInf;
#pragma unroll
        for (int i = 0; i < 4; ++i) { v[i] = sp[h][lane + 64 * i]; mx = fmaxf(mx, v[i]); }
        mx = wave_max(mx);   // finite: token c0 < ctx is in this chunk
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = expf(v[i] - mx);
            sp[h][lane + 64 * i] = p;
            sum += p;
        }
        sum = wave_sum(sum);
        if (lane == 0) { mstat[h] = mx; lstat[h] = sum; }
    }
    __syncthreads();

    // ---- phase 3: P.V ----------------------------------------------------------
    constexpr int DL = D / 64;
    float acc[REP][DL];
#pragma unroll
    for (int h = 0; h < REP; ++h)
#pragma unroll
        for (int i = 0; i < DL; ++i) acc[h][i] = 0.f;
    const int t0 = wave * 64, t1 = min(t0 + 64, ctx - c0);
#pragma unroll 4
    for (int t = t0; t < t1; ++t) {
        const int jj = c0 + t;
        float vv[DL];
        if constexpr (Q8) {
            const float sc = vs[jj];
#pragma unroll
            for (int i = 0; i < DL; ++i) vv[i] = (float)vq[hb + (size_t)jj * D + lane + 64 * i] * sc;
        } else {
#pragma unroll
            for (int i = 0; i < DL; ++i) vv[i] = vf[hb + (size_t)jj * D + lane + 64 * i];
        }
#pragma unroll
        for (int h = 0; h < REP; ++h) {
            const float p = sp[h][t];
#pragma unroll
            for (int i = 0; i < DL; ++i) acc[h][i] += p * vv[i];
        }
    }
#pragma unroll
    for (int h = 0; h < REP; ++h)
#pragma unroll
        for (int i = 0; i < DL; ++i) red[wave][h][lane + 64 * i] = acc[h][i];
    __syncthreads();
    for (int i = tid; i < REP * D; i += 256) {
        const int h = i / D, dd = i % D;
        pout[(size_t)h * n_splits * (D + 2) + dd] =
            red[0][h][dd] + red[1][h][dd] + red[2][h][dd] + red[3][h][dd];
    }
    if (tid < REP) {
        pout[(size_t)tid * n_splits * (D + 2) + D] = mstat[tid];
        pout[(size_t)tid * n_splits * (D + 2) + D + 1] = lstat[tid];
    }
}

template <int D>
__global__ __launch_bounds__(D) void attn_combine_kernel(const float* __restrict__ part, int n_splits,
                                                         float* __restrict__ out) {
    const int h = blockIdx.x, d = threadIdx.x;
    const float* p = part + (size_t)h * n_splits * (D + 2);
    float M = kNegInf;
    for (int s = 0; s < n_splits; ++s) M = fmaxf(M, p[(size_t)s * (D + 2) + D]);
    float L = 0.f, o = 0.f;
    if (M != kNegInf) {
        for (int s = 0; s < n_splits; ++s) {
            const float ms = p[(size_t)s * (D + 2) + D];
            if (ms == kNegInf) continue;
            const float w = expf(ms - M);
            L += w * p[(size_t)s * (D + 2) + D + 1];
            o += w * p[(size_t)s * (D + 2) + d];
        }
    }
    out[(size_t)h * D + d] = (L > 0.f) ? o * (1.f / L) : 0.f;
}

// ---- general f32 attention: one thread per query row, 64x64 tiles --------------
template <int D>
__global__ __launch_bounds__(64) void attn_f32_tiled_kernel(const float* __restrict__ Q,
                                                            const float* __restrict__ K,
                                                            const float* __restrict__ V,
                                                            float* __restrict__ O, int T, int ctx,
                                                            int d, float scale, int causal) {
    __shared__ __align__(16) float Kt[64][D];
    __shared__ __align__(16) float Vt[64][D];
    const int h = blockIdx.y, q0 = blockIdx.x * 64, lane = threadIdx.x, qi = q0 + lane;
    const float* Qh = Q + (size_t)h * T * d;
    const float* Kh = K + (size_t)h * ctx * d;
    const float* Vh = V + (size_t)h * ctx * d;
    float qv[D], acc[D];
#pragma unroll
    for (int i = 0; i < D; ++i) {
        qv[i] = (qi < T && i < d) ? Qh[(size_t)qi * d + i] : 0.f;
        acc[i] = 0.f;
    }
    float m = kNegInf, l = 0.f;
    const int past = ctx - T;
    const int br = min(64, T - q0);
    const int k_limit = causal ? min(ctx, q0 + br + past) : ctx;
    const int qpos = qi + past;

    for (int k0 = 0; k0 < k_limit; k0 += 64) {
        const int bc = min(64, k_limit - k0);
        for (int i = lane; i < 64 * D; i += 64) {
            const int r = i / D, c = i % D;
            const bool ok = r < bc && c < d;
            Kt[r][c] = ok ? Kh[(size_t)(k0 + r) * d + c] : 0.f;
            Vt[r][c] = ok ? Vh[(size_t)(k0 + r) * d + c] : 0.f;
        }
        __syncthreads();
        for (int j0 = 0; j0 < bc; j0 += 16) {
            float s[16], bmax = kNegInf;
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
                const int j = j0 + jj;
                float dot = 0.f;
#pragma unroll
                for (int i = 0; i < D; i += 4) {
                    const float4 kv = *reinterpret_cast<const float4*>(&Kt[j][i]);
                    dot += qv[i] * kv.x + qv[i + 1] * kv.y + qv[i + 2] * kv.z + qv[i + 3] * kv.w;
                }
                float sj = dot * scale;
                if (j >= bc || (causal && k0 + j > qpos)) sj = kNegInf;
                s[jj] = sj;
                bmax = fmaxf(bmax, sj);
            }
            if (bmax != kNegInf) {
                const float m_new = fmaxf(m, bmax);
                float bsum = 0.f;
#pragma unroll
                for (int jj = 0; jj < 16; ++jj) { s[jj] = expf(s[jj] - m_new); bsum += s[jj]; }
                const float corr = (m == kNegInf) ? 0.f : expf(m - m_new);
                l = l * corr + bsum;
#pragma unroll
                for (int i = 0; i < D; ++i) acc[i] *= corr;
#pragma unroll
                for (int jj = 0; jj < 16; ++jj) {
                    const float p = s[jj];
#pragma unroll
                    for (int i = 0; i < D; i += 4) {
                        const float4 vv = *reinterpret_cast<const float4*>(&Vt[j0 + jj][i]);
                        acc[i] += p * vv.x; acc[i + 1] += p * vv.y;
                        acc[i + 2] += p * vv.z; acc[i + 3] += p * vv.w;
                    }
                }
                m = m_new;
            }
        }
        __syncthreads();
    }
    if (qi < T) {
        const float inv = (l > 0.f) ? 1.f / l : 0.f;
        float* Oh = O + (size_t)h * T * d + (size_t)qi * d;
        for (int i = 0; i < d; ++i) Oh[i] = acc[i] * inv;
    }
}

}  // namespace

int attn_decode_splits(int max_ctx) { return (max_ctx + kChunk - 1) / kChunk; }

int launch_attn_decode(hipStream_t s, const float* q, const int8_t* kq, const int8_t* vq,
                       const float* ks, const float* vs, const float* kf, const float* vf,
                       long head_stride, int n_heads, int n_kv, int d_head, int ctx_len,
                       const int* ctx_dev, int n_splits, float scale, float* part, float* out) {
    VH_ARG(n_kv > 0 && n_heads % n_kv == 0, "attn_decode: n_heads %d not a multiple of n_kv %d",
           n_heads, n_kv);
    const int rep = n_heads / n_kv;
    VH_ARG(d_head == 64 || d_head == 128, "attn_decode: d_head %d not in {64,128}", d_head);
    VH_ARG(rep == 1 || rep == 2 || rep == 4 || rep == 8, "attn_decode: GQA group %d not in {1,2,4,8}", rep);
    VH_ARG(n_splits >= 1, "attn_decode: no splits");
    if (!ctx_dev)
        VH_ARG(ctx_len >= 1 && ctx_len <= n_splits * kChunk, "attn_decode: ctx_len %d outside [1,%d]",
               ctx_len, n_splits * kChunk);
    const bool q8 = kq != nullptr;
    VH_ARG(q8 ? (vq && ks && vs) : (kf && vf), "attn_decode: missing K/V operands");
    dim3 grid(n_splits, n_kv), block(256);
#define VH_AD(D, R, Q)                                                                          \
    hipLaunchKernelGGL((attn_decode_partial_kernel<D, R, Q>), grid, block, 0, s, q, kq, vq, ks,  \
                       vs, kf, vf, head_stride, ctx_len, ctx_dev, n_splits, scale, part)
#define VH_AD_R(D, Q)                       \
    switch (rep) {                          \
        case 1: VH_AD(D, 1, Q); break;      \
        case 2: VH_AD(D, 2, Q); break;      \
        case 4: VH_AD(D, 4, Q); break;      \
        default: VH_AD(D, 8, Q); break;     \
    }
    if (d_head == 64) {
        if (q8) { VH_AD_R(64, true) } else { VH_AD_R(64, false) }
    } else {
        if (q8) { VH_AD_R(128, true) } else { VH_AD_R(128, false) }
    }
#undef VH_AD_R
#undef VH_AD
    VH_LAUNCHED();
    if (d_head == 64)
        hipLaunchKernelGGL((attn_combine_kernel<64>), dim3(n_heads), dim3(64), 0, s, part, n_splits, out);
    else
        hipLaunchKernelGGL((attn_combine_kernel<128>), dim3(n_heads), dim3(128), 0, s, part, n_splits, out);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_attn_f32_tiled(hipStream_t s, const float* Q, const float* K, const float* V, float* O,
                          int n_h, int T, int ctx_len, int d_h, float scale, int causal) {
    VH_ARG(n_h >= 1 && T >= 1 && ctx_len >= 1, "attn_f32: empty shape");
    VH_ARG(d_h >= 1 && d_h <= 128, "attn_f32: d_h %d outside [1,128]", d_h);
    VH_ARG(T <= ctx_len || !causal, "attn_f32: causal with T > ctx_len");
    dim3 grid((T + 63) / 64, n_h), block(64);
#define VH_AT(D) hipLaunchKernelGGL((attn_f32_tiled_kernel<D>), grid, block, 0, s, Q, K, V, O, T, \
                                    ctx_len, d_h, scale, causal)
    if (d_h <= 8) VH_AT(8);
    else if (d_h <= 16) VH_AT(16);
    else if (d_h <= 32) VH_AT(32);
    else if (d_h <= 64) VH_AT(64);
    else VH_AT(128);
#undef VH_AT
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

}  // namespace vlrf_hip
