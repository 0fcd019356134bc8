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
// Decode design (gfx950): split-K over the context.  A 256-lane workgroup owns
// one KV head and a 64-token chunk, so each K/V byte is loaded and dequantized
// once and reused by all REP query heads of the GQA group.  Phase 1: lane t of
// wave w scores token c0+t over dimension quarter w against the REP queries
// (LDS broadcast reads of q); the quarters are summed in LDS.  Phase 2:
// per-head chunk max / sum with DPP + shuffle wave reductions.  Phase 3: P.V
// with lanes along d_head (coalesced rows per token), reduced across waves in
// LDS.  Partials (m, l, acc[d]) per (head, chunk) are merged by a combine
// kernel with the log-sum-exp rescale.  With a device-side position the
// kernel also applies RoPE to q and to the new k and quantizes + stores the
// new K/V row before attending (the decode step's fused form).
#include "../internal.hpp"

#include <cmath>

namespace vlrf_hip {
namespace {

constexpr int kChunk = 64;        // tokens per split-K workgroup
constexpr int kMaxSplits = 512;   // contexts up to 32768 tokens
constexpr float kNegInf = -INFINITY;

__device__ __forceinline__ float block_max256(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_max(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return v;
}

// RoPE of one pair (rope.hpp:90-96), each product rounded separately.
__device__ __forceinline__ void rope2(float x0, float x1, float c, float s, float* y0, float* y1) {
#pragma clang fp contract(off)
    const float a = x0 * c, b = x1 * s, e = x1 * c, f = x0 * s;
    *y0 = a - b;
    *y1 = e + f;
}

template <int D, int REP, bool Q8, bool FUSED>
__global__ __launch_bounds__(256) void attn_decode_partial_kernel(
    const float* __restrict__ q, const int8_t* kq, const int8_t* vq, const float* ks, const float* vs,
    const float* __restrict__ kf, const float* __restrict__ vf, long head_stride, int ctx_len,
    const int* __restrict__ ctx_dev, int n_splits, float scale, float* __restrict__ part, DecodeFuse fz) {
    constexpr int DQ = D / 4;                  // dims per wave in the score phase
    constexpr int DL = D / 64;                 // 4-dim groups per lane in the P.V phase
    __shared__ __align__(16) float qs[REP][D];
    __shared__ float sp4[4][REP][kChunk];      // score partials per dim quarter
    __shared__ float red[4][REP][D];
    __shared__ float mstat[REP], lstat[REP];
    __shared__ float rmax[4];
    __shared__ float krow[FUSED ? 1024 : 1], vrow[FUSED ? 1024 : 1];
    __shared__ __align__(16) float newk[FUSED ? D : 1], newv[FUSED ? D : 1];

    const int split = blockIdx.x, g = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int HALF = D / 2;
    int pos = -1, ctx;
    if constexpr (FUSED) {
        pos = *ctx_dev;          // tokens before this one
        ctx = pos + 1;
    } else {
        ctx = ctx_dev ? (*ctx_dev + ctx_len) : ctx_len;
    }
    // Rows past the cache capacity are never read, even if the device-side
    // position were corrupt (the host checks capacity before queuing).
    ctx = min(ctx, (int)(head_stride / D));
    const int c0 = split * kChunk;
    const size_t hb = (size_t)g * head_stride;

    float* pout = part + (size_t)(g * REP) * n_splits * (D + 2) + (size_t)split * (D + 2);
    if (c0 >= ctx) {   // chunk past the context: empty partial
        for (int i = tid; i < REP * (D + 2); i += 256) {
            const int h = i / (D + 2), dd = i % (D + 2);
            pout[(size_t)h * n_splits * (D + 2) + dd] = dd == D ? kNegInf : 0.f;
        }
        return;
    }
    const int nt = min(kChunk, ctx - c0);       // valid tokens of the chunk
    const bool has_new = FUSED && pos >= c0 && pos < c0 + kChunk;

    // Vector loads complete in issue order, so the small L2-resident operands
    // (queries, RoPE tables, the new K/V row) are requested first, then the
    // cache stream, and every load is branch-free (out-of-range tokens read
    // row c0, which is in bounds, and are masked where they are used): a load
    // in a branch, or a value converted right after its load, would make the
    // wave wait for the whole stream early.
    constexpr int PAIRS = REP * HALF, PPT = (PAIRS + 255) / 256;
    const bool rot = FUSED && pos < fz.max_seq;   // rope.hpp:84: positions >= max_seq stay unrotated
    float qlo[PPT], qhi[PPT];
#pragma unroll
    for (int p = 0; p < PPT; ++p) {
        const int i = min(tid + 256 * p, PAIRS - 1), h = i / HALF, j = i - h * HALF;
        const float* qh = q + (size_t)(g * REP + h) * D;
        qlo[p] = qh[j];
        qhi[p] = qh[j + HALF];
    }
    float cw = 1.f, sw = 0.f;
    if (rot) {
        cw = fz.cos_t[(size_t)pos * HALF + (tid & (HALF - 1))];
        sw = fz.sin_t[(size_t)pos * HALF + (tid & (HALF - 1))];
    }
    constexpr int NPT = FUSED ? 4 : 1;            // new-row floats per thread (row <= 1024)
    float kn[NPT], vn[NPT];
    if constexpr (FUSED) {
        const int row = fz.n_kv * D;
#pragma unroll
        for (int p = 0; p < NPT; ++p) {
            const int i = min(tid + 256 * p, row - 1);
            kn[p] = fz.k_new[i];
            vn[p] = fz.v_new[i];
        }
    }

    // The cache stream: this thread's K slice (token lane, dims of this wave)
    // and its V words (tokens wave*16 + t4 + 4i, dims 4dg..), kept as raw codes.
    const int t4 = lane >> 4, dg = lane & 15;
    constexpr int KW = Q8 ? DQ / 16 : DQ / 4;      // 16-byte words of the K slice
    uint4 kraw[KW];
    uint4 vraw[4][DL];                             // Q8: .x holds 4 codes; f32: 4 floats
    float ksc = 1.f, vsc[4] = {1.f, 1.f, 1.f, 1.f};
    {
        const int jt = lane < nt ? c0 + lane : c0;
#pragma unroll
        for (int i = 0; i < KW; ++i) {
            if constexpr (Q8)
                kraw[i] = *reinterpret_cast<const uint4*>(kq + hb + (size_t)jt * D + wave * DQ + 16 * i);
            else
                kraw[i] = *reinterpret_cast<const uint4*>(kf + hb + (size_t)jt * D + wave * DQ + 4 * i);
        }
        if constexpr (Q8) ksc = ks[jt];
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int t = wave * 16 + t4 + 4 * it;
            const int jj = t < nt ? c0 + t : c0;
            if constexpr (Q8) vsc[it] = vs[jj];
#pragma unroll
            for (int dl = 0; dl < DL; ++dl) {
                if constexpr (Q8) {
                    vraw[it][dl].x = *reinterpret_cast<const uint32_t*>(vq + hb + (size_t)jj * D + dl * 64 + dg * 4);
                } else {
                    vraw[it][dl] = *reinterpret_cast<const uint4*>(vf + hb + (size_t)jj * D + dl * 64 + dg * 4);
                }
            }
        }
    }

    // ---- queries of the GQA group (RoPE at the device position when fused) -------
    {
        float* cst = sp4[0][0];                    // RoPE table row, staged before phase 1 reuses sp4
        if (rot && tid < HALF) { cst[tid] = cw; cst[HALF + tid] = sw; }
        __syncthreads();
#pragma unroll
        for (int p = 0; p < PPT; ++p) {
            const int i = tid + 256 * p;
            if (i < PAIRS) {
                const int h = i / HALF, j = i - h * HALF;
                if (rot) rope2(qlo[p], qhi[p], cst[j], cst[HALF + j], &qs[h][j], &qs[h][j + HALF]);
                else { qs[h][j] = qlo[p]; qs[h][j + HALF] = qhi[p]; }
            }
        }
        // ---- decode fusion: the current token's K/V row ----------------------------
        // attention.hpp:109-128: RoPE on k, then KVCache::append quantizes the whole
        // row (quantize_row_q8_0, kv_cache.hpp:102-117) before attention reads it.
        // Every chunk holding `pos` quantizes the row itself and uses the dequantized
        // values for that token; the workgroup of KV head g stores head g's codes,
        // KV head 0 stores the row scales.
        if constexpr (FUSED) {
            if (has_new) {
                const int row = fz.n_kv * D;
#pragma unroll
                for (int p = 0; p < NPT; ++p) {
                    const int i = tid + 256 * p;
                    if (i < row) { krow[i] = kn[p]; vrow[i] = vn[p]; }
                }
                __syncthreads();
                if (rot) {
                    for (int i = tid; i < fz.n_kv * HALF; i += 256) {
                        const int h = i / HALF, j = i - h * HALF;
                        float* kh = krow + h * D;
                        const float x0 = kh[j], x1 = kh[j + HALF];
                        rope2(x0, x1, cst[j], cst[HALF + j], &kh[j], &kh[j + HALF]);
                    }
                }
                __syncthreads();
                float ak = 0.f, av = 0.f;
                for (int i = tid; i < row; i += 256) { ak = fmaxf(ak, fabsf(krow[i])); av = fmaxf(av, fabsf(vrow[i])); }
                ak = block_max256(ak, rmax);
                av = block_max256(av, rmax);
                const float sk = ak != 0.f ? ak / 127.f : 0.f, sv = av != 0.f ? av / 127.f : 0.f;
                const float ik = ak != 0.f ? 1.f / sk : 0.f, iv = av != 0.f ? 1.f / sv : 0.f;
                for (int i = tid; i < D; i += 256) {
                    const int a = ak != 0.f ? min(127, max(-127, (int)roundf(krow[g * D + i] * ik))) : 0;
                    const int b = av != 0.f ? min(127, max(-127, (int)roundf(vrow[g * D + i] * iv))) : 0;
                    newk[i] = (float)a * sk;
                    newv[i] = (float)b * sv;
                    fz.kq_w[hb + (size_t)pos * D + i] = (int8_t)a;
                    fz.vq_w[hb + (size_t)pos * D + i] = (int8_t)b;
                }
                if (g == 0 && tid == 0) { fz.ks_w[pos] = sk; fz.vs_w[pos] = sv; }
            }
        }
        __syncthreads();
    }

    // ---- phase 1: partial scores over this wave's quarter of d_head --------------
    {
        float kd[DQ];
        if (FUSED && has_new && c0 + lane == pos) {
#pragma unroll
            for (int i = 0; i < DQ; ++i) kd[i] = newk[wave * DQ + i];
        } else {
#pragma unroll
            for (int i = 0; i < KW; ++i) {
                const uint32_t w[4] = {kraw[i].x, kraw[i].y, kraw[i].z, kraw[i].w};
                if constexpr (Q8) {
#pragma unroll
                    for (int k = 0; k < 16; ++k)   // dequantize_row_q8_0
                        kd[16 * i + k] = (float)(int8_t)(w[k >> 2] >> (8 * (k & 3))) * ksc;
                } else {
#pragma unroll
                    for (int k = 0; k < 4; ++k) kd[4 * i + k] = __uint_as_float(w[k]);
                }
            }
        }
#pragma unroll
        for (int h = 0; h < REP; ++h) {
            float dsum = 0.f;
#pragma unroll
            for (int i = 0; i < DQ; i += 4) {
                const float4 qv = *reinterpret_cast<const float4*>(&qs[h][wave * DQ + i]);
                dsum += qv.x * kd[i] + qv.y * kd[i + 1] + qv.z * kd[i + 2] + qv.w * kd[i + 3];
            }
            sp4[wave][h][lane] = dsum;
        }
    }
    __syncthreads();

    // ---- phase 2: per-head chunk max and sum (DPP/shuffle wave reductions) --------
    for (int h = wave; h < REP; h += 4) {
        float sc = kNegInf;
        if (lane < nt) sc = ((sp4[0][h][lane] + sp4[1][h][lane]) + (sp4[2][h][lane] + sp4[3][h][lane])) * scale;
        const float mx = wave_max(sc);   // finite: token c0 < ctx is in this chunk
        const float p = expf(sc - mx);
        sp4[0][h][lane] = p;
        const float sum = wave_sum(p);
        if (lane == 0) { mstat[h] = mx; lstat[h] = sum; }
    }
    __syncthreads();

    // ---- phase 3: P.V (lane = 4 dims x token offset t4, wave = 16 tokens) ----------
    float acc[REP][DL][4];
#pragma unroll
    for (int h = 0; h < REP; ++h)
#pragma unroll
        for (int dl = 0; dl < DL; ++dl)
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[h][dl][k] = 0.f;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int t = wave * 16 + t4 + 4 * it;
        if (t < nt) {
            float vd[DL][4];
            if (FUSED && has_new && c0 + t == pos) {
#pragma unroll
                for (int dl = 0; dl < DL; ++dl)
#pragma unroll
                    for (int k = 0; k < 4; ++k) vd[dl][k] = newv[dl * 64 + dg * 4 + k];
            } else {
#pragma unroll
                for (int dl = 0; dl < DL; ++dl) {
                    if constexpr (Q8) {
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            vd[dl][k] = (float)(int8_t)(vraw[it][dl].x >> (8 * k)) * vsc[it];
                    } else {
                        vd[dl][0] = __uint_as_float(vraw[it][dl].x); vd[dl][1] = __uint_as_float(vraw[it][dl].y);
                        vd[dl][2] = __uint_as_float(vraw[it][dl].z); vd[dl][3] = __uint_as_float(vraw[it][dl].w);
                    }
                }
            }
#pragma unroll
            for (int h = 0; h < REP; ++h) {
                const float p = sp4[0][h][t];
#pragma unroll
                for (int dl = 0; dl < DL; ++dl)
#pragma unroll
                    for (int k = 0; k < 4; ++k) acc[h][dl][k] += p * vd[dl][k];
            }
        }
    }
#pragma unroll
    for (int h = 0; h < REP; ++h)
#pragma unroll
        for (int dl = 0; dl < DL; ++dl)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float a = acc[h][dl][k];
                a += __shfl_xor(a, 16);
                a += __shfl_xor(a, 32);
                if (t4 == 0) red[wave][h][dl * 64 + dg * 4 + k] = a;
            }
    __syncthreads();
    for (int i = tid; i < REP * D; i += 256) {
        const int h = i / D, dd = i % D;
        pout[(size_t)h * n_splits * (D + 2) + dd] =
            (red[0][h][dd] + red[1][h][dd]) + (red[2][h][dd] + red[3][h][dd]);
    }
    if (tid < REP) {
        pout[(size_t)tid * n_splits * (D + 2) + D] = mstat[tid];
        pout[(size_t)tid * n_splits * (D + 2) + D + 1] = lstat[tid];
    }
}

// Log-sum-exp merge of the per-chunk partials of one query head.  The 256
// threads form G = 256/D groups of D lanes (one lane per dimension); group gi
// merges splits gi, gi+G, ... in passes of B splits whose loads are all issued
// before any is used (index clamped, masked afterwards), then the G group
// results are merged through LDS.
template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ part, int n_splits,
                                                           float* __restrict__ out) {
    constexpr int G = 256 / D, B = 16;
    __shared__ float sm[G][D], sl[G][D], so[G][D];
    const int h = blockIdx.x, gi = threadIdx.x / D, d = threadIdx.x - gi * D;
    const float* p = part + (size_t)h * n_splits * (D + 2);
    float M = kNegInf, L = 0.f, o = 0.f;
    for (int s0 = gi; s0 < n_splits; s0 += G * B) {
        float pm[B], pl[B], po[B];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float* ps = p + (size_t)min(s0 + b * G, n_splits - 1) * (D + 2);
            pm[b] = ps[D];
            pl[b] = ps[D + 1];
            po[b] = ps[d];
        }
        float mb = kNegInf;
#pragma unroll
        for (int b = 0; b < B; ++b)
            if (s0 + b * G < n_splits) mb = fmaxf(mb, pm[b]);
        const float mn = fmaxf(M, mb);
        if (mn != kNegInf) {
            const float c = M == kNegInf ? 0.f : expf(M - mn);
            L *= c;
            o *= c;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                if (s0 + b * G < n_splits && pm[b] != kNegInf) {
                    const float w = expf(pm[b] - mn);
                    L += w * pl[b];
                    o += w * po[b];
                }
            }
            M = mn;
        }
    }
    sm[gi][d] = M;
    sl[gi][d] = L;
    so[gi][d] = o;
    __syncthreads();
    if (gi == 0) {
        float mt = kNegInf;
#pragma unroll
        for (int k = 0; k < G; ++k) mt = fmaxf(mt, sm[k][d]);
        float lt = 0.f, ot = 0.f;
        if (mt != kNegInf) {
#pragma unroll
            for (int k = 0; k < G; ++k) {
                if (sm[k][d] != kNegInf) {
                    const float w = expf(sm[k][d] - mt);
                    lt += w * sl[k][d];
                    ot += w * so[k][d];
                }
            }
        }
        out[(size_t)h * D + d] = (lt > 0.f) ? ot * (1.f / lt) : 0.f;
    }
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
                       const int* ctx_dev, int n_splits, float scale, float* part, float* out,
                       const DecodeFuse* fuse) {
    VH_ARG(n_kv > 0 && n_heads % n_kv == 0, "attn_decode: n_heads %d not a multiple of n_kv %d",
           n_heads, n_kv);
    const int rep = n_heads / n_kv;
    VH_ARG(d_head == 64 || d_head == 128, "attn_decode: d_head %d not in {64,128}", d_head);
    VH_ARG(rep == 1 || rep == 2 || rep == 4 || rep == 8, "attn_decode: GQA group %d not in {1,2,4,8}", rep);
    VH_ARG(n_splits >= 1 && n_splits <= kMaxSplits, "attn_decode: %d splits outside [1,%d]", n_splits,
           kMaxSplits);
    if (!ctx_dev)
        VH_ARG(ctx_len >= 1 && ctx_len <= n_splits * kChunk, "attn_decode: ctx_len %d outside [1,%d]",
               ctx_len, n_splits * kChunk);
    const bool q8 = kq != nullptr;
    VH_ARG(q8 ? (vq && ks && vs) : (kf && vf), "attn_decode: missing K/V operands");
    DecodeFuse fz{};
    if (fuse) {
        VH_ARG(q8 && ctx_dev, "attn_decode: fusion needs the Q8 cache and a device position");
        VH_ARG(fuse->n_kv == n_kv && n_kv * d_head <= 1024, "attn_decode: bad fusion row");
        fz = *fuse;
    }
    dim3 grid(n_splits, n_kv), block(256);
#define VH_AD(D, R, Q, FU)                                                                          \
    hipLaunchKernelGGL((attn_decode_partial_kernel<D, R, Q, FU>), grid, block, 0, s, q, kq, vq, ks,  \
                       vs, kf, vf, head_stride, ctx_len, ctx_dev, n_splits, scale, part, fz)
#define VH_AD_R(D, Q, FU)                       \
    switch (rep) {                              \
        case 1: VH_AD(D, 1, Q, FU); break;      \
        case 2: VH_AD(D, 2, Q, FU); break;      \
        case 4: VH_AD(D, 4, Q, FU); break;      \
        default: VH_AD(D, 8, Q, FU); break;     \
    }
    if (d_head == 64) {
        if (fuse) { VH_AD_R(64, true, true) }
        else if (q8) { VH_AD_R(64, true, false) }
        else { VH_AD_R(64, false, false) }
    } else {
        if (fuse) { VH_AD_R(128, true, true) }
        else if (q8) { VH_AD_R(128, true, false) }
        else { VH_AD_R(128, false, false) }
    }
#undef VH_AD_R
#undef VH_AD
    VH_LAUNCHED();
    if (d_head == 64)
        hipLaunchKernelGGL((attn_combine_kernel<64>), dim3(n_heads), dim3(256), 0, s, part, n_splits, out);
    else
        hipLaunchKernelGGL((attn_combine_kernel<128>), dim3(n_heads), dim3(256), 0, s, part, n_splits, out);
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
