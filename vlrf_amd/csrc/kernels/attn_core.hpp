// attn_core.hpp - the decode attention of one query head over one block of
// cache rows, shared by the stand-alone decode kernel (attention.hip) and the
// fused QKV + attention launch (qkv_attn.hip).
//
// Reference semantics: AttentionBlock::flash_attn_head (attention.hpp:207-309)
// for T = 1 (non-causal, attention.hpp:171), scale 1/sqrt(d_h)
// (attention.hpp:373-374); with decode fusion the token's K/V row is rotated
// (rope.hpp:90-96) and stored (kv_cache.hpp:102-117) before attention reads it
// back (attention.hpp:109-145).
//
// Layout: NW waves of 64 lanes; wave w scores the 64 rows c0 + 64w + lane
// against q (lane = token; the softmax max and sum are wave reductions) and
// accumulates P.V with lane (tg, dg) = (lane/4, lane%4) owning dims
// 16dg..16dg+15 over tokens tg + 16j, the V rows read as 16-element pieces.
// The waves' (m, l, acc) are merged in LDS with the log-sum-exp rule.  Under
// fusion the row at `pos` is left out of the rounds (its cache row may not be
// written yet) and merged as one more entry (score q.k_stored, weight 1, value
// the stored V row).
#pragma once

#include "../internal.hpp"
#include "gemv_core.hpp"

#include <cmath>

namespace vlrf_hip {
namespace attn {

constexpr int D = 64, HALF = 32;
constexpr float kNegInf = -INFINITY;

using gemv::s8f;
__device__ __forceinline__ float4 s8f4(uint32_t w) { return make_float4(s8f<0>(w), s8f<1>(w), s8f<2>(w), s8f<3>(w)); }

// RoPE of one pair (rope.hpp:90-96), each product rounded separately.
__device__ __forceinline__ void rope2(float x0, float x1, float c, float s, float* y0, float* y1) {
#pragma clang fp contract(off)
    const float a = x0 * c, b = x1 * s, e = x1 * c, f = x0 * s;
    *y0 = a - b;
    *y1 = e + f;
}

// Elements 4i..4i+3 of a 64-element row held as 16-byte words, as f32.
template <int KVT>
__device__ __forceinline__ float4 row4(const uint4* wds, int i) {
    if constexpr (KVT == VLRF_HIP_KV_Q8_0) {
        const uint4 k = wds[i >> 2];
        const uint32_t u = (i & 3) == 0 ? k.x : (i & 3) == 1 ? k.y : (i & 3) == 2 ? k.z : k.w;
        return make_float4((float)(int8_t)u, (float)(int8_t)(u >> 8), (float)(int8_t)(u >> 16),
                           (float)(int8_t)(u >> 24));
    } else if constexpr (KVT == VLRF_HIP_KV_F16) {
        const uint4 k = wds[i >> 1];
        const uint32_t a = (i & 1) ? k.z : k.x, b = (i & 1) ? k.w : k.y;
        return make_float4(f16_bits_to_f32(a & 0xFFFFu), f16_bits_to_f32(a >> 16), f16_bits_to_f32(b & 0xFFFFu),
                           f16_bits_to_f32(b >> 16));
    } else {
        const uint4 k = wds[i];
        return make_float4(__uint_as_float(k.x), __uint_as_float(k.y), __uint_as_float(k.z), __uint_as_float(k.w));
    }
}

template <int KVT>
struct KV {
    static constexpr int EB = KVT == VLRF_HIP_KV_Q8_0 ? 1 : KVT == VLRF_HIP_KV_F16 ? 2 : 4;   // bytes per element
    static constexpr int KW = D * EB / 16;   // 16-byte words of a K row
    static constexpr int VW = EB;            // 16-byte words of a 16-element V piece
};

// One round of cache rows in registers: the K row of token base + lane, the V
// pieces of tokens base + tg + 16j (dims 16dg..16dg+15), and the Q8_0 row scales.
template <int KVT>
struct Round {
    uint4 k[KV<KVT>::KW];
    uint4 v[4][KV<KVT>::VW];
    float ks, vs;
};

// Loads the round of wave w starting at row base (rows clamped into the cache;
// rows past the context are masked where they are used).
// Global-memory views: a pointer read from a table in memory is otherwise a
// flat pointer, and flat loads also count against the LDS counter.
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4v gu32x4v;
typedef const __attribute__((address_space(1))) float gfloat;
__device__ __forceinline__ uint4 gload16(const int8_t* p) {
    const u32x4v t = *(gu32x4v*)p;
    return make_uint4(t.x, t.y, t.z, t.w);
}

template <int KVT>
__device__ __forceinline__ void load_round(Round<KVT>& R, const int8_t* kc, const int8_t* vc, const float* ks,
                                           const float* vs, size_t hb, int base, int cap, int lane) {
    constexpr int EB = KV<KVT>::EB;
    const int tg = lane >> 2, dg = lane & 3;
    const int t = min(base + lane, cap - 1);
#pragma unroll
    for (int i = 0; i < KV<KVT>::KW; ++i)
        R.k[i] = gload16(kc + (hb + (size_t)t * D) * EB + 16 * i);
    R.ks = KVT == VLRF_HIP_KV_Q8_0 ? *(gfloat*)(ks + t) : 1.f;
    R.vs = KVT == VLRF_HIP_KV_Q8_0 ? *(gfloat*)(vs + t) : 1.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int tv = min(base + tg + 16 * j, cap - 1);
#pragma unroll
        for (int i = 0; i < KV<KVT>::VW; ++i)
            R.v[j][i] = gload16(vc + (hb + (size_t)tv * D + 16 * dg) * EB + 16 * i);
    }
}

// Element j of the token's stored K or V row: quantized (Q8_0: clamp(round(x
// * inv)) with the row scale sc, zero for an all-zero row, kv_cache.hpp:102-117),
// converted to F16 bits (kv_cache.hpp:68-97) or kept (F32); stored when wr, and
// the value attention reads back returned.
template <int KVT>
__device__ __forceinline__ float store_elem(int8_t* row, int j, float x, float sc, float inv, bool nz, bool wr) {
    if constexpr (KVT == VLRF_HIP_KV_Q8_0) {
        const int c = nz ? min(127, max(-127, (int)roundf(x * inv))) : 0;
        if (wr) row[j] = (int8_t)c;
        return (float)c * sc;
    } else if constexpr (KVT == VLRF_HIP_KV_F16) {
        const uint16_t hb16 = f32_to_f16_kv(x);
        if (wr) reinterpret_cast<uint16_t*>(row)[j] = hb16;
        return f16_bits_to_f32(hb16);
    } else {
        if (wr) reinterpret_cast<float*>(row)[j] = x;
        return x;
    }
}

template <int NW>
struct Smem {
    __align__(16) float qs[D];
    __align__(16) float nk[D];       // the new token's stored row of KV head g, read back
    __align__(16) float nv[D];
    float amax[2 * NW];              // per-wave maxima of the new K and V rows
    __align__(16) float pbuf[NW][64];   // p (times the V row scale) of the wave's round
    float wm[NW], wl[NW];
    __align__(16) float wacc[NW][D];
};

// Inputs of the new token (fused): thread t holds K RoPE pair t (k0, k1) of
// the row's n_kv heads and V elements t and t + 64*NW (vn, vn2), and the RoPE
// table entries (rc, rs) of pair index lane % 32 at the token's position
// (every pair a thread rotates has that index; cos 1, sin 0 when unfused).
struct NewRow {
    float k0 = 0.f, k1 = 0.f, vn = 0.f, vn2 = 0.f;
    float rc = 1.f, rs = 0.f;
};

// The RoPE table entries of nr for the token at pos (rope.hpp:62-69 tables).
__device__ __forceinline__ void rope_row(NewRow& nr, const DecodeFuse& fz, int pos) {
    const int trow = min(pos, fz.max_seq - 1);
    const int j = threadIdx.x & (HALF - 1);
    nr.rc = fz.cos_t[(size_t)trow * HALF + j];
    nr.rs = fz.sin_t[(size_t)trow * HALF + j];
}

// The attention of query head h (KV head g, whose rows start at element hb of
// the cache) over rows [c0, c0 + 64*NW) of a context of ctx rows, for the
// wave's loaded round R.  q0/q1 (wave 0, lane j < 32): q[j], q[j + 32].
// FUSED: pos is the new token's row, rot whether RoPE applies, has_new whether
// the row lies in this block; `writer` (the group's first head) stores head g's
// elements of the row in the cache and `scale_writer` (query head 0) the Q8_0
// row scales.  out(tid, acc, m, l) is called for tid < 64 with the
// unnormalised result.
template <int KVT, bool FUSED, int NW, class Out>
__device__ __forceinline__ void chunk(Smem<NW>& sm, const Round<KVT>& R, float q0, float q1, const NewRow& nr, bool writer,
                                      bool scale_writer, int g, int c0, int cap, size_t hb, int ctx, int pos, bool rot,
                                      bool has_new, float scale, const DecodeFuse& fz, Out&& out) {
    constexpr bool Q8 = KVT == VLRF_HIP_KV_Q8_0;
    constexpr int EB = KV<KVT>::EB, NT = 64 * NW;
    constexpr bool V2 = NT < 512;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int tg = lane >> 2, dg = lane & 3;
    const int npairs = FUSED ? fz.n_kv * HALF : 0, nrow = FUSED ? fz.n_kv * D : 0;
    float k0 = nr.k0, k1 = nr.k1;
    const float rc = nr.rc, rs = nr.rs;

    // ---- q of head h (wave 0) and, fused, the new row's RoPE and maxima -------------
    if (w == 0 && lane < HALF) {
        if (rot) rope2(q0, q1, rc, rs, &sm.qs[lane], &sm.qs[lane + HALF]);
        else { sm.qs[lane] = q0; sm.qs[lane + HALF] = q1; }
    }
    if constexpr (FUSED) {
        // attention.hpp:109-128: RoPE on k, then KVCache::append stores the row
        // before attention reads it back: Q8_0 quantizes the whole row with one
        // scale (kv_cache.hpp:102-117); the row maxima are merged through LDS and
        // the row is quantized after the rounds, off their critical path.
        if (has_new) {
            if (tid < npairs && rot) rope2(k0, k1, rc, rs, &k0, &k1);
            if constexpr (Q8) {
                float ak = wave_max(tid < npairs ? fmaxf(fabsf(k0), fabsf(k1)) : 0.f);
                float av = tid < nrow ? fabsf(nr.vn) : 0.f;
                if (V2 && tid + NT < nrow) av = fmaxf(av, fabsf(nr.vn2));
                av = wave_max(av);
                if (lane == 0) { sm.amax[w] = ak; sm.amax[NW + w] = av; }
            }
        }
    }
    __syncthreads();

    // ---- the wave's round -----------------------------------------------------------
    const int nrounds = (ctx - c0 + 63) / 64;
    float m_run = kNegInf, l_run = 0.f, acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    if (w < nrounds) {
        const int base = c0 + w * 64;
        // scores: lane = token base + lane; the new token (fused) is merged at the end
        const int t = base + lane;
        float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
        for (int i = 0; i < D / 4; ++i) {
            const float4 qv = *reinterpret_cast<const float4*>(&sm.qs[4 * i]);
            const float4 kf = row4<KVT>(R.k, i);
            s0 += qv.x * kf.x;
            s1 += qv.y * kf.y;
            s2 += qv.z * kf.z;
            s3 += qv.w * kf.w;
        }
        const bool live = t < ctx && t != pos;
        const float sc = live ? ((s0 + s1) + (s2 + s3)) * R.ks * scale : kNegInf;
        const float mx = fmaxf(m_run, wave_max(sc));
        const float corr = m_run == kNegInf ? 0.f : expf(m_run - mx);
        const float pe = live ? expf(sc - mx) : 0.f;
        l_run = l_run * corr + wave_sum(pe);
        m_run = mx;
        sm.pbuf[w][lane] = pe * R.vs;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // P.V: lane (tg, dg) over tokens tg + 16j of the round, dims 16dg..16dg+15
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] *= corr;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float pp = sm.pbuf[w][tg + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v4 = row4<KVT>(R.v[j], i);
                acc[4 * i] += pp * v4.x;
                acc[4 * i + 1] += pp * v4.y;
                acc[4 * i + 2] += pp * v4.z;
                acc[4 * i + 3] += pp * v4.w;
            }
        }
        __builtin_amdgcn_wave_barrier();
    }

    // ---- fused: quantize and store the new row; the merge reads it back from LDS -----
    // (F16 converts each element, kv_cache.hpp:68-97; F32 copies.)  The group's
    // first head stores head g's elements, never past the cache.
    if (FUSED && has_new) {
        float ak = 0.f, av = 0.f, sk = 1.f, sv = 1.f, ik = 0.f, iv = 0.f;
        if constexpr (Q8) {
#pragma unroll
            for (int k = 0; k < NW; ++k) {
                ak = fmaxf(ak, sm.amax[k]);
                av = fmaxf(av, sm.amax[NW + k]);
            }
            sk = ak != 0.f ? ak / 127.f : 0.f;
            sv = av != 0.f ? av / 127.f : 0.f;
            ik = ak != 0.f ? 1.f / sk : 0.f;
            iv = av != 0.f ? 1.f / sv : 0.f;
        }
        const bool wr = writer && pos < cap;
        int8_t* krow = fz.kq_w + (hb + (size_t)pos * D) * EB;
        int8_t* vrow = fz.vq_w + (hb + (size_t)pos * D) * EB;
        auto put = [&](int8_t* row, int j, float x, float sc, float inv, bool nz) -> float {
            return store_elem<KVT>(row, j, x, sc, inv, nz, wr);
        };
        if (tid < npairs && tid / HALF == g) {
            const int j = tid % HALF;
            sm.nk[j] = put(krow, j, k0, sk, ik, ak != 0.f);
            sm.nk[j + HALF] = put(krow, j + HALF, k1, sk, ik, ak != 0.f);
        }
        if (tid < nrow && tid / D == g) sm.nv[tid % D] = put(vrow, tid % D, nr.vn, sv, iv, av != 0.f);
        if (V2 && tid + NT < nrow && (tid + NT) / D == g)
            sm.nv[(tid + NT) % D] = put(vrow, (tid + NT) % D, nr.vn2, sv, iv, av != 0.f);
        if constexpr (Q8) {
            if (scale_writer && tid == 0 && pos < cap) { fz.ks_w[pos] = sk; fz.vs_w[pos] = sv; }
        }
    }

    // ---- merge: lanes of a dim group, then the waves -------------------------------
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        // sum over the 16 lanes tg of dim group dg: rotations by 4 and 8 within a
        // 16-lane row (DPP row_ror), then the row and half exchanges
        float v = acc[e];
        v += dpp_f<0x124>(v);
        v += dpp_f<0x128>(v);
        float2 t = swap_rows16(v, v);
        v = t.x + t.y;
        t = swap_halves32(v, v);
        acc[e] = t.x + t.y;
    }
    if (tg == 0) {
#pragma unroll
        for (int e = 0; e < 16; ++e) sm.wacc[w][16 * dg + e] = acc[e];
    }
    if (lane == 0) { sm.wm[w] = m_run; sm.wl[w] = l_run; }
    __syncthreads();
    if (tid < D) {
        // The new token (fused): score q . k_stored, weight 1, value its stored V row.
        float sn = kNegInf;
        if (FUSED && has_new) {
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
            for (int i = 0; i < D / 4; ++i) {
                const float4 qv = *reinterpret_cast<const float4*>(&sm.qs[4 * i]);
                const float4 kv = *reinterpret_cast<const float4*>(&sm.nk[4 * i]);
                a0 += qv.x * kv.x;
                a1 += qv.y * kv.y;
                a2 += qv.z * kv.z;
                a3 += qv.w * kv.w;
            }
            sn = ((a0 + a1) + (a2 + a3)) * scale;
        }
        float mt = sn;
#pragma unroll
        for (int k = 0; k < NW; ++k) mt = fmaxf(mt, sm.wm[k]);
        float lt = 0.f, ot = 0.f;
        if (FUSED && has_new) {
            lt = expf(sn - mt);
            ot = lt * sm.nv[tid];
        }
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            if (sm.wm[k] != kNegInf) {
                const float c = expf(sm.wm[k] - mt);
                lt += c * sm.wl[k];
                ot += c * sm.wacc[k][tid];
            }
        }
        out(tid, ot, mt, lt);
    }
}


// ---- one chunk without the token's row (the fused QKV + attention launch) ----------
// The attention of query head h over the cache rows [c0, min(c0 + 64*NW, pos))
// for the wave's loaded round R: every row before the token, none of it (the
// token's key is merged as its own partial).  The head's rotated q is in
// sm.qs (stage_q, before a workgroup barrier).
//
// Arranged for latency: the chunk's maximum score is formed first (one more
// barrier), so every wave exponentiates against it and the waves' P.V sums
// merge by plain addition, with no rescaling and no exponentials in the merge.
// Q8_0 codes are converted with one sign-extending byte-select conversion
// each, to the same values as the signed extraction.  (Converting them as
// unsigned bytes and taking the bias out afterwards, as the M = 1 GEMV does,
// loses bits to cancellation here: measured 4e-5 to 8e-5 against 1e-6 on the
// logits.)  out(tid, acc, m, l) for tid < 64: the unnormalised partial.
template <int NW>
struct SmemQ {
    __align__(16) float qs[D];
    float wmax[NW], wl[NW];
    __align__(16) float pbuf[NW][64];
    __align__(16) float wacc[NW][D];
};

// q of the head into sm.qs, rotated (lanes j < 32 of one wave: q[j], q[j + 32]
// before RoPE; rc, rs the table entries of pair j).  The caller's next
// workgroup barrier publishes it to chunk_q.
template <int NW>
__device__ __forceinline__ void stage_q(SmemQ<NW>& sm, float q0, float q1, float rc, float rs, bool rot) {
    const int lane = threadIdx.x & 63;
    float y0 = q0, y1 = q1;
    if (rot) rope2(q0, q1, rc, rs, &y0, &y1);
    if (lane < HALF) { sm.qs[lane] = y0; sm.qs[lane + HALF] = y1; }
}

template <int KVT, int NW, class Out>
__device__ __forceinline__ void chunk_q(SmemQ<NW>& sm, const Round<KVT>& R, int c0, int pos, float scale, Out&& out) {
    static_assert(KVT == VLRF_HIP_KV_Q8_0 || KVT == VLRF_HIP_KV_F16, "Q8_0 / F16 caches");
    constexpr bool Q8 = KVT == VLRF_HIP_KV_Q8_0;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int tg = lane >> 2, dg = lane & 3;

    // scores: lane = row c0 + 64w + lane (rows from pos on are masked)
    const int t = c0 + w * 64 + lane;
    const bool live = t < pos;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
    for (int i = 0; i < D / 4; ++i) {
        const float4 qv = *reinterpret_cast<const float4*>(&sm.qs[4 * i]);
        float4 kf;
        if constexpr (Q8) {
            const uint4 kw = R.k[i >> 2];
            kf = s8f4((i & 3) == 0 ? kw.x : (i & 3) == 1 ? kw.y : (i & 3) == 2 ? kw.z : kw.w);
        } else {
            kf = row4<KVT>(R.k, i);
        }
        s0 += qv.x * kf.x;
        s1 += qv.y * kf.y;
        s2 += qv.z * kf.z;
        s3 += qv.w * kf.w;
    }
    const float sc = live ? ((s0 + s1) + (s2 + s3)) * R.ks * scale : kNegInf;
    const float wm = wave_max(sc);
    if (lane == 0) sm.wmax[w] = wm;
    __syncthreads();
    float M = sm.wmax[0];
#pragma unroll
    for (int k = 1; k < NW; ++k) M = fmaxf(M, sm.wmax[k]);
    const float pe = live ? __expf(sc - M) : 0.f;   // hardware exp (~1 ulp), on the chunk's serial path
    const float lw = wave_sum(pe);
    sm.pbuf[w][lane] = pe * R.vs;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // P.V: lane (tg, dg) over rows tg + 16j of the wave, dims 16dg..16dg+15
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float pp = sm.pbuf[w][tg + 16 * j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float4 v4;
            if constexpr (Q8) {
                const uint4 vw = R.v[j][0];
                v4 = s8f4(i == 0 ? vw.x : i == 1 ? vw.y : i == 2 ? vw.z : vw.w);
            } else {
                v4 = row4<KVT>(R.v[j], i);
            }
            acc[4 * i] += pp * v4.x;
            acc[4 * i + 1] += pp * v4.y;
            acc[4 * i + 2] += pp * v4.z;
            acc[4 * i + 3] += pp * v4.w;
        }
    }
    // Sum over the 16 lanes tg of dim group dg as a reduce-scatter: each
    // exchange halves the values a lane holds, so 15 exchanges replace 64.
    // Lane bits (t3 t2 | t1 t0 d1 d0), tg = t3t2t1t0: rows of 16 lanes differ
    // in t3t2.  (1) rows t2=0/1 swap halves of acc (permlane16): lanes keep
    // dims 8*t2 + [0,8); (2) halves t3=0/1 (permlane32): 4*t3 + [0,4); (3)
    // lanes t1=0/1, 8 apart in a row (DPP rotate by 8): 2*t1 + [0,2); (4)
    // lanes t0=0/1, 4 apart (rotate by 4 one way, 12 the other): t0.  The lane
    // then holds dim 16*dg + 8*t2 + 4*t3 + 2*t1 + t0, summed over tg.
    {
        const int t0 = tg & 1, t1 = (tg >> 1) & 1, t2 = (tg >> 2) & 1, t3 = tg >> 3;
        float v1[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float2 x = swap_rows16(acc[e], acc[e + 8]);
            v1[e] = x.x + x.y;
        }
        float v2[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float2 x = swap_halves32(v1[e], v1[e + 4]);
            v2[e] = x.x + x.y;
        }
        float v3[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float own = t1 ? v2[e + 2] : v2[e];
            const float send = t1 ? v2[e] : v2[e + 2];
            v3[e] = own + dpp_f<0x128>(send);
        }
        const float own = t0 ? v3[1] : v3[0];
        const float send = t0 ? v3[0] : v3[1];
        // row_ror:N reads lane (p - N) mod 16: rotate by 12 reaches p + 4, by 4
        // p - 4.  Both rotations run on every lane and a bit mask picks one: a
        // rotation left to a branch would run with its source lanes switched
        // off and read zeros.
        const float g4 = dpp_f<0x124>(send), g12 = dpp_f<0x12C>(send);
        const int pick = -t0;
        const float got = __int_as_float((__float_as_int(g4) & pick) | (__float_as_int(g12) & ~pick));
        sm.wacc[w][16 * dg + 8 * t2 + 4 * t3 + 2 * t1 + t0] = own + got;
    }
    if (lane == 0) sm.wl[w] = lw;
    __syncthreads();
    if (tid < D) {
        float ot = 0.f, lt = 0.f;
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            ot += sm.wacc[k][tid];
            lt += sm.wl[k];
        }
        out(tid, ot, M, lt);
    }
}

// ---- d_head 128: one chunk without the token's row --------------------------------
// The 8B-shape heads (d_head 128, Q8_0 cache) in the arrangement of chunk_q:
// wave w scores rows c0 + 64w + lane (lane = token, its 128 codes in eight
// 16-byte words), every wave exponentiates against the chunk's common
// maximum, and P.V runs with lane (tg, dg) = (lane / 8, lane % 8) owning dims
// 16dg..16dg+15 over rows tg + 8j (j < 8).  The 8 lanes tg of a dim group are
// summed by a reduce-scatter (lane bits: dg = bits 0-2, tg = bits 3-5):
// permlane16 pairs bit 4, permlane32 bit 5, a DPP rotation by 8 bit 3, so each
// lane ends with two dims, 16*dg + 8*t1 + 4*t2 + 2*t0 + {0, 1}.
constexpr int D128 = 128, HALF128 = 64;

struct Round128 {
    uint4 k[8];        // token base + lane: codes 16i..16i+15
    uint4 v[8];        // token base + tg + 8j: codes 16dg..16dg+15
    float ks, vs;      // row scales of token base + lane
};

__device__ __forceinline__ void load_round128(Round128& R, const int8_t* kc, const int8_t* vc, const float* ks,
                                              const float* vs, size_t hb, int base, int cap, int lane) {
    const int tg = lane >> 3, dg = lane & 7;
    const int t = min(base + lane, cap - 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) R.k[i] = gload16(kc + hb + (size_t)t * D128 + 16 * i);
    R.ks = *(gfloat*)(ks + t);
    R.vs = *(gfloat*)(vs + t);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int tv = min(base + tg + 8 * j, cap - 1);
        R.v[j] = gload16(vc + hb + (size_t)tv * D128 + 16 * dg);
    }
}

template <int NW>
struct SmemQ128 {
    __align__(16) float qs[D128];
    float wmax[NW], wl[NW];
    __align__(16) float pbuf[NW][64];
    __align__(16) float wacc[NW][D128];
};

// q0/q1 (wave 0, lane j): q[j], q[j + 64] before RoPE (rc, rs: the table
// entries of pair j).  out(tid, acc, m, l) for tid < 128: the unnormalised
// partial over rows [c0, min(c0 + 64*NW, pos)).
template <int NW, class Out>
__device__ __forceinline__ void chunk_q128(SmemQ128<NW>& sm, const Round128& R, float q0, float q1, float rc,
                                           float rs, bool rot, int c0, int pos, float scale, Out&& out) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int tg = lane >> 3, dg = lane & 7;
    if (w == 0) {
        float y0 = q0, y1 = q1;
        if (rot) rope2(q0, q1, rc, rs, &y0, &y1);
        sm.qs[lane] = y0;
        sm.qs[lane + HALF128] = y1;
    }
    __syncthreads();

    const int t = c0 + w * 64 + lane;
    const bool live = t < pos;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
    for (int i = 0; i < D128 / 4; ++i) {
        const float4 qv = *reinterpret_cast<const float4*>(&sm.qs[4 * i]);
        const uint4 kw = R.k[i >> 2];
        const float4 kf = s8f4((i & 3) == 0 ? kw.x : (i & 3) == 1 ? kw.y : (i & 3) == 2 ? kw.z : kw.w);
        s0 += qv.x * kf.x;
        s1 += qv.y * kf.y;
        s2 += qv.z * kf.z;
        s3 += qv.w * kf.w;
    }
    const float sc = live ? ((s0 + s1) + (s2 + s3)) * R.ks * scale : kNegInf;
    const float wm = wave_max(sc);
    if (lane == 0) sm.wmax[w] = wm;
    __syncthreads();
    float M = sm.wmax[0];
#pragma unroll
    for (int k = 1; k < NW; ++k) M = fmaxf(M, sm.wmax[k]);
    const float pe = live ? __expf(sc - M) : 0.f;   // hardware exp (~1 ulp), on the chunk's serial path
    const float lw = wave_sum(pe);
    sm.pbuf[w][lane] = pe * R.vs;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float pp = sm.pbuf[w][tg + 8 * j];
        const uint4 vw = R.v[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v4 = s8f4(i == 0 ? vw.x : i == 1 ? vw.y : i == 2 ? vw.z : vw.w);
            acc[4 * i] += pp * v4.x;
            acc[4 * i + 1] += pp * v4.y;
            acc[4 * i + 2] += pp * v4.z;
            acc[4 * i + 3] += pp * v4.w;
        }
    }
    {
        const int t0 = tg & 1, t1 = (tg >> 1) & 1, t2 = tg >> 2;
        float v1[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {   // rows differing in bit 4 (t1): dims 8*t1 + [0, 8)
            const float2 x = swap_rows16(acc[e], acc[e + 8]);
            v1[e] = x.x + x.y;
        }
        float v2[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {   // halves (bit 5, t2): 4*t2 + [0, 4)
            const float2 x = swap_halves32(v1[e], v1[e + 4]);
            v2[e] = x.x + x.y;
        }
        float v3[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {   // lanes 8 apart in a row (bit 3, t0): 2*t0 + [0, 2)
            const float own = t0 ? v2[e + 2] : v2[e];
            const float send = t0 ? v2[e] : v2[e + 2];
            v3[e] = own + dpp_f<0x128>(send);
        }
        const int d = 16 * dg + 8 * t1 + 4 * t2 + 2 * t0;
        sm.wacc[w][d] = v3[0];
        sm.wacc[w][d + 1] = v3[1];
    }
    if (lane == 0) sm.wl[w] = lw;
    __syncthreads();
    if (tid < D128) {
        float ot = 0.f, lt = 0.f;
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            ot += sm.wacc[k][tid];
            lt += sm.wl[k];
        }
        out(tid, ot, M, lt);
    }
}

}  // namespace attn
}  // namespace vlrf_hip
