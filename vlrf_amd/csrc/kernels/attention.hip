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
// Decode design (gfx950): split-K over the context.  A 512-lane workgroup owns
// one KV head and a 64-token chunk, so each K/V byte is loaded and dequantized
// once per workgroup and reused by all REP query heads of the GQA group.
// Scores: lane t of every wave holds the K row of token c0+t and scores it
// against REP/8 query heads over the full head dimension (LDS broadcast reads
// of q); the softmax max and sum are wave reductions (DPP + shuffles), so no
// workgroup-level reduction is needed.  P.V: the chunk's V rows are staged
// dequantized in LDS and each thread accumulates its own (head, dim) outputs
// over the 64 tokens.  Two workgroup barriers in all.  Partials
// (m, l, acc[d]) per (head, chunk) are merged by a combine kernel with the
// log-sum-exp rescale.  With a device-side position the kernel also applies
// RoPE to q and to the new k and quantizes + stores the new K/V row before
// attending (the decode step's fused form).
//
// The decode step itself (d_head 64, caches of 513..8192 rows) runs the
// single-pass kernel below in chunked form instead: one query head and one
// 512-row chunk per workgroup, a (m, l, acc) partial per chunk, merged by the
// O projection's GEMV prologue, so the step has no combine launch; caches of
// at most 512 rows take the single pass over the whole context.  The
// stand-alone calls (vlrf_hip_attn_decode, vlrf_hip_attn_f32 at T = 1) at
// d_head 64 run attn_decode_chunks_kernel: the same chunk code on 64..512-row
// chunks, merged in the same launch by each head's last workgroup; the
// split-K kernel and its combine serve d_head 128 and longer contexts.
#include "../internal.hpp"
#include "attn_core.hpp"

#include <cmath>
#include <cstdlib>

namespace vlrf_hip {
namespace {

constexpr int kChunk = 64;        // tokens per split-K workgroup
constexpr int kAttnThreads = 512;  // lanes per decode-attention workgroup (8 waves)
constexpr int kMaxSplits = 512;   // contexts up to 32768 tokens
constexpr float kNegInf = -INFINITY;

using attn::rope2;

// KVT: cache element type VLRF_HIP_KV_Q8_0 (int8 codes, f32 scale per token row),
// VLRF_HIP_KV_F16 (the reference's f16 bits) or VLRF_HIP_KV_F32; kc/vc address the
// elements ([n_kv][head_stride/D][D]) as bytes.
template <int D, int REP, int KVT, bool FUSED>
__global__ __launch_bounds__(kAttnThreads) void attn_decode_partial_kernel(
    const float* __restrict__ q, const int8_t* kc, const int8_t* vc, const float* ks, const float* vs,
    long head_stride, int ctx_len, const int* __restrict__ ctx_dev, int n_splits, float scale,
    float* __restrict__ part, DecodeFuse fz) {
    constexpr bool Q8 = KVT == VLRF_HIP_KV_Q8_0, H16 = KVT == VLRF_HIP_KV_F16;
    constexpr int EB = Q8 ? 1 : H16 ? 2 : 4;             // bytes per cache element
    constexpr int HALF = D / 2;
    static_assert(HALF == 32 || HALF == 64, "a RoPE pair index is tid % HALF only for HALF | 64");
    constexpr int NT = kAttnThreads, NW = NT / 64;
    constexpr int HPW = REP >= NW ? REP / NW : 1;        // query heads scored per wave
    constexpr int KW = D * EB / 16;                      // 16-byte words of one K row
    constexpr int EPW = 16 / EB;                         // elements per 16-byte word
    constexpr int VE = kChunk * D / NT;                  // V elements staged per thread
    constexpr int VD = VE * EB / 4;                      // their dwords
    static_assert(VD % 2 == 0 && VD <= 16, "V staging granularity");
    __shared__ __align__(16) float qs[REP][D];
    __shared__ __align__(16) float vsm[kChunk][D];       // the chunk's dequantized V rows
    __shared__ __align__(16) float pr[REP][kChunk];      // softmax numerators
    __shared__ float mstat[REP], lstat[REP];
    __shared__ __align__(16) float newk[FUSED ? D : 1];
    __shared__ float amax[FUSED ? 2 * NW : 1];          // per-wave maxima of the new K and V rows

    const int split = blockIdx.x, g = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cap = (int)(head_stride / D);       // cache rows
    const int c0 = split * kChunk;
    const size_t hb = (size_t)g * head_stride;

    // Vector loads complete in issue order, so the small L2-resident operands
    // (queries, the new K/V row) are requested first, then the cache stream,
    // and every load is branch-free (rows are clamped into the cache and
    // masked where they are used): a load in a branch, or a value converted
    // right after its load, would make the wave wait for the whole stream early.
    constexpr int PAIRS = REP * HALF, PPT = (PAIRS + NT - 1) / NT;
    float qlo[PPT], qhi[PPT];
#pragma unroll
    for (int p = 0; p < PPT; ++p) {
        const int i = min(tid + NT * p, PAIRS - 1), h = i / HALF, j = i - h * HALF;
        const float* qh = q + (size_t)(g * REP + h) * D;
        qlo[p] = qh[j];
        qhi[p] = qh[j + HALF];
    }
    // Fused decode: the new token's row spread over the workgroup (rows of at
    // most 1024 elements): thread t holds K RoPE pair t and V elements t, t + NT.
    float nk0 = 0.f, nk1 = 0.f, nv0 = 0.f, nv1 = 0.f;
    if constexpr (FUSED) {
        const int npairs = fz.n_kv * HALF, nrow = fz.n_kv * D;
        const int i = min(tid, npairs - 1), h = i / HALF, j = i - h * HALF;
        nk0 = fz.k_new[h * D + j];
        nk1 = fz.k_new[h * D + j + HALF];
        nv0 = fz.v_new[min(tid, nrow - 1)];
        nv1 = fz.v_new[min(tid + NT, nrow - 1)];
    }
    // The cache stream, kept as raw codes: lane l of every wave reads the whole
    // K row of token c0+l (the waves' repeats are L1 hits); thread t stages
    // VE elements of the V row of token c0 + t*VE/D.
    const int jt = min(c0 + lane, cap - 1);
    uint4 kraw[KW];
#pragma unroll
    for (int i = 0; i < KW; ++i)
        kraw[i] = *reinterpret_cast<const uint4*>(kc + (hb + (size_t)jt * D) * EB + 16 * i);
    const float ksc = Q8 ? ks[jt] : 1.f;
    const int tv = tid / (D / VE), pv = tid % (D / VE);
    const int jv = min(c0 + tv, cap - 1);
    uint2 vraw[VD / 2];
#pragma unroll
    for (int i = 0; i < VD / 2; ++i)
        vraw[i] = *reinterpret_cast<const uint2*>(vc + (hb + (size_t)jv * D + pv * VE) * EB + 8 * i);
    const float vsc = Q8 ? vs[jv] : 1.f;

    // The device position is read only now: none of the addresses above depend
    // on it, so its latency overlaps the cache stream.
    const int dpos = (FUSED || ctx_dev) ? *ctx_dev : 0;   // fused: always a device position
    int ctx = FUSED ? dpos + 1 : (ctx_dev ? dpos + ctx_len : ctx_len);   // FUSED: dpos = tokens before this one
    // Rows past the cache capacity are never read, even if the device-side
    // position were corrupt (the host checks capacity before queuing).
    ctx = min(ctx, cap);
    const int pos = FUSED ? dpos : -1;
    float* pout = part + (size_t)(g * REP) * n_splits * (D + 2) + (size_t)split * (D + 2);
    if (c0 >= ctx) {   // chunk past the context: empty partial
        for (int i = tid; i < REP * (D + 2); i += NT) {
            const int h = i / (D + 2), dd = i % (D + 2);
            pout[(size_t)h * n_splits * (D + 2) + dd] = dd == D ? kNegInf : 0.f;
        }
        return;
    }
    const int nt = min(kChunk, ctx - c0);       // valid tokens of the chunk
    const bool has_new = FUSED && pos >= c0 && pos < c0 + kChunk;
    const bool rot = FUSED && pos < fz.max_seq;   // rope.hpp:84: positions >= max_seq stay unrotated
    // Every RoPE pair this thread rotates (q pairs tid + NT*p, and for wave 0
    // the new k pairs lane + 64p) has pair index tid % HALF, so one table entry
    // per thread serves them all.
    float rc = 1.f, rs = 0.f;
    if constexpr (FUSED) {
        const int trow = min(pos, fz.max_seq - 1);   // used only when rot
        rc = fz.cos_t[(size_t)trow * HALF + (tid & (HALF - 1))];
        rs = fz.sin_t[(size_t)trow * HALF + (tid & (HALF - 1))];
    }

    // ---- queries of the GQA group (RoPE at the device position when fused) -------
#pragma unroll
    for (int p = 0; p < PPT; ++p) {
        const int i = tid + NT * p;
        if (i < PAIRS) {
            const int h = i / HALF, j = i - h * HALF;
            if (rot) rope2(qlo[p], qhi[p], rc, rs, &qs[h][j], &qs[h][j + HALF]);
            else { qs[h][j] = qlo[p]; qs[h][j + HALF] = qhi[p]; }
        }
    }

    // ---- V chunk into LDS as f32 (dequantize_row_q8_0 / f16_to_f32); rows past
    // the context are zero, and the new token's row is written by wave 0 below.
    if (!(has_new && c0 + tv == pos)) {
        float* dst = &vsm[tv][pv * VE];
        const bool live = c0 + tv < ctx;
#pragma unroll
        for (int i = 0; i < VD / 2; ++i) {
            const uint32_t w[2] = {vraw[i].x, vraw[i].y};
            if constexpr (Q8) {
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    float4 o;
                    o.x = live ? (float)(int8_t)(w[k]) * vsc : 0.f;
                    o.y = live ? (float)(int8_t)(w[k] >> 8) * vsc : 0.f;
                    o.z = live ? (float)(int8_t)(w[k] >> 16) * vsc : 0.f;
                    o.w = live ? (float)(int8_t)(w[k] >> 24) * vsc : 0.f;
                    *reinterpret_cast<float4*>(dst + 8 * i + 4 * k) = o;
                }
            } else if constexpr (H16) {
                float4 o;
                o.x = live ? f16_bits_to_f32(w[0] & 0xFFFFu) : 0.f;
                o.y = live ? f16_bits_to_f32(w[0] >> 16) : 0.f;
                o.z = live ? f16_bits_to_f32(w[1] & 0xFFFFu) : 0.f;
                o.w = live ? f16_bits_to_f32(w[1] >> 16) : 0.f;
                *reinterpret_cast<float4*>(dst + 4 * i) = o;
            } else {
                float2 o;
                o.x = live ? __uint_as_float(w[0]) : 0.f;
                o.y = live ? __uint_as_float(w[1]) : 0.f;
                *reinterpret_cast<float2*>(dst + 2 * i) = o;
            }
        }
    }

    // ---- decode fusion: the current token's K/V row (the chunk holding it)
    // attention.hpp:109-128: RoPE on k, then KVCache::append stores the row
    // before attention reads it: Q8_0 quantizes the whole row (quantize_row_q8_0,
    // kv_cache.hpp:102-117), F16 converts each element (f32_to_f16, :68-97), F32
    // copies.  Every chunk holding `pos` converts the row itself and uses the
    // stored values for that token; the workgroup of KV head g stores head g's
    // elements, KV head 0 the Q8_0 row scales.  The whole workgroup shares the
    // work (one pair and up to two V elements per thread): the row maxima are
    // wave reductions merged through LDS at the barrier below, so the chain
    // before the scores is a few dozen instructions long.
    const int npairs = FUSED ? fz.n_kv * HALF : 0, nrow = FUSED ? fz.n_kv * D : 0;
    if constexpr (FUSED) {
        if (has_new) {
            if (tid < npairs && rot) rope2(nk0, nk1, rc, rs, &nk0, &nk1);
            if constexpr (Q8) {
                float ak = tid < npairs ? fmaxf(fabsf(nk0), fabsf(nk1)) : 0.f;
                float av = tid < nrow ? fabsf(nv0) : 0.f;
                if (tid + NT < nrow) av = fmaxf(av, fabsf(nv1));
                ak = wave_max(ak);
                av = wave_max(av);
                if (lane == 0) { amax[wave] = ak; amax[NW + wave] = av; }
            }
        }
    }
    __syncthreads();
    // The row's stored form stays in registers and is written to the cache at
    // the end of the kernel: one counter covers vector loads and stores, so a
    // store issued here would make the later waits for the cache stream wait
    // for the store as well.
    uint32_t kb0 = 0, kb1 = 0, vb0 = 0, vb1 = 0;
    float sk = 1.f, sv = 1.f;
    if constexpr (FUSED) {
        if (has_new) {
            float ak = 0.f, av = 0.f, ik = 0.f, iv = 0.f;
            if constexpr (Q8) {
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    ak = fmaxf(ak, amax[w]);
                    av = fmaxf(av, amax[NW + w]);
                }
                sk = ak != 0.f ? ak / 127.f : 0.f;
                sv = av != 0.f ? av / 127.f : 0.f;
                ik = ak != 0.f ? 1.f / sk : 0.f;
                iv = av != 0.f ? 1.f / sv : 0.f;
            }
            float* vnew = vsm[pos - c0];
            // the stored bits of one element; *back = the value attention reads back
            auto enc = [&](float x, float sc, float inv, bool nz, float* back) -> uint32_t {
                if constexpr (Q8) {
                    const int c = nz ? min(127, max(-127, (int)roundf(x * inv))) : 0;
                    *back = (float)c * sc;
                    return (uint32_t)c;
                } else if constexpr (H16) {
                    const uint16_t hb16 = f32_to_f16_kv(x);
                    *back = f16_bits_to_f32(hb16);
                    return hb16;
                } else {
                    *back = x;
                    return __float_as_uint(x);
                }
            };
            if (tid < npairs && tid / HALF == g) {
                const int j = tid % HALF;
                kb0 = enc(nk0, sk, ik, ak != 0.f, &newk[j]);
                kb1 = enc(nk1, sk, ik, ak != 0.f, &newk[j + HALF]);
            }
            if (tid < nrow && tid / D == g) vb0 = enc(nv0, sv, iv, av != 0.f, &vnew[tid % D]);
            if (tid + NT < nrow && (tid + NT) / D == g) vb1 = enc(nv1, sv, iv, av != 0.f, &vnew[(tid + NT) % D]);
            __syncthreads();   // the stored K row, before the scores read it
        }
    }

    // ---- scores and softmax: lane = token, HPW heads per wave, full d_head ------
    // One wave per SIMD leaves no other wave to hide LDS latency, so each
    // head's q row is read in one batch and the dot products use four
    // independent accumulators.  Codes are converted once; the row scale is
    // applied to the finished dot (exact integers times q, then one scale).
    {
        const bool live = lane < nt;
        float kv[D];
        float kscale = ksc;
#pragma unroll
        for (int i = 0; i < KW; ++i) {
            const uint32_t w[4] = {kraw[i].x, kraw[i].y, kraw[i].z, kraw[i].w};
            if constexpr (Q8) {
#pragma unroll
                for (int k = 0; k < 16; ++k) kv[16 * i + k] = (float)(int8_t)(w[k >> 2] >> (8 * (k & 3)));
            } else if constexpr (H16) {
#pragma unroll
                for (int k = 0; k < 8; ++k) kv[8 * i + k] = f16_bits_to_f32((w[k >> 1] >> (16 * (k & 1))) & 0xFFFFu);
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) kv[4 * i + k] = __uint_as_float(w[k]);
            }
        }
        if constexpr (FUSED) {
            if (has_new && c0 + lane == pos) {     // the new token: its stored row, as read back
#pragma unroll
                for (int j = 0; j < D; ++j) kv[j] = newk[j];
                kscale = 1.f;
            }
        }
#pragma unroll
        for (int hh = 0; hh < HPW; ++hh) {
            const int h = wave * HPW + hh;
            if (h < REP) {
                float4 qv[D / 4];
#pragma unroll
                for (int i = 0; i < D / 4; ++i) qv[i] = *reinterpret_cast<const float4*>(&qs[h][4 * i]);
                float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
                for (int i = 0; i < D / 4; ++i) {
                    s0 += qv[i].x * kv[4 * i];
                    s1 += qv[i].y * kv[4 * i + 1];
                    s2 += qv[i].z * kv[4 * i + 2];
                    s3 += qv[i].w * kv[4 * i + 3];
                }
                const float sdot = ((s0 + s1) + (s2 + s3)) * kscale;
                const float sc = live ? sdot * scale : kNegInf;
                const float mx = wave_max(sc);   // finite: token c0 < ctx is in this chunk
                const float pe = live ? expf(sc - mx) : 0.f;
                const float sum = wave_sum(pe);
                pr[h][lane] = pe;
                if (lane == 0) { mstat[h] = mx; lstat[h] = sum; }
            }
        }
    }
    __syncthreads();

    // ---- P.V: thread = (head, dim), over the chunk's tokens from LDS -------------
    // LDS reads in batches of 16 tokens, two accumulators per output.
    for (int i = tid; i < REP * D; i += NT) {
        const int h = i / D, d = i - h * D;
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int t0 = 0; t0 < kChunk; t0 += 16) {
            float4 pp[4];
            float vv[16];
#pragma unroll
            for (int k = 0; k < 4; ++k) pp[k] = *reinterpret_cast<const float4*>(&pr[h][t0 + 4 * k]);
#pragma unroll
            for (int k = 0; k < 16; ++k) vv[k] = vsm[t0 + k][d];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                a += pp[k].x * vv[4 * k] + pp[k].y * vv[4 * k + 1];
                b += pp[k].z * vv[4 * k + 2] + pp[k].w * vv[4 * k + 3];
            }
        }
        pout[(size_t)h * n_splits * (D + 2) + d] = a + b;
    }
    if (tid < REP) {
        pout[(size_t)tid * n_splits * (D + 2) + D] = mstat[tid];
        pout[(size_t)tid * n_splits * (D + 2) + D + 1] = lstat[tid];
    }
    // ---- fused: the new row into the cache (head g's elements; KV head 0 the scales)
    if constexpr (FUSED) {
        if (has_new) {
            int8_t* krow_w = fz.kq_w + (hb + (size_t)pos * D) * EB;
            int8_t* vrow_w = fz.vq_w + (hb + (size_t)pos * D) * EB;
            auto st = [&](int8_t* row, int j, uint32_t b) {
                if constexpr (Q8) row[j] = (int8_t)b;
                else if constexpr (H16) reinterpret_cast<uint16_t*>(row)[j] = (uint16_t)b;
                else reinterpret_cast<uint32_t*>(row)[j] = b;
            };
            if (tid < npairs && tid / HALF == g) {
                st(krow_w, tid % HALF, kb0);
                st(krow_w, tid % HALF + HALF, kb1);
            }
            if (tid < nrow && tid / D == g) st(vrow_w, tid % D, vb0);
            if (tid + NT < nrow && (tid + NT) / D == g) st(vrow_w, (tid + NT) % D, vb1);
            if constexpr (Q8) {
                if (g == 0 && tid == 0) { fz.ks_w[pos] = sk; fz.vs_w[pos] = sv; }
            }
        }
    }
}

// ---- single-pass decode over a short cache (d_head 64, <= 512 rows) -------------
// One 512-lane workgroup per query head and no split partials: the combine
// kernel's launch and its round trip through memory disappear.
// Wave w takes the 64-token rounds r*8 + w; in a round lane t scores token
// (r*8 + w)*64 + t against q (from LDS), the wave keeps its own online
// softmax (m, l) with wave reductions, and accumulates P.V with lane
// (tg, dg) = (lane/4, lane%4) owning dims 16dg..16dg+15 over tokens tg + 16j,
// reading the V elements as 16-element row pieces (each load a contiguous run)
// and the Q8_0 row scales folded into p.  Each wave loads its one round up
// front (attn::load_round, attn::chunk).  At the end the 16 lanes of a dim
// group are summed with xor shuffles and the waves' (m, l, acc) are merged in
// LDS with the log-sum-exp rule.  The fused
// form rotates and stores the new token's row in every workgroup (identical
// results; the group's first head writes it), leaves the token at `pos` out
// of the rounds (its cache row may not be written yet) and adds it to the
// final merge as one more entry: score q.k_stored, weight 1, value the stored
// V row.  KVT: VLRF_HIP_KV_Q8_0 codes + row scales, VLRF_HIP_KV_F16 bits, VLRF_HIP_KV_F32.
// Measured on the MI355X (32q/4kv Q8_0, d 64, stream launches): single pass
// 5.8 / 7.0 / 8.6 / 11.9 us at ctx 64 / 512 / 1024 / 2048 against 6.9 / 7.7 /
// 7.8 / 8.1 us for split-K + combine.  One workgroup's memory parallelism caps
// the single pass beyond a few hundred tokens, so it takes caches of up to 512
// rows.
constexpr int kSPWaves = 8, kSPRounds = 1, kSPDepth = 1;   // rounds per wave, rounds in flight
constexpr int kSPMaxCtx = kSPWaves * 64 * kSPRounds;   // cache rows the single pass covers
// Chunked form (CH tokens per workgroup, one query head each): partials of
// kChunkStride floats -- acc[0..63] (unnormalised), m at 64, l at 65 --
// merged by the next GEMV's prologue.
constexpr int kChunksMaxCtx = 8192;   // the one-launch chunked form: at most 16 chunks of 512 rows
constexpr int kCH = 512, kChunkStride = kAttnChunkStride;   // 256 / 1024: 0.645 / 0.673 ms per step against 0.620

// CH > 0 (fused decode only): the same algorithm on one CH-token chunk of the
// cache per workgroup, NW = CH/64 waves of one round, for query head h of
// chunk s; the result is the chunk's partial (m, l, acc) at out[h][s][*]
// (kChunkStride floats), the new token merged only by the chunk holding it.
template <int KVT, int REP, bool FUSED, int CH = 0>
__global__ __launch_bounds__(CH ? CH : 64 * kSPWaves) void attn_decode_single_kernel(
    const float* __restrict__ q, const int8_t* kc, const int8_t* vc, const float* ks, const float* vs,
    long head_stride, int ctx_len, const int* __restrict__ ctx_dev, float scale, float* __restrict__ out,
    DecodeFuse fz, int nch) {
    static_assert(CH == 0 || (FUSED && CH % 64 == 0), "chunks: fused decode, whole rounds");
    static_assert(kSPRounds == 1 && kSPDepth == 1, "attn::chunk runs one round per wave");
    constexpr int D = attn::D, HALF = attn::HALF, NW = CH ? CH / 64 : kSPWaves;
    __shared__ attn::Smem<NW> sm;

    int h, g, c0 = 0, chunk = 0;
    if constexpr (CH > 0) {
        // The REP query heads of chunk (g, s) run on one XCD (workgroup b on XCD
        // b % 8), so the chunk's K/V rows come from HBM once and then from that
        // L2; placement only affects speed.
        const int b = blockIdx.x, k = b >> 3, r = k % REP, pc = (b & 7) + 8 * (k / REP);
        if (pc >= fz.n_kv * nch) return;
        g = pc / nch;
        chunk = pc - g * nch;
        h = g * REP + r;
        c0 = chunk * CH;
    } else {
        h = blockIdx.x;
        g = h / REP;
    }
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int cap = (int)(head_stride / D);
    const size_t hb = (size_t)g * head_stride;

    // Loads first, all branch-free with rows clamped into the cache (masked at use):
    // q, the new row (fused), the round's K/V, and only then the device position.
    float q0 = 0.f, q1 = 0.f;
    if (w == 0) {
        const int j = lane & (HALF - 1);
        q0 = q[(size_t)h * D + j];
        q1 = q[(size_t)h * D + j + HALF];
    }
    // The new row (fused; n_kv <= 8, so at most 512 elements): thread t holds K
    // RoPE pair t and V elements t and (with 256 threads) t + NT.
    constexpr int NT = 64 * NW;
    attn::NewRow nr;
    if constexpr (FUSED) {
        const int npairs = fz.n_kv * HALF, nrow = fz.n_kv * D;
        const int i = min(tid, npairs - 1), hh = i / HALF, j = i - hh * HALF;
        nr.k0 = fz.k_new[hh * D + j];
        nr.k1 = fz.k_new[hh * D + j + HALF];
        nr.vn = fz.v_new[min(tid, nrow - 1)];
        if constexpr (NT < 512) nr.vn2 = fz.v_new[min(tid + NT, nrow - 1)];
    }
    attn::Round<KVT> R;
    attn::load_round<KVT>(R, kc, vc, ks, vs, hb, c0 + w * 64, cap, lane);
    // Every K/V load is issued before the device position's load and the wait on
    // it (the RoPE table rows depend on it): left to the scheduler, that wait
    // lands between the K and the V loads.
    __builtin_amdgcn_sched_barrier(0);

    const int dpos = (FUSED || ctx_dev) ? *ctx_dev : 0;   // fused: always a device position
    int ctx = FUSED ? dpos + 1 : (ctx_dev ? dpos + ctx_len : ctx_len);
    ctx = min(ctx, cap);
    const int pos = FUSED ? dpos : -1;
    const bool rot = FUSED && pos < fz.max_seq;      // rope.hpp:84: positions >= max_seq stay unrotated
    const bool has_new = FUSED && (CH == 0 || (pos >= c0 && pos < c0 + CH));
    if constexpr (FUSED) attn::rope_row(nr, fz, pos);
    // A chunk past the context takes no early exit: it runs no round and the merge
    // writes its empty partial (acc 0, m -inf, l 0).  An exit on the device
    // position here lets the compiler sink the K/V loads below that position's
    // load, adding its round trip to every workgroup.
    attn::chunk<KVT, FUSED, NW>(sm, R, q0, q1, nr, h % REP == 0, h == 0, g, c0, cap, hb, ctx, pos, rot, has_new, scale, fz,
                                [&](int t, float ot, float mt, float lt) {
                                    if constexpr (CH > 0) {   // the chunk's partial, unnormalised
                                        float* pp = out + ((size_t)h * nch + chunk) * kChunkStride;
                                        pp[t] = ot;
                                        if (t == 0) { pp[D] = mt; pp[D + 1] = lt; }
                                    } else {
                                        out[(size_t)h * D + t] = lt > 0.f ? ot * (1.f / lt) : 0.f;
                                    }
                                });
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

// ---- prefill: causal attention of T new tokens on the matrix cores ------------
// Reference: AttentionBlock::forward with T > 1 (attention.hpp:89-186): the new
// K/V rows are quantized into the cache first (N6 order), then each query row
// attends the dequantized cache rows kpos <= qpos (attention.hpp:232,253-261)
// with scale 1/sqrt(d_h); flash_attn_head's online softmax (attention.hpp:207-309).
//
// Design: a workgroup = one KV head g and 8/REP blocks of 32 consecutive query
// tokens, 8 waves; wave w serves query head g*REP + w%REP on query block w/REP,
// so each K/V tile (64 keys, dequantized to bf16 in LDS, V transposed) is
// shared by the REP heads of the GQA group and 256/REP queries.  Each thread
// stages 16 elements of one key; the next tile's elements are loaded into
// registers before the current tile is computed, so their latency hides
// behind the matrix work.  A wave skips tiles that lie wholly past its last
// query (it still joins the barriers).  The wave
// computes S^T = K.Q^T and O^T = V^T.P^T with v_mfma_f32_32x32x16_bf16: in that
// orientation lane l owns query l%32 (both lane halves), so the softmax max and
// sum are one cross-half exchange (v_permlane32_swap), the rescale multiplies
// the lane's own accumulators, and P re-enters the second product through the
// same register exchange.
constexpr int kPQ = 32, kPK = 64;         // queries per wave, keys per tile
constexpr float kLazy = 8.f;              // log2 headroom of the prefill softmax's reference max

// Raw cache elements of one staging item (16 consecutive elements of one key
// row, K and V) held in registers between their load and the LDS store.
template <int KVT>
struct RawKV {
    static constexpr int W = KVT == VLRF_HIP_KV_Q8_0 ? 1 : KVT == VLRF_HIP_KV_F16 ? 2 : 4;   // uint4 per 16 elements
    uint4 k[W], v[W];
    float sk, sv;
};

template <int KVT>
__device__ __forceinline__ void load_raw(RawKV<KVT>& r, const int8_t* kq, const int8_t* vq, const float* ks,
                                         const float* vs, size_t e0, int row) {
    constexpr int EB = RawKV<KVT>::W;                 // bytes per element = uint4 per 16 elements
#pragma unroll
    for (int i = 0; i < RawKV<KVT>::W; ++i) {
        r.k[i] = *reinterpret_cast<const uint4*>(kq + e0 * EB + 16 * i);
        r.v[i] = *reinterpret_cast<const uint4*>(vq + e0 * EB + 16 * i);
    }
    if constexpr (KVT == VLRF_HIP_KV_Q8_0) {
        r.sk = ks[row];
        r.sv = vs[row];
    }
}

// The 16 elements -> f32 (Q8_0 codes times the row scale, f16 widened); zero where !live.
template <int KVT>
__device__ __forceinline__ void raw_f32(const uint4 (&w)[RawKV<KVT>::W], float scale, bool live, float (&o)[16]) {
    if constexpr (KVT == VLRF_HIP_KV_Q8_0) {
        const uint32_t u[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
#pragma unroll
        for (int e = 0; e < 16; ++e) o[e] = (float)(int8_t)(u[e >> 2] >> (8 * (e & 3))) * (live ? scale : 0.f);
    } else if constexpr (KVT == VLRF_HIP_KV_F16) {
        const uint32_t u[8] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w};
#pragma unroll
        for (int e = 0; e < 16; ++e) o[e] = live ? f16_bits_to_f32((u[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) : 0.f;
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            o[4 * k] = live ? __uint_as_float(w[k].x) : 0.f;
            o[4 * k + 1] = live ? __uint_as_float(w[k].y) : 0.f;
            o[4 * k + 2] = live ? __uint_as_float(w[k].z) : 0.f;
            o[4 * k + 3] = live ? __uint_as_float(w[k].w) : 0.f;
        }
    }
}

__device__ __forceinline__ float2 half_swap(float a, float b) { return swap_halves32(a, b); }

// Column (key) of V^T row d in LDS: groups of 8 keys XOR-swizzled by the row's
// 16-dim block, so the 8 stagers of one key (8 blocks of 16 dims) hit distinct
// banks, while every 8-key run an MFMA operand reads stays contiguous.
__device__ __forceinline__ int vt_col(int d, int key) { return key ^ (8 * ((d >> 4) & 7)); }

template <int D, int REP, int KVT>
__global__ __launch_bounds__(512) void attn_prefill_kernel(
    const float* __restrict__ qkv, int ld, const int8_t* __restrict__ kq, const int8_t* __restrict__ vq,
    const float* __restrict__ ks, const float* __restrict__ vs, long head_stride, int T, int pos0,
    float scale, int n_heads, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    uint16_t* __restrict__ out) {
    typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
    typedef float f32x16 __attribute__((ext_vector_type(16)));
    constexpr int NT = 512, NQB = 8 / REP;           // waves: REP heads x NQB query blocks
    constexpr int KS = D + 8, VS = kPK + 8;          // padded LDS row strides (bf16)
    constexpr int ITEMS = kPK * (D / 16);            // staging items of 16 elements per tile
    static_assert(ITEMS <= NT, "one staging item per thread");
    // Double-buffered: tile kt + 1 is staged into the other buffer as soon as
    // a thread has finished computing tile kt, so one barrier per tile.
    __shared__ __align__(16) __bf16 Ks2[2][kPK * KS];   // K tile [key][d]
    __shared__ __align__(16) __bf16 Vt2[2][D * VS];     // V tile transposed [d][vt_col(d, key)]

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, hh = lane >> 5, lq = lane & 31;
    const int g = blockIdx.y, h = g * REP + w % REP;
    // Query blocks of 32 in zig-zag order 0, n-1, 1, n-2, ...: the workgroup's
    // NQB consecutive entries pair early (short) and late (long) causal rows,
    // so every workgroup holds about the same number of wave-tiles.
    const int nblk = (T + kPQ - 1) / kPQ;
    auto zigzag = [nblk](int i) { return (i & 1) ? nblk - 1 - (i >> 1) : i >> 1; };
    int qlast = 0;                                   // the workgroup's last query position
#pragma unroll
    for (int j = 0; j < NQB; ++j) {
        const int i = blockIdx.x * NQB + j;
        if (i < nblk) qlast = max(qlast, pos0 + min(kPQ * zigzag(i) + kPQ, T) - 1);
    }
    const int iw = blockIdx.x * NQB + w / REP;
    const int q0 = iw < nblk ? kPQ * zigzag(iw) : T; // this wave's first query (T: no block)
    const int qi = min(q0 + lq, T - 1);              // clamped: rows past T are not stored
    const int qpos = pos0 + qi;
    const size_t hb = (size_t)g * head_stride;
    const int wave_last = pos0 + min(q0 + kPQ, T) - 1;   // this wave's last query position (q0 < T)

    bf16x8 qf[D / 16];                               // B operand: query lq, dims 16kk + 8hh + e
    {
        // The lane's dims j and j + D/2 (groups kk and kk + D/32) are a RoPE
        // pair (rope.hpp:90-96): the query is rotated here, on load, at its
        // position pos0 + qi, by the same separately rounded products as the
        // per-row RoPE.
        const float* qr = qkv + (size_t)qi * ld + (size_t)h * D;
        float xv[D / 16][8];
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
            const float4 a = *reinterpret_cast<const float4*>(qr + 16 * kk + 8 * hh);
            const float4 b = *reinterpret_cast<const float4*>(qr + 16 * kk + 8 * hh + 4);
            xv[kk][0] = a.x; xv[kk][1] = a.y; xv[kk][2] = a.z; xv[kk][3] = a.w;
            xv[kk][4] = b.x; xv[kk][5] = b.y; xv[kk][6] = b.z; xv[kk][7] = b.w;
        }
        {
            const float* ct = cos_t + (size_t)(pos0 + qi) * (D / 2);
            const float* st = sin_t + (size_t)(pos0 + qi) * (D / 2);
#pragma unroll
            for (int kk = 0; kk < D / 32; ++kk) {
                const float4 c0 = *reinterpret_cast<const float4*>(ct + 16 * kk + 8 * hh);
                const float4 c1 = *reinterpret_cast<const float4*>(ct + 16 * kk + 8 * hh + 4);
                const float4 s0 = *reinterpret_cast<const float4*>(st + 16 * kk + 8 * hh);
                const float4 s1 = *reinterpret_cast<const float4*>(st + 16 * kk + 8 * hh + 4);
                const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
                const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    attn::rope2(xv[kk][e], xv[kk + D / 32][e], cv[e], sv[e], &xv[kk][e], &xv[kk + D / 32][e]);
            }
        }
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk)
            qf[kk] = bf16x8{(__bf16)xv[kk][0], (__bf16)xv[kk][1], (__bf16)xv[kk][2], (__bf16)xv[kk][3],
                            (__bf16)xv[kk][4], (__bf16)xv[kk][5], (__bf16)xv[kk][6], (__bf16)xv[kk][7]};
    }
    f32x16 o[D / 32];
#pragma unroll
    for (int c = 0; c < D / 32; ++c) o[c] = f32x16{};
    float m_run = kNegInf, l_run = 0.f;              // running max (base-2 scaled) and sum
    const float sl2 = scale * 1.4426950408889634f;   // scale * log2(e)

    const int kv_end = pos0 + T;                             // cache rows written
    const int ntile = qlast / kPK + 1;
    // Staging item of this thread: key it / (D/16), dims 16 * (it % (D/16)) .. +15.
    const int it = threadIdx.x, skey = it / (D / 16), spart = it % (D / 16);
    const bool stager = it < ITEMS;
    RawKV<KVT> raw;
    auto fetch = [&](int kt) {                       // tile kt's elements into registers
        const int kp = kt * kPK + skey, kr = kp < kv_end ? kp : 0;
        load_raw<KVT>(raw, kq, vq, ks, vs, hb + (size_t)kr * D + 16 * spart, kr);
    };
    // Registers (tile kt) -> LDS buffer buf as bf16 (rows past kv_end zero).
    auto stage = [&](int kt, int buf) {
        __bf16* Ks = Ks2[buf];
        __bf16* Vt = Vt2[buf];
        const int kv0 = kt * kPK;
        if (stager) {
            const bool live = kv0 + skey < kv_end;
            float kf[16], vf[16];                    // dequantize_row_q8_0 / f16_to_f32
            raw_f32<KVT>(raw.k, KVT == VLRF_HIP_KV_Q8_0 ? raw.sk : 1.f, live, kf);
            raw_f32<KVT>(raw.v, KVT == VLRF_HIP_KV_Q8_0 ? raw.sv : 1.f, live, vf);
            bf16x8 k0, k1;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                k0[e] = (__bf16)kf[e];
                k1[e] = (__bf16)kf[8 + e];
            }
            *reinterpret_cast<bf16x8*>(&Ks[skey * KS + 16 * spart]) = k0;
            *reinterpret_cast<bf16x8*>(&Ks[skey * KS + 16 * spart + 8]) = k1;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int d = 16 * spart + e;
                Vt[d * VS + vt_col(d, skey)] = (__bf16)vf[e];
            }
        }
    };
    if (stager) fetch(0);
    stage(0, 0);
    if (stager && ntile > 1) fetch(1);
    __syncthreads();
    for (int kt = 0; kt < ntile; ++kt) {
        const int kv0 = kt * kPK;
        const __bf16* Ks = Ks2[kt & 1];
        const __bf16* Vt = Vt2[kt & 1];
        if (q0 < T && kv0 <= wave_last) {            // tiles wholly past this wave's queries: nothing to do
            // S^T = K . Q^T for the two 32-key blocks of the tile.
            f32x16 sc[2] = {f32x16{}, f32x16{}};
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int kk = 0; kk < D / 16; ++kk) {
                    const bf16x8 a = *reinterpret_cast<const bf16x8*>(&Ks[(32 * kb + lq) * KS + 16 * kk + 8 * hh]);
                    sc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], sc[kb], 0, 0, 0);
                }
            // Causal mask (key r(v) = 8(v/4) + 4hh + v%4 of the block), only on
            // tiles that cross the wave's diagonal.
            if (kv0 + kPK - 1 > pos0 + q0) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int kp = kv0 + 32 * kb + 8 * (v >> 2) + 4 * hh + (v & 3);
                        if (kp > qpos) sc[kb][v] = kNegInf;
                    }
            }
            // Online softmax in base 2: exp(s*scale - m) = 2^(s*scale*log2(e) - m'),
            // the max taken on raw scores (scale > 0); masked scores give 2^-inf = 0.
            // The reference point m_run moves only when a tile's max passes it by
            // more than kLazy (so p <= 2^kLazy, exact in f32 and bf16 range): the
            // rescale of l and O by 2^(m_old - m_new) is then rare, and skipped
            // by the whole wave when no lane moved (the result is the same ratio).
            float mx = kNegInf;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sc[kb][v]);
            {
                const float2 t = half_swap(mx, mx);    // [lo, lo], [hi, hi]
                mx = fmaxf(t.x, t.y);
            }
            const float mt = mx * sl2;
            const bool grow = mt > m_run + kLazy;    // always on the first tile (key 0 is in it)
            const float mn = grow ? mt : m_run;
            const float corr = grow ? __builtin_amdgcn_exp2f(m_run - mn) : 1.f;   // 0 on the first tile
            float sum = 0.f;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(sc[kb][v], sl2, -mn));
                    sc[kb][v] = p;
                    sum += p;
                }
            {
                const float2 t = half_swap(sum, sum);
                sum = t.x + t.y;                         // lo + hi in both halves
            }
            l_run = l_run * corr + sum;
            m_run = mn;
            if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
                for (int c = 0; c < D / 32; ++c)
#pragma unroll
                    for (int v = 0; v < 16; ++v) o[c][v] *= corr;
            }

            // O^T += V^T . P^T, 16 keys per step.  The B operand of lane (hh, q)
            // needs keys 16s + 8hh + e: v-group 2s+hh, elements 0..3 from lane
            // half 0 and 4..7 from half 1.  One half-swap of (group 2s, group
            // 2s+1) delivers exactly that in both halves: [A_lo, B_lo] gives
            // elements 0..3, [A_hi, B_hi] elements 4..7.
#pragma unroll
            for (int kk2 = 0; kk2 < kPK / 16; ++kk2) {
                const int kb = kk2 >> 1, s2 = kk2 & 1;
                bf16x8 b;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float2 t = half_swap(sc[kb][8 * s2 + e], sc[kb][8 * s2 + 4 + e]);
                    b[e] = (__bf16)t.x;
                    b[4 + e] = (__bf16)t.y;
                }
#pragma unroll
                for (int c = 0; c < D / 32; ++c) {
                    const int d = 32 * c + lq;
                    const bf16x8 a = *reinterpret_cast<const bf16x8*>(&Vt[d * VS + vt_col(d, 16 * kk2 + 8 * hh)]);
                    o[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, o[c], 0, 0, 0);
                }
            }
        }
        if (kt + 1 < ntile) {   // the buffer tile kt - 1 used: every thread passed the last barrier
            stage(kt + 1, (kt + 1) & 1);
            // The tile after next: its loads land while tile kt + 1 is computed.
            if (stager && kt + 2 < ntile) fetch(kt + 2);
        }
        __syncthreads();
    }

    // out[q][h*D + d] = O / l (output acc * (1/l), attention.hpp:300-307), d = 32c + 8(v/4) + 4hh + v%4.
    if (q0 + lq < T) {
        const float inv = 1.f / l_run;
        uint16_t* orow = out + (size_t)(q0 + lq) * n_heads * D + (size_t)h * D;
#pragma unroll
        for (int c = 0; c < D / 32; ++c)
#pragma unroll
            for (int vg = 0; vg < 4; ++vg) {
                uint2 pk;
                pk.x = pack_bf16(o[c][4 * vg] * inv, o[c][4 * vg + 1] * inv);
                pk.y = pack_bf16(o[c][4 * vg + 2] * inv, o[c][4 * vg + 3] * inv);
                *reinterpret_cast<uint2*>(orow + 32 * c + 8 * vg + 4 * hh) = pk;
            }
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

// ---- chunked form at d_head 128 (Q8_0 cache) ---------------------------------------
// The decode step's attention for 8B-shape heads: one workgroup per query
// head and 512-row chunk of the cache (REP heads of a chunk on one XCD, as
// above), each writing the unnormalised partial (acc[0..127], m, l) of the
// rows before the token; one more workgroup (the last) rotates the token's K
// row, quantizes the K and V rows into the cache (kv_cache.hpp:102-117) and
// writes every head's partial of the new key (m = q.k_stored * scale, l = 1,
// acc = v_stored) as partial nch, so the O projection's prologue merges the
// chunks and then the new key: the order of the reference's online softmax
// (attention.hpp:207-309), where the token's key comes last.
constexpr int kChunkStride128 = attn::D128 + 4;

struct NewRow128Smem {
    __align__(16) float nk[8 * attn::D128];   // the stored K / V rows read back
    __align__(16) float nv[8 * attn::D128];
    float amax[2 * (kCH / 64)];
};

__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);   // row_half_mirror
    v += dpp_f<0x140>(v);   // row_mirror
    return v;
}

__device__ void new_row128(const float* __restrict__ q, long head_stride, int pos, int n_heads, float scale,
                           const DecodeFuse& fz, int nch) {
    __shared__ NewRow128Smem sm;
    constexpr int NT = kCH, W = kCH / 64, D = attn::D128, HALF = attn::HALF128;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int G = fz.n_kv, npairs = G * HALF, nrow = G * D, rep = n_heads / G, nparts = nch + 1;
    const int trow = min(pos, fz.max_seq - 1);
    const bool rot = pos < fz.max_seq;   // rope.hpp:84: positions >= max_seq stay unrotated
    // thread t: K pair t (head t / 64, dims j and j + 64), V elements t and t + 512
    const int kp = min(tid, npairs - 1), kh = kp / HALF, kj = kp - kh * HALF;
    float k0 = fz.k_new[kh * D + kj], k1 = fz.k_new[kh * D + kj + HALF];
    const float v0 = fz.v_new[min(tid, nrow - 1)], v1 = fz.v_new[min(tid + NT, nrow - 1)];
    if (tid < npairs && rot)
        attn::rope2(k0, k1, fz.cos_t[(size_t)trow * HALF + kj], fz.sin_t[(size_t)trow * HALF + kj], &k0, &k1);
    const float ak_w = wave_max(tid < npairs ? fmaxf(fabsf(k0), fabsf(k1)) : 0.f);
    float av_l = tid < nrow ? fabsf(v0) : 0.f;
    if (tid + NT < nrow) av_l = fmaxf(av_l, fabsf(v1));
    const float av_w = wave_max(av_l);
    if (lane == 0) { sm.amax[w] = ak_w; sm.amax[W + w] = av_w; }
    __syncthreads();
    float ak = 0.f, av = 0.f;
#pragma unroll
    for (int k = 0; k < W; ++k) {
        ak = fmaxf(ak, sm.amax[k]);
        av = fmaxf(av, sm.amax[W + k]);
    }
    const float sk = ak != 0.f ? ak / 127.f : 0.f, sv = av != 0.f ? av / 127.f : 0.f;
    const float ik = ak != 0.f ? 1.f / sk : 0.f, iv = av != 0.f ? 1.f / sv : 0.f;
    if (tid < npairs) {
        int8_t* krow = fz.kq_w + (size_t)kh * head_stride + (size_t)pos * D;
        sm.nk[kh * D + kj] = attn::store_elem<VLRF_HIP_KV_Q8_0>(krow, kj, k0, sk, ik, ak != 0.f, true);
        sm.nk[kh * D + kj + HALF] = attn::store_elem<VLRF_HIP_KV_Q8_0>(krow, kj + HALF, k1, sk, ik, ak != 0.f, true);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int e = tid + u * NT;
        if (e < nrow) {
            const int vh = e / D, vj = e - vh * D;
            int8_t* vrow = fz.vq_w + (size_t)vh * head_stride + (size_t)pos * D;
            sm.nv[e] = attn::store_elem<VLRF_HIP_KV_Q8_0>(vrow, vj, u ? v1 : v0, sv, iv, av != 0.f, true);
        }
    }
    if (tid == 0) { fz.ks_w[pos] = sk; fz.vs_w[pos] = sv; }
    __syncthreads();
    // Head hh's new-key score: 16 threads a head, 4 RoPE pairs each, summed
    // over the 16-lane row.
    for (int hh0 = 0; hh0 < n_heads; hh0 += NT / 16) {
        const int hh = hh0 + tid / 16, sub = tid & 15;
        const int hq = min(hh, n_heads - 1), g = hq / rep;
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = 4 * sub + i;
            float y0 = q[(size_t)hq * D + j], y1 = q[(size_t)hq * D + j + HALF];
            if (rot)
                attn::rope2(y0, y1, fz.cos_t[(size_t)trow * HALF + j], fz.sin_t[(size_t)trow * HALF + j], &y0, &y1);
            a += y0 * sm.nk[g * D + j] + y1 * sm.nk[g * D + j + HALF];
        }
        a = row16_sum(a);
        if (hh < n_heads && sub == 0) {
            float* pp = fz.chunks + ((size_t)hh * nparts + nch) * kChunkStride128;
            pp[D] = a * scale;
            pp[D + 1] = 1.f;
        }
    }
    for (int e = tid; e < n_heads * D; e += NT) {
        const int hh = e / D, d = e - hh * D;
        fz.chunks[((size_t)hh * nparts + nch) * kChunkStride128 + d] = sm.nv[(hh / rep) * D + d];
    }
}

template <int REP>
__global__ __launch_bounds__(kCH) void attn_chunk128_kernel(const float* __restrict__ q, const int8_t* kc,
                                                            const int8_t* vc, const float* ks, const float* vs,
                                                            long head_stride, const int* __restrict__ pos_dev,
                                                            float scale, DecodeFuse fz, int nch, int na) {
    constexpr int D = attn::D128, HALF = attn::HALF128, NW = kCH / 64;
    const int b = blockIdx.x;
    const int cap = (int)(head_stride / D);
    if (b == na) {
        new_row128(q, head_stride, min(*pos_dev, cap - 1), REP * fz.n_kv, scale, fz, nch);
        return;
    }
    __shared__ attn::SmemQ128<NW> sm;
    const int k = b >> 3, r = k % REP, pc = (b & 7) + 8 * (k / REP);
    if (pc >= fz.n_kv * nch) return;
    const int g = pc / nch, chunk = pc - g * nch, h = g * REP + r, c0 = chunk * kCH;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const size_t hb = (size_t)g * head_stride;
    attn::Round128 R;
    attn::load_round128(R, kc, vc, ks, vs, hb, c0 + w * 64, cap, lane);
    float q0 = 0.f, q1 = 0.f;
    if (w == 0) {
        q0 = q[(size_t)h * D + lane];
        q1 = q[(size_t)h * D + lane + HALF];
    }
    // The K/V loads stay above the device position's load and the exit below.
    __builtin_amdgcn_sched_barrier(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const int pos = min(*pos_dev, cap - 1);   // the host checks capacity before queuing
    float* pp = fz.chunks + ((size_t)h * (nch + 1) + chunk) * kChunkStride128;
    if (c0 >= pos) {   // no cache row before the token: the empty partial (acc 0, m -inf, l 0)
        if (tid < D) pp[tid] = 0.f;
        if (tid == 0) { pp[D] = attn::kNegInf; pp[D + 1] = 0.f; }
        return;
    }
    const int trow = min(pos, fz.max_seq - 1);
    const float rc = fz.cos_t[(size_t)trow * HALF + lane], rs = fz.sin_t[(size_t)trow * HALF + lane];
    attn::chunk_q128<NW>(sm, R, q0, q1, rc, rs, pos < fz.max_seq, c0, pos, scale,
                         [&](int t, float ot, float mt, float lt) {
                             pp[t] = ot;
                             if (t == 0) { pp[D] = mt; pp[D + 1] = lt; }
                         });
}


// ---- stand-alone decode attention in one launch ----------------------------------
// vlrf_hip_attn_decode / attn_f32 at T = 1 (AttentionBlock::flash_attn_head for
// one query row over the cache, attention.hpp:207-309, non-causal): workgroup
// (query head h, chunk c) runs attn::chunk over cache rows [c*CH, c*CH + CH)
// and stores its unnormalised partial (acc[64], m, l; stride D + 2) device-
// coherent; once those stores are acknowledged one thread adds 1 to the head's
// counter (its own 128-byte line in the context's counter array, zero between
// calls).  The workgroup that brings it to nch resets it and merges the head's
// partials in chunk order with the log-sum-exp rule (the same result whichever
// workgroup comes last): out = sum_c e^(m_c - M) acc_c / sum_c e^(m_c - M) l_c.
// nch = ceil(ctx_len / CH) <= kAttnMaxChunks; rows at or past the context are
// masked.  The REP query heads of a chunk run on one XCD (workgroup b on XCD
// b % 8), as in the fused step, so a chunk's K/V rows come from HBM once.
template <int KVT, int REP, int CH>
__global__ __launch_bounds__(CH) void attn_decode_chunks_kernel(
    const float* __restrict__ q, const int8_t* kc, const int8_t* vc, const float* ks, const float* vs,
    long head_stride, int ctx_len, float scale, float* __restrict__ out, float* __restrict__ part,
    int* __restrict__ ctr, int n_kv, int nch) {
    constexpr int D = attn::D, HALF = attn::HALF, NW = CH / 64, PS = D + 2;
    __shared__ attn::Smem<NW> sm;
    __shared__ int last;
    const int b = blockIdx.x, k = b >> 3, r = k % REP, pc = (b & 7) + 8 * (k / REP);
    if (pc >= n_kv * nch) return;   // padding of the grid: no counter, no partial
    const int g = pc / nch, chunk = pc - g * nch, h = g * REP + r, c0 = chunk * CH;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int cap = (int)(head_stride / D);
    const size_t hb = (size_t)g * head_stride;
    float q0 = 0.f, q1 = 0.f;
    if (w == 0) {
        const int j = lane & (HALF - 1);
        q0 = q[(size_t)h * D + j];
        q1 = q[(size_t)h * D + j + HALF];
    }
    attn::Round<KVT> R;
    attn::load_round<KVT>(R, kc, vc, ks, vs, hb, c0 + w * 64, cap, lane);
    const int ctx = min(ctx_len, cap);
    const DecodeFuse fz{};
    const attn::NewRow nr;
    float* pp = part + ((size_t)h * nch + chunk) * PS;
    attn::chunk<KVT, false, NW>(sm, R, q0, q1, nr, false, false, g, c0, cap, hb, ctx, -1, false, false, scale, fz,
                                [&](int t, float ot, float mt, float lt) {
                                    __hip_atomic_store(&pp[t], ot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                    if (t == 0) {
                                        __hip_atomic_store(&pp[D], mt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                        __hip_atomic_store(&pp[D + 1], lt, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT);
                                    }
                                });
    __builtin_amdgcn_s_waitcnt(0x0F70);   // this wave's stores acknowledged (vmcnt 0)
    __syncthreads();
    if (tid == 0) {
        int* c = ctr + (size_t)h * kSmallTileCtrStride;
        last = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nch - 1;
        if (last) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last || tid >= D) return;
    // The merge: lane d of wave 0, every chunk's loads issued before any use.
    const float* ph = part + (size_t)h * nch * PS;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ph), 0, nch * PS * 4,
                                                                        0x00020000);
    float pm[kAttnMaxChunks], pl[kAttnMaxChunks], pa[kAttnMaxChunks];
#pragma unroll
    for (int c = 0; c < kAttnMaxChunks; ++c) {
        const int o = (c < nch ? c : nch - 1) * PS;
        pm[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (o + D) * 4, 0, 16));
        pl[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (o + D + 1) * 4, 0, 16));
        pa[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (o + tid) * 4, 0, 16));
    }
    float M = kNegInf;
#pragma unroll
    for (int c = 0; c < kAttnMaxChunks; ++c)
        if (c < nch) M = fmaxf(M, pm[c]);
    float L = 0.f, O = 0.f;
    if (M != kNegInf) {
#pragma unroll
        for (int c = 0; c < kAttnMaxChunks; ++c)
            if (c < nch && pm[c] != kNegInf) {
                const float wgt = expf(pm[c] - M);
                L += wgt * pl[c];
                O += wgt * pa[c];
            }
    }
    out[(size_t)h * D + tid] = L > 0.f ? O * (1.f / L) : 0.f;
}

}  // namespace

int attn_decode_splits(int max_ctx) { return (max_ctx + kChunk - 1) / kChunk; }

int attn_decode_chunks(int cap, int d_head, int n_kv) {
    const int n = (cap + kCH - 1) / kCH;
    return d_head == 64 && n_kv <= 8 && cap > kSPMaxCtx && n <= kAttnMaxChunks ? n : 0;
}

int attn_decode_chunks128(int cap, int n_heads, int n_kv, int kv_dtype) {
    const int n = (cap + kCH - 1) / kCH;
    const int rep = n_kv > 0 ? n_heads / n_kv : 0;
    return kv_dtype == VLRF_HIP_KV_Q8_0 && n_kv >= 1 && n_kv <= 8 && n_heads % n_kv == 0 &&
                   (rep == 1 || rep == 2 || rep == 4 || rep == 8) && n + 1 <= kAttnMaxChunks
               ? n : 0;
}

int launch_attn_decode(hipStream_t s, const float* q, const void* kc, const void* vc, const float* ks,
                       const float* vs, int kv_dtype, long head_stride, int n_heads, int n_kv, int d_head,
                       int ctx_len, const int* ctx_dev, int n_splits, float scale, float* part, float* out,
                       const DecodeFuse* fuse, int* ctr) {
    VH_ARG(n_kv > 0 && n_heads % n_kv == 0, "attn_decode: n_heads %d not a multiple of n_kv %d",
           n_heads, n_kv);
    const int rep = n_heads / n_kv;
    VH_ARG(d_head == 64 || d_head == 128, "attn_decode: d_head %d not in {64,128}", d_head);
    VH_ARG(rep == 1 || rep == 2 || rep == 4 || rep == 8, "attn_decode: GQA group %d not in {1,2,4,8}", rep);
    VH_ARG(n_splits >= 1 && n_splits <= kMaxSplits, "attn_decode: %d splits outside [1,%d]", n_splits,
           kMaxSplits);
    VH_ARG(kv_dtype == VLRF_HIP_KV_F32 || kv_dtype == VLRF_HIP_KV_F16 || kv_dtype == VLRF_HIP_KV_Q8_0,
           "attn_decode: cache dtype %d", kv_dtype);
    if (!ctx_dev)
        VH_ARG(ctx_len >= 1 && ctx_len <= n_splits * kChunk, "attn_decode: ctx_len %d outside [1,%d]",
               ctx_len, n_splits * kChunk);
    VH_ARG(kc && vc && (kv_dtype != VLRF_HIP_KV_Q8_0 || (ks && vs)), "attn_decode: missing K/V operands");
    DecodeFuse fz{};
    if (fuse) {
        VH_ARG(ctx_dev, "attn_decode: fusion needs a device position");
        VH_ARG(fuse->n_kv == n_kv && n_kv * d_head <= 1024, "attn_decode: bad fusion row");
        fz = *fuse;
    }
    const int8_t* k8 = static_cast<const int8_t*>(kc);
    const int8_t* v8 = static_cast<const int8_t*>(vc);
    if (fuse && fz.nch > 0 && d_head == 128) {
        // d_head 128 chunked form: nch chunk partials and the new key's (nch + 1 per head).
        VH_ARG(fz.chunks && fz.nch == attn_decode_chunks128((int)(head_stride / d_head), n_heads, n_kv, kv_dtype),
               "attn_decode: d_head 128 chunked form for %d chunks does not apply", fz.nch);
        VH_ARG(fz.k_new && fz.v_new && fz.cos_t && fz.sin_t, "attn_decode: d_head 128 chunked form needs the row");
        const int na = 8 * rep * ((n_kv * fz.nch + 7) / 8);
        const dim3 cgrid(na + 1);
#define VH_C128(R)                                                                                              \
    VH_LAUNCH((attn_chunk128_kernel<R>), cgrid, dim3(kCH), 0, s, q, k8, v8, ks, vs, head_stride, ctx_dev,       \
                       scale, fz, fz.nch, na)
        switch (rep) {
            case 1: VH_C128(1); break;
            case 2: VH_C128(2); break;
            case 4: VH_C128(4); break;
            default: VH_C128(8); break;
        }
#undef VH_C128
        VH_LAUNCHED();
        return VLRF_HIP_OK;
    }
    if (fuse && fz.nch > 0) {
        // Chunked form: REP workgroups per (KV head, chunk), grouped by XCD
        // (8 slots per group of 8 chunk indices); partials for the next GEMV.
        VH_ARG(fz.chunks && fz.nch == attn_decode_chunks((int)(head_stride / d_head), d_head, n_kv),
               "attn_decode: chunked form for %d chunks does not apply", fz.nch);
        const dim3 cgrid(8 * rep * ((n_kv * fz.nch + 7) / 8));
#define VH_CHK(KT, R)                                                                                         \
    VH_LAUNCH((attn_decode_single_kernel<KT, R, true, kCH>), cgrid, dim3(kCH), 0, s, q, k8, v8, ks, vs,       \
                       head_stride, ctx_len, ctx_dev, scale, fz.chunks, fz, fz.nch)
#define VH_CHK_R(KT)                     \
    switch (rep) {                       \
        case 1: VH_CHK(KT, 1); break;    \
        case 2: VH_CHK(KT, 2); break;    \
        case 4: VH_CHK(KT, 4); break;    \
        default: VH_CHK(KT, 8); break;   \
    }
        switch (kv_dtype) {
            case VLRF_HIP_KV_Q8_0: VH_CHK_R(VLRF_HIP_KV_Q8_0) break;
            case VLRF_HIP_KV_F16: VH_CHK_R(VLRF_HIP_KV_F16) break;
            default: VH_CHK_R(VLRF_HIP_KV_F32) break;
        }
#undef VH_CHK_R
#undef VH_CHK
        VH_LAUNCHED();
        return VLRF_HIP_OK;
    }
    static const bool chunks_on = [] {
        const char* e = std::getenv("VLRF_HIP_ATTN_CHUNKS");   // "0": the split-K pair of launches instead
        return !(e && e[0] == '0');
    }();
    if (chunks_on && !fuse && ctr && !ctx_dev && d_head == 64 && ctx_len <= kChunksMaxCtx &&
        n_heads <= kSmallMaxTiles) {
        // One launch: the smallest chunk (64..512 rows) that splits the context
        // into at most kAttnMaxChunks chunks; nch <= ceil(ctx_len / 64) = n_splits,
        // so the partials fit the split-K buffer.
        int CHR = 64;
        while ((ctx_len + CHR - 1) / CHR > kAttnMaxChunks) CHR *= 2;
        const int nch = (ctx_len + CHR - 1) / CHR;
        const dim3 cgrid(8 * rep * ((n_kv * nch + 7) / 8));
#define VH_CC(KT, R, C)                                                                                        \
    VH_LAUNCH((attn_decode_chunks_kernel<KT, R, C>), cgrid, dim3(C), 0, s, q, k8, v8, ks, vs, head_stride,     \
              ctx_len, scale, out, part, ctr, n_kv, nch)
#define VH_CC_R(KT, C)                      \
    switch (rep) {                          \
        case 1: VH_CC(KT, 1, C); break;     \
        case 2: VH_CC(KT, 2, C); break;     \
        case 4: VH_CC(KT, 4, C); break;     \
        default: VH_CC(KT, 8, C); break;    \
    }
#define VH_CC_T(C)                                                 \
    switch (kv_dtype) {                                            \
        case VLRF_HIP_KV_Q8_0: VH_CC_R(VLRF_HIP_KV_Q8_0, C) break; \
        case VLRF_HIP_KV_F16: VH_CC_R(VLRF_HIP_KV_F16, C) break;   \
        default: VH_CC_R(VLRF_HIP_KV_F32, C) break;                \
    }
        switch (CHR) {
            case 64: VH_CC_T(64) break;
            case 128: VH_CC_T(128) break;
            case 256: VH_CC_T(256) break;
            default: VH_CC_T(512) break;
        }
#undef VH_CC_T
#undef VH_CC_R
#undef VH_CC
        VH_LAUNCHED();
        return VLRF_HIP_OK;
    }
    if (d_head == 64 && head_stride / d_head <= kSPMaxCtx && (!fuse || n_kv <= 8)) {
#define VH_SP(KT, R, FU)                                                                                     \
    VH_LAUNCH((attn_decode_single_kernel<KT, R, FU>), dim3(n_heads), dim3(64 * kSPWaves), 0, s, q, k8,       \
                       v8, ks, vs, head_stride, ctx_len, ctx_dev, scale, out, fz, 0)
#define VH_SP_R(KT, FU)                       \
    switch (rep) {                            \
        case 1: VH_SP(KT, 1, FU); break;      \
        case 2: VH_SP(KT, 2, FU); break;      \
        case 4: VH_SP(KT, 4, FU); break;      \
        default: VH_SP(KT, 8, FU); break;     \
    }
#define VH_SP_T(FU)                                                 \
    switch (kv_dtype) {                                             \
        case VLRF_HIP_KV_Q8_0: VH_SP_R(VLRF_HIP_KV_Q8_0, FU) break; \
        case VLRF_HIP_KV_F16: VH_SP_R(VLRF_HIP_KV_F16, FU) break;   \
        default: VH_SP_R(VLRF_HIP_KV_F32, FU) break;                \
    }
        if (fuse) { VH_SP_T(true) }
        else { VH_SP_T(false) }
#undef VH_SP_T
#undef VH_SP_R
#undef VH_SP
        VH_LAUNCHED();
        return VLRF_HIP_OK;
    }
    dim3 grid(n_splits, n_kv), block(kAttnThreads);
#define VH_AD(D, R, T, FU)                                                                          \
    VH_LAUNCH((attn_decode_partial_kernel<D, R, T, FU>), grid, block, 0, s, q, k8, v8, ks,          \
                       vs, head_stride, ctx_len, ctx_dev, n_splits, scale, part, fz)
#define VH_AD_R(D, T, FU)                       \
    switch (rep) {                              \
        case 1: VH_AD(D, 1, T, FU); break;      \
        case 2: VH_AD(D, 2, T, FU); break;      \
        case 4: VH_AD(D, 4, T, FU); break;      \
        default: VH_AD(D, 8, T, FU); break;     \
    }
#define VH_AD_T(D, FU)                                                   \
    switch (kv_dtype) {                                                  \
        case VLRF_HIP_KV_Q8_0: VH_AD_R(D, VLRF_HIP_KV_Q8_0, FU) break;   \
        case VLRF_HIP_KV_F16: VH_AD_R(D, VLRF_HIP_KV_F16, FU) break;     \
        default: VH_AD_R(D, VLRF_HIP_KV_F32, FU) break;                  \
    }
    if (d_head == 64) {
        if (fuse) { VH_AD_T(64, true) }
        else { VH_AD_T(64, false) }
    } else {
        if (fuse) { VH_AD_T(128, true) }
        else { VH_AD_T(128, false) }
    }
#undef VH_AD_T
#undef VH_AD_R
#undef VH_AD
    VH_LAUNCHED();
    if (d_head == 64)
        VH_LAUNCH((attn_combine_kernel<64>), dim3(n_heads), dim3(256), 0, s, part, n_splits, out);
    else
        VH_LAUNCH((attn_combine_kernel<128>), dim3(n_heads), dim3(256), 0, s, part, n_splits, out);
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

int launch_attn_prefill(hipStream_t s, const float* qkv, int ld, const KVLayer& L, int T, int pos0,
                        int n_heads, int n_kv, int d_head, int max_seq, float scale, const float* cos_t,
                        const float* sin_t, uint16_t* out) {
    VH_ARG(n_kv > 0 && n_heads % n_kv == 0, "attn_prefill: n_heads %d not a multiple of n_kv %d", n_heads, n_kv);
    const int rep = n_heads / n_kv;
    VH_ARG(d_head == 64 || d_head == 128, "attn_prefill: d_head %d not in {64,128}", d_head);
    VH_ARG(rep == 1 || rep == 2 || rep == 4 || rep == 8, "attn_prefill: GQA group %d not in {1,2,4,8}", rep);
    VH_ARG(T >= 1 && pos0 >= 0 && pos0 + T <= max_seq, "attn_prefill: positions [%d,%d) outside the cache",
           pos0, pos0 + T);
    VH_ARG(ld % 4 == 0, "attn_prefill: row stride %d not a multiple of 4", ld);
    VH_ARG(cos_t && sin_t, "attn_prefill: missing RoPE tables");
    const int nqb = 8 / rep;                        // query blocks of 32 per workgroup (8 waves)
    dim3 grid(((T + kPQ - 1) / kPQ + nqb - 1) / nqb, n_kv);
#define VH_AP(D, R, KT)                                                                                 \
    hipLaunchKernelGGL((attn_prefill_kernel<D, R, KT>), grid, dim3(512), 0, s, qkv, ld, L.k, L.v, L.ks, \
                       L.vs, (long)max_seq * d_head, T, pos0, scale, n_heads, cos_t, sin_t, out)
#define VH_AP_R(D, KT)                      \
    switch (rep) {                          \
        case 1: VH_AP(D, 1, KT); break;     \
        case 2: VH_AP(D, 2, KT); break;     \
        case 4: VH_AP(D, 4, KT); break;     \
        default: VH_AP(D, 8, KT); break;    \
    }
#define VH_AP_T(D)                                                  \
    switch (L.dtype) {                                              \
        case VLRF_HIP_KV_Q8_0: VH_AP_R(D, VLRF_HIP_KV_Q8_0) break;  \
        case VLRF_HIP_KV_F16: VH_AP_R(D, VLRF_HIP_KV_F16) break;    \
        default: VH_AP_R(D, VLRF_HIP_KV_F32) break;                 \
    }
    if (d_head == 64) { VH_AP_T(64) } else { VH_AP_T(128) }
#undef VH_AP_T
#undef VH_AP_R
#undef VH_AP
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

}  // namespace vlrf_hip
