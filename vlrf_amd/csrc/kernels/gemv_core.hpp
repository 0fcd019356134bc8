// gemv_core.hpp - building blocks of the M = 1 dequant GEMV, shared by the
// stand-alone kernel (qlinear.hip) and the fused QKV + attention launch
// (qkv_attn.hip).
//
// Reference contract: compute::linear -> ops::gemm(x, W, y, 1, 0, false, true)
// at M = 1 (include/model/compute.hpp:58-68, ops.hpp:212-252) on weights
// decoded from GGUF Q8_0/Q4_0 blocks (tools/converter/convert_gguf.py:233-263);
// RMSNorm (ops.hpp:488-498) and SwiGLU (ops.hpp:409-441) fused at its edges.
//
// The workgroup (kGemvWaves waves) stages the activation vector (times the
// norm weight when RMSNorm is fused; 1/rms multiplies the finished dots) in
// LDS once, behind a single barrier, in a lane-interleaved layout: the i-th
// float4 of lane l for chunk c sits at [(c*EPL/4 + i)*64 + l], so every
// ds_read_b128 of a wave touches 64 consecutive float4 (no bank conflicts).  A
// wave owns RPW rows (SwiGLU: RPW gate/up row pairs) at a time; lane l covers
// EPL consecutive columns of each chunk of 64*EPL columns, so one 16-byte load
// per lane per chunk streams a contiguous 1 KiB run of a row (Q8_0: 16 codes,
// Q4_0: 32 nibbles).  Codes are loaded nontemporal (streamed once per step)
// and decoded with v_cvt_f32_ubyte*: Q8_0 codes are biased by 128 (xor 0x80),
// Q4_0 nibbles are used as stored, and the bias is removed once per chunk with
// the lane's sum of x (sum (q+b)x - b*sum x = sum qx).
#pragma once

#include "../internal.hpp"

#include <cmath>

namespace vlrf_hip {
namespace gemv {

template <int WT>
struct Gemv;
// EPL: codes per lane and chunk.  Each code becomes an f32 in one instruction:
// Q8_0 codes as signed bytes (s8f); Q4_0 codes n - 8 as (n - 8) / 16 (s4f), so
// their block scales are taken times SCALE = 16 (exact).
template <>
struct Gemv<VLRF_HIP_DT_Q8_0> { static constexpr int EPL = 16; static constexpr float SCALE = 1.f; };
template <>
struct Gemv<VLRF_HIP_DT_Q4_0> { static constexpr int EPL = 32; static constexpr float SCALE = 16.f; };

constexpr float kNegInfF = -INFINITY;
constexpr int kGemvMaxK = 6144;          // staged activations: 24 KiB of LDS
// Plain and residual forms with one row per wave also take the d_ff-wide
// rows of an 8B-shape down projection (56 KiB of LDS, two workgroups a CU).
constexpr int kGemvWideMaxK = 14336;
constexpr int kGemvMaxGroups = 512;      // workgroups of the row loop (2 per CU)
constexpr int kGemvMaxOneGroups = 768;   // one row per wave up to 3 workgroups per CU
constexpr int kGemvWaves = 8;            // waves per workgroup (one staged copy of x)
constexpr int kGemvThreads = 64 * kGemvWaves;

// Signed byte K of a word as f32 in one instruction (SDWA source select with
// sign extension; the compiler otherwise extracts the byte first).
template <int K>
__device__ __forceinline__ float s8f(uint32_t w) {
    float r;
    if constexpr (K == 0)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(w));
    else if constexpr (K == 1)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(w));
    else if constexpr (K == 2)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(w));
    else
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(w));
    return r;
}

// (n - 8) / 16 for the nibble n in bits 0-3 of byte K of w ^ 0x88888888: the
// flipped top bit makes the sign-extended 4-bit value n - 8, and the
// conversion (v_cvt_off_f32_i4, the byte chosen by an SDWA source select)
// divides it by 16.
template <int K>
__device__ __forceinline__ float s4f(uint32_t w) {
    float r;
    if constexpr (K == 0)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(w));
    else if constexpr (K == 1)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(w));
    else if constexpr (K == 2)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(w));
    else
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(w));
    return r;
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
// Global-memory views: a pointer read from a table in memory is otherwise a
// flat pointer, and flat loads also count against the LDS counter.
typedef const __attribute__((address_space(1))) u32x4 gu32x4;
typedef const __attribute__((address_space(1))) uint16_t gu16;

// Activation chunks (NC) of a K-wide row, the float4 slots they stage and the
// float4 each thread stages.
template <int WT, int NC>
struct Shape {
    static constexpr int EPL = Gemv<WT>::EPL;
    static constexpr int CW = 64 * EPL;
    static constexpr int XF4 = NC * CW / 4;
    static constexpr int PER = (XF4 + kGemvThreads - 1) / kGemvThreads;
};

template <int NM, int RPW, int NC>
struct GemvRegs {
    uint4 w[NM][RPW][NC];
    uint32_t s[NM][RPW][NC];      // raw f16 scale bits, converted at use
};

// Branch-free loads: a lane whose (row, chunk) lies outside the matrix reads
// the first 16 bytes and the first scale of the matrix instead (always in
// bounds) and gemv_compute gives it a zero scale.  A load inside a bounds
// branch would be followed by a wait for its result at the end of the branch,
// and since loads return in issue order that wait would serialise the stream.
template <int WT, int NM, int RPW, int NC>
__device__ __forceinline__ void gemv_load(GemvRegs<NM, RPW, NC>& R, const uint8_t* __restrict__ qa,
                                          const __half* __restrict__ da, const uint8_t* __restrict__ qb,
                                          const __half* __restrict__ db, int row0, int N, int K,
                                          int lane) {
    constexpr int EPL = Gemv<WT>::EPL;
    constexpr int CW = 64 * EPL;
    const size_t qrow = WT == VLRF_HIP_DT_Q8_0 ? (size_t)K : (size_t)K / 2;
    const int kb = K / 32;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const uint8_t* q = m ? qb : qa;
        const uint16_t* d = reinterpret_cast<const uint16_t*>(m ? db : da);
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int row = row0 + r;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int e0 = c * CW + lane * EPL;
                const bool in = row < N && e0 < K;
                const size_t qo = in ? (size_t)row * qrow + (size_t)c * 1024 + lane * 16 : 0;
                const size_t so = in ? (size_t)row * kb + e0 / 32 : 0;
                // Streamed once per step: nontemporal, so the codes do not
                // displace the activations and scales from the caches.
                const u32x4 t = __builtin_nontemporal_load((gu32x4*)(q + qo));
                R.w[m][r][c] = make_uint4(t.x, t.y, t.z, t.w);
                R.s[m][r][c] = ((gu16*)d)[so];
            }
        }
    }
}

// The rows' dot products with the staged x; out(row, value) is called by every
// lane of the wave with the finished value of each of its RPW rows (silu(g)*u
// for SwiGLU), 1/rms applied.
template <int WT, int NM, int RPW, int NC, bool SWIGLU, class Out>
__device__ __forceinline__ void gemv_compute(const GemvRegs<NM, RPW, NC>& R, const float4* xs4,
                                             float inv, int row0, int N, int K,
                                             int lane, Out&& out) {
    constexpr int EPL = Gemv<WT>::EPL;
    float acc[NM][RPW];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < RPW; ++r) acc[m][r] = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        float xv[EPL];
#pragma unroll
        for (int i = 0; i < EPL / 4; ++i) {
            const float4 v = xs4[(c * (EPL / 4) + i) * 64 + lane];
            xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const uint32_t u[4] = {R.w[m][r][c].x, R.w[m][r][c].y, R.w[m][r][c].z, R.w[m][r][c].w};
                float p = 0.f;
                if constexpr (WT == VLRF_HIP_DT_Q8_0) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        p += s8f<0>(u[j]) * xv[4 * j];
                        p += s8f<1>(u[j]) * xv[4 * j + 1];
                        p += s8f<2>(u[j]) * xv[4 * j + 2];
                        p += s8f<3>(u[j]) * xv[4 * j + 3];
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        // byte 4j+k holds elements 2(4j+k) (low nibble) and 2(4j+k)+1 (high)
                        const uint32_t w = u[j] ^ 0x88888888u, w4 = w >> 4;
                        p += s4f<0>(w) * xv[8 * j];
                        p += s4f<0>(w4) * xv[8 * j + 1];
                        p += s4f<1>(w) * xv[8 * j + 2];
                        p += s4f<1>(w4) * xv[8 * j + 3];
                        p += s4f<2>(w) * xv[8 * j + 4];
                        p += s4f<2>(w4) * xv[8 * j + 5];
                        p += s4f<3>(w) * xv[8 * j + 6];
                        p += s4f<3>(w4) * xv[8 * j + 7];
                    }
                }
                const bool in = row0 + r < N && c * (64 * EPL) + lane * EPL < K;
                const float sc = in ? __half2float(__ushort_as_half((unsigned short)R.s[m][r][c])) * Gemv<WT>::SCALE : 0.f;
                acc[m][r] = fmaf(sc, p, acc[m][r]);
            }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        float o = wave_sum(acc[0][r]) * inv;
        if constexpr (SWIGLU) {
            const float u = wave_sum(acc[1][r]) * inv;
            // silu(g) * u (ops.hpp:409-441) with the hardware exp and
            // reciprocal (about 1 ulp each): once per row and wave, on the
            // finished dots, where the correctly rounded forms cost ~20
            // instructions
            o = u * (o * __builtin_amdgcn_rcpf(1.f + __expf(-o)));
        }
        out(row0 + r, o);
    }
}

// Decode attention output in its chunked form (head dim 64) merged into the
// thread's x slots: slot p holds elements 4f..4f+3 (f = tid + p*threads) of
// head 4f/64, merged from its nparts chunk partials (pa(p, c): the chunk's
// unnormalised acc for the slot, pml(p, c): its (m, l)) with the log-sum-exp
// rule of the reference's online softmax (attention.hpp:207-309).  NP bounds
// nparts at compile time.
template <int PER, int NP, class PA, class PML>
__device__ __forceinline__ void gemv_merge(PA&& pa, PML&& pml, int nparts, int XF4, int K, int tid,
                                           float4 (&v)[PER]) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int f = tid + p * kGemvThreads;
        const bool in = f < XF4 && 4 * f < K;
        float mt = kNegInfF;
#pragma unroll
        for (int c = 0; c < NP; ++c)
            if (c < nparts) mt = fmaxf(mt, pml(p, c).x);
        float lt = 0.f;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int c = 0; c < NP; ++c) {
            if (c < nparts) {
                const float2 ml = pml(p, c);
                if (ml.x != kNegInfF) {
                    const float4 a = pa(p, c);
                    const float wgt = __expf(ml.x - mt);   // hardware exp (~1 ulp)
                    lt += wgt * ml.y;
                    o.x += wgt * a.x;
                    o.y += wgt * a.y;
                    o.z += wgt * a.z;
                    o.w += wgt * a.w;
                }
            }
        }
        const float il = lt > 0.f ? __builtin_amdgcn_rcpf(lt) : 0.f;   // hardware reciprocal (~1 ulp)
        v[p] = in ? make_float4(o.x * il, o.y * il, o.z * il, o.w * il) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// Stages the thread's x slots v (times the norm weight gw when NORM) in the
// lane-interleaved layout with one barrier: RMSNorm (ops.hpp:488-498) is per
// row, so W.((x*inv)*w) = inv * W.(x*w) and 1/rms (inv) is applied to the
// dots.
template <int WT, int NC, bool NORM>
__device__ __forceinline__ void gemv_stage(const float4 (&v)[Shape<WT, NC>::PER], const float4 (&gw)[Shape<WT, NC>::PER],
                                           float4* xs4, float* red, int K, float eps, float& inv) {
    constexpr int EPL = Gemv<WT>::EPL, CW = Shape<WT, NC>::CW;
    constexpr int XF4 = Shape<WT, NC>::XF4, PER = Shape<WT, NC>::PER;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < PER; ++p)
        ss += v[p].x * v[p].x + v[p].y * v[p].y + v[p].z * v[p].z + v[p].w * v[p].w;
    if constexpr (NORM) {
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
    }
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int f = tid + p * kGemvThreads;
        if (f < XF4) {
            float4 o = v[p];
            if (NORM && 4 * f < K) {
                const float4 g = gw[p];
                o.x = o.x * g.x; o.y = o.y * g.y;
                o.z = o.z * g.z; o.w = o.w * g.w;
            }
            const int e = 4 * f, c = e / CW, r = e - c * CW, l = r / EPL, i = (r - l * EPL) / 4;
            xs4[(c * (EPL / 4) + i) * 64 + l] = o;
        }
    }
    __syncthreads();
    inv = 1.f;
    if constexpr (NORM) {
        ss = 0.f;
#pragma unroll
        for (int w = 0; w < kGemvWaves; ++w) ss += red[w];
        // 1/rms with the hardware reciprocal square root and reciprocal
        // (~1 ulp each; the scale is applied to the finished dots)
        inv = __builtin_amdgcn_rsqf(ss * __builtin_amdgcn_rcpf((float)K) + eps);
    }
}

// The M = 1 GEMV of workgroup blk of nblk: y[row] = W[row] . x for the rows
// of its waves, handed to st(row, value) (lane 0, row < N).
// XM: bit 0 = RMSNorm fused (norm_w), bit 1 = x is row *x_row of a table (with
// the raw row copied to x_copy), bit 2 = residual added (by st).  Compile-time: the
// kernel branches on no argument (measured in the decode step, same box:
// 0.706 -> 0.686 ms/step for the norm and gather bits).
template <int WT, int NC, int RPW, bool SWIGLU, int XM, class Store>
__device__ __forceinline__ void gemv_body(const uint8_t* __restrict__ qa, const __half* __restrict__ da,
                                          const uint8_t* __restrict__ qb, const __half* __restrict__ db, int N,
                                          int K, const float* __restrict__ x, const int* __restrict__ x_row,
                                          float* x_copy, const float* __restrict__ norm_w, float eps, int nparts,
                                          int blk, int nblk, Store&& st) {
    using S = Shape<WT, NC>;
    constexpr int NM = SWIGLU ? 2 : 1;
    constexpr int NT = kGemvThreads;
    // XM & 8: x is decode attention output in its chunked form (head dim HD:
    // 64, or 128 with XM & 32): element e is dim e % HD of head e / HD, merged
    // here from the nparts chunk partials of that head (HD + 4 floats each:
    // acc, m, l; log-sum-exp, attention.hpp:207-309's rule).
    constexpr bool MERGE = XM & 8;
    constexpr int HD = (XM & 32) ? 128 : 64, CS = HD + 4;
    static_assert(HD != 64 || CS == kAttnChunkStride, "partial layout");
    // XM & 16: every wave has at most one row (N <= the grid's row step), so
    // the second register set of the pipeline is neither loaded nor held.
    constexpr bool ONE = XM & 16;
    constexpr int XF4 = S::XF4, PER = S::PER;
    constexpr int NP = MERGE ? kAttnMaxChunks / PER : 1;   // chunks a merge holds in registers
    __shared__ float4 xs4[XF4];
    __shared__ float red[kGemvWaves];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nwaves = nblk * kGemvWaves;
    int row0 = (blk * kGemvWaves + wave) * RPW;
    const int rstep = nwaves * RPW;

    // x_row: x is row *x_row of a table (the embedding gather of the first
    // layer, ops.hpp:615-626); workgroup 0 copies the raw row to x_copy.
    //
    // Vector loads return in issue order, so the activations and the norm
    // weight are requested first: the staging below then overlaps the weight
    // stream instead of waiting behind it.  (Loading each wave's slice of x
    // into registers instead of staging it once per workgroup was measured
    // slower: 16 waves per CU re-reading x and the norm weight cost more L1
    // bandwidth than the two barriers.)
    float inv = 1.f;                                  // 1/rms, applied to the finished dots
    GemvRegs<NM, RPW, NC> A, B;
    {
        constexpr bool NORM = XM & 1, GATHER = XM & 2;
        const float* xs = GATHER ? x + (size_t)(*x_row) * K : x;
        float4 v[PER], gw[PER];
        float4 pa[PER][NP];
        float2 pml[PER][NP];
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int f = tid + p * NT;            // float4 index in x
            const bool in = f < XF4 && 4 * f < K;
            if constexpr (MERGE) {                 // the head's chunk words, before any use (the 16
                                                   // threads of a head share the (m, l) loads in L1)
                const int e = in ? 4 * f : 0;
                const float* ph = x + (size_t)(e / HD) * nparts * CS + (e % HD);
#pragma unroll
                for (int c = 0; c < NP; ++c)
                    if (c < nparts) {
                        pa[p][c] = *reinterpret_cast<const float4*>(ph + (size_t)c * CS);
                        pml[p][c] = *reinterpret_cast<const float2*>(ph - (e % HD) + (size_t)c * CS + HD);
                    }
            } else {
                const float4 t = reinterpret_cast<const float4*>(xs)[in ? f : 0];
                v[p] = in ? t : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        if constexpr (NORM) {
#pragma unroll
            for (int p = 0; p < PER; ++p) {
                const int f = tid + p * NT;
                gw[p] = reinterpret_cast<const float4*>(norm_w)[(f < XF4 && 4 * f < K) ? f : 0];
            }
        }
        // Every wave's activation requests enter the CU's memory pipeline
        // before any weight request, so x is not queued behind the stream.
        __builtin_amdgcn_s_barrier();
        gemv_load<WT, NM, RPW, NC>(A, qa, da, qb, db, row0, N, K, lane);
        if constexpr (!ONE) gemv_load<WT, NM, RPW, NC>(B, qa, da, qb, db, row0 + rstep, N, K, lane);

        if constexpr (MERGE)
            gemv_merge<PER, NP>([&](int p, int c) { return pa[p][c]; }, [&](int p, int c) { return pml[p][c]; },
                                      nparts, XF4, K, tid, v);
        if (GATHER && x_copy && blk == 0) {
#pragma unroll
            for (int p = 0; p < PER; ++p) {
                const int f = tid + p * NT;
                if (f < XF4 && 4 * f < K) reinterpret_cast<float4*>(x_copy)[f] = v[p];
            }
        }
        gemv_stage<WT, NC, NORM>(v, gw, xs4, red, K, eps, inv);
    }

    auto store = [&](int row, float out) {
        if (lane == 0 && row < N) st(row, out);
    };
    if constexpr (ONE) {
        if (row0 < N) gemv_compute<WT, NM, RPW, NC, SWIGLU>(A, xs4, inv, row0, N, K, lane, store);
        return;
    }
    // Loads stay unconditional inside the loop as well (see gemv_load).
    for (; row0 < N; row0 += 2 * rstep) {
        const int r1 = row0 + rstep;
        gemv_compute<WT, NM, RPW, NC, SWIGLU>(A, xs4, inv, row0, N, K, lane, store);
        if (r1 >= N) break;
        const int r2 = r1 + rstep;
        gemv_load<WT, NM, RPW, NC>(A, qa, da, qb, db, r2, N, K, lane);
        gemv_compute<WT, NM, RPW, NC, SWIGLU>(B, xs4, inv, r1, N, K, lane, store);
        if (r2 >= N) break;
        gemv_load<WT, NM, RPW, NC>(B, qa, da, qb, db, r2 + rstep, N, K, lane);
    }
}

}  // namespace gemv
}  // namespace vlrf_hip
