// qlinear.hip - dequant-fused quantized linear y[M,N] = x[M,K] . W[N,K]^T.
//
// Reference contract: compute::linear -> ops::gemm(x, W, y, 1, 0, false, true)
// (include/model/compute.hpp:58-68, ops.hpp:170-310) on weights decoded from
// GGUF Q8_0/Q4_0 blocks (tools/converter/convert_gguf.py:233-263).
//
// Design (gfx950, wave64): a wave owns RPW output rows and walks K in tiles
// of 1024 that the whole workgroup stages in LDS (optionally RMS-normalised on
// the way in).  Within a tile, lane l reads EPL consecutive weights per
// sub-chunk at offset 64*EPL*j + EPL*l, so each weight load instruction of a
// wave covers one contiguous 256/512 B run of the row (coalesced), and the
// matching activation reads from LDS are contiguous across lanes
// (conflict-free).  Weights are dequantized in registers: codes -> f32, a
// per-lane partial dot over the lane's EPL elements, then one FMA with the
// block scale.  The K reduction across lanes is a DPP/shuffle wave sum.
#include "../internal.hpp"
#include "gemv_core.hpp"

namespace vlrf_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kTile = 1024;
constexpr int kRPW = 2;

template <int WT> struct WT_;
template <> struct WT_<VLRF_HIP_DT_Q8_0> { static constexpr int EPL = 4; };
template <> struct WT_<VLRF_HIP_DT_Q4_0> { static constexpr int EPL = 8; };
template <> struct WT_<VLRF_HIP_DT_F32>  { static constexpr int EPL = 4; };

// Partial dot of the lane's EPL weights of row n starting at column c with the
// staged activations xr (EPL floats per activation row, stride kTile).
template <int WT, int MT>
__device__ __forceinline__ void lane_dot(const uint8_t* __restrict__ q, const __half* __restrict__ d,
                                         const float* __restrict__ f, int n, int K, int c,
                                         const float* __restrict__ xr, int M, float (&acc)[MT]) {
    constexpr int EPL = WT_<WT>::EPL;
    float w[EPL];
    float scale = 1.f;
    if constexpr (WT == VLRF_HIP_DT_Q8_0) {
        const uint32_t u = *reinterpret_cast<const uint32_t*>(q + (size_t)n * K + c);
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = (float)(int8_t)(u >> (8 * i));
        scale = __half2float(d[(size_t)n * (K / 32) + c / 32]);
    } else if constexpr (WT == VLRF_HIP_DT_Q4_0) {
        const uint32_t u = *reinterpret_cast<const uint32_t*>(q + (size_t)n * (K / 2) + c / 2);
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = (float)((int)((u >> (4 * i)) & 0xFu) - 8);
        scale = __half2float(d[(size_t)n * (K / 32) + c / 32]);
    } else {
        const float4 v = *reinterpret_cast<const float4*>(f + (size_t)n * K + c);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if (m < M) {
            const float* xm = xr + m * kTile;
            float p = 0.f;
#pragma unroll
            for (int i = 0; i < EPL; i += 4) {
                const float4 xv = *reinterpret_cast<const float4*>(xm + i);
                p += w[i] * xv.x + w[i + 1] * xv.y + w[i + 2] * xv.z + w[i + 3] * xv.w;
            }
            if constexpr (WT == VLRF_HIP_DT_F32) acc[m] += p;
            else acc[m] += scale * p;
        }
    }
}

template <int WT, int MT, bool SWIGLU>
__global__ __launch_bounds__(kThreads) void qlinear_kernel(
    const uint8_t* __restrict__ qa, const __half* __restrict__ da, const float* __restrict__ fa,
    const uint8_t* __restrict__ qb, const __half* __restrict__ db, const float* __restrict__ fb,
    int N, int K, int M, const float* __restrict__ x, const float* __restrict__ norm_w, float eps,
    const float* residual, float* y) {
    constexpr int EPL = WT_<WT>::EPL;
    constexpr int SUB = kTile / (64 * EPL);
    __shared__ __align__(16) float xs[MT * kTile];
    __shared__ float inv_rms[MT];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = (blockIdx.x * kWaves + wave) * kRPW;

    if (norm_w) {
        // ops::rms_norm (ops.hpp:488-498): inv = 1 / sqrt(sum(x^2)/D + eps).
        for (int m = wave; m < M; m += kWaves) {
            float ss = 0.f;
            for (int k = lane; k < K; k += 64) {
                const float v = x[(size_t)m * K + k];
                ss += v * v;
            }
            ss = wave_sum(ss);
            if (lane == 0) inv_rms[m] = 1.f / sqrtf(ss / (float)K + eps);
        }
        __syncthreads();
    }

    float acc[kRPW][MT], accb[kRPW][MT];
#pragma unroll
    for (int r = 0; r < kRPW; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) { acc[r][m] = 0.f; accb[r][m] = 0.f; }

    for (int k0 = 0; k0 < K; k0 += kTile) {
        const int kt = min(kTile, K - k0);
        for (int i = tid; i < MT * kTile; i += kThreads) {
            const int m = i / kTile, kk = i - m * kTile;
            float v = 0.f;
            if (m < M && kk < kt) {
                v = x[(size_t)m * K + k0 + kk];
                if (norm_w) v = v * inv_rms[m] * norm_w[k0 + kk];
            }
            xs[i] = v;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < SUB; ++j) {
            const int e = j * 64 * EPL + lane * EPL;
            if (e < kt) {
#pragma unroll
                for (int r = 0; r < kRPW; ++r) {
                    const int n = row0 + r;
                    if (n < N) {
                        lane_dot<WT, MT>(qa, da, fa, n, K, k0 + e, xs + e, M, acc[r]);
                        if constexpr (SWIGLU) lane_dot<WT, MT>(qb, db, fb, n, K, k0 + e, xs + e, M, accb[r]);
                    }
                }
            }
        }
        __syncthreads();
    }

#pragma unroll
    for (int r = 0; r < kRPW; ++r) {
        const int n = row0 + r;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < M) {
                const float s = wave_sum(acc[r][m]);
                float out = s;
                if constexpr (SWIGLU) {
                    // silu_inplace(g) then multiply_inplace(h, g) (ops.hpp:409-441)
                    const float u = wave_sum(accb[r][m]);
                    const float g = s / (1.f + expf(-s));
                    out = u * g;
                }
                if (lane == 0 && n < N) {
                    if (residual) out = out + residual[(size_t)m * N + n];
                    y[(size_t)m * N + n] = out;
                }
            }
        }
    }
}

template <int WT, bool SWIGLU>
int dispatch_m(hipStream_t s, const DevWeight& a, const DevWeight* b, const float* x, float* y,
               int M, const float* norm_w, float eps, const float* residual) {
    const int rows_per_block = kWaves * kRPW;
    dim3 grid((a.N + rows_per_block - 1) / rows_per_block), block(kThreads);
    const uint8_t* qb = b ? b->q : nullptr;
    const __half* db = b ? b->d : nullptr;
    const float* fb = b ? b->f : nullptr;
#define VH_QL(MT)                                                                           \
    hipLaunchKernelGGL((qlinear_kernel<WT, MT, SWIGLU>), grid, block, 0, s, a.q, a.d, a.f,  \
                       qb, db, fb, a.N, a.K, M, x, norm_w, eps, residual, y)
    if (M == 1) VH_QL(1);
    else if (M <= 4) VH_QL(4);
    else VH_QL(16);
#undef VH_QL
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

// ---- M = 1 decode GEMV (building blocks in gemv_core.hpp) ------------------------
// Waves walk their rows with a two-deep register pipeline: the next rows'
// weights are in flight while the current ones are reduced, and the first
// rows' loads are issued before the activations are staged -- after a barrier
// that puts every wave's activation loads ahead of them, since a CU's vector
// memory requests are served in order.
using gemv::Gemv;
using gemv::GemvRegs;
using gemv::kGemvMaxGroups;
using gemv::kGemvMaxK;
using gemv::kGemvMaxOneGroups;
using gemv::kGemvWaves;

// XM & 64 (argmax form): besides y, the workgroup's largest output and its
// first row go to argp[blockIdx.x] (value, row bits) -- the first level of the
// greedy step's argmax (transformer.hpp:43-47), so the step kernel reduces one
// pair per workgroup instead of every logit.  A wave meets its rows in
// increasing order, so keeping strictly larger values keeps the first maximum.
template <int WT, int NC, int RPW, bool SWIGLU, int XM>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv_kernel(
    const uint8_t* __restrict__ qa, const __half* __restrict__ da, const uint8_t* __restrict__ qb,
    const __half* __restrict__ db, int N, int K, const float* __restrict__ x,
    const int* __restrict__ x_row, float* x_copy, const float* __restrict__ norm_w, float eps,
    const float* residual, float* y, int nparts, float2* argp) {
    constexpr int GM = XM & ~64;   // the GEMV's own form
    float best = -INFINITY;
    int bidx = -1;                 // lane 0 of each wave
    gemv::gemv_body<WT, NC, RPW, SWIGLU, GM>(qa, da, qb, db, N, K, x, x_row, x_copy, norm_w, eps, nparts, blockIdx.x,
                                              gridDim.x, [&](int row, float out) {
                                                  if constexpr ((XM & 4) != 0) out = out + residual[row];
                                                  y[row] = out;
                                                  if constexpr ((XM & 64) != 0)
                                                      if (bidx < 0 || out > best) { best = out; bidx = row; }
                                              });
    if constexpr ((XM & 64) != 0) {
        __shared__ float sb[kGemvWaves];
        __shared__ int si[kGemvWaves];
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        if (lane == 0) { sb[wave] = best; si[wave] = bidx; }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w = 0; w < kGemvWaves; ++w)
                if (si[w] >= 0 && (bidx < 0 || sb[w] > best || (sb[w] == best && si[w] < bidx))) {
                    best = sb[w];
                    bidx = si[w];
                }
            argp[blockIdx.x] = make_float2(best, __int_as_float(bidx));
        }
    }
}

// The wide-row form (K up to kGemvWideMaxK, one row per wave) held to 128
// VGPRs, so that two workgroups share a CU: an 8B-shape down projection's
// 512 workgroups then run in one pass over the 256 CUs.
template <int WT, int NC, int XM>
__global__ __launch_bounds__(64 * kGemvWaves) __attribute__((amdgpu_waves_per_eu(4))) void gemv_wide_kernel(
    const uint8_t* __restrict__ qa, const __half* __restrict__ da, int N, int K, const float* __restrict__ x,
    const float* residual, float* y) {
    gemv::gemv_body<WT, NC, 1, false, XM>(qa, da, nullptr, nullptr, N, K, x, nullptr, nullptr, nullptr, 0.f, 0,
                                          blockIdx.x, gridDim.x, [&](int row, float out) {
                                              if constexpr ((XM & 4) != 0) out = out + residual[row];
                                              y[row] = out;
                                          });
}

template <int WT, bool SWIGLU>
int launch_gemv(hipStream_t s, const DevWeight& a, const DevWeight* b, const float* x, float* y,
                const float* norm_w, float eps, const float* residual, const int* x_row = nullptr,
                float* x_copy = nullptr, int nparts = 0, int head_dim = 64, float2* argp = nullptr) {
    constexpr int CW = 64 * Gemv<WT>::EPL;
    const int nc = (a.K + CW - 1) / CW;
    const uint8_t* qb = b ? b->q : nullptr;
    const __half* db = b ? b->d : nullptr;
    VH_ARG(!x_row || (norm_w && !SWIGLU), "gemv: a gathered row needs the fused norm");
    VH_ARG(!(residual && SWIGLU), "gemv: no residual on the SwiGLU form");
    VH_ARG(!nparts || (!x_row && !norm_w && !SWIGLU && nparts <= kAttnMaxChunks && a.K % 64 == 0),
           "gemv: chunk merge takes a plain x of whole 64-wide heads and at most %d chunks", kAttnMaxChunks);
    const int groups1 = (a.N + kGemvWaves - 1) / kGemvWaves;
    const bool one = groups1 <= kGemvMaxOneGroups;       // RPW 1: one row per wave
    VH_ARG(!argp || (norm_w && !x_row && !residual && !nparts && !one && !SWIGLU),
           "gemv: the argmax form is the normalised LM head's row loop");
    const int xm = (x_row ? 2 : 0) | (norm_w ? 1 : 0) | (residual ? 4 : 0) | (nparts ? 8 : 0) | (one ? 16 : 0) |
                   (nparts && head_dim == 128 ? 32 : 0) | (argp ? 64 : 0);
    VH_ARG(!nparts || head_dim == 64 || (head_dim == 128 && xm == 60 && a.K % 128 == 0),
           "gemv: chunk merge of head dim %d (form %d)", head_dim, xm);
#define VH_GEMV_XM(NC, RPW, XM)                                                                            \
    do {                                                                                                   \
        const int groups = (a.N + kGemvWaves * (RPW)-1) / (kGemvWaves * (RPW));                            \
        dim3 grid(((XM)&16) || groups < kGemvMaxGroups ? groups : kGemvMaxGroups);                         \
        VH_LAUNCH((gemv_kernel<WT, NC, RPW, SWIGLU, XM>), grid, dim3(64 * kGemvWaves), 0, s, a.q, a.d, qb, \
                  db, a.N, a.K, x, x_row, x_copy, norm_w, eps, residual, y, nparts, argp);                 \
    } while (0)
#define VH_GEMV(NC, RPW)                                                  \
    do {                                                                  \
        if (xm == 0) VH_GEMV_XM(NC, RPW, 0);                              \
        else if (xm == 1) VH_GEMV_XM(NC, RPW, 1);                         \
        else if (xm == 65) VH_GEMV_XM(NC, RPW, 65);                       \
        else if (xm == 16) VH_GEMV_XM(NC, RPW, 16);                       \
        else if (xm == 17) VH_GEMV_XM(NC, RPW, 17);                       \
        else if constexpr (!SWIGLU) {                                     \
            if (xm == 3) VH_GEMV_XM(NC, RPW, 3);                          \
            else if (xm == 4) VH_GEMV_XM(NC, RPW, 4);                     \
            else if (xm == 5) VH_GEMV_XM(NC, RPW, 5);                     \
            else if (xm == 7) VH_GEMV_XM(NC, RPW, 7);                     \
            else if (xm == 12) VH_GEMV_XM(NC, RPW, 12);                   \
            else if (xm == 19) VH_GEMV_XM(NC, RPW, 19);                   \
            else if (xm == 20) VH_GEMV_XM(NC, RPW, 20);                   \
            else if (xm == 21) VH_GEMV_XM(NC, RPW, 21);                   \
            else if (xm == 23) VH_GEMV_XM(NC, RPW, 23);                   \
            else if (xm == 28) VH_GEMV_XM(NC, RPW, 28);                   \
            else if (xm == 60) VH_GEMV_XM(NC, RPW, 60);                   \
        }                                                                 \
    } while (0)
    if (nc <= 1) {
        VH_GEMV(1, 1);
    } else if (nc <= 2) {
        VH_GEMV(2, 1);
    } else if (nc <= 3) {
        VH_GEMV(3, 1);
    } else if (WT == VLRF_HIP_DT_Q8_0 && nc == 4) {
        // K = 4096 (the 8B shape's d_model): 2 activation slots per thread.
        if constexpr (WT == VLRF_HIP_DT_Q8_0) VH_GEMV(4, 1);
    } else if (WT == VLRF_HIP_DT_Q8_0 && nc <= 6) {
        // Q4_0 chunks are 2048 wide, so K <= kGemvMaxK needs at most 3 of them.
        if constexpr (WT == VLRF_HIP_DT_Q8_0) VH_GEMV(6, 1);
    } else {
        // Wide rows (K <= kGemvWideMaxK): one row per wave, plain or with the
        // residual, one register set (14 / 7 chunks of 16 bytes per lane).
        constexpr int NCW = WT == VLRF_HIP_DT_Q8_0 ? 14 : 7;
        VH_ARG(!SWIGLU && nc <= NCW && (xm == 16 || xm == 20), "gemv: K %d too large for the M=1 path (form %d)",
               a.K, xm);
        if constexpr (!SWIGLU) {
            const dim3 grid((a.N + kGemvWaves - 1) / kGemvWaves);
            if (xm == 16)
                VH_LAUNCH((gemv_wide_kernel<WT, NCW, 16>), grid, dim3(64 * kGemvWaves), 0, s, a.q, a.d, a.N, a.K,
                          x, residual, y);
            else
                VH_LAUNCH((gemv_wide_kernel<WT, NCW, 20>), grid, dim3(64 * kGemvWaves), 0, s, a.q, a.d, a.N, a.K,
                          x, residual, y);
        }
    }
#undef VH_GEMV
#undef VH_GEMV_XM
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

// The LDS-staged GEMV covers K up to kGemvMaxK columns in every form.
bool gemv_fits(const DevWeight& w) {
    return (w.dtype == VLRF_HIP_DT_Q8_0 || w.dtype == VLRF_HIP_DT_Q4_0) && w.K <= kGemvMaxK;
}

// ... and up to kGemvWideMaxK in the plain / residual forms with one row per
// wave (N <= 8 * kGemvMaxOneGroups).
bool gemv_wide_fits(const DevWeight& w) {
    return (w.dtype == VLRF_HIP_DT_Q8_0 || w.dtype == VLRF_HIP_DT_Q4_0) && w.K <= gemv::kGemvWideMaxK &&
           (w.N + kGemvWaves - 1) / kGemvWaves <= kGemvMaxOneGroups;
}

int check_weight(const DevWeight& w) {
    VH_ARG(w.N > 0 && w.K > 0, "qlinear: empty weight");
    VH_ARG(w.dtype == VLRF_HIP_DT_F32 || w.dtype == VLRF_HIP_DT_Q8_0 || w.dtype == VLRF_HIP_DT_Q4_0,
           "qlinear: unsupported weight dtype %d", w.dtype);
    VH_ARG(w.K % 32 == 0, "qlinear: K=%d must be a multiple of 32", w.K);
    if (w.dtype == VLRF_HIP_DT_F32) VH_ARG(w.f != nullptr, "qlinear: f32 weight not allocated");
    else VH_ARG(w.q != nullptr && w.d != nullptr, "qlinear: quantized weight not allocated");
    return VLRF_HIP_OK;
}

}  // namespace

int launch_qlinear(hipStream_t s, const DevWeight& w, const float* x, float* y, int M,
                   const float* norm_w, float eps, const float* residual) {
    int rc = check_weight(w);
    if (rc) return rc;
    VH_ARG(M >= 1 && M <= 16, "qlinear: M=%d outside [1,16]", M);
    VH_ARG(x && y, "qlinear: null activation pointer");
    if (M == 1 && (gemv_fits(w) || (!norm_w && gemv_wide_fits(w)))) {
        if (w.dtype == VLRF_HIP_DT_Q8_0) return launch_gemv<VLRF_HIP_DT_Q8_0, false>(s, w, nullptr, x, y, norm_w, eps, residual);
        return launch_gemv<VLRF_HIP_DT_Q4_0, false>(s, w, nullptr, x, y, norm_w, eps, residual);
    }
    switch (w.dtype) {
        case VLRF_HIP_DT_Q8_0: return dispatch_m<VLRF_HIP_DT_Q8_0, false>(s, w, nullptr, x, y, M, norm_w, eps, residual);
        case VLRF_HIP_DT_Q4_0: return dispatch_m<VLRF_HIP_DT_Q4_0, false>(s, w, nullptr, x, y, M, norm_w, eps, residual);
        default:           return dispatch_m<VLRF_HIP_DT_F32, false>(s, w, nullptr, x, y, M, norm_w, eps, residual);
    }
}

bool qlinear_argmax_supported(const DevWeight& w) {
    return gemv_fits(w) && (w.N + kGemvWaves - 1) / kGemvWaves > kGemvMaxOneGroups;
}

int launch_qlinear_argmax(hipStream_t s, const DevWeight& w, const float* x, float* y, const float* norm_w,
                          float eps, float2* pairs, int* npairs) {
    int rc = check_weight(w);
    if (rc) return rc;
    VH_ARG(qlinear_argmax_supported(w) && norm_w && x && y && pairs, "qlinear_argmax: not supported");
    const int groups = (w.N + kGemvWaves - 1) / kGemvWaves;
    *npairs = groups < kGemvMaxGroups ? groups : kGemvMaxGroups;
    if (w.dtype == VLRF_HIP_DT_Q8_0)
        return launch_gemv<VLRF_HIP_DT_Q8_0, false>(s, w, nullptr, x, y, norm_w, eps, nullptr, nullptr, nullptr, 0, 64, pairs);
    return launch_gemv<VLRF_HIP_DT_Q4_0, false>(s, w, nullptr, x, y, norm_w, eps, nullptr, nullptr, nullptr, 0, 64, pairs);
}

bool qlinear_gather_supported(const DevWeight& w) { return gemv_fits(w); }

int qlinear_merge_max_chunks(const DevWeight& w) {
    if (!gemv_fits(w) || w.K % 64) return 0;
    const int cw = w.dtype == VLRF_HIP_DT_Q8_0 ? 64 * Gemv<VLRF_HIP_DT_Q8_0>::EPL : 64 * Gemv<VLRF_HIP_DT_Q4_0>::EPL;
    int nc = (w.K + cw - 1) / cw;
    if (nc > 4 || (nc == 4 && w.dtype != VLRF_HIP_DT_Q8_0)) nc = 6;   // instantiated: 1, 2, 3, 4 (Q8_0), 6
    const int per = (nc * cw / 4 + 64 * kGemvWaves - 1) / (64 * kGemvWaves);
    return kAttnMaxChunks / per;
}

int launch_qlinear_merge(hipStream_t s, const DevWeight& w, const float* chunks, int nch, const float* residual,
                         float* y, int head_dim) {
    int rc = check_weight(w);
    if (rc) return rc;
    VH_ARG(chunks && y && residual && nch >= 1, "qlinear_merge: bad arguments");
    VH_ARG(gemv_fits(w), "qlinear_merge: weight does not take the M=1 GEMV path");
    VH_ARG(nch <= qlinear_merge_max_chunks(w), "qlinear_merge: %d chunks, at most %d for K %d", nch,
           qlinear_merge_max_chunks(w), w.K);
    VH_ARG(head_dim == 64 || head_dim == 128, "qlinear_merge: head dim %d", head_dim);
    if (w.dtype == VLRF_HIP_DT_Q8_0)
        return launch_gemv<VLRF_HIP_DT_Q8_0, false>(s, w, nullptr, chunks, y, nullptr, 0.f, residual, nullptr, nullptr, nch,
                                                head_dim);
    return launch_gemv<VLRF_HIP_DT_Q4_0, false>(s, w, nullptr, chunks, y, nullptr, 0.f, residual, nullptr, nullptr, nch,
                                            head_dim);
}

int launch_qlinear_gather(hipStream_t s, const DevWeight& w, const float* table, const int* row,
                          float* x_copy, float* y, const float* norm_w, float eps) {
    int rc = check_weight(w);
    if (rc) return rc;
    VH_ARG(gemv_fits(w), "qlinear_gather: weight dtype %d / K %d not supported", w.dtype, w.K);
    if (w.dtype == VLRF_HIP_DT_Q8_0)
        return launch_gemv<VLRF_HIP_DT_Q8_0, false>(s, w, nullptr, table, y, norm_w, eps, nullptr, row, x_copy);
    return launch_gemv<VLRF_HIP_DT_Q4_0, false>(s, w, nullptr, table, y, norm_w, eps, nullptr, row, x_copy);
}

int launch_qlinear_swiglu(hipStream_t s, const DevWeight& wg, const DevWeight& wu,
                          const float* x, float* h, int M, const float* norm_w, float eps) {
    int rc = check_weight(wg);
    if (rc) return rc;
    rc = check_weight(wu);
    if (rc) return rc;
    VH_ARG(wg.N == wu.N && wg.K == wu.K && wg.dtype == wu.dtype,
           "swiglu: gate/up shapes or dtypes differ");
    VH_ARG(M >= 1 && M <= 16, "swiglu: M=%d outside [1,16]", M);
    if (M == 1 && gemv_fits(wg)) {
        if (wg.dtype == VLRF_HIP_DT_Q8_0) return launch_gemv<VLRF_HIP_DT_Q8_0, true>(s, wg, &wu, x, h, norm_w, eps, nullptr);
        return launch_gemv<VLRF_HIP_DT_Q4_0, true>(s, wg, &wu, x, h, norm_w, eps, nullptr);
    }
    switch (wg.dtype) {
        case VLRF_HIP_DT_Q8_0: return dispatch_m<VLRF_HIP_DT_Q8_0, true>(s, wg, &wu, x, h, M, norm_w, eps, nullptr);
        case VLRF_HIP_DT_Q4_0: return dispatch_m<VLRF_HIP_DT_Q4_0, true>(s, wg, &wu, x, h, M, norm_w, eps, nullptr);
        default:           return dispatch_m<VLRF_HIP_DT_F32, true>(s, wg, &wu, x, h, M, norm_w, eps, nullptr);
    }
}

}  // namespace vlrf_hip
