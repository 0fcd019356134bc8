// gemm.hip - dequant-fused MFMA GEMM for the prefill path (M > 16 rows).
//
// Reference contract: compute::linear -> ops::gemm(x, W, y, 1, 0, false, true)
// (include/model/compute.hpp:58-68, ops.hpp:254-305 for M >= 4) on weights
// decoded from GGUF Q8_0/Q4_0 blocks (tools/converter/convert_gguf.py:233-263).
// The reference computes in f32; this path rounds the activations and the
// decoded weights to bf16 and accumulates in f32 on the matrix cores (the
// 1e-2 tolerance class of bf16 paths).
//
// Design (gfx950): C[M,N] = A[M,K] . W[N,K]^T with A in bf16 and W as split
// GGUF blocks (codes [N][K], f16 scales [N][K/32]).  A 256-lane workgroup owns
// a 128x128 tile of C; each wave a 64x64 quarter as 2x2 v_mfma_f32_32x32x16_bf16
// blocks.  K advances in steps of 64: the next step's A rows and weight codes
// are loaded into registers while the matrix cores work on the current step,
// then the codes are dequantized (code * scale -> bf16) on their way into the
// other LDS buffer, so W is read from HBM once per tile column as 1.06 B
// (Q8_0) or 0.56 B (Q4_0) per weight.  LDS rows are padded by 16 bytes so the
// 32 lanes of an operand read hit distinct banks.  Epilogues: store f32,
// add a residual, or SwiGLU (two weights, silu(g)*u) with bf16 output.
#include "../internal.hpp"

namespace vlrf_hip {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kGemmThreads = 256;
constexpr int kLds = kBK + 8;            // bf16 per LDS row (16 bytes of padding)

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return bf16_bits(lo) | (bf16_bits(hi) << 16);
}

// One K step of global operands held in registers between load and LDS store.
// Thread t covers row t/2 of the tile and half t%2 of the 64 columns.
template <int WT, int NM>
struct GemmStage {
    uint4 a[4];                          // 32 bf16 of A
    uint4 w[NM][WT == VLRF_DT_Q8_0 ? 2 : 1];   // 32 codes (Q8_0) or 32 nibbles (Q4_0)
    uint32_t s[NM];                      // raw f16 scale of the 32-element block
};

template <int WT, int NM>
__device__ __forceinline__ void gemm_load(GemmStage<WT, NM>& st, const uint16_t* __restrict__ A,
                                          const uint8_t* qa, const __half* da, const uint8_t* qb,
                                          const __half* db, int m0, int n0, int k0, int M, int N, int K) {
    const int t = threadIdx.x, r = t >> 1, hf = t & 1;
    const int am = min(m0 + r, M - 1), wn = min(n0 + r, N - 1);   // clamped: rows past M/N are not stored
    const uint4* ap = reinterpret_cast<const uint4*>(A + (size_t)am * K + k0 + 32 * hf);
#pragma unroll
    for (int i = 0; i < 4; ++i) st.a[i] = ap[i];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const uint8_t* q = m ? qb : qa;
        const uint16_t* d = reinterpret_cast<const uint16_t*>(m ? db : da);
        if constexpr (WT == VLRF_DT_Q8_0) {
            const uint4* wp = reinterpret_cast<const uint4*>(q + (size_t)wn * K + k0 + 32 * hf);
            st.w[m][0] = wp[0];
            st.w[m][1] = wp[1];
        } else {
            st.w[m][0] = *reinterpret_cast<const uint4*>(q + (size_t)wn * (K / 2) + (k0 + 32 * hf) / 2);
        }
        st.s[m] = d[(size_t)wn * (K / 32) + k0 / 32 + hf];
    }
}

template <int WT, int NM>
__device__ __forceinline__ void gemm_store(const GemmStage<WT, NM>& st, uint16_t* As, uint16_t* Bs) {
    const int t = threadIdx.x, r = t >> 1, hf = t & 1;
    uint4* ad = reinterpret_cast<uint4*>(As + r * kLds + 32 * hf);
#pragma unroll
    for (int i = 0; i < 4; ++i) ad[i] = st.a[i];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const float sc = __half2float(__ushort_as_half((unsigned short)st.s[m]));
        float v[32];
        if constexpr (WT == VLRF_DT_Q8_0) {
            const uint32_t u[8] = {st.w[m][0].x, st.w[m][0].y, st.w[m][0].z, st.w[m][0].w,
                                   st.w[m][1].x, st.w[m][1].y, st.w[m][1].z, st.w[m][1].w};
#pragma unroll
            for (int j = 0; j < 32; ++j) v[j] = (float)(int8_t)(u[j >> 2] >> (8 * (j & 3))) * sc;
        } else {
            const uint32_t u[4] = {st.w[m][0].x, st.w[m][0].y, st.w[m][0].z, st.w[m][0].w};
#pragma unroll
            for (int j = 0; j < 16; ++j) {    // byte j: element 2j (low nibble), 2j+1 (high)
                const uint32_t b = (u[j >> 2] >> (8 * (j & 3))) & 0xFFu;
                v[2 * j] = (float)((int)(b & 0xFu) - 8) * sc;
                v[2 * j + 1] = (float)((int)(b >> 4) - 8) * sc;
            }
        }
        uint4* bd = reinterpret_cast<uint4*>(Bs + (size_t)m * kBN * kLds + r * kLds + 32 * hf);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            bd[i] = make_uint4(pack_bf16(v[8 * i], v[8 * i + 1]), pack_bf16(v[8 * i + 2], v[8 * i + 3]),
                               pack_bf16(v[8 * i + 4], v[8 * i + 5]), pack_bf16(v[8 * i + 6], v[8 * i + 7]));
    }
}

// EPI: 0 = store f32, 1 = f32 + residual, 2 = SwiGLU silu(g)*u (NM = 2) stored
// as bf16 (the next GEMM's operand), 3 = SwiGLU stored as f32.
template <int WT, int EPI>
__global__ __launch_bounds__(kGemmThreads) void mfma_qgemm_kernel(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ qa, const __half* __restrict__ da,
    const uint8_t* __restrict__ qb, const __half* __restrict__ db, int M, int N, int K,
    const float* __restrict__ residual, void* __restrict__ out) {
    constexpr int NM = EPI >= 2 ? 2 : 1;
    __shared__ __align__(16) uint16_t As[2][kBM * kLds];
    __shared__ __align__(16) uint16_t Bs[2][NM * kBN * kLds];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;

    f32x16 acc[NM][2][2];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[m][i][j] = f32x16{};

    GemmStage<WT, NM> st;
    gemm_load<WT, NM>(st, A, qa, da, qb, db, m0, n0, 0, M, N, K);
    gemm_store<WT, NM>(st, As[0], Bs[0]);
    __syncthreads();

    const int nk = K / kBK;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        // Unconditional (the last step reloads its own tile, unused): a conditional
        // load would leave the staging registers to a merge the compiler spills.
        gemm_load<WT, NM>(st, A, qa, da, qb, db, m0, n0, min(kt + 1, nk - 1) * kBK, M, N, K);
        const uint16_t* as = As[cur];
        const uint16_t* bs = Bs[cur];
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const int kc = kk * 16 + 8 * (lane >> 5);      // this lane's 8 k of the 16
            bf16x8 af[2], bf[NM][2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const bf16x8*>(as + (64 * wm + 32 * i + (lane & 31)) * kLds + kc);
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    bf[m][j] = *reinterpret_cast<const bf16x8*>(bs + (size_t)m * kBN * kLds +
                                                                 (64 * wn + 32 * j + (lane & 31)) * kLds + kc);
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[m][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[m][j], acc[m][i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) gemm_store<WT, NM>(st, As[cur ^ 1], Bs[cur ^ 1]);
        __syncthreads();
    }

    // Accumulator v of block (i, j) holds C[row][col] with
    // row = 32i + 8(v/4) + 4(lane/32) + v%4 and col = 32j + lane%32 (of the wave's 64x64).
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + 64 * wm + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                const int col = n0 + 64 * wn + 32 * j + (lane & 31);
                if (row < M && col < N) {
                    const size_t o = (size_t)row * N + col;
                    if constexpr (EPI >= 2) {
                        const float g = acc[0][i][j][v], u = acc[1][i][j][v];
                        const float hv = u * (g / (1.f + expf(-g)));   // silu(g) * u, ops.hpp:409-441
                        if constexpr (EPI == 2) reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)bf16_bits(hv);
                        else reinterpret_cast<float*>(out)[o] = hv;
                    } else if constexpr (EPI == 1) {
                        reinterpret_cast<float*>(out)[o] = acc[0][i][j][v] + residual[o];
                    } else {
                        reinterpret_cast<float*>(out)[o] = acc[0][i][j][v];
                    }
                }
            }
}

// out[r][:] = bf16(w ? rmsnorm(x[r]) * w : x[r]), one 256-lane workgroup per row
// (ops.hpp:488-498: sum of squares, 1/sqrt(mean + eps), (x * inv) * w).
__global__ __launch_bounds__(256) void rows_to_bf16_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ w,
                                                           uint16_t* __restrict__ out, int D, float eps) {
    __shared__ float red[4];
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* xr = x + (size_t)r * D;
    float inv = 1.f;
    if (w) {
        float ss = 0.f;
        for (int i = tid; i < D; i += 256) ss += xr[i] * xr[i];
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        inv = 1.f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)D + eps);
    }
    uint16_t* o = out + (size_t)r * D;
    for (int i = tid; i < D; i += 256) o[i] = (uint16_t)bf16_bits(w ? xr[i] * inv * w[i] : xr[i]);
}

int check_qgemm(const DevWeight& w, int M) {
    VH_ARG(w.dtype == VLRF_DT_Q8_0 || w.dtype == VLRF_DT_Q4_0,
           "qgemm: the MFMA path takes Q8_0/Q4_0 weights (dtype %d)", w.dtype);
    VH_ARG(w.q != nullptr && w.d != nullptr, "qgemm: weight not allocated");
    VH_ARG(w.K % kBK == 0, "qgemm: K=%d must be a multiple of %d", w.K, kBK);
    VH_ARG(M >= 1, "qgemm: M=%d", M);
    return VLRF_HIP_OK;
}

}  // namespace

int launch_rows_to_bf16(hipStream_t s, const float* x, const float* w, uint16_t* out, int rows, int D,
                        float eps) {
    VH_ARG(x && out && rows >= 1 && D >= 1, "rows_to_bf16: bad arguments");
    hipLaunchKernelGGL(rows_to_bf16_kernel, dim3(rows), dim3(256), 0, s, x, w, out, D, eps);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_qgemm(hipStream_t s, const DevWeight& w, const uint16_t* a, int M, const float* residual,
                 float* y) {
    int rc = check_qgemm(w, M);
    if (rc) return rc;
    VH_ARG(a && y, "qgemm: null operand");
    dim3 grid((w.N + kBN - 1) / kBN, (M + kBM - 1) / kBM), block(kGemmThreads);
#define VH_QG(WT, EPI)                                                                                 \
    hipLaunchKernelGGL((mfma_qgemm_kernel<WT, EPI>), grid, block, 0, s, a, w.q, w.d, nullptr, nullptr, \
                       M, w.N, w.K, residual, (void*)y)
    if (w.dtype == VLRF_DT_Q8_0) {
        if (residual) VH_QG(VLRF_DT_Q8_0, 1); else VH_QG(VLRF_DT_Q8_0, 0);
    } else {
        if (residual) VH_QG(VLRF_DT_Q4_0, 1); else VH_QG(VLRF_DT_Q4_0, 0);
    }
#undef VH_QG
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_qgemm_swiglu(hipStream_t s, const DevWeight& wg, const DevWeight& wu, const uint16_t* a,
                        int M, void* h, bool h_bf16) {
    int rc = check_qgemm(wg, M);
    if (rc) return rc;
    rc = check_qgemm(wu, M);
    if (rc) return rc;
    VH_ARG(wg.N == wu.N && wg.K == wu.K && wg.dtype == wu.dtype, "qgemm_swiglu: gate/up differ");
    VH_ARG(a && h, "qgemm_swiglu: null operand");
    dim3 grid((wg.N + kBN - 1) / kBN, (M + kBM - 1) / kBM), block(kGemmThreads);
#define VH_QS(WT, EPI)                                                                                  \
    hipLaunchKernelGGL((mfma_qgemm_kernel<WT, EPI>), grid, block, 0, s, a, wg.q, wg.d, wu.q, wu.d, M, wg.N, \
                       wg.K, nullptr, h)
    if (wg.dtype == VLRF_DT_Q8_0) {
        if (h_bf16) VH_QS(VLRF_DT_Q8_0, 2); else VH_QS(VLRF_DT_Q8_0, 3);
    } else {
        if (h_bf16) VH_QS(VLRF_DT_Q4_0, 2); else VH_QS(VLRF_DT_Q4_0, 3);
    }
#undef VH_QS
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

}  // namespace vlrf_hip
