// ops.hip - the engine's remaining per-op backend calls on the device
// (IBackend::gemm / layer_norm / softmax_inplace / gelu_inplace / add_inplace,
// include/backend/ibackend.hpp:61-70), used by GPT-2-family models.
//
// Semantics follow the CPU ops (include/model/ops.hpp): gemm :170-310
// (C = beta*C first -- beta == 0 writes zeros -- then alpha*op(A)*op(B) added;
// op = transpose when transA / transB), layer_norm :443-476 (mean, variance of
// the deviations, (x - mean) * (1/sqrt(var + eps)) * w + b), softmax_inplace
// :501-540 (row max, exp(x - max), x * (1/(sum + 1e-9))), gelu_inplace
// :390-404 (tanh approximation 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3)))),
// add_inplace :344-356.  f32 throughout; reductions are tree-ordered, so
// results agree with the sequential CPU loops to f32 rounding.
#include "../internal.hpp"

#include <cmath>

namespace vlrf_hip {
namespace {

// f32 GEMM: a 256-lane workgroup owns a 64x64 tile of C, each lane a 4x4 block
// (rows ty + 16i, columns tx + 16j, so LDS reads of a wave are broadcast or
// conflict-free); K in steps of 16 staged through LDS.  op(A)[m][k] and
// op(B)[k][n] are gathered with the transposes applied on the way into LDS.
constexpr int kGT = 64, kGK = 16;

__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                       float* C, int M, int N, int K, int lda, int ldb, int ldc,
                                                       float alpha, float beta, int transA, int transB) {
    __shared__ float As[kGK][kGT + 1];
    __shared__ float Bs[kGK][kGT + 1];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int m0 = blockIdx.y * kGT, n0 = blockIdx.x * kGT;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += kGK) {
        for (int i = tid; i < kGT * kGK; i += 256) {
            // A tile element (m, k): lanes walk k fastest when A is row-major in k
            const int r = transA ? i % kGT : i / kGK, c = transA ? i / kGT : i % kGK;
            const int m = m0 + r, k = k0 + c;
            float a = 0.f;
            if (m < M && k < K) a = transA ? A[(size_t)k * lda + m] : A[(size_t)m * lda + k];
            As[c][r] = a;
            const int rb = transB ? i / kGK : i % kGT, cb = transB ? i % kGK : i / kGT;   // (n, k)
            const int n = n0 + rb, kb = k0 + cb;
            float b = 0.f;
            if (n < N && kb < K) b = transB ? B[(size_t)n * ldb + kb] : B[(size_t)kb * ldb + n];
            Bs[cb][rb] = b;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kGK; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[kk][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = m0 + ty + 16 * i, n = n0 + tx + 16 * j;
            if (m < M && n < N) {
                float* c = C + (size_t)m * ldc + n;
                const float prev = beta == 0.f ? 0.f : (beta == 1.f ? *c : *c * beta);
                *c = prev + alpha * acc[i][j];
            }
        }
}

__device__ __forceinline__ float block_sum(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float block_max(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_max(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__global__ __launch_bounds__(256) void layer_norm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                         const float* __restrict__ b, float* out, int D,
                                                         float eps) {
    __shared__ float red[4];
    const float* r = x + (size_t)blockIdx.x * D;
    float s = 0.f;
    for (int j = threadIdx.x; j < D; j += 256) s += r[j];
    const float mean = block_sum(s, red) / (float)D;
    float v = 0.f;
    for (int j = threadIdx.x; j < D; j += 256) {
        const float d = r[j] - mean;
        v += d * d;
    }
    const float var = block_sum(v, red) / (float)D + eps;
    const float inv = 1.f / sqrtf(var);
    float* o = out + (size_t)blockIdx.x * D;
    for (int j = threadIdx.x; j < D; j += 256) o[j] = (r[j] - mean) * inv * w[j] + b[j];
}

__global__ __launch_bounds__(256) void softmax_kernel(float* x, int D) {
    __shared__ float red[4];
    float* r = x + (size_t)blockIdx.x * D;
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < D; j += 256) mx = fmaxf(mx, r[j]);
    mx = block_max(mx, red);
    float s = 0.f;
    for (int j = threadIdx.x; j < D; j += 256) {
        const float e = expf(r[j] - mx);
        r[j] = e;
        s += e;
    }
    const float inv = 1.f / (block_sum(s, red) + 1e-9f);
    for (int j = threadIdx.x; j < D; j += 256) r[j] *= inv;
}

__global__ __launch_bounds__(256) void gelu_kernel(float* x, int64_t n) {
    constexpr float c1 = 0.7978845608028654f, c2 = 0.044715f;   // sqrt(2/pi), ops.hpp:393-394
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float v = x[i];
        const float inner = c1 * (v + c2 * v * v * v);
        x[i] = 0.5f * v * (1.f + tanhf(inner));
    }
}

__global__ __launch_bounds__(256) void add_kernel(float* dst, const float* __restrict__ src, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        dst[i] += src[i];
}

int grid_1d(int64_t n) {
    const int64_t g = (n + 255) / 256;
    return (int)(g < 4096 ? (g < 1 ? 1 : g) : 4096);
}

}  // namespace

int launch_gemm_f32(hipStream_t s, const float* A, const float* B, float* C, int M, int N, int K, int lda,
                    int ldb, int ldc, float alpha, float beta, bool transA, bool transB) {
    VH_ARG(A && B && C, "gemm_f32: null operand");
    VH_ARG(M >= 1 && N >= 1 && K >= 1, "gemm_f32: empty shape %dx%dx%d", M, N, K);
    VH_ARG(lda >= (transA ? M : K) && ldb >= (transB ? K : N) && ldc >= N, "gemm_f32: leading dimension too small");
    dim3 grid((N + kGT - 1) / kGT, (M + kGT - 1) / kGT);
    hipLaunchKernelGGL(gemm_f32_kernel, grid, dim3(256), 0, s, A, B, C, M, N, K, lda, ldb, ldc, alpha, beta,
                       (int)transA, (int)transB);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_layer_norm(hipStream_t s, const float* x, const float* w, const float* b, float* out, int rows, int D,
                      float eps) {
    VH_ARG(x && w && b && out && rows >= 1 && D >= 1, "layer_norm: bad arguments");
    hipLaunchKernelGGL(layer_norm_kernel, dim3(rows), dim3(256), 0, s, x, w, b, out, D, eps);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_softmax(hipStream_t s, float* x, int rows, int D) {
    VH_ARG(x && rows >= 1 && D >= 1, "softmax: bad arguments");
    hipLaunchKernelGGL(softmax_kernel, dim3(rows), dim3(256), 0, s, x, D);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_gelu(hipStream_t s, float* x, int64_t n) {
    VH_ARG(x && n >= 0, "gelu: bad arguments");
    if (n == 0) return VLRF_HIP_OK;
    hipLaunchKernelGGL(gelu_kernel, dim3(grid_1d(n)), dim3(256), 0, s, x, n);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_add(hipStream_t s, float* dst, const float* src, int64_t n) {
    VH_ARG(dst && src && n >= 0, "add: bad arguments");
    if (n == 0) return VLRF_HIP_OK;
    hipLaunchKernelGGL(add_kernel, dim3(grid_1d(n)), dim3(256), 0, s, dst, src, n);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

}  // namespace vlrf_hip
