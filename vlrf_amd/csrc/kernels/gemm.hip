// gemm.hip - dequant-fused linear layers on the matrix cores.
//
// Reference contract: compute::linear -> ops::gemm(x, W, y, 1, 0, false, true)
// (include/model/compute.hpp:58-68, ops.hpp:170-310) on weights decoded from
// GGUF Q8_0/Q4_0 blocks (tools/converter/convert_gguf.py:233-263).
//
// 1. Prefill GEMM (M > 16 rows).  The reference computes in f32; this path
// rounds the activations and the decoded weights to bf16 and accumulates in
// f32 (the 1e-2 tolerance class of bf16 paths).  For 17 <= M <= 128,
// mfma_qgemm_kernel:  C[M,N] = A[M,K] . W[N,K]^T
// with A in bf16 and W as split GGUF blocks (codes [N][K], f16 scales
// [N][K/32]).  A workgroup owns a BM x BN tile of C, each wave a block of
// v_mfma_f32_32x32x16_bf16 tiles.  K advances in steps of BK: the next step's
// A rows and weight codes are loaded into registers while the matrix cores
// work on the current step, then the codes are dequantized (code * scale ->
// bf16) on their way into the other LDS buffer, so W is read from HBM once per
// tile column as 1.06 B (Q8_0) or 0.56 B (Q4_0) per weight.  LDS rows are
// padded by 16 bytes so the lanes of an operand read hit distinct banks.
// Epilogues: store f32, add a residual, or SwiGLU (two weights, silu(g)*u).
// Weights with M > 128 take mfma_qgemm_lds_kernel instead (below): the
// same arithmetic with operands brought into a 3-stage LDS ring by
// direct-to-LDS loads and codes decoded in registers next to the MFMAs.
//
// 2. Small M (2..16 rows, ops.hpp:142-168,254-305 for M = 2..16) with
// f32-class accuracy.  Q8_0/Q4_0 codes are integers of at most 8 bits, exact
// in bf16, so one v_mfma_f32_16x16x32_bf16 multiplies the codes of one 32-wide
// block of 16 weight rows with 32 activations of 16 rows exactly, and the
// block scale is applied to the f32 result afterwards.  The activations are
// split into bf16 hi + lo (x = hi + lo to about 2^-17 relative), two MFMAs per
// block, so the products carry ~16 significant bits of x and accumulate in
// f32: results agree with the f32 reference to ~1e-5 relative.
#include "../internal.hpp"
#include "gemv_core.hpp"

namespace vlrf_hip {
namespace {

// silu(g) * u (ops.hpp:409-441: g / (1 + exp(-g)) times u) for the bf16-class
// GEMM epilogues: the hardware exp2 and reciprocal (about 1 ulp each) instead
// of the library expf and the correctly rounded division, whose extra
// instructions sat in every tile's epilogue.  g -> -inf gives -0 as the
// division does; the f32-class paths keep the exact form.
__device__ __forceinline__ float silu_mul_fast(float g, float u) {
    return u * (g * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f)));
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Tile configuration: BM x BN tile of C per workgroup, K steps of BK, WM x WN
// waves each owning a (BM/WM) x (BN/WN) block of 32x32 MFMA tiles.
template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct TileCfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    static constexpr int NT = 64 * WM * WN;
    static constexpr int LDS = BK + 8;            // bf16 per LDS row (16 bytes of padding)
    static constexpr int EA = BM * BK / NT;       // A elements (bf16) staged per thread
    static constexpr int EB = BN * BK / NT;       // weight elements staged per thread (per matrix)
    static constexpr int MI = BM / WM / 32, NI = BN / WN / 32;
    static_assert(EA % 8 == 0 && BK % EA == 0, "A staging granularity");
    static_assert((EB == 8 || EB == 16 || EB == 32) && BK % EB == 0, "weight staging granularity");
    static_assert(MI >= 1 && NI >= 1 && BK % 32 == 0, "tile shape");
};

// Raw weight bytes of EB elements: Q8_0 one byte each, Q4_0 a nibble each.
template <int WT, int EB>
struct WBytes { static constexpr int DW = WT == VLRF_HIP_DT_Q8_0 ? EB / 4 : EB / 8; };

template <int DW>
__device__ __forceinline__ void load_dwords(uint32_t (&o)[DW], const uint8_t* p) {
    if constexpr (DW == 8) {
        const uint4 a = reinterpret_cast<const uint4*>(p)[0], b = reinterpret_cast<const uint4*>(p)[1];
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
    } else if constexpr (DW == 4) {
        const uint4 a = *reinterpret_cast<const uint4*>(p);
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    } else if constexpr (DW == 2) {
        const uint2 a = *reinterpret_cast<const uint2*>(p);
        o[0] = a.x; o[1] = a.y;
    } else {
        o[0] = *reinterpret_cast<const uint32_t*>(p);
    }
}

// One K step of global operands held in registers between load and LDS store.
template <class C, int WT, int NM>
struct GemmStage {
    uint4 a[C::EA / 8];
    uint32_t w[NM][WBytes<WT, C::EB>::DW];
    uint32_t s[NM];                      // raw f16 scale of the 32-element block
};

template <class C, int WT, int NM>
__device__ __forceinline__ void gemm_load(GemmStage<C, WT, NM>& st, const uint16_t* __restrict__ A,
                                          const uint8_t* qa, const __half* da, const uint8_t* qb,
                                          const __half* db, int m0, int n0, int k0, int M, int N, int K) {
    const int t = threadIdx.x;
    {
        const int r = t / (C::BK / C::EA), pa = t % (C::BK / C::EA);
        const int am = min(m0 + r, M - 1);          // clamped: rows past M are not stored
        const uint4* ap = reinterpret_cast<const uint4*>(A + (size_t)am * K + k0 + pa * C::EA);
#pragma unroll
        for (int i = 0; i < C::EA / 8; ++i) st.a[i] = ap[i];
    }
    const int r = t / (C::BK / C::EB), pb = t % (C::BK / C::EB);
    const int wn = min(n0 + r, N - 1);              // clamped: rows past N are not stored
    const int kb = k0 + pb * C::EB;                 // first element; one 32-block per thread
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const uint8_t* q = m ? qb : qa;
        const uint16_t* d = reinterpret_cast<const uint16_t*>(m ? db : da);
        if constexpr (WT == VLRF_HIP_DT_Q8_0) load_dwords(st.w[m], q + (size_t)wn * K + kb);
        else load_dwords(st.w[m], q + (size_t)wn * (K / 2) + kb / 2);
        st.s[m] = d[(size_t)wn * (K / 32) + kb / 32];
    }
}

template <class C, int WT, int NM>
__device__ __forceinline__ void gemm_store(const GemmStage<C, WT, NM>& st, uint16_t* As, uint16_t* Bs) {
    const int t = threadIdx.x;
    {
        const int r = t / (C::BK / C::EA), pa = t % (C::BK / C::EA);
        uint4* ad = reinterpret_cast<uint4*>(As + r * C::LDS + pa * C::EA);
#pragma unroll
        for (int i = 0; i < C::EA / 8; ++i) ad[i] = st.a[i];
    }
    const int r = t / (C::BK / C::EB), pb = t % (C::BK / C::EB);
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const float sc = __half2float(__ushort_as_half((unsigned short)st.s[m]));
        float v[C::EB];
        if constexpr (WT == VLRF_HIP_DT_Q8_0) {
#pragma unroll
            for (int j = 0; j < C::EB; ++j) v[j] = (float)(int8_t)(st.w[m][j >> 2] >> (8 * (j & 3))) * sc;
        } else {
#pragma unroll
            for (int j = 0; j < C::EB / 2; ++j) {    // byte j: element 2j (low nibble), 2j+1 (high)
                const uint32_t b = (st.w[m][j >> 2] >> (8 * (j & 3))) & 0xFFu;
                v[2 * j] = (float)((int)(b & 0xFu) - 8) * sc;
                v[2 * j + 1] = (float)((int)(b >> 4) - 8) * sc;
            }
        }
        uint4* bd = reinterpret_cast<uint4*>(Bs + (size_t)m * C::BN * C::LDS + r * C::LDS + pb * C::EB);
#pragma unroll
        for (int i = 0; i < C::EB / 8; ++i)
            bd[i] = make_uint4(pack_bf16(v[8 * i], v[8 * i + 1]), pack_bf16(v[8 * i + 2], v[8 * i + 3]),
                               pack_bf16(v[8 * i + 4], v[8 * i + 5]), pack_bf16(v[8 * i + 6], v[8 * i + 7]));
    }
}

// EPI: 0 = store f32, 1 = f32 + residual, 2 = SwiGLU silu(g)*u (NM = 2) stored
// as bf16 (the next GEMM's operand), 3 = SwiGLU stored as f32.
template <class C, int WT, int EPI>
__global__ __launch_bounds__(C::NT) void mfma_qgemm_kernel(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ qa, const __half* __restrict__ da,
    const uint8_t* __restrict__ qb, const __half* __restrict__ db, int M, int N, int K,
    const float* __restrict__ residual, void* __restrict__ out) {
    constexpr int NM = EPI >= 2 ? 2 : 1;
    constexpr int MI = C::MI, NI = C::NI, LD = C::LDS;
    __shared__ __align__(16) uint16_t As[2][C::BM * LD];
    __shared__ __align__(16) uint16_t Bs[2][NM * C::BN * LD];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / C::WN, wn = wave % C::WN;
    const int m0 = blockIdx.y * C::BM, n0 = blockIdx.x * C::BN;
    const int rm = wm * (C::BM / C::WM), rn = wn * (C::BN / C::WN);

    f32x16 acc[NM][MI][NI];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j) acc[m][i][j] = f32x16{};

    GemmStage<C, WT, NM> st;
    gemm_load<C, WT, NM>(st, A, qa, da, qb, db, m0, n0, 0, M, N, K);
    gemm_store<C, WT, NM>(st, As[0], Bs[0]);
    __syncthreads();

    const int nk = K / C::BK;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        // Unconditional (the last step reloads its own tile, unused): a conditional
        // load would leave the staging registers to a merge the compiler spills.
        gemm_load<C, WT, NM>(st, A, qa, da, qb, db, m0, n0, min(kt + 1, nk - 1) * C::BK, M, N, K);
        const uint16_t* as = As[cur];
        const uint16_t* bs = Bs[cur];
#pragma unroll
        for (int kk = 0; kk < C::BK / 16; ++kk) {
            const int kc = kk * 16 + 8 * (lane >> 5);      // this lane's 8 k of the 16
            bf16x8 af[MI], bf[NM][NI];
#pragma unroll
            for (int i = 0; i < MI; ++i)
                af[i] = *reinterpret_cast<const bf16x8*>(as + (rm + 32 * i + (lane & 31)) * LD + kc);
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int j = 0; j < NI; ++j)
                    bf[m][j] = *reinterpret_cast<const bf16x8*>(bs + (size_t)m * C::BN * LD +
                                                                 (rn + 32 * j + (lane & 31)) * LD + kc);
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NI; ++j)
                        acc[m][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[m][j], acc[m][i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) gemm_store<C, WT, NM>(st, As[cur ^ 1], Bs[cur ^ 1]);
        __syncthreads();
    }

    // Accumulator v of block (i, j) holds C[row][col] with
    // row = 32i + 8(v/4) + 4(lane/32) + v%4 and col = 32j + lane%32 (of the wave's block).
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + rm + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                const int col = n0 + rn + 32 * j + (lane & 31);
                if (row < M && col < N) {
                    const size_t o = (size_t)row * N + col;
                    if constexpr (EPI >= 2) {
                        const float g = acc[0][i][j][v], u = acc[1][i][j][v];
                        const float hv = silu_mul_fast(g, u);
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

// The register-staged configuration for 17 <= M <= 128 (128-row tiles, where
// the direct-to-LDS kernel's 256-row tiles would be mostly padding): 128x128x64,
// 4 waves.  Both prefill kernels step K by 64, so K % 64 == 0 covers them.
using CfgSmall = TileCfg<128, 128, 64, 2, 2>;
constexpr int kBK = 64;

template <class C, int EPI>
void launch_cfg(hipStream_t s, int wt, const uint16_t* a, const DevWeight& w0, const DevWeight* w1, int M,
                const float* residual, void* out) {
    const dim3 grid((w0.N + C::BN - 1) / C::BN, (M + C::BM - 1) / C::BM), block(C::NT);
    const uint8_t* qb = w1 ? w1->q : nullptr;
    const __half* db = w1 ? w1->d : nullptr;
    if (wt == VLRF_HIP_DT_Q8_0)
        hipLaunchKernelGGL((mfma_qgemm_kernel<C, VLRF_HIP_DT_Q8_0, EPI>), grid, block, 0, s, a, w0.q, w0.d, qb, db,
                           M, w0.N, w0.K, residual, out);
    else
        hipLaunchKernelGGL((mfma_qgemm_kernel<C, VLRF_HIP_DT_Q4_0, EPI>), grid, block, 0, s, a, w0.q, w0.d, qb, db,
                           M, w0.N, w0.K, residual, out);
}

// ---- prefill GEMM with direct-to-LDS loads ---------------------------------------
// C[M,N] = A[M,K] . W[N,K]^T for Q8_0/Q4_0 W and M > 128: workgroup tile 256 x 128
// (per weight matrix; SwiGLU computes gate and up tiles together), 8 waves as
// 2 along M x 4 along N, so each wave owns a 128 x 32 block per matrix (four
// 32x32 MFMA tiles) and each weight code is decoded by only two waves.
// K advances in steps of 64 through a 3-stage LDS ring filled by
// global_load_lds_dwordx4 (the loads write LDS without passing through
// registers): stage = A rows as bf16 (32 KB), the raw codes of the tile's weight
// rows (8 KB per matrix for Q8_0, 4 KB for Q4_0) and their two f16 block
// scales.  16-byte chunks are XOR-swizzled within a row (A: chunk ^
// ((row >> 1) & 7); Q8_0 codes: chunk ^ ((row >> 2) & 3); Q4_0: chunk ^
// ((row >> 3) & 1)) so the MFMA operand reads of consecutive rows spread over
// the banks; the loads realise the swizzle by choosing which global chunk
// each lane fetches (lane l always writes LDS bytes 16l..16l+15 of its wave's
// 1 KB destination).  One barrier per K step: wait until this wave's loads of
// the step have landed, barrier, issue the loads of step k+2 into the buffer
// step k-1 used, compute step k.  The MFMA k order within a 32-element block
// is permuted (lane half h takes elements 16h..16h+15 of block p -- Q8_0 code
// chunk 2p+h, Q4_0 bytes 8h..8h+7 of chunk p -- and slices q = 0, 1 their two
// halves; A uses the same permutation), so a lane reads its codes in one LDS
// read; codes are decoded in registers (code * scale rounded to bf16) just
// before use.
namespace lds_gemm {

// BM: 256 rows of A (waves 2 x 4 over 128 x 32 blocks) or 128 (64 x 32 blocks).
constexpr int BN = 128, NT = 512, WN = 32;
template <int BM> struct ATile {
    static constexpr int WM = BM / 2, MI = WM / 32;
    static constexpr int A_B = BM * 128;                 // one K step of A: BM rows x 64 bf16
    static constexpr int A_IT = A_B / (NT * 16);         // 16-byte loads per thread
};
template <int WT, int NM, int BM> struct Stage {
    static constexpr int A_IT = ATile<BM>::A_IT;
    static constexpr int CB = WT == VLRF_HIP_DT_Q8_0 ? 64 : 32;   // code bytes of a row per K step
    static constexpr int W_B = NM * BN * CB;  // codes: NM*BN rows
    static constexpr int S_B = NM * BN * 4;   // two f16 block scales per row
    static constexpr int W_TI = W_B / 1024;   // 1 KB code loads per step (wave w issues w, w+8, ...)
    static constexpr int W_IT = (W_TI + 7) / 8;
    static constexpr int S_WAVES = NM * BN / 64;
    // Loads of one step by the wave that issues fewest: waiting until at most this
    // many are outstanding leaves only the newer step in flight for every wave.
    static constexpr int LPS = A_IT + W_TI / 8 + (S_WAVES >= 8 ? 1 : 0);
    static constexpr int WAIT = (LPS & 15) | (7 << 4) | (15 << 8) | ((LPS >> 4) << 14);   // s_waitcnt vmcnt(LPS)
    static_assert(W_TI >= 1 && S_WAVES <= 8, "stage shape");
};

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) char*)(p);
}
// Direct-to-LDS loads (lane l writes LDS base + size*l; base wave-uniform, in M0).
// Written as asm so that the compiler's wait insertion, which cannot tell these
// LDS writes apart from the stage being read, does not wait for every load in
// flight before each LDS read; the kernel orders them with explicit vmcnt waits
// and barriers instead.  Loads complete in issue order, so these extra loads
// only make the compiler's own vmcnt waits stricter.
__device__ __forceinline__ void dma16(const void* g, uint32_t base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(g), "s"(__builtin_amdgcn_readfirstlane(base)) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
                 :: "v"(g), "s"(__builtin_amdgcn_readfirstlane(base)) : "memory", "m0");
}
__device__ __forceinline__ int swz_a(int r) { return (r >> 1) & 7; }
// code chunk swizzle within a row: Q8_0 rows of 4 chunks, Q4_0 rows of 2
template <int WT> __device__ __forceinline__ int swz_w(int n) {
    return WT == VLRF_HIP_DT_Q8_0 ? (n >> 2) & 3 : (n >> 3) & 1;
}

// The tile's results: accumulator v of MFMA tile i holds row 32i + 8(v/4) +
// 4h + v%4, column l32 of the wave's block.  EPI 0 plain, 1 + residual,
// 2 / 3 silu(gate) * up as bf16 / f32 (NM 2: gate, up), 4 / 5 wide (NM 2: the
// two BN-column halves of one weight) plain / + residual.
template <int NM, int EPI, int BM>
__device__ __forceinline__ void store_tile(const f32x16 (&acc)[NM][ATile<BM>::MI], int m0, int n0, int wm, int wn,
                                           int h, int l32, int M, int N, int ldo, const float* __restrict__ residual,
                                           void* __restrict__ out) {
    constexpr int WM = ATile<BM>::WM, MI = ATile<BM>::MI;
    constexpr bool WIDE = EPI >= 4;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int row = m0 + wm * WM + 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
            const int col = n0 + wn * WN + l32;
            if constexpr (WIDE) {
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    if (row < M && col + m * BN < N) {
                        const size_t o = (size_t)row * ldo + col + m * BN;
                        if constexpr (EPI == 5) reinterpret_cast<float*>(out)[o] = acc[m][i][v] + residual[o];
                        else reinterpret_cast<float*>(out)[o] = acc[m][i][v];
                    }
                }
            } else if (row < M && col < N) {
                const size_t o = (size_t)row * ldo + col;
                if constexpr (EPI >= 2) {
                    const float g = acc[0][i][v], u = acc[NM - 1][i][v];
                    const float hv = silu_mul_fast(g, u);
                    if constexpr (EPI == 2) reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)bf16_bits(hv);
                    else reinterpret_cast<float*>(out)[o] = hv;
                } else if constexpr (EPI == 1) {
                    reinterpret_cast<float*>(out)[o] = acc[0][i][v] + residual[o];
                } else {
                    reinterpret_cast<float*>(out)[o] = acc[0][i][v];
                }
            }
        }
}

}  // namespace lds_gemm

// ldo: the row stride of out and residual (N, or the whole width when this
// launch covers a column range of a wider output).
template <int WT, int NM, int EPI, int BM>
__global__ __launch_bounds__(lds_gemm::NT) void mfma_qgemm_lds_kernel(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ qa, const __half* __restrict__ da,
    const uint8_t* __restrict__ qb, const __half* __restrict__ db, int M, int N, int K, int ldo,
    const float* __restrict__ residual, void* __restrict__ out) {
    using namespace lds_gemm;
    using S = Stage<WT, NM, BM>;
    constexpr int WM = ATile<BM>::WM, MI = ATile<BM>::MI, A_B = ATile<BM>::A_B, A_IT = ATile<BM>::A_IT;
    constexpr int CB = S::CB, RPI = 1024 / CB, CPR = CB / 16;   // rows / chunks per 1 KB load
    __shared__ __align__(16) uint8_t A0[A_B], A1[A_B], A2[A_B];
    __shared__ __align__(16) uint8_t W0[S::W_B], W1[S::W_B], W2[S::W_B];
    __shared__ __align__(16) uint8_t S0[S::S_B], S1[S::S_B], S2[S::S_B];
    const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    // EPI 4 / 5 (wide): one matrix, NM = 2 halves of a 2*BN-row tile (its rows
    // n0 .. n0 + 2*BN - 1), stored as is / plus the residual.
    constexpr bool WIDE = EPI >= 4;
    static_assert(!WIDE || NM == 2, "a wide tile is two halves");
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN * (WIDE ? 2 : 1);

    // Load sources of K step 0 (step k adds 128 B of A, 64 B of codes, 4 B of
    // scales) and the wave-uniform offsets of their destinations in a stage.
    // Rows past M or N load the last row (in bounds; never stored).
    const char* ga[A_IT];
    uint32_t la[A_IT];
#pragma unroll
    for (int it = 0; it < A_IT; ++it) {
        const int r0 = (it * 8 + wave) * 8, r = r0 + (lane >> 3), c = (lane & 7) ^ swz_a(r);
        ga[it] = reinterpret_cast<const char*>(A + (size_t)min(m0 + r, M - 1) * K + c * 8);
        la[it] = r0 * 128;
    }
    const char* gw[S::W_IT];
    uint32_t lw[S::W_IT];
    const size_t rowb = WT == VLRF_HIP_DT_Q8_0 ? (size_t)K : (size_t)K / 2;   // code bytes of a weight row
#pragma unroll
    for (int it = 0; it < S::W_IT; ++it) {
        const int li = min(it * 8 + wave, S::W_TI - 1);   // waves past the last load: never issued
        const int r0 = li * RPI, n = r0 + lane / CPR, c = (lane % CPR) ^ swz_w<WT>(n);
        const int gn = min(n0 + (WIDE ? n : n % BN), N - 1);
        gw[it] = reinterpret_cast<const char*>((n / BN ? qb : qa) + (size_t)gn * rowb + c * 16);
        lw[it] = r0 * CB;
    }
    const bool sload = wave < S::S_WAVES;
    const char* gs = nullptr;
    if (sload) {
        const int n = wave * 64 + lane, gn = min(n0 + (WIDE ? n : n % BN), N - 1);
        gs = reinterpret_cast<const char*>((n / BN ? db : da) + (size_t)gn * (K / 32));
    }
    const uint32_t bA[3] = {lds_addr(A0), lds_addr(A1), lds_addr(A2)};
    const uint32_t bW[3] = {lds_addr(W0), lds_addr(W1), lds_addr(W2)};
    const uint32_t bS[3] = {lds_addr(S0), lds_addr(S1), lds_addr(S2)};
    auto load = [&](int kt, int buf) {
#pragma unroll
        for (int it = 0; it < A_IT; ++it) dma16(ga[it] + (size_t)kt * 128, bA[buf] + la[it]);
#pragma unroll
        for (int it = 0; it < S::W_IT; ++it)
            if (it * 8 + wave < S::W_TI) dma16(gw[it] + (size_t)kt * CB, bW[buf] + lw[it]);
        if (sload) dma4(gs + (size_t)kt * 4, bS[buf] + wave * 256);
    };

    f32x16 acc[NM][MI];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int i = 0; i < MI; ++i) acc[m][i] = f32x16{};

    auto compute = [&](const uint8_t* As, const uint8_t* Ws, const uint8_t* Ss) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {             // 32-element block p of the step
            bf16x8 bfr[NM][2];
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const int n = m * BN + wn * WN + l32;
                const uint32_t s2 = *reinterpret_cast<const uint32_t*>(Ss + n * 4);
                const float sc = __half2float(__ushort_as_half((unsigned short)(p ? s2 >> 16 : s2 & 0xFFFFu)));
                if constexpr (WT == VLRF_HIP_DT_Q8_0) {
                    // Q8_0: lane half h takes code chunk 2p + h (16 codes), slice q its half q
                    const int c = 2 * p + h;
                    const uint4 u = *reinterpret_cast<const uint4*>(Ws + n * CB + 16 * (c ^ swz_w<WT>(n)));
                    const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                    for (int q = 0; q < 2; ++q)
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            bfr[m][q][e] = (__bf16)((float)(int8_t)(w4[2 * q + (e >> 2)] >> (8 * (e & 3))) * sc);
                } else {
                    // Q4_0: chunk p is the block; lane half h takes its bytes 8h..8h+7 (elements
                    // 16h..16h+15, byte j = element 2j low nibble, 2j+1 high), slice q 4 of them
                    const uint2 u = *reinterpret_cast<const uint2*>(Ws + n * CB + 16 * (p ^ swz_w<WT>(n)) + 8 * h);
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        const uint32_t wd = q ? u.y : u.x;
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            bfr[m][q][e] = (__bf16)((float)((int)((wd >> (4 * e)) & 0xFu) - 8) * sc);
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                bf16x8 afr[MI];
#pragma unroll
                for (int i = 0; i < MI; ++i) {
                    const int r = wm * WM + 32 * i + l32, c = 2 * (2 * p + h) + q;
                    afr[i] = *reinterpret_cast<const bf16x8*>(As + r * 128 + 16 * (c ^ swz_a(r)));
                }
#pragma unroll
                for (int m = 0; m < NM; ++m)
#pragma unroll
                    for (int i = 0; i < MI; ++i)
                        acc[m][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afr[i], bfr[m][q], acc[m][i], 0, 0, 0);
            }
        }
    };

    const int nk = K / 64;
    load(0, 0);
    if (nk > 1) load(1, 1);
    // Unrolled by the ring size so each step names its buffers statically.
    for (int kt = 0; kt < nk; kt += 3) {
#define VH_LDS_STEP(KT, AS, WS, SS, NEXT)                                                  \
        if (KT < nk) {                                                                     \
            if (KT + 1 < nk) __builtin_amdgcn_s_waitcnt(S::WAIT);                          \
            else __builtin_amdgcn_s_waitcnt(0);                                            \
            __builtin_amdgcn_s_barrier();                                                  \
            asm volatile("" ::: "memory");                                                 \
            if (KT + 2 < nk) load(KT + 2, NEXT);                                           \
            compute(AS, WS, SS);                                                           \
        }
        VH_LDS_STEP(kt, A0, W0, S0, 2)
        VH_LDS_STEP(kt + 1, A1, W1, S1, 0)
        VH_LDS_STEP(kt + 2, A2, W2, S2, 1)
#undef VH_LDS_STEP
    }

    lds_gemm::store_tile<NM, EPI, BM>(acc, m0, n0, wm, wn, h, l32, M, N, ldo, residual, out);
}

// ---- GEMM over bf16 weights ---------------------------------------------------
// out = A . W^T with W the weight's bf16 expansion (rows [N][K]): A tiles of BM
// rows and weight tiles of BN rows are staged in LDS by direct-to-LDS loads
// (BK elements = 2 BK bytes of a row per K step, the 16-byte chunks of row r
// swizzled by (r / 2) mod chunks, for both) and read straight into the MFMA
// operands, so no wave decodes codes.  WR x WC
// waves; a wave owns WM = BM / WR rows of A (MI MFMA tiles of 32) and
// WNR = BN / WC weight rows (NB blocks of 32).  SwiGLU tiles hold BN / 2 gate
// rows, then the same BN / 2 up rows; a wave's first NB / 2 blocks are gate
// rows and the others the matching up rows, so its outputs are
// WM x WNR / 2.  The ring holds as many stages as fit in the 160 KiB of LDS,
// at most four.
template <int BM_, int BN_, int WR_, int WC_, int BK_ = 64, int NSMAX = 4> struct BTile {
    static constexpr int BM = BM_, BN = BN_, WR = WR_, WC = WC_, BK = BK_;
    static constexpr int NW = WR * WC, NT = 64 * NW;
    static constexpr int WM = BM / WR, MI = WM / 32;
    static constexpr int WNR = BN / WC, NB = WNR / 32;
    static constexpr int RB = 2 * BK, CPR = RB / 16, RPL = 1024 / RB;   // row bytes, chunks, rows per 1 KiB
    static constexpr int NG = BK / 16;                                   // MFMA k groups per step
    static constexpr int A_B = BM * RB, W_B = BN * RB, ST = A_B + W_B;
    static constexpr int A_IT = BM / (RPL * NW), W_IT = BN / (RPL * NW);   // 1 KiB loads per wave and step
    static constexpr int NS = 160 * 1024 / ST < NSMAX ? 160 * 1024 / ST : NSMAX;
    static constexpr int LPS = A_IT + W_IT;
    static_assert(BK == 32 || BK == 64, "K step");
    static_assert(NS >= 2 && (NS - 1) * LPS < 64, "ring");
    static_assert(A_IT * RPL * NW == BM && W_IT * RPL * NW == BN && MI >= 1 && NB >= 2 && NB % 2 == 0, "tile shape");
    // Every row a lane reads is l32 mod 16, so all share one swizzle.
    static_assert(WM % 16 == 0 && WNR % 32 == 0, "row swizzle");
    __device__ static int swz(int r) { return (r >> 1) & (CPR - 1); }
};

// EPI: 0 plain, 1 + residual, 2 / 3 silu(gate) * up as bf16 / f32.
template <class T, int EPI>
__global__ __launch_bounds__(T::NT) void mfma_bgemm_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ ba, const uint16_t* __restrict__ bb, int M, int N,
    int K, int kl, int ldo, const float* __restrict__ residual, void* __restrict__ out) {
    using lds_gemm::dma16;
    using lds_gemm::lds_addr;
    constexpr int MI = T::MI, NB = T::NB, WM = T::WM, WNR = T::WNR, BN = T::BN;
    constexpr int A_B = T::A_B, ST = T::ST, NS = T::NS, LPS = T::LPS, NW = T::NW;
    constexpr int RB = T::RB, CPR = T::CPR, RPL = T::RPL, NG = T::NG;
    // EPI 6 / 7: raw partial sums of K slice blockIdx.z (plain / gate and up).
    constexpr bool SWIGLU = EPI == 2 || EPI == 3 || EPI == 7, PARTIAL = EPI >= 6;
    __shared__ __align__(16) uint8_t lds[NS * ST];
    const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / T::WC, wn = wave % T::WC;
    const int m0 = blockIdx.y * T::BM;
    const int n0 = blockIdx.x * (SWIGLU ? BN / 2 : BN);   // first output column
    const int k0 = blockIdx.z * kl;                        // this launch's K range: k0 .. k0 + kl (rows K long)

    // Sources of K step 0 (step k adds RB bytes) and destinations: wave w's
    // load `it` fills rows RPL (NW it + w) .. + RPL - 1 of the tile, lane l row
    // + l / CPR, its 16-byte chunk (l % CPR) ^ swizzle.  Rows past M or N load
    // the last row (in bounds; never stored).
    const char* ga[T::A_IT];
    const char* gb[T::W_IT];
#pragma unroll
    for (int it = 0; it < T::A_IT; ++it) {
        const int r = (it * NW + wave) * RPL + lane / CPR, c = (lane % CPR) ^ T::swz(r);
        ga[it] = reinterpret_cast<const char*>(A + (size_t)min(m0 + r, M - 1) * K + k0 + c * 8);
    }
#pragma unroll
    for (int it = 0; it < T::W_IT; ++it) {
        const int t = (it * NW + wave) * RPL + lane / CPR, c = (lane % CPR) ^ T::swz(t);
        const bool up = SWIGLU && t >= BN / 2;
        const int gn = min(n0 + (up ? t - BN / 2 : t), N - 1);
        gb[it] = reinterpret_cast<const char*>((up ? bb : ba) + (size_t)gn * K + k0 + c * 8);
    }
    const uint32_t base = lds_addr(lds);
    auto load = [&](int kt, int buf) {
        const uint32_t sa = base + buf * ST, sb = sa + A_B;
#pragma unroll
        for (int it = 0; it < T::A_IT; ++it) dma16(ga[it] + (size_t)kt * RB, sa + (it * NW + wave) * 1024);
#pragma unroll
        for (int it = 0; it < T::W_IT; ++it) dma16(gb[it] + (size_t)kt * RB, sb + (it * NW + wave) * 1024);
    };

    f32x16 acc[NB][MI];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < MI; ++i) acc[b][i] = f32x16{};

    // A K step is NG groups g = 2p + q of 16 elements (lane half h holds the
    // 16-byte chunk 2(2p + h) + q).  A wave's weight block b starts at tile
    // row wb + boff(b): wb = wn * WNR (plain) or wn * WNR / 2 (SwiGLU: gate
    // blocks, then the up blocks BN / 2 rows further).
    const int sw = T::swz(l32);
    const int a_off = (wm * WM + l32) * RB;
    const int b_off = A_B + ((SWIGLU ? wn * (WNR / 2) : wn * WNR) + l32) * RB;
    auto boff = [](int b) {
        return SWIGLU ? ((b < NB / 2 ? 0 : BN / 2) + 32 * (b % (NB / 2))) * RB : 32 * b * RB;
    };
    bf16x8 fa[2][MI], fb[2][NB];
    auto rd = [&](const uint8_t* St, int g, bf16x8 (&a)[MI], bf16x8 (&b)[NB]) {
        const int x = 16 * ((2 * (2 * (g >> 1) + h) + (g & 1)) ^ sw);
        const uint8_t* pa = St + a_off + x;
        const uint8_t* pb = St + b_off + x;
#pragma unroll
        for (int i = 0; i < MI; ++i) a[i] = *reinterpret_cast<const bf16x8*>(pa + i * 32 * RB);
#pragma unroll
        for (int j = 0; j < NB; ++j) b[j] = *reinterpret_cast<const bf16x8*>(pb + boff(j));
    };
    auto mm = [&](const bf16x8 (&a)[MI], const bf16x8 (&b)[NB]) {
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < MI; ++i)
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[j][i], 0, 0, 0);
    };
    // One phase: group g's MFMAs (operands in a / b) interleaved one for one
    // with the LDS reads of the next group into the other register set
    // (scheduling-group barriers pin the order; left alone, the compiler sinks
    // each read next to its use and reuses one register set, so every group's
    // read latency sits in series with its MFMAs).
    constexpr int NR = MI + NB, NMF = MI * NB;
    auto phase = [&](const bf16x8 (&a)[MI], const bf16x8 (&b)[NB], const uint8_t* St, int g, bf16x8 (&na)[MI],
                     bf16x8 (&nb)[NB]) {
        mm(a, b);
        rd(St, g, na, nb);
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);              // one MFMA
            if (i < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // one LDS read
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // The phase after a step's barrier: the same MFMAs and next-group reads,
    // with the refill of stage `buf` (step kt) spread over the MFMAs (PER
    // direct-to-LDS loads after each), so the loads leave under the MFMAs
    // instead of holding them up.
    constexpr int PER = (LPS + NMF - 1) / NMF;
    static_assert(NR <= NMF, "one read per MFMA");
    auto phase_refill = [&](const bf16x8 (&a)[MI], const bf16x8 (&b)[NB], const uint8_t* St, int g,
                            bf16x8 (&na)[MI], bf16x8 (&nb)[NB], int kt, int buf) {
        const int x = 16 * ((2 * (2 * (g >> 1) + h) + (g & 1)) ^ sw);
        const uint8_t* pa = St + a_off + x;
        const uint8_t* pb = St + b_off + x;
        const uint32_t sa = base + buf * ST, sb = sa + A_B;
#pragma unroll
        for (int j = 0, n = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < MI; ++i, ++n) {
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[j][i], 0, 0, 0);
                if (n < MI) na[n] = *reinterpret_cast<const bf16x8*>(pa + n * 32 * RB);
                else if (n < NR) nb[n - MI] = *reinterpret_cast<const bf16x8*>(pb + boff(n - MI));
#pragma unroll
                for (int l = n * PER; l < (n + 1) * PER && l < LPS; ++l) {
                    if (l < T::A_IT) dma16(ga[l] + (size_t)kt * RB, sa + (l * NW + wave) * 1024);
                    else dma16(gb[l - T::A_IT] + (size_t)kt * RB, sb + ((l - T::A_IT) * NW + wave) * 1024);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
    };

    // The ring: NS stages, stage k % NS holds step k.  A step's barrier sits
    // before its last group's MFMAs, whose operands are already in registers:
    // past it every wave has read the whole stage, so the stage is refilled
    // with step k + NS under those MFMAs, and the next step's first group is
    // read from LDS under them too.  Each load is issued NS - 1 steps before
    // the barrier that waits for it.  Every step issues its refill, with the
    // step index clamped to the last one (past the end a stage gets a copy of
    // the last step, which is never read, or, in the last step, of its own
    // bytes), so the count of loads in flight is the same at every wait.  No
    // MFMA sits under a branch (the accumulators would be copied at the
    // join): after the last step the first group of the next stage is read
    // all the same (in bounds, unused).
    constexpr int W_ALL = 0x70;                                                           // vmcnt(0) lgkmcnt(0)
    constexpr int W_IN = ((NS - 2) * LPS & 15) | (7 << 4) | (((NS - 2) * LPS >> 4) << 14);   // vmcnt((NS-2) LPS) lgkmcnt(0)
    constexpr int W_PRO = ((NS - 1) * LPS & 15) | (7 << 4) | (15 << 8) | (((NS - 1) * LPS >> 4) << 14);
    const int nk = kl / T::BK;
#pragma unroll
    for (int j = 0; j < NS; ++j) load(min(j, nk - 1), j);
    __builtin_amdgcn_s_waitcnt(W_PRO);   // step 0's loads in: the newer NS - 1 stages pending
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    rd(lds, 0, fa[0], fb[0]);
    __builtin_amdgcn_sched_barrier(0);
    int st = 0;   // stage of step k
    for (int k = 0; k < nk; ++k) {
        const uint8_t* St = lds + st * ST;
        const int sn = st + 1 == NS ? 0 : st + 1;
        phase(fa[0], fb[0], St, 1, fa[1], fb[1]);
        if constexpr (NG == 4) {
            phase(fa[1], fb[1], St, 2, fa[0], fb[0]);
            phase(fa[0], fb[0], St, 3, fa[1], fb[1]);
        }
        if (k + 1 < nk) {
            // step k + 1's loads are in (steps k + 2 .. k + NS - 1 may be pending)
            __builtin_amdgcn_s_waitcnt(W_IN);
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        }
        phase_refill(fa[1], fb[1], lds + sn * ST, 0, fa[0], fb[0], min(k + NS, nk - 1), st);
        st = sn;
    }
    __builtin_amdgcn_s_waitcnt(W_ALL);   // no load into LDS outlives the workgroup

    // Accumulator v of tile (j, i) holds row 32i + 8(v/4) + 4h + v%4 of the
    // wave's rows, weight row l32 of block j.
    if constexpr (PARTIAL) {
        // Slice z's sums at out + z M ldo: plain column n at n, SwiGLU gate at
        // n and up at N + n (ldo >= 2N).
        float* P = static_cast<float*>(out) + (size_t)blockIdx.z * M * ldo;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + wm * WM + 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
                if (row >= M) continue;
#pragma unroll
                for (int j = 0; j < (SWIGLU ? NB / 2 : NB); ++j) {
                    const int col = n0 + (SWIGLU ? wn * (WNR / 2) : wn * WNR) + 32 * j + l32;
                    if (col < N) {
                        P[(size_t)row * ldo + col] = acc[j][i][v];
                        if constexpr (SWIGLU) P[(size_t)row * ldo + N + col] = acc[j + NB / 2][i][v];
                    }
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int row = m0 + wm * WM + 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
            if (row >= M) continue;
            if constexpr (SWIGLU) {
#pragma unroll
                for (int j = 0; j < NB / 2; ++j) {
                    const int col = n0 + wn * (WNR / 2) + 32 * j + l32;
                    if (col < N) {
                        const size_t o = (size_t)row * ldo + col;
                        const float g = acc[j][i][v], u = acc[j + NB / 2][i][v];
                        const float hv = silu_mul_fast(g, u);
                        if constexpr (EPI == 2) reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)bf16_bits(hv);
                        else reinterpret_cast<float*>(out)[o] = hv;
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const int col = n0 + wn * WNR + 32 * j + l32;
                    if (col < N) {
                        const size_t o = (size_t)row * ldo + col;
                        if constexpr (EPI == 1) reinterpret_cast<float*>(out)[o] = acc[j][i][v] + residual[o];
                        else reinterpret_cast<float*>(out)[o] = acc[j][i][v];
                    }
                }
            }
        }
}

// One thread's codes of one K step (QB bytes: two or one 16-byte loads, or
// one 8-byte load) and the f16 scale of their block (zero-extended), loaded
// by inline assembly (see mfma_dqgemm_kernel).
typedef uint32_t dq_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t dq_u32x2 __attribute__((ext_vector_type(2)));
template <int QB>
struct DqCodes {
    static constexpr int NQ = QB >= 16 ? QB / 16 : 1;   // loads of the codes
    typedef typename std::conditional<(QB >= 16), dq_u32x4, dq_u32x2>::type V;
    V q[NQ];
    uint32_t d;
    __device__ __forceinline__ uint32_t word(int j) const {
        if constexpr (QB >= 16) return q[j >> 2][j & 3];
        else return q[0][j];
    }
    __device__ __forceinline__ void load(const uint8_t* p, const __half* ps) {
        if constexpr (QB >= 16) {
            asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(q[0]) : "v"(p));
            if constexpr (NQ == 2) asm volatile("global_load_dwordx4 %0, %1, off offset:16" : "=v"(q[NQ - 1]) : "v"(p));
        } else {
            asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(q[0]) : "v"(p));
        }
        asm volatile("global_load_ushort %0, %1, off" : "=v"(d) : "v"(ps));
    }
    // Wait until at most N vector-memory operations are pending; the
    // registers pass through the statement, so no use of them precedes it.
    template <int N>
    __device__ __forceinline__ void wait() {
        if constexpr (NQ == 2) asm volatile("s_waitcnt vmcnt(%3)" : "+v"(q[0]), "+v"(q[NQ - 1]), "+v"(d) : "n"(N));
        else asm volatile("s_waitcnt vmcnt(%2)" : "+v"(q[0]), "+v"(d) : "n"(N));
    }
};

// The same GEMM over Q8_0 / Q4_0 codes, dequantized into LDS tiles: A is staged by
// direct-to-LDS loads in a two-stage ring as above; the weight tile of each K
// step is loaded as codes into registers (thread t: row t / TPR, the codes
// of part t % TPR of the row's 64 and their f16 scale), decoded there to
// bf16(code * scale) -- the conversion of the bf16 expansion -- and written
// into one of two bf16 tile buffers laid out (and swizzled) as the ring's
// weight stage, so the MFMA phases are the bf16 kernel's, on the same
// operands in the same order: results equal the bf16-expansion GEMM's bit for
// bit.  Each code is decoded once per workgroup.
//
// Step k decodes tile k + 1 into the buffer step k - 1 read, under its first
// two groups' MFMAs (five to ten VALU instructions after each).  The codes of
// tile k + 1 were loaded at the end of step k - 2, with A of step k, into the
// register set (k + 1) % 2 (the loop is unrolled by two steps); the codes of
// step k + 3 follow A of step k + 2 at the end of step k.  The code loads are
// issued from inline assembly, so the compiler places no wait of its own for
// them (its count would hold up the A loads issued after them too): step k
// waits for its codes with A of step k + 1 and the codes of step k + 2 still
// in flight (vmcnt(A_IT + LW)), its barrier for A of step k + 1 with the
// codes of step k + 2 in flight (vmcnt(LW)).  With the decode under one
// group's MFMAs and the codes loaded one step later (the compiler's waits)
// the 8B layer ran 1.23 against 1.12 ms for the in-register decode; as here,
// 1.05 ms.
template <class T, int WT, int EPI, int NSA>
__global__ __launch_bounds__(T::NT) void mfma_dqgemm_kernel(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ qa, const __half* __restrict__ da,
    const uint8_t* __restrict__ qb, const __half* __restrict__ db, int M, int N, int K, int kl, int ldo,
    const float* __restrict__ residual, void* __restrict__ out) {
    using lds_gemm::dma16;
    using lds_gemm::lds_addr;
    constexpr int MI = T::MI, NB = T::NB, WM = T::WM, WNR = T::WNR, BN = T::BN;
    constexpr int A_B = T::A_B, NW = T::NW, RB = T::RB, CPR = T::CPR, RPL = T::RPL;
    constexpr int W_B = BN * RB;
    // EPI 6 / 7: raw partial sums of K slice blockIdx.z (plain / gate and up).
    constexpr bool SWIGLU = EPI == 2 || EPI == 3 || EPI == 7, PARTIAL = EPI >= 6;
    constexpr bool Q4 = WT == VLRF_HIP_DT_Q4_0;
    constexpr int TPR = T::NT / BN;              // threads per weight row
    constexpr int CPT = 64 / TPR;                // codes per thread and K step
    constexpr int NC = CPT / 8;                  // its 8-code chunks
    constexpr int RBQ = Q4 ? 32 : 64;            // code bytes of a row per K step
    constexpr int QB = Q4 ? CPT / 2 : CPT;       // code bytes per thread and K step
    using Codes = DqCodes<QB>;
    constexpr int LW = Codes::NQ + 1;            // loads per code set (the codes, the scale)
    static_assert(T::BK == 64 && T::NG == 4 && T::NT % BN == 0 && (TPR == 2 || TPR == 4), "code split");
    static_assert(NSA >= 2 && NSA * A_B + 2 * W_B <= 160 * 1024, "LDS");
    // Loads in flight at each wait (step j ends with A of step j + NSA, then
    // the codes of step j + 3): at step k's start the codes of step k + 1 are
    // in with the last step's pair pending; at its barrier A of step k + 1,
    // with the codes of step k + 1 (NSA > 2) and NSA - 2 later pairs pending;
    // at the prologue's barrier A of step 0, with everything after it pending.
    constexpr int VM_CODES = T::A_IT + LW;
    constexpr int VM_BAR = LW + (NSA - 2) * (T::A_IT + LW);
    constexpr int VM_PRO = (NSA - 1) * T::A_IT + 2 * LW;
    static_assert(VM_PRO < 16 && VM_BAR < 16, "vmcnt immediates in four bits");
    constexpr int W_BAR = VM_BAR | (7 << 4);                  // lgkmcnt(0) too: W writes and reads done
    constexpr int W_PRO = VM_PRO | (7 << 4) | (15 << 8);
    __shared__ __align__(16) uint8_t lds[NSA * A_B + 2 * W_B];
    const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / T::WC, wn = wave % T::WC;
    const int m0 = blockIdx.y * T::BM;
    const int n0 = blockIdx.x * (SWIGLU ? BN / 2 : BN);   // first output column
    const int k0 = blockIdx.z * kl;                        // this launch's K range: k0 .. k0 + kl (rows K long)

    const char* ga[T::A_IT];
#pragma unroll
    for (int it = 0; it < T::A_IT; ++it) {
        const int r = (it * NW + wave) * RPL + lane / CPR, c = (lane % CPR) ^ T::swz(r);
        ga[it] = reinterpret_cast<const char*>(A + (size_t)min(m0 + r, M - 1) * K + k0 + c * 8);
    }
    const uint32_t base = lds_addr(lds);
    auto load_a = [&](int kt, int buf) {
        const uint32_t sa = base + buf * A_B;
#pragma unroll
        for (int it = 0; it < T::A_IT; ++it) dma16(ga[it] + (size_t)kt * RB, sa + (it * NW + wave) * 1024);
    };
    // This thread's codes: tile row wr, part pt of each K step's 64 (CPT
    // codes from byte CPT pt; block 2 kt + CPT pt / 32 of the row).  A wave
    // decodes 64 / TPR rows; lanes 8m .. 8m + 7, whose 16-byte LDS writes go
    // out together, take rows (m & 1) + 2j + (16 / TPR)(m >> 1) of them, j <
    // 8 / TPR: rows of distinct swizzles, so the eight writes of a chunk
    // fill the eight 16-byte slots of a 128-byte row (rows t / TPR: two-way
    // bank conflicts, rows 2i and 2i + 1 sharing a swizzle).
    const int pt = lane % TPR, m8 = lane >> 3;
    const int wr = wave * (64 / TPR) + (m8 & 1) + 2 * ((lane / TPR) % (8 / TPR)) + (16 / TPR) * (m8 >> 1);
    const bool wup = SWIGLU && wr >= BN / 2;
    const int gnr = min(n0 + (wup ? wr - BN / 2 : wr), N - 1);
    const uint8_t* qrow = (wup ? qb : qa) + (size_t)gnr * (K / 64 * RBQ) + k0 / 64 * RBQ + QB * pt;
    const __half* drow = (wup ? db : da) + (size_t)gnr * (K / 32) + k0 / 32 + CPT * pt / 32;
    int woff[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) woff[c] = NSA * A_B + wr * RB + 16 * ((NC * pt + c) ^ T::swz(wr));
    // Register sets of the codes (two, alternating by step).
    Codes cq0, cq1;
    auto load_w = [&](int kt, Codes& q) { q.load(qrow + (size_t)kt * RBQ, drow + 2 * kt); };
    // Chunks c0 .. c1 - 1 (8 codes each) of the thread's codes -> bf16 (the
    // expansion's conversion), into W buffer wb.  Q8_0: signed bytes times
    // the scale; Q4_0 (element 2b + i in nibble i of byte b): (n - 8) / 16
    // (one conversion a code, gemv::s4f) times 16 x the scale, exact, so the
    // same bf16 as (n - 8) x scale.
    auto store_w = [&](const Codes& q, int wb, int c0, int c1) {
        const float sc = __half2float(__ushort_as_half((unsigned short)q.d)) * (Q4 ? 16.f : 1.f);
#pragma unroll
        for (int c = c0; c < c1; ++c) {
            bf16x8 v;
            if constexpr (Q4) {
                const uint32_t x = q.word(c) ^ 0x88888888u, x4 = x >> 4;
                v[0] = (__bf16)(gemv::s4f<0>(x) * sc);
                v[1] = (__bf16)(gemv::s4f<0>(x4) * sc);
                v[2] = (__bf16)(gemv::s4f<1>(x) * sc);
                v[3] = (__bf16)(gemv::s4f<1>(x4) * sc);
                v[4] = (__bf16)(gemv::s4f<2>(x) * sc);
                v[5] = (__bf16)(gemv::s4f<2>(x4) * sc);
                v[6] = (__bf16)(gemv::s4f<3>(x) * sc);
                v[7] = (__bf16)(gemv::s4f<3>(x4) * sc);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = (__bf16)((float)(int8_t)(q.word(2 * c + (e >> 2)) >> (8 * (e & 3))) * sc);
            }
            *reinterpret_cast<bf16x8*>(lds + woff[c] + wb * W_B) = v;
        }
    };

    f32x16 acc[NB][MI];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < MI; ++i) acc[b][i] = f32x16{};

    const int sw = T::swz(l32);
    const int a_off = (wm * WM + l32) * RB;
    const int b_off = NSA * A_B + ((SWIGLU ? wn * (WNR / 2) : wn * WNR) + l32) * RB;
    auto boff = [](int b) {
        return SWIGLU ? ((b < NB / 2 ? 0 : BN / 2) + 32 * (b % (NB / 2))) * RB : 32 * b * RB;
    };
    bf16x8 fa[2][MI], fb[2][NB];
    // group g of the step in A stage sa, W buffer wb
    auto rd = [&](int sa, int wb, int g, bf16x8 (&a)[MI], bf16x8 (&b)[NB]) {
        const int x = 16 * ((2 * (2 * (g >> 1) + h) + (g & 1)) ^ sw);
        const uint8_t* pa = lds + sa * A_B + a_off + x;
        const uint8_t* pb = lds + wb * W_B + b_off + x;
#pragma unroll
        for (int i = 0; i < MI; ++i) a[i] = *reinterpret_cast<const bf16x8*>(pa + i * 32 * RB);
#pragma unroll
        for (int j = 0; j < NB; ++j) b[j] = *reinterpret_cast<const bf16x8*>(pb + boff(j));
    };
    auto mm = [&](const bf16x8 (&a)[MI], const bf16x8 (&b)[NB]) {
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < MI; ++i)
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[j][i], 0, 0, 0);
    };
    constexpr int NR = MI + NB, NMF = MI * NB;
    auto phase = [&](const bf16x8 (&a)[MI], const bf16x8 (&b)[NB], int sa, int wb, int g, bf16x8 (&na)[MI],
                     bf16x8 (&nb)[NB]) {
        mm(a, b);
        rd(sa, wb, g, na, nb);
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);              // one MFMA
            if (i < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // one LDS read
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // A phase with chunks c0 .. c1 - 1 of the next tile's decode spread over its MFMAs.
    constexpr int DQ_V = (20 * (NC / 2) + NMF - 1) / NMF;   // decode VALU per MFMA (about 20 per chunk)
    auto phase_dq = [&](const bf16x8 (&a)[MI], const bf16x8 (&b)[NB], int sa, int wb, int g, bf16x8 (&na)[MI],
                        bf16x8 (&nb)[NB], const Codes& q, int wnext, int c0, int c1) {
        mm(a, b);
        rd(sa, wb, g, na, nb);
        store_w(q, wnext, c0, c1);
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);              // one MFMA
            if (i < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // one LDS read
            __builtin_amdgcn_sched_group_barrier(0x002, DQ_V, 0);           // decode VALU
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // After a step's barrier: the last group's MFMAs, the next step's first
    // reads, and the refill (A of step kta into stage sa_fill, spread over the
    // MFMAs, then the codes of step ktw into the register set given).
    constexpr int PER = (T::A_IT + NMF - 1) / NMF;
    auto phase_refill = [&](const bf16x8 (&a)[MI], const bf16x8 (&b)[NB], int sa, int wb, bf16x8 (&na)[MI],
                            bf16x8 (&nb)[NB], int kta, int sa_fill, int ktw, Codes& q) {
        const int x = 16 * ((2 * h) ^ sw);
        const uint8_t* pa = lds + sa * A_B + a_off + x;
        const uint8_t* pb = lds + wb * W_B + b_off + x;
        const uint32_t sfa = base + sa_fill * A_B;
#pragma unroll
        for (int j = 0, n = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < MI; ++i, ++n) {
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[j][i], 0, 0, 0);
                if (n < MI) na[n] = *reinterpret_cast<const bf16x8*>(pa + n * 32 * RB);
                else if (n < NR) nb[n - MI] = *reinterpret_cast<const bf16x8*>(pb + boff(n - MI));
#pragma unroll
                for (int l = n * PER; l < (n + 1) * PER && l < T::A_IT; ++l)
                    dma16(ga[l] + (size_t)kta * RB, sfa + (l * NW + wave) * 1024);
                if (n == NMF - 1) load_w(ktw, q);
                __builtin_amdgcn_sched_barrier(0);
            }
        // Reads beyond one per MFMA (one 32-row block per wave: MI + NB > MI NB).
#pragma unroll
        for (int n = NMF; n < NR; ++n) {
            if (n < MI) na[n] = *reinterpret_cast<const bf16x8*>(pa + n * 32 * RB);
            else nb[n - MI] = *reinterpret_cast<const bf16x8*>(pb + boff(n - MI));
        }
    };

    // Prologue, so that every step finds the same loads in flight: codes 0
    // (decoded into W buffer 0), then A 0 .. NSA - 3, and the pairs (A
    // NSA - 2, codes 1), (A NSA - 1, codes 2).
    const int nk = kl / T::BK;
    load_w(0, cq0);
    cq0.template wait<0>();
    store_w(cq0, 0, 0, NC);
#pragma unroll
    for (int j = 0; j < NSA - 2; ++j) load_a(min(j, nk - 1), j);
    load_a(min(NSA - 2, nk - 1), NSA - 2);
    load_w(min(1, nk - 1), cq1);
    load_a(min(NSA - 1, nk - 1), NSA - 1);
    load_w(min(2, nk - 1), cq0);
    __builtin_amdgcn_s_waitcnt(W_PRO);
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0) alone: the tile's LDS writes done
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    rd(0, 0, 0, fa[0], fb[0]);
    __builtin_amdgcn_sched_barrier(0);

    // Step k: A stage k % NSA (st), W buffer k % 2; decodes the codes of step
    // k + 1 (set qn) into W buffer (k + 1) % 2; set qn then takes the codes of
    // step k + 3, A stage st A of step k + NSA.
    int st = 0;
    auto step = [&](int k, Codes& qn) {
        const int s = k & 1, s1 = s ^ 1, sn = st + 1 == NSA ? 0 : st + 1;
        qn.template wait<VM_CODES>();
        phase_dq(fa[0], fb[0], st, s, 1, fa[1], fb[1], qn, s1, 0, NC / 2);
        phase_dq(fa[1], fb[1], st, s, 2, fa[0], fb[0], qn, s1, NC / 2, NC);
        phase(fa[0], fb[0], st, s, 3, fa[1], fb[1]);
        __builtin_amdgcn_s_waitcnt(W_BAR);   // A of step k + 1 in; W writes and reads done
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        phase_refill(fa[1], fb[1], sn, s1, fa[0], fb[0], min(k + NSA, nk - 1), st, min(k + 3, nk - 1), qn);
        st = sn;
    };
    for (int k = 0; k < nk; k += 2) {
        step(k, cq1);
        step(k + 1, cq0);
    }
    cq0.template wait<0>();   // nothing outlives the workgroup
    cq1.template wait<0>();

    // Accumulator v of tile (j, i) holds row 32i + 8(v/4) + 4h + v%4 of the
    // wave's rows, weight row l32 of block j.
    if constexpr (PARTIAL) {
        // Slice z's sums at out + z M ldo: plain column n at n, SwiGLU gate at
        // n and up at N + n (ldo >= 2N).
        float* P = static_cast<float*>(out) + (size_t)blockIdx.z * M * ldo;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + wm * WM + 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
                if (row >= M) continue;
#pragma unroll
                for (int j = 0; j < (SWIGLU ? NB / 2 : NB); ++j) {
                    const int col = n0 + (SWIGLU ? wn * (WNR / 2) : wn * WNR) + 32 * j + l32;
                    if (col < N) {
                        P[(size_t)row * ldo + col] = acc[j][i][v];
                        if constexpr (SWIGLU) P[(size_t)row * ldo + N + col] = acc[j + NB / 2][i][v];
                    }
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int row = m0 + wm * WM + 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
            if (row >= M) continue;
            if constexpr (SWIGLU) {
#pragma unroll
                for (int j = 0; j < NB / 2; ++j) {
                    const int col = n0 + wn * (WNR / 2) + 32 * j + l32;
                    if (col < N) {
                        const size_t o = (size_t)row * ldo + col;
                        const float g = acc[j][i][v], u = acc[j + NB / 2][i][v];
                        const float hv = silu_mul_fast(g, u);
                        if constexpr (EPI == 2) reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)bf16_bits(hv);
                        else reinterpret_cast<float*>(out)[o] = hv;
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const int col = n0 + wn * WNR + 32 * j + l32;
                    if (col < N) {
                        const size_t o = (size_t)row * ldo + col;
                        if constexpr (EPI == 1) reinterpret_cast<float*>(out)[o] = acc[j][i][v] + residual[o];
                        else reinterpret_cast<float*>(out)[o] = acc[j][i][v];
                    }
                }
            }
        }
}

// bf16 expansion of Q8_0 / Q4_0 rows, a quarter block (8 elements) per
// thread, so a wave's code loads and 16-byte stores are each one contiguous
// run: element = bf16(code * scale) with the conversion the GEMM's in-register
// decode uses, so both GEMM forms multiply identical operands.  Q8_0 code e
// is element e; Q4_0 byte j holds elements 2j (low nibble) and 2j + 1 (high),
// both minus 8 (the oracle's orc_dequant_q4_0).
template <int WT>
__global__ __launch_bounds__(256) void expand_bf16_kernel(const uint8_t* __restrict__ q, const __half* __restrict__ d,
                                                          uint16_t* __restrict__ out, size_t nparts) {
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;   // elements 8t .. 8t + 7, of block t / 4
    if (t >= nparts) return;
    const float sc = __half2float(d[t >> 2]);
    int e[8];
    if constexpr (WT == VLRF_HIP_DT_Q8_0) {
        const uint2 u = *reinterpret_cast<const uint2*>(q + t * 8);   // block t / 4, codes 8 (t % 4) ..
        const uint32_t w[2] = {u.x, u.y};
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = (int8_t)(w[i >> 2] >> (8 * (i & 3)));
    } else {
        const uint32_t u = *reinterpret_cast<const uint32_t*>(q + t * 4);   // block t / 4, bytes 4 (t % 4) ..
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = (int)((u >> (4 * i)) & 0xFu) - 8;
    }
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const __bf16 lo = (__bf16)((float)e[2 * i] * sc), hi = (__bf16)((float)e[2 * i + 1] * sc);
        o[i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
    *reinterpret_cast<uint4*>(out + t * 8) = make_uint4(o[0], o[1], o[2], o[3]);
}

// Rows [n0, n0 + nn) of the weights (columns of the output), BM-row tiles of A.
template <int WT, int EPI, int BM>
void launch_lds_wt(hipStream_t s, const uint16_t* a, const DevWeight& w0, const DevWeight* w1, int M, int n0,
                   int nn, const float* residual, void* out) {
    constexpr int TN = lds_gemm::BN * (EPI >= 4 ? 2 : 1);
    const dim3 grid((nn + TN - 1) / TN, (M + BM - 1) / BM);
    const size_t rowb = WT == VLRF_HIP_DT_Q8_0 ? (size_t)w0.K : (size_t)w0.K / 2;
    const uint8_t* qa = w0.q + (size_t)n0 * rowb;
    const __half* da = w0.d + (size_t)n0 * (w0.K / 32);
    const float* res = residual ? residual + n0 : nullptr;
    void* o = EPI == 2 ? (void*)(static_cast<uint16_t*>(out) + n0) : (void*)(static_cast<float*>(out) + n0);
    if constexpr (EPI >= 4)   // wide: both halves from the one matrix
        hipLaunchKernelGGL((mfma_qgemm_lds_kernel<WT, 2, EPI, BM>), grid, dim3(lds_gemm::NT), 0, s, a, qa, da, qa, da,
                           M, nn, w0.K, w0.N, res, o);
    else if constexpr (EPI >= 2)   // SwiGLU: gate and up tiles together
        hipLaunchKernelGGL((mfma_qgemm_lds_kernel<WT, 2, EPI, BM>), grid, dim3(lds_gemm::NT), 0, s, a, qa, da,
                           w1->q + (size_t)n0 * rowb, w1->d + (size_t)n0 * (w0.K / 32), M, nn, w0.K, w0.N, res, o);
    else
        hipLaunchKernelGGL((mfma_qgemm_lds_kernel<WT, 1, EPI, BM>), grid, dim3(lds_gemm::NT), 0, s, a, qa, da, qa, da,
                           M, nn, w0.K, w0.N, res, o);
}

// Over the weights' bf16 expansions: columns [n0, n0 + nn) of the output.
template <class T, int EPI>
void launch_bgemm(hipStream_t s, const uint16_t* a, const DevWeight& w0, const DevWeight* w1, int M, int n0, int nn,
                  const float* residual, void* out) {
    constexpr int TN = EPI >= 2 ? T::BN / 2 : T::BN;   // output columns per tile
    const dim3 grid((nn + TN - 1) / TN, (M + T::BM - 1) / T::BM);
    const uint16_t* ba = w0.bf + (size_t)n0 * w0.K;
    const uint16_t* bb = EPI >= 2 ? w1->bf + (size_t)n0 * w0.K : ba;
    const float* res = residual ? residual + n0 : nullptr;
    void* o = EPI == 2 ? (void*)(static_cast<uint16_t*>(out) + n0) : (void*)(static_cast<float*>(out) + n0);
    hipLaunchKernelGGL((mfma_bgemm_kernel<T, EPI>), grid, dim3(T::NT), 0, s, a, ba, bb, M, nn, w0.K, w0.K, w0.N, res, o);
}

template <int EPI, int BM>
void launch_lds(hipStream_t s, const uint16_t* a, const DevWeight& w0, const DevWeight* w1, int M, int n0, int nn,
                const float* residual, void* out) {
    if (w0.dtype == VLRF_HIP_DT_Q8_0) launch_lds_wt<VLRF_HIP_DT_Q8_0, EPI, BM>(s, a, w0, w1, M, n0, nn, residual, out);
    else launch_lds_wt<VLRF_HIP_DT_Q4_0, EPI, BM>(s, a, w0, w1, M, n0, nn, residual, out);
}

// Tile plan of an M > 128 GEMM on the lds ring (one workgroup per CU: the
// ring takes 99-147 KiB of LDS).  Plain and residual GEMMs take 256 x 256
// tiles (two 128-row halves of the weight: twice the MFMA work per staged
// byte) where they still give at least 3/4 of a round of workgroups, else
// 256 x 128 (O and down of the 8B layer at T = 2048 ran 1.335 against 1.166 ms
// per layer wide, and slower again as 128 x 256 tiles, whose waves decode
// twice the codes per MFMA).  A last round of 256-row tiles at most half full
// (SwiGLU's 896 tiles at T = 2048) is run instead as 128-row tiles over its
// columns: twice as many, each with half the MFMA work but the same decode
// work per wave, so the round takes more than half as long (8B layer at
// T = 2048: 1.1667 -> 1.1555 ms, same-box A/B).
struct LdsPlan {
    bool wide = false;   // 2 x BN weight rows per tile (plain / residual GEMMs)
    int n_split = 0;     // > 0: columns [n_split, N) in a second launch of 128-row tiles
};

LdsPlan lds_plan(int M, int N, bool swiglu, int cus) {
    LdsPlan p;
    const int mt = (M + 255) / 256;
    const long wide_groups = (long)((N + 2 * lds_gemm::BN - 1) / (2 * lds_gemm::BN)) * mt;
    p.wide = !swiglu && 4 * wide_groups >= 3L * cus;
    const int tn = p.wide ? 2 * lds_gemm::BN : lds_gemm::BN;   // weight rows per tile (of each matrix)
    const int nt = (N + tn - 1) / tn;
    const long full = (long)nt * mt, rem = full % cus;
    if (N % tn == 0 && full >= cus && rem > 0 && 2 * rem <= cus && rem % mt == 0)
        p.n_split = (int)((nt - rem / mt) * tn);
    return p;
}

// Runs a plan: EPI of the narrow form (the wide form is EPI + 4 for 0 / 1).
template <int EPI>
void launch_lds_plan(hipStream_t s, const LdsPlan& p, const uint16_t* a, const DevWeight& w0, const DevWeight* w1,
                     int M, const float* residual, void* out) {
    constexpr int EW = EPI <= 1 ? EPI + 4 : EPI;
    const int n1 = p.n_split ? p.n_split : w0.N;
    if (p.wide) launch_lds<EW, 256>(s, a, w0, w1, M, 0, n1, residual, out);
    else launch_lds<EPI, 256>(s, a, w0, w1, M, 0, n1, residual, out);
    if (p.n_split) {
        if (p.wide) launch_lds<EW, 128>(s, a, w0, w1, M, p.n_split, w0.N - p.n_split, residual, out);
        else launch_lds<EPI, 128>(s, a, w0, w1, M, p.n_split, w0.N - p.n_split, residual, out);
    }
}

int lds_cus();

// Tile plan of the GEMM over bf16 expansions, on the rule of lds_plan: 256 x 256
// tiles (8 waves of 128 x 64) where they give at least 3/4 of a round of
// workgroups, else 128 x 256 tiles (8 waves of 64 x 64; no decode, so 128-row
// tiles cost no extra work per MFMA); a last round of 256-row tiles at most
// half full runs as 128-row tiles over its columns.  Measured at the 8B layer
// (T = 2048), slower than this plan: four waves per workgroup with larger
// wave tiles (64 x 128, 128 x 64, 128 x 128; one wave per SIMD) by 12-29%;
// 32-element K steps (a ring four stages deep, twice the barriers) by 4-11%;
// two workgroups per CU (128 x 128 or 64 x 256 tiles of 4 waves, two-stage
// rings of 64-80 KiB, so one workgroup's barrier leaves the other computing)
// by 8-25%; a third weight-tile stage for the 256 x 256 tiles (rings of two A
// and three weight stages, all 160 KiB, weight loads leading by two steps) by
// 0-2%; for the residual GEMMs at M = 2048, N = 4096 (O and down, one round of
// 128 x 256 tiles), 256 x 256 tiles split two ways over K (256 workgroups, the
// second of a tile's halves to finish adding the first's partial sums, read
// back through agent-coherent loads) by 3-4% for the layer: O 134 against
// 94 us, down 316 against 281 us (with agent-scope fences in the join
// instead, which write back and invalidate the XCD's L2 under the workgroups
// still computing: 207 and 382 us); an XCD-aware tile order (each XCD a run
// of tiles, M fastest) and a ring of five 32-element half-steps (half the
// loads leading by two steps) by 2-6% (stand-alone SwiGLU GEMM, cycle counts).
template <class BBig, class BHalf, int EPI>
void launch_bgemm_plan_t(hipStream_t s, const uint16_t* a, const DevWeight& w0, const DevWeight* w1, int M,
                         const float* residual, void* out) {
    const int cus = lds_cus(), N = w0.N;
    const int tn = EPI >= 2 ? BBig::BN / 2 : BBig::BN;   // output columns per tile
    const int mt = (M + BBig::BM - 1) / BBig::BM, nt = (N + tn - 1) / tn;
    const long full = (long)mt * nt, rem = full % cus;
    if (EPI < 2 && 4 * full < 3L * cus) {
        launch_bgemm<BHalf, EPI>(s, a, w0, w1, M, 0, N, residual, out);
        return;
    }
    int n_split = N;
    if (N % tn == 0 && full >= cus && rem > 0 && 2 * rem <= cus && rem % mt == 0) n_split = (int)((nt - rem / mt) * tn);
    launch_bgemm<BBig, EPI>(s, a, w0, w1, M, 0, n_split, residual, out);
    if (n_split < N) launch_bgemm<BHalf, EPI>(s, a, w0, w1, M, n_split, N - n_split, residual, out);
}

template <int EPI>
void launch_bgemm_plan(hipStream_t s, const uint16_t* a, const DevWeight& w0, const DevWeight* w1, int M,
                       const float* residual, void* out) {
    launch_bgemm_plan_t<BTile<256, 256, 2, 4>, BTile<128, 256, 2, 4>, EPI>(s, a, w0, w1, M, residual, out);
}

// Over Q8_0 codes decoded into LDS tiles (mfma_dqgemm_kernel): columns [n0, n0 + nn).
template <class T, int EPI>
void launch_dqgemm(hipStream_t s, const uint16_t* a, const DevWeight& w0, const DevWeight* w1, int M, int n0,
                   int nn, const float* residual, void* out) {
    constexpr int TN = EPI >= 2 ? T::BN / 2 : T::BN;
    const dim3 grid((nn + TN - 1) / TN, (M + T::BM - 1) / T::BM);
    const size_t nd = (size_t)n0 * (w0.K / 32);
    const size_t rowb = w0.dtype == VLRF_HIP_DT_Q8_0 ? (size_t)w0.K : (size_t)w0.K / 2;
    const uint8_t* qa = w0.q + (size_t)n0 * rowb;
    const __half* da = w0.d + nd;
    const uint8_t* qb = EPI >= 2 ? w1->q + (size_t)n0 * rowb : qa;
    const __half* db = EPI >= 2 ? w1->d + nd : da;
    const float* res = residual ? residual + n0 : nullptr;
    void* o = EPI == 2 ? (void*)(static_cast<uint16_t*>(out) + n0) : (void*)(static_cast<float*>(out) + n0);
    // Two A stages: three (the 128-row tiles in 112 KiB, the 256-row ones in
    // 160 KiB) ran the 8B layer 0.5-1% slower.
    constexpr int NSA = 2;
    if (w0.dtype == VLRF_HIP_DT_Q8_0)
        hipLaunchKernelGGL((mfma_dqgemm_kernel<T, VLRF_HIP_DT_Q8_0, EPI, NSA>), grid, dim3(T::NT), 0, s, a, qa, da, qb, db,
                           M, nn, w0.K, w0.K, w0.N, res, o);
    else
        hipLaunchKernelGGL((mfma_dqgemm_kernel<T, VLRF_HIP_DT_Q4_0, EPI, NSA>), grid, dim3(T::NT), 0, s, a, qa, da, qb, db,
                           M, nn, w0.K, w0.K, w0.N, res, o);
}

// Q8_0 / Q4_0 weights with K a multiple of 128 (whole 64-element K-step pairs).
bool dqgemm_supported(const DevWeight& w) {
    const char* e = getenv("VLRF_HIP_PREFILL_DQ");   // "0": the in-register decode instead
    return !(e && e[0] == '0') && (w.dtype == VLRF_HIP_DT_Q8_0 || w.dtype == VLRF_HIP_DT_Q4_0) && w.K % 128 == 0;
}

// The tile plan of launch_bgemm_plan_t over codes, with half tiles of half
// the columns rather than half the rows.
template <int EPI>
void launch_dqgemm_plan(hipStream_t s, const uint16_t* a, const DevWeight& w0, const DevWeight* w1, int M,
                        const float* residual, void* out) {
    // 512 x 128 tiles (the A ring and two weight tiles in 160 KiB; half the
    // decode per MFMA, twice the A bytes) ran the 8B layer 0.6% slower.
    using BBig = BTile<256, 256, 2, 4>;
    // Half tiles of 256 x 128 (8 waves of 64 x 64): half the decode per
    // workgroup and step of 128 x 256 tiles, the same MFMA work (8B layer at
    // T = 2048: 1.081 against 1.053 ms with 128 x 256 half tiles).
    using BHalf = BTile<256, 128, 4, 2>;
    const int cus = lds_cus(), N = w0.N;
    const int tn = EPI >= 2 ? BBig::BN / 2 : BBig::BN;
    const int mt = (M + BBig::BM - 1) / BBig::BM, nt = (N + tn - 1) / tn;
    const long full = (long)mt * nt, rem = full % cus;
    if (EPI < 2 && 4 * full < 3L * cus) {
        launch_dqgemm<BHalf, EPI>(s, a, w0, w1, M, 0, N, residual, out);
        return;
    }
    int n_split = N;
    if (N % tn == 0 && full >= cus && rem > 0 && 2 * rem <= cus && rem % mt == 0) n_split = (int)((nt - rem / mt) * tn);
    launch_dqgemm<BBig, EPI>(s, a, w0, w1, M, 0, n_split, residual, out);
    if (n_split < N) launch_dqgemm<BHalf, EPI>(s, a, w0, w1, M, n_split, N - n_split, residual, out);
}

// ---- 17 <= M <= 128: mfma_dqgemm_kernel with K split over blockIdx.z ------------
// One tile row (64 x 256 tiles for M <= 64, 128 x 128 above) leaves a GEMM of
// these M with one workgroup per 128-256 weight rows: 16-48 of the 256 CUs at
// the 1.1B and 8B shapes, each streaming its rows' whole K.  The K steps are
// split into S contiguous slices instead, each slice's f32 sums written to a
// partial buffer ([S][M][N], SwiGLU [S][M][2N]: gate, then up), and
// splitk_reduce_kernel adds the slices in order (the same sum on every run)
// and applies the epilogue.  S is the largest divisor of K / 128 whose
// workgroups fit one round of the CUs and whose slices keep at least 8 K
// steps (the pipeline's prologue and the partial stores are per slice; 8B
// QKV at M = 128, 48 column tiles: 4 slices 26.8 us, 8 slices 1.5 rounds
// 30.2 us).  Measured while S was the smallest divisor reaching a round:
// summed over M = 17, 32, 64, 65, 100, 128 at four 1.1B / 8B shapes (Q8_0),
// 689 us against 693 with 4 steps, 703 with 2, and 765 aiming at two
// workgroups per CU; capping S further so that the partials (written and
// read back, mostly from the caches) move no more bytes than the weight cost
// 6% over M = 17, 64, 128 and both dtypes (706 against 663 us).

// out[r][n] = sum over z of P[z][r][n] (EPI 0), + residual (1, in place
// allowed), silu(sum of gate) * (sum of up) as bf16 (2) or f32 (3).
// N % 4 == 0: four columns a thread (VEC), the same sums element by element.
template <int EPI>
__global__ __launch_bounds__(256) void splitk_reduce4_kernel(const float* __restrict__ P, int S, int M, int N,
                                                             int ldp, const float* residual, void* out) {
    const size_t idx = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (idx >= (size_t)M * N) return;
    const int row = (int)(idx / N), col = (int)(idx % N);
    const size_t zs = (size_t)M * ldp;
    const float* p = P + (size_t)row * ldp + col;
    float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int z = 0; z < S; ++z) {
        const float4 t = *reinterpret_cast<const float4*>(p + z * zs);
        g.x += t.x; g.y += t.y; g.z += t.z; g.w += t.w;
    }
    if constexpr (EPI >= 2) {
        float4 u = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int z = 0; z < S; ++z) {
            const float4 t = *reinterpret_cast<const float4*>(p + z * zs + N);
            u.x += t.x; u.y += t.y; u.z += t.z; u.w += t.w;
        }
        const float h0 = silu_mul_fast(g.x, u.x), h1 = silu_mul_fast(g.y, u.y);
        const float h2 = silu_mul_fast(g.z, u.z), h3 = silu_mul_fast(g.w, u.w);
        if constexpr (EPI == 2)
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + idx) =
                make_uint2(bf16_bits(h0) | (bf16_bits(h1) << 16), bf16_bits(h2) | (bf16_bits(h3) << 16));
        else
            *reinterpret_cast<float4*>(static_cast<float*>(out) + idx) = make_float4(h0, h1, h2, h3);
    } else {
        if constexpr (EPI == 1) {
            const float4 r = *reinterpret_cast<const float4*>(residual + idx);
            g.x += r.x; g.y += r.y; g.z += r.z; g.w += r.w;
        }
        *reinterpret_cast<float4*>(static_cast<float*>(out) + idx) = g;
    }
}

template <int EPI>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ P, int S, int M, int N,
                                                            int ldp, const float* residual, void* out) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)M * N) return;
    const int row = (int)(idx / N), col = (int)(idx % N);
    const size_t zs = (size_t)M * ldp;
    const float* p = P + (size_t)row * ldp + col;
    float g = 0.f;
    for (int z = 0; z < S; ++z) g += p[z * zs];
    if constexpr (EPI >= 2) {
        float u = 0.f;
        for (int z = 0; z < S; ++z) u += p[z * zs + N];
        const float hv = silu_mul_fast(g, u);
        if constexpr (EPI == 2) static_cast<uint16_t*>(out)[idx] = (uint16_t)bf16_bits(hv);
        else static_cast<float*>(out)[idx] = hv;
    } else if constexpr (EPI == 1) {
        static_cast<float*>(out)[idx] = g + residual[idx];
    } else {
        static_cast<float*>(out)[idx] = g;
    }
}

template <int EPI>
void launch_splitk_reduce(hipStream_t s, const float* part, int S, int M, int N, int ldp, const float* residual,
                          void* out) {
    const size_t n = (size_t)M * N;
    if (N % 4 == 0)
        hipLaunchKernelGGL((splitk_reduce4_kernel<EPI>), dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, s, part, S,
                           M, N, ldp, residual, out);
    else
        hipLaunchKernelGGL((splitk_reduce_kernel<EPI>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, part, S, M,
                           N, ldp, residual, out);
}

using SplitTile64 = BTile<64, 256, 2, 4>;     // M <= 64: 8 waves of 32 x 64
using SplitTile128 = BTile<128, 128, 4, 2>;   // 65 <= M <= 128: 8 waves of 32 x 64

int splitk_slices(const DevWeight& w, int M, bool swiglu, int cus) {
    const int bn = M <= 64 ? SplitTile64::BN : SplitTile128::BN;
    const long nt = (w.N + (swiglu ? bn / 2 : bn) - 1) / (swiglu ? bn / 2 : bn);
    const int kb = w.K / 128;
    constexpr int kMinSteps = 8;   // K steps per slice at least (2 and 4 measured slower in sum)
    int S = 1;
    for (int d = 1; d <= kb; ++d) {
        if (kb % d) continue;
        if (w.K / 64 / d < kMinSteps || (d > 1 && nt * d > cus)) break;
        S = d;
    }
    return S;
}

template <class T, int WT, int EPI>
void launch_dq_split_t(hipStream_t s, const uint16_t* a, const DevWeight& w0, const DevWeight* w1, int M, int S,
                       const float* residual, void* out, float* part) {
    constexpr bool SW = EPI >= 2;
    constexpr int TN = SW ? T::BN / 2 : T::BN;
    const int N = w0.N, K = w0.K;
    const dim3 grid((N + TN - 1) / TN, (M + T::BM - 1) / T::BM, S);
    const uint8_t* qb = SW ? w1->q : w0.q;
    const __half* db = SW ? w1->d : w0.d;
    if (S == 1) {
        hipLaunchKernelGGL((mfma_dqgemm_kernel<T, WT, EPI, 2>), grid, dim3(T::NT), 0, s, a, w0.q, w0.d, qb, db, M, N,
                           K, K, N, residual, out);
        return;
    }
    const int ldp = SW ? 2 * N : N;
    hipLaunchKernelGGL((mfma_dqgemm_kernel<T, WT, SW ? 7 : 6, 2>), grid, dim3(T::NT), 0, s, a, w0.q, w0.d, qb, db, M,
                       N, K, K / S, ldp, nullptr, part);
    launch_splitk_reduce<EPI>(s, part, S, M, N, ldp, residual, out);
}

template <int EPI>
void launch_dq_split(hipStream_t s, const uint16_t* a, const DevWeight& w0, const DevWeight* w1, int M, int S,
                     const float* residual, void* out, float* part) {
    if (w0.dtype == VLRF_HIP_DT_Q8_0) {
        if (M <= 64) launch_dq_split_t<SplitTile64, VLRF_HIP_DT_Q8_0, EPI>(s, a, w0, w1, M, S, residual, out, part);
        else launch_dq_split_t<SplitTile128, VLRF_HIP_DT_Q8_0, EPI>(s, a, w0, w1, M, S, residual, out, part);
    } else {
        if (M <= 64) launch_dq_split_t<SplitTile64, VLRF_HIP_DT_Q4_0, EPI>(s, a, w0, w1, M, S, residual, out, part);
        else launch_dq_split_t<SplitTile128, VLRF_HIP_DT_Q4_0, EPI>(s, a, w0, w1, M, S, residual, out, part);
    }
}

// ---- M > 128 with few tiles: the same K split --------------------------------
// The plans above fill the GPU at the 8B shapes only from about T = 2048: at
// M = 256 the O and down GEMMs have 32 tiles.  Below a round of 256-row
// x 128-column output tiles, both forms (over the bf16 expansions and over
// the codes) split K into the same S slices -- the largest divisor of K / 128
// whose workgroups still fit one round, slices of at least 8 K steps -- with
// the partial buffer and splitk_reduce_kernel of the 17..128-row path, so
// the two forms still multiply and add the same numbers in the same order.
// (8B layer, same box: against aiming at 3/4 of a round from below half a
// round, T = 1024 0.677 -> 0.600 ms, its O and down now split in two; T =
// 256 .. 768 within noise.  Aiming at a full round: T = 256 0.291 ms.)
int big_split_slices(int M, int N, int K, int cus) {
    const long g0 = (long)((M + 255) / 256) * ((N + 127) / 128);
    const char* e = getenv("VLRF_HIP_PREFILL_SPLIT");   // "0": the unsplit plans at every M > 128
    if ((e && e[0] == '0') || K % 128 || g0 >= cus) return 1;
    const int kb = K / 128;
    int S = 1;
    for (int d = 1; d <= kb; ++d) {
        if (kb % d) continue;
        if (K / 64 / d < 8 || g0 * d > cus) break;
        S = d;
    }
    return S;
}

template <class T, int EPI>
void launch_bgemm_split_t(hipStream_t s, const uint16_t* a, const DevWeight& w0, const DevWeight* w1, int M, int S,
                          const float* residual, void* out, float* part) {
    constexpr bool SW = EPI >= 2;
    constexpr int TN = SW ? T::BN / 2 : T::BN;
    const int N = w0.N, K = w0.K, ldp = SW ? 2 * N : N;
    const dim3 grid((N + TN - 1) / TN, (M + T::BM - 1) / T::BM, S);
    hipLaunchKernelGGL((mfma_bgemm_kernel<T, SW ? 7 : 6>), grid, dim3(T::NT), 0, s, a, w0.bf, SW ? w1->bf : w0.bf, M,
                       N, K, K / S, ldp, nullptr, part);
    launch_splitk_reduce<EPI>(s, part, S, M, N, ldp, residual, out);
}

// bf16: over the expansions (of both matrices for SwiGLU); else over the codes.
template <int EPI>
void launch_big_split(hipStream_t s, bool bf16, const uint16_t* a, const DevWeight& w0, const DevWeight* w1, int M,
                      int S, const float* residual, void* out, float* part) {
    using TP = BTile<256, 128, 4, 2>;   // plain: 256 x 128 tiles
    using TS = BTile<256, 256, 2, 4>;   // SwiGLU: 256 rows x 128 gate and 128 up rows
    using T = typename std::conditional<(EPI >= 2), TS, TP>::type;
    if (bf16) launch_bgemm_split_t<T, EPI>(s, a, w0, w1, M, S, residual, out, part);
    else if (w0.dtype == VLRF_HIP_DT_Q8_0) launch_dq_split_t<T, VLRF_HIP_DT_Q8_0, EPI>(s, a, w0, w1, M, S, residual, out, part);
    else launch_dq_split_t<T, VLRF_HIP_DT_Q4_0, EPI>(s, a, w0, w1, M, S, residual, out, part);
}

// out[r][:] = bf16(w ? rmsnorm(x[r]) * w : x[r]), one 256-lane workgroup per row
// (ops.hpp:488-498: sum of squares, 1/sqrt(mean + eps), (x * inv) * w).
// Rows of D % 4 == 0 and D <= 4096 are read once, as float4 held in registers
// (NV = 4 per thread; D <= 8192 / 16384 with NV = 8 / 16), and written as 4
// packed bf16; others take the element loop (NV = 0).
template <int NV>
__global__ __launch_bounds__(256) void rows_to_bf16_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ w,
                                                           uint16_t* __restrict__ out, int D, float eps) {
    __shared__ float red[4];
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* xr = x + (size_t)r * D;
    uint16_t* o = out + (size_t)r * D;
    auto inv_rms = [&](float ss) {
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        return 1.f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)D + eps);
    };
    if constexpr (NV > 0) {
        const int n4 = D / 4;
        float4 v[NV], g[NV];
#pragma unroll
        for (int p = 0; p < NV; ++p) {
            const int f = tid + 256 * p;
            v[p] = f < n4 ? reinterpret_cast<const float4*>(xr)[f] : make_float4(0.f, 0.f, 0.f, 0.f);
            if (w) g[p] = f < n4 ? reinterpret_cast<const float4*>(w)[f] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float inv = 1.f;
        if (w) {
            float ss = 0.f;
#pragma unroll
            for (int p = 0; p < NV; ++p) ss += v[p].x * v[p].x + v[p].y * v[p].y + v[p].z * v[p].z + v[p].w * v[p].w;
            inv = inv_rms(ss);
        }
#pragma unroll
        for (int p = 0; p < NV; ++p) {
            const int f = tid + 256 * p;
            if (f < n4) {
                float4 t = v[p];
                if (w) t = make_float4(t.x * inv * g[p].x, t.y * inv * g[p].y, t.z * inv * g[p].z, t.w * inv * g[p].w);
                reinterpret_cast<uint2*>(o)[f] = make_uint2(pack_bf16(t.x, t.y), pack_bf16(t.z, t.w));
            }
        }
    } else {
        float inv = 1.f;
        if (w) {
            float ss = 0.f;
            for (int i = tid; i < D; i += 256) ss += xr[i] * xr[i];
            inv = inv_rms(ss);
        }
        for (int i = tid; i < D; i += 256) o[i] = (uint16_t)bf16_bits(w ? xr[i] * inv * w[i] : xr[i]);
    }
}

// ---- small M on the matrix cores ------------------------------------------------
// y[M,N] = x[M,K] . W^T for 2 <= M <= 16, W Q8_0/Q4_0 with K % 256 == 0, in one
// kernel.  qlinear_small_kernel<.., NW>: workgroup (gx, gy) owns the 16*NW
// weight rows of tile gx and the 256-column slices gy, gy + gridDim.y, ...
// (NW = 4 waves by default: 64-row tiles, about three workgroups per CU at
// the configuration's shapes).  Per slice it
// stages the 16 x 256 activations (rows >= M zero, times the norm weight when
// given) in LDS as bf16 hi and lo planes, laid out [block][row][32] so that
// lane (c, g) of a wave reads its MFMA operand, row c, columns 8g..8g+7 of a
// block, as 16 contiguous bytes and the wave's 64 reads cover one KiB.  Wave w
// owns rows 16w..16w+15 of the tile.  It loads their codes and scales with
// 16-byte (codes) and 4-byte (scales) lane loads over contiguous runs of each
// row, as the M = 1 GEMV does, and transposes them through LDS: lane (c, g)
// then reads the codes of row c, columns 8g..8g+7 of each block (A operand),
// one MFMA per plane multiplies them with the block's activations, and the
// f32 result D (lane (m, g) holds rows 4g+v, v = 0..3, column m) takes the
// block scales of those rows.  The workgroup's partial [128][M] tile goes to
// P[gy][mat][n][16], and with a norm the slice's sum of x^2 per row to
// SS[gx][gy][16], as device-coherent stores; once they are acknowledged one
// thread adds 1 to the row tile's counter (its own 128-byte line).  The
// workgroup that brings it to the slice count (the last of the tile's
// slices) resets it and reduces the tile: the partials of every slice added
// in slice order (deterministic, whichever workgroup comes last), then the
// epilogue.  With a norm, x is scaled by w before the product and by inv_rms
// after it: rms_norm is per row, so W.((x*inv)*w) = inv * W.(x*w)
// (ops.hpp:488-498, rounded differently).  The counters belong to the
// context (kSmallTileCtrStride ints per row tile, zero at creation, zero
// again after every call), so calls need no clearing and none is recorded
// under graph capture; calls on one context are serialised by its stream.
constexpr int kSmallSlice = 256;         // K columns per slice (8 blocks)

__device__ __forceinline__ float wave32_sum(float v) {     // sum over each half-wave
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    const float2 t = swap_rows16(v, v);
    return t.x + t.y;
}

// Four floats at byte offset off of the buffer rs, written device-coherent by
// another workgroup (sc1 load; rs is uniform, the offset per lane).
__device__ __forceinline__ float4 ld_agent4(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v v = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 16));
    return make_float4(v.x, v.y, v.z, v.w);
}

// Codes of one lane's 8 columns of a block -> bf16 (exact).
template <int WT>
__device__ __forceinline__ bf16x8 codes_bf16(uint2 c) {
    bf16x8 r;
    if constexpr (WT == VLRF_HIP_DT_Q8_0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            r[e] = (__bf16)(float)(int8_t)(c.x >> (8 * e));
            r[4 + e] = (__bf16)(float)(int8_t)(c.y >> (8 * e));
        }
    } else {                                  // byte j: element 2j low nibble, 2j+1 high
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = (__bf16)(float)((int)((c.x >> (4 * e)) & 0xFu) - 8);
    }
    return r;
}

template <int WT, int NM, int EPI, int NW>
__global__ __launch_bounds__(64 * NW) void qlinear_small_kernel(
    const uint8_t* __restrict__ qa, const __half* __restrict__ da, const uint8_t* __restrict__ qb,
    const __half* __restrict__ db, int N, int K, int M, const float* __restrict__ x,
    const float* __restrict__ norm_w, float eps, const float* __restrict__ residual, float* __restrict__ y,
    float* __restrict__ P, float* __restrict__ SS, int* __restrict__ tile_ctr) {
    constexpr int CB = WT == VLRF_HIP_DT_Q8_0 ? 256 : 128;   // code bytes of a row per slice
    constexpr int CS = CB + 16;                          // padded LDS row stride
    constexpr int LPR = CB / 16;                         // lanes per row in a coalesced load
    constexpr int CL = 16 * LPR / 64;                    // 16-byte code loads per lane and matrix
    __shared__ __align__(16) uint16_t xh[8 * 16 * 32];
    __shared__ __align__(16) uint16_t xl[8 * 16 * 32];
    __shared__ __align__(16) uint8_t cs[NM][NW][16 * CS];  // per wave: its 16 rows' codes
    __shared__ __align__(16) uint32_t ssc[NM][NW][16 * 4]; // per wave: 16 rows x 8 f16 scales
    constexpr int ROWS = 16 * NW, NI = 512 / (64 * NW);   // rows per workgroup; staging items per thread
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int rbase = blockIdx.x * ROWS + 16 * wave;
    const int ns = K / kSmallSlice;
    const size_t rowb = WT == VLRF_HIP_DT_Q8_0 ? (size_t)K : (size_t)K / 2;
    // staging: item e = tid + 64 NW i converts row e/32, columns 8(e%32) .. +7 of the slice
    const int sk = 8 * (tid & 31);
    float ss[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) ss[i] = 0.f;
    f32x4 acc[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int sl = blockIdx.y; sl < ns; sl += gridDim.y) {
        const int k0 = sl * kSmallSlice;
        // Activations first (L2, needed first), then the codes and scales (HBM):
        // loads complete in order, so the staging below waits for x only.
        float4 a0[NI], a1[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int sm = (tid >> 5) + 2 * NW * i;
            a0[i] = a1[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (sm < M) {
                const float4* xp = reinterpret_cast<const float4*>(x + (size_t)sm * K + k0 + sk);
                a0[i] = xp[0];
                a1[i] = xp[1];
            }
        }
        // Codes: load i of lane l covers row LPR-group i*64/LPR + l/LPR, bytes
        // 16(l % LPR) .. +15 of the row's slice: runs of CB contiguous bytes.
        uint4 cv[NM][CL];
        uint32_t sv[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const uint8_t* q = m ? qb : qa;
            const __half* d = m ? db : da;
#pragma unroll
            for (int i = 0; i < CL; ++i) {
                const int r = min(rbase + i * (64 / LPR) + lane / LPR, N - 1);
                cv[m][i] = *reinterpret_cast<const uint4*>(q + r * rowb + (size_t)k0 * CB / kSmallSlice +
                                                           16 * (lane % LPR));
            }
            const int r = min(rbase + (lane >> 2), N - 1);      // 16 rows x 4 dwords of scales
            sv[m] = *reinterpret_cast<const uint32_t*>(d + (size_t)r * (K / 32) + k0 / 32 + 2 * (lane & 3));
        }
#pragma unroll
        for (int it = 0; it < NI; ++it) {
            const int sm = (tid >> 5) + 2 * NW * it;
            float4 b0 = a0[it], b1 = a1[it];
            if (sm < M) {
                ss[it] += b0.x * b0.x + b0.y * b0.y + b0.z * b0.z + b0.w * b0.w +
                          b1.x * b1.x + b1.y * b1.y + b1.z * b1.z + b1.w * b1.w;
                if (norm_w) {
                    const float4* wp = reinterpret_cast<const float4*>(norm_w + k0 + sk);
                    const float4 w0 = wp[0], w1 = wp[1];
                    b0 = make_float4(b0.x * w0.x, b0.y * w0.y, b0.z * w0.z, b0.w * w0.w);
                    b1 = make_float4(b1.x * w1.x, b1.y * w1.y, b1.z * w1.z, b1.w * w1.w);
                }
            }
            const float v[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
            uint32_t h[4], l[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h[i] = pack_bf16(v[2 * i], v[2 * i + 1]);
                l[i] = pack_bf16(v[2 * i] - __uint_as_float(h[i] << 16),
                                 v[2 * i + 1] - __uint_as_float(h[i] & 0xFFFF0000u));
            }
            const int o = (sk >> 5) * 512 + sm * 32 + (sk & 31);
            *reinterpret_cast<uint4*>(xh + o) = make_uint4(h[0], h[1], h[2], h[3]);
            *reinterpret_cast<uint4*>(xl + o) = make_uint4(l[0], l[1], l[2], l[3]);
        }
#pragma unroll
        for (int m = 0; m < NM; ++m) {
#pragma unroll
            for (int i = 0; i < CL; ++i)
                *reinterpret_cast<uint4*>(&cs[m][wave][(i * (64 / LPR) + lane / LPR) * CS + 16 * (lane % LPR)]) =
                    cv[m][i];
            ssc[m][wave][lane] = sv[m];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int xo = (j * 16 + c) * 32 + 8 * g;
            const bf16x8 bh = *reinterpret_cast<const bf16x8*>(xh + xo);
            const bf16x8 bl = *reinterpret_cast<const bf16x8*>(xl + xo);
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                uint2 code;
                if constexpr (WT == VLRF_HIP_DT_Q8_0)
                    code = *reinterpret_cast<const uint2*>(&cs[m][wave][c * CS + 32 * j + 8 * g]);
                else
                    code = make_uint2(*reinterpret_cast<const uint32_t*>(&cs[m][wave][c * CS + 16 * j + 4 * g]), 0u);
                const bf16x8 a = codes_bf16<WT>(code);
                f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl, t, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const uint32_t wd = ssc[m][wave][(4 * g + v) * 4 + (j >> 1)];
                    const float sv2 = __half2float(__ushort_as_half((unsigned short)(wd >> (16 * (j & 1)))));
                    acc[m][v] += sv2 * t[v];
                }
            }
        }
        __syncthreads();                      // before the next slice overwrites the staging
    }

    // This slice's partials, device-coherent (the tile's last workgroup may
    // run on another XCD): columns m < M only.
    const int S = gridDim.y;
    float* Pw = P + (size_t)blockIdx.y * NM * N * 16;
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int n = rbase + 4 * g + v;
            if (n < N && c < M)
                __hip_atomic_store(&Pw[((size_t)m * N + n) * 16 + c], acc[m][v], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    if (SS) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int sm = (tid >> 5) + 2 * NW * i;
            const float t = wave32_sum(ss[i]);   // threads 32r .. 32r+31 hold row r
            if ((tid & 31) == 0 && sm < M)
                __hip_atomic_store(&SS[((size_t)blockIdx.x * S + blockIdx.y) * 16 + sm], t, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);       // this wave's stores acknowledged (vmcnt 0)
    __shared__ int last;
    __syncthreads();
    if (tid == 0) {
        int* ctr = tile_ctr + (size_t)blockIdx.x * kSmallTileCtrStride;
        last = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
        if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;

    // The tile's reduction: thread (row r = tid / 4, columns 4q..4q+3).
    const int r = tid >> 2, q4 = tid & 3, n = blockIdx.x * ROWS + r;
    if (n >= N || 4 * q4 >= M) return;
    // Byte offsets stay below 2^32: the partials are S * NM * N * 64 bytes and
    // the host bounds that (qlinear_small_scratch).
    const uint32_t st = (uint32_t)NM * N * 64;                      // bytes per slice
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(P, 0, 0x7fffffff, 0x00020000);
    float4 o[NM];
#pragma unroll
    for (int j = 0; j < NM; ++j) {
        const uint32_t base = (uint32_t)(((size_t)j * N + n) * 64 + 16 * q4);
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        int sl = 0;
        for (; sl + 4 <= S; sl += 4) {        // four independent loads in flight, added in slice order
            float4 v4[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v4[u] = ld_agent4(prs, base + (uint32_t)(sl + u) * st);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                t.x += v4[u].x; t.y += v4[u].y; t.z += v4[u].z; t.w += v4[u].w;
            }
        }
        for (; sl < S; ++sl) {
            const float4 v4 = ld_agent4(prs, base + (uint32_t)sl * st);
            t.x += v4.x; t.y += v4.y; t.z += v4.z; t.w += v4.w;
        }
        o[j] = t;
    }
    float inv[4] = {1.f, 1.f, 1.f, 1.f};
    if (SS) {
        const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(SS, 0, 0x7fffffff, 0x00020000);
        float4 ssum = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int sl = 0; sl < S; ++sl) {
            const float4 v4 = ld_agent4(srs, (uint32_t)((((size_t)blockIdx.x * S + sl) * 16 + 4 * q4) * 4));
            ssum.x += v4.x; ssum.y += v4.y; ssum.z += v4.z; ssum.w += v4.w;
        }
        const float sv[4] = {ssum.x, ssum.y, ssum.z, ssum.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) inv[u] = 1.f / sqrtf(sv[u] / (float)K + eps);
    }
    const float o0[4] = {o[0].x, o[0].y, o[0].z, o[0].w};
    float o1[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (NM == 2) {
        o1[0] = o[1].x; o1[1] = o[1].y; o1[2] = o[1].z; o1[3] = o[1].w;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int m = 4 * q4 + u;
        if (m >= M) break;
        const size_t off = (size_t)m * N + n;
        float out = o0[u] * inv[u];
        if constexpr (EPI >= 2) {
            const float gv = out, uv = o1[u] * inv[u];
            out = uv * (gv / (1.f + expf(-gv)));   // silu(g) * u, ops.hpp:409-441
        }
        if constexpr (EPI == 1) out += residual[off];
        y[off] = out;
    }
}

// Workgroup columns: one per slice (every workgroup loads once and computes
// once) up to about 1024 workgroups (4 per CU); beyond that columns take
// several slices, which bounds the partial-sum scratch.
int small_grid_y(int N, int K, int rows) {
    const int groups = (N + rows - 1) / rows, ns = K / kSmallSlice;
    const int want = (1024 + groups - 1) / groups;
    return want < ns ? want : ns;
}

// Waves per workgroup of the small-M kernel (16 rows each): 4 (VLRF_HIP_SMALL_WAVES=8: 8).
int small_waves() {
    static int nw = 0;
    if (!nw) {
        const char* e = getenv("VLRF_HIP_SMALL_WAVES");
        nw = e && std::atoi(e) == 8 ? 8 : 4;
    }
    return nw;
}

// Compute units of the current device (the tile plan's round size).
int lds_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            cus = n;
        else
            cus = 256;
    }
    return cus;
}

int check_qgemm(const DevWeight& w, int M) {
    VH_ARG(w.dtype == VLRF_HIP_DT_Q8_0 || w.dtype == VLRF_HIP_DT_Q4_0,
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
    if (D % 4 == 0 && D <= 4096)
        hipLaunchKernelGGL(rows_to_bf16_kernel<4>, dim3(rows), dim3(256), 0, s, x, w, out, D, eps);
    else if (D % 4 == 0 && D <= 8192)
        hipLaunchKernelGGL(rows_to_bf16_kernel<8>, dim3(rows), dim3(256), 0, s, x, w, out, D, eps);
    else if (D % 4 == 0 && D <= 16384)
        hipLaunchKernelGGL(rows_to_bf16_kernel<16>, dim3(rows), dim3(256), 0, s, x, w, out, D, eps);
    else
        hipLaunchKernelGGL(rows_to_bf16_kernel<0>, dim3(rows), dim3(256), 0, s, x, w, out, D, eps);
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

// Makes the weight's bf16 expansion on first use (an allocation and one
// kernel).  Never while `s` is being captured into a graph: the allocation
// would be recorded mid-capture, so the GEMM then decodes the codes in its
// tiles instead (the same results to the 1e-2 class, a little slower).
bool weight_expand_bf16(hipStream_t s, const DevWeight& w) {
    if (w.bf) return true;
    const char* e = getenv("VLRF_HIP_PREFILL_BF16");
    if ((e && e[0] == '0') || !w.q || !w.d || (w.dtype != VLRF_HIP_DT_Q8_0 && w.dtype != VLRF_HIP_DT_Q4_0)) return false;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        return false;
    }
    const size_t n = (size_t)w.N * w.K, nb = n / 32;
    uint16_t* bf = nullptr;
    if (hipMalloc(&bf, n * sizeof(uint16_t)) != hipSuccess) {
        (void)hipGetLastError();   // not an error: the GEMM decodes the codes instead
        return false;
    }
    const size_t np = nb * 4;   // quarter blocks, one per thread
    const dim3 grid((unsigned)((np + 255) / 256));
    if (w.dtype == VLRF_HIP_DT_Q8_0) hipLaunchKernelGGL(expand_bf16_kernel<VLRF_HIP_DT_Q8_0>, grid, dim3(256), 0, s, w.q, w.d, bf, np);
    else hipLaunchKernelGGL(expand_bf16_kernel<VLRF_HIP_DT_Q4_0>, grid, dim3(256), 0, s, w.q, w.d, bf, np);
    if (hipGetLastError() != hipSuccess) {
        (void)hipFree(bf);
        return false;
    }
    w.bf = bf;
    return true;
}

// 17 <= M <= 128 over codes with K split: the partial-buffer bytes the call
// needs (0 when it runs unsplit or on another kernel).
static bool dq_split_path(const DevWeight& w, int M) { return M >= 17 && M <= 128 && dqgemm_supported(w); }

size_t qgemm_part_bytes(const DevWeight& w, int M, bool swiglu) {
    int S = 1;
    if (M > 128) S = big_split_slices(M, w.N, w.K, lds_cus());
    else if (dq_split_path(w, M)) S = splitk_slices(w, M, swiglu, lds_cus());
    return S > 1 ? (size_t)S * M * w.N * (swiglu ? 2 : 1) * sizeof(float) : 0;
}

int launch_qgemm(hipStream_t s, const DevWeight& w, const uint16_t* a, int M, const float* residual,
                 float* y, float* part) {
    int rc = check_qgemm(w, M);
    if (rc) return rc;
    VH_ARG(a && y, "qgemm: null operand");
    if (M > 128) {
        weight_expand_bf16(s, w);
        const int S = part ? big_split_slices(M, w.N, w.K, lds_cus()) : 1;
        if (S > 1 && (w.bf || dqgemm_supported(w))) {
            if (residual) launch_big_split<1>(s, w.bf != nullptr, a, w, nullptr, M, S, residual, y, part);
            else launch_big_split<0>(s, w.bf != nullptr, a, w, nullptr, M, S, nullptr, y, part);
        } else if (w.bf) {
            if (residual) launch_bgemm_plan<1>(s, a, w, nullptr, M, residual, y);
            else launch_bgemm_plan<0>(s, a, w, nullptr, M, nullptr, y);
        } else if (dqgemm_supported(w)) {
            if (residual) launch_dqgemm_plan<1>(s, a, w, nullptr, M, residual, y);
            else launch_dqgemm_plan<0>(s, a, w, nullptr, M, nullptr, y);
        } else {
            const LdsPlan p = lds_plan(M, w.N, false, lds_cus());
            if (residual) launch_lds_plan<1>(s, p, a, w, nullptr, M, residual, y);
            else launch_lds_plan<0>(s, p, a, w, nullptr, M, nullptr, y);
        }
    } else if (dq_split_path(w, M) && (part || qgemm_part_bytes(w, M, false) == 0)) {
        const int S = splitk_slices(w, M, false, lds_cus());
        if (residual) launch_dq_split<1>(s, a, w, nullptr, M, S, residual, y, part);
        else launch_dq_split<0>(s, a, w, nullptr, M, S, nullptr, y, part);
    } else {
        if (residual) launch_cfg<CfgSmall, 1>(s, w.dtype, a, w, nullptr, M, residual, y);
        else launch_cfg<CfgSmall, 0>(s, w.dtype, a, w, nullptr, M, nullptr, y);
    }
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

int launch_qgemm_swiglu(hipStream_t s, const DevWeight& wg, const DevWeight& wu, const uint16_t* a,
                        int M, void* h, bool h_bf16, float* part) {
    int rc = check_qgemm(wg, M);
    if (rc) return rc;
    rc = check_qgemm(wu, M);
    if (rc) return rc;
    VH_ARG(wg.N == wu.N && wg.K == wu.K && wg.dtype == wu.dtype, "qgemm_swiglu: gate/up differ");
    VH_ARG(a && h, "qgemm_swiglu: null operand");
    if (M > 128) {
        const bool both = weight_expand_bf16(s, wg) && weight_expand_bf16(s, wu);
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (!both && wg.bf && !wu.bf && hipStreamIsCapturing(s, &cs) == hipSuccess &&
            cs == hipStreamCaptureStatusNone) {
            (void)hipFree(wg.bf);   // both or neither (no free while capturing)
            wg.bf = nullptr;
        }
        const int S = part ? big_split_slices(M, wg.N, wg.K, lds_cus()) : 1;
        if (S > 1 && (both || dqgemm_supported(wg))) {
            if (h_bf16) launch_big_split<2>(s, both, a, wg, &wu, M, S, nullptr, h, part);
            else launch_big_split<3>(s, both, a, wg, &wu, M, S, nullptr, h, part);
        } else if (both) {
            if (h_bf16) launch_bgemm_plan<2>(s, a, wg, &wu, M, nullptr, h);
            else launch_bgemm_plan<3>(s, a, wg, &wu, M, nullptr, h);
        } else if (dqgemm_supported(wg)) {
            if (h_bf16) launch_dqgemm_plan<2>(s, a, wg, &wu, M, nullptr, h);
            else launch_dqgemm_plan<3>(s, a, wg, &wu, M, nullptr, h);
        } else {
            const LdsPlan p = lds_plan(M, wg.N, true, lds_cus());
            if (h_bf16) launch_lds_plan<2>(s, p, a, wg, &wu, M, nullptr, h);
            else launch_lds_plan<3>(s, p, a, wg, &wu, M, nullptr, h);
        }
    } else if (dq_split_path(wg, M) && (part || qgemm_part_bytes(wg, M, true) == 0)) {
        const int S = splitk_slices(wg, M, true, lds_cus());
        if (h_bf16) launch_dq_split<2>(s, a, wg, &wu, M, S, nullptr, h, part);
        else launch_dq_split<3>(s, a, wg, &wu, M, S, nullptr, h, part);
    } else {
        if (h_bf16) launch_cfg<CfgSmall, 2>(s, wg.dtype, a, wg, &wu, M, nullptr, h);
        else launch_cfg<CfgSmall, 3>(s, wg.dtype, a, wg, &wu, M, nullptr, h);
    }
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

bool qlinear_small_supported(const DevWeight& w) {
    return (w.dtype == VLRF_HIP_DT_Q8_0 || w.dtype == VLRF_HIP_DT_Q4_0) && w.q && w.d && w.K % kSmallSlice == 0;
}

int qlinear_small_tiles(int N) { const int rows = 16 * small_waves(); return (N + rows - 1) / rows; }

size_t qlinear_small_scratch(int N, int K, bool two) {
    const size_t S = (size_t)small_grid_y(N, K, 16 * small_waves()), tiles = (size_t)qlinear_small_tiles(N);
    return S * (two ? 2 : 1) * (size_t)N * 16 * sizeof(float) + tiles * S * 16 * sizeof(float);
}

int launch_qlinear_small(hipStream_t s, const DevWeight& w0, const DevWeight* w1, const float* x,
                         int M, const float* norm_w, float eps, const float* residual, float* scratch,
                         int* tile_ctr, int tile_ctr_tiles, float* y) {
    VH_ARG(M >= 2 && M <= 16, "qlinear_small: M=%d outside [2,16]", M);
    VH_ARG(qlinear_small_supported(w0), "qlinear_small: dtype %d / K %d not supported", w0.dtype, w0.K);
    if (w1) VH_ARG(w1->N == w0.N && w1->K == w0.K && w1->dtype == w0.dtype && w1->q && w1->d,
                   "qlinear_small: gate/up differ");
    VH_ARG(x && y && scratch && tile_ctr, "qlinear_small: null pointer");
    VH_ARG(!(w1 && residual), "qlinear_small: no residual on the SwiGLU form");
    const int NW = small_waves();
    const int N = w0.N, K = w0.K, S = small_grid_y(N, K, 16 * NW), NM = w1 ? 2 : 1;
    VH_ARG(qlinear_small_tiles(N) <= tile_ctr_tiles, "qlinear_small: %d row tiles, the context counts %d",
           qlinear_small_tiles(N), tile_ctr_tiles);
    VH_ARG(qlinear_small_scratch(N, K, w1 != nullptr) < 0x7fffffffu, "qlinear_small: partials exceed 2 GiB");
    float* P = scratch;
    float* SS = norm_w ? scratch + (size_t)S * NM * N * 16 : nullptr;
    const dim3 grid(qlinear_small_tiles(N), S);
    const uint8_t* qb = w1 ? w1->q : nullptr;
    const __half* db = w1 ? w1->d : nullptr;
#define VH_SMALL(WT, NMV, EPIV)                                                                                 \
    do {                                                                                                        \
        if (NW == 8)                                                                                            \
            hipLaunchKernelGGL((qlinear_small_kernel<WT, NMV, EPIV, 8>), grid, dim3(512), 0, s, w0.q, w0.d, qb, \
                               db, N, K, M, x, norm_w, eps, residual, y, P, SS, tile_ctr);                      \
        else                                                                                                    \
            hipLaunchKernelGGL((qlinear_small_kernel<WT, NMV, EPIV, 4>), grid, dim3(256), 0, s, w0.q, w0.d, qb, \
                               db, N, K, M, x, norm_w, eps, residual, y, P, SS, tile_ctr);                      \
    } while (0)
#define VH_SMALL_T(WT)                                         \
    do {                                                       \
        if (w1) VH_SMALL(WT, 2, 3);                            \
        else if (residual) VH_SMALL(WT, 1, 1);                 \
        else VH_SMALL(WT, 1, 0);                               \
    } while (0)
    if (w0.dtype == VLRF_HIP_DT_Q8_0) VH_SMALL_T(VLRF_HIP_DT_Q8_0);
    else VH_SMALL_T(VLRF_HIP_DT_Q4_0);
#undef VH_SMALL_T
#undef VH_SMALL
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

}  // namespace vlrf_hip
