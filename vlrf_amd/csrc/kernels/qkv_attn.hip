// qkv_attn.hip - a layer's QKV projection and its decode attention in ONE
// launch: the first two kernels of the per-kernel decode step, fused.
//
// Reference: AttentionBlock::forward (attention.hpp:89-186) for T = 1 after
// the pre-norm (transformer_block.hpp:141-159): q, k, v = W{q,k,v} .
// rmsnorm(x) (ops.hpp:478-499, compute.hpp:64-68), RoPE on q and k
// (rope.hpp:90-96), the K/V row appended to the cache (kv_cache.hpp:102-117),
// then attention over the cache (attention.hpp:207-309).
//
// Why one launch.  The attention of query head h needs only 64 outputs of the
// QKV projection for its query and the 2 x n_kv x 64 of the token's K/V row,
// not the whole projection; its cache rows do not depend on this step at all.
// So the grid holds the projection's workgroups first and the attention's
// after them: an attention workgroup issues its cache rows' loads (and the
// RoPE table row) at once, while the projection streams its weights, then
// waits for exactly the words it needs.  The projection publishes its outputs
// as tagged words (tagged.hpp: value | epoch << 32, one device-scope store per
// word; the step's epoch is state[3], advanced by the argmax kernel), so the
// wait needs no counter, fence or clearing.  A kernel boundary, the
// attention's launch and its first-byte latency leave the critical path.
//
// Progress: the attention workgroups only wait for lower-numbered ones, which
// the hardware dispatches first on every XCD, and the projection's never
// wait.  The wait is bounded anyway (QkvAttnParams::limit on the wall clock):
// one that runs out sets `status` and leaves, and the host reports it.
//
// Arithmetic: the projection is gemv_body (the M = 1 GEMV of the per-kernel
// step) and the attention attn::chunk (the chunked decode attention), on the
// same operands in the same order as the two kernels they replace.
#include "../internal.hpp"
#include "attn_core.hpp"
#include "gemv_core.hpp"
#include "tagged.hpp"

namespace vlrf_hip {
namespace {

using namespace tagged;
constexpr int kChunkRows = kAttnChunkRows;   // one workgroup: 8 waves x one 64-row round
constexpr int kPhaseAttention = 2;

__device__ __forceinline__ Ctl ctl(const QkvAttnParams& P, uint32_t tag) {
    Ctl c;
    c.rs = __builtin_amdgcn_make_buffer_rsrc(P.tags, 0, P.N * 8, 0x00020000);
    c.tag = tag;
    c.status = P.status;
    c.t0 = wall_clock64();
    c.limit = P.limit;
    c.phase = kPhaseAttention;
    c.layer = P.layer;
    return c;
}

// ---- the token's K/V row (one workgroup) -------------------------------------------
// attention.hpp:109-145 for T = 1: RoPE on k (rope.hpp:90-96), KVCache::append
// (kv_cache.hpp:102-117: the Q8_0 row, all n_kv heads, under one scale per K
// and per V row), and the new key's share of every query head's attention,
// which the chunks leave out: the partial (acc = v_stored, m = q.k_stored *
// scale, l = 1) at index nch of the head's partials, merged by the O
// projection after the cache chunks, the order of the reference's online
// softmax, where the token's key comes last.
struct NewRowSmem {
    __align__(16) float qs[kQkvAttnMaxD];   // q of every head, rotated
    __align__(16) float nk[8 * attn::D];    // the stored K / V row read back
    __align__(16) float nv[8 * attn::D];
    float amax[2 * gemv::kGemvWaves];
    int oks[gemv::kGemvWaves];
};

template <int KVT>
__device__ void new_row(const QkvAttnParams& P, uint32_t tag) {
    __shared__ NewRowSmem sm;
    constexpr int NT = gemv::kGemvThreads, W = gemv::kGemvWaves;
    constexpr bool Q8 = KVT == VLRF_HIP_KV_Q8_0;
    const DecodeFuse& fz = P.fz;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int G = fz.n_kv, D = P.K, H = G * P.rep, npairs = G * attn::HALF, nrow = G * attn::D;
    const int nparts = fz.nch + 1;
    const int cap = (int)(P.head_stride / attn::D);
    const int pos = min(P.state[1], cap - 1);
    const bool rot = pos < fz.max_seq;
    attn::NewRow nr;                          // RoPE table entries of pair index tid % 32
    attn::rope_row(nr, fz, pos);
    // Words: q pairs tid and tid + 512 (D / 2 <= 1024 pairs), this thread's K
    // pair and V element.
    Ctl c = ctl(P, tag);
    const int qp0 = tid, qp1 = tid + NT, nqp = D / 2;
    auto qword = [&](int pr, int half) {   // pair pr = (head, j): elements j and j + 32 of the head
        const int hh = pr / attn::HALF, jj = pr - hh * attn::HALF;
        return (hh * attn::D + jj + half * attn::HALF) * 8;
    };
    const int kp = min(tid, npairs - 1), kh = kp / attn::HALF, kj = kp - kh * attn::HALF;
    int off[7] = {qword(min(qp0, nqp - 1), 0), qword(min(qp0, nqp - 1), 1), qword(min(qp1, nqp - 1), 0),
                  qword(min(qp1, nqp - 1), 1), (D + kh * attn::D + kj) * 8,
                  (D + kh * attn::D + kj + attn::HALF) * 8, (D + nrow + min(tid, nrow - 1)) * 8};
    bool use[7] = {qp0 < nqp, qp0 < nqp, qp1 < nqp, qp1 < nqp, tid < npairs, tid < npairs, tid < nrow};
    u32x2 v[7];
    const bool ok = poll_direct<7, u32x2>(c, off, use, v);
    if (!block_ok(ok, sm.oks)) return;
    auto f = [&](int i) { return __uint_as_float(v[i].x); };
    // q of every head, rotated (pair index = lane % 32 for both of the thread's pairs)
    if (qp0 < nqp) {
        const int hh = qp0 / attn::HALF, jj = qp0 - hh * attn::HALF;
        float y0 = f(0), y1 = f(1);
        if (rot) attn::rope2(f(0), f(1), nr.rc, nr.rs, &y0, &y1);
        sm.qs[hh * attn::D + jj] = y0;
        sm.qs[hh * attn::D + jj + attn::HALF] = y1;
    }
    if (qp1 < nqp) {
        const int hh = qp1 / attn::HALF, jj = qp1 - hh * attn::HALF;
        float y0 = f(2), y1 = f(3);
        if (rot) attn::rope2(f(2), f(3), nr.rc, nr.rs, &y0, &y1);
        sm.qs[hh * attn::D + jj] = y0;
        sm.qs[hh * attn::D + jj + attn::HALF] = y1;
    }
    float k0 = f(4), k1 = f(5);
    const float vn = f(6);
    if (tid < npairs && rot) attn::rope2(k0, k1, nr.rc, nr.rs, &k0, &k1);
    if constexpr (Q8) {
        const float ak = wave_max(tid < npairs ? fmaxf(fabsf(k0), fabsf(k1)) : 0.f);
        const float av = wave_max(tid < nrow ? fabsf(vn) : 0.f);
        if (lane == 0) { sm.amax[w] = ak; sm.amax[W + w] = av; }
    }
    __syncthreads();
    float ak = 0.f, av = 0.f, sk = 1.f, sv = 1.f, ik = 0.f, iv = 0.f;
    if constexpr (Q8) {
#pragma unroll
        for (int k = 0; k < W; ++k) {
            ak = fmaxf(ak, sm.amax[k]);
            av = fmaxf(av, sm.amax[W + k]);
        }
        sk = ak != 0.f ? ak / 127.f : 0.f;
        sv = av != 0.f ? av / 127.f : 0.f;
        ik = ak != 0.f ? 1.f / sk : 0.f;
        iv = av != 0.f ? 1.f / sv : 0.f;
    }
    constexpr int EB = attn::KV<KVT>::EB;
    if (tid < npairs) {
        int8_t* krow = fz.kq_w + ((size_t)kh * P.head_stride + (size_t)pos * attn::D) * EB;
        sm.nk[kh * attn::D + kj] = attn::store_elem<KVT>(krow, kj, k0, sk, ik, ak != 0.f, true);
        sm.nk[kh * attn::D + kj + attn::HALF] = attn::store_elem<KVT>(krow, kj + attn::HALF, k1, sk, ik, ak != 0.f, true);
    }
    if (tid < nrow) {
        const int vh = tid / attn::D, vj = tid - vh * attn::D;
        int8_t* vrow = fz.vq_w + ((size_t)vh * P.head_stride + (size_t)pos * attn::D) * EB;
        sm.nv[tid] = attn::store_elem<KVT>(vrow, vj, vn, sv, iv, av != 0.f, true);
    }
    if constexpr (Q8) {
        if (tid == 0) { fz.ks_w[pos] = sk; fz.vs_w[pos] = sv; }
    }
    __syncthreads();
    // The new key's partial of head h: score q.k_stored, weight 1, value the
    // stored V row.  Each head's dot runs on one 16-lane row, 4 dims a lane,
    // summed by row rotations (one thread per head reading its head's q row
    // had every lane of a read on one LDS bank).
    static_assert(attn::D == 16 * 4, "16 lanes x 4 dims per head");
    for (int h0 = 0; h0 < H; h0 += NT / 16) {
        const int hh = h0 + (tid >> 4), i = tid & 15, hc = min(hh, H - 1);
        const float4 qv = *reinterpret_cast<const float4*>(&sm.qs[hc * attn::D + 4 * i]);
        const float4 kv = *reinterpret_cast<const float4*>(&sm.nk[(hc / P.rep) * attn::D + 4 * i]);
        float a = (qv.x * kv.x + qv.y * kv.y) + (qv.z * kv.z + qv.w * kv.w);
        a += dpp_f<0x128>(a);   // row_ror:8
        a += dpp_f<0x124>(a);   // row_ror:4
        a += dpp_f<0x122>(a);   // row_ror:2
        a += dpp_f<0x121>(a);   // row_ror:1: every lane of the row holds the sum
        if (i == 0 && hh < H) {
            float* pp = fz.chunks + ((size_t)hh * nparts + fz.nch) * kAttnChunkStride;
            pp[attn::D] = a * P.scale;
            pp[attn::D + 1] = 1.f;
        }
    }
    for (int e = tid; e < H * attn::D; e += NT) {
        const int hh = e / attn::D, d = e - hh * attn::D;
        fz.chunks[((size_t)hh * nparts + fz.nch) * kAttnChunkStride + d] = sm.nv[(hh / P.rep) * attn::D + d];
    }
}

// 128 VGPRs at most (4 waves per SIMD): two workgroups per CU, so the
// attention's workgroups are resident beside the projection's.
template <int WT, int KVT, int NC, bool GATHER>
__global__ __launch_bounds__(gemv::kGemvThreads) __attribute__((amdgpu_waves_per_eu(4))) void qkv_attn_kernel(
    QkvAttnParams P) {
    static_assert(gemv::kGemvThreads == kChunkRows, "one thread per chunk row");
    const int b = blockIdx.x;
    const uint32_t tag = (uint32_t)P.state[3];
    if (b < P.nq) {
        // The projection: one row per wave, RMSNorm fused; layer 0 gathers the
        // token's embedding row (ops.hpp:615-626), copied to the residual stream.
        constexpr int XM = 16 | 1 | (GATHER ? 2 : 0);
        gemv::gemv_body<WT, NC, 1, false, XM>(P.qa, P.da, nullptr, nullptr, P.N, P.K, P.x,
                                              GATHER ? P.state : nullptr, P.x_copy, P.norm_w, P.eps, 0, b, P.nq,
                                              [&](int row, float o) { put_word(P.tags + row, __float_as_uint(o), tag); });
        return;
    }

    if (b == P.nq + P.na) {
        new_row<KVT>(P, tag);
        return;
    }

    // ---- attention: query head h over cache rows [c0, c0 + 512) -----------------
    // The REP query heads of chunk (g, s) run on one XCD (workgroup b on XCD
    // b % 8, and nq is a multiple of 8), so the chunk's K/V rows come from HBM
    // once and then from that L2; placement only affects speed.  The token's
    // own row is left out (the new-row workgroup writes it meanwhile) and
    // enters the O projection's merge as one more partial.
    __shared__ attn::SmemQ<8> sm;
    __shared__ int oks[gemv::kGemvWaves];
    const DecodeFuse& fz = P.fz;
    const int ab = b - P.nq, rep = P.rep, nch = fz.nch, nparts = nch + 1;
    const int k = ab >> 3, r = k % rep, pc = (ab & 7) + 8 * (k / rep);
    if (pc >= fz.n_kv * nch) return;
    const int g = pc / nch, chunk = pc - g * nch, h = g * rep + r, c0 = chunk * kChunkRows;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int cap = (int)(P.head_stride / attn::D);
    const size_t hb = (size_t)g * P.head_stride;

    attn::Round<KVT> R;
    attn::load_round<KVT>(R, fz.kq_w, fz.vq_w, fz.ks_w, fz.vs_w, hb, c0 + w * 64, cap, lane);
    const int pos = min(P.state[1], cap - 1);   // the host checks capacity before queuing
    attn::NewRow nr;
    attn::rope_row(nr, fz, pos);
    issue_before_wait();
    float* pp = fz.chunks + ((size_t)h * nparts + chunk) * kAttnChunkStride;
    if (c0 >= pos) {   // no cache row before the token: the empty partial (acc 0, m -inf, l 0), no wait
        if (tid < attn::D) pp[tid] = 0.f;
        if (tid == 0) { pp[attn::D] = attn::kNegInf; pp[attn::D + 1] = 0.f; }
        return;
    }
    // Input: q of head h (wave 0, lanes j < 32: dims j and j + 32), from the 8
    // projection workgroups of head h, polled by wave 0 alone.
    Ctl c = ctl(P, tag);
    const int j = lane & (attn::HALF - 1);
    int off[2] = {(h * attn::D + j) * 8, (h * attn::D + j + attn::HALF) * 8};
    bool use[2] = {true, true};
    u32x2 v[2];
    bool ok = true;
    if (w == 0) {
        ok = poll_direct<2, u32x2>(c, off, use, v);
        // rope.hpp:84: positions >= max_seq stay unrotated.  Staged before the
        // barrier that also publishes the workgroup's wait results.
        if (ok)
            attn::stage_q<8>(sm, __uint_as_float(v[0].x), __uint_as_float(v[1].x), nr.rc, nr.rs, pos < fz.max_seq);
    }
    if (!block_ok(ok, oks)) return;
    // the chunk's partial, unnormalised
    attn::chunk_q<KVT, 8>(sm, R, c0, pos, P.scale, [&](int t, float ot, float mt, float lt) {
        pp[t] = ot;
        if (t == 0) { pp[attn::D] = mt; pp[attn::D + 1] = lt; }
    });
}

int qkv_chunks(int w_dtype, int K) {
    const int cw = 64 * (w_dtype == VLRF_HIP_DT_Q8_0 ? gemv::Gemv<VLRF_HIP_DT_Q8_0>::EPL : gemv::Gemv<VLRF_HIP_DT_Q4_0>::EPL);
    return (K + cw - 1) / cw;
}

}  // namespace

// Applies where the per-kernel step would run the M = 1 GEMV with one row per
// wave for the projection (d_model <= 2048) and the chunked decode attention
// (d_head 64, at most 8 KV heads, at most 15 chunks: 16 partials per head).
bool qkv_attn_supported(int w_dtype, int N, int K, int nch, int n_kv) {
    if (w_dtype != VLRF_HIP_DT_Q8_0 && w_dtype != VLRF_HIP_DT_Q4_0) return false;
    const int nc = qkv_chunks(w_dtype, K);
    if (nc > (w_dtype == VLRF_HIP_DT_Q8_0 ? 2 : 1) || K > kQkvAttnMaxD) return false;
    return nch > 0 && nch + 1 <= kAttnMaxChunks && n_kv >= 1 && n_kv <= 8 &&
           (N + gemv::kGemvWaves - 1) / gemv::kGemvWaves <= gemv::kGemvMaxOneGroups && N == K + 2 * n_kv * attn::D;
}

int qkv_attn_blocks(int rep, int n_kv, int nch) { return 8 * rep * ((n_kv * nch + 7) / 8); }

int launch_qkv_attn(hipStream_t s, const QkvAttnParams& p, int w_dtype, int kv_dtype, bool gather) {
    VH_ARG(qkv_attn_supported(w_dtype, p.N, p.K, p.fz.nch, p.fz.n_kv), "qkv_attn: shape not supported");
    VH_ARG(p.tags && p.status && p.state && p.fz.chunks && p.rep >= 1 && p.fz.n_kv * p.rep * attn::D == p.K,
           "qkv_attn: bad arguments");
    VH_ARG(p.nq % 8 == 0 && p.nq * gemv::kGemvWaves >= p.N, "qkv_attn: %d projection workgroups for %d rows", p.nq,
           p.N);
    VH_ARG(!gather || p.x_copy, "qkv_attn: the gather needs the residual stream");
    // An F32 cache's rounds need more registers than this kernel keeps (it would spill).
    VH_ARG(kv_dtype == VLRF_HIP_KV_Q8_0 || kv_dtype == VLRF_HIP_KV_F16, "qkv_attn: cache dtype %d not fused", kv_dtype);
    VH_ARG(p.na == qkv_attn_blocks(p.rep, p.fz.n_kv, p.fz.nch), "qkv_attn: %d attention workgroups", p.na);
    const dim3 grid(p.nq + p.na + 1), block(gemv::kGemvThreads);
    const int nc = qkv_chunks(w_dtype, p.K);
#define VH_QA(WT, KT, NC)                                                                                  \
    do {                                                                                                   \
        if (gather) VH_LAUNCH((qkv_attn_kernel<WT, KT, NC, true>), grid, block, 0, s, p);                  \
        else VH_LAUNCH((qkv_attn_kernel<WT, KT, NC, false>), grid, block, 0, s, p);                        \
    } while (0)
#define VH_QA_KV(WT, NC)                                               \
    if (kv_dtype == VLRF_HIP_KV_Q8_0) VH_QA(WT, VLRF_HIP_KV_Q8_0, NC); \
    else VH_QA(WT, VLRF_HIP_KV_F16, NC);
    if (w_dtype == VLRF_HIP_DT_Q8_0) {
        if (nc == 1) { VH_QA_KV(VLRF_HIP_DT_Q8_0, 1) }
        else { VH_QA_KV(VLRF_HIP_DT_Q8_0, 2) }
    } else {
        VH_QA_KV(VLRF_HIP_DT_Q4_0, 1)
    }
#undef VH_QA_KV
#undef VH_QA
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

}  // namespace vlrf_hip
