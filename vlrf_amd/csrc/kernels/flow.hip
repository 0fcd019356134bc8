// flow.hip - one decode step of the whole model as ONE kernel launch.
//
// Reference: TransformerModel::forward for one token with the KV cache
// (transformer.hpp:335-424), pre-norm blocks (transformer_block.hpp:141-159),
// AttentionBlock::forward (attention.hpp:89-186), FeedForward::forward SwiGLU
// (feedforward.hpp:50-77), greedy argmax (transformer.hpp:43-47).
//
// Design.  The per-kernel step pays a launch, a first-byte latency and a
// ramp-down at every one of its 5 kernels per layer.  Here the workgroups of
// all phases of all layers form one grid, ordered by dependency:
//
//   per layer: QKV | attention (+ the chunks' merge) | O + residual | gate/up | down
//   then:      LM head | argmax
//
// Each workgroup first issues the loads that do not depend on this step (its
// weight rows, its block of KV cache rows, the RoPE table row), then waits for
// its inputs, which lower-numbered workgroups publish as tagged 64-bit words:
// value bits in the low half, the step's epoch in the high half, written with
// one device-scope store.  A word is valid when its tag is the current epoch,
// so a reader needs no fence, no flag and no counter (the word is its own
// flag), and the buffers never need clearing (every layer has its own,
// rewritten once per step).  Readers poll with cache-bypassing (sc1) loads:
// the L2 of another XCD would otherwise keep serving the stale line.  A failed
// poll waits on one "gate" word, written by a producer that finishes late,
// before polling everything again, which keeps the workgroups that are already
// resident for later phases from flooding the fabric (measured in isolation:
// 2.9 -> 1.85 us per exchange).
//
// Progress: the hardware dispatches a kernel's workgroups in increasing order
// on each XCD and a workgroup only waits for lower-numbered ones, so the
// lowest unfinished workgroup is always resident or dispatchable: no co-
// residency is assumed.  Every wait is bounded anyway (FlowParams::limit on
// the wall clock): a wait that runs out records the failure in `status`, and
// every other wait sees the flag and leaves, so the grid always drains and the
// host reports the error.
//
// Arithmetic: every phase runs the code of the per-kernel step
// (gemv_core.hpp, attn_core.hpp) on the same operands in the same order; the
// two steps agree to a few ULP (the compiler may contract a multiply-add
// differently in the two contexts) and give the same token streams.
#include "../internal.hpp"
#include "attn_core.hpp"
#include "gemv_core.hpp"
#include "tagged.hpp"

#include <algorithm>

namespace vlrf_hip {
namespace {

using namespace tagged;
using gemv::Gemv;
using gemv::GemvRegs;
using gemv::kGemvThreads;
using gemv::kGemvWaves;
using gemv::Shape;

constexpr int kPart = kAttnChunkStride;      // words per (head, chunk) partial: acc[64], m, l, 2 pad
constexpr int kChunkRows = 512;              // cache rows per attention workgroup (8 waves x 64)
constexpr int kRpwQKV = 2, kRpwGU = 2;       // rows per wave of the QKV and gate/up phases

enum : int { kPhQKV = 1, kPhAtt, kPhO, kPhGU, kPhDown, kPhLM, kPhArgmax };

static_assert(sizeof(FlowParams) <= 4096, "the one-launch step's arguments exceed 4 KiB");

struct Smem {
    float red[kGemvWaves];
    int ok[kGemvWaves];   // per-wave poll results (block_ok)
    float best[kGemvWaves];
    int bidx[kGemvWaves];
};

template <int WT, int KVT, int NCD, int NCF>
struct Step {
    static constexpr int NTH = kGemvThreads;
    // LDS: the staged x of the widest phase, or the attention's workspace and
    // its merge of the head's chunk partials.
    static constexpr int kStageBytes = std::max(Shape<WT, NCD>::XF4, Shape<WT, NCF>::XF4) * 16;
    static constexpr int kAttBytes = (int)sizeof(attn::Smem<8>) + kAttnMaxChunks * kPart * 4;
    static constexpr int kPoolBytes = std::max(kStageBytes, kAttBytes);

    // ---- a GEMV phase: 8 waves x RPW rows each, rows (blk*8 + wave)*RPW + r ---------
    // x from the tagged vector at word xw (or, layer 0's QKV, the embedding row
    // of the token, x_plain), times norm_w when NORM; residual (RPW 1) from the
    // tagged word res_w + row, or res_plain[row]; output tagged at out_w + row.
    template <int NC, int NM, int RPW, bool NORM>
    static __device__ void gemv_phase(const Ctl& c, Smem& sm, float4* xs4, const FlowParams& P, const uint8_t* qa,
                                      const __half* da, const uint8_t* qb, const __half* db, int N, int K, int blk,
                                      long long xw, const float* x_plain, const float* norm_w, long long res_w,
                                      const float* res_plain, long long out_w) {
        using S = Shape<WT, NC>;
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int row0 = (blk * kGemvWaves + wave) * RPW;
        GemvRegs<NM, RPW, NC> A;
        gemv::gemv_load<WT, NM, RPW, NC>(A, qa, da, qb, db, row0, N, K, lane);
        float4 v[S::PER], gw[S::PER];
        if constexpr (NORM) load_norm<WT, NC>(norm_w, K, gw);
        float res = 0.f;
        if (RPW == 1 && res_plain) res = res_plain[min(row0, N - 1)];
        issue_before_wait();
        bool ok = true;
        if (x_plain) {
#pragma unroll
            for (int p = 0; p < S::PER; ++p) {
                const int f = tid + p * NTH;
                const bool in = f < S::XF4 && 4 * f < K;
                const float4 t = reinterpret_cast<const float4*>(x_plain)[in ? f : 0];
                v[p] = in ? t : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        } else {
            ok = poll_x<WT, NC>(c, xw, K, v);
        }
        if (RPW == 1 && res_w >= 0 && ok) ok = poll_word(c, (int)((res_w + min(row0, N - 1)) * 8), lane == 0, &res);
        if (!block_ok(ok, sm.ok)) return;
        float inv;
        gemv::gemv_stage<WT, NC, NORM>(v, gw, xs4, sm.red, K, P.eps, inv);
        const bool with_res = RPW == 1 && (res_plain || res_w >= 0);
        if (row0 < N)
            gemv::gemv_compute<WT, NM, RPW, NC, NM == 2>(A, xs4, inv, row0, N, K, lane, [&](int row, float o) {
                if (lane == 0 && row < N) {
                    if (with_res) o = o + res;
                    put_word(P.arena + out_w + row, __float_as_uint(o), c.tag);
                }
            });
    }

    // ---- attention: query head h over one 512-row chunk of the cache --------------
    // The head's last chunk (its highest workgroup) also merges the head's
    // chunk partials into the attention output, with the log-sum-exp rule and
    // operation order of gemv::gemv_merge.
    static __device__ void att_phase(const Ctl& c, unsigned char* pool, Smem& fs, const FlowParams& P, int l, int b) {
        attn::Smem<8>& sm = *reinterpret_cast<attn::Smem<8>*>(pool);
        float* raw = reinterpret_cast<float*>(pool + sizeof(attn::Smem<8>));   // [nch][kPart]
        const int rep = P.rep, nch = P.nch;
        // The REP query heads of chunk (g, s) run on one XCD (workgroup b % 8):
        // the chunk's K/V rows come from HBM once, then from that L2.
        const int k = b >> 3, r = k % rep, pc = (b & 7) + 8 * (k / rep);
        if (pc >= P.G * nch) return;
        const int g = pc / nch, chunk = pc - g * nch, h = g * rep + r, c0 = chunk * kChunkRows;
        const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
        const FlowLayer& Ly = P.layers[l];
        const int cap = P.S;
        const size_t hb = (size_t)g * cap * attn::D;
        attn::Round<KVT> R;
        attn::load_round<KVT>(R, Ly.kc, Ly.vc, Ly.ks, Ly.vs, hb, c0 + w * 64, cap, lane);
        const int pos = min(P.state[1], cap - 1);   // the host checks capacity before queuing
        const int ctx = pos + 1;
        DecodeFuse fz;
        fz.cos_t = P.cos_t;
        fz.sin_t = P.sin_t;
        fz.kq_w = Ly.kc;
        fz.vq_w = Ly.vc;
        fz.ks_w = Ly.ks;
        fz.vs_w = Ly.vs;
        fz.n_kv = P.G;
        fz.max_seq = P.S;
        attn::NewRow nr;
        attn::rope_row(nr, fz, pos);
        issue_before_wait();
        const long long pw0 = P.a.part + (long long)l * P.a.ld_part + (long long)h * nch * kPart;
        const long long pw = pw0 + (long long)chunk * kPart;
        if (c0 >= ctx) {   // past the context: the empty partial (acc 0, m -inf, l 0)
            if (tid < attn::D) put_word(P.arena + pw + tid, 0u, c.tag);
            if (tid == 0) {
                put_word(P.arena + pw + 64, __float_as_uint(attn::kNegInf), c.tag);
                put_word(P.arena + pw + 65, 0u, c.tag);
                put_word(P.arena + pw + 66, 0u, c.tag);
                put_word(P.arena + pw + 67, 0u, c.tag);
            }
        } else {
            // Inputs from the QKV phase: q (wave 0: dims j, j + 32), the new row's
            // K pair and V element of this thread (all n_kv heads: the Q8_0 row
            // scale covers the whole row).
            const long long qw = P.a.qkv + (long long)l * P.a.ld_qkv;
            const int npairs = P.G * attn::HALF, nrow = P.G * attn::D;
            const int j = lane & (attn::HALF - 1);
            const int i = min(tid, npairs - 1), hh = i / attn::HALF, jj = i - hh * attn::HALF;
            int off[5] = {(int)((qw + h * attn::D + j) * 8), (int)((qw + h * attn::D + j + attn::HALF) * 8),
                          (int)((qw + P.D + hh * attn::D + jj) * 8),
                          (int)((qw + P.D + hh * attn::D + jj + attn::HALF) * 8),
                          (int)((qw + P.D + nrow + min(tid, nrow - 1)) * 8)};
            bool use[5] = {w == 0, w == 0, tid < npairs, tid < npairs, tid < nrow};
            u32x2 v[5];
            const bool ok = poll<5, u32x2>(c, off, use, v, (int)((qw + P.D + 2 * nrow - 1) * 8));
            if (!block_ok(ok, fs.ok)) return;
            nr.k0 = __uint_as_float(v[2].x);
            nr.k1 = __uint_as_float(v[3].x);
            nr.vn = __uint_as_float(v[4].x);
            const bool rot = pos < P.S;
            const bool has_new = pos >= c0 && pos < c0 + kChunkRows;
            attn::chunk<KVT, true, 8>(sm, R, __uint_as_float(v[0].x), __uint_as_float(v[1].x), nr, r == 0, h == 0, g,
                                      c0, cap, hb, ctx, pos, rot, has_new, P.scale, fz,
                                      [&](int t, float ot, float mt, float lt) {
                                          put_word(P.arena + pw + t, __float_as_uint(ot), c.tag);
                                          if (t == 0) {
                                              put_word(P.arena + pw + 64, __float_as_uint(mt), c.tag);
                                              put_word(P.arena + pw + 65, __float_as_uint(lt), c.tag);
                                              put_word(P.arena + pw + 66, 0u, c.tag);
                                              put_word(P.arena + pw + 67, 0u, c.tag);
                                          }
                                      });
        }
        if (chunk != nch - 1) return;
        // ---- the head's merger: every chunk partial (16-byte pieces, at most one per
        // thread), gated on the chunk holding the token (the one that finishes last).
        const int npieces = nch * kPart / 2;
        int off[1] = {(int)((pw0 + 2 * min(tid, npieces - 1)) * 8)};
        bool use[1] = {tid < npieces};
        u32x4 v[1];
        const bool ok = poll<1, u32x4>(c, off, use, v, (int)((pw0 + (long long)P.gate_chunk * kPart) * 8));
        if (use[0]) {
            raw[2 * tid] = __uint_as_float(v[0].x);
            raw[2 * tid + 1] = __uint_as_float(v[0].z);
        }
        if (!block_ok(ok, fs.ok)) return;
        if (tid < attn::D) {
            float mt = gemv::kNegInfF;
            for (int cc = 0; cc < nch; ++cc) mt = fmaxf(mt, raw[cc * kPart + 64]);
            float lt = 0.f, o = 0.f;
            for (int cc = 0; cc < nch; ++cc) {
                const float m = raw[cc * kPart + 64];
                if (m != gemv::kNegInfF) {
                    const float wgt = expf(m - mt);
                    lt += wgt * raw[cc * kPart + 65];
                    o += wgt * raw[cc * kPart + tid];
                }
            }
            const float il = lt > 0.f ? 1.f / lt : 0.f;
            put_word(P.arena + P.a.att + (long long)l * P.a.ld_x + h * attn::D + tid, __float_as_uint(o * il), c.tag);
        }
    }

    // ---- LM head over the final norm + the block's first maximum --------------------
    static __device__ void lm_phase(const Ctl& c, Smem& sm, float4* xs4, const FlowParams& P, int blk) {
        using S = Shape<WT, NCD>;
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int N = P.V, K = P.D;
        const int rstep = P.plan.nlm * kGemvWaves;
        int row0 = blk * kGemvWaves + wave;
        GemvRegs<1, 1, NCD> A, B;
        gemv::gemv_load<WT, 1, 1, NCD>(A, P.lm_q, P.lm_d, nullptr, nullptr, row0, N, K, lane);
        gemv::gemv_load<WT, 1, 1, NCD>(B, P.lm_q, P.lm_d, nullptr, nullptr, row0 + rstep, N, K, lane);
        float4 v[S::PER], gw[S::PER];
        load_norm<WT, NCD>(P.ln_final, K, gw);
        issue_before_wait();
        const bool ok = poll_x<WT, NCD>(c, P.a.x2 + (long long)(P.L - 1) * P.a.ld_x, K, v);
        if (!block_ok(ok, sm.ok)) return;
        float inv;
        gemv::gemv_stage<WT, NCD, true>(v, gw, xs4, sm.red, K, P.eps, inv);
        // First maximum of the rows the wave visits (rows ascend; ties keep the
        // lower index), as std::max_element over the logits.
        float best = -INFINITY;
        int idx = -1;
        auto store = [&](int row, float o) {
            if (row < N) {
                if (lane == 0) P.logits[row] = o;
                if (idx < 0 || best < o) { best = o; idx = row; }
            }
        };
        for (; row0 < N; row0 += 2 * rstep) {
            const int r1 = row0 + rstep;
            gemv::gemv_compute<WT, 1, 1, NCD, false>(A, xs4, inv, row0, N, K, lane, store);
            if (r1 >= N) break;
            const int r2 = r1 + rstep;
            gemv::gemv_load<WT, 1, 1, NCD>(A, P.lm_q, P.lm_d, nullptr, nullptr, r2, N, K, lane);
            gemv::gemv_compute<WT, 1, 1, NCD, false>(B, xs4, inv, r1, N, K, lane, store);
            if (r2 >= N) break;
            gemv::gemv_load<WT, 1, 1, NCD>(B, P.lm_q, P.lm_d, nullptr, nullptr, r2 + rstep, N, K, lane);
        }
        if (lane == 0) { sm.best[wave] = best; sm.bidx[wave] = idx; }
        __syncthreads();
        if (tid == 0) {
            best = sm.best[0];
            idx = sm.bidx[0];
            for (int w2 = 1; w2 < kGemvWaves; ++w2) {
                const float ov = sm.best[w2];
                const int oi = sm.bidx[w2];
                if (oi >= 0 && (idx < 0 || best < ov || (best == ov && oi < idx))) { best = ov; idx = oi; }
            }
            uint64_t* o = P.arena + P.a.lm + 2 * blk;
            put_word(o, __float_as_uint(best), c.tag);
            put_word(o + 1, (uint32_t)idx, c.tag);
        }
    }

    // ---- argmax over the LM blocks' maxima; the step state advances ------------------
    static __device__ void argmax_phase(const Ctl& c, Smem& sm, const FlowParams& P) {
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int n = P.plan.nlm;
        int off[1] = {(int)((P.a.lm + 2 * min(tid, n - 1)) * 8)};
        bool use[1] = {tid < n};
        u32x4 r[1];
        const bool ok = poll<1, u32x4>(c, off, use, r, (int)((P.a.lm + 2 * (n - 1) + 1) * 8));
        if (!block_ok(ok, sm.ok)) return;
        float best = tid < n ? __uint_as_float(r[0].x) : -INFINITY;
        int idx = tid < n ? (int)r[0].z : -1;
        auto take = [&](float ov, int oi) {
            if (oi >= 0 && (idx < 0 || best < ov || (best == ov && oi < idx))) { best = ov; idx = oi; }
        };
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(best, o);
            const int oi = __shfl_xor(idx, o);
            take(ov, oi);
        }
        if (lane == 0) { sm.best[wave] = best; sm.bidx[wave] = idx; }
        __syncthreads();
        if (tid == 0) {
            best = sm.best[0];
            idx = sm.bidx[0];
            for (int w2 = 1; w2 < kGemvWaves; ++w2) take(sm.best[w2], sm.bidx[w2]);
            const int tok = idx < 0 ? 0 : idx;
            P.state[0] = tok;
            const int g = P.state[2];
            if (g < P.gen_cap) P.gen_ids[g] = tok;
            P.state[2] = g + 1;
            P.state[1] = P.state[1] + 1;
            // Last: every workgroup of the step has read the epoch (each published
            // a word tagged with it, and this workgroup consumed them all).
            P.state[3] = (int)(c.tag + 1u);
        }
    }
};

// At most 128 VGPRs (4 waves per SIMD): two workgroups per CU stay resident,
// so a phase's successors are already streaming their weights while it waits.
template <int WT, int KVT, int NCD, int NCF>
__global__ __launch_bounds__(gemv::kGemvThreads) __attribute__((amdgpu_waves_per_eu(4))) void flow_step_kernel(
    FlowParams P) {
    using St = Step<WT, KVT, NCD, NCF>;
    __shared__ Smem sm;
    __shared__ __align__(16) unsigned char pool[St::kPoolBytes];
    const FlowPlan& pl = P.plan;
    const int b = blockIdx.x;
    Ctl c;
    c.rs = __builtin_amdgcn_make_buffer_rsrc(P.arena, 0, (int)(P.a.words * 8), 0x00020000);
    c.status = P.status;
    c.t0 = wall_clock64();
    c.limit = P.limit;
    c.layer = b < P.L * pl.per_layer ? b / pl.per_layer : P.L;
    int r = b - c.layer * pl.per_layer;
    c.tag = (uint32_t)P.state[3];
    float4* xs4 = reinterpret_cast<float4*>(pool);
    const int l = c.layer;
    if (l < P.L) {
        const FlowLayer& Ly = P.layers[l];
        const long long x2prev = P.a.x2 + (long long)(l - 1) * P.a.ld_x;
        const float* emb = P.embed + (size_t)P.state[0] * P.D;   // layer 0's input: the token's row
        if (r < pl.nq) {
            c.phase = kPhQKV;
            St::template gemv_phase<NCD, 1, kRpwQKV, true>(c, sm, xs4, P, Ly.q[0], Ly.d[0], nullptr, nullptr,
                                                           P.D + 2 * P.G * attn::D, P.D, r, x2prev,
                                                           l == 0 ? emb : nullptr, Ly.ln1, -1, nullptr,
                                                           P.a.qkv + (long long)l * P.a.ld_qkv);
            return;
        }
        r -= pl.nq;
        if (r < pl.na) {
            c.phase = kPhAtt;
            St::att_phase(c, pool, sm, P, l, r);
            return;
        }
        r -= pl.na;
        if (r < pl.no) {
            c.phase = kPhO;
            St::template gemv_phase<NCD, 1, 1, false>(c, sm, xs4, P, Ly.q[1], Ly.d[1], nullptr, nullptr, P.D, P.D, r,
                                                      P.a.att + (long long)l * P.a.ld_x, nullptr, nullptr,
                                                      l == 0 ? -1 : x2prev, l == 0 ? emb : nullptr,
                                                      P.a.x1 + (long long)l * P.a.ld_x);
            return;
        }
        r -= pl.no;
        if (r < pl.ngu) {
            c.phase = kPhGU;
            St::template gemv_phase<NCD, 2, kRpwGU, true>(c, sm, xs4, P, Ly.q[2], Ly.d[2], Ly.q[3], Ly.d[3], P.F,
                                                          P.D, r, P.a.x1 + (long long)l * P.a.ld_x, nullptr, Ly.ln2,
                                                          -1, nullptr, P.a.h + (long long)l * P.a.ld_h);
            return;
        }
        r -= pl.ngu;
        c.phase = kPhDown;
        St::template gemv_phase<NCF, 1, 1, false>(c, sm, xs4, P, Ly.q[4], Ly.d[4], nullptr, nullptr, P.D, P.F, r,
                                                  P.a.h + (long long)l * P.a.ld_h, nullptr, nullptr,
                                                  P.a.x1 + (long long)l * P.a.ld_x, nullptr,
                                                  P.a.x2 + (long long)l * P.a.ld_x);
        return;
    }
    if (r < pl.nlm) {
        c.phase = kPhLM;
        St::lm_phase(c, sm, xs4, P, r);
        return;
    }
    if (r == pl.nlm) {
        c.phase = kPhArgmax;
        St::argmax_phase(c, sm, P);
    }
}

constexpr int ceil8(int n) { return (n + 7) / 8 * 8; }
int nchunks(int w_dtype, int K) {
    const int cw = 64 * (w_dtype == VLRF_DT_Q8_0 ? Gemv<VLRF_DT_Q8_0>::EPL : Gemv<VLRF_DT_Q4_0>::EPL);
    return (K + cw - 1) / cw;
}

// The instantiated chunk counts (activation chunks of a d_model row, of a
// d_ff row): Q8_0 (1, 1) and (2, 6), Q4_0 (1, 1) and (1, 3).
bool pick_nc(int w_dtype, int D, int F, int* ncd, int* ncf) {
    const int a = nchunks(w_dtype, D), b = nchunks(w_dtype, F);
    if (a <= 1 && b <= 1) { *ncd = 1; *ncf = 1; return true; }
    if (w_dtype == VLRF_DT_Q8_0 && a <= 2 && b <= 6) { *ncd = 2; *ncf = 6; return true; }
    if (w_dtype == VLRF_DT_Q4_0 && a <= 1 && b <= 3) { *ncd = 1; *ncf = 3; return true; }
    return false;
}

}  // namespace

// The one-launch step applies when the per-kernel step would use the M = 1
// GEMV and the chunked decode attention for every phase: Q8_0/Q4_0 weights
// (the LM head in the same format), d_head 64, at most 8 KV heads, activation
// widths with an instantiated chunk count, at most kFlowMaxLayers layers and
// 15 cache chunks (7680 rows).
FlowShape flow_shape(int w_dtype, int lm_dtype, int kv_dtype, int L, int D, int F, int H, int G, int dh, int V,
                     int S) {
    FlowShape f;
    int ncd = 0, ncf = 0;
    if ((w_dtype != VLRF_DT_Q8_0 && w_dtype != VLRF_DT_Q4_0) || lm_dtype != w_dtype) return f;
    if (kv_dtype != VLRF_KV_Q8_0 && kv_dtype != VLRF_KV_F16 && kv_dtype != VLRF_KV_F32) return f;
    if (dh != attn::D || G < 1 || G > 8 || H % G != 0 || D != H * dh || L < 1 || L > kFlowMaxLayers) return f;
    if (D % 32 || F % 32 || !pick_nc(w_dtype, D, F, &ncd, &ncf)) return f;
    const int nch = (S + kChunkRows - 1) / kChunkRows;
    if (nch > kAttnMaxChunks || nch * kPart / 2 > kGemvThreads) return f;   // the merger polls one piece per thread
    const int rep = H / G;
    f.nch = nch;
    FlowPlan& p = f.plan;
    p.nq = ceil8((D + 2 * G * dh + kGemvWaves * kRpwQKV - 1) / (kGemvWaves * kRpwQKV));
    p.na = 8 * rep * ((G * nch + 7) / 8);
    p.no = ceil8((D + kGemvWaves - 1) / kGemvWaves);
    p.ngu = ceil8((F + kGemvWaves * kRpwGU - 1) / (kGemvWaves * kRpwGU));
    p.nd = p.no;
    p.per_layer = p.nq + p.na + p.no + p.ngu + p.nd;
    p.nlm = std::min(ceil8((V + kGemvWaves - 1) / kGemvWaves), gemv::kGemvMaxGroups);
    p.total = L * p.per_layer + p.nlm + 8;
    auto even = [](long long n) { return (n + 1) / 2 * 2; };
    FlowArena& a = f.a;
    a.ld_qkv = (int)even(D + 2 * G * dh);
    a.ld_part = H * nch * kPart;
    a.ld_x = (int)even(D);
    a.ld_h = (int)even(F);
    long long o = 0;
    a.qkv = o; o += (long long)L * a.ld_qkv;
    a.part = o; o += (long long)L * a.ld_part;
    a.att = o; o += (long long)L * a.ld_x;
    a.x1 = o; o += (long long)L * a.ld_x;
    a.h = o; o += (long long)L * a.ld_h;
    a.x2 = o; o += (long long)L * a.ld_x;
    a.lm = o; o += 2LL * p.nlm;
    a.words = even(o);
    if (a.words * 8 >= (1LL << 31)) return f;   // byte offsets are 32-bit
    f.ok = true;
    return f;
}

// The gate of the attention merger's wait: the chunk holding the token at pos
// (the one with the most work: its rounds plus the row's quantization).
int flow_gate_chunk(const FlowShape& f, int pos) { return std::min(pos / kChunkRows, f.nch - 1); }

int launch_flow_step(hipStream_t s, const FlowParams& p) {
    VH_ARG(p.plan.total > 0 && p.arena && p.status && p.state, "flow: not planned");
    VH_ARG(p.L >= 1 && p.L <= kFlowMaxLayers, "flow: %d layers (at most %d)", p.L, kFlowMaxLayers);
    int ncd = 0, ncf = 0;
    VH_ARG(pick_nc(p.w_dtype, p.D, p.F, &ncd, &ncf), "flow: no instantiation for d_model %d / d_ff %d", p.D, p.F);
    const dim3 grid(p.plan.total), block(gemv::kGemvThreads);
#define VH_FLOW(WT, KT, A, B) hipLaunchKernelGGL((flow_step_kernel<WT, KT, A, B>), grid, block, 0, s, p)
#define VH_FLOW_KV(WT, A, B)                                      \
    switch (p.kv_dtype) {                                         \
        case VLRF_KV_Q8_0: VH_FLOW(WT, VLRF_KV_Q8_0, A, B); break; \
        case VLRF_KV_F16: VH_FLOW(WT, VLRF_KV_F16, A, B); break;   \
        default: VH_FLOW(WT, VLRF_KV_F32, A, B); break;            \
    }
    if (p.w_dtype == VLRF_DT_Q8_0) {
        if (ncd == 1) { VH_FLOW_KV(VLRF_DT_Q8_0, 1, 1) }
        else { VH_FLOW_KV(VLRF_DT_Q8_0, 2, 6) }
    } else {
        if (ncf == 1) { VH_FLOW_KV(VLRF_DT_Q4_0, 1, 1) }
        else { VH_FLOW_KV(VLRF_DT_Q4_0, 1, 3) }
    }
#undef VH_FLOW_KV
#undef VH_FLOW
    VH_LAUNCHED();
    return VLRF_HIP_OK;
}

}  // namespace vlrf_hip
