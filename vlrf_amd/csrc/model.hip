// model.hip - device-resident decode step of a Llama-style decoder.
//
// Reference: TransformerModel::forward (transformer.hpp:335-424) for one token
// with the KV cache, TransformerBlock::forward_v2 pre-norm order
// (transformer_block.hpp:141-159), AttentionBlock::forward (attention.hpp:89-186),
// FeedForward::forward SwiGLU (feedforward.hpp:50-77), greedy argmax
// (transformer.hpp:43-47).
//
// Per layer the step queues five kernels (six where the chunked attention
// form does not apply):
//   qlinear(Wqkv, rmsnorm(x; ln1))        Q,K,V in one pass over the fused rows
//   attn_decode                           RoPE on q,k and the Q8_0 append of the
//                                         token's K/V row, fused with attention
//                                         over the quantized cache: per query head
//                                         and 512-row chunk a (m, l, acc) partial
//                                         (else split-K partials + attn_combine)
//   qlinear(Wo, merge(chunks)) + x        the chunks' log-sum-exp merge in the
//                                         GEMV prologue, residual in the epilogue
//   swiglu(Wg, Wu, rmsnorm(x; ln2))       silu(g) * u in the epilogue
//   qlinear(Wd, h) + x
// then rmsnorm + LM head and argmax, which writes the next token id and
// advances the device-side position.  The token and position live in device
// memory, so the whole step is captured once as a HIP graph and replayed with
// no host round trip between steps.
//
#include "internal.hpp"
#include "runtime.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

using namespace vlrf_hip;

namespace {

enum : int { kLn1 = 0, kLn2, kQ, kK, kV, kO, kGate, kUp, kDown, kPerLayer };

struct Layer {
    float* ln1 = nullptr;
    float* ln2 = nullptr;
    DevWeight wqkv, wo, wg, wu, wd;
    KVLayer kv;
    unsigned set = 0;
};

}  // namespace

struct vlrf_hip_model {
    Ctx* ctx = nullptr;
    vlrf_hip_model_config cfg{};
    int D = 0, F = 0, H = 0, G = 0, dh = 0, dkv = 0, L = 0, V = 0, S = 0;
    float* embed = nullptr;
    float* ln_final = nullptr;
    DevWeight lm_head;
    bool embed_set = false, ln_final_set = false, lm_head_set = false;
    std::vector<Layer> layers;
    const float* cos_t = nullptr;
    const float* sin_t = nullptr;
    float *x = nullptr, *qkv = nullptr, *att = nullptr, *h = nullptr, *logits = nullptr, *part = nullptr;
    float2* argpairs = nullptr;   // [512] the LM head's per-workgroup (max, first index)
    int nch = 0;               // decode attention in chunked form (merged by the O GEMV) when > 0
    int nparts = 0;            // partials per head: nch, plus the token's own key when fused
    float* chunks = nullptr;   // its partials [H][nparts][kAttnChunkStride]
    int* state = nullptr;      // [0] token, [1] position, [2] generated count, [3] epoch (>= 1)
    int* gen_ids = nullptr;    // [S]
    int* prompt = nullptr;     // [S] staged prompt ids
    int* pinned = nullptr;     // host pinned [8]
    int n_splits = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    // kGraphSteps steps in one graph, for runs of that many steps: the gap
    // between two graph launches is paid once per kGraphSteps steps.
    hipGraph_t graph_n = nullptr;
    hipGraphExec_t exec_n = nullptr;
    bool use_graph = true;     // VLRF_HIP_GRAPH=0: queue the step's kernels directly
    // Fused QKV + attention launch (kernels/qkv_attn.hip) where it applies
    // (VLRF_HIP_QKV_ATTN=0 queues the two kernels instead).
    bool qkv_attn = false;
    bool chunk_new = false;         // d_head 128 chunked attention: the new key is partial nch
    uint64_t* qkv_tags = nullptr;   // [L][D + 2*dkv] tagged projection outputs
    int* step_status = nullptr;     // [4] failure flag, workgroup, phase, layer
    long long wait_limit = 0;       // wall-clock ticks a wait may last
    int pos = 0;               // host mirror of state[1]
    // Batched prefill (matrix cores) work buffers, sized for pf_cap rows.
    int pf_cap = 0;
    float* pf_x = nullptr;         // [T][D] residual stream
    float* pf_qkv = nullptr;       // [T][D + 2*dkv]
    uint16_t* pf_a = nullptr;      // [T][D] bf16 normalised rows
    uint16_t* pf_att = nullptr;    // [T][D] bf16 attention output
    uint16_t* pf_h = nullptr;      // [T][F] bf16 SwiGLU output
    int* pf_ids = nullptr;         // [T]
    float* pf_part = nullptr;      // K-split partial sums of the GEMMs of 17..128 rows
    size_t pf_part_bytes = 0;

    bool ready() const {
        if (!embed_set || !ln_final_set || !lm_head_set) return false;
        for (auto& l : layers)
            if (l.set != (1u << kPerLayer) - 1) return false;
        return true;
    }
};

namespace {

// Labels the launches that follow for an installed LaunchTimer.
void lk(int kind) {
    if (LaunchTimer* t = launch_timer()) t->cur_kind = kind;
}

int enqueue_step(vlrf_hip_model* m, hipStream_t s) {
    // Layer 0's QKV projection gathers the embedding row itself when it can.
    const bool gather = qlinear_gather_supported(m->layers[0].wqkv);
    lk(VLRF_HIP_LK_OTHER);
    int rc = gather ? VLRF_HIP_OK : launch_embed(s, m->embed, m->state, m->x, m->D);
    const float eps = m->cfg.norm_eps;
    const float scale = 1.f / std::sqrt((float)m->dh);   // attention.hpp:373-374
    for (int l = 0; l < m->L && !rc; ++l) {
        Layer& Ly = m->layers[l];
        float* q = m->qkv;
        float* k = m->qkv + m->D;
        float* v = m->qkv + m->D + m->dkv;
        DecodeFuse fz;
        fz.k_new = k;
        fz.v_new = v;
        fz.cos_t = m->cos_t;
        fz.sin_t = m->sin_t;
        fz.kq_w = Ly.kv.k;
        fz.vq_w = Ly.kv.v;
        fz.ks_w = Ly.kv.ks;
        fz.vs_w = Ly.kv.vs;
        fz.n_kv = m->G;
        fz.max_seq = m->S;
        fz.chunks = m->chunks;
        fz.nch = m->nch;
        if (m->qkv_attn) {   // one launch: the projection's rows feed the attention as tagged words
            QkvAttnParams p;
            p.qa = Ly.wqkv.q;
            p.da = Ly.wqkv.d;
            p.N = Ly.wqkv.N;
            p.K = Ly.wqkv.K;
            p.x = l == 0 && gather ? m->embed : m->x;
            p.x_copy = l == 0 && gather ? m->x : nullptr;
            p.norm_w = Ly.ln1;
            p.eps = eps;
            p.nq = (p.N + 63) / 64 * 8;
            p.rep = m->H / m->G;
            p.na = qkv_attn_blocks(p.rep, m->G, m->nch);
            p.tags = m->qkv_tags + (size_t)l * p.N;
            p.head_stride = (long)m->S * m->dh;
            p.fz = fz;
            p.scale = scale;
            p.state = m->state;
            p.status = m->step_status;
            p.limit = m->wait_limit;
            p.layer = l;
            lk(VLRF_HIP_LK_QKV);
            if (!rc) rc = launch_qkv_attn(s, p, m->cfg.weight_dtype, m->cfg.kv_dtype, l == 0 && gather);
        } else {
            lk(VLRF_HIP_LK_QKV);
            if (!rc) {
                if (l == 0 && gather)   // embedding_lookup (ops.hpp:615-626) fused: x = embed[token]
                    rc = launch_qlinear_gather(s, Ly.wqkv, m->embed, m->state, m->x, m->qkv, Ly.ln1, eps);
                else
                    rc = launch_qlinear(s, Ly.wqkv, m->x, m->qkv, 1, Ly.ln1, eps, nullptr);
            }
            lk(VLRF_HIP_LK_ATTN);
            if (!rc) rc = launch_attn_decode(s, q, Ly.kv.k, Ly.kv.v, Ly.kv.ks, Ly.kv.vs, Ly.kv.dtype,
                                             (long)m->S * m->dh, m->H, m->G, m->dh, 1, m->state + 1,
                                             m->n_splits, scale, m->part, m->att, &fz);
        }
        lk(VLRF_HIP_LK_O);
        if (!rc) rc = m->nch ? launch_qlinear_merge(s, Ly.wo, m->chunks, m->nparts, m->x, m->x, m->dh)
                             : launch_qlinear(s, Ly.wo, m->att, m->x, 1, nullptr, 0.f, m->x);
        lk(VLRF_HIP_LK_GATE_UP);
        if (!rc) rc = launch_qlinear_swiglu(s, Ly.wg, Ly.wu, m->x, m->h, 1, Ly.ln2, eps);
        lk(VLRF_HIP_LK_DOWN);
        if (!rc) rc = launch_qlinear(s, Ly.wd, m->h, m->x, 1, nullptr, 0.f, m->x);
    }
    if (qlinear_argmax_supported(m->lm_head)) {
        // The LM head's workgroups leave (max, first index) pairs: the argmax
        // step reduces those instead of the 32000 logits.
        int np = 0;
        lk(VLRF_HIP_LK_LM_HEAD);
        if (!rc) rc = launch_qlinear_argmax(s, m->lm_head, m->x, m->logits, m->ln_final, eps, m->argpairs, &np);
        lk(VLRF_HIP_LK_ARGMAX);
        if (!rc) rc = launch_argmax_pairs_step(s, m->argpairs, np, m->state, m->gen_ids, m->S);
    } else {
        lk(VLRF_HIP_LK_LM_HEAD);
        if (!rc) rc = launch_qlinear(s, m->lm_head, m->x, m->logits, 1, m->ln_final, eps, nullptr);
        lk(VLRF_HIP_LK_ARGMAX);
        if (!rc) rc = launch_argmax_step(s, m->logits, m->V, m->state, m->gen_ids, m->S);
    }
    return rc;
}

// Steps per launch of the multi-step graph: 16 steps in one graph ran
// 0.5258-0.5271 against 0.5294-0.5305 ms per step with one step per graph
// (4 steps: 0.5275-0.5282), same box.
constexpr int kGraphSteps = 16;

// Captures `steps` decode steps into *graph / *exec.
int capture_steps(vlrf_hip_model* m, int steps, hipGraph_t* graph, hipGraphExec_t* exec) {
    hipStream_t s = m->ctx->stream;
    VH_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int rc = VLRF_HIP_OK;
    for (int i = 0; i < steps && !rc; ++i) rc = enqueue_step(m, s);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s, &g);
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) {
        set_error("graph capture failed: %s", hipGetErrorString(e));
        return VLRF_HIP_ERR_RUNTIME;
    }
    *graph = g;
    VH_CHECK(hipGraphInstantiate(exec, g, nullptr, nullptr, 0));
    return VLRF_HIP_OK;
}

int ensure_graph(vlrf_hip_model* m) {
    if (m->exec || !m->use_graph) return VLRF_HIP_OK;
    int rc = capture_steps(m, 1, &m->graph, &m->exec);
    if (!rc) rc = capture_steps(m, kGraphSteps, &m->graph_n, &m->exec_n);
    return rc;
}

void drop_graphs(vlrf_hip_model* m) {
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    if (m->exec_n) (void)hipGraphExecDestroy(m->exec_n);
    if (m->graph_n) (void)hipGraphDestroy(m->graph_n);
    m->exec = m->exec_n = nullptr;
    m->graph = m->graph_n = nullptr;
}

// One decode step on the context stream: the captured graph, or the same
// kernels queued one by one when graphs are switched off.
int launch_step(vlrf_hip_model* m) {
    if (!m->use_graph) return enqueue_step(m, m->ctx->stream);
    VH_CHECK(hipGraphLaunch(m->exec, m->ctx->stream));
    return VLRF_HIP_OK;
}

// After the queued steps have finished: a launch whose wait for another
// workgroup's output ran out (the fused QKV + attention launch) left its flag; report it, clear it and move to a fresh
// epoch (the failed step may have published words of the old one), and take
// the device position as the host's.
int check_waits(vlrf_hip_model* m) {
    int* status = m->step_status;
    if (!status) return VLRF_HIP_OK;
    hipStream_t s = m->ctx->stream;
    int* st = m->pinned + 4;
    VH_CHECK(hipMemcpyAsync(st, status, 4 * sizeof(int), hipMemcpyDeviceToHost, s));
    VH_CHECK(hipStreamSynchronize(s));
    if (!st[0]) return VLRF_HIP_OK;
    const int blk = st[1], ph = st[2], layer = st[3];
    VH_CHECK(hipMemsetAsync(status, 0, 4 * sizeof(int), s));
    VH_CHECK(hipMemcpyAsync(m->pinned, m->state, 4 * sizeof(int), hipMemcpyDeviceToHost, s));
    VH_CHECK(hipStreamSynchronize(s));
    m->pinned[3] += 1;
    m->pos = m->pinned[1];
    VH_CHECK(hipMemcpyAsync(m->state, m->pinned, 4 * sizeof(int), hipMemcpyHostToDevice, s));
    VH_CHECK(hipStreamSynchronize(s));
    set_error("decode step: a wait for another workgroup's output ran out (workgroup %d, phase %d, layer %d)",
              blk, ph, layer);
    return VLRF_HIP_ERR_RUNTIME;
}

int check_ready(vlrf_hip_model* m) {
    VH_ARG(m != nullptr, "model: null handle");
    VH_CHECK(hipSetDevice(m->ctx->device));
    VH_ARG(m->ready(), "model: not every weight has been set");
    return ensure_graph(m);
}

int parse_layer(const std::string& name, int* layer, std::string* rest) {
    if (name.compare(0, 7, "layers.") != 0) return -1;
    size_t dot = name.find('.', 7);
    if (dot == std::string::npos) return -1;
    *layer = std::atoi(name.substr(7, dot - 7).c_str());
    *rest = name.substr(dot + 1);
    return 0;
}

int upload_f32(hipStream_t s, float* dst, const void* host, size_t n) {
    VH_CHECK(hipMemcpyAsync(dst, host, n * sizeof(float), hipMemcpyHostToDevice, s));
    VH_CHECK(hipStreamSynchronize(s));
    return VLRF_HIP_OK;
}

}  // namespace

extern "C" {

int vlrf_hip_model_create(vlrf_hip_ctx_t ctx, const vlrf_hip_model_config* cfg, vlrf_hip_model_t* out) {
    VH_ARG(ctx && cfg && out, "model_create: null argument");
    *out = nullptr;
    VH_CHECK(hipSetDevice(ctx->device));
    const auto& c = *cfg;
    // ModelConfig::check (config.hpp:127-140) plus what the kernels assume.
    VH_ARG(c.d_model > 0 && c.n_heads > 0 && c.d_model % c.n_heads == 0, "model: d_model %% n_heads != 0");
    VH_ARG(c.n_kv_heads > 0 && c.n_heads % c.n_kv_heads == 0, "model: n_heads %% n_kv_heads != 0");
    VH_ARG(c.n_layers > 0 && c.max_seq_len > 0 && c.vocab_size > 0 && c.d_ff > 0, "model: bad sizes");
    const int dh = c.d_model / c.n_heads;
    VH_ARG(dh == 64 || dh == 128, "model: d_head %d not in {64,128}", dh);
    const int rep = c.n_heads / c.n_kv_heads;
    VH_ARG(rep == 1 || rep == 2 || rep == 4 || rep == 8, "model: GQA group %d not in {1,2,4,8}", rep);
    VH_ARG(c.n_kv_heads * dh <= 1024, "model: kv row %d exceeds 1024", c.n_kv_heads * dh);
    VH_ARG(c.d_model % 32 == 0 && c.d_ff % 32 == 0, "model: d_model and d_ff must be multiples of 32");
    VH_ARG(c.weight_dtype == VLRF_HIP_DT_Q8_0 || c.weight_dtype == VLRF_HIP_DT_Q4_0 || c.weight_dtype == VLRF_HIP_DT_F32,
           "model: unsupported weight dtype %d", c.weight_dtype);
    VH_ARG(c.kv_dtype == VLRF_HIP_KV_F32 || c.kv_dtype == VLRF_HIP_KV_F16 || c.kv_dtype == VLRF_HIP_KV_Q8_0,
           "model: unsupported KV cache dtype %d", c.kv_dtype);

    auto* m = new (std::nothrow) vlrf_hip_model();
    if (!m) return VLRF_HIP_ERR_NOMEM;
    m->ctx = ctx;
    m->cfg = c;
    m->D = c.d_model; m->F = c.d_ff; m->H = c.n_heads; m->G = c.n_kv_heads; m->dh = dh;
    m->dkv = c.n_kv_heads * dh; m->L = c.n_layers; m->V = c.vocab_size; m->S = c.max_seq_len;
    m->n_splits = attn_decode_splits(m->S);
    m->layers.resize(m->L);
    if (const char* g = std::getenv("VLRF_HIP_GRAPH")) m->use_graph = std::strcmp(g, "0") != 0;

    int rc = VLRF_HIP_OK;
    auto dalloc = [&](void** p, size_t bytes) {
        if (rc) return;
        if (hipMalloc(p, bytes) != hipSuccess) {
            set_error("model_create: hipMalloc(%zu) failed", bytes);
            rc = VLRF_HIP_ERR_NOMEM;
        }
    };
    dalloc((void**)&m->embed, (size_t)m->V * m->D * 4);
    dalloc((void**)&m->ln_final, (size_t)m->D * 4);
    dalloc((void**)&m->x, (size_t)m->D * 4);
    dalloc((void**)&m->qkv, (size_t)(m->D + 2 * m->dkv) * 4);
    dalloc((void**)&m->att, (size_t)m->D * 4);
    dalloc((void**)&m->h, (size_t)m->F * 4);
    dalloc((void**)&m->logits, (size_t)m->V * 4);
    dalloc((void**)&m->argpairs, 512 * sizeof(float2));
    dalloc((void**)&m->part, (size_t)m->H * m->n_splits * (dh + 2) * 4);
    // Chunked decode attention when the O projection's GEMV can merge it.
    m->nch = c.weight_dtype == VLRF_HIP_DT_Q8_0 || c.weight_dtype == VLRF_HIP_DT_Q4_0
                 ? attn_decode_chunks(m->S, dh, m->G) : 0;
    DevWeight wo_shape;
    wo_shape.dtype = c.weight_dtype;
    wo_shape.N = m->D;
    wo_shape.K = m->H * dh;
    if (m->nch && (wo_shape.K != m->D || m->nch > qlinear_merge_max_chunks(wo_shape))) m->nch = 0;
    // The fused QKV + attention launch, which always takes the chunked form
    // (one 512-row chunk for the caches the single-pass kernel would cover):
    // Q8_0/F16 caches (an F32 cache's rounds need more registers than the
    // fused kernel keeps: it would spill).
    const char* qa_env = std::getenv("VLRF_HIP_QKV_ATTN");
    if (!(qa_env && std::strcmp(qa_env, "0") == 0) && c.kv_dtype != VLRF_HIP_KV_F32 && dh == 64 && m->G <= 8 &&
        wo_shape.K == m->D) {
        const int n = (m->S + kAttnChunkRows - 1) / kAttnChunkRows;
        if (n + 1 <= qlinear_merge_max_chunks(wo_shape) &&
            qkv_attn_supported(c.weight_dtype, m->D + 2 * m->dkv, m->D, n, m->G)) {
            m->nch = n;
            m->qkv_attn = true;
        }
    }
    // d_head 128 (the 8B shape): the chunked form with the new key as its own
    // partial, where the O projection's GEMV can merge nch + 1 partials.
    if (dh == 128 && (c.weight_dtype == VLRF_HIP_DT_Q8_0 || c.weight_dtype == VLRF_HIP_DT_Q4_0) && wo_shape.K == m->D) {
        const int n = attn_decode_chunks128(m->S, m->H, m->G, c.kv_dtype);
        if (n && n + 1 <= qlinear_merge_max_chunks(wo_shape)) {
            m->nch = n;
            m->chunk_new = true;
        }
    }
    m->nparts = m->nch + (m->qkv_attn || m->chunk_new ? 1 : 0);
    if (m->nch) dalloc((void**)&m->chunks, (size_t)m->H * m->nparts * (dh + 4) * 4);
    // Zero words carry no epoch (the epoch starts at 1).
    auto tagged = [&](uint64_t** p, size_t words) {
        dalloc((void**)p, words * 8);
        if (!rc && hipMemset(*p, 0, words * 8) != hipSuccess) {
            set_error("model_create: clearing the tagged words failed");
            rc = VLRF_HIP_ERR_RUNTIME;
        }
    };
    if (m->qkv_attn) tagged(&m->qkv_tags, (size_t)m->L * (m->D + 2 * m->dkv));
    if (m->qkv_attn) {
        dalloc((void**)&m->step_status, 4 * sizeof(int));
        if (!rc && hipMemset(m->step_status, 0, 4 * sizeof(int)) != hipSuccess) {
            set_error("model_create: clearing the status words failed");
            rc = VLRF_HIP_ERR_RUNTIME;
        }
    }
    {
        // A wait for another workgroup's output may last 0.5 s
        // (VLRF_HIP_WAIT_US overrides it: the tests shorten it to exercise the
        // failure path).
        int rate_khz = 0;
        if (!rc && hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, ctx->device) != hipSuccess) {
            set_error("model_create: no wall-clock rate");
            rc = VLRF_HIP_ERR_RUNTIME;
        }
        long long wait_us = 500000;
        if (const char* w = std::getenv("VLRF_HIP_WAIT_US")) wait_us = std::atoll(w);
        m->wait_limit = (long long)rate_khz * wait_us / 1000;
    }
    dalloc((void**)&m->state, 4 * sizeof(int));
    dalloc((void**)&m->gen_ids, (size_t)m->S * sizeof(int));
    dalloc((void**)&m->prompt, (size_t)m->S * sizeof(int));
    const size_t kvdata = (size_t)m->G * m->S * dh * kv_elem_bytes(c.kv_dtype);
    for (auto& Ly : m->layers) {
        dalloc((void**)&Ly.ln1, (size_t)m->D * 4);
        dalloc((void**)&Ly.ln2, (size_t)m->D * 4);
        Ly.kv.dtype = c.kv_dtype;
        dalloc((void**)&Ly.kv.k, kvdata);
        dalloc((void**)&Ly.kv.v, kvdata);
        if (c.kv_dtype == VLRF_HIP_KV_Q8_0) {
            dalloc((void**)&Ly.kv.ks, (size_t)m->S * 4);
            dalloc((void**)&Ly.kv.vs, (size_t)m->S * 4);
        }
        if (!rc) rc = weight_alloc(Ly.wqkv, c.weight_dtype, m->D + 2 * m->dkv, m->D);
        if (!rc) rc = weight_alloc(Ly.wo, c.weight_dtype, m->D, m->D);
        if (!rc) rc = weight_alloc(Ly.wg, c.weight_dtype, m->F, m->D);
        if (!rc) rc = weight_alloc(Ly.wu, c.weight_dtype, m->F, m->D);
        if (!rc) rc = weight_alloc(Ly.wd, c.weight_dtype, m->D, m->F);
    }
    if (!rc && hipHostMalloc((void**)&m->pinned, 8 * sizeof(int), hipHostMallocDefault) != hipSuccess) {
        set_error("model_create: hipHostMalloc failed");
        rc = VLRF_HIP_ERR_NOMEM;
    }
    if (!rc) {   // the epoch starts at 1: the zeroed tagged words carry none
        m->pinned[0] = m->pinned[1] = m->pinned[2] = 0;
        m->pinned[3] = 1;
        if (hipMemcpy(m->state, m->pinned, 4 * sizeof(int), hipMemcpyHostToDevice) != hipSuccess) {
            set_error("model_create: state upload failed");
            rc = VLRF_HIP_ERR_RUNTIME;
        }
    }
    if (!rc) rc = ctx->rope_tables(m->S, dh, c.rope_theta, &m->cos_t, &m->sin_t);
    if (!rc) rc = vlrf_hip_model_reset(m);
    if (rc) {
        vlrf_hip_model_destroy(m);
        return rc;
    }
    *out = m;
    return VLRF_HIP_OK;
}

void vlrf_hip_model_destroy(vlrf_hip_model_t m) {
    if (!m) return;
    (void)hipSetDevice(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    drop_graphs(m);
    for (auto& Ly : m->layers) {
        for (void* p : {(void*)Ly.ln1, (void*)Ly.ln2, (void*)Ly.kv.k, (void*)Ly.kv.v, (void*)Ly.kv.ks,
                        (void*)Ly.kv.vs})
            if (p) (void)hipFree(p);
        weight_release(Ly.wqkv);
        weight_release(Ly.wo);
        weight_release(Ly.wg);
        weight_release(Ly.wu);
        weight_release(Ly.wd);
    }
    weight_release(m->lm_head);
    for (void* p : {(void*)m->embed, (void*)m->ln_final, (void*)m->x, (void*)m->qkv, (void*)m->att,
                    (void*)m->h, (void*)m->logits, (void*)m->argpairs, (void*)m->part, (void*)m->chunks, (void*)m->state,
                    (void*)m->gen_ids, (void*)m->prompt})
        if (p) (void)hipFree(p);
    for (void* p : {(void*)m->pf_x, (void*)m->pf_qkv, (void*)m->pf_a, (void*)m->pf_att, (void*)m->pf_h,
                    (void*)m->pf_ids, (void*)m->pf_part, (void*)m->qkv_tags,
                    (void*)m->step_status})
        if (p) (void)hipFree(p);
    if (m->pinned) (void)hipHostFree(m->pinned);
    delete m;
}

int vlrf_hip_model_set_weight(vlrf_hip_model_t m, const char* name, const void* host, int dtype,
                              int rows, int cols) {
    VH_ARG(m && name && host, "set_weight: null argument");
    VH_CHECK(hipSetDevice(m->ctx->device));
    hipStream_t s = m->ctx->stream;
    const std::string n(name);
    auto need = [&](int dt, int r, int c) -> int {
        VH_ARG(dtype == dt && rows == r && cols == c,
               "set_weight %s: expected dtype %d [%d,%d], got dtype %d [%d,%d]", name, dt, r, c, dtype,
               rows, cols);
        return VLRF_HIP_OK;
    };
    int rc;
    if (n == "embed.weight") {
        if ((rc = need(VLRF_HIP_DT_F32, m->V, m->D))) return rc;
        if ((rc = upload_f32(s, m->embed, host, (size_t)m->V * m->D))) return rc;
        m->embed_set = true;
        return VLRF_HIP_OK;
    }
    if (n == "ln_final.weight") {
        if ((rc = need(VLRF_HIP_DT_F32, 1, m->D))) return rc;
        if ((rc = upload_f32(s, m->ln_final, host, m->D))) return rc;
        m->ln_final_set = true;
        return VLRF_HIP_OK;
    }
    if (n == "lm_head.weight") {
        VH_ARG(rows == m->V && cols == m->D, "set_weight lm_head: shape [%d,%d] != [%d,%d]", rows, cols,
               m->V, m->D);
        if (m->lm_head.dtype != dtype || !(m->lm_head.q || m->lm_head.f)) {
            VH_CHECK(hipStreamSynchronize(s));
            // The captured step graphs hold the old pointers: drop them.
            drop_graphs(m);
            weight_release(m->lm_head);
            if ((rc = weight_alloc(m->lm_head, dtype, m->V, m->D))) return rc;
        }
        if ((rc = weight_upload_rows(s, m->lm_head, host, 0, m->V))) return rc;
        m->lm_head_set = true;
        return VLRF_HIP_OK;
    }
    int l = -1;
    std::string rest;
    VH_ARG(parse_layer(n, &l, &rest) == 0 && l >= 0 && l < m->L, "set_weight: unknown tensor %s", name);
    Layer& Ly = m->layers[l];
    const int wdt = m->cfg.weight_dtype;
    if (rest == "ln1.weight" || rest == "ln2.weight") {
        if ((rc = need(VLRF_HIP_DT_F32, 1, m->D))) return rc;
        const bool one = rest == "ln1.weight";
        if ((rc = upload_f32(s, one ? Ly.ln1 : Ly.ln2, host, m->D))) return rc;
        Ly.set |= 1u << (one ? kLn1 : kLn2);
        return VLRF_HIP_OK;
    }
    struct Slot { const char* key; DevWeight* w; int row0, rows, cols, bit; };
    const Slot slots[] = {
        {"attn.q_proj.weight", &Ly.wqkv, 0, m->D, m->D, kQ},
        {"attn.k_proj.weight", &Ly.wqkv, m->D, m->dkv, m->D, kK},
        {"attn.v_proj.weight", &Ly.wqkv, m->D + m->dkv, m->dkv, m->D, kV},
        {"attn.o_proj.weight", &Ly.wo, 0, m->D, m->D, kO},
        {"ffn.gate.weight", &Ly.wg, 0, m->F, m->D, kGate},
        {"ffn.fc1.weight", &Ly.wu, 0, m->F, m->D, kUp},
        {"ffn.fc2.weight", &Ly.wd, 0, m->D, m->F, kDown},
    };
    for (const auto& sl : slots) {
        if (rest != sl.key) continue;
        if ((rc = need(wdt, sl.rows, sl.cols))) return rc;
        if ((rc = weight_upload_rows(s, *sl.w, host, sl.row0, sl.rows))) return rc;
        Ly.set |= 1u << sl.bit;
        return VLRF_HIP_OK;
    }
    set_error("set_weight: unknown tensor %s", name);
    return VLRF_HIP_ERR_ARG;
}

int vlrf_hip_model_reset(vlrf_hip_model_t m) {
    VH_ARG(m != nullptr, "model_reset: null handle");
    VH_CHECK(hipSetDevice(m->ctx->device));
    hipStream_t s = m->ctx->stream;
    const size_t kvdata = (size_t)m->G * m->S * m->dh * kv_elem_bytes(m->cfg.kv_dtype);
    for (auto& Ly : m->layers) {
        VH_CHECK(hipMemsetAsync(Ly.kv.k, 0, kvdata, s));
        VH_CHECK(hipMemsetAsync(Ly.kv.v, 0, kvdata, s));
        if (Ly.kv.ks) VH_CHECK(hipMemsetAsync(Ly.kv.ks, 0, (size_t)m->S * 4, s));
        if (Ly.kv.vs) VH_CHECK(hipMemsetAsync(Ly.kv.vs, 0, (size_t)m->S * 4, s));
    }
    VH_CHECK(hipMemsetAsync(m->state, 0, 3 * sizeof(int), s));   // the epoch (state[3]) runs on
    VH_CHECK(hipStreamSynchronize(s));
    m->pos = 0;
    return VLRF_HIP_OK;
}

int vlrf_hip_model_used(vlrf_hip_model_t m) { return m ? m->pos : -1; }

int vlrf_hip_model_get_config(vlrf_hip_model_t m, vlrf_hip_model_config* out) {
    VH_ARG(m && out, "model_get_config: null argument");
    *out = m->cfg;
    return VLRF_HIP_OK;
}

int vlrf_hip_model_step(vlrf_hip_model_t m, int32_t token, int32_t* next, float* logits) {
    int rc = check_ready(m);
    if (rc) return rc;
    VH_ARG(token >= 0 && token < m->V, "model_step: token %d outside [0,%d)", token, m->V);
    if (m->pos + 1 > m->S) {
        set_error("KVCache::append: exceeds max_seq_len (%d + 1 > %d)", m->pos, m->S);
        return VLRF_HIP_ERR_OVERFLOW;
    }
    hipStream_t s = m->ctx->stream;
    m->pinned[0] = token;
    VH_CHECK(hipMemcpyAsync(m->state, m->pinned, sizeof(int), hipMemcpyHostToDevice, s));
    if ((rc = launch_step(m))) return rc;
    VH_CHECK(hipMemcpyAsync(m->pinned, m->state, sizeof(int), hipMemcpyDeviceToHost, s));
    if (logits) VH_CHECK(hipMemcpyAsync(logits, m->logits, (size_t)m->V * 4, hipMemcpyDeviceToHost, s));
    VH_CHECK(hipStreamSynchronize(s));
    if ((rc = check_waits(m))) return rc;
    m->pos += 1;
    if (next) *next = m->pinned[0];
    return VLRF_HIP_OK;
}

int vlrf_hip_model_prefill(vlrf_hip_model_t m, const int32_t* ids, int n, int32_t* next) {
    int rc = check_ready(m);
    if (rc) return rc;
    VH_ARG(ids != nullptr && n >= 1, "model_prefill: empty prompt");
    for (int i = 0; i < n; ++i)
        VH_ARG(ids[i] >= 0 && ids[i] < m->V, "model_prefill: token %d outside [0,%d)", ids[i], m->V);
    if (m->pos + n > m->S) {
        set_error("KVCache::append: exceeds max_seq_len (%d + %d > %d)", m->pos, n, m->S);
        return VLRF_HIP_ERR_OVERFLOW;
    }
    hipStream_t s = m->ctx->stream;
    VH_CHECK(hipMemcpyAsync(m->prompt, ids, (size_t)n * sizeof(int), hipMemcpyHostToDevice, s));
    VH_CHECK(hipStreamSynchronize(s));
    for (int i = 0; i < n; ++i) {
        VH_CHECK(hipMemcpyAsync(m->state, m->prompt + i, sizeof(int), hipMemcpyDeviceToDevice, s));
        if ((rc = launch_step(m))) return rc;
    }
    VH_CHECK(hipMemcpyAsync(m->pinned, m->state, sizeof(int), hipMemcpyDeviceToHost, s));
    VH_CHECK(hipStreamSynchronize(s));
    if ((rc = check_waits(m))) return rc;
    m->pos += n;
    if (next) *next = m->pinned[0];
    return VLRF_HIP_OK;
}

namespace {

// Grows the batched-prefill buffers to hold T rows (waits for queued work first).
int prefill_reserve(vlrf_hip_model* m, int T) {
    // The GEMMs' K-split partial sums at T rows (every layer has layer 0's shapes).
    size_t need = 0;
    if (!m->layers.empty()) {
        const Layer& L0 = m->layers[0];
        need = std::max({qgemm_part_bytes(L0.wqkv, T, false), qgemm_part_bytes(L0.wo, T, false),
                         qgemm_part_bytes(L0.wg, T, true), qgemm_part_bytes(L0.wd, T, false)});
    }
    if (need > m->pf_part_bytes) {
        VH_CHECK(hipStreamSynchronize(m->ctx->stream));
        if (m->pf_part) (void)hipFree(m->pf_part);
        m->pf_part = nullptr;
        m->pf_part_bytes = 0;
        if (hipMalloc(&m->pf_part, need) != hipSuccess) {
            set_error("prefill: hipMalloc(%zu) failed", need);
            return VLRF_HIP_ERR_NOMEM;
        }
        m->pf_part_bytes = need;
    }
    if (T <= m->pf_cap) return VLRF_HIP_OK;
    VH_CHECK(hipStreamSynchronize(m->ctx->stream));
    for (void** p : {(void**)&m->pf_x, (void**)&m->pf_qkv, (void**)&m->pf_a, (void**)&m->pf_att,
                     (void**)&m->pf_h, (void**)&m->pf_ids}) {
        if (*p) (void)hipFree(*p);
        *p = nullptr;
    }
    m->pf_cap = 0;
    const size_t t = (size_t)T;
    const size_t sizes[6] = {t * m->D * 4, t * (m->D + 2 * m->dkv) * 4, t * m->D * 2, t * m->D * 2,
                             t * m->F * 2, t * 4};
    void** ptrs[6] = {(void**)&m->pf_x, (void**)&m->pf_qkv, (void**)&m->pf_a, (void**)&m->pf_att,
                      (void**)&m->pf_h, (void**)&m->pf_ids};
    for (int i = 0; i < 6; ++i) {
        if (hipMalloc(ptrs[i], sizes[i]) != hipSuccess) {
            set_error("prefill: hipMalloc(%zu) failed", sizes[i]);
            return VLRF_HIP_ERR_NOMEM;
        }
    }
    m->pf_cap = T;
    return VLRF_HIP_OK;
}

// All layers over T embedded rows (device [T][D]) at cache positions m->pos..:
// TransformerBlock::forward_v2 pre-norm order (transformer_block.hpp:141-159)
// with AttentionBlock::forward's T > 1 path (attention.hpp:89-186: RoPE, K/V
// appended to the cache, causal attention).  Layer 0 reads the rows from
// x_in, the residual stream lives in pf_x, and the last layer's down
// projection writes x_out (either may be pf_x; x_out may be x_in), so the
// rows are never copied in or out.
int enqueue_prefill_layers(vlrf_hip_model* m, const float* x_in, float* x_out, int T) {
    hipStream_t s = m->ctx->stream;
    const float eps = m->cfg.norm_eps;
    const float scale = 1.f / std::sqrt((float)m->dh);          // attention.hpp:373-374
    const int ld = m->D + 2 * m->dkv;
    float* x = m->pf_x;
    int rc = VLRF_HIP_OK;
    for (int l = 0; l < m->L && !rc; ++l) {
        Layer& Ly = m->layers[l];
        const float* src = l == 0 ? x_in : x;                    // the stream entering layer l
        float* dst = l == m->L - 1 ? x_out : x;                  // and leaving it
        rc = launch_rows_to_bf16(s, src, Ly.ln1, m->pf_a, T, m->D, eps);
        if (!rc) rc = launch_qgemm(s, Ly.wqkv, m->pf_a, T, nullptr, m->pf_qkv, m->pf_part);
        // k rotated and appended here; q rotated by the attention as it loads it
        if (!rc) rc = launch_prefill_rope_append(s, Ly.kv, m->pf_qkv, ld, T, m->H, m->G, m->dh, m->S, m->pos,
                                                 m->cos_t, m->sin_t);
        if (!rc) rc = launch_attn_prefill(s, m->pf_qkv, ld, Ly.kv, T, m->pos, m->H, m->G, m->dh, m->S, scale,
                                          m->cos_t, m->sin_t, m->pf_att);
        if (!rc) rc = launch_qgemm(s, Ly.wo, m->pf_att, T, src, x, m->pf_part);   // x = src + att . Wo^T
        if (!rc) rc = launch_rows_to_bf16(s, x, Ly.ln2, m->pf_a, T, m->D, eps);
        if (!rc) rc = launch_qgemm_swiglu(s, Ly.wg, Ly.wu, m->pf_a, T, m->pf_h, true, m->pf_part);
        if (!rc) rc = launch_qgemm(s, Ly.wd, m->pf_h, T, x, dst, m->pf_part);   // dst = x + h . Wd^T
    }
    return rc;
}

int check_prefill(vlrf_hip_model* m, int T) {
    int rc = check_ready(m);
    if (rc) return rc;
    VH_ARG(T >= 1, "prefill: no rows");
    VH_ARG(m->cfg.weight_dtype == VLRF_HIP_DT_Q8_0 || m->cfg.weight_dtype == VLRF_HIP_DT_Q4_0,
           "prefill_mfma: needs Q8_0/Q4_0 weights (dtype %d)", m->cfg.weight_dtype);
    VH_ARG(m->D % 64 == 0 && m->F % 64 == 0, "prefill_mfma: d_model %d / d_ff %d not multiples of 64",
           m->D, m->F);
    if (m->pos + T > m->S) {
        set_error("KVCache::append: exceeds max_seq_len (%d + %d > %d)", m->pos, T, m->S);
        return VLRF_HIP_ERR_OVERFLOW;
    }
    return prefill_reserve(m, T);
}

}  // namespace

int vlrf_hip_model_forward_hidden(vlrf_hip_model_t m, const float* x, int T, float* out) {
    int rc = check_prefill(m, T);
    if (rc) return rc;
    VH_ARG(x && out, "forward_hidden: null buffer");
    hipStream_t s = m->ctx->stream;
    if ((rc = enqueue_prefill_layers(m, x, out, T))) return rc;
    m->pos += T;
    m->pinned[0] = 0;
    m->pinned[1] = m->pos;
    m->pinned[2] = 0;
    VH_CHECK(hipMemcpyAsync(m->state, m->pinned, 3 * sizeof(int), hipMemcpyHostToDevice, s));
    VH_CHECK(hipStreamSynchronize(s));
    return VLRF_HIP_OK;
}

int vlrf_hip_model_prefill_mfma(vlrf_hip_model_t m, const int32_t* ids, int n, int32_t* next) {
    int rc = check_prefill(m, n);
    if (rc) return rc;
    VH_ARG(ids != nullptr, "prefill_mfma: null ids");
    for (int i = 0; i < n; ++i)
        VH_ARG(ids[i] >= 0 && ids[i] < m->V, "prefill_mfma: token %d outside [0,%d)", ids[i], m->V);
    hipStream_t s = m->ctx->stream;
    VH_CHECK(hipMemcpyAsync(m->pf_ids, ids, (size_t)n * sizeof(int), hipMemcpyHostToDevice, s));
    if ((rc = launch_embed_rows(s, m->embed, m->pf_ids, m->pf_x, n, m->D))) return rc;   // ops.hpp:615-626
    if ((rc = enqueue_prefill_layers(m, m->pf_x, m->pf_x, n))) return rc;
    // transformer.hpp:399-414: final norm and LM head on the last row, greedy argmax.
    if ((rc = launch_qlinear(s, m->lm_head, m->pf_x + (size_t)(n - 1) * m->D, m->logits, 1, m->ln_final,
                             m->cfg.norm_eps, nullptr)))
        return rc;
    if ((rc = launch_argmax_step(s, m->logits, m->V, m->state, m->gen_ids, m->S))) return rc;
    VH_CHECK(hipMemcpyAsync(m->pinned, m->state, sizeof(int), hipMemcpyDeviceToHost, s));
    VH_CHECK(hipStreamSynchronize(s));
    if (next) *next = m->pinned[0];
    m->pos += n;
    m->pinned[1] = m->pos;
    m->pinned[2] = 0;
    VH_CHECK(hipMemcpyAsync(m->state + 1, m->pinned + 1, 2 * sizeof(int), hipMemcpyHostToDevice, s));
    VH_CHECK(hipStreamSynchronize(s));
    return VLRF_HIP_OK;
}

int vlrf_hip_model_kv_read(vlrf_hip_model_t m, int layer, int row0, int n, int8_t* k_q, int8_t* v_q,
                           float* k_s, float* v_s) {
    VH_ARG(m != nullptr, "model_kv_read: null handle");
    VH_ARG(layer >= 0 && layer < m->L, "model_kv_read: layer %d out of range", layer);
    VH_ARG(row0 >= 0 && n >= 0 && row0 + n <= m->S, "model_kv_read: rows out of range");
    VH_CHECK(hipSetDevice(m->ctx->device));
    return kv_rows_to_host(m->ctx->stream, m->layers[layer].kv, m->G, m->dh, m->S, row0, n, k_q, v_q, k_s, v_s);
}

int vlrf_hip_model_generate_async(vlrf_hip_model_t m, int32_t first, int n_steps) {
    int rc = check_ready(m);
    if (rc) return rc;
    VH_ARG(first >= 0 && first < m->V, "model_generate: token %d outside [0,%d)", first, m->V);
    VH_ARG(n_steps >= 1, "model_generate: n_steps %d < 1", n_steps);
    if (m->pos + n_steps > m->S) {
        set_error("KVCache::append: exceeds max_seq_len (%d + %d > %d)", m->pos, n_steps, m->S);
        return VLRF_HIP_ERR_OVERFLOW;
    }
    hipStream_t s = m->ctx->stream;
    VH_CHECK(hipStreamSynchronize(s));   // the pinned staging word is free again
    m->pinned[0] = first;
    m->pinned[1] = m->pos;
    m->pinned[2] = 0;
    VH_CHECK(hipMemcpyAsync(m->state, m->pinned, 3 * sizeof(int), hipMemcpyHostToDevice, s));
    int i = 0;
    if (m->exec_n)   // the steps need no host input: whole runs of kGraphSteps
        for (; i + kGraphSteps <= n_steps; i += kGraphSteps) VH_CHECK(hipGraphLaunch(m->exec_n, s));
    for (; i < n_steps; ++i)
        if ((rc = launch_step(m))) return rc;
    m->pos += n_steps;
    return VLRF_HIP_OK;
}

int vlrf_hip_model_read_generated(vlrf_hip_model_t m, int32_t* out_ids, int n) {
    VH_ARG(m && out_ids && n >= 0 && n <= m->S, "read_generated: bad arguments");
    VH_CHECK(hipSetDevice(m->ctx->device));
    hipStream_t s = m->ctx->stream;
    VH_CHECK(hipMemcpyAsync(out_ids, m->gen_ids, (size_t)n * sizeof(int), hipMemcpyDeviceToHost, s));
    VH_CHECK(hipStreamSynchronize(s));
    return check_waits(m);
}

int vlrf_hip_model_time_launches(vlrf_hip_model_t m, int32_t first, int n_steps, double us[VLRF_HIP_LK_KINDS],
                                 int calls[VLRF_HIP_LK_KINDS]) {
    int rc = check_ready(m);
    if (rc) return rc;
    VH_ARG(us && calls, "time_launches: null output");
    VH_ARG(first >= 0 && first < m->V, "time_launches: token %d outside [0,%d)", first, m->V);
    VH_ARG(n_steps >= 1 && n_steps <= 256, "time_launches: n_steps %d outside [1,256]", n_steps);
    if (m->pos + n_steps > m->S) {
        set_error("KVCache::append: exceeds max_seq_len (%d + %d > %d)", m->pos, n_steps, m->S);
        return VLRF_HIP_ERR_OVERFLOW;
    }
    for (int k = 0; k < VLRF_HIP_LK_KINDS; ++k) {
        us[k] = 0.0;
        calls[k] = 0;
    }
    hipStream_t s = m->ctx->stream;
    // At most 6 launches per layer plus 3 per step (stand-alone attention with
    // its combine, the embedding, the LM head and the argmax).
    const int cap = n_steps * (6 * m->L + 3);
    std::vector<hipEvent_t> ev(2 * (size_t)cap, nullptr);
    std::vector<int> kind(cap, 0);
    LaunchTimer t;
    t.start = ev.data();
    t.stop = ev.data() + cap;
    t.kind = kind.data();
    t.cap = cap;
    auto destroy = [&]() {
        for (hipEvent_t e : ev)
            if (e) (void)hipEventDestroy(e);
    };
    for (auto& e : ev)
        if (hipEventCreate(&e) != hipSuccess) {
            destroy();
            set_error("time_launches: hipEventCreate failed");
            return VLRF_HIP_ERR_RUNTIME;
        }
    if (hipStreamSynchronize(s) != hipSuccess) {
        destroy();
        set_error("time_launches: stream synchronisation failed");
        return VLRF_HIP_ERR_RUNTIME;
    }
    m->pinned[0] = first;
    m->pinned[1] = m->pos;
    m->pinned[2] = 0;
    if (hipMemcpyAsync(m->state, m->pinned, 3 * sizeof(int), hipMemcpyHostToDevice, s) != hipSuccess) {
        destroy();
        set_error("time_launches: state upload failed");
        return VLRF_HIP_ERR_RUNTIME;
    }
    launch_timer() = &t;
    for (int i = 0; i < n_steps && !rc; ++i) rc = enqueue_step(m, s);
    launch_timer() = nullptr;
    if (!rc) m->pos += n_steps;
    if (!rc && hipStreamSynchronize(s) != hipSuccess) {
        set_error("time_launches: the timed steps failed");
        rc = VLRF_HIP_ERR_RUNTIME;
    }
    for (int j = 0; j < t.n && !rc; ++j) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, t.start[j], t.stop[j]) != hipSuccess) {
            set_error("time_launches: no timing for launch %d", j);
            rc = VLRF_HIP_ERR_RUNTIME;
            break;
        }
        us[t.kind[j]] += ms * 1e3;
        calls[t.kind[j]] += 1;
    }
    destroy();
    if (rc) return rc;
    return check_waits(m);
}

int vlrf_hip_model_generate(vlrf_hip_model_t m, int32_t first, int n_steps, int32_t* out_ids) {
    int rc = vlrf_hip_model_generate_async(m, first, n_steps);
    if (rc) return rc;
    return vlrf_hip_model_read_generated(m, out_ids, n_steps);
}

int vlrf_hip_model_step_bytes(vlrf_hip_model_t m, int ctx_len, double out[3]) {
    VH_ARG(m && out && ctx_len >= 1, "step_bytes: bad arguments");
    double w = 0.0;
    for (auto& Ly : m->layers)
        for (const DevWeight* dw : {&Ly.wqkv, &Ly.wo, &Ly.wg, &Ly.wu, &Ly.wd})
            w += (double)weight_device_bytes(dw->dtype, dw->N, dw->K);
    w += (double)weight_device_bytes(m->lm_head.dtype, m->V, m->D);
    // K and V elements of the context (plus one f32 scale per row for Q8_0), per layer.
    const bool q8 = m->cfg.kv_dtype == VLRF_HIP_KV_Q8_0;
    const double kv = (double)m->L * (2.0 * ctx_len * m->dkv * kv_elem_bytes(m->cfg.kv_dtype) +
                                      (q8 ? 2.0 * ctx_len * 4.0 : 0.0));
    // Norm weights (2 per layer + final) and the embedding row.
    const double other = (2.0 * m->L + 1.0) * m->D * 4.0 + m->D * 4.0;
    out[0] = w;
    out[1] = kv;
    out[2] = other;
    return VLRF_HIP_OK;
}

}  // extern "C"
