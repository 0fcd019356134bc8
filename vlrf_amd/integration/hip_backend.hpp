// hip_backend.hpp - IBackend implementation for the VLRF engine, over the C ABI
// of libvlrf_hip.so (include/vlrf_hip.h).
//
// Drop-in location in the engine tree: include/backend/hip_backend.hpp,
// included by backend.hpp after ibackend.hpp and registered through
// BackendRegistry::try_hip() (reference include/backend/backend.hpp:544-578).
// It mirrors OpenCLBackend's contract (backend.hpp:191-492): host Tensors in,
// host Tensors out, and any unsupported shape or device failure runs the CPU
// op instead.  Unlike the reference's default sdp_attention
// (ibackend.hpp:79-82 -> ops::sdp_attention, which slices K/V with T instead
// of ctx_len when T != ctx_len), the CPU fallback here is a correct per-head
// softmax attention.
//
// The decode hot path does not go through this per-op interface: it uses
// HipDecoder (hip_decoder.hpp), which keeps weights, KV cache and activations
// resident on the device.  This class serves the generic IBackend callers:
// compute::gemm / compute::linear (compute.hpp:37-101) and
// AttentionBlock::sdp_heads (attention.hpp:376-392).
#pragma once

#include "ibackend.hpp"
#include "vlrf_hip.h"

#include <cmath>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#ifndef VLRF_HIP_BACKEND_TYPE
#define VLRF_HIP_BACKEND_TYPE BackendType::HIP   // enum value added by the integration patch
#endif

namespace vlrf {
namespace backend {

class HipBackend : public IBackend {
public:
    HipBackend() = default;
    HipBackend(const HipBackend&) = delete;
    HipBackend& operator=(const HipBackend&) = delete;
    ~HipBackend() override { release(); }

    // BackendRegistry::try_hip(): true when a gfx950 device is usable.
    bool try_init(int device = 0) {
        release();
        if (vlrf_hip_init(device, &ctx_) != VLRF_HIP_OK) {
            info_ = std::string("HIP: unavailable (") + vlrf_hip_last_error() + ")";
            ctx_ = nullptr;
            return false;
        }
        char buf[256];
        vlrf_hip_device_info(ctx_, buf, sizeof(buf));
        info_ = buf;
        return true;
    }

    vlrf_hip_ctx_t context() const { return ctx_; }

    BackendType type() const override { return VLRF_HIP_BACKEND_TYPE; }
    std::string device_info() const override { return info_; }
    bool is_available() const override { return ctx_ != nullptr; }
    std::string capabilities() const override {
        return "HIP backend (gfx950)\n"
               "  gemm: linear x.W^T, 1<=M<=16, K%32==0 on device (weights cached); other shapes\n"
               "        with >= 2^22 multiply-adds on device (f32), smaller ones CPU\n"
               "  sdp_attention: fused flash attention on device (d_h<=128)\n"
               "  layer_norm/softmax/gelu/add: device for >= 65536 elements, CPU below\n"
               "  decode step: HipDecoder (device-resident Q8_0/Q4_0 weights, F32/F16/Q8_0 KV cache)";
    }
    void synchronize() const override {
        if (ctx_) vlrf_hip_sync(ctx_);
    }

    // Tensors stay host-side at this interface (as OpenCLBackend).
    Tensor to_device(Tensor const& t) const override { return t; }
    Tensor to_host(Tensor const& t) const override { return t; }

    void gemm(Tensor const& A, Tensor const& B, Tensor& C, float alpha, float beta, bool tA,
              bool tB) const override {
        if (ctx_ && !tA && tB && alpha == 1.f && beta == 0.f && linear_on_device(A, B, C)) return;
        if (ctx_ && gemm_on_device(A, B, C, alpha, beta, tA, tB)) return;
        fallback_.gemm(A, B, C, alpha, beta, tA, tB);
    }
    void layer_norm(Tensor const& x, Tensor const& w, Tensor const& b, Tensor& out,
                    float eps) const override {
        if (ctx_ && layer_norm_on_device(x, w, b, out, eps)) return;
        fallback_.layer_norm(x, w, b, out, eps);
    }
    void softmax_inplace(Tensor& t) const override {
        if (ctx_ && t.ndim() >= 1 && t.numel() >= kDeviceMin &&
            inplace_on_device(t, nullptr, [&](float* p) {
                return vlrf_hip_softmax(ctx_, p, (int)(t.numel() / t.dim(t.ndim() - 1)), t.dim(t.ndim() - 1));
            }))
            return;
        fallback_.softmax_inplace(t);
    }
    void gelu_inplace(Tensor& t) const override {
        if (ctx_ && t.numel() >= kDeviceMin &&
            inplace_on_device(t, nullptr, [&](float* p) { return vlrf_hip_gelu(ctx_, p, t.numel()); }))
            return;
        fallback_.gelu_inplace(t);
    }
    void add_inplace(Tensor& dst, Tensor const& src) const override {
        if (ctx_ && dst.numel() >= kDeviceMin && src.numel() == dst.numel() &&
            inplace_on_device(dst, &src, [&](float* p) {
                return vlrf_hip_add(ctx_, p, static_cast<const float*>(bq_.p), dst.numel());
            }))
            return;
        fallback_.add_inplace(dst, src);
    }

    // Q [n_h,T,d_h], K/V [n_h,ctx,d_h] -> [n_h,T,d_h]; scale 1/sqrt(d_h) as the
    // fused-kernel contract of the reference (attention.hpp:376-392).
    Tensor sdp_attention(Tensor const& Q, Tensor const& K, Tensor const& V,
                         bool causal) const override {
        Tensor out;
        if (ctx_ && attention_on_device(Q, K, V, causal, out)) return out;
        return attention_cpu(Q, K, V, causal);
    }

private:
    // Elementwise and row ops go to the device from this many elements on:
    // below it the host round trip costs more than the CPU op.
    static constexpr int64_t kDeviceMin = 1 << 16;
    static constexpr double kGemmDeviceMin = 4194304.0;   // multiply-adds

    struct Buf {
        void* p = nullptr;
        size_t n = 0;
    };

    bool grow(Buf& b, size_t bytes) const {
        if (b.n >= bytes) return true;
        if (b.p) vlrf_hip_free(ctx_, b.p);
        b.p = nullptr;
        b.n = 0;
        if (vlrf_hip_malloc(ctx_, bytes, &b.p) != VLRF_HIP_OK) return false;
        b.n = bytes;
        return true;
    }

    // compute::linear: C[M,N] = A[M,K] . B[N,K]^T.  B is usually a weight of
    // the WeightMap, uploaded once and reused; the cache is keyed by B's
    // storage and offset, holds a weak reference to the storage (a freed
    // tensor's address can be reused by a new one) and the shape, as the SYCL
    // backend's device cache does (sycl_backend.hpp:715-749).  Contents are
    // taken as immutable while the storage lives, as for every engine weight.
    bool linear_on_device(Tensor const& A, Tensor const& B, Tensor& C) const {
        if (A.ndim() != 2 || B.ndim() != 2 || C.ndim() != 2 || !B.storage) return false;
        const int M = A.dim(0), K = A.dim(1), N = B.dim(0);
        if (B.dim(1) != K || C.dim(0) != M || C.dim(1) != N) return false;
        if (M < 1 || M > 16 || K % 32 != 0) return false;
        const auto key = std::make_pair(static_cast<const void*>(B.storage.get()), B.offset);
        auto it = wcache_.find(key);
        if (it != wcache_.end() &&
            (it->second.owner.expired() || it->second.N != N || it->second.K != K)) {
            vlrf_hip_weight_free(it->second.w);
            wcache_.erase(it);
            it = wcache_.end();
        }
        vlrf_hip_weight_t w = nullptr;
        if (it != wcache_.end()) {
            w = it->second.w;
        } else {
            if (vlrf_hip_weight_upload(ctx_, B.data_ptr(), VLRF_HIP_DT_F32, N, K, &w) != VLRF_HIP_OK)
                return false;
            wcache_.emplace(key, Cached{w, B.storage, N, K});
        }
        const size_t xb = sizeof(float) * (size_t)M * K, yb = sizeof(float) * (size_t)M * N;
        if (!grow(bx_, xb) || !grow(by_, yb)) return false;
        if (vlrf_hip_h2d(ctx_, bx_.p, A.data_ptr(), xb) != VLRF_HIP_OK) return false;
        if (vlrf_hip_qlinear(ctx_, w, static_cast<const float*>(bx_.p), static_cast<float*>(by_.p), M,
                             nullptr, 0.f, nullptr) != VLRF_HIP_OK)
            return false;
        return vlrf_hip_d2h(ctx_, C.data_ptr(), by_.p, yb) == VLRF_HIP_OK;
    }

    // ops::gemm (ops.hpp:170-310) on the device: A, B and C (when beta != 0)
    // uploaded, C downloaded.
    bool gemm_on_device(Tensor const& A, Tensor const& B, Tensor& C, float alpha, float beta, bool tA,
                        bool tB) const {
        if (A.ndim() != 2 || B.ndim() != 2 || C.ndim() != 2) return false;
        const int M = tA ? A.dim(1) : A.dim(0), K = tA ? A.dim(0) : A.dim(1);
        const int N = tB ? B.dim(0) : B.dim(1), KB = tB ? B.dim(1) : B.dim(0);
        if (KB != K || C.dim(0) != M || C.dim(1) != N || (double)M * N * K < kGemmDeviceMin) return false;
        const size_t ab = sizeof(float) * A.numel(), bb = sizeof(float) * B.numel(), cb = sizeof(float) * C.numel();
        if (!grow(bq_, ab) || !grow(bk_, bb) || !grow(bo_, cb)) return false;
        if (vlrf_hip_h2d(ctx_, bq_.p, A.data_ptr(), ab) || vlrf_hip_h2d(ctx_, bk_.p, B.data_ptr(), bb) ||
            (beta != 0.f && vlrf_hip_h2d(ctx_, bo_.p, C.data_ptr(), cb)))
            return false;
        if (vlrf_hip_gemm_f32(ctx_, static_cast<const float*>(bq_.p), static_cast<const float*>(bk_.p),
                              static_cast<float*>(bo_.p), M, N, K, A.dim(1), B.dim(1), N, alpha, beta, tA, tB))
            return false;
        return vlrf_hip_d2h(ctx_, C.data_ptr(), bo_.p, cb) == VLRF_HIP_OK;
    }

    bool layer_norm_on_device(Tensor const& x, Tensor const& w, Tensor const& b, Tensor& out, float eps) const {
        if (x.ndim() < 1 || x.numel() < kDeviceMin) return false;
        const int D = x.dim(x.ndim() - 1);
        if (w.numel() != D || b.numel() != D) return false;
        const size_t xb = sizeof(float) * x.numel(), wb = sizeof(float) * D;
        if (!grow(bq_, xb) || !grow(bk_, wb) || !grow(bv_, wb) || !grow(bo_, xb)) return false;
        if (vlrf_hip_h2d(ctx_, bq_.p, x.data_ptr(), xb) || vlrf_hip_h2d(ctx_, bk_.p, w.data_ptr(), wb) ||
            vlrf_hip_h2d(ctx_, bv_.p, b.data_ptr(), wb))
            return false;
        if (vlrf_hip_layer_norm(ctx_, static_cast<const float*>(bq_.p), static_cast<const float*>(bk_.p),
                                static_cast<const float*>(bv_.p), static_cast<float*>(bo_.p),
                                (int)(x.numel() / D), D, eps))
            return false;
        if (out.numel() != x.numel()) out = Tensor(x.shape);   // ops::layer_norm's like(x)
        return vlrf_hip_d2h(ctx_, out.data_ptr(), bo_.p, xb) == VLRF_HIP_OK;
    }

    // t uploaded to bo_ (and src, when given, to bq_), op(bo_) run, t downloaded.
    template <class Op>
    bool inplace_on_device(Tensor& t, Tensor const* src, Op op) const {
        const size_t tb = sizeof(float) * t.numel();
        if (!grow(bo_, tb) || (src && !grow(bq_, tb))) return false;
        if (vlrf_hip_h2d(ctx_, bo_.p, t.data_ptr(), tb) || (src && vlrf_hip_h2d(ctx_, bq_.p, src->data_ptr(), tb)))
            return false;
        if (op(static_cast<float*>(bo_.p)) != VLRF_HIP_OK) return false;
        return vlrf_hip_d2h(ctx_, t.data_ptr(), bo_.p, tb) == VLRF_HIP_OK;
    }

    bool attention_on_device(Tensor const& Q, Tensor const& K, Tensor const& V, bool causal,
                             Tensor& out) const {
        if (Q.ndim() != 3 || K.ndim() != 3 || V.ndim() != 3) return false;
        const int n_h = Q.dim(0), T = Q.dim(1), d = Q.dim(2), ctx = K.dim(1);
        if (K.dim(0) != n_h || V.dim(0) != n_h || K.dim(2) != d || V.dim(2) != d || V.dim(1) != ctx)
            return false;
        if (d < 1 || d > 128 || (causal && T > ctx)) return false;
        const size_t qb = sizeof(float) * Q.numel(), kb = sizeof(float) * K.numel();
        if (!grow(bq_, qb) || !grow(bk_, kb) || !grow(bv_, kb) || !grow(bo_, qb)) return false;
        if (vlrf_hip_h2d(ctx_, bq_.p, Q.data_ptr(), qb) || vlrf_hip_h2d(ctx_, bk_.p, K.data_ptr(), kb) ||
            vlrf_hip_h2d(ctx_, bv_.p, V.data_ptr(), kb))
            return false;
        const float scale = 1.f / std::sqrt((float)d);
        if (vlrf_hip_attn_f32(ctx_, static_cast<const float*>(bq_.p), static_cast<const float*>(bk_.p),
                              static_cast<const float*>(bv_.p), static_cast<float*>(bo_.p), n_h, T, ctx,
                              d, scale, causal ? 1 : 0) != VLRF_HIP_OK)
            return false;
        out = Tensor({n_h, T, d});
        return vlrf_hip_d2h(ctx_, out.data_ptr(), bo_.p, qb) == VLRF_HIP_OK;
    }

    // Correct CPU fallback: per head, softmax(Q K^T * scale + causal mask) V
    // with the causal rule key > query + (ctx - T) (attention.hpp:232,253-261).
    static Tensor attention_cpu(Tensor const& Q, Tensor const& K, Tensor const& V, bool causal) {
        const int n_h = Q.dim(0), T = Q.dim(1), d = Q.dim(2), ctx = K.dim(1);
        Tensor out({n_h, T, d});
        const float scale = 1.f / std::sqrt((float)d);
        std::vector<float> s(ctx);
        for (int h = 0; h < n_h; ++h) {
            const float* q = Q.data_ptr() + (size_t)h * T * d;
            const float* k = K.data_ptr() + (size_t)h * ctx * d;
            const float* v = V.data_ptr() + (size_t)h * ctx * d;
            float* o = out.data_ptr() + (size_t)h * T * d;
            for (int i = 0; i < T; ++i) {
                const int last = causal ? i + (ctx - T) : ctx - 1;
                float mx = -std::numeric_limits<float>::infinity();
                for (int j = 0; j <= last && j < ctx; ++j) {
                    float dot = 0.f;
                    for (int c = 0; c < d; ++c) dot += q[(size_t)i * d + c] * k[(size_t)j * d + c];
                    s[j] = dot * scale;
                    if (s[j] > mx) mx = s[j];
                }
                float l = 0.f;
                for (int c = 0; c < d; ++c) o[(size_t)i * d + c] = 0.f;
                for (int j = 0; j <= last && j < ctx; ++j) {
                    const float p = std::exp(s[j] - mx);
                    l += p;
                    for (int c = 0; c < d; ++c) o[(size_t)i * d + c] += p * v[(size_t)j * d + c];
                }
                const float inv = l > 0.f ? 1.f / l : 0.f;
                for (int c = 0; c < d; ++c) o[(size_t)i * d + c] *= inv;
            }
        }
        return out;
    }

    void release() {
        if (!ctx_) return;
        for (auto& kv : wcache_) vlrf_hip_weight_free(kv.second.w);
        wcache_.clear();
        for (Buf* b : {&bx_, &by_, &bq_, &bk_, &bv_, &bo_}) {
            if (b->p) vlrf_hip_free(ctx_, b->p);
            b->p = nullptr;
            b->n = 0;
        }
        vlrf_hip_shutdown(ctx_);
        ctx_ = nullptr;
    }

    vlrf_hip_ctx_t ctx_ = nullptr;
    std::string info_{"HIP: not initialised"};
    CpuBackend fallback_;
    struct Cached {
        vlrf_hip_weight_t w;
        std::weak_ptr<TensorStorage> owner;
        int N, K;
    };
    mutable std::map<std::pair<const void*, int64_t>, Cached> wcache_;
    mutable Buf bx_, by_, bq_, bk_, bv_, bo_;
};

}  // namespace backend
}  // namespace vlrf
