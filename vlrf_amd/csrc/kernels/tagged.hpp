// tagged.hpp - exchange of values between the workgroups of one launch as
// tagged 64-bit words (the fused QKV + attention launch, qkv_attn.hip).
//
// A word holds the value's bits in its low half and the producer's epoch in
// its high half, written with one device-scope store; it is valid when its tag
// is the reader's epoch, so a reader needs no fence, flag or counter (the word
// is its own flag) and the buffers never need clearing.  Readers poll with
// cache-bypassing (sc1) loads: the L2 of another XCD would otherwise keep
// serving the stale line.  A failed poll waits on one "gate" word, written by
// a producer that finishes late, before polling everything again, which keeps
// waiting workgroups from flooding the fabric.  Every wait is bounded on the
// wall clock: one that runs out records (block, phase, layer) in `status` and
// every other wait sees the flag and gives up, so a launch always drains.
#pragma once

#include "../internal.hpp"
#include "gemv_core.hpp"

namespace vlrf_hip {
namespace tagged {

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kSc1 = 16;   // buffer cache policy: device-coherent (sc1)

__device__ __forceinline__ void put_word(uint64_t* p, uint32_t bits, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct Ctl {
    __amdgpu_buffer_rsrc_t rs;   // the tagged arena
    uint32_t tag;
    int* status;
    long long t0, limit;
    int phase, layer;
};

// Records the first failing wait (block, phase, layer) and raises the flag.
__device__ inline void fail(const Ctl& c) {
    int expected = 0;
    if (__hip_atomic_compare_exchange_strong(&c.status[0], &expected, 1, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT)) {
        __hip_atomic_store(&c.status[1], (int)blockIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&c.status[2], c.phase, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&c.status[3], c.layer, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Keeps the loads above it (weights, cache rows) above the wait that follows:
// their results are used only after the wait, on the path where it succeeds,
// and the compiler otherwise sinks them there, so the weight stream would
// start only once the inputs are in.  A compiler-only fence: it emits nothing
// and, unlike an asm memory clobber, makes the compiler wait for nothing.
__device__ __forceinline__ void issue_before_wait() { __atomic_signal_fence(__ATOMIC_SEQ_CST); }

// One pass over the wave's N pieces (VT = u32x2: one tagged word at each byte
// offset; u32x4: two words); true when every used piece carries the tag.
template <int N, class VT>
__device__ __forceinline__ bool poll_pass(const Ctl& c, const int (&off)[N], const bool (&use)[N], VT (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if constexpr (sizeof(VT) == 16) v[i] = __builtin_amdgcn_raw_buffer_load_b128(c.rs, off[i], 0, kSc1);
        else v[i] = __builtin_amdgcn_raw_buffer_load_b64(c.rs, off[i], 0, kSc1);
    }
    bool ok = true;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        bool good = v[i].y == c.tag;
        if constexpr (sizeof(VT) == 16) good = good && v[i].w == c.tag;
        if (use[i] && !good) ok = false;
    }
    return __all(ok);
}

// Polls until every used piece of the wave is valid; after a failed pass it
// waits for the gate word (byte offset `gate`) before the next full pass.
// False when the wait ran out (recorded) or another workgroup failed.
template <int N, class VT>
__device__ inline bool poll(const Ctl& c, const int (&off)[N], const bool (&use)[N], VT (&v)[N], int gate) {
    if (poll_pass<N, VT>(c, off, use, v)) return true;
    for (;;) {
        const u32x2 g = __builtin_amdgcn_raw_buffer_load_b64(c.rs, gate, 0, kSc1);
        if (__hip_atomic_load(c.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
        if (wall_clock64() - c.t0 > c.limit) {
            fail(c);
            return false;
        }
        if (g.y == c.tag) {
            if (poll_pass<N, VT>(c, off, use, v)) return true;
            __builtin_amdgcn_s_sleep(1);
        } else {
            __builtin_amdgcn_s_sleep(2);
        }
    }
}

// Polls until every used piece of the wave is valid, re-reading all of them
// (for waves that read few words: no gate).  The clock is read after every
// failed pass, the failure flag (a memory round trip of its own) after every
// 8th, so a pass costs one round trip.  False when the wait ran out
// (recorded) or another workgroup failed.
template <int N, class VT>
__device__ inline bool poll_direct(const Ctl& c, const int (&off)[N], const bool (&use)[N], VT (&v)[N]) {
    for (int it = 1;; ++it) {
        if (poll_pass<N, VT>(c, off, use, v)) return true;
        if (wall_clock64() - c.t0 > c.limit) {
            fail(c);
            return false;
        }
        if ((it & 7) == 0 && __hip_atomic_load(c.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
    }
}

// One tagged word (byte offset off, read by the lanes with use set).
__device__ __forceinline__ bool poll_word(const Ctl& c, int off, bool use, float* out) {
    int o[1] = {off};
    bool u[1] = {use};
    u32x2 r[1];
    const bool ok = poll<1, u32x2>(c, o, u, r, off);
    *out = __uint_as_float(r[0].x);
    return ok;
}

// Every wave has polled (ok: its own result); true when the whole workgroup
// may go on.  slots: one LDS int per wave, written before the barrier and read
// after it (a caller that polls again must pass another barrier first).
__device__ __forceinline__ bool block_ok(bool ok, int* slots) {
    if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = ok;
    __syncthreads();
    bool all = true;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) all = all && slots[w] != 0;
    return all;
}

// The thread's x slots (float4 f = tid + p*threads, elements 4f..4f+3) of a
// tagged K-vector at word offset w0, polled; gate: its last word.
template <int WT, int NC>
__device__ __forceinline__ bool poll_x(const Ctl& c, long long w0, int K, float4 (&v)[gemv::Shape<WT, NC>::PER]) {
    constexpr int PER = gemv::Shape<WT, NC>::PER, XF4 = gemv::Shape<WT, NC>::XF4;
    int off[2 * PER];
    bool use[2 * PER];
    u32x4 r[2 * PER];
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int f = threadIdx.x + p * gemv::kGemvThreads;
        const bool in = f < XF4 && 4 * f < K;
        off[2 * p] = (int)((w0 + (in ? 4 * f : 0)) * 8);
        off[2 * p + 1] = off[2 * p] + 16;
        use[2 * p] = use[2 * p + 1] = in;
    }
    const bool ok = poll<2 * PER, u32x4>(c, off, use, r, (int)((w0 + K - 1) * 8));
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const bool in = use[2 * p];
        v[p] = in ? make_float4(__uint_as_float(r[2 * p].x), __uint_as_float(r[2 * p].z),
                                __uint_as_float(r[2 * p + 1].x), __uint_as_float(r[2 * p + 1].z))
                  : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    return ok;
}

template <int WT, int NC>
__device__ __forceinline__ void load_norm(const float* w, int K, float4 (&gw)[gemv::Shape<WT, NC>::PER]) {
    constexpr int PER = gemv::Shape<WT, NC>::PER, XF4 = gemv::Shape<WT, NC>::XF4;
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int f = threadIdx.x + p * gemv::kGemvThreads;
        gw[p] = reinterpret_cast<const float4*>(w)[(f < XF4 && 4 * f < K) ? f : 0];
    }
}

}  // namespace tagged
}  // namespace vlrf_hip
