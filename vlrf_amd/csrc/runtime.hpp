// runtime.hpp - the context object behind vlrf_hip_ctx_t.
#pragma once

#include "internal.hpp"

#include <vector>

struct vlrf_hip_ctx {
    int device = 0;
    int num_cus = 0;
    char name[256] = {0};
    hipStream_t stream = nullptr;   // default priority, non-blocking
    hipEvent_t ev0 = nullptr, ev1 = nullptr;

    struct RopeTab {
        int max_seq = 0, d_head = 0;
        float theta = 0.f;
        float* cos_t = nullptr;
        float* sin_t = nullptr;
    };
    std::vector<RopeTab> ropes;      // RoPE tables per (max_seq, d_head, theta)
    void* scratch_buf = nullptr;     // split-K partials of the standalone ops
    size_t scratch_bytes = 0;
    float* noalloc_scratch = nullptr;   // this device's fixed array for vlrf_hip_attn_decode_noalloc
    int* small_tile_ctr = nullptr;      // small-M linear: row-tile counters (zero between calls)

    // Device cos/sin tables built on the host as RopeCache::init does.
    int rope_tables(int max_seq, int d_head, float theta, const float** c, const float** s);
    // Grows the shared scratch buffer (waits for queued work before regrowing).
    int scratch(size_t bytes, float** out);
    ~vlrf_hip_ctx();
};

namespace vlrf_hip {
using Ctx = ::vlrf_hip_ctx;
}
