// format.cpp - host-side block formats and synthetic seeded data.
//
// Block layouts are the GGUF ones the reference's converter decodes
// (tools/converter/convert_gguf.py:233-263): Q8_0 = [f16 d][32 x int8] (34 B),
// Q4_0 = [f16 d][16 B], byte j = element 2j (low nibble) | element 2j+1 (high
// nibble), value (nibble - 8) * d.  The reference has no encoder; the ones
// below are this backend's own (closed form, documented in vlrf_hip.h).
#include <cmath>
#include <cstdint>
#include <cstring>
#include <algorithm>
#include <thread>
#include <vector>

#include "../../../include/vlrf_hip.h"

namespace {

uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint16_t)(sign | (a > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);   // >= 65520 rounds to inf
    if (a < 0x38800000u) {                                       // below 2^-14: subnormal
        float v;
        std::memcpy(&v, &a, 4);
        return (uint16_t)(sign | (uint32_t)std::lrintf(v * 16777216.0f));  // exact scaling, RNE
    }
    uint32_t h = ((a >> 23) - 112u) << 10 | ((a & 0x7FFFFFu) >> 13);
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int ee = 1;
            while (!(m & 0x400u)) { m <<= 1; --ee; }
            m &= 0x3FFu;
            bits = sign | ((uint32_t)(ee + 112) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

template <class F>
void parallel_blocks(int64_t nblocks, F&& fn) {
    unsigned hw = std::thread::hardware_concurrency();
    int nt = (int)std::min<int64_t>(std::max(1u, std::min(hw, 16u)), std::max<int64_t>(1, nblocks / 4096));
    if (nt <= 1) { fn(0, nblocks); return; }
    std::vector<std::thread> ts;
    int64_t chunk = (nblocks + nt - 1) / nt;
    for (int t = 0; t < nt; ++t) {
        int64_t lo = t * chunk, hi = std::min(nblocks, lo + chunk);
        if (lo < hi) ts.emplace_back([&fn, lo, hi] { fn(lo, hi); });
    }
    for (auto& t : ts) t.join();
}

inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return splitmix64(seed ^ splitmix64(stream * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull));
}

}  // namespace

extern "C" {

int vlrf_quantize_q8_0(const float* src, void* dst, int64_t n) {
    if (!src || !dst || n < 0 || n % 32) return VLRF_HIP_ERR_ARG;
    uint8_t* out = static_cast<uint8_t*>(dst);
    parallel_blocks(n / 32, [&](int64_t b0, int64_t b1) {
        for (int64_t b = b0; b < b1; ++b) {
            const float* x = src + b * 32;
            uint8_t* blk = out + b * 34;
            float amax = 0.f;
            for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[i]));
            const uint16_t d16 = f32_to_f16_rne(amax / 127.f);
            const float d = f16_to_f32(d16);
            const float id = d != 0.f ? 1.f / d : 0.f;
            std::memcpy(blk, &d16, 2);
            for (int i = 0; i < 32; ++i) {
                long q = std::lroundf(x[i] * id);
                q = std::min(127L, std::max(-127L, q));
                blk[2 + i] = (uint8_t)(int8_t)q;
            }
        }
    });
    return VLRF_HIP_OK;
}

int vlrf_quantize_q4_0(const float* src, void* dst, int64_t n) {
    if (!src || !dst || n < 0 || n % 32) return VLRF_HIP_ERR_ARG;
    uint8_t* out = static_cast<uint8_t*>(dst);
    parallel_blocks(n / 32, [&](int64_t b0, int64_t b1) {
        for (int64_t b = b0; b < b1; ++b) {
            const float* x = src + b * 32;
            uint8_t* blk = out + b * 18;
            float amax = 0.f, mx = 0.f;
            for (int i = 0; i < 32; ++i)
                if (std::fabs(x[i]) > amax) { amax = std::fabs(x[i]); mx = x[i]; }
            const uint16_t d16 = f32_to_f16_rne(mx / -8.f);
            const float d = f16_to_f32(d16);
            const float id = d != 0.f ? 1.f / d : 0.f;
            std::memcpy(blk, &d16, 2);
            for (int j = 0; j < 16; ++j) {
                int lo = (int)(x[2 * j] * id + 8.5f), hi = (int)(x[2 * j + 1] * id + 8.5f);
                lo = std::min(15, std::max(0, lo));
                hi = std::min(15, std::max(0, hi));
                blk[2 + j] = (uint8_t)(lo | (hi << 4));
            }
        }
    });
    return VLRF_HIP_OK;
}

int vlrf_dequantize(const void* src, int dtype, float* dst, int64_t n) {
    if (!src || !dst || n < 0) return VLRF_HIP_ERR_ARG;
    const uint8_t* in = static_cast<const uint8_t*>(src);
    if (dtype == VLRF_HIP_DT_F32) {
        std::memcpy(dst, src, sizeof(float) * (size_t)n);
        return VLRF_HIP_OK;
    }
    if (n % 32) return VLRF_HIP_ERR_ARG;
    if (dtype == VLRF_HIP_DT_Q8_0) {
        parallel_blocks(n / 32, [&](int64_t b0, int64_t b1) {
            for (int64_t b = b0; b < b1; ++b) {
                uint16_t d16;
                std::memcpy(&d16, in + b * 34, 2);
                const float d = f16_to_f32(d16);
                for (int i = 0; i < 32; ++i) dst[b * 32 + i] = (float)(int8_t)in[b * 34 + 2 + i] * d;
            }
        });
        return VLRF_HIP_OK;
    }
    if (dtype == VLRF_HIP_DT_Q4_0) {
        parallel_blocks(n / 32, [&](int64_t b0, int64_t b1) {
            for (int64_t b = b0; b < b1; ++b) {
                uint16_t d16;
                std::memcpy(&d16, in + b * 18, 2);
                const float d = f16_to_f32(d16);
                for (int j = 0; j < 16; ++j) {
                    const uint8_t byte = in[b * 18 + 2 + j];
                    dst[b * 32 + 2 * j] = (float)((int)(byte & 0x0F) - 8) * d;
                    dst[b * 32 + 2 * j + 1] = (float)((int)(byte >> 4) - 8) * d;
                }
            }
        });
        return VLRF_HIP_OK;
    }
    return VLRF_HIP_ERR_ARG;
}

int vlrf_synth_normal(uint64_t seed, uint64_t stream, float std_dev, float* out, int64_t n) {
    if (!out || n < 0) return VLRF_HIP_ERR_ARG;
    const uint64_t key = stream_key(seed, stream);
    const int64_t npairs = (n + 1) / 2;
    parallel_blocks(npairs, [&](int64_t p0, int64_t p1) {
        for (int64_t p = p0; p < p1; ++p) {
            const uint64_t a = splitmix64(key + 2 * (uint64_t)p);
            const uint64_t b = splitmix64(key + 2 * (uint64_t)p + 1);
            const double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;   // (0, 1]
            const double u2 = (double)(b >> 11) * 0x1.0p-53;         // [0, 1)
            const double r = std::sqrt(-2.0 * std::log(u1));
            const double th = 6.283185307179586 * u2;
            out[2 * p] = (float)((double)std_dev * r * std::cos(th));
            if (2 * p + 1 < n) out[2 * p + 1] = (float)((double)std_dev * r * std::sin(th));
        }
    });
    return VLRF_HIP_OK;
}

int vlrf_synth_tokens(uint64_t seed, uint64_t stream, int vocab, int32_t* out, int64_t n) {
    if (!out || n < 0 || vocab <= 0) return VLRF_HIP_ERR_ARG;
    const uint64_t key = stream_key(seed, stream);
    for (int64_t i = 0; i < n; ++i) out[i] = (int32_t)(splitmix64(key + (uint64_t)i) % (uint64_t)vocab);
    return VLRF_HIP_OK;
}

}  // extern "C"
