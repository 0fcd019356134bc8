// nfw.cpp - NFW weight files and loading them into a device model.
//
// Reference format (include/model/weights.hpp:58-62, parse_header :289-339;
// writer tools/converter/nfw_writer.py:11-27): header <u32 magic 0x4E465746,
// u32 version, u32 count, u32 reserved>, then per tensor <u16 name length,
// name, u8 ndim, i32 dims[ndim], i64 numel, [v2: u8 dtype], payload>.  Version
// 1 holds f32 payloads; version 2 adds the dtype byte, 0 = F32 and 1 = F16.
// Version 3 (this backend's extension) keeps the version-2 layout and adds
// block dtypes whose payload is the GGUF blocks themselves, numel/32 blocks in
// row-major element order: 2 = Q4_0 (18 B per block), 8 = Q8_0 (34 B per
// block) -- the GGML type numbers, so a converter copies GGUF tensors through
// byte for byte (tools/converter/convert_gguf.py:193-263 decodes them instead).
//
// The loader maps the engine's tensor names onto a vlrf_hip model through the
// public ABI: F16 payloads are widened with the reference's f16_to_f32
// (weights.hpp:76-96), a block-quantized embedding table is decoded to f32
// (the model gathers f32 rows), projection and LM-head blocks go to the device
// unchanged, and all-zero bias tensors (the converters write zero biases for
// bias-free models) are accepted and dropped.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../../include/vlrf_hip.h"

namespace vlrf_hip {
void set_error(const char* fmt, ...);   // api.hip: thread-local message for vlrf_hip_last_error
}

struct vlrf_nfw {
    std::string path;
    uint32_t version = 0;
    struct Entry {
        std::string name;
        int dtype = 0, ndim = 0;
        int32_t dims[8] = {0};
        int64_t numel = 0, bytes = 0, offset = 0;
    };
    std::vector<Entry> t;
};

namespace {

constexpr uint32_t kMagic = 0x4E465746u;

int64_t payload_bytes(int dtype, int64_t numel) {
    switch (dtype) {
        case VLRF_NFW_F32: return numel * 4;
        case VLRF_NFW_F16: return numel * 2;
        case VLRF_NFW_Q8_0: return numel % 32 ? -1 : numel / 32 * 34;
        case VLRF_NFW_Q4_0: return numel % 32 ? -1 : numel / 32 * 18;
        default: return -1;
    }
}

struct File {
    FILE* f = nullptr;
    explicit File(const char* p) : f(std::fopen(p, "rb")) {}
    ~File() {
        if (f) std::fclose(f);
    }
    bool read(void* dst, size_t n) { return std::fread(dst, 1, n, f) == n; }
};

// weights.hpp:76-96 f16_to_f32: exact, subnormals normalised, inf/NaN kept.
float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            e = 1;
            while (!(m & 0x400u)) { m <<= 1; --e; }
            m &= 0x3FFu;
            bits = sign | ((e + 112u) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float v;
    std::memcpy(&v, &bits, 4);
    return v;
}

bool ends_with(const std::string& s, const char* suf) {
    const size_t n = std::strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

// Allocation failures (a header that asks for more than the host holds) are
// returned as VLRF_HIP_ERR_NOMEM instead of escaping the C ABI.
template <class Fn>
int guarded(const char* what, Fn&& fn) {
    try {
        return fn();
    } catch (std::bad_alloc const&) {
        vlrf_hip::set_error("%s: host allocation failed", what);
    } catch (std::length_error const&) {
        vlrf_hip::set_error("%s: host allocation failed (size out of range)", what);
    }
    return VLRF_HIP_ERR_NOMEM;
}

}  // namespace

extern "C" {

static int nfw_open(const char* path, vlrf_nfw_t* out) {
    using vlrf_hip::set_error;
    if (!path || !out) { set_error("nfw_open: null argument"); return VLRF_HIP_ERR_ARG; }
    *out = nullptr;
    File f(path);
    if (!f.f) { set_error("nfw_open: cannot open '%s'", path); return VLRF_HIP_ERR_ARG; }
    uint32_t hdr[4];
    if (!f.read(hdr, sizeof hdr)) { set_error("nfw_open: '%s' is too short", path); return VLRF_HIP_ERR_ARG; }
    if (hdr[0] != kMagic) {
        set_error("nfw_open: bad magic 0x%08X (expected 0x4E465746) in '%s'", hdr[0], path);
        return VLRF_HIP_ERR_ARG;
    }
    if (hdr[1] < 1 || hdr[1] > 3) {
        set_error("nfw_open: unsupported version %u in '%s'", hdr[1], path);
        return VLRF_HIP_ERR_ARG;
    }
    std::unique_ptr<vlrf_nfw> h(new vlrf_nfw());
    h->path = path;
    h->version = hdr[1];
    std::fseek(f.f, 0, SEEK_END);
    const int64_t size = std::ftell(f.f);
    std::fseek(f.f, 16, SEEK_SET);
    for (uint32_t i = 0; i < hdr[2]; ++i) {
        vlrf_nfw::Entry e;
        uint16_t nl = 0;
        uint8_t nd = 0;
        if (!f.read(&nl, 2)) goto truncated;
        e.name.resize(nl);
        if (nl && !f.read(&e.name[0], nl)) goto truncated;
        if (!f.read(&nd, 1)) goto truncated;
        if (nd > 8) { set_error("nfw_open: tensor '%s' has %d dims", e.name.c_str(), nd); return VLRF_HIP_ERR_ARG; }
        e.ndim = nd;
        if (nd && !f.read(e.dims, 4 * nd)) goto truncated;
        if (!f.read(&e.numel, 8)) goto truncated;
        if (h->version >= 2) {
            uint8_t dt;
            if (!f.read(&dt, 1)) goto truncated;
            e.dtype = dt;
        }
        if (h->version == 2 && e.dtype > VLRF_NFW_F16) {
            set_error("nfw_open: dtype %d of '%s' needs version 3", e.dtype, e.name.c_str());
            return VLRF_HIP_ERR_ARG;
        }
        {
            // Every dtype stores at least 18 bytes per 32 elements, so a numel
            // beyond twice the bytes left cannot be in the file; checking that
            // first keeps the size products below in range.
            const int64_t left = size - std::ftell(f.f);
            if (e.numel > 2 * left) goto truncated;
            if (e.numel < 0) {   // before any size product: a negative count must not reach one
                set_error("nfw_open: tensor '%s' has a negative element count", e.name.c_str());
                return VLRF_HIP_ERR_ARG;
            }
            int64_t prod = 1;
            bool dims_ok = true;
            for (int d = 0; d < nd && dims_ok; ++d)
                dims_ok = e.dims[d] >= 0 && !__builtin_mul_overflow(prod, (int64_t)e.dims[d], &prod);
            if (!dims_ok) {
                set_error("nfw_open: tensor '%s' has a negative or overflowing dimension", e.name.c_str());
                return VLRF_HIP_ERR_ARG;
            }
            e.bytes = payload_bytes(e.dtype, e.numel);
            if (e.numel < 0 || (nd && prod != e.numel) || e.bytes < 0) {
                set_error("nfw_open: tensor '%s': dtype %d, numel %lld inconsistent", e.name.c_str(), e.dtype,
                          (long long)e.numel);
                return VLRF_HIP_ERR_ARG;
            }
            if ((e.dtype == VLRF_NFW_Q8_0 || e.dtype == VLRF_NFW_Q4_0) && (nd < 1 || e.dims[nd - 1] % 32)) {
                set_error("nfw_open: block tensor '%s' needs a last dimension divisible by 32", e.name.c_str());
                return VLRF_HIP_ERR_ARG;
            }
        }
        e.offset = std::ftell(f.f);
        if (e.offset + e.bytes > size) goto truncated;
        std::fseek(f.f, (long)e.bytes, SEEK_CUR);
        h->t.push_back(std::move(e));
    }
    *out = h.release();
    return VLRF_HIP_OK;
truncated:
    set_error("nfw_open: '%s' is truncated", path);
    return VLRF_HIP_ERR_ARG;
}

int vlrf_nfw_open(const char* path, vlrf_nfw_t* out) {
    if (out) *out = nullptr;
    return guarded("nfw_open", [&] { return nfw_open(path, out); });
}

void vlrf_nfw_close(vlrf_nfw_t f) { delete f; }

int vlrf_nfw_version(vlrf_nfw_t f) { return f ? (int)f->version : VLRF_HIP_ERR_ARG; }

int vlrf_nfw_count(vlrf_nfw_t f) { return f ? (int)f->t.size() : VLRF_HIP_ERR_ARG; }

int vlrf_nfw_find(vlrf_nfw_t f, const char* name) {
    if (!f || !name) return VLRF_HIP_ERR_ARG;
    for (size_t i = 0; i < f->t.size(); ++i)
        if (f->t[i].name == name) return (int)i;
    return -1;
}

int vlrf_nfw_tensor_info(vlrf_nfw_t f, int i, const char** name, int* dtype, int* ndim, int32_t* dims,
                         int64_t* numel, int64_t* bytes) {
    if (!f || i < 0 || i >= (int)f->t.size()) {
        vlrf_hip::set_error("nfw_tensor_info: index %d out of range", i);
        return VLRF_HIP_ERR_ARG;
    }
    const auto& e = f->t[i];
    if (name) *name = e.name.c_str();
    if (dtype) *dtype = e.dtype;
    if (ndim) *ndim = e.ndim;
    if (dims) std::memcpy(dims, e.dims, sizeof(int32_t) * e.ndim);
    if (numel) *numel = e.numel;
    if (bytes) *bytes = e.bytes;
    return VLRF_HIP_OK;
}

int vlrf_nfw_read(vlrf_nfw_t f, int i, void* dst, int64_t cap) {
    if (!f || !dst || i < 0 || i >= (int)f->t.size()) {
        vlrf_hip::set_error("nfw_read: bad arguments");
        return VLRF_HIP_ERR_ARG;
    }
    const auto& e = f->t[i];
    if (cap < e.bytes) {
        vlrf_hip::set_error("nfw_read: '%s' needs %lld bytes, buffer has %lld", e.name.c_str(), (long long)e.bytes,
                            (long long)cap);
        return VLRF_HIP_ERR_ARG;
    }
    File fh(f->path.c_str());
    if (!fh.f || std::fseek(fh.f, (long)e.offset, SEEK_SET) != 0 || !fh.read(dst, (size_t)e.bytes)) {
        vlrf_hip::set_error("nfw_read: read error on '%s'", e.name.c_str());
        return VLRF_HIP_ERR_ARG;
    }
    return VLRF_HIP_OK;
}

static int nfw_read_f32(vlrf_nfw_t f, int i, float* dst, int64_t n) {
    if (!f || !dst || i < 0 || i >= (int)f->t.size()) {
        vlrf_hip::set_error("nfw_read_f32: bad arguments");
        return VLRF_HIP_ERR_ARG;
    }
    const auto& e = f->t[i];
    if (n < e.numel) {
        vlrf_hip::set_error("nfw_read_f32: '%s' has %lld elements, buffer %lld", e.name.c_str(),
                            (long long)e.numel, (long long)n);
        return VLRF_HIP_ERR_ARG;
    }
    if (e.dtype == VLRF_NFW_F32) return vlrf_nfw_read(f, i, dst, n * 4);
    std::vector<uint8_t> raw((size_t)e.bytes);
    int rc = vlrf_nfw_read(f, i, raw.data(), e.bytes);
    if (rc) return rc;
    if (e.dtype == VLRF_NFW_F16) {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(raw.data());
        for (int64_t k = 0; k < e.numel; ++k) dst[k] = half_to_float(h[k]);
        return VLRF_HIP_OK;
    }
    return vlrf_dequantize(raw.data(), e.dtype == VLRF_NFW_Q8_0 ? VLRF_HIP_DT_Q8_0 : VLRF_HIP_DT_Q4_0, dst, e.numel);
}

int vlrf_nfw_read_f32(vlrf_nfw_t f, int i, float* dst, int64_t n) {
    return guarded("nfw_read_f32", [&] { return nfw_read_f32(f, i, dst, n); });
}

static int model_load_nfw(vlrf_hip_model_t m, const char* path, int* n_loaded) {
    using vlrf_hip::set_error;
    if (n_loaded) *n_loaded = 0;
    vlrf_hip_model_config cfg;
    int rc = vlrf_hip_model_get_config(m, &cfg);
    if (rc) return rc;
    vlrf_nfw_t f = nullptr;
    if ((rc = vlrf_nfw_open(path, &f))) return rc;
    std::unique_ptr<vlrf_nfw, void (*)(vlrf_nfw_t)> guard(f, vlrf_nfw_close);
    int loaded = 0;
    for (int i = 0; i < (int)f->t.size(); ++i) {
        const auto& e = f->t[i];
        const std::string& n = e.name;
        if (ends_with(n, ".bias")) {                  // zero biases of bias-free models
            std::vector<float> b((size_t)e.numel);
            if ((rc = vlrf_nfw_read_f32(f, i, b.data(), e.numel))) return rc;
            for (float v : b)
                if (v != 0.f) {
                    set_error("load_nfw: '%s' is a non-zero bias; the device model has no bias terms", n.c_str());
                    return VLRF_HIP_ERR_ARG;
                }
            continue;
        }
        const bool f32_slot = n == "embed.weight" || ends_with(n, "ln1.weight") || ends_with(n, "ln2.weight") ||
                              n == "ln_final.weight";
        const int rows = e.ndim >= 2 ? e.dims[0] : 1;
        const int cols = e.ndim >= 1 ? e.dims[e.ndim - 1] : 1;
        if (f32_slot || e.dtype == VLRF_NFW_F32 || e.dtype == VLRF_NFW_F16) {
            if (!f32_slot && cfg.weight_dtype != VLRF_HIP_DT_F32 && n != "lm_head.weight") {
                set_error("load_nfw: '%s' is %s but the model's projections are block type %d "
                          "(create the model with weight_dtype F32, or store the tensor as Q8_0/Q4_0)",
                          n.c_str(), e.dtype == VLRF_NFW_F16 ? "F16" : "F32", cfg.weight_dtype);
                return VLRF_HIP_ERR_ARG;
            }
            std::vector<float> v((size_t)e.numel);
            if ((rc = vlrf_nfw_read_f32(f, i, v.data(), e.numel))) return rc;
            rc = vlrf_hip_model_set_weight(m, n.c_str(), v.data(), VLRF_HIP_DT_F32, rows, cols);
        } else {
            std::vector<uint8_t> raw((size_t)e.bytes);
            if ((rc = vlrf_nfw_read(f, i, raw.data(), e.bytes))) return rc;
            rc = vlrf_hip_model_set_weight(m, n.c_str(), raw.data(), e.dtype, rows, cols);
        }
        if (rc) return rc;
        ++loaded;
    }
    if (n_loaded) *n_loaded = loaded;
    return VLRF_HIP_OK;
}

int vlrf_hip_model_load_nfw(vlrf_hip_model_t m, const char* path, int* n_loaded) {
    if (n_loaded) *n_loaded = 0;
    return guarded("load_nfw", [&] { return model_load_nfw(m, path, n_loaded); });
}

}  // extern "C"
