// nfw_fuzz.cpp - host-side fuzz of the NFW parser (vlrf_amd/csrc/host/nfw.cpp),
// built with AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/test_nfw_fuzz.py: every truncation of each seed file and random byte
// mutations of it (header-heavy for half of them), each written to a file,
// opened, and every tensor read in full and into too-small buffers.  Usage:
//   nfw_fuzz <tmpfile> <iterations per seed> <seed files...>
// The model-loading entry points the parser's translation unit references
// are stubbed (never called here).
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <cstdarg>
#include <random>
#include <string>
#include <vector>
#include "vlrf_hip.h"

namespace vlrf_hip {
void set_error(const char* fmt, ...) { (void)fmt; }
}
extern "C" int vlrf_hip_model_get_config(vlrf_hip_model_t, vlrf_hip_model_config*) { return VLRF_HIP_ERR_ARG; }
extern "C" int vlrf_hip_model_set_weight(vlrf_hip_model_t, const char*, const void*, int, int, int) { return VLRF_HIP_ERR_ARG; }

static std::vector<uint8_t> slurp(const char* p) {
    FILE* f = fopen(p, "rb"); std::vector<uint8_t> v;
    if (!f) return v;
    fseek(f, 0, SEEK_END); long n = ftell(f); fseek(f, 0, SEEK_SET);
    v.resize(n); if (fread(v.data(), 1, n, f) != (size_t)n) v.clear(); fclose(f); return v;
}
static long opened = 0, rejected = 0;
static void try_file(const std::vector<uint8_t>& d, const char* tmp) {
    FILE* f = fopen(tmp, "wb"); if (!d.empty()) fwrite(d.data(), 1, d.size(), f); fclose(f);
    vlrf_nfw_t h = nullptr;
    if (vlrf_nfw_open(tmp, &h) != VLRF_HIP_OK) { ++rejected; return; }
    ++opened;
    const int n = vlrf_nfw_count(h);
    for (int i = -1; i <= n; ++i) {
        const char* name = nullptr; int dt = 0, nd = 0; int32_t dims[8]; int64_t numel = 0, bytes = 0;
        if (vlrf_nfw_tensor_info(h, i, &name, &dt, &nd, dims, &numel, &bytes) != VLRF_HIP_OK) continue;
        if (name) vlrf_nfw_find(h, name);
        if (bytes >= 0 && bytes < (64 << 20)) {
            std::vector<uint8_t> buf((size_t)bytes + 1);
            vlrf_nfw_read(h, i, buf.data(), bytes);
            vlrf_nfw_read(h, i, buf.data(), bytes / 2);   // too small: must be refused, not overrun
        }
        if (numel >= 0 && numel < (16 << 20)) {
            std::vector<float> fb((size_t)numel + 1);
            vlrf_nfw_read_f32(h, i, fb.data(), numel);
            if (numel > 0) vlrf_nfw_read_f32(h, i, fb.data(), numel - 1);
        }
    }
    vlrf_nfw_close(h);
}
int main(int argc, char** argv) {
    if (argc < 4) { printf("usage: nfw_fuzz <tmpfile> <iterations> <seeds...>\n"); return 2; }
    const char* tmp = argv[1];
    const int iters = atoi(argv[2]);
    std::mt19937_64 rng(12345);
    for (int a = 3; a < argc; ++a) {
        const auto seed = slurp(argv[a]);
        if (seed.empty()) { printf("cannot read %s\n", argv[a]); return 1; }
        for (size_t L = 0; L < seed.size(); ++L) try_file(std::vector<uint8_t>(seed.begin(), seed.begin() + L), tmp);
        for (int it = 0; it < iters; ++it) {
            auto d = seed;
            const int k = 1 + (int)(rng() % 4);
            for (int j = 0; j < k; ++j) {
                const size_t pos = rng() % std::min<size_t>(d.size(), it % 2 ? d.size() : 96);   // header-heavy half
                const int mode = (int)(rng() % 4);
                if (mode == 0) d[pos] ^= (uint8_t)(1u << (rng() % 8));
                else if (mode == 1) d[pos] = 0xFF;
                else if (mode == 2) d[pos] = 0x00;
                else d[pos] = (uint8_t)rng();
            }
            if (rng() % 8 == 0) d.resize(rng() % (d.size() + 1));
            try_file(d, tmp);
        }
        printf("%s: done\n", argv[a]);
    }
    printf("opened %ld, rejected %ld\n", opened, rejected);
    return 0;
}
