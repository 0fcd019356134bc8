// engine_hip_driver.cpp - the engine's own C API (src/api/vlrf_api.cpp with
// vlrf_amd/integration/engine_hip.patch applied, built with -DVLRF_USE_HIP)
// selecting the HIP backend: vlrf_generate_ids must return the CPU
// backend's ids (reference vlrf_api.cpp:417-462 -> TransformerModel::generate,
// transformer.hpp:439-547).
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile target `engine` builds it into
// oracle/_ref/engine_hip; tests/test_integration.py writes the model (an .nfw
// file with config.json beside it) and runs it.
//   engine_hip <weights.nfw>
// Cases: greedy with the engine's default F32 KV cache and with a Q8_0 cache
// (vlrf_set_kv_cache_type), and a request past max_seq_len; after each run
// vlrf_context_length must report what the CPU backend reports (the prompt
// plus one row per generated token, transformer.hpp:324-326,444-482).  Each
// prints PASS/FAIL; exit status 0 = all pass.
#include "vlrf.h"

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace {

int g_fail = 0;

void report(bool ok, const std::string& what) {
    std::printf("%s %s\n", ok ? "PASS" : "FAIL", what.c_str());
    std::fflush(stdout);
    if (!ok) ++g_fail;
}

std::vector<int32_t> run(VlrfModel m, std::vector<int32_t> const& prompt, int max_new) {
    std::vector<int32_t> out(prompt.size() + max_new + 8);
    int32_t n = (int32_t)out.size();
    const VlrfStatus st = vlrf_generate_ids(m, prompt.data(), (int32_t)prompt.size(), out.data(), &n, max_new,
                                            nullptr, nullptr);
    if (st != VLRF_OK) {
        std::printf("vlrf_generate_ids: %s\n", vlrf_status_str(st));
        return {};
    }
    out.resize(n);
    return out;
}

void compare(VlrfModel m, std::vector<int32_t> const& prompt, int max_new, const std::string& what) {
    if (vlrf_set_backend(VLRF_BACKEND_CPU) != VLRF_OK) { report(false, what + ": CPU backend"); return; }
    const std::vector<int32_t> cpu = run(m, prompt, max_new);
    const int32_t cpu_ctx = vlrf_context_length(m);
    if (vlrf_set_backend(VLRF_BACKEND_HIP) != VLRF_OK) { report(false, what + ": HIP backend unavailable"); return; }
    const std::string info = vlrf_backend_info();
    const std::vector<int32_t> hip = run(m, prompt, max_new);
    const int32_t hip_ctx = vlrf_context_length(m);
    int first = -1;
    for (size_t i = 0; i < cpu.size() && i < hip.size(); ++i)
        if (cpu[i] != hip[i]) { first = (int)i; break; }
    std::printf("  %s: backend [%s], cpu %zu ids, hip %zu ids, first difference %d\n", what.c_str(), info.c_str(),
                cpu.size(), hip.size(), first);
    report(!cpu.empty() && cpu.size() == hip.size() && first < 0 && info.find("HIP") != std::string::npos,
           "engine vlrf_generate_ids, HIP backend == CPU backend: " + what);
    std::printf("  %s: vlrf_context_length cpu %d, hip %d\n", what.c_str(), cpu_ctx, hip_ctx);
    report(cpu_ctx == hip_ctx && cpu_ctx > 0, "engine vlrf_context_length after generate, HIP == CPU: " + what);
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s weights.nfw\n", argv[0]);
        return 2;
    }
    VlrfModel m = vlrf_create_model();
    VlrfStatus st = vlrf_load_weights(m, argv[1], nullptr);
    if (st != VLRF_OK) {
        std::printf("FAIL vlrf_load_weights: %s\n", vlrf_status_str(st));
        return 1;
    }
    VlrfModelParams p;
    std::memset(&p, 0, sizeof p);
    vlrf_get_params(m, &p);
    p.use_sampling = 0;                      // config.json loads with sampling on
    vlrf_set_generation_params(m, &p);
    std::printf("[model] %s\n", vlrf_model_summary(m));

    std::vector<int32_t> prompt(40);
    uint32_t s = 12345u;
    for (auto& t : prompt) {
        s = s * 1664525u + 1013904223u;
        t = (int32_t)((s >> 8) % (uint32_t)p.vocab_size);
    }
    compare(m, prompt, 48, "48 greedy steps, KV f32");
    vlrf_set_kv_cache_type(m, VLRF_KV_Q8_0);
    compare(m, prompt, 48, "48 greedy steps, KV q8_0");
    compare(m, prompt, 4 * p.max_seq_len, "max_new_tokens past max_seq_len");
    vlrf_free_model(m);
    std::printf("%s: %d failure(s)\n", g_fail ? "FAILED" : "OK", g_fail);
    return g_fail ? 1 : 0;
}
