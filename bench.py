"""Decode benchmark of the MI355X HIP backend (one GPU).

Workload (the metric's configuration): a random-init
Llama-style 1.1B model (22 layers, hidden 2048, FFN 5632 SwiGLU, 32/4 heads,
head_dim 64, vocab 32000) with Q8_0 weights and a Q8_0 KV cache.  The cache is
filled to 2048 tokens of seeded random ids (untimed: 2048-W prompt tokens
through the decode step, then W warm-up decode steps), then exactly `steps`
greedy decode steps are timed with HIP events on the library's stream
(context 2048 -> 2048+steps).  value = steps / time (tok/s).

step_kernels: after the timed steps, as many more greedy steps with the
step's kernels queued one by one and every launch timed by its own start/stop
events (vlrf_hip_model_time_launches: hipExtLaunchKernel stamps the kernel's
own begin and end, so no marker sits between launches), on the library's
stream.  Per kernel kind: average us per launch, launches and us per step,
algorithmic bytes per launch at the middle context, and the GB/s and fraction
of the 8 TB/s peak they imply (the metric's attention + GEMV breakdown), with
the committed rocprofv3 trace's average beside it (rocprof_us, from
profiles/decode_step_llama1b_{q8,q4}_kernel_stats.md).

roofline: the dominant kernel of the step by time per step, from step_kernels
(the fused RMSNorm + QKV + RoPE + KV append + attention launch at this shape).
`traffic` is null: a rocprofv3 counter pass over that launch has not been run
(a profiler crash inside its dispatch interception).

roofline_gemv: the fused RMSNorm + gate/up dequant-GEMV with the SwiGLU
epilogue (52% of a step's bytes), timed with HIP events over launches that
rotate through 12 distinct weight pairs (295 MB, more than the 256 MB
Infinity Cache), so the bytes come from HBM; its `traffic` is the HBM bytes
per launch that rocprofv3 counted (FETCH_SIZE and WRITE_SIZE passes over
`bench.py --roofline-only`, each scaled by the same counter on a plain 256 MiB
device copy), read from profiles/gemv_swiglu_q8_1b_pmc.txt.

cpu_baseline: the oracle's restatement of the reference decode step
(oracle/vlrf_oracle.c: f32 decoded weights, AVX2 streaming GEMV, full-cache
dequant, per-head flash attention) at context 2048 on every hardware thread
of the process's CPU set (nproc and the CPU model in the line), up to 32
steps within about 20 s.

    python bench.py [--gpus 1] [--steps 128] [--warmup 8] [--dtype q8_0|q4_0]
    python bench.py --roofline-only     # copy calibration + roofline launches only
    python bench.py --prefill           # config 5: one Llama-8B-shape layer, T=2048 prefill
    python bench.py --decode-8b [--layers 4]   # decode at the 8B layer shape (d_head 128)
    python bench.py --configs           # configs 1-3: kernel-level GB/s, one JSON line each
    python bench.py --summarize-trace run_kernel_trace.csv --steps 128 --launches-per-step 90
    python bench.py --summarize-runs run_kernel_trace.csv --skip 2 --runs 5   # prefill runs

--prefill prints its own line: one Llama-8B-shape
layer (hidden 4096, 32/8 heads, head_dim 128, FFN 14336 SwiGLU, Q8_0 weights
dequantized into the GEMM tiles) over a causal 2048-token prompt of N(0,1)
embedded rows, on the matrix cores (bf16 operands, f32 accumulation), each run
from an empty cache; the variant over bf16 copies of the weights is reported
beside it as `bf16_expansion`.  FLOPs per
layer = 2*T*(D*(D+2*dkv) + D*D + 3*D*F) + 4*H*d*T*T/2 = 927.7 GFLOP; the
roofline is the dense bf16 MFMA peak (2.5 PFLOP/s).

--configs (BASELINE.json configs[0..2]) prints one line per kernel case, each
timed with HIP events over launches that rotate through distinct instances
totalling more than the 256 MB Infinity Cache, plus the latency of one
instance repeated (cache-warm):
  cfg1  f32 attention Q[8,1,64], K/V[8,512,64], non-causal: 2,101,248 B/call;
  cfg2  decode attention over a Q8_0 cache, 32 q / 4 kv heads, d 64, ctx 4096:
        2,146,304 B/call (codes, row scales, q, out);
  cfg3  quantized linear up 5632x2048 and down 2048x5632, Q8_0 and Q4_0,
        M = 1, 4, 16: weight bytes + 4*M*(K+N) per call.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0   # MI355X published HBM3E bandwidth
PMC_SUMMARY = os.path.join(ROOT, "profiles", "gemv_swiglu_q8_1b_pmc.txt")
COPY_BYTES = 256 << 20  # calibration copy size for the PMC passes


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_roofline(ctx, V, F, cfg, dtype, launches=96):
    """Live HIP-event timing of the gate/up SwiGLU dequant-GEMV at the step's shape."""
    D, Fd = cfg["d_model"], cfg["d_ff"]
    pairs = []
    for i in range(12):
        g = F.quantize(F.normal(99, f"bench.g{i}", Fd * D, 0.02), dtype)
        u = F.quantize(F.normal(99, f"bench.u{i}", Fd * D, 0.02), dtype)
        pairs.append((V.QuantWeight(ctx, g, dtype, Fd, D), V.QuantWeight(ctx, u, dtype, Fd, D)))
    x = ctx.to_device(F.normal(99, "bench.x", D))
    nw = ctx.to_device(np.ones(D, np.float32))
    h = ctx.alloc(Fd * 4)
    for i in range(24):                       # warm-up
        wg, wu = pairs[i % 12]
        ctx.qlinear_swiglu(wg, wu, x, h, 1, nw, 1e-5)
    ctx.sync()
    ctx.timer_start()
    for i in range(launches):
        wg, wu = pairs[i % 12]
        ctx.qlinear_swiglu(wg, wu, x, h, 1, nw, 1e-5)
    ms = ctx.timer_stop()
    per_launch_s = ms / 1e3 / launches
    wbytes = 2 * pairs[0][0].device_bytes
    algo = wbytes + D * 4 * 2 + Fd * 4          # weights + x + norm weight + h
    achieved = algo / per_launch_s / 1e9
    chunk = 64 * (16 if dtype == V.DT_Q8_0 else 32)      # K columns per lane-chunk of one wave
    # XM: 1 fused RMSNorm, + 16 when every wave holds one row (at most 768 workgroups of 8 rows)
    xm = 1 | (16 if (Fd + 7) // 8 <= 768 else 0)
    name = "gemv_kernel<%d, %d, 1, true, %d>" % (dtype, (D + chunk - 1) // chunk, xm)
    return {"kernel": name + " (RMSNorm + gate/up %dx%d + SwiGLU)" % (Fd, D),
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": pmc_traffic(dtype),
            "bytes_per_launch": int(algo), "us_per_launch": round(per_launch_s * 1e6, 3),
            "launches": launches}


def pmc_traffic(dtype):
    """HBM bytes per launch from the committed rocprofv3 PMC summary (Q8_0 only)."""
    if dtype != 8 or not os.path.exists(PMC_SUMMARY):
        return None
    for line in open(PMC_SUMMARY):
        if line.startswith("traffic_bytes_per_launch"):
            return int(float(line.split("=")[1]))
    return None


def copy_calibration(ctx):
    """Three plain device copies of COPY_BYTES (the runtime's blit copy
    kernel), so that a PMC pass can relate FETCH_SIZE / WRITE_SIZE to a known
    byte count."""
    src, dst = ctx.alloc(COPY_BYTES), ctx.alloc(COPY_BYTES)
    src.zero()
    for _ in range(3):
        dst.copy_from(src)
    ctx.sync()
    log(f"[bench] copy calibration: 3 x {COPY_BYTES} B device copy")
    src.free()
    dst.free()


MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 matrix peak


def prefill_flops(cfg, T):
    D, F, H = cfg["d_model"], cfg["d_ff"], cfg["n_heads"]
    dh = D // H
    dkv = cfg["n_kv_heads"] * dh
    gemm = 2.0 * T * (D * (D + 2 * dkv) + D * D + 3 * D * F)
    attn = 4.0 * H * dh * T * T / 2          # QK^T and PV over the causal half
    return gemm + attn


def prefill_runs(ctx, model, x, out, warmup, steps):
    """warmup + steps layer prefills from an empty cache: (mean ms of the
    timed runs, ms of the first run)."""
    times, first_ms = [], None
    for i in range(warmup + steps):
        model.reset()
        ctx.timer_start()
        model.forward_hidden(x, out)
        ms = ctx.timer_stop()
        if first_ms is None:
            first_ms = ms
        if i >= warmup:
            times.append(ms)
    return float(np.mean(times)), first_ms


def prefill_bench(a, V, F):
    """One Llama-8B-shape layer, T-token causal prefill (MFMA path).

    value: the stated workload of the configuration, quantized weights
    dequantized into the GEMM's LDS tiles (VLRF_HIP_PREFILL_BF16=0: no bf16
    copy of any weight exists).  Beside it, `bf16_expansion`: the same layer
    once each weight has a bf16 expansion (2 bytes per weight, made by the
    first GEMM of more than 128 rows on it), timed after its first run, with
    the first run (which makes the expansions) reported as well."""
    dtype = V.DT_Q8_0 if a.dtype == "q8_0" else V.DT_Q4_0
    T = a.prefill_tokens
    cfg = F.llama8b_layer(dtype, max_seq_len=T)
    ctx = V.Context(0)
    log("[prefill]", ctx.device_info())
    t0 = time.time()
    model = V.Model(ctx, cfg)
    F.load_model(model, a.seed)
    log(f"[prefill] weights generated and uploaded in {time.time() - t0:.1f}s")
    x = ctx.to_device(F.normal(a.seed, "prefill.x", T * cfg["d_model"]))
    out = ctx.alloc(T * cfg["d_model"] * 4)
    fl = prefill_flops(cfg, T)
    os.environ["VLRF_HIP_PREFILL_BF16"] = "0"
    ms, _ = prefill_runs(ctx, model, x, out, a.warmup, a.steps)
    os.environ["VLRF_HIP_PREFILL_BF16"] = "1"
    bms, bfirst = prefill_runs(ctx, model, x, out, 1, a.steps)
    tflops = fl / (ms / 1e3) / 1e12
    btflops = fl / (bms / 1e3) / 1e12
    log(f"[prefill] in-tile dequant {ms:.4f} ms ({tflops:.1f} TFLOP/s); bf16 expansions {bms:.4f} ms "
        f"({btflops:.1f} TFLOP/s), first run with the expansion {bfirst:.4f} ms")
    return {
        "metric": "prefill TFLOP/s of one Llama-8B-shape layer, T=%d" % T,
        "value": round(tflops, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 operands, f32 accumulate, %s weights dequantized in the GEMM tiles, q8_0 KV" % a.dtype,
        "data": "synthetic: seeded N(0,0.02) weights, N(0,1) embedded rows",
        "config": {"workload": "llama-8B-shape layer prefill, causal T=%d from an empty cache" % T,
                   "weights": a.dtype, "hidden": 4096, "ffn": 14336, "heads": "32/8", "head_dim": 128},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "flops_per_step": fl},
        # The weights' bf16 expansions (2 bytes per weight beside the blocks),
        # made once by the first run: not the configuration's workload.
        "bf16_expansion": {"tflops": round(btflops, 1), "ms_per_step": round(bms, 4),
                           "frac": round(btflops / MFMA_BF16_PEAK_TFLOPS, 4),
                           "first_run_ms_with_expansion": round(bfirst, 4)},
    }


def timed(ctx, fn, n_inst, launches):
    """Mean ms per launch over `launches` calls fn(i % n_inst), after a warm-up."""
    for i in range(min(launches, 2 * n_inst)):
        fn(i % n_inst)
    ctx.sync()
    ctx.timer_start()
    for i in range(launches):
        fn(i % n_inst)
    return ctx.timer_stop() / launches


def config_line(name, workload, bytes_per_call, ms_rot, ms_warm, extra=None):
    gbs = bytes_per_call / (ms_rot / 1e3) / 1e9
    out = {"metric": name, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
           "config": {"workload": workload}, "bytes_per_call": int(bytes_per_call),
           "us_per_call_rotating": round(ms_rot * 1e3, 3), "us_per_call_repeated": round(ms_warm * 1e3, 3),
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbs / HBM_PEAK_GBS, 4)}}
    if extra:
        out.update(extra)
    return out


def configs_bench(V, F):
    """Kernel-level measurements of configs 1-3 through the C ABI."""
    ctx = V.Context(0)
    log("[configs]", ctx.device_info())
    lines = []

    # cfg1: f32 fused attention, 8 heads, T=1, ctx 512, d 64, non-causal.
    nh, T, L, d = 8, 1, 512, 64
    n1 = 128
    kv_elems = nh * L * d
    K = ctx.to_device(np.tile(F.normal(5, "cfg1.k", kv_elems), n1))
    Vb = ctx.to_device(np.tile(F.normal(5, "cfg1.v", kv_elems), n1))
    Q = ctx.to_device(np.tile(F.normal(5, "cfg1.q", nh * d), n1))
    O = ctx.alloc(n1 * nh * d * 4)
    f4 = 4

    def cfg1(i):
        V.check(V.lib().vlrf_hip_attn_f32(ctx.h, Q.ptr + i * nh * d * f4, K.ptr + i * kv_elems * f4,
                                          Vb.ptr + i * kv_elems * f4, O.ptr + i * nh * d * f4,
                                          nh, T, L, d, 0.125, 0))
    b1 = 2 * kv_elems * 4 + 2 * nh * d * 4
    lines.append(config_line("cfg1 f32 attention GB/s", "Q[8,1,64] K/V[8,512,64] f32, non-causal, "
                             "128 instances rotating", b1, timed(ctx, cfg1, n1, 512),
                             timed(ctx, cfg1, 1, 512)))
    del K, Vb, Q, O

    # cfg2: decode attention over a Q8_0 cache, 128 caches (one per "layer").
    n2, ctxl, nkv, nq = 128, 4096, 4, 32
    kv = V.KVCache(ctx, n2, ctxl, nkv, d)
    k = ctx.to_device(F.normal(6, "cfg2.k", ctxl * nkv * d))
    v = ctx.to_device(F.normal(6, "cfg2.v", ctxl * nkv * d))
    for layer in range(n2):
        kv.append(layer, k, v, ctxl)
    del k, v
    q = ctx.to_device(F.normal(6, "cfg2.q", nq * d))
    o = ctx.alloc(nq * d * 4)

    def cfg2(i):
        kv.attention_decode(i, q, o, nq, ctxl, 0.125)
    b2 = 2 * ctxl * nkv * d + 2 * ctxl * 4 + 2 * nq * d * 4
    lines.append(config_line("cfg2 Q8_0-KV GQA decode attention GB/s",
                             "32 q / 4 kv heads, d 64, ctx 4096, 128 caches rotating", b2,
                             timed(ctx, cfg2, n2, 512), timed(ctx, cfg2, 1, 512)))
    del kv

    # cfg3: quantized linear, 24 weight copies per shape (> 256 MB for Q8_0).
    for dtype, dname in ((V.DT_Q8_0, "q8_0"), (V.DT_Q4_0, "q4_0")):
        for wname, N, Kd in (("up", 5632, 2048), ("down", 2048, 5632)):
            n3 = 24 if dtype == V.DT_Q8_0 else 48
            base = F.quantize(F.normal(7, f"cfg3.{wname}", N * Kd, 0.02), dtype)
            ws = [V.QuantWeight(ctx, base, dtype, N, Kd) for _ in range(n3)]
            # M = 64 and 128 beside the configuration's 1, 4, 16: the
            # K-split matrix-core GEMM of 17..128 rows.
            for M in (1, 4, 16, 64, 128):
                x = ctx.to_device(F.normal(7, f"cfg3.x{M}", M * Kd))
                y = ctx.alloc(M * N * 4)

                def cfg3(i):
                    ctx.qlinear(ws[i], x, y, M)
                b3 = ws[0].device_bytes + 4 * M * (Kd + N)
                lines.append(config_line(
                    f"cfg3 quantized linear GB/s ({wname} {N}x{Kd} {dname} M={M})",
                    f"y[{M},{N}] = x[{M},{Kd}] . W^T, {dname} weights, {n3} copies rotating", b3,
                    timed(ctx, cfg3, n3, 8 * n3), timed(ctx, cfg3, 1, 8 * n3),
                    {"gflop_per_call": round(2e-9 * M * N * Kd, 4)}))
            del ws
    for line in lines:
        print(json.dumps(line), flush=True)


def weight_bytes(dtype, rows, cols):
    """Device bytes of a quantized weight: codes plus one f16 scale per 32."""
    codes = rows * cols if dtype == 8 else rows * cols // 2
    return codes + rows * (cols // 32) * 2




def kernel_bytes(cfg, dtype, ctx_len, nparts):
    """Algorithmic HBM bytes per launch of each kind at context ctx_len: the
    weights once, the cache rows attention reads, activations in and out."""
    D, Fd, H, G = cfg["d_model"], cfg["d_ff"], cfg["n_heads"], cfg["n_kv_heads"]
    dh = D // H
    dkv, V_ = G * dh, cfg["vocab_size"]
    part = H * nparts * 68 * 4
    kv_read = ctx_len * dkv * 2 + ctx_len * 4 * 2          # K and V codes + row scales
    return {
        "qkv_attn": weight_bytes(dtype, D + 2 * dkv, D) + kv_read + D * 8 + 2 * dkv + 8 + part,
        "o_proj": weight_bytes(dtype, D, D) + part + D * 8,
        "gate_up": 2 * weight_bytes(dtype, Fd, D) + D * 8 + Fd * 4,
        "down": weight_bytes(dtype, D, Fd) + Fd * 4 + D * 8,
        # The LM head's workgroups (at most 512) also leave one (max, index)
        # pair each, and the argmax step reduces only those.
        "lm_head": weight_bytes(dtype, V_, D) + D * 8 + V_ * 4 + 512 * 8,
        "argmax": 512 * 8,
    }


KERNEL_KINDS = (  # (kind, pattern in the profile's kernel name)
    ("qkv_attn", "qkv_attn_kernel<"),
    ("o_proj", ", false, 28>"),
    ("gate_up", ", true, 17>"),
    ("down", ", false, 20>"),
    ("lm_head", ", false, 65>"),
    ("argmax", "argmax_pairs_step_kernel"),
)


def profile_kernel_us(wname):
    """Average us per launch of each kind in the committed rocprofv3 kernel
    trace of the same workload (profiles/decode_step_llama1b_{q8,q4}_kernel_stats.md),
    for comparison with the live event timing."""
    path = os.path.join(ROOT, "profiles", f"decode_step_llama1b_{wname[:2]}_kernel_stats.md")
    if not os.path.exists(path):
        return None, None
    calls, tot = {}, {}
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) < 7 or not cells[1].replace(".", "").isdigit():
            continue
        for kind, pat in KERNEL_KINDS:
            if pat in cells[0]:
                n, us = float(cells[1]), float(cells[2])
                calls[kind] = calls.get(kind, 0.0) + n
                tot[kind] = tot.get(kind, 0.0) + n * us
    return {k: round(tot[k] / calls[k], 3) for k in calls}, os.path.relpath(path, ROOT)


def step_kernels(model, cfg, dtype, wname, first, steps, ctx_first):
    """Live per-kernel breakdown of the decode step: `steps` greedy steps with
    every launch timed by its own start/stop events (vlrf_hip_model_time_launches,
    the kernels queued one by one), at contexts ctx_first..ctx_first+steps-1.
    Per kind: average us per launch, launches per step, algorithmic bytes per
    launch at the middle context and the GB/s and fraction of peak they imply."""
    live = model.time_launches(first, steps)
    ctx_mid = ctx_first + steps // 2
    nparts = (cfg["max_seq_len"] + 511) // 512 + 1
    nb = kernel_bytes(cfg, dtype, ctx_mid, nparts)
    prof, src = profile_kernel_us(wname)
    out = {}
    for kind, (us_sum, n) in live.items():
        us = us_sum / n
        row = {"us": round(us, 3), "calls_per_step": round(n / steps, 2), "us_per_step": round(us_sum / steps, 2)}
        if kind in nb:
            gbs = nb[kind] / (us * 1e-6) / 1e9
            row.update({"bytes": int(nb[kind]), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)})
        if prof and kind in prof:
            row["rocprof_us"] = prof[kind]
        out[kind] = row
    res = {"kernels": out, "timing": "hipExtLaunchKernel start/stop events per launch, %d steps" % steps,
           "contexts": [ctx_first, ctx_first + steps - 1], "bytes_at_ctx": ctx_mid}
    if src:
        res["rocprof_source"] = src
    return res


def dominant_roofline(sk):
    """The roofline object for the step's dominant kernel by time per step."""
    kind, row = max(((k, r) for k, r in sk["kernels"].items() if "bytes" in r), key=lambda kv: kv[1]["us_per_step"])
    names = {"qkv_attn": "qkv_attn_kernel (RMSNorm + QKV projection + RoPE + KV append + chunked attention)",
             "gate_up": "gemv_kernel (RMSNorm + gate/up + SwiGLU)", "down": "gemv_kernel (down + residual)",
             "o_proj": "gemv_kernel (partials merge + O projection + residual)",
             "lm_head": "gemv_kernel (final RMSNorm + LM head + argmax pairs)"}
    return {"kernel": names.get(kind, kind), "kind": kind, "bound": "hbm", "achieved": row["GB/s"],
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": row["frac"], "traffic": None,
            "bytes_per_launch": row["bytes"], "us_per_launch": row["us"], "us_per_step": row["us_per_step"],
            "timing": sk["timing"]}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_plan(cfg, ctx_len, max_steps):
    """The oracle model's own configuration for the CPU leg: its cache holds
    the ctx_len - 1 filled rows, the warm-up step and up to max_steps timed
    steps, whatever cache the GPU model was sized for (the GPU run's --steps
    does not bound the CPU sample)."""
    ocfg = dict(cfg)
    ocfg["max_seq_len"] = ctx_len + max_steps + 1
    return ocfg


def _cpu_decode_rate(om, ocfg, ctx_len, budget_s, max_steps):
    """(steps, tok/s) of decode steps from a cache of ctx_len - 1 seeded rows."""
    om.reset()
    om.fill_kv(ctx_len - 1, seed=7)
    tok = 1
    t0 = time.perf_counter()
    tok = om.forward([tok])                   # warm-up step: the cache now holds ctx_len rows
    warm = time.perf_counter() - t0
    room = ocfg["max_seq_len"] - om.used      # rows left for timed steps
    n = max(1, min(max_steps, room, int(budget_s / max(warm, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(n):
        tok = om.forward([tok])
    return n, n / (time.perf_counter() - t0)


def _port_threads(threads):
    if threads is None:
        try:
            threads = len(os.sched_getaffinity(0))
        except AttributeError:
            threads = os.cpu_count() or 1
    return max(1, threads)


def cpu_baseline(cfg, f32w, ctx_len, gpu_steps, budget_s=20.0, max_steps=32, threads=None,
                 prefer_ref=True, port_budget_s=8.0):
    """Decode steps at context ctx_len on the CPU: the reference's own
    TransformerModel (oracle/_ref, built from its sources with its default
    flags; its thread pool takes every hardware thread) when that library is
    present, with the C restatement (every hardware thread of the process's
    CPU set) timed beside it as `port`; else the restatement alone.  Both
    start from the same seeded Q8_0 cache rows instead of a CPU prefill."""
    import oracle
    ocfg = cpu_baseline_plan(cfg, ctx_len, max_steps)
    pt = _port_threads(threads)
    port_what = f"oracle restatement, {pt} threads = every hardware thread of the process's CPU set"
    out = {"unit": "tok/s", "nproc": os.cpu_count(), "cpu": cpu_model()}
    if prefer_ref and oracle.ref() is not None:
        om = oracle.RefModel(ocfg, f32w)
        n, rate = _cpu_decode_rate(om, ocfg, ctx_len, budget_s, max_steps)
        del om
        rt = oracle.RefModel.threads()
        what = f"reference TransformerModel built from its sources, its own pool of {rt} threads"
        om = oracle.Model(ocfg, f32w, n_threads=pt)
        pn, prate = _cpu_decode_rate(om, ocfg, ctx_len, port_budget_s, max_steps)
        del om
        out.update(value=round(rate, 3), cores=rt, kind="reference",
                   port={"value": round(prate, 3), "cores": pt, "steps": pn})
    else:
        om = oracle.Model(ocfg, f32w, n_threads=pt)
        n, rate = _cpu_decode_rate(om, ocfg, ctx_len, budget_s, max_steps)
        del om
        what = port_what
        out.update(value=round(rate, 3), cores=pt, kind="port")
    out["sample"] = (f"{n} decode steps (the GPU timed {gpu_steps}) of the 1.1B-shape f32-decoded model at "
                     f"context {ctx_len}-{ctx_len + n} ({what}, Q8_0 KV cache filled with seeded codes "
                     f"instead of a CPU prefill)")
    return {k: out[k] for k in ("value", "unit", "cores", "kind", "port", "nproc", "cpu", "sample") if k in out}


def summarize_trace(path, steps, per_step):
    """The last `steps` decode steps of a rocprofv3 kernel trace (CSV): the
    runtime's own copy and fill kernels left out, the remaining dispatches
    taken from the end, steps x per_step of them; per-kernel average
    duration and time per step, as markdown."""
    import csv
    rows = [r for r in csv.DictReader(open(path)) if not r["Kernel_Name"].startswith("__amd_rocclr")]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    tail = rows[-steps * per_step:]
    agg = {}
    for r in tail:
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        name = r["Kernel_Name"]
        agg.setdefault(name, []).append(d)
    span = (int(tail[-1]["End_Timestamp"]) - int(tail[0]["Start_Timestamp"])) / 1e3
    total = sum(sum(v) for v in agg.values())
    print(f"{len(tail)} dispatches = {steps} steps x {per_step}; span {span / steps:.1f} us/step, "
          f"kernel time {total / steps:.1f} us/step\n")
    print("| kernel | calls/step | avg us | min us | max us | us/step | % |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for name, v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        short = name.replace("void ", "").replace("vlrf_hip::(anonymous namespace)::", "")
        short = short.split("(")[0]
        print(f"| {short} | {len(v) / steps:.2f} | {np.mean(v):.2f} | {np.min(v):.2f} | {np.max(v):.2f} | "
              f"{sum(v) / steps:.1f} | {100 * sum(v) / total:.1f} |")


def summarize_runs(path, skip, nruns, clock_ghz=2.4, simds=1024):
    """Per-kernel averages over runs [skip, skip + nruns) of a rocprofv3 CSV
    (kernel trace or counter collection), a run being the dispatches between
    two groups of the runtime's own copy/fill kernels (model.reset() before
    each layer prefill).  With SQ_VALU_MFMA_BUSY_CYCLES in the file: the MFMA
    busy fraction of each kernel, busy cycles / (duration x clock x SIMDs)."""
    import csv
    import collections
    disp = collections.OrderedDict()
    for r in csv.DictReader(open(path)):
        k = r.get("Dispatch_Id") or r.get("Correlation_Id")
        e = disp.setdefault(k, {"name": r["Kernel_Name"], "t0": int(r["Start_Timestamp"]),
                                "us": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3})
        if "Counter_Name" in r:
            e[r["Counter_Name"]] = float(r["Counter_Value"])
    runs, cur = [], []
    for e in sorted(disp.values(), key=lambda e: e["t0"]):
        if e["name"].startswith("__amd_rocclr"):
            if cur:
                runs.append(cur)
                cur = []
            continue
        cur.append(e)
    if cur:
        runs.append(cur)
    sel = runs[skip:skip + nruns]
    agg = collections.OrderedDict()
    for run in sel:
        for e in run:
            n = e["name"].replace("void ", "").replace("vlrf_hip::(anonymous namespace)::", "")
            agg.setdefault(n.replace("vlrf_hip::", "").split("(")[0], []).append(e)
    mfma = any("SQ_VALU_MFMA_BUSY_CYCLES" in e for run in sel for e in run)
    tot_us = sum(e["us"] for run in sel for e in run) / max(1, len(sel))
    print(f"runs {skip}..{skip + len(sel) - 1} of {len(runs)} (dispatches per run {[len(r) for r in sel]}); "
          f"kernel time per run {tot_us:.1f} us\n")
    head = "| kernel | calls/run | avg us | min us | max us | us/run |" + (" MFMA busy |" if mfma else "")
    print(head)
    print("|---|---:|---:|---:|---:|---:|" + ("---:|" if mfma else ""))
    busy_tot = 0.0
    for n, es in agg.items():
        us = [e["us"] for e in es]
        line = (f"| {n} | {len(es) / len(sel):.2f} | {np.mean(us):.2f} | {np.min(us):.2f} | {np.max(us):.2f} | "
                f"{sum(us) / len(sel):.1f} |")
        if mfma:
            mb = np.mean([e.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) for e in es])
            busy_tot += mb * len(es) / len(sel)
            line += f" {mb / (np.mean(us) * 1e-6 * clock_ghz * 1e9 * simds):.3f} |"
        print(line)
    if mfma:
        print(f"\nwhole run: MFMA busy {busy_tot / (tot_us * 1e-6 * clock_ghz * 1e9 * simds):.3f} "
              f"of the run's kernel time ({clock_ghz} GHz x {simds} SIMDs)")


def decode8b_bench(a, V, F):
    """Decode at the Llama-8B layer shape (the d_head 128 path): `layers` layers
    (hidden 4096, 32/8 heads, FFN 14336) + a 32000-row LM head, cache filled to
    ctx by the MFMA prefill, then `steps` timed greedy steps; us per layer
    includes the LM head's share."""
    dtype = V.DT_Q8_0 if a.dtype == "q8_0" else V.DT_Q4_0
    ctx = V.Context(0)
    cfg = F.llama8b_layer(dtype, max_seq_len=a.ctx + a.warmup + a.steps + 8, n_layers=a.layers,
                          vocab_size=32000)
    m = V.Model(ctx, cfg)
    F.load_model(m, a.seed)
    prompt = F.tokens(a.seed, "bench8b.prompt", a.ctx, cfg["vocab_size"])
    nxt = m.prefill_mfma(prompt)
    if a.warmup:
        nxt = int(m.generate_ids(nxt, a.warmup)[-1])
    used = m.used
    ctx.sync()
    ctx.timer_start()
    m.generate_async(nxt, a.steps)
    ms = ctx.timer_stop()
    step_bytes = [sum(m.step_bytes(used + i)) for i in range(a.steps)]
    gbs = sum(step_bytes) / (ms / 1e3) / 1e9
    return {
        "metric": "decode us per layer at the Llama-8B shape",
        "value": round(ms / a.steps / a.layers * 1e3, 2),
        "unit": "us/layer",
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms / a.steps, 4),
        "higher_is_better": False,
        "dtype": f"f32 compute, {a.dtype} weights, q8_0 KV",
        "data": "synthetic: seeded N(0,0.02) weights, random token ids",
        "config": {"workload": "llama-8B-shape greedy decode, ctx %d->%d, batch 1" % (used, used + a.steps),
                   "layers": a.layers, "hidden": 4096, "ffn": 14336, "heads": "32/8", "head_dim": 128,
                   "vocab": 32000},
        "step_roofline": {"bytes_per_step": int(np.mean(step_bytes)), "achieved": round(gbs, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)},
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=2048)
    ap.add_argument("--dtype", default="q8_0", choices=["q8_0", "q4_0"])
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-roofline", action="store_true")
    ap.add_argument("--summarize-trace", metavar="CSV",
                    help="print a markdown table of a rocprofv3 kernel trace's last --steps steps")
    ap.add_argument("--launches-per-step", type=int, default=90)
    ap.add_argument("--summarize-runs", metavar="CSV",
                    help="per-kernel table of runs [--skip, --skip + --runs) of a rocprofv3 CSV (prefill runs)")
    ap.add_argument("--skip", type=int, default=0)
    ap.add_argument("--runs", type=int, default=1)
    ap.add_argument("--roofline-only", action="store_true",
                    help="run the copy calibration and the roofline launches only (PMC passes)")
    ap.add_argument("--prefill", action="store_true",
                    help="config 5: one Llama-8B-shape layer prefill on the matrix cores")
    ap.add_argument("--prefill-tokens", type=int, default=2048)
    ap.add_argument("--decode-8b", action="store_true",
                    help="decode at the Llama-8B layer shape (d_head 128), us per layer")
    ap.add_argument("--layers", type=int, default=4, help="--decode-8b: layers of the model")
    ap.add_argument("--configs", action="store_true",
                    help="configs 1-3: kernel-level GB/s of attention and quantized linear")
    a = ap.parse_args()

    if a.summarize_trace:
        summarize_trace(a.summarize_trace, a.steps, a.launches_per_step)
        return
    if a.summarize_runs:
        summarize_runs(a.summarize_runs, a.skip, a.runs)
        return

    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path; "
              "the sharding of the decode step is described, not built.", file=sys.stderr)
        sys.exit(2)

    import vlrf_amd as V
    from vlrf_amd import formats as F

    if a.configs:
        configs_bench(V, F)
        return

    if a.decode_8b:
        if a.steps == 128:           # the 1.1B default; 32 steps of an 8B-shape model suffice
            a.steps = 32
        print(json.dumps(decode8b_bench(a, V, F)), flush=True)
        return

    if a.prefill:
        if a.steps == 128:           # the decode default; a layer prefill is ~ms
            a.steps = 10
        print(json.dumps(prefill_bench(a, V, F)), flush=True)
        return

    dtype = V.DT_Q8_0 if a.dtype == "q8_0" else V.DT_Q4_0
    # Room for the timed steps and, after them, as many steps timed launch by launch.
    cfg = F.llama_1b(max_seq_len=a.ctx + 2 * a.steps, weight_dtype=dtype)
    ctx = V.Context(0)
    log("[bench]", ctx.device_info())
    if a.roofline_only:
        copy_calibration(ctx)
        print(json.dumps({"roofline": gemv_roofline(ctx, V, F, cfg, dtype)}), flush=True)
        return

    t0 = time.time()
    model = V.Model(ctx, cfg)
    f32w = F.load_model(model, a.seed, want_f32=not a.no_cpu_baseline)
    log(f"[bench] weights generated and uploaded in {time.time() - t0:.1f}s")

    prompt = F.tokens(a.seed, "bench.prompt", a.ctx - a.warmup, cfg["vocab_size"])
    model.reset()
    t0 = time.time()
    nxt = model.prefill(prompt)
    ctx.sync()
    log(f"[bench] {prompt.size} prompt tokens through the decode step in {time.time() - t0:.2f}s")
    if a.warmup:
        warm = model.generate_ids(nxt, a.warmup)
        nxt = int(warm[-1])
    assert model.used == a.ctx, model.used

    ctx.sync()
    wall0 = time.perf_counter()
    ctx.timer_start()
    model.generate_async(nxt, a.steps)
    ms = ctx.timer_stop()
    wall = time.perf_counter() - wall0
    ids = model.read_generated(a.steps)
    log(f"[bench] {a.steps} steps: {ms:.3f} ms (events), {wall * 1e3:.3f} ms (wall); "
        f"first ids {ids[:8].tolist()}")

    tok_s = a.steps / (ms / 1e3)
    step_bytes = [sum(model.step_bytes(a.ctx + i)) for i in range(a.steps)]
    step_gbs = sum(step_bytes) / (ms / 1e3) / 1e9

    out = {
        "metric": "decode tok/s at 1.1B-shape ctx 2048",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms / a.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"f32 compute, {a.dtype} weights, q8_0 KV",
        "data": "synthetic: seeded N(0,0.02) weights, random token ids",
        "config": {"workload": "llama-1.1B-shape greedy decode, ctx 2048->%d, batch 1"
                   % (a.ctx + a.steps), "weights": a.dtype, "kv_cache": "q8_0 per token row",
                   "layers": 22, "hidden": 2048, "ffn": 5632, "heads": "32/4", "vocab": 32000},
        "step_roofline": {"bytes_per_step": int(np.mean(step_bytes)), "achieved": round(step_gbs, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
    }
    if not a.no_roofline:
        # The step's kernels timed one by one over the next `steps` steps: the
        # dominant one by time per step is the roofline; gate/up with weights
        # rotating through more than the memory-side cache is reported beside it.
        sk = step_kernels(model, cfg, dtype, a.dtype, int(ids[-1]), a.steps, a.ctx + a.steps)
        out["step_kernels"] = sk
        out["roofline"] = dominant_roofline(sk)
        log(f"[bench] dominant kernel {out['roofline']['kind']}: {out['roofline']['us_per_launch']} us, "
            f"frac {out['roofline']['frac']}")
    del model
    if not a.no_roofline:
        out["roofline_gemv"] = gemv_roofline(ctx, V, F, cfg, dtype)
    if not a.no_cpu_baseline:
        # The GPU line is complete at this point: a failure of the CPU leg is
        # reported in the line instead of discarding the GPU measurement.
        log("[bench] cpu baseline ...")
        try:
            out["cpu_baseline"] = cpu_baseline(cfg, f32w, a.ctx, a.steps)
        except Exception as e:       # noqa: BLE001 - reported, not hidden
            log(f"[bench] cpu baseline failed: {e!r}")
            out["cpu_baseline"] = {"value": None, "error": repr(e)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
