"""bench.py's host-side logic on the CPU: the CPU-baseline leg must complete
whatever --steps the GPU run was given (the driver runs --steps 20, the
default is 128), with its step count bounded by the CPU model's own cache."""
import importlib.util
import os

import pytest

from vlrf_amd import formats as F

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("use_ref", [False, True])
@pytest.mark.parametrize("gpu_steps", [1, 20, 128])
def test_cpu_baseline_fits_the_oracle_cache(gpu_steps, use_ref):
    """The GPU model is sized ctx + steps (as main() sizes it); the CPU leg
    runs up to max_steps steps after filling ctx - 1 rows and one warm-up
    step, and must not overflow for any gpu_steps, on the C restatement and
    on the reference model (when oracle/_ref was built)."""
    import oracle
    if use_ref and oracle.ref() is None:
        pytest.skip("oracle/_ref/libvlrf_ref.so not built")
    b = _bench()
    ctx_len = 96
    cfg = F.tiny(n_layers=1, max_seq_len=ctx_len + gpu_steps)
    w = F.make_f32_weights(cfg, 3)
    out = b.cpu_baseline(cfg, w, ctx_len, gpu_steps, budget_s=1e9, max_steps=32, threads=2,
                         prefer_ref=use_ref)
    assert out["value"] > 0
    if use_ref:
        assert out["kind"] == "reference" and out["cores"] == oracle.RefModel.threads()
        assert out["port"]["value"] > 0 and out["port"]["cores"] == 2
    else:
        assert out["cores"] == 2 and out["kind"] == "port" and "port" not in out
    assert f"the GPU timed {gpu_steps}" in out["sample"]
    assert f"context {ctx_len}-{ctx_len + 32}" in out["sample"]     # all 32 steps ran


def test_cpu_baseline_plan_leaves_room():
    b = _bench()
    cfg = F.llama_1b(max_seq_len=2048 + 20)
    ocfg = b.cpu_baseline_plan(cfg, 2048, 32)
    assert ocfg["max_seq_len"] >= (2048 - 1) + 1 + 32
    assert cfg["max_seq_len"] == 2068          # the GPU config is not modified
