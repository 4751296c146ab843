"""bench.py's host-side pieces that run without a GPU: the end-to-end CPU
baseline (the reference's decode-step forward restated in f32 over the
engine's weights, attention through the oracle) on a reduced model."""
import pytest


@pytest.fixture(scope="module")
def bench(pa, oracle):
    import bench as b
    return b


def test_cpu_baseline_e2e_runs_on_host(bench, pa):
    from vllm_lite_amd import e2e

    cfg = e2e.qwen25_05b()
    cfg.layers, cfg.vocab = 2, 2048
    w = e2e.Weights(cfg, seed=4, device="cpu")
    lens = [64, 130, 300, 17] * 2
    out = bench.cpu_baseline_e2e(cfg, w, lens, 32, budget_s=0.2)
    assert out["kind"] == "port" and out["unit"] == "tokens/s"
    assert out["value"] > 0 and out["cores"] >= 1
    assert "decode steps" in out["sample"]

