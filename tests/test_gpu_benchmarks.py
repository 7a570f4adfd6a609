"""Benchmark harness on MI355X: the kernel sweep (accuracy-checked cases), and
the inference and comparison commands on a small random-init checkpoint saved
to a temporary directory."""

import json
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_kernel_sweep_writes_checked_records(device, tmp_path, monkeypatch):
    from reskv_amd.benchmarks import kernels

    out = tmp_path / "kernels.json"
    monkeypatch.setattr(sys, "argv", ["kernels", "--batch-sizes", "1", "2", "--seq-len", "256", "--output", str(out)])
    kernels.main()
    report = json.loads(out.read_text())
    assert report["gpu_arch"].startswith("gfx950") and len(report["records"]) == 4
    for record in report["records"]:
        assert record["split_invariance_max_abs"] <= 2e-3
        assert record["decode_ms"] > 0 and record["compression_ms"] > 0 and record["cache_bytes"] > 0


def test_kernel_sweep_releases_previous_case(device, tmp_path, monkeypatch):
    """Each case's inputs and compressed payloads are released before the next
    case allocates its own (reskv tests/test_benchmark.py:17-45)."""
    import weakref

    from reskv_amd.benchmarks import kernels

    tracked = []
    original_inputs, original_compress = kernels._inputs, kernels.compress

    def inputs(*args, **kwargs):
        assert all(ref() is None for ref in tracked)
        return original_inputs(*args, **kwargs)

    def compress(*args, **kwargs):
        cache = original_compress(*args, **kwargs)
        tracked.extend(weakref.ref(x) for x in (*args[:2], cache.key.payload, cache.value.payload))
        return cache

    monkeypatch.setattr(kernels, "_inputs", inputs)
    monkeypatch.setattr(kernels, "compress", compress)
    monkeypatch.setattr(kernels, "median_event_ms", lambda fn: 0.0)
    monkeypatch.setattr(sys, "argv", ["kernels", "--batch-sizes", "1", "2", "--seq-len", "128", "--output",
                                      str(tmp_path / "kernels.json")])
    kernels.main()
    assert tracked and all(ref() is None for ref in tracked)


def test_kernel_sweep_against_the_fp32_checker(device):
    """The sweep's own inputs and caches, checked by the float32 port of the oracle."""
    from oracle import torch_checker
    from reskv_amd.benchmarks import kernels

    for rec in kernels.sweep([1, 2], 512, [0.5, 0.75], checker=torch_checker.attention):
        assert rec["max_abs_error"] <= 2e-3, rec


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory):
    from transformers import LlamaConfig, LlamaForCausalLM

    path = tmp_path_factory.mktemp("tiny-llama")
    torch.manual_seed(0)
    cfg = LlamaConfig(vocab_size=1000, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=1, max_position_embeddings=4096)
    LlamaForCausalLM(cfg).half().save_pretrained(path)
    return path


@pytest.mark.parametrize("method", ["reskv", "dense"])
def test_inference_report(device, checkpoint, tmp_path, monkeypatch, method):
    from reskv_amd.benchmarks import inference

    out = tmp_path / f"{method}.json"
    monkeypatch.setattr(sys, "argv", ["inference", "--model", str(checkpoint), "--method", method, "--input-length",
                                      "200", "--new-tokens", "12", "--warmup", "1", "--repeats", "2", "--output",
                                      str(out)])
    inference.main()
    report = json.loads(out.read_text())
    assert report["method"] == method and len(report["records"]) == 2
    for record in report["records"]:
        assert record["decode_steps"] == 11 and record["finite_last_logits"] and record["tpot_ms"] > 0
    if method == "reskv":
        assert report["kernel_plan"]["layout"] == "structured"


def test_compare_runs_both_methods(device, checkpoint, tmp_path, monkeypatch):
    from reskv_amd.benchmarks import compare

    monkeypatch.setattr(sys, "argv", ["compare", "--model", str(checkpoint), "--batch-sizes", "1", "--input-length",
                                      "200", "--new-tokens", "8", "--warmup", "0", "--repeats", "1", "--output",
                                      str(tmp_path)])
    compare.main()
    summary = json.loads((tmp_path / "summary.json").read_text())
    assert not summary["errors"] and sorted(r["method"] for r in summary["runs"]) == ["dense", "reskv"]
