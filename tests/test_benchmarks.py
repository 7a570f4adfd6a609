"""Benchmark harness on CPU with mocks (the reference's tests/test_benchmark.py):
GPU gate, entry points refusing before output, dense attention phases, decode
counts, cache byte accounting, atomic reports, deterministic inputs and report
comparison; plus the float32 reference checker against the golden fixtures."""

import argparse
import importlib
import sys
from contextlib import contextmanager
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from reskv_amd.benchmarks import timing

GOLDEN = Path(__file__).resolve().parent / "golden"


def _gpu(monkeypatch, arch, name="AMD Radeon Graphics"):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "get_device_name", lambda *a: name)
    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda *a: SimpleNamespace(gcnArchName=arch))


@pytest.mark.parametrize("arch", ["gfx950:sramecc+:xnack-", "gfx950"])
def test_benchmark_gpu_accepts_mi355x(monkeypatch, arch):
    _gpu(monkeypatch, arch)
    timing.validate_gpu(argparse.ArgumentParser())


@pytest.mark.parametrize("arch", ["gfx942:sramecc+:xnack-", "gfx90a", "gfx1100", ""])
def test_benchmark_gpu_rejects_other_architectures(monkeypatch, capsys, arch):
    _gpu(monkeypatch, arch)
    with pytest.raises(SystemExit) as error:
        timing.validate_gpu(argparse.ArgumentParser())
    assert error.value.code == 2
    message = capsys.readouterr().err
    assert timing.BENCHMARK_GPU in message and "detected AMD Radeon Graphics" in message


def test_benchmark_gpu_rejects_missing_gpu(monkeypatch, capsys):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda *a: pytest.fail("GPU must not be queried"))
    with pytest.raises(SystemExit) as error:
        timing.validate_gpu(argparse.ArgumentParser())
    assert error.value.code == 2
    assert "no ROCm GPU is available" in capsys.readouterr().err


@pytest.mark.parametrize("module,arguments", [
    ("inference", ["--model", "/missing-model", "--method", "reskv"]),
    ("inference", ["--model", "/missing-model", "--method", "dense"]),
    ("kernels", []),
    ("compare", ["--model", "/missing-model", "--methods", "reskv", "dense"]),
])
def test_benchmark_entry_points_reject_gpu_before_output(tmp_path, monkeypatch, capsys, module, arguments):
    entry = importlib.import_module("reskv_amd.benchmarks." + module)
    target = tmp_path / "results"
    monkeypatch.setattr(sys, "argv", [module, *arguments, "--output", str(target)])
    _gpu(monkeypatch, "gfx942:sramecc+:xnack-", "AMD Instinct MI300X")
    if module == "compare":
        monkeypatch.setattr(entry.subprocess, "run", lambda *a, **kw: pytest.fail("child process launched"))
    with pytest.raises(SystemExit) as error:
        entry.main()
    assert error.value.code == 2
    assert "detected AMD Instinct MI300X" in capsys.readouterr().err
    assert not target.exists()


def _no_gpu_memory_stats(monkeypatch):
    for name in ("synchronize", "reset_peak_memory_stats"):
        monkeypatch.setattr(torch.cuda, name, lambda: None)
    for name in ("max_memory_allocated", "max_memory_reserved"):
        monkeypatch.setattr(torch.cuda, name, lambda: 0)


@pytest.mark.parametrize("new_tokens", [1, 4])
def test_dense_attention_phases_and_decode_count(monkeypatch, new_tokens):
    flash_active = False

    @contextmanager
    def flash_context(backend):
        nonlocal flash_active
        assert backend == timing.SDPBackend.FLASH_ATTENTION
        flash_active = True
        try:
            yield
        finally:
            flash_active = False

    class Model:
        implementation = "sdpa"

        def __init__(self):
            self.calls = []

        def set_attn_implementation(self, implementation):
            self.implementation = implementation

        def __call__(self, ids, **kwargs):
            self.calls.append((ids.shape[-1], self.implementation, flash_active))
            return SimpleNamespace(logits=torch.tensor([[[0.0, 1.0, 0.0]]]), past_key_values=SimpleNamespace(layers=[]))

    monkeypatch.setattr(timing, "sdpa_kernel", flash_context)
    _no_gpu_memory_stats(monkeypatch)
    model = Model()
    for _ in range(2):
        model.calls.clear()
        record = timing.run(model, torch.ones(1, 8, dtype=torch.long), new_tokens, dense=True)
        assert len(model.calls) == new_tokens
        assert model.calls[0] == (8, "sdpa", True)
        assert model.calls[1:] == [(1, "eager", False)] * (new_tokens - 1)
        assert record["finite_last_logits"] and record["decode_steps"] == new_tokens - 1
        assert (record["tpot_ms"] is None) == (new_tokens == 1)


def test_cache_storage_deduplication():
    from dataclasses import dataclass

    @dataclass
    class Payload:
        data: torch.Tensor
        native_view: torch.Tensor

    storage = torch.zeros(64, dtype=torch.float16)
    other = torch.ones(8)
    packed = Payload(storage[:16], storage.view(8, 8))
    layer_cache = SimpleNamespace(layers=[SimpleNamespace(compressed=packed, keys=other, values=other[:2])])
    tuple_cache = (([storage[:2], storage[3:4]], {"values": other}, 8, None),)
    expected = storage.untyped_storage().nbytes() + other.untyped_storage().nbytes()
    assert timing.cache_bytes(layer_cache) == timing.cache_bytes(tuple_cache) == expected


def test_cache_bytes_of_the_resKV_cache_counts_capacity_buffers_once():
    from reskv_amd import ResKVKernelConfig
    from reskv_amd.cache import ResKVCache

    cache = ResKVCache(ResKVKernelConfig(), 2)
    x = torch.zeros(1, 1, 10, 128, dtype=torch.float16)
    for layer in cache.layers:
        layer.update(x, x, {"raw_keys": x})  # ring only: three [1, 1, 96, 128] buffers
    assert timing.cache_bytes(cache) == 2 * 3 * 96 * 128 * 2


def test_nonfinite_report_does_not_replace_existing_results(tmp_path):
    output = tmp_path / "result.json"
    output.write_text('{"complete": true}\n', encoding="utf-8")
    with pytest.raises(ValueError):
        timing.write_report(output, {"throughput_tps": float("nan")})
    assert output.read_text(encoding="utf-8") == '{"complete": true}\n'
    assert sorted(p.name for p in tmp_path.iterdir()) == ["result.json"]


@pytest.mark.parametrize("new_tokens", [1, 4])
def test_tuple_cache_continuation(monkeypatch, new_tokens):
    calls = []
    cache = ((torch.zeros(1), [torch.ones(2)], 7),)

    def model(ids, *, use_cache, past_key_values=None):
        assert use_cache
        if calls:
            assert past_key_values is cache and ids.tolist() == [[2]]
        else:
            assert past_key_values is None and ids.shape[-1] == 8
        calls.append(ids)
        return SimpleNamespace(logits=torch.tensor([[[0.0, 1.0, 2.0]]]), past_key_values=cache)

    _no_gpu_memory_stats(monkeypatch)
    record = timing.run(model, torch.ones(1, 8, dtype=torch.long), new_tokens, logits_to_keep=False)
    assert len(calls) == new_tokens
    assert record["decode_steps"] == new_tokens - 1
    assert record["cache_bytes"] == 12
    assert (record["tpot_ms"] is None) == (new_tokens == 1)


def test_deterministic_inputs():
    first, digest = timing.make_inputs(32000, 2, 64, 42, device="cpu")
    second, same = timing.make_inputs(32000, 2, 64, 42, device="cpu")
    changed, different = timing.make_inputs(32000, 2, 64, 43, device="cpu")
    assert torch.equal(first, second) and digest == same
    assert not torch.equal(first, changed) and digest != different
    tiny, _ = timing.make_inputs(12, 1, 16, 42, device="cpu")
    assert tiny.min() >= 0 and tiny.max() < 12


@pytest.mark.parametrize("field", ["input_ids_sha256", "git_commit", "source_sha256", "model_dtype", "gpu", "torch",
                                   "hip", "decode_steps", "finite_last_logits"])
def test_comparison_rejects_incompatible_measurements(field):
    from copy import deepcopy

    from reskv_amd.benchmarks.compare import validate_reports

    report = {"model": "model", "model_dtype": "fp16", "batch_size": 1, "input_length": 8, "new_tokens": 4,
              "seed": 42, "input_ids_sha256": "abc", "git_commit": "def", "source_sha256": "abc123", "gpu": "gpu",
              "torch": "2.10.0+rocm7.0", "hip": "7.0", "repeats": 1, "warmup": 1,
              "records": [{"decode_steps": 3, "finite_last_logits": True}]}
    other = deepcopy(report)
    validate_reports([report, other])
    if field in other:
        other[field] = "changed"
    else:
        other["records"][0][field] = False if field == "finite_last_logits" else 4
    with pytest.raises(ValueError):
        validate_reports([report, other])


@pytest.mark.parametrize("key", ["bitmap64", "bitmap32", "tiled64", "struct32", "sint4", "q4n64", "q2n64"])
def test_reference_checker_matches_golden_attention(key):
    """The float32 torch checker used by the kernel sweep reproduces the float64 oracle fixtures
    (5e-4: float32 RoPE and sums; a wrong format or index gives errors above 1e-2)."""
    from reskv_amd.config import KernelPlan
    from reskv_amd.reference import reference_attention
    from reskv_amd.tensors import CompressedKV, CompressedTensor

    plans = {"bitmap64": KernelPlan("unstructured", "deferred", 16, 64, 2, 0),
             "bitmap32": KernelPlan("unstructured", "deferred", 16, 32, 2, 0),
             "tiled64": KernelPlan("tiled", "per_token", 16, 64, 4, 0),
             "struct32": KernelPlan("structured", "deferred", 16, 32, 4, 20),
             "sint4": KernelPlan("structured", "deferred", 4, 32, 4, 20),
             "q4n64": KernelPlan("unstructured", "per_token", 4, 64, 16, 0),
             "q2n64": KernelPlan("unstructured", "per_token", 2, 64, 16, 0)}
    with np.load(GOLDEN / "encoders.npz", allow_pickle=False) as f:
        enc = {k: f[k] for k in f.files}
    with np.load(GOLDEN / "decode.npz", allow_pickle=False) as f:
        dec = {k: f[k] for k in f.files}
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731

    def one(side):
        meta, scale = enc.get(f"{side}_{key}_meta"), enc.get(f"{side}_{key}_scale")
        return CompressedTensor(t(enc[side + "c"]), t(enc[side + "i"]), t(enc[f"{side}_{key}_payload"]),
                                None if meta is None else t(meta), None if scale is None else t(scale), plans[key])

    cache = CompressedKV(one("k"), one("v"))
    freq = (500000.0 ** (-torch.arange(64).float() / 64)).float()
    pos, start = int(dec["position"]), int(dec["start"])
    out = reference_attention(t(dec["q"]), cache, position=pos, start_position=start, inv_freq=freq)
    assert np.abs(out.double().numpy() - dec[f"{key}_out"]).max() <= 5e-4
    recent = (t(dec["q_rot"]), t(dec["k_recent"]), t(dec["v_recent"]))
    out = reference_attention(t(dec["q"]), cache, position=pos, start_position=start, inv_freq=freq, recent=recent)
    assert np.abs(out.double().numpy() - dec[f"{key}_out_recent"]).max() <= 5e-4
