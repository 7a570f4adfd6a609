"""The benchmark commands on the CPU, with the GPU and the model mocked: the
gfx950 gate (and that every command applies it before writing anything), the
dense baseline's per-phase attention selection, decode step counts, storage
accounting, atomic reports, deterministic prompts and the comparison's
report validation.  Follows the coverage of the reference's
tests/test_benchmark.py with tests of this harness's own design."""

import argparse
import importlib
import sys
from contextlib import contextmanager
from copy import deepcopy
from types import SimpleNamespace

import pytest
import torch

from reskv_amd.benchmarks import common, compare, timing


def _fake_gpu(monkeypatch, arch, name="AMD Radeon Graphics"):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "get_device_name", lambda *a: name)
    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda *a: SimpleNamespace(gcnArchName=arch))


def _gate_exit(capsys):
    with pytest.raises(SystemExit) as exc:
        common.require_gpu(argparse.ArgumentParser())
    assert exc.value.code == 2
    return capsys.readouterr().err


@pytest.mark.parametrize("arch", ["gfx950", "gfx950:sramecc+:xnack-"])
def test_gate_accepts_gfx950(monkeypatch, arch):
    _fake_gpu(monkeypatch, arch)
    common.require_gpu(argparse.ArgumentParser())


@pytest.mark.parametrize("arch", ["gfx942:sramecc+:xnack-", "gfx90a", "gfx1100", ""])
def test_gate_rejects_other_architectures(monkeypatch, capsys, arch):
    _fake_gpu(monkeypatch, arch)
    err = _gate_exit(capsys)
    assert common.GPU_LABEL in err and "detected AMD Radeon Graphics" in err


def test_gate_without_a_gpu_never_queries_one(monkeypatch, capsys):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    monkeypatch.setattr(torch.cuda, "get_device_properties", lambda *a: pytest.fail("GPU queried"))
    assert "no ROCm GPU is available" in _gate_exit(capsys)


@pytest.mark.parametrize("module,argv", [
    ("inference", ["--model", "/missing-model", "--method", "reskv"]),
    ("inference", ["--model", "/missing-model", "--method", "dense"]),
    ("kernels", []),
    ("compare", ["--model", "/missing-model", "--methods", "reskv", "dense"]),
])
def test_commands_stop_at_the_gate_before_any_output(tmp_path, monkeypatch, capsys, module, argv):
    cmd = importlib.import_module("reskv_amd.benchmarks." + module)
    target = tmp_path / "out"
    monkeypatch.setattr(sys, "argv", [module, *argv, "--output", str(target)])
    _fake_gpu(monkeypatch, "gfx942:sramecc+:xnack-", "AMD Instinct MI300X")
    if module == "compare":
        monkeypatch.setattr(cmd.subprocess, "run", lambda *a, **k: pytest.fail("child process started"))
    with pytest.raises(SystemExit) as exc:
        cmd.main()
    assert exc.value.code == 2 and "detected AMD Instinct MI300X" in capsys.readouterr().err
    assert not target.exists()


def _quiet_allocator(monkeypatch):
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a: None)
    monkeypatch.setattr(torch.cuda, "reset_peak_memory_stats", lambda *a: None)
    monkeypatch.setattr(torch.cuda, "max_memory_allocated", lambda *a: 0)
    monkeypatch.setattr(torch.cuda, "max_memory_reserved", lambda *a: 0)


class _RecordingModel:
    """Logs (input length, attention implementation, flash backend active) per forward."""

    def __init__(self, state):
        self.state, self.impl, self.log = state, "sdpa", []

    def set_attn_implementation(self, impl):
        self.impl = impl

    def __call__(self, ids, **kwargs):
        self.log.append((ids.shape[-1], self.impl, self.state["flash"]))
        return SimpleNamespace(logits=torch.tensor([[[0.0, 3.0, 1.0]]]), past_key_values=SimpleNamespace(layers=[]))


@pytest.mark.parametrize("new_tokens", [1, 5])
def test_dense_run_switches_attention_per_phase(monkeypatch, new_tokens):
    state = {"flash": False}

    @contextmanager
    def fake_sdpa(backend):
        assert backend == timing.SDPBackend.FLASH_ATTENTION
        state["flash"] = True
        yield
        state["flash"] = False

    monkeypatch.setattr(timing, "sdpa_kernel", fake_sdpa)
    _quiet_allocator(monkeypatch)
    model = _RecordingModel(state)
    rec = timing.greedy_run(model, torch.ones(1, 6, dtype=torch.long), new_tokens, dense=True)
    assert model.log == [(6, "sdpa", True)] + [(1, "eager", False)] * (new_tokens - 1)
    assert rec["decode_steps"] == new_tokens - 1 and rec["finite_last_logits"]
    assert (rec["tpot_ms"] is None) == (new_tokens == 1) and rec["throughput_tps"] > 0


@pytest.mark.parametrize("new_tokens", [1, 3])
def test_tuple_cache_is_fed_back_and_counted(monkeypatch, new_tokens):
    cache = ((torch.zeros(2), [torch.ones(3)], 5),)
    seen = []

    def model(ids, *, use_cache, past_key_values=None):
        assert use_cache
        assert (past_key_values is cache) == bool(seen)
        if seen:
            assert ids.tolist() == [[1]]  # the argmax of the logits below
        seen.append(ids.shape[-1])
        return SimpleNamespace(logits=torch.tensor([[[0.0, 2.0, 1.0]]]), past_key_values=cache)

    _quiet_allocator(monkeypatch)
    rec = timing.greedy_run(model, torch.ones(1, 9, dtype=torch.long), new_tokens, logits_to_keep=False)
    assert seen == [9] + [1] * (new_tokens - 1)
    assert rec["cache_bytes"] == 2 * 4 + 3 * 4


def test_storage_is_counted_once_per_backing_buffer():
    from dataclasses import dataclass

    @dataclass
    class Holder:
        a: torch.Tensor
        b: torch.Tensor

    base = torch.zeros(32, dtype=torch.float16)
    other = torch.ones(6)
    layered = SimpleNamespace(layers=[SimpleNamespace(compressed=Holder(base[:4], base.view(4, 8)), keys=other,
                                                      values=other[1:])])
    nested = ({"k": [base[2:], base[:1]], "v": other}, 7, None)
    want = base.untyped_storage().nbytes() + other.untyped_storage().nbytes()
    assert common.storage_bytes(layered) == common.storage_bytes(nested) == want


def test_storage_of_the_device_cache_counts_its_ring_buffers():
    from reskv_amd import ResKVKernelConfig
    from reskv_amd.cache import ResKVCache

    cache = ResKVCache(ResKVKernelConfig(), 2)
    x = torch.zeros(1, 1, 10, 128, dtype=torch.float16)
    for layer in cache.layers:
        layer.update(x, x, {"raw_keys": x})  # ring only: three [1, 1, 96, 128] fp16 buffers per layer
    assert common.storage_bytes(cache) == 2 * 3 * 96 * 128 * 2


def test_a_nonfinite_report_leaves_the_old_one(tmp_path):
    path = tmp_path / "r.json"
    path.write_text("old\n")
    with pytest.raises(ValueError):
        common.save_json(path, {"tpot_ms": float("inf")})
    assert path.read_text() == "old\n" and [p.name for p in tmp_path.iterdir()] == ["r.json"]
    text = common.save_json(path, {"tpot_ms": 1.5})
    assert path.read_text() == text and '"tpot_ms": 1.5' in text


def test_prompts_are_reproducible_and_in_range():
    a, da = common.prompt_ids(32000, 2, 50, 42, device="cpu")
    b, db = common.prompt_ids(32000, 2, 50, 42, device="cpu")
    c, dc = common.prompt_ids(32000, 2, 50, 7, device="cpu")
    assert torch.equal(a, b) and da == db and not torch.equal(a, c) and da != dc
    assert int(a.min()) >= 128
    small, _ = common.prompt_ids(10, 1, 40, 42, device="cpu")
    assert int(small.min()) >= 9 and int(small.max()) < 10


def _report():
    return {"method": "reskv", "model": "m", "model_dtype": "fp16", "batch_size": 1, "input_length": 8,
            "new_tokens": 3, "seed": 42, "input_ids_sha256": "x", "git_commit": "c", "source_sha256": "s",
            "gpu": "g", "torch": "t", "hip": "h", "repeats": 2, "warmup": 0,
            "records": [{"decode_steps": 2, "finite_last_logits": True, "prefill_ms": 1.0, "decode_ms": 2.0,
                         "tpot_ms": 1.0, "throughput_tps": 3.0, "peak_allocated_bytes": 10}] * 2}


@pytest.mark.parametrize("field", list(compare.SHARED_FIELDS) + ["decode_steps", "finite_last_logits", "records"])
def test_comparison_rejects_reports_that_differ(field):
    a, b = _report(), _report()
    compare.validate_reports([a, b])
    if field in compare.SHARED_FIELDS:
        b[field] = "other"
    elif field == "records":
        b["records"] = b["records"][:1]
    else:
        b["records"] = deepcopy(b["records"])
        b["records"][1][field] = False if field == "finite_last_logits" else 5
    with pytest.raises(ValueError):
        compare.validate_reports([a, b])


def test_summary_row_takes_medians():
    rep = _report()
    rep["records"] = [dict(rep["records"][0], decode_ms=x, peak_allocated_bytes=x) for x in (1.0, 5.0, 3.0)]
    row = compare.summary_row(rep, "p.json")
    assert row["decode_ms"] == 3.0 and row["peak_allocated_bytes"] == 5.0 and row["result"] == "p.json"
