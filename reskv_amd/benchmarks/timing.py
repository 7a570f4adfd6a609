"""Greedy decoding of a Hugging Face causal LM, timed per phase.

One *run* is a prefill forward over the prompt followed by new_tokens - 1
single-token forwards that feed back the argmax; the phases are timed with a
device synchronisation at each boundary, and the peak allocator statistics
are read per phase.  The dense baseline prefills with SDPA's flash backend and
decodes with eager attention (the reference's methodology,
benchmarks/timing.py:96-145), the ResKV model uses its own attention
throughout.  Record fields are the reference's.
"""

import time
from contextlib import contextmanager, nullcontext

import torch
from torch.nn.attention import SDPBackend, sdpa_kernel

from .common import prompt_ids, provenance, storage_bytes


class _Phase:
    """Wall time (ms, synchronised on both ends) and peak allocator bytes of one phase."""

    def __enter__(self):
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        self._t0 = time.perf_counter()
        return self

    def __exit__(self, *exc):
        torch.cuda.synchronize()
        self.ms = (time.perf_counter() - self._t0) * 1000.0
        self.peak = torch.cuda.max_memory_allocated()
        self.reserved = torch.cuda.max_memory_reserved()
        return False


@contextmanager
def _dense_attention(model, phase):
    """Prefill: SDPA restricted to its flash backend; decode: eager attention."""
    if phase == "prefill":
        model.set_attn_implementation("sdpa")
        with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
            yield
    else:
        model.set_attn_implementation("eager")
        yield


def greedy_run(model, ids, new_tokens, *, dense=False, logits_to_keep=True):
    """One timed run; returns the record of its phases."""
    if new_tokens < 1:
        raise ValueError("new_tokens must be positive")
    extra = {"use_cache": True}
    if logits_to_keep:
        extra["logits_to_keep"] = 1
    mode = (lambda phase: _dense_attention(model, phase)) if dense else (lambda phase: nullcontext())
    with _Phase() as pre, mode("prefill"):
        out = model(ids, **extra)
    if out.logits.shape[-2] != 1:
        raise RuntimeError("benchmark requires final-position logits; check the model compatibility patch")
    steps = new_tokens - 1
    with _Phase() as dec, mode("decode"):
        for _ in range(steps):
            nxt = out.logits[:, -1].argmax(-1, keepdim=True)
            out = model(nxt, past_key_values=out.past_key_values, **extra)
    decode_ms = dec.ms if steps else 0.0
    total_ms = pre.ms + decode_ms
    return {
        "prefill_ms": pre.ms,
        "decode_ms": decode_ms,
        "total_ms": total_ms,
        "tpot_ms": decode_ms / steps if steps else None,
        "throughput_tps": ids.shape[0] * new_tokens / (total_ms / 1000.0),
        "decode_steps": steps,
        "prefill_peak_allocated_bytes": pre.peak,
        "decode_peak_allocated_bytes": dec.peak,
        "peak_allocated_bytes": max(pre.peak, dec.peak),
        "peak_reserved_bytes": max(pre.reserved, dec.reserved),
        "cache_bytes": storage_bytes(out.past_key_values),
        "finite_last_logits": bool(out.logits.isfinite().all()),
    }


def repeated_runs(model, ids, args, **options):
    """``args.warmup`` short runs (at most 8 tokens) on the measured shape, then
    ``args.repeats`` full runs with the allocator cache emptied before each."""
    with torch.inference_mode():
        for _ in range(args.warmup):
            greedy_run(model, ids, min(args.new_tokens, 8), **options)
        records = []
        for _ in range(args.repeats):
            torch.cuda.empty_cache()
            rec = greedy_run(model, ids, args.new_tokens, **options)
            if not rec["finite_last_logits"]:
                raise RuntimeError("nonfinite logits in benchmark")
            records.append(rec)
    return records


def run_header(args, ids_digest, transformers_version):
    """Report fields that identify the inputs and the environment of a run."""
    return {
        **provenance(),
        "model": args.model,
        "batch_size": args.batch_size,
        "input_length": args.input_length,
        "new_tokens": args.new_tokens,
        "decode_steps": args.new_tokens - 1,
        "seed": args.seed,
        "input_ids_sha256": ids_digest,
        "warmup": args.warmup,
        "repeats": args.repeats,
        "transformers": transformers_version,
    }


__all__ = ["greedy_run", "repeated_runs", "run_header", "prompt_ids"]
