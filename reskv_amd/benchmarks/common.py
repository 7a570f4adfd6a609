"""Pieces shared by the benchmark commands (``kernels``, ``inference``,
``compare``): the GPU gate, the common argument set, deterministic prompts,
storage accounting, event timing, provenance and atomic JSON reports.

The record fields, command-line flags and input recipe follow the
reference's harness (benchmarks/timing.py, kernels.py, compare.py) so that
reports of the two can be read side by side; the gate accepts the MI355X,
identified by its gfx950 architecture (the marketing name the runtime
reports depends on the installed device-name table).
"""

import hashlib
import json
import os
import subprocess
from datetime import datetime, timezone
from pathlib import Path

import torch

GPU_ARCH = "gfx950"
GPU_LABEL = "AMD Instinct MI355X (gfx950)"
_ROOT = Path(__file__).resolve().parents[2]


# ---------------------------------------------------------------------------
# gate and arguments
# ---------------------------------------------------------------------------

def require_gpu(parser):
    """Exit through ``parser.error`` (status 2) unless the benchmark GPU is present."""
    if not torch.cuda.is_available():
        parser.error(f"performance benchmarks require {GPU_LABEL}; no ROCm GPU is available")
    arch = str(getattr(torch.cuda.get_device_properties(0), "gcnArchName", "")).split(":")[0].strip()
    if arch != GPU_ARCH:
        name = " ".join(torch.cuda.get_device_name().split())
        parser.error(f"performance benchmarks require {GPU_LABEL}; detected {name} ({arch or 'unknown arch'})")


# (flag, argparse options) of the run description shared by inference and compare
_RUN_FLAGS = (
    ("--model", {"required": True}),
    ("--input-length", {"type": int, "default": 8192}),
    ("--new-tokens", {"type": int, "default": 2048}),
    ("--seed", {"type": int, "default": 42}),
    ("--warmup", {"type": int, "default": 1}),
    ("--repeats", {"type": int, "default": 3}),
)
_METHOD_FLAGS = (
    ("--sparsity", {"type": float, "choices": [0.5, 0.75], "default": 0.75, "help": "Fraction of residuals discarded"}),
    ("--dtype", {"choices": ["fp16", "bf16"], "default": "fp16"}),
    ("--reskv-implementation", {"choices": ["default", "unstructure"], "default": "default",
                                "help": "ResKV implementation; default selects automatically for the sparsity "
                                        "and batch size"}),
)


def declare_run(parser, *, many_batches=False):
    """Add the run description (model, batch size(s), lengths, seed, warmup, repeats) and the method flags."""
    for flag, options in _RUN_FLAGS:
        parser.add_argument(flag, **options)
    if many_batches:
        parser.add_argument("--batch-sizes", type=int, nargs="+", default=[1, 4, 8, 16, 32])
    else:
        parser.add_argument("--batch-size", type=int, default=1)
    for flag, options in _METHOD_FLAGS:
        parser.add_argument(flag, **options)


def check_run(parser, args):
    batches = getattr(args, "batch_sizes", None) or [args.batch_size]
    if min(*batches, args.input_length, args.new_tokens, args.repeats) < 1 or args.warmup < 0:
        parser.error("batch size, lengths and repeats must be positive; warmup must be nonnegative")


def kernel_config_for(args):
    """The ResKV configuration a run's flags select."""
    from .. import ResKVKernelConfig

    layout = "unstructured" if args.reskv_implementation == "unstructure" else "auto"
    return ResKVKernelConfig(sparsity=args.sparsity, layout=layout)


# ---------------------------------------------------------------------------
# inputs, storage, timing
# ---------------------------------------------------------------------------

def prompt_ids(vocab_size, batch_size, length, seed, device="cuda"):
    """Token ids drawn on the CPU from a seeded generator -- identical on every
    machine and interpreter -- in [min(128, vocab - 1), vocab), and their sha256."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    ids = torch.randint(min(128, vocab_size - 1), vocab_size, (batch_size, length), generator=gen)
    return ids.to(device), hashlib.sha256(ids.numpy().tobytes()).hexdigest()


_CACHE_ATTRS = ("keys", "values", "raw_keys", "compressed")


def storage_bytes(obj) -> int:
    """Bytes of the distinct storages reachable from ``obj``: tensors inside
    dicts, sequences, dataclasses, objects with ``layers`` (cache containers)
    or with the layer-cache attributes; views of one storage count once."""
    seen = {}
    stack = [obj]
    while stack:
        item = stack.pop()
        if item is None:
            continue
        if isinstance(item, torch.Tensor):
            st = item.untyped_storage()
            seen[(item.device, st.data_ptr())] = st.nbytes()
        elif isinstance(item, dict):
            stack.extend(item.values())
        elif isinstance(item, (list, tuple)):
            stack.extend(item)
        elif hasattr(item, "__dataclass_fields__") and not isinstance(item, type):
            stack.extend(getattr(item, name) for name in item.__dataclass_fields__)
        elif hasattr(item, "layers"):
            stack.append(item.layers)
        else:
            stack.extend(getattr(item, name, None) for name in _CACHE_ATTRS)
    return sum(seen.values())


def median_event_ms(fn, *, warmup=5, repeats=50, windows=5):
    """Median over ``windows`` event-timed windows of ``repeats`` calls, in ms per call."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    per_call = []
    for _ in range(windows):
        begin, finish = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record()
        for _ in range(repeats):
            fn()
        finish.record()
        finish.synchronize()
        per_call.append(begin.elapsed_time(finish) / repeats)
    return sorted(per_call)[len(per_call) // 2]


# ---------------------------------------------------------------------------
# provenance and reports
# ---------------------------------------------------------------------------

def _git(*args):
    return subprocess.run(["git", "-C", str(_ROOT), *args], capture_output=True, text=True, check=True).stdout.strip()


def git_commit():
    """HEAD of this checkout, ``-dirty`` when tracked files differ; None outside git."""
    try:
        head, changes = _git("rev-parse", "HEAD"), _git("status", "--porcelain", "--untracked-files=no")
    except (OSError, subprocess.CalledProcessError):
        return None
    return f"{head}-dirty" if changes else head


def source_sha256():
    """Digest over the runtime sources (Python, HIP, the C header), edits included."""
    digest = hashlib.sha256()
    files = [p for base in ("reskv_amd", "include") for p in (_ROOT / base).rglob("*")
             if p.is_file() and p.suffix in (".py", ".hip", ".h", ".json")]
    for path in sorted(files):
        digest.update(path.relative_to(_ROOT).as_posix().encode() + b"\0" + path.read_bytes())
    return digest.hexdigest()


def provenance():
    props = torch.cuda.get_device_properties(0)
    return {"timestamp": datetime.now(timezone.utc).isoformat(), "gpu": torch.cuda.get_device_name(),
            "gpu_arch": str(getattr(props, "gcnArchName", "")), "torch": torch.__version__,
            "hip": torch.version.hip, "git_commit": git_commit(), "source_sha256": source_sha256()}


def save_json(path, value):
    """Write ``value`` as JSON to ``path`` atomically and return the text.  Nonfinite
    numbers fail before any file is touched, so an earlier report survives."""
    text = json.dumps(value, indent=2, allow_nan=False) + "\n"
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    partial = path.with_name(f".{path.name}.{os.getpid()}.partial")
    try:
        partial.write_text(text, encoding="utf-8")
        os.replace(partial, path)
    finally:
        partial.unlink(missing_ok=True)
    return text
