"""Report files and provenance for the benchmark harness (reskv/_io.py:40-84)."""

import hashlib
import json
import subprocess
import tempfile
from pathlib import Path

_ROOT = Path(__file__).resolve().parents[1]


def write_json(path, value):
    """Replace a complete JSON report atomically; nonfinite numbers are rejected
    before anything is written, so an existing report survives a bad run."""
    text = json.dumps(value, indent=2, allow_nan=False)
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    temporary = None
    try:
        with tempfile.NamedTemporaryFile(mode="w", encoding="utf-8", dir=path.parent, delete=False) as stream:
            temporary = Path(stream.name)
            stream.write(text + "\n")
        temporary.replace(path)
        temporary = None
    finally:
        if temporary is not None:
            temporary.unlink(missing_ok=True)
    return path


def git_commit():
    """HEAD of this checkout, with ``-dirty`` for uncommitted tracked changes; None outside git."""
    try:
        head = subprocess.run(["git", "-C", str(_ROOT), "rev-parse", "HEAD"], capture_output=True, text=True,
                              check=True).stdout.strip()
        dirty = subprocess.run(["git", "-C", str(_ROOT), "status", "--porcelain", "--untracked-files=no"],
                               capture_output=True, text=True, check=True).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        return None
    return head + ("-dirty" if dirty else "")


def source_sha256():
    """Digest of the runtime sources (Python, HIP and the C header), uncommitted edits included."""
    digest = hashlib.sha256()
    for base in (_ROOT / "reskv_amd", _ROOT / "include"):
        for path in sorted(base.rglob("*")):
            if path.is_file() and path.suffix in (".py", ".hip", ".h", ".json"):
                digest.update(path.relative_to(_ROOT).as_posix().encode() + b"\0")
                digest.update(path.read_bytes())
    return digest.hexdigest()
