"""Kernel configuration and resolved launch plans.

Interface mirror of ``reskv/config.py:57-248`` (``ResKVKernelConfig``,
``KernelPlan``, ``resolve``).  The field names, validation messages and the
plan-selection table are kept identical because callers (compression, the
decode dispatcher, saved checkpoints, benchmark records) depend on them; the
code itself is written for this package.  Importing this module does not
import torch.
"""

from dataclasses import asdict, dataclass, fields
from typing import Literal

# Accepted values, one place each (reskv/config.py:136-157).
_SPARSITIES = (0.5, 0.75)
_BITS = (2, 4, 16)
_LAYOUTS = ("auto", "unstructured", "tiled", "structured")
_FUSIONS = ("auto", "per_token", "deferred")
_TOKENS_PER_WARP = (2, 4, 8, 12, 16)


def _is_int(value) -> bool:
    return type(value) is int


@dataclass(frozen=True)
class ResKVKernelConfig:
    """Compression and fused-decode settings (reskv/config.py:96-130).

    sparsity: fraction of residual channels discarded per token (0.5 or 0.75).
    bits: residual width; 16 keeps sparse FP16 residuals, 4/2 quantize them.
    layout: residual mask layout (``unstructured`` top-|r|, ``structured``
        4 of every 16, ``tiled`` fixed 16-dim tiles at 50%, or ``auto``).
    centroid_fusion: ``per_token`` or ``deferred`` Value-centroid handling
        (``auto`` follows ``resolve``).
    num_clusters / max_clusters: K-means centroids at prefill / the cap
        reached by appending one centroid per compressed decode group.
    group_size: tokens compressed together during decode.
    recent_size: most recent tokens kept dense.
    kmeans_iterations: Lloyd iterations at prefill.
    rope_mode: ``model`` frequencies or ``theta``-derived ones.
    softmax_mode: ``online`` or ``fixed_shift`` (structured INT4 only).
    """

    sparsity: float = 0.5
    bits: Literal[2, 4, 16] = 16
    layout: Literal["auto", "unstructured", "tiled", "structured"] = "auto"
    centroid_fusion: Literal["auto", "per_token", "deferred"] = "auto"
    num_clusters: int = 32
    max_clusters: int = 64
    group_size: int = 64
    recent_size: int = 32
    kmeans_iterations: int = 10
    rope_mode: Literal["model", "theta"] = "model"
    softmax_mode: Literal["online", "fixed_shift"] = "online"

    def __post_init__(self):
        counts = ("num_clusters", "max_clusters", "group_size", "recent_size", "kmeans_iterations")
        for name in counts:
            if not _is_int(getattr(self, name)):
                raise ValueError(f"{name} must be an integer")
        if self.sparsity not in _SPARSITIES:
            raise ValueError("sparsity must be 0.5 or 0.75 (discarded fraction)")
        if not _is_int(self.bits) or self.bits not in _BITS:
            raise ValueError("bits must be 2, 4, or 16 (FP16 sparse-only)")
        if self.layout not in _LAYOUTS:
            raise ValueError("unknown sparsity layout")
        if self.centroid_fusion not in _FUSIONS:
            raise ValueError("centroid_fusion must be auto, per_token or deferred")
        if not 1 <= self.num_clusters <= self.max_clusters <= 64:
            raise ValueError("require 1 <= num_clusters <= max_clusters <= 64")
        if self.group_size <= 0 or self.recent_size < 0 or self.kmeans_iterations <= 0:
            raise ValueError("group_size/iterations must be positive; recent_size nonnegative")
        if self.rope_mode not in ("model", "theta"):
            raise ValueError("rope_mode must be 'model' or 'theta'")
        if self.softmax_mode not in ("online", "fixed_shift"):
            raise ValueError("softmax_mode must be 'online' or 'fixed_shift'")
        int4_75 = self.bits == 4 and self.sparsity == 0.75
        if self.softmax_mode == "fixed_shift" and not int4_75:
            raise ValueError("fixed_shift softmax requires sparse75 INT4")
        if self.layout == "structured" and (self.sparsity != 0.75 or self.bits == 2):
            raise ValueError("structured layout requires sparsity=0.75 and bits=4 or 16")
        if self.layout == "tiled" and (self.bits != 16 or self.sparsity != 0.5):
            raise ValueError("tiled masks support only FP16 residuals at sparsity 0.5")

    @property
    def keep_ratio(self) -> float:
        return 1.0 - self.sparsity

    @property
    def nnz(self) -> int:
        """Retained residual channels per 128-dim head vector."""
        return int(128 * self.keep_ratio)

    def to_dict(self) -> dict:
        return asdict(self)

    def _auto_layout(self) -> str:
        if self.layout != "auto":
            return self.layout
        return "structured" if (self.sparsity == 0.75 and self.bits != 2) else "unstructured"

    def _auto_fusion(self, layout: str, batch_size: int) -> str:
        if self.centroid_fusion != "auto":
            return self.centroid_fusion
        quantized_unstructured = self.bits != 16 and layout == "unstructured"
        if layout == "tiled" or quantized_unstructured:
            return "per_token"
        if layout == "structured" and batch_size <= 2:
            return "per_token"
        return "deferred"

    def _schedule(self, layout: str, fusion: str, batch_size: int):
        """(tokens_per_warp, splits) exactly as reskv/config.py:192-208."""
        if layout == "structured":
            if self.bits == 4 and fusion == "per_token" and batch_size >= 8:
                return 4, 16
            if self.bits == 4 and fusion == "deferred":
                if batch_size >= 32:
                    return 4, 10
                if batch_size >= 8:
                    return 8, 14
                return 4, 20
            return 4, 20
        base_tpw = 4 if fusion == "per_token" else 2
        if self.bits == 16:
            return base_tpw, 0
        if batch_size <= 2:
            return 16, 40
        if batch_size <= 4:
            return 8, 20
        return (12 if batch_size == 8 else 16), 0

    def resolve(self, batch_size: int) -> "KernelPlan":
        """Select layout, centroid fusion and launch schedule for a batch size."""
        if not _is_int(batch_size) or batch_size < 1:
            raise ValueError("batch_size must be a positive integer")
        layout = self._auto_layout()
        fusion = self._auto_fusion(layout, batch_size)
        if layout == "tiled" and fusion != "per_token":
            raise ValueError("tiled masks require per_token centroid fusion")
        if layout == "unstructured" and self.bits == 16 and fusion != "deferred":
            raise ValueError("unstructured FP16 requires deferred centroid fusion")
        if layout == "unstructured" and self.bits != 16 and fusion != "per_token":
            raise ValueError("unstructured quantized caches require per_token centroid fusion")
        fixed = self.softmax_mode == "fixed_shift"
        if fixed and (layout != "structured" or fusion != "deferred"):
            raise ValueError("fixed_shift requires structured layout with deferred centroid fusion")
        tpw, splits = self._schedule(layout, fusion, batch_size)
        return KernelPlan(layout, fusion, self.bits, self.nnz, tpw, splits, fixed)


def _model_settings(model_config, settings, config_type, key):
    """Explicit settings, or the ones stored at ``model_config.<key>``; stored back.

    Mirrors reskv/config.py:220-234 (checkpoint round trip of the settings).
    """
    if settings is not None and not isinstance(settings, config_type):
        raise TypeError(f"expected {config_type.__name__}, got {type(settings).__name__}")
    if settings is None:
        stored = getattr(model_config, key, None)
        if stored is None:
            stored = {}
        known = {f.name for f in fields(config_type)}
        if not isinstance(stored, dict) or set(stored) - known:
            raise ValueError(
                f"checkpoint compression settings do not match {config_type.__name__}; "
                "pass an explicit configuration"
            )
        settings = config_type(**stored)
    setattr(model_config, key, settings.to_dict())
    return settings


@dataclass(frozen=True)
class KernelPlan:
    """Resolved implementation for one batch size (reskv/config.py:237-287).

    layout / centroid_fusion / bits / nnz describe the stored format;
    tokens_per_warp and splits are schedule hints (splits 0 lets the
    kernel choose); fixed_shift selects the structured-INT4 softmax variant.
    """

    layout: str
    centroid_fusion: str
    bits: int
    nnz: int
    tokens_per_warp: int
    splits: int
    fixed_shift: bool = False

    def __post_init__(self):
        for name in ("bits", "nnz", "tokens_per_warp", "splits"):
            if not _is_int(getattr(self, name)):
                raise ValueError(f"{name} must be an integer")
        if type(self.fixed_shift) is not bool:
            raise ValueError("fixed_shift must be a boolean")
        if self.layout not in ("unstructured", "tiled", "structured") or self.bits not in _BITS:
            raise ValueError("invalid resolved layout or bit width")
        if self.centroid_fusion not in ("per_token", "deferred") or self.nnz not in (32, 64):
            raise ValueError("invalid resolved centroid fusion or retained dimension count")
        if self.tokens_per_warp not in _TOKENS_PER_WARP or self.splits < 0:
            raise ValueError("invalid warp or split schedule")
        if self.layout == "structured" and (self.nnz != 32 or self.bits == 2):
            raise ValueError("invalid indexed residual configuration")
        if self.layout == "tiled" and (
            self.bits != 16 or self.nnz != 64 or self.centroid_fusion != "per_token"
        ):
            raise ValueError("invalid tiled residual configuration")
        if self.layout == "unstructured":
            wanted = "deferred" if self.bits == 16 else "per_token"
            if self.centroid_fusion != wanted:
                raise ValueError("invalid residual bit width and centroid fusion")
        if self.fixed_shift and not (
            self.layout == "structured" and self.bits == 4 and self.centroid_fusion == "deferred"
        ):
            raise ValueError("fixed shift requires indexed INT4 deferred fusion")

    @property
    def payload_width(self) -> int:
        """Last-dim width of the payload tensor (reskv/tensors.py:71-78)."""
        if self.bits == 16:
            return self.nnz
        return 4 if self.layout == "structured" else 4 * self.bits

    @property
    def metadata_spec(self):
        """(words, dtype name) of per-token metadata, or None (reskv/tensors.py:79-88)."""
        if self.bits == 16 or self.layout == "structured":
            words = 2 if (self.layout == "unstructured" or self.bits == 4) else 4
            return words, ("int64" if self.layout == "unstructured" else "int32")
        return None

    def to_dict(self) -> dict:
        return asdict(self)
