"""Compressed K/V cache containers (the ``reskv.tensors`` surface,
reskv/tensors.py:11-162).

A ``CompressedTensor`` is a record of device tensors whose expected dtypes and
widths follow from its ``KernelPlan``: ``_Layout`` derives them once, and
``_violations`` walks an ordered list of rules, raising the first one that
fails (the order and wording are the reference's, which callers match on).
The record also carries ``_native``: the [B*H, ...] views the C ABI receives.
A view into a larger capacity buffer (rows of each (batch, head) block evenly
strided, 16-byte aligned) is passed as is, so the device cache's history is
read in place; anything else is made contiguous.  All arithmetic runs in the
HIP library.
"""

from dataclasses import dataclass, field

import torch

from .config import KernelPlan

_ID_DTYPES = (torch.int8, torch.int16, torch.int32, torch.int64)
_STORED = ("cluster_ids", "payload", "metadata", "scale")  # tensors that grow along T


@dataclass(frozen=True)
class _Layout:
    """What a plan's residual format stores per token."""

    payload_dtype: torch.dtype
    payload_width: int
    meta: tuple | None      # (words, dtype) or None
    scaled: bool

    @staticmethod
    def of(plan: KernelPlan) -> "_Layout":
        spec = plan.metadata_spec
        meta = None if spec is None else (spec[0], getattr(torch, spec[1]))
        dtype = torch.float16 if plan.bits == 16 else torch.int32
        return _Layout(dtype, plan.payload_width, meta, plan.bits != 16)


def _violations(ct: "CompressedTensor"):
    """(failed, message) pairs in the order they are checked."""
    c, ids, p = ct.centroids, ct.cluster_ids, ct.payload
    lay = _Layout.of(ct.plan)
    yield c.ndim != 4 or c.shape[-1] != 128, "centroids must have shape [B,H,C,128]"
    yield ids.ndim != 3 or ids.shape[:2] != c.shape[:2], "cluster IDs must have shape [B,H,T]"
    yield not 1 <= c.shape[2] <= 64, "centroid count must be between 1 and 64"
    yield p.ndim != 4 or p.shape[:3] != ids.shape, "payload must have shape [B,H,T,words_or_values]"
    yield (any(t is not None and t.device != c.device for t in (ids, p, ct.metadata, ct.scale)),
           "all cache tensors must share a device")
    yield c.dtype != torch.float16, "centroids must be FP16"
    yield p.dtype != lay.payload_dtype, "payload dtype does not match the compression plan"
    yield min(ids.shape) < 1, "cache dimensions must be nonempty"
    yield ids.dtype not in _ID_DTYPES, "cluster IDs must be integer tensors"
    yield p.shape[-1] != lay.payload_width, "payload width does not match the compression plan"
    m = ct.metadata
    if lay.meta is None:
        yield m is not None, "quantized unstructured payloads do not use sparse metadata"
    else:
        words, dtype = lay.meta
        yield (m is None or tuple(m.shape) != (*ids.shape, words) or m.dtype != dtype,
               "sparse metadata shape/dtype does not match the compression plan")
    s = ct.scale
    if lay.scaled:
        yield (s is None or tuple(s.shape) != tuple(ids.shape) or s.dtype != torch.float16,
               "quantized scales must be FP16 [B,H,T]")
    else:
        yield s is not None, "FP16 sparse-only caches do not use quantization scales"


def _kernel_view(t: torch.Tensor) -> torch.Tensor:
    """t itself when its token rows are dense and 16-byte aligned, else a contiguous copy."""
    rows_dense = t.stride(-1) == 1 and (t.dim() == 2 or t.shape[-2] == 1 or t.stride(-2) == t.shape[-1])
    aligned = (t.storage_offset() * t.element_size()) % 16 == 0
    return t if rows_dense and aligned else t.contiguous()


@dataclass
class CompressedTensor:
    """Compressed K or V cache of shape [B, H, T, 128] for one layer.

    centroids: FP16 [B, H, C, 128] cluster centres (1 <= C <= 64).
    cluster_ids: per-token centroid index [B, H, T], stored as int8.
    payload: FP16 [B, H, T, nnz] kept residuals (bits 16) or int32 words of
        packed signed codes (bits 4/2).
    metadata: residual positions -- int64 [.., 2] MSB-first bitmaps
        (unstructured FP16), int32 [.., 4] tile codes (tiled / structured
        FP16), int32 [.., 2] 2-bit selections (structured INT4) -- or None
        for unstructured quantized payloads.
    scale: FP16 [B, H, T] per-token quantisation scale, or None for FP16.
    plan: the KernelPlan that produced this tensor.
    """

    centroids: torch.Tensor
    cluster_ids: torch.Tensor
    payload: torch.Tensor
    metadata: torch.Tensor | None
    scale: torch.Tensor | None
    plan: KernelPlan
    _native: tuple = field(default=(), init=False, repr=False)

    def __post_init__(self):
        for failed, message in _violations(self):
            if failed:
                raise ValueError(message)
        if self.cluster_ids.dtype != torch.int8:
            self.cluster_ids = self.cluster_ids.to(torch.int8).contiguous()
        b, h, t = self.cluster_ids.shape
        flat = lambda x, *tail: None if x is None else _kernel_view(x.reshape(b * h, *tail))  # noqa: E731
        self._native = (flat(self.centroids, -1, 128), flat(self.cluster_ids, t), flat(self.payload, t, -1),
                        flat(self.metadata, t, -1), flat(self.scale, t))

    @property
    def seq_len(self) -> int:
        return self.cluster_ids.shape[-1]

    @property
    def tensors(self) -> tuple:
        """All stored tensors, including the flattened views handed to the kernels."""
        return (self.centroids, *(getattr(self, n) for n in _STORED), *self._native)

    @property
    def nbytes(self) -> int:
        return _storage_bytes(self.tensors)

    def _rebuild(self, centroids, fn) -> "CompressedTensor":
        grown = {n: (None if getattr(self, n) is None else fn(n)) for n in _STORED}
        return CompressedTensor(centroids, grown["cluster_ids"], grown["payload"], grown["metadata"],
                                grown["scale"], self.plan)

    def append(self, other: "CompressedTensor") -> "CompressedTensor":
        """This history followed by ``other`` along T, with ``other``'s (newer,
        possibly longer) centroid table (reskv/tensors.py:105-119)."""
        if self.plan != other.plan:
            raise ValueError("cannot concatenate different cache plans")
        return self._rebuild(other.centroids, lambda n: torch.cat((getattr(self, n), getattr(other, n)), dim=2))

    def index_select(self, index: torch.Tensor) -> "CompressedTensor":
        """The batch rows ``index`` (beam reordering)."""
        pick = lambda x: x.index_select(0, index.to(x.device))  # noqa: E731
        return self._rebuild(pick(self.centroids), lambda n: pick(getattr(self, n)))


@dataclass
class CompressedKV:
    key: CompressedTensor
    value: CompressedTensor

    def __post_init__(self):
        if self.key.plan != self.value.plan or self.key.cluster_ids.shape != self.value.cluster_ids.shape:
            raise ValueError("K/V compression plans and token dimensions must agree")
        if self.key.centroids.device != self.value.centroids.device:
            raise ValueError("K/V caches must share a device")

    @property
    def seq_len(self) -> int:
        return self.key.seq_len

    @property
    def nbytes(self) -> int:
        return _storage_bytes((*self.key.tensors, *self.value.tensors))


def _storage_bytes(tensors) -> int:
    """Bytes of the distinct storages behind ``tensors`` (views share one)."""
    storages = {(t.device, t.untyped_storage().data_ptr()): t.untyped_storage().nbytes()
                for t in tensors if isinstance(t, torch.Tensor)}
    return sum(storages.values())
