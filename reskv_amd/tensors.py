"""Compressed K/V cache containers.

Interface mirror of ``reskv/tensors.py:11-162``: the same fields, shape/dtype
contract per layout, int8 cluster ids and the flattened ``_native`` views that
the decode kernels receive.  The containers only hold device tensors; all
arithmetic happens in the HIP library.
"""

from dataclasses import dataclass, field

import torch

from .config import KernelPlan

_ID_DTYPES = (torch.int8, torch.int16, torch.int32, torch.int64)


def _rows(t: torch.Tensor) -> torch.Tensor:
    """t when its innermost dimensions are dense (a [BH, T(, W)] block view), else a contiguous copy."""
    inner_dense = t.stride(-1) == 1 and (t.dim() == 2 or t.stride(-2) == t.shape[-1] or t.shape[-2] == 1)
    aligned = (t.storage_offset() * t.element_size()) % 16 == 0
    return t if inner_dense and aligned else t.contiguous()


def _check_metadata(plan: KernelPlan, metadata, shape3):
    spec = plan.metadata_spec
    if spec is None:
        if metadata is not None:
            raise ValueError("quantized unstructured payloads do not use sparse metadata")
        return
    words, dtype_name = spec
    dtype = getattr(torch, dtype_name)
    if metadata is None or tuple(metadata.shape) != (*shape3, words) or metadata.dtype != dtype:
        raise ValueError("sparse metadata shape/dtype does not match the compression plan")


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
        c, ids, p = self.centroids, self.cluster_ids, self.payload
        if c.ndim != 4 or c.shape[-1] != 128:
            raise ValueError("centroids must have shape [B,H,C,128]")
        if ids.ndim != 3 or ids.shape[:2] != c.shape[:2]:
            raise ValueError("cluster IDs must have shape [B,H,T]")
        if not 1 <= c.shape[2] <= 64:
            raise ValueError("centroid count must be between 1 and 64")
        if p.ndim != 4 or p.shape[:3] != ids.shape:
            raise ValueError("payload must have shape [B,H,T,words_or_values]")
        members = (c, ids, p, self.metadata, self.scale)
        if any(t is not None and t.device != c.device for t in members):
            raise ValueError("all cache tensors must share a device")
        if c.dtype != torch.float16:
            raise ValueError("centroids must be FP16")
        want = torch.float16 if self.plan.bits == 16 else torch.int32
        if p.dtype != want:
            raise ValueError("payload dtype does not match the compression plan")
        b, h, t = ids.shape
        if min(b, h, t) < 1:
            raise ValueError("cache dimensions must be nonempty")
        if ids.dtype not in _ID_DTYPES:
            raise ValueError("cluster IDs must be integer tensors")
        if p.shape[-1] != self.plan.payload_width:
            raise ValueError("payload width does not match the compression plan")
        _check_metadata(self.plan, self.metadata, (b, h, t))
        if self.plan.bits != 16:
            s = self.scale
            if s is None or tuple(s.shape) != (b, h, t) or s.dtype != torch.float16:
                raise ValueError("quantized scales must be FP16 [B,H,T]")
        elif self.scale is not None:
            raise ValueError("FP16 sparse-only caches do not use quantization scales")
        # int8 ids; tensors that are views into larger capacity buffers (rows of
        # each (batch, head) block evenly strided) stay views: the kernels read
        # them in place, and [B, H] merge into one dimension without a copy.
        self.cluster_ids = ids if ids.dtype == torch.int8 else ids.to(torch.int8).contiguous()
        bh = b * h
        self._native = (
            _rows(c.reshape(bh, -1, 128)),
            _rows(self.cluster_ids.reshape(bh, t)),
            _rows(p.reshape(bh, t, -1)),
            None if self.metadata is None else _rows(self.metadata.reshape(bh, t, -1)),
            None if self.scale is None else _rows(self.scale.reshape(bh, t)),
        )

    @property
    def seq_len(self) -> int:
        return self.cluster_ids.shape[-1]

    @property
    def tensors(self) -> tuple:
        """All stored tensors, including the flattened views handed to the kernels."""
        return (self.centroids, self.cluster_ids, self.payload, self.metadata, self.scale, *self._native)

    @property
    def nbytes(self) -> int:
        return _storage_bytes(self.tensors)

    def append(self, other: "CompressedTensor") -> "CompressedTensor":
        """Concatenate along T, taking the newer centroid table (reskv/tensors.py:105-119)."""
        if self.plan != other.plan:
            raise ValueError("cannot concatenate different cache plans")

        def cat(a, b):
            return None if a is None else torch.cat((a, b), dim=2)

        return CompressedTensor(
            other.centroids,
            cat(self.cluster_ids, other.cluster_ids),
            cat(self.payload, other.payload),
            cat(self.metadata, other.metadata),
            cat(self.scale, other.scale),
            self.plan,
        )

    def index_select(self, index: torch.Tensor) -> "CompressedTensor":
        def take(t):
            return None if t is None else t.index_select(0, index.to(t.device))

        return CompressedTensor(
            take(self.centroids),
            take(self.cluster_ids),
            take(self.payload),
            take(self.metadata),
            take(self.scale),
            self.plan,
        )


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
    """Bytes in unique backing storages; views of one storage count once."""
    seen = {}
    for t in tensors:
        if isinstance(t, torch.Tensor):
            storage = t.untyped_storage()
            seen[(t.device, storage.data_ptr())] = storage.nbytes()
    return sum(seen.values())
