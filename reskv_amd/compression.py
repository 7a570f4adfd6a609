"""Clustering and residual compression through one K/V API.

Mirror of ``reskv/compression.py:12-170``: ``cluster``, ``_incremental_cluster``,
``_encode`` and ``compress`` keep their names, arguments, validation messages
and results.  The arithmetic runs in the gfx950 library: Lloyd iterations in
``reskv_kmeans`` (``reskv_kmeans_kv`` for a layer's K and V together), assignment of decode groups in ``reskv_kmeans_assign`` and
all four residual encoders (including the unstructured FP16 bitmap encoder
that the reference runs as a chain of PyTorch ops).
"""

import torch

from ._extension import load_extension
from .config import KernelPlan, ResKVKernelConfig
from .tensors import CompressedKV, CompressedTensor


def _validate(x: torch.Tensor):
    if x.ndim != 4 or x.shape[-1] != 128 or not x.is_cuda or x.dtype != torch.float16:
        raise ValueError("expected FP16 CUDA tensor [batch, kv_heads, tokens, 128]")
    if min(x.shape[:3]) < 1:
        raise ValueError("batch, head and token dimensions must be nonempty")


def _initial_centers(data: torch.Tensor, count: int) -> torch.Tensor:
    """Initial centres [BH, C, 128] fp32 (reskv/compression.py:28-36).

    T >= C: the tokens at ``linspace(0, T-1, C).long()``; T < C: every token plus
    C - T jittered copies of random tokens (not deterministic, as in the reference).
    """
    t = data.shape[1]
    if t < count:
        idx = torch.randint(t, (count - t,), device=data.device)
        extra = data[:, idx] + torch.randn_like(data[:, idx]) * 0.01
        return torch.cat((data.clone(), extra), dim=1).float().contiguous()
    idx = torch.linspace(0, t - 1, count, device=data.device).long()
    return data[:, idx].float().contiguous()


def cluster(x: torch.Tensor, count: int = 32, iterations: int = 10, *, value: bool = False):
    """Lloyd clustering of K (fp32 centres, empty clusters kept) or V (fp16 centres, empty -> 0).

    Returns (centres fp16 [B, H, C, 128], ids int32 [B, H, T]); the ids are the
    last assignment, made against the centres before the final update.
    """
    b, h, t, d = x.shape
    count = min(count, t) if value else count
    data = x.reshape(b * h, t, d).contiguous()
    init = _initial_centers(data, count)
    if value:
        init = init.half().float()  # V centres live in fp16 (reskv/compression.py:27)
    ext = load_extension("compression", device_index=x.device.index or 0)
    centers, ids = ext.kmeans(data.half().contiguous(), init, iterations, value)
    return centers.reshape(b, h, count, d), ids.reshape(b, h, t)


def cluster_kv(key: torch.Tensor, value: torch.Tensor, count: int = 32, iterations: int = 10):
    """``cluster(key, ...)`` and ``cluster(value, ..., value=True)`` as one launch sequence.

    Returns ((k_centres, k_ids), (v_centres, v_ids)), equal to the two separate
    calls (reskv/compression.py:164-165).  Below ``count`` tokens V caps its
    centroid count at T, so the two runs have different sizes and run apart.
    """
    b, h, t, d = key.shape
    if t < count:
        return cluster(key, count, iterations), cluster(value, count, iterations, value=True)
    kd = key.reshape(b * h, t, d).contiguous()
    vd = value.reshape(b * h, t, d).contiguous()
    ik = _initial_centers(kd, count)
    iv = _initial_centers(vd, count).half().float()  # V centres live in fp16
    ext = load_extension("compression", device_index=key.device.index or 0)
    (kc, ki), (vc, vi) = ext.kmeans_kv(kd, vd, ik, iv, iterations)
    return ((kc.reshape(b, h, count, d), ki.reshape(b, h, t)), (vc.reshape(b, h, count, d), vi.reshape(b, h, t)))


def _incremental_cluster(x, centers, config, *, value=False):
    """Append the group mean while under the centroid cap, then assign (reskv/compression.py:56-69)."""
    b, h, t, d = x.shape
    if centers.shape[2] < config.max_clusters:
        centers = torch.cat((centers, x.mean(2, keepdim=True)), dim=2)
    ext = load_extension("compression", device_index=x.device.index or 0)
    ids = ext.kmeans_assign(x.reshape(b * h, t, d).contiguous(), centers.reshape(b * h, -1, d).float().contiguous(),
                            value)
    return centers, ids.reshape(b, h, t)


def _encode(x, centers, ids, plan, *, value=False):
    """Residual encoding of one tensor with the plan's format (reskv/compression.py:72-101)."""
    ids = ids.int().contiguous()
    centers = centers.half().contiguous()
    x = x.contiguous()
    ext = load_extension("compression", device_index=x.device.index or 0)
    if plan.bits == 16 and plan.layout == "unstructured":
        payload, metadata = ext.compress_bitmap(x, centers, ids, plan.nnz)
        scale = None
    elif plan.bits == 16:
        payload, metadata = ext.compress_fp16(x, centers, ids, plan.nnz, plan.layout == "structured")
        scale = None
    elif plan.layout == "structured":
        payload, metadata, scale = ext.compress_structured_int4(x, centers, ids)
    else:
        payload, scale = ext.compress_quantized(x, centers, ids, plan.nnz, plan.bits)
        metadata = None
    return CompressedTensor(centers, ids, payload, metadata, scale, plan)


@torch.no_grad()
def compress(
    key: torch.Tensor,
    value: torch.Tensor,
    config: ResKVKernelConfig | None = None,
    *,
    previous: CompressedKV | None = None,
    clustering: tuple | None = None,
    plan: KernelPlan | None = None,
) -> CompressedKV:
    """Compress pre-RoPE K and unrotated V; optionally append a decode group.

    ``clustering=((k_centers, k_ids), (v_centers, v_ids))`` reuses external
    clustering; ``previous`` extends the shared centroid tables during
    generation (reskv/compression.py:104-170).
    """
    config = ResKVKernelConfig() if config is None else config
    if not isinstance(config, ResKVKernelConfig):
        raise TypeError("compress requires ResKVKernelConfig; ResKVConfig is for accuracy evaluation")
    _validate(key)
    _validate(value)
    if key.shape != value.shape or key.device != value.device:
        raise ValueError("K and V must have identical shapes and devices")
    plan = plan or (previous.key.plan if previous else config.resolve(key.shape[0]))
    if plan.bits != config.bits or plan.nnz != int(128 * config.keep_ratio):
        raise ValueError("compression plan and configuration disagree")
    if config.layout != "auto" and plan.layout != config.layout:
        raise ValueError("compression plan violates the requested layout")
    if config.centroid_fusion != "auto" and plan.centroid_fusion != config.centroid_fusion:
        raise ValueError("compression plan violates the requested centroid fusion")
    if plan.fixed_shift != (config.softmax_mode == "fixed_shift"):
        raise ValueError("compression plan and softmax configuration disagree")
    if previous is not None and (
        previous.key.cluster_ids.shape[:2] != key.shape[:2] or previous.key.centroids.device != key.device
    ):
        raise ValueError("previous cache has incompatible dimensions or device")
    if previous is not None and max(previous.key.centroids.shape[2], previous.value.centroids.shape[2]) > (
        config.max_clusters
    ):
        raise ValueError("previous cache exceeds the configured centroid limit")
    if clustering is not None and previous is not None:
        raise ValueError("provide clustering or previous, not both")
    if clustering is not None:
        (kc, ki), (vc, vi) = clustering
        for centers, ids in ((kc, ki), (vc, vi)):
            if centers.shape[:2] != key.shape[:2] or centers.ndim != 4 or centers.shape[-1] != 128:
                raise ValueError("external centers must have shape [B,H,C,128]")
            if not 1 <= centers.shape[2] <= config.max_clusters or ids.shape != key.shape[:3]:
                raise ValueError("external clustering has incompatible sizes")
            if centers.device != key.device or ids.device != key.device:
                raise ValueError("external clustering must share the K/V device")
            if ids.dtype not in (torch.int8, torch.int16, torch.int32, torch.int64):
                raise ValueError("cluster IDs must be integer tensors")
            if bool(((ids < 0) | (ids >= centers.shape[2])).any()):
                raise ValueError("external cluster IDs are out of range")
    elif previous is not None:
        k, v = _compress_group(key, value, config, previous, plan)
        return CompressedKV(previous.key.append(k), previous.value.append(v))
    else:
        (kc, ki), (vc, vi) = cluster_kv(key, value, config.num_clusters, config.kmeans_iterations)
    k = _encode(key, kc, ki, plan)
    v = _encode(value, vc, vi, plan, value=True)
    return CompressedKV(k, v)


def _compress_group(key, value, config, previous, plan):
    """One decode group against the shared centroid tables of ``previous``
    (reskv/compression.py:160-169 without the final append): the group's own
    compressed K and V, each carrying the extended centroid table."""
    kc, ki = _incremental_cluster(key, previous.key.centroids, config)
    vc, vi = _incremental_cluster(value, previous.value.centroids, config, value=True)
    return _encode(key, kc, ki, plan), _encode(value, vc, vi, plan, value=True)
