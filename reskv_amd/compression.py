"""Clustering and residual compression through one K/V API (the
``reskv.compression`` surface, reskv/compression.py:12-170).

``cluster``, ``_incremental_cluster``, ``_encode`` and ``compress`` keep the
reference's names, arguments, validation messages and results.  Their work is
native: Lloyd iterations in ``reskv_kmeans`` (``reskv_kmeans_kv`` runs a
layer's K and V as one launch sequence), decode-group assignment in
``reskv_kmeans_assign``, and all four residual encoders, including the
unstructured FP16 bitmap encoder that the reference runs as a chain of
PyTorch ops.  ``compress`` is organised as: resolve the plan, run the
argument rules, obtain the clustering from one of three sources (external,
the previous cache's tables, or fresh K-means), encode, append.
"""

import torch

from ._extension import load_extension
from .config import KernelPlan, ResKVKernelConfig
from .tensors import CompressedKV, CompressedTensor

_ID_DTYPES = (torch.int8, torch.int16, torch.int32, torch.int64)


def _validate(x: torch.Tensor):
    if x.ndim != 4 or x.shape[-1] != 128 or not x.is_cuda or x.dtype != torch.float16:
        raise ValueError("expected FP16 CUDA tensor [batch, kv_heads, tokens, 128]")
    if min(x.shape[:3]) < 1:
        raise ValueError("batch, head and token dimensions must be nonempty")


def _ops(x: torch.Tensor):
    return load_extension("compression", device_index=x.device.index or 0)


def _initial_centers(data: torch.Tensor, count: int) -> torch.Tensor:
    """Initial centres [BH, C, 128] fp32 when T < C (reskv/compression.py:28-33):
    every token plus C - T jittered copies of random tokens (not deterministic,
    as in the reference).  For T >= C the library takes the tokens at
    ``linspace(0, T-1, C).long()`` itself (``reskv_linspace_rows``,
    reskv/compression.py:34-36)."""
    t = data.shape[1]
    pick = data[:, torch.randint(t, (count - t,), device=data.device)]
    return torch.cat((data, pick + torch.randn_like(pick) * 0.01), dim=1).float().contiguous()


def cluster(x: torch.Tensor, count: int = 32, iterations: int = 10, *, value: bool = False):
    """Lloyd clustering of K (fp32 distances and centres, empty clusters kept)
    or V (the fp16 ``cdist`` rule, fp16 centres, empty -> 0).

    Returns (centres fp16 [B, H, C, 128], ids int32 [B, H, T]); the ids are the
    last assignment, made against the centres before the final update.
    """
    b, h, t, d = x.shape
    if value:
        count = min(count, t)
    rows = x.reshape(b * h, t, d).contiguous()
    init = None  # T >= C: the library gathers the linspace tokens itself
    if t < count:
        init = _initial_centers(rows, count)
        if value:
            init = init.half().float()  # V centres live in fp16 (reskv/compression.py:27)
    centers, ids = _ops(x).kmeans(rows, init, iterations, value, count)
    return centers.view(b, h, count, d), ids.view(b, h, t)


def cluster_kv(key: torch.Tensor, value: torch.Tensor, count: int = 32, iterations: int = 10):
    """``(cluster(key, ...), cluster(value, ..., value=True))`` as one launch sequence.

    Each half equals its separate call (reskv/compression.py:164-165).  Below
    ``count`` tokens V caps its centroid count at T, so the two runs have
    different sizes and run apart.
    """
    b, h, t, d = key.shape
    if t < count:
        return cluster(key, count, iterations), cluster(value, count, iterations, value=True)
    krows = key.reshape(b * h, t, d).contiguous()
    vrows = value.reshape(b * h, t, d).contiguous()
    # the linspace tokens of both tensors, gathered by the library (T >= C here)
    (kc, ki), (vc, vi) = _ops(key).kmeans_kv(krows, vrows, None, None, iterations, count)
    shape_c, shape_i = (b, h, count, d), (b, h, t)
    return (kc.view(shape_c), ki.view(shape_i)), (vc.view(shape_c), vi.view(shape_i))


def _incremental_cluster(x, centers, config, *, value=False):
    """Append the group mean as a new centre while under the cap, then assign
    each token (reskv/compression.py:56-69)."""
    b, h, t, d = x.shape
    if centers.shape[2] < config.max_clusters:
        centers = torch.cat((centers, x.mean(2, keepdim=True)), dim=2)
    table = centers.reshape(b * h, -1, d).float().contiguous()
    ids = _ops(x).kmeans_assign(x.reshape(b * h, t, d).contiguous(), table, value)
    return centers, ids.view(b, h, t)


def _encode(x, centers, ids, plan, *, value=False):
    """Residual encoding of one tensor in the plan's format (reskv/compression.py:72-101).

    Returns a CompressedTensor; ``value`` is accepted for the reference's
    signature (K and V encode alike here: every encoder breaks magnitude ties
    towards the lower channel)."""
    ops = _ops(x)
    x, centers, ids = x.contiguous(), centers.half().contiguous(), ids.int().contiguous()
    metadata = scale = None
    if plan.bits == 16:
        if plan.layout == "unstructured":
            payload, metadata = ops.compress_bitmap(x, centers, ids, plan.nnz)
        else:
            payload, metadata = ops.compress_fp16(x, centers, ids, plan.nnz, plan.layout == "structured")
    elif plan.layout == "structured":
        payload, metadata, scale = ops.compress_structured_int4(x, centers, ids)
    else:
        payload, scale = ops.compress_quantized(x, centers, ids, plan.nnz, plan.bits)
    return CompressedTensor(centers, ids, payload, metadata, scale, plan)


def _encode_kv(key, value, k_clusters, v_clusters, plan):
    """``(_encode(key, ...), _encode(value, ..., value=True))``; the FP16
    formats run K and V in one launch (reskv/compression.py:166-167)."""
    (kc, ki), (vc, vi) = k_clusters, v_clusters
    if plan.bits != 16:
        return _encode(key, kc, ki, plan), _encode(value, vc, vi, plan, value=True)
    ops = _ops(key)
    kx, kc, ki = key.contiguous(), kc.half().contiguous(), ki.int().contiguous()
    vx, vc, vi = value.contiguous(), vc.half().contiguous(), vi.int().contiguous()
    if plan.layout == "unstructured":
        (kp, km), (vp, vm) = ops.compress_bitmap_kv(kx, kc, ki, vx, vc, vi, plan.nnz)
    else:
        (kp, km), (vp, vm) = ops.compress_fp16_kv(kx, kc, ki, vx, vc, vi, plan.nnz, plan.layout == "structured")
    return CompressedTensor(kc, ki, kp, km, None, plan), CompressedTensor(vc, vi, vp, vm, None, plan)


# ---------------------------------------------------------------------------
# compress: argument rules, then one of three clustering sources
# ---------------------------------------------------------------------------

def _plan_rules(plan: KernelPlan, config: ResKVKernelConfig):
    yield (plan.bits != config.bits or plan.nnz != int(128 * config.keep_ratio),
           "compression plan and configuration disagree")
    yield (config.layout != "auto" and plan.layout != config.layout,
           "compression plan violates the requested layout")
    yield (config.centroid_fusion != "auto" and plan.centroid_fusion != config.centroid_fusion,
           "compression plan violates the requested centroid fusion")
    yield plan.fixed_shift != (config.softmax_mode == "fixed_shift"), "compression plan and softmax configuration disagree"


def _previous_rules(previous: CompressedKV, key: torch.Tensor, config: ResKVKernelConfig):
    yield (previous.key.cluster_ids.shape[:2] != key.shape[:2] or previous.key.centroids.device != key.device,
           "previous cache has incompatible dimensions or device")
    largest = max(previous.key.centroids.shape[2], previous.value.centroids.shape[2])
    yield largest > config.max_clusters, "previous cache exceeds the configured centroid limit"


def _external_rules(centers: torch.Tensor, ids: torch.Tensor, key: torch.Tensor, config: ResKVKernelConfig):
    yield (centers.shape[:2] != key.shape[:2] or centers.ndim != 4 or centers.shape[-1] != 128,
           "external centers must have shape [B,H,C,128]")
    yield (not 1 <= centers.shape[2] <= config.max_clusters or ids.shape != key.shape[:3],
           "external clustering has incompatible sizes")
    yield centers.device != key.device or ids.device != key.device, "external clustering must share the K/V device"
    yield ids.dtype not in _ID_DTYPES, "cluster IDs must be integer tensors"
    yield bool(((ids < 0) | (ids >= centers.shape[2])).any()), "external cluster IDs are out of range"


def _enforce(rules):
    for failed, message in rules:
        if failed:
            raise ValueError(message)


def _clusters(key, value, config, previous, clustering):
    """((K centres, K ids), (V centres, V ids)) from the one source given."""
    if clustering is not None:
        for centers, ids in clustering:
            _enforce(_external_rules(centers, ids, key, config))
        return clustering
    if previous is not None:
        return (_incremental_cluster(key, previous.key.centroids, config),
                _incremental_cluster(value, previous.value.centroids, config, value=True))
    return cluster_kv(key, value, config.num_clusters, config.kmeans_iterations)


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
    """Compress pre-RoPE K and unrotated V; with ``previous``, encode one
    decode group against its centroid tables and return the extended cache.

    ``clustering=((k_centers, k_ids), (v_centers, v_ids))`` reuses an external
    clustering (controlled benchmarks).
    """
    if config is None:
        config = ResKVKernelConfig()
    if not isinstance(config, ResKVKernelConfig):
        raise TypeError("compress requires ResKVKernelConfig; ResKVConfig is for accuracy evaluation")
    _validate(key)
    _validate(value)
    if key.shape != value.shape or key.device != value.device:
        raise ValueError("K and V must have identical shapes and devices")
    if plan is None:
        plan = previous.key.plan if previous is not None else config.resolve(key.shape[0])
    _enforce(_plan_rules(plan, config))
    if previous is not None:
        _enforce(_previous_rules(previous, key, config))
        if clustering is not None:
            raise ValueError("provide clustering or previous, not both")
    k_clusters, v_clusters = _clusters(key, value, config, previous, clustering)
    k, v = _encode_kv(key, value, k_clusters, v_clusters, plan)
    if previous is not None:
        return CompressedKV(previous.key.append(k), previous.value.append(v))
    return CompressedKV(k, v)


def _compress_group(key, value, config, previous, plan):
    """One decode group against the shared centroid tables of ``previous``:
    the group's own K and V CompressedTensors, each carrying the extended
    centroid table (the device cache appends them in place)."""
    k_clusters, v_clusters = _clusters(key, value, config, previous, None)
    return _encode_kv(key, value, k_clusters, v_clusters, plan)
