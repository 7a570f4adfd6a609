"""Decode attention over a compressed cache: the ``reskv._attention.attention``
surface (reskv/_attention.py:10-144) on this library's engine.

The reference dispatches to one of two operator families and, when a dense
recent window is given, joins it in separate steps (fp32 scores by
``torch.bmm``, then a merge launch).  Here every plan runs through one call of
the C ABI: the cache's formats become descriptors, and the recent window is
joined inside the split-K merge kernel (``reskv_decode_recent``), so a decode
step is two kernel launches whatever the plan.  The family operators of
``load_extension`` compute the same function for callers that use them
directly.  Argument names, defaults, shapes and the ``ValueError`` messages
are the reference's, since callers and tests match on them.
"""

import torch

from ._extension import decode_step
from .tensors import CompressedKV

_GQA_RATIOS = (1, 4, 8)


def _cache_heads(query, cache):
    """(B, Hq, Hk) after the query/cache compatibility checks of the reference."""
    if query.ndim != 4 or query.shape[2:] != (1, 128) or not query.is_cuda or query.dtype != torch.float16:
        raise ValueError("query must be FP16 CUDA [batch, query_heads, 1, 128]")
    key, value = cache.key, cache.value
    if query.device != key.payload.device or query.device != value.payload.device:
        raise ValueError("query and cache must be on the same CUDA device")
    batch, heads = int(query.shape[0]), int(query.shape[1])
    kv_heads = int(key.centroids.shape[1])
    if batch != key.centroids.shape[0] or key.seq_len != value.seq_len:
        raise ValueError("query/cache batch or K/V sequence lengths differ")
    if key.plan != value.plan:
        raise ValueError("K and V plans differ")
    if heads % kv_heads or heads // kv_heads not in _GQA_RATIOS:
        raise ValueError("supported query/kv head ratios are 1, 4, and 8")
    return batch, heads, kv_heads


def _recent_window(recent, query, batch, kv_heads):
    """The dense window as contiguous (q_rot [B*Hq,128], k_rot, v) or None when empty."""
    if recent is None:
        return None
    q_rot, k_rot, v = recent
    if k_rot.shape[2] == 0:
        return None
    if (q_rot.shape != query.shape or k_rot.shape != v.shape or k_rot.dim() != 4 or k_rot.shape[3] != 128
            or tuple(k_rot.shape[:2]) != (batch, kv_heads)):
        raise ValueError("recent Q/K/V shapes do not match the compressed cache")
    if any(t.device != query.device or t.dtype != torch.float16 for t in (q_rot, k_rot, v)):
        raise ValueError("recent tensors must be FP16 on the query device")
    return q_rot.reshape(-1, 128).contiguous(), k_rot.contiguous(), v.contiguous()


@torch.no_grad()
def attention(
    query: torch.Tensor,
    cache: CompressedKV,
    *,
    position: int,
    start_position: int = 0,
    rope_theta: float = 500000.0,
    inv_freq: torch.Tensor | None = None,
    scaling: float | None = None,
    recent: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
    splits: int = 0,
):
    """Decode raw (pre-RoPE) Q [B, Hq, 1, 128] against the compressed pre-RoPE
    K and V of ``cache``; returns fp16 of Q's shape.

    ``recent`` = (rotated Q, rotated K, V) of dense tokens joined in the same
    softmax; ``inv_freq`` = the model's 64 RoPE frequencies (default: derived
    from ``rope_theta``); ``splits`` = 0 picks the split count from the CU
    occupancy.
    """
    batch, heads, kv_heads = _cache_heads(query, cache)
    if position < start_position + cache.seq_len - 1:
        raise ValueError("query position precedes compressed tokens")
    if inv_freq is not None and (inv_freq.shape != (64,) or inv_freq.device != query.device):
        raise ValueError("inv_freq must be [64] on the query CUDA device")
    window = _recent_window(recent, query, batch, kv_heads)
    out = decode_step(
        query.reshape(batch * heads, 128).contiguous(), cache, heads,
        position=int(position), start_position=int(start_position),
        scaling=128 ** -0.5 if scaling is None else float(scaling),
        inv_freq=inv_freq, rope_theta=float(rope_theta), splits=int(splits), recent=window,
    )
    return out.view(batch, heads, 1, 128)
