"""Fused decode over the compressed cache with an exact joint softmax for recent tokens.

Mirror of ``reskv/_attention.py:10-144``: same signature, validation and
result.  Dispatch goes to the per-token (``attention``) or deferred
(``cluster_mass``) operator family selected by the plan, exactly as the
reference does; both families run the same split-K HIP engine, whose split
count is chosen from the 256-CU occupancy (``splits=0``) rather than the
plan's hint tuned for another GPU.  The dense recent window is merged by the
in-kernel-score variant of ``merge_recent`` for both families (the reference
computes deferred-family scores with a separate ``torch.bmm``).
"""

import torch

from ._extension import load_extension
from .tensors import CompressedKV


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
    """Decode raw Q [B,H,1,128] against compressed pre-RoPE K and V.

    ``recent`` is (rotated Q, rotated K, V); ``inv_freq`` holds the model's 64
    RoPE frequencies, omitted -> theta-derived.  Output has the shape of Q.
    """
    if query.ndim != 4 or query.shape[2:] != (1, 128) or not query.is_cuda or query.dtype != torch.float16:
        raise ValueError("query must be FP16 CUDA [batch, query_heads, 1, 128]")
    b, nh = query.shape[:2]
    kh = cache.key.centroids.shape[1]
    if query.device != cache.key.payload.device or query.device != cache.value.payload.device:
        raise ValueError("query and cache must be on the same CUDA device")
    if b != cache.key.centroids.shape[0] or cache.key.seq_len != cache.value.seq_len:
        raise ValueError("query/cache batch or K/V sequence lengths differ")
    if cache.key.plan != cache.value.plan:
        raise ValueError("K and V plans differ")
    if nh % kh or nh // kh not in (1, 4, 8):
        raise ValueError("supported query/kv head ratios are 1, 4, and 8")
    if position < start_position + cache.seq_len - 1:
        raise ValueError("query position precedes compressed tokens")
    plan = cache.key.plan
    family = "attention" if plan.centroid_fusion == "per_token" else "cluster_mass"
    ext = load_extension(family, plan, query.device.index or 0)
    q = query.reshape(b * nh, 128).contiguous()
    kc, ki, kp, km, ks = cache.key._native
    vc, vi, vp, vm, vs = cache.value._native
    scale = 128**-0.5 if scaling is None else float(scaling)
    if inv_freq is None:
        freq = torch.empty(0, dtype=torch.float32, device=query.device)
    else:
        if inv_freq.shape != (64,) or inv_freq.device != query.device:
            raise ValueError("inv_freq must be [64] on the query CUDA device")
        freq = inv_freq.float().contiguous()
    empty = query.new_empty(0)
    suffix = (kh, nh, int(start_position), int(position), float(rope_theta), scale)
    if plan.centroid_fusion == "deferred":
        if plan.layout == "unstructured":
            out, m, normalizer = ext.decode_fp16(q, kc, ki, kp, km, vc, vi, vp, vm, *suffix, True, splits, freq)
        else:
            fn = ext.decode_structured_int4 if plan.bits == 4 else ext.decode_structured_fp16
            out, m, normalizer = fn(
                q, kc, ki, kp, km, ks if ks is not None else empty, vc, vi, vp, vm,
                vs if vs is not None else empty, *suffix, True, splits, freq,
            )
    elif plan.layout == "unstructured":
        out, m, normalizer = ext.decode_quantized(
            q, kc, ki, kp, ks, vc, vi, vp, vs, *suffix, plan.bits, plan.bits, splits, freq
        )
    else:
        fn = ext.decode_int4 if plan.bits == 4 else ext.decode_fp16
        out, m, normalizer = fn(
            q, kc, ki, kp, km, ks if ks is not None else empty, vc, vi, vp, vm,
            vs if vs is not None else empty, *suffix, splits, freq,
        )
    if recent is not None and recent[1].shape[2] > 0:
        qr, kr, vr = recent
        if qr.shape != query.shape or kr.shape != vr.shape or kr.shape[:2] != (b, kh):
            raise ValueError("recent Q/K/V shapes do not match the compressed cache")
        if any(x.device != query.device or x.dtype != torch.float16 for x in recent):
            raise ValueError("recent tensors must be FP16 on the query device")
        merge = load_extension("attention", None, query.device.index or 0).merge_recent
        out = merge(out, m, normalizer, qr.reshape(b * nh, 128).contiguous(), kr.contiguous(), vr.contiguous(),
                    kh, nh, scale)
    return out.reshape(b, nh, 1, 128)
