"""FP32 reconstruction and attention of a compressed cache, for numerical checks.

Counterpart of ``reskv/reference.py:12-91``, the reference package's own
diagnostic checker, which its benchmark harness uses to validate each measured
case (``reskv_amd.benchmarks.kernels``).  It runs plain torch on whatever
device the cache lives on.  No operator of this package calls it: ``compress``
and ``attention`` run only the HIP library and raise when it is missing.
"""

import torch

from .tensors import CompressedKV, CompressedTensor


def _signed(codes, bits):
    half = 1 << (bits - 1)
    return (codes ^ half) - half


def reconstruct(tensor: CompressedTensor) -> torch.Tensor:
    """Centre + residual of every token, float32 [B, H, T, 128]."""
    ids = tensor.cluster_ids.long()
    b, h, t = ids.shape
    dev = ids.device
    plan = tensor.plan
    dims = torch.arange(128, device=dev)
    if plan.layout == "unstructured" and plan.bits != 16:
        # dim d: word d // (32/bits), bit field (d % (32/bits)) * bits, signed codes times the scale
        per = 32 // plan.bits
        words = tensor.payload.long()[..., dims // per]
        codes = (words >> ((dims % per) * plan.bits)) & ((1 << plan.bits) - 1)
        residual = _signed(codes, plan.bits).float() * tensor.scale.float()[..., None]
    elif plan.layout == "unstructured":
        # dim d kept when bit 63 - d % 64 of word d // 64 is set; values in dim order
        words = tensor.metadata[..., dims // 64]
        kept = ((words >> (63 - dims % 64)) & 1).bool()
        order = kept.long().cumsum(-1) - 1
        residual = torch.where(kept, tensor.payload.gather(-1, order.clamp_min(0)).float(), 0.0)
    elif plan.bits == 4:
        # 32 subgroups of four dims, one kept each: a 2-bit position and a signed nibble
        sub = torch.arange(32, device=dev)
        nibbles = (tensor.payload.long()[..., sub // 8] >> ((sub % 8) * 4)) & 15
        values = _signed(nibbles, 4).float() * tensor.scale.float()[..., None]
        local = (tensor.metadata.long()[..., sub // 16] >> ((sub % 16) * 2)) & 3
        residual = torch.zeros(b, h, t, 128, device=dev, dtype=torch.float32)
        residual.scatter_(-1, local + 4 * sub, values)
    else:
        # word w holds the codes of tiles 2w (low half) and 2w + 1 (high half)
        tiles = torch.arange(8, device=dev)
        codes = (tensor.metadata.long()[..., tiles // 2] >> ((tiles % 2) * 16)) & 0xFFFF
        if plan.layout == "structured":
            slot = torch.arange(4, device=dev)
            within = (codes[..., None] >> (4 * slot)) & 15  # four ascending in-tile indices
            target = (within + 16 * tiles[:, None]).reshape(b, h, t, 32)
            residual = torch.zeros(b, h, t, 128, device=dev, dtype=torch.float32)
            residual.scatter_(-1, target, tensor.payload.float())
        else:
            bit = torch.arange(16, device=dev)
            kept = ((codes[..., None] >> bit) & 1).bool().reshape(b, h, t, 128)
            order = kept.long().cumsum(-1) - 1
            residual = torch.where(kept, tensor.payload.gather(-1, order.clamp_min(0)).float(), 0.0)
    centres = tensor.centroids.float().gather(2, ids[..., None].expand(-1, -1, -1, 128))
    return centres + residual


def rotate(x: torch.Tensor, positions: torch.Tensor, frequencies: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE in float32 at absolute positions (angle = fp32(position * frequency))."""
    angles = positions.float()[..., None] * frequencies.float()
    cos, sin = angles.cos(), angles.sin()
    lo, hi = x.float().chunk(2, dim=-1)
    return torch.cat((lo * cos - hi * sin, hi * cos + lo * sin), dim=-1)


def reference_attention(query: torch.Tensor, cache: CompressedKV, *, position: int, start_position: int = 0,
                        rope_theta: float = 500000.0, inv_freq: torch.Tensor | None = None,
                        scaling: float | None = None, recent: tuple | None = None) -> torch.Tensor:
    """Softmax attention of ``query`` [B, Hq, 1, 128] over the reconstructed cache
    (compressed tokens at positions start_position..) and optional dense recent
    tokens ``(query_rot, k_rot, v)``; float32 [B, Hq, 1, 128]."""
    k, v = reconstruct(cache.key), reconstruct(cache.value)
    b, kv_heads, t, _ = k.shape
    heads = query.shape[1]
    group = heads // kv_heads
    dev = query.device
    freq = inv_freq if inv_freq is not None else rope_theta ** (-torch.arange(64, device=dev).float() / 64)
    q = rotate(query, torch.tensor([position], device=dev), freq)
    k = rotate(k, torch.arange(start_position, start_position + t, device=dev), freq)
    k = k.repeat_interleave(group, 1)
    v = v.repeat_interleave(group, 1)
    scale = 128 ** -0.5 if scaling is None else scaling
    scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    if recent is not None:
        q_rot, k_rot, v_rec = recent
        kr = k_rot.float().repeat_interleave(group, 1)
        scores = torch.cat((scores, torch.matmul(q_rot.float(), kr.transpose(-1, -2).contiguous()) * scale), dim=-1)
        v = torch.cat((v, v_rec.float().repeat_interleave(group, 1)), dim=2)
    return torch.matmul(scores.softmax(-1), v)
