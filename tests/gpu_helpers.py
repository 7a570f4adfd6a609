"""Shared inputs and oracle adapters for the GPU parity tests."""

import numpy as np
import torch

from oracle import reskv_oracle as o

ATOL = 2e-3  # max-abs bound on fp16 attention outputs (softmax-weighted sum)


def np_(t):
    return t.detach().cpu().numpy()


def oracle_format(plan):
    if plan.bits == 16:
        return {"unstructured": "bitmap", "tiled": "tiled", "structured": "structured"}[plan.layout]
    return "struct_int4" if plan.layout == "structured" else "quant"


def dense(ct):
    """Oracle reconstruction (float64 [B,H,T,128]) of a GPU CompressedTensor."""
    plan = ct.plan
    meta = None if ct.metadata is None else np_(ct.metadata)
    scale = None if ct.scale is None else np_(ct.scale)
    return o.reconstruct(oracle_format(plan), np_(ct.centroids), np_(ct.cluster_ids).astype(np.int64),
                         np_(ct.payload), meta, scale, bits=plan.bits)


def expected_attention(q, cache, *, position, start_position=0, inv_freq=None, rope_theta=500000.0,
                       scaling=None, recent=None):
    freq = None if inv_freq is None else np_(inv_freq)
    rec = None if recent is None else tuple(np_(x).astype(np.float64) for x in recent)
    return o.reference_attention(np_(q).astype(np.float64), dense(cache.key), dense(cache.value),
                                 position=position, start_position=start_position, freq=freq,
                                 rope_theta=rope_theta, scaling=scaling, recent=rec)


def expected_attention_two_step(q, cache, *, position, start_position=0, inv_freq=None, rope_theta=500000.0,
                                scaling=None, recent=None):
    """The reference's structure for a recent window: the compressed result is
    an fp16 op output, then joined with the recent tokens (merge_recent).
    Float64 [B, Hq, 1, 128]; without a window the same as expected_attention."""
    if recent is None:
        return expected_attention(q, cache, position=position, start_position=start_position, inv_freq=inv_freq,
                                  rope_theta=rope_theta, scaling=scaling)
    freq = None if inv_freq is None else np_(inv_freq)
    qq = np_(q).astype(np.float64)
    out, m, l = o.compressed_stats(qq, dense(cache.key), dense(cache.value), position=position,
                                   start_position=start_position, freq=freq, rope_theta=rope_theta,
                                   scaling=scaling)
    out16 = out.astype(np.float16).astype(np.float64)
    q_r, k_r, v_r = (np_(x).astype(np.float64) for x in recent)
    g = q.shape[1] // k_r.shape[1]
    scale = 128 ** -0.5 if scaling is None else scaling
    scores = (q_r @ np.swapaxes(np.repeat(k_r, g, axis=1), -1, -2))[..., 0, :] * scale
    return o.merge_recent(out16, m, l, scores, np.repeat(v_r, g, axis=1))[:, :, None]


def seeded(seed):
    return torch.Generator().manual_seed(seed)


def reference_test_inputs(b=1, t=256, heads=1, gqa=4, seed=123, device="cuda"):
    """The synthetic recipe of reskv tests/test_cuda.py:27-36 (values 0.5 N(0,1), centres 0.1 N(0,1))."""
    g = seeded(seed)
    k = (torch.randn(b, heads, t, 128, generator=g) * 0.5).half()
    v = (torch.randn(b, heads, t, 128, generator=g) * 0.5).half()
    q = (torch.randn(b, heads * gqa, 1, 128, generator=g) * 0.5).half()
    kc = (torch.randn(b, heads, 32, 128, generator=g) * 0.1).half()
    vc = (torch.randn(b, heads, 32, 128, generator=g) * 0.1).half()
    ki = torch.randint(32, (b, heads, t), generator=g, dtype=torch.int32)
    vi = torch.randint(32, (b, heads, t), generator=g, dtype=torch.int32)
    to = lambda x: x.to(device)  # noqa: E731
    return to(k), to(v), to(q), ((to(kc), to(ki)), (to(vc), to(vi)))


def outlier_kv(b, heads, t, seed, device="cuda", gqa=4):
    """Config-0 distributions: K = N(0,1) * LogNormal(0,1) per channel with 4 outlier
    channels x10 per head; V ~ N(0,1); one query per head ~ N(0,1)."""
    g = seeded(seed)
    scale = torch.exp(torch.randn(1, heads, 1, 128, generator=g))
    for h in range(heads):
        idx = torch.randperm(128, generator=g)[:4]
        scale[0, h, 0, idx] *= 10.0
    k = (torch.randn(b, heads, t, 128, generator=g) * scale).half()
    v = torch.randn(b, heads, t, 128, generator=g).half()
    q = torch.randn(b, heads * gqa, 1, 128, generator=g).half()
    return k.to(device), v.to(device), q.to(device)


def theta_freq(theta=500000.0, device="cuda"):
    return (theta ** (-torch.arange(64, device=device).float() / 64)).float()
