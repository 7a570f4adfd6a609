"""Seeded random sweep of decode parity against the float64 oracle.

Each case draws a plan (every layout / fusion / bit width combination the
reference's case matrix has, reskv tests/test_cuda.py), batch, KV heads, GQA
ratio 1/4/8, T (including 1, tile and split boundaries), 1-64 centroids, a
start offset, the query position, an explicit or automatic split count and an
optional recent window of 1-300 tokens (one to three join chunks), with
Gaussian or config-0 outlier-channel keys.

Bound per output element: max(2e-3, 1.5 fp16 ulp of the expected value).
For |x| < 2 that is the 2e-3 of the parity bar; above it, 2e-3 is less than
one fp16 step (1.95e-3 on [2, 4)), and the output passes through two fp16
roundings when a recent window is joined (the compressed result, then the
joined one), as in the reference's decode op followed by merge_recent, so the
expected value for those cases follows that structure
(expected_attention_two_step).
"""

import random

import numpy as np
import pytest
import torch

from oracle import reskv_oracle as o
from reskv_amd import ResKVKernelConfig, attention, compress
from tests.gpu_helpers import ATOL, expected_attention_two_step, np_, outlier_kv, seeded, theta_freq

pytestmark = pytest.mark.gpu

COMBOS = [(16, 0.5, "unstructured", "deferred"), (16, 0.75, "unstructured", "deferred"),
          (16, 0.5, "tiled", "per_token"), (16, 0.75, "structured", "per_token"),
          (16, 0.75, "structured", "deferred"), (4, 0.5, "unstructured", "per_token"),
          (4, 0.75, "unstructured", "per_token"), (2, 0.5, "unstructured", "per_token"),
          (2, 0.75, "unstructured", "per_token"), (4, 0.75, "structured", "per_token"),
          (4, 0.75, "structured", "deferred")]
CHUNKS, PER_CHUNK = 8, 20


def _case(index, device):
    rnd = random.Random(1009 * index + 7)
    bits, sp, lay, fus = rnd.choice(COMBOS)
    b = rnd.choice([1, 2, 3, 5])
    h = rnd.choice([1, 2, 8])
    gqa = rnd.choice([1, 4, 8])
    t = rnd.choice([1, 2, 15, 16, 17, 63, 64, 65, 127, 129, 300, 777, 1024, 1500, 2500])
    nc = rnd.choice([1, 4, 16, 32, 64])
    start = rnd.choice([0, 0, 3, 37])
    pos = start + t - 1 + rnd.choice([0, 0, 1, 20])
    splits = rnd.choice([0, 0, 0, 1, 3, 7])
    tr = rnd.choice([0, 0, 0, 1, 31, 96, 129, 300])
    g = seeded(7919 * index + 3)
    if rnd.random() < 0.5:
        k, v, q = outlier_kv(b, h, t, seed=31 * index + 1, gqa=gqa, device=device)
    else:
        k = (torch.randn(b, h, t, 128, generator=g) * 0.5).half().to(device)
        v = (torch.randn(b, h, t, 128, generator=g) * 0.5).half().to(device)
        q = (torch.randn(b, h * gqa, 1, 128, generator=g) * 0.5).half().to(device)
    kc = (torch.randn(b, h, nc, 128, generator=g) * 0.1).half().to(device)
    vc = (torch.randn(b, h, nc, 128, generator=g) * 0.1).half().to(device)
    ki = torch.randint(nc, (b, h, t), generator=g, dtype=torch.int32).to(device)
    vi = torch.randint(nc, (b, h, t), generator=g, dtype=torch.int32).to(device)
    cfg = ResKVKernelConfig(bits=bits, sparsity=sp, layout=lay, centroid_fusion=fus)
    cache = compress(k, v, cfg, clustering=((kc, ki), (vc, vi)))
    freq = theta_freq(device=device)
    recent = None
    if tr:
        kr = torch.randn(b, h, tr, 128, generator=g).half().to(device)
        vr = torch.randn(b, h, tr, 128, generator=g).half().to(device)
        qr = torch.from_numpy(o.rotate(np_(q).astype(np.float64), np.array([pos + tr]), np_(freq))).half()
        recent = (qr.to(device), kr, vr)
    desc = dict(index=index, bits=bits, sparsity=sp, layout=lay, fusion=fus, b=b, h=h, gqa=gqa, t=t, nc=nc,
                start=start, pos=pos, splits=splits, tr=tr)
    return cache, q, freq, pos, start, splits, recent, desc


@pytest.mark.parametrize("chunk", range(CHUNKS))
def test_random_decode_cases_against_the_oracle(device, chunk):
    for index in range(chunk * PER_CHUNK, (chunk + 1) * PER_CHUNK):
        cache, q, freq, pos, start, splits, recent, desc = _case(index, device)
        out = attention(q, cache, position=pos, start_position=start, inv_freq=freq, splits=splits, recent=recent)
        ref = expected_attention_two_step(q, cache, position=pos, start_position=start, inv_freq=freq, recent=recent)
        err = np.abs(np_(out).astype(np.float64) - ref)
        ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
        bound = np.maximum(ATOL, 1.5 * ulp)
        worst = int((err - bound).argmax())
        assert (err <= bound).all(), (desc, float(err.flat[worst]), float(ref.flat[worst]))
