"""Seeded random sweep of both merge_recent ops against the oracle's joint softmax.

Each case draws B, KV heads, the GQA ratio (1/4/8), a recent window Tr of
0-513 tokens (within and across the 128-token join chunks), compressed
statistics (m from -8 to 8, l from 0.5 to 200) and recent scores that may
exceed m or fall far below it, then runs

- the deferred family's op with precomputed fp32 scores
  (``load_extension("cluster_mass").merge_recent``, cluster_mass.cu:1461-1508),
- the per-token family's op with the rotated query and keys
  (``load_extension("attention").merge_recent``, attention.cu:839-906; Tr >= 1),

and compares both with ``oracle.merge_recent`` in float64 (pinned against the
joint softmax of the concatenated tokens in tests/test_oracle.py).  Bound per
output element: max(2e-3, 1.5 fp16 ulp of the expected value).
"""

import random

import numpy as np
import pytest
import torch

from oracle import reskv_oracle as o
from tests.gpu_helpers import ATOL, np_, seeded

pytestmark = pytest.mark.gpu

CHUNKS, PER_CHUNK = 3, 20


@pytest.fixture(scope="module")
def exts(device):
    from reskv_amd._extension import load_extension

    return load_extension("cluster_mass"), load_extension("attention")


def _bound_ok(got, ref):
    err = np.abs(np_(got).astype(np.float64) - ref)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    return (err <= np.maximum(ATOL, 1.5 * ulp)).all(), float(err.max())


@pytest.mark.parametrize("chunk", range(CHUNKS))
def test_random_recent_merges_against_the_oracle(exts, device, chunk):
    deferred, per_token = exts
    for index in range(chunk * PER_CHUNK, (chunk + 1) * PER_CHUNK):
        rnd = random.Random(6007 * index + 13)
        b, kh, gqa = rnd.choice([1, 2, 3]), rnd.choice([1, 2, 8]), rnd.choice([1, 4, 8])
        nh = kh * gqa
        tr = rnd.choice([0, 1, 2, 31, 127, 128, 129, 255, 300, 513])
        scale = 128 ** -0.5
        g = seeded(9001 + index)
        comp_out = torch.randn(b * nh, 128, generator=g).half()
        comp_m = (torch.rand(b * nh, generator=g) * 16 - 8).float()
        comp_l = (torch.rand(b * nh, generator=g) * 199.5 + 0.5).float()
        q = (torch.randn(b * nh, 128, generator=g) * rnd.choice([0.5, 1.0, 3.0])).half()
        k = torch.randn(b, kh, tr, 128, generator=g).half()
        v = torch.randn(b, kh, tr, 128, generator=g).half()
        desc = dict(index=index, b=b, kh=kh, gqa=gqa, tr=tr)
        # scaled scores as the reference's Python computes them for the deferred op (fp32)
        qf = q.float().reshape(b, kh, gqa, 128)
        scores = (torch.matmul(qf, k.float().transpose(-1, -2).contiguous()) * scale).reshape(b, nh, tr).contiguous()
        v_rep = np.repeat(np_(v).astype(np.float64), gqa, axis=1)  # [B, nh, Tr, 128]
        ref = o.merge_recent(np_(comp_out).astype(np.float64).reshape(b, nh, 128), np_(comp_m).reshape(b, nh),
                             np_(comp_l).reshape(b, nh), np_(scores).astype(np.float64), v_rep)
        dev = [t.to(device) for t in (comp_out, comp_m, comp_l, scores, v)]
        out = deferred.merge_recent(*dev, kh, nh)
        ok, worst = _bound_ok(out.reshape(b, nh, 128), ref)
        assert ok, ("deferred", desc, worst)
        if tr == 0:
            continue
        out = per_token.merge_recent(dev[0], dev[1], dev[2], q.to(device), k.to(device), dev[4], kh, nh, scale)
        ok, worst = _bound_ok(out.reshape(b, nh, 128), ref)
        assert ok, ("per-token", desc, worst)
