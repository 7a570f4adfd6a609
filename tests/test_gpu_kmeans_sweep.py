"""Seeded random sweep of the HIP k-means against the oracle, one Lloyd step at a time.

Each case draws B, H, T (from the centre count up to 3000), the centre count
(1 to 64), the iteration count n (1 to 5), K or V and a data kind (Gaussian,
config-0 outlier channels, tokens of widely different norms, a coarse grid
with exact ties).
The device run is deterministic, so the run with n - 1 iterations yields the
centres that the n-th assignment used (the linspace tokens for n = 1): V's
fp16 centres as returned, K's fp32 centres as the member means of that run's
ids (the library returns K centres rounded to fp16).  Then:

- the n-th ids equal the oracle's assignment against those centres: K
  wherever the exact margin exceeds fp32 rounding of the distances and of
  the member sums; V on every token the oracle does not flag as within fp32
  accumulation error of an fp16 rounding midpoint; on the coarse grid at
  n = 1 every distance is exact in fp32, so ids must equal the oracle's
  everywhere, lowest index on ties;
- the n-th centres are the oracle's update from those ids within one fp16
  step.
"""

import random

import numpy as np
import pytest
import torch

from oracle import reskv_oracle as o
from reskv_amd.compression import cluster
from tests.gpu_helpers import np_, outlier_kv, seeded

pytestmark = pytest.mark.gpu

KINDS = ["normal", "outliers", "scaled", "grid"]
CHUNKS, PER_CHUNK = 4, 10


def _data(kind, b, h, t, seed):
    g = seeded(seed)
    if kind == "normal":
        return torch.randn(b, h, t, 128, generator=g).half()
    if kind == "outliers":
        k, _, _ = outlier_kv(b, h, t, seed, device="cpu")
        return k
    if kind == "scaled":  # per-token scales from LogNormal(0, 1)
        return (torch.randn(b, h, t, 128, generator=g) * torch.exp(torch.randn(b, h, t, 1, generator=g))).half()
    return (torch.randint(-4, 5, (b, h, t, 128), generator=g).float() * 0.25).half()  # grid


def _within_one_fp16_step(got, ref):
    got = np.asarray(got, dtype=np.float16)
    ref = np.asarray(ref, dtype=np.float64).astype(np.float16)
    up = np.nextafter(ref, np.float16(np.inf))
    dn = np.nextafter(ref, np.float16(-np.inf))
    return ((got == ref) | (got == up) | (got == dn)).all()


def _k_safe(data, centres, margin, exact_centres):
    """Tokens whose K assignment is decided beyond fp32 rounding of the
    distances and, for centres that are fp32 member means, beyond the shift
    a 1e-5 relative error of every centre entry can cause."""
    row_scale = (data * data).sum(-1) + (centres * centres).sum(-1).max(-1)[:, None]
    bound = 1e-5 * row_scale
    if not exact_centres:
        err = 1e-5 * (np.abs(centres) + 1e-3)
        shift = np.einsum("ntd,ncd->ntc", np.abs(data), err) + (np.abs(centres) * err).sum(-1)[:, None, :]
        bound = bound + 4.0 * shift.max(-1)
    return margin > bound


@pytest.mark.parametrize("chunk", range(CHUNKS))
def test_random_kmeans_steps_against_the_oracle(device, chunk):
    for index in range(chunk * PER_CHUNK, (chunk + 1) * PER_CHUNK):
        rnd = random.Random(7907 * index + 5)
        b, h = rnd.choice([1, 2]), rnd.choice([1, 3])
        count = rnd.choice([1, 2, 7, 16, 32, 64])
        t = rnd.choice([count, count + 1, 100, 257, 1000, 3000])
        t = max(t, count)
        n = rnd.choice([1, 2, 3, 5])
        value = rnd.random() < 0.5
        kind = rnd.choice(KINDS)
        desc = dict(index=index, b=b, h=h, t=t, count=count, n=n, value=value, kind=kind)
        x = _data(kind, b, h, t, 300 + index).to(device)
        centres_n, ids_n = cluster(x, count, n, value=value)
        data16 = np_(x).reshape(b * h, t, 128)
        data = data16.astype(np.float64)
        if n == 1:
            prev = data[:, o.linspace_indices(t, count)]
        else:
            prev_t, prev_ids = cluster(x, count, n - 1, value=value)
            prev = np_(prev_t).reshape(b * h, count, 128).astype(np.float64)
            if not value:  # the fp32 centres: member means (empty clusters keep theirs)
                prev = o.update_centres(data, np_(prev_ids).reshape(b * h, t).astype(np.int64), prev, count)
                if n == 2:
                    first = data[:, o.linspace_indices(t, count)]
                    empty = np.eye(count)[np_(prev_ids).reshape(b * h, t)].sum(1) == 0
                    prev = np.where(empty[..., None], first, prev)
        gids = np_(ids_n).reshape(b * h, t).astype(np.int64)
        exact = kind == "grid" and n == 1  # every product and sum exact in fp32
        if value:
            ora = o.assign_value(data16, prev.astype(np.float16))
            if exact:
                assert np.array_equal(gids, ora), desc
            else:
                amb = o.value_ambiguous(data16, prev.astype(np.float16))
                # grid norms are exact sums that can sit on an fp16 midpoint;
                # elsewhere ambiguity is rare
                assert (amb.mean() < 0.02 if kind != "grid" else (~amb).mean() > 0.3), desc
                assert np.array_equal(gids[~amb], ora[~amb]), desc
        else:
            ora, margin = o.assign(data, prev)
            if exact:
                assert np.array_equal(gids, ora), desc
            else:
                safe = _k_safe(data, prev, margin, exact_centres=n == 1)
                assert safe.mean() > (0.8 if kind != "grid" else 0.3), desc
                assert np.array_equal(gids[safe], ora[safe]), desc
        ref = o.update_centres(data, gids, prev, count, value=value)
        assert _within_one_fp16_step(np_(centres_n).reshape(b * h, count, 128), ref), desc
