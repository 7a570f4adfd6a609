"""HIP k-means against the CPU oracle.

K follows the fp32 rule: ids equal the exact-distance ids wherever the
nearest/second-nearest margin exceeds fp32 rounding.  V follows the reference's
fp16 ``cdist`` rule (compression.py:27, 38): ids equal the oracle's
``assign_value`` on every token the oracle does not flag as sitting within fp32
accumulation error of an fp16 rounding midpoint.  Centres are always checked:
the oracle recomputes one update from the GPU's own ids, which the GPU centres
must match within one fp16 step.
"""

import numpy as np
import pytest
import torch

from oracle import reskv_oracle as o
from reskv_amd.compression import _incremental_cluster, cluster, cluster_kv
from reskv_amd import ResKVKernelConfig
from tests.gpu_helpers import np_, outlier_kv, seeded

pytestmark = pytest.mark.gpu


def _tie_free_equal(gpu_ids, ora_ids, margin, data, centers):
    """Equal ids wherever the exact margin exceeds fp32 rounding of that row's distances.

    The device forms |c|^2 - 2<x, c> in fp32 over 128 channels; its error is a
    few ulps of |x|^2 + |c|^2, so a margin of 1e-5 of that sum is safely decided.
    """
    row_scale = (data * data).sum(-1) + (centers * centers).sum(-1).max(-1)[:, None]
    safe = margin > 1e-5 * row_scale
    assert safe.mean() > 0.9
    assert np.array_equal(gpu_ids[safe], ora_ids[safe])


def _within_one_fp16_step(got, ref):
    """Every entry of got (fp16) is ref (fp16) or one of its fp16 neighbours."""
    got = np.asarray(got, dtype=np.float16)
    ref = np.asarray(ref, dtype=np.float64).astype(np.float16)
    up = np.nextafter(ref, np.float16(np.inf))
    dn = np.nextafter(ref, np.float16(-np.inf))
    ok = (got == ref) | (got == up) | (got == dn)
    assert ok.all(), f"{(~ok).sum()} centre entries beyond one fp16 step"
    return (got == ref).mean()


def _check_one_iteration(x, value, count=32):
    """One Lloyd iteration from the linspace init: ids against the oracle rule,
    centres against the oracle's update from the GPU ids."""
    b, h, t, _ = x.shape
    centers, ids = cluster(x, count, 1, value=value)
    data16 = np_(x).reshape(b * h, t, 128)
    data = data16.astype(np.float64)
    init = data[:, o.linspace_indices(t, count)]
    gids = np_(ids).reshape(b * h, t).astype(np.int64)
    if value:
        ora = o.assign_value(data16, init.astype(np.float16))
        amb = o.value_ambiguous(data16, init.astype(np.float16))
        assert amb.mean() < 0.005
        assert np.array_equal(gids[~amb], ora[~amb])
        # the exact (K) rule disagrees with the reference's V rule on some tokens,
        # which this test would catch if the device used it
        exact, _ = o.assign(data, init)
        differ = (exact != ora) & ~amb
        assert differ.any()
        assert np.array_equal(gids[differ], ora[differ])
    else:
        ora, margin = o.assign(data, init)
        _tie_free_equal(gids, ora, margin, data, init)
    ref = o.update_centres(data, gids, init, count, value=value)
    frac = _within_one_fp16_step(np_(centers).reshape(b * h, count, 128), ref)
    assert frac > 0.99
    return gids


@pytest.mark.parametrize("value", [False, True])
def test_single_iteration_matches_oracle(device, value):
    k, v, _ = outlier_kv(1, 4, 1000, seed=21 if not value else 22)
    _check_one_iteration(v if value else k, value)


@pytest.mark.parametrize("value", [False, True])
def test_single_iteration_at_config1_shape(device, value):
    """Config 1: 8 heads x 8192 tokens, outlier-channel K, N(0,1) V."""
    k, v, _ = outlier_kv(1, 8, 8192, seed=41)
    _check_one_iteration(v if value else k, value)


@pytest.mark.parametrize("value", [False, True])
def test_separated_mixture_full_run(device, value):
    g = seeded(3)
    means = torch.randn(1, 2, 8, 128, generator=g) * 4
    member = torch.randint(8, (1, 2, 2048), generator=g)
    # one linspace-initialised token per true cluster, so Lloyd never splits a
    # cluster and every assignment is decided by a wide margin
    member[..., torch.from_numpy(o.linspace_indices(2048, 8))] = torch.arange(8)
    x = means.gather(2, member[..., None].expand(-1, -1, -1, 128)) + torch.randn(1, 2, 2048, 128, generator=g) * 0.3
    x = x.half().to(device)
    centers, ids = cluster(x, 8, 10, value=value)
    ec, eids, margin = o.kmeans(np_(x), 8, 10, value=value)
    assert margin > (10.0 if value else 100.0)
    assert np.array_equal(np_(ids), eids)
    _within_one_fp16_step(np_(centers), ec)


@pytest.mark.parametrize("count", [1, 32])
def test_value_cluster_mean_does_not_overflow(device, count):
    # known answer of reskv tests/test_cuda.py:161-169
    data = torch.full((1, 1, 8192, 128), 20.0, device=device, dtype=torch.float16)
    centers, assignments = cluster(data, count=count, iterations=2, value=True)
    assert torch.isfinite(centers).all()
    restored = centers.gather(2, assignments.long().unsqueeze(-1).expand_as(data))
    assert torch.equal(restored, data)


def test_value_ties_take_the_lowest_index(device):
    """Two different fp16 squared distances with one fp16 root (256.25 and 256
    both give 16): the reference's fp16 cdist picks the lower index, which the
    exact rule would not."""
    x = torch.zeros(1, 1, 64, 128, dtype=torch.float16)
    x[0, 0, 0, 1], x[0, 0, 0, 2] = 16.0, 0.5      # linspace picks tokens 0, 21, 42, 63
    x[0, 0, 21, 0] = 16.0
    x[0, 0, 42, 3] = 40.0
    x[0, 0, 63, 4] = 40.0
    # every other token sits at the origin; token 5's distances to centres 0 and 1: 256.25 vs 256
    _, ids = cluster(x.to(device), 4, 1, value=True)
    assert int(ids[0, 0, 5]) == 0
    exact, _ = o.assign(np_(x).reshape(1, 64, 128).astype(np.float64),
                        np_(x).reshape(1, 64, 128)[:, o.linspace_indices(64, 4)].astype(np.float64))
    assert exact[0, 5] == 1
    assert np.array_equal(np_(ids).reshape(1, 64), o.assign_value(np_(x).reshape(1, 64, 128),
                                                                   np_(x).reshape(1, 64, 128)[:, [0, 21, 42, 63]]))


def test_short_input_key_clustering(device):
    x = torch.randn(1, 2, 5, 128, device=device).half()
    centers, ids = cluster(x, 8, 3)
    assert centers.shape == (1, 2, 8, 128) and torch.isfinite(centers).all()
    assert int(ids.min()) >= 0 and int(ids.max()) < 8
    vc, vi = cluster(x, 8, 3, value=True)  # V caps the count at T
    assert vc.shape == (1, 2, 5, 128)


@pytest.mark.parametrize("value", [False, True])
def test_incremental_cluster_matches_oracle(device, value):
    g = seeded(8)
    x = torch.randn(2, 2, 64, 128, generator=g).half().to(device)
    c = torch.randn(2, 2, 20, 128, generator=g).half().to(device)
    cfg = ResKVKernelConfig(num_clusters=20, max_clusters=21)
    c2, ids = _incremental_cluster(x, c, cfg, value=value)
    ec, eids, _ = o.incremental_cluster(np_(x), np_(c), 21, value=value)
    assert c2.shape[2] == 21
    assert np.array_equal(np_(c2), ec)  # the fp16 group mean, correctly rounded
    if value:
        d = o.incremental_value_distances(np_(x), ec).reshape(4, 64, 21)
        srt = np.sort(d, -1)
        safe = (srt[..., 1] - srt[..., 0]) > 1e-4 * np.abs(srt[..., 0]).max()
        assert safe.mean() > 0.9
        assert np.array_equal(np_(ids).reshape(4, 64)[safe], eids.reshape(4, 64)[safe])
    else:
        data = np_(x).astype(np.float64).reshape(4, 64, 128)
        cen = np_(c2).astype(np.float64).reshape(4, 21, 128)
        _, margin = o.assign(data, cen)
        _tie_free_equal(np_(ids).reshape(4, -1), eids.reshape(4, -1), margin, data, cen)
    c3, _ = _incremental_cluster(x, c2, cfg, value=value)  # at the cap: no new centre
    assert c3.shape[2] == 21


def test_incremental_value_rule_differs_from_exact(device):
    """The decode-group V rule rounds |x|^2 + |c|^2 to fp16 first; on
    near-equidistant centres that decides the id differently from the exact
    distance, and the device follows the reference."""
    g = seeded(9)
    x = (torch.randn(1, 8, 64, 128, generator=g) * 2).half()
    c = (torch.randn(1, 8, 40, 128, generator=g) * 2).half()
    cfg = ResKVKernelConfig(num_clusters=40, max_clusters=40)
    _, ids = _incremental_cluster(x.to(device), c.to(device), cfg, value=True)
    d = o.incremental_value_distances(np_(x), np_(c)).reshape(8 * 64, 40)
    ora = np.argmin(d, -1)
    srt = np.sort(d, -1)
    safe = (srt[:, 1] - srt[:, 0]) > 1e-4 * np.abs(srt[:, 0]).max()
    got = np_(ids).reshape(-1)
    assert np.array_equal(got[safe], ora[safe])


@pytest.mark.parametrize("t,count", [(1000, 32), (300, 20), (2100, 64), (40, 8)])
def test_paired_kv_clustering_equals_separate_runs(device, t, count):
    """K and V in one launch sequence give exactly the two separate runs' results."""
    k, v, _ = outlier_kv(2, 3, t, seed=31)
    (kc, ki), (vc, vi) = cluster_kv(k, v, count, 5)
    ek, eki = cluster(k, count, 5)
    ev, evi = cluster(v, count, 5, value=True)
    assert torch.equal(ki, eki) and torch.equal(vi, evi)
    assert torch.equal(kc, ek) and torch.equal(vc, ev)


def test_paired_kv_clustering_at_config1_scale(device):
    """Config 1 shape: the separate runs (256 workgroups, centre operands in
    registers) and the paired run (512 workgroups, operands from LDS) agree exactly."""
    k, v, _ = outlier_kv(1, 8, 8192, seed=41)
    (kc, ki), (vc, vi) = cluster_kv(k, v, 32, 3)
    ek, eki = cluster(k, 32, 3)
    ev, evi = cluster(v, 32, 3, value=True)
    assert torch.equal(ki, eki) and torch.equal(vi, evi)
    assert torch.equal(kc, ek) and torch.equal(vc, ev)


@pytest.mark.parametrize("t,count", [(8156, 32), (333, 64), (64, 64), (17, 1)])
def test_library_linspace_init_equals_explicit_centres(device, t, count):
    """Initial centres gathered by the library (reskv_linspace_rows on the
    device) give exactly the run from the same tokens passed as fp32 centres,
    for K, V and the paired sequence."""
    from reskv_amd._extension import load_extension

    ops = load_extension("compression")
    k, v, _ = outlier_kv(1, 4, t, seed=53)
    rows_k, rows_v = (x.reshape(4, t, 128).contiguous() for x in (k, v))
    idx = torch.from_numpy(o.linspace_indices(t, count)).to(device)
    init_k, init_v = rows_k[:, idx].float(), rows_v[:, idx].float()
    for rows, init, value in ((rows_k, init_k, False), (rows_v, init_v, True)):
        got = ops.kmeans(rows, None, 3, value, count)
        want = ops.kmeans(rows, init, 3, value)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
    got = ops.kmeans_kv(rows_k, rows_v, None, None, 3, count)
    want = ops.kmeans_kv(rows_k, rows_v, init_k, init_v, 3)
    for g, w in zip(got, want):
        assert torch.equal(g[0], w[0]) and torch.equal(g[1], w[1])
