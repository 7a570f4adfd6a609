"""HIP k-means vs the float64 oracle.

Assignments must be equal wherever the oracle's nearest/second-nearest margin
exceeds fp32 rounding; centres agree within fp16 rounding of the member mean.
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


@pytest.mark.parametrize("value", [False, True])
def test_single_iteration_matches_oracle(device, value):
    x, _, _ = outlier_kv(1, 4, 1000, seed=21) if not value else (None, None, None)
    if value:
        _, x, _ = outlier_kv(1, 4, 1000, seed=22)
    centers, ids = cluster(x, 32, 1, value=value)
    ec, eids, _ = o.kmeans(np_(x), 32, 1, value=value)
    data = np_(x).astype(np.float64).reshape(4, 1000, 128)
    init = data[:, o.linspace_indices(1000, 32)]
    _, margin = o.assign(data, init)
    _tie_free_equal(np_(ids).reshape(4, -1), eids.reshape(4, -1), margin, data, init)
    if np.array_equal(np_(ids), eids):
        ref = ec.astype(np.float64)
        got = np_(centers).astype(np.float64)
        assert np.abs(got - ref).max() <= 2e-3 * max(1.0, np.abs(ref).max())


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
    assert margin > 100.0
    assert np.array_equal(np_(ids), eids)
    assert np.abs(np_(centers).astype(np.float64) - ec.astype(np.float64)).max() <= 4e-3


@pytest.mark.parametrize("count", [1, 32])
def test_value_cluster_mean_does_not_overflow(device, count):
    # known answer of reskv tests/test_cuda.py:161-169
    data = torch.full((1, 1, 8192, 128), 20.0, device=device, dtype=torch.float16)
    centers, assignments = cluster(data, count=count, iterations=2, value=True)
    assert torch.isfinite(centers).all()
    restored = centers.gather(2, assignments.long().unsqueeze(-1).expand_as(data))
    assert torch.equal(restored, data)


def test_short_input_key_clustering(device):
    x = torch.randn(1, 2, 5, 128, device=device).half()
    centers, ids = cluster(x, 8, 3)
    assert centers.shape == (1, 2, 8, 128) and torch.isfinite(centers).all()
    assert int(ids.min()) >= 0 and int(ids.max()) < 8
    vc, vi = cluster(x, 8, 3, value=True)  # V caps the count at T
    assert vc.shape == (1, 2, 5, 128)


def test_incremental_cluster_matches_oracle(device):
    g = seeded(8)
    x = torch.randn(2, 2, 64, 128, generator=g).half().to(device)
    c = torch.randn(2, 2, 20, 128, generator=g).half().to(device)
    cfg = ResKVKernelConfig(num_clusters=20, max_clusters=21)
    c2, ids = _incremental_cluster(x, c, cfg)
    ec, eids, _ = o.incremental_cluster(np_(x), np_(c), 21)
    assert c2.shape[2] == 21
    assert np.abs(np_(c2).astype(np.float64) - ec.astype(np.float64)).max() <= 1e-3
    data = np_(x).astype(np.float64).reshape(4, 64, 128)
    cen = np_(c2).astype(np.float64).reshape(4, 21, 128)
    _, margin = o.assign(data, cen)
    _tie_free_equal(np_(ids).reshape(4, -1), eids.reshape(4, -1), margin, data, cen)
    c3, _ = _incremental_cluster(x, c2, cfg)  # at the cap: no new centre
    assert c3.shape[2] == 21


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
