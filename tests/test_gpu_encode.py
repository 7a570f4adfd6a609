"""HIP residual encoders vs the oracle: bit-exact payloads, metadata, codes and scales."""

import numpy as np
import pytest
import torch

from oracle import reskv_oracle as o
from tests.gpu_helpers import np_, outlier_kv, seeded

pytestmark = pytest.mark.gpu


def _case(kind, b, h, t, c, seed, device):
    g = seeded(seed)
    if kind == "normal":
        x = torch.randn(b, h, t, 128, generator=g).half()
        cen = (torch.randn(b, h, c, 128, generator=g) * 0.1).half()
    elif kind == "ties":  # coarse grid -> many equal |fp16(r)|
        x = (torch.randint(-4, 5, (b, h, t, 128), generator=g).float() * 0.25).half()
        cen = (torch.randint(-2, 3, (b, h, c, 128), generator=g).float() * 0.25).half()
    elif kind == "zeros":  # r == 0 everywhere: all-tie selection, zero scales
        x = torch.zeros(b, h, t, 128).half()
        cen = torch.zeros(b, h, c, 128).half()
    else:  # outlier channels (config-0 distribution)
        x, _, _ = outlier_kv(b, h, t, seed, device="cpu")
        cen = (torch.randn(b, h, c, 128, generator=g) * 0.5).half()
    ids = torch.randint(c, (b, h, t), generator=g, dtype=torch.int32)
    if kind == "normal":
        ids[..., :3] = torch.tensor([-5, c, c + 7], dtype=torch.int32)  # clamped, as the reference does
    return x.to(device), cen.to(device), ids.to(device)


KINDS = ["normal", "ties", "zeros", "outliers"]


@pytest.fixture(scope="module")
def ext(device):
    from reskv_amd._extension import load_extension

    return load_extension("compression")


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("nnz", [64, 32, 1, 127, 128])
def test_bitmap_encoder(ext, device, kind, nnz):
    x, c, ids = _case(kind, 2, 3, 77, 5, 1, device)
    payload, meta = ext.compress_bitmap(x, c, ids, nnz)
    ep, em = o.encode_bitmap(np_(x), np_(c), np_(ids), nnz)
    assert np.array_equal(np_(meta), em)
    assert np.array_equal(np_(payload).view(np.uint16), ep.view(np.uint16))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("nnz,struct", [(64, False), (32, True), (32, False), (16, False)])
def test_qtile_encoder(ext, device, kind, nnz, struct):
    x, c, ids = _case(kind, 1, 4, 131, 7, 2, device)
    payload, meta = ext.compress_fp16(x, c, ids, nnz, struct)
    ep, em = o.encode_qtile(np_(x), np_(c), np_(ids), nnz, struct)
    assert np.array_equal(np_(meta), em)
    assert np.array_equal(np_(payload).view(np.uint16), ep.view(np.uint16))


@pytest.mark.parametrize("kind", KINDS)
def test_struct_int4_encoder(ext, device, kind):
    x, c, ids = _case(kind, 2, 2, 65, 3, 3, device)
    qp, qm, qs = ext.compress_structured_int4(x, c, ids)
    ep, em, es = o.encode_struct_int4(np_(x), np_(c), np_(ids))
    assert np.array_equal(np_(qm), em)
    assert np.array_equal(np_(qs).view(np.uint16), es.view(np.uint16))
    assert np.array_equal(np_(qp), ep)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("nnz", [64, 32])
def test_multibit_encoder(ext, device, kind, bits, nnz):
    x, c, ids = _case(kind, 1, 3, 90, 4, 4, device)
    qt, qs = ext.compress_quantized(x, c, ids, nnz, bits)
    et, es = o.encode_multibit(np_(x), np_(c), np_(ids), nnz, bits)
    assert np.array_equal(np_(qs).view(np.uint16), es.view(np.uint16))
    assert np.array_equal(np_(qt), et)


def test_encoders_at_config1_scale_round_trip(ext, device):
    """Config 1 shape (B=1, 8 heads, T=8192): structured and bitmap encoders on outlier K;
    the oracle reconstruction of the HIP output keeps exactly the top residuals."""
    x, _, _ = outlier_kv(1, 8, 8192, 11)
    g = seeded(12)
    c = (torch.randn(1, 8, 32, 128, generator=g) * 0.5).half().to(device)
    ids = torch.randint(32, (1, 8, 8192), generator=g, dtype=torch.int32).to(device)
    p, m = ext.compress_fp16(x, c, ids, 32, True)
    ep, em = o.encode_qtile(np_(x), np_(c), np_(ids), 32, True)
    assert np.array_equal(np_(m), em) and np.array_equal(np_(p).view(np.uint16), ep.view(np.uint16))
    p, m = ext.compress_bitmap(x, c, ids, 32)
    ep, em = o.encode_bitmap(np_(x), np_(c), np_(ids), 32)
    assert np.array_equal(np_(m), em) and np.array_equal(np_(p).view(np.uint16), ep.view(np.uint16))


@pytest.mark.parametrize("t", [77, 300])
@pytest.mark.parametrize("fmt,nnz,struct", [("bitmap", 64, None), ("bitmap", 32, None), ("bitmap", 24, None),
                                            ("tile", 32, True), ("tile", 32, False), ("tile", 64, False)])
def test_kv_encoders_equal_single_tensor_calls(ext, device, t, fmt, nnz, struct):
    """K and V in one launch (different data, 5 and 3 centroids) give exactly the two single calls' results."""
    k, kc, ki = _case("normal", 2, 3, t, 5, 3, device)
    v, vc, vi = _case("ties", 2, 3, t, 3, 4, device)
    if fmt == "bitmap":
        pair = ext.compress_bitmap_kv(k, kc, ki, v, vc, vi, nnz)
        single = (ext.compress_bitmap(k, kc, ki, nnz), ext.compress_bitmap(v, vc, vi, nnz))
    else:
        pair = ext.compress_fp16_kv(k, kc, ki, v, vc, vi, nnz, struct)
        single = (ext.compress_fp16(k, kc, ki, nnz, struct), ext.compress_fp16(v, vc, vi, nnz, struct))
    for got, want in zip(pair, single):
        for a, b in zip(got, want):
            assert torch.equal(a, b)


def test_encoder_rejects_bad_inputs(ext, device):
    x = torch.zeros(1, 1, 4, 128, dtype=torch.float16, device=device)
    c = torch.zeros(1, 1, 2, 128, dtype=torch.float16, device=device)
    ids = torch.zeros(1, 1, 4, dtype=torch.int32, device=device)
    with pytest.raises(RuntimeError, match="int32"):
        ext.compress_fp16(x, c, ids.long(), 32, True)
    with pytest.raises(RuntimeError, match="4:16"):
        ext.compress_fp16(x, c, ids, 64, True)
    with pytest.raises(RuntimeError, match="float16"):
        ext.compress_bitmap(x.float(), c, ids, 32)
    with pytest.raises(RuntimeError, match="identical shapes"):
        ext.compress_bitmap_kv(x, c, ids, x[:, :, :2].contiguous(), c, ids[:, :, :2].contiguous(), 32)


def test_layouts_have_different_selection_semantics(device):
    """75% unstructured and 75% structured keep the same number of values per
    token (32) but select different ones: global top-32 against the top 4 of
    every 16-channel tile (reskv tests/test_cuda.py:92-97).  (The bit-exact
    checks of each encoder against its oracle are the tests above.)"""
    from reskv_amd import ResKVKernelConfig, compress
    from tests.gpu_helpers import dense, reference_test_inputs

    k, v, _, c = reference_test_inputs(t=64)
    u = compress(k, v, ResKVKernelConfig(bits=16, sparsity=0.75, layout="unstructured"), clustering=c)
    s = compress(k, v, ResKVKernelConfig(bits=16, sparsity=0.75, layout="structured"), clustering=c)
    assert u.key.payload.shape[-1] == s.key.payload.shape[-1] == 32
    du, ds = dense(u.key), dense(s.key)
    assert not np.array_equal(du, ds)
    # every structured tile keeps exactly four channels; the unstructured rows do not
    kept_s = (ds - dense_centroids(s.key)) != 0
    kept_u = (du - dense_centroids(u.key)) != 0
    assert (kept_s.reshape(*kept_s.shape[:-1], 8, 16).sum(-1) <= 4).all()
    assert (kept_u.reshape(*kept_u.shape[:-1], 8, 16).sum(-1) > 4).any()


def dense_centroids(ct):
    """Each token's centroid row (float64 [B, H, T, 128])."""
    cent = np_(ct.centroids).astype(np.float64)
    ids = np_(ct.cluster_ids).astype(np.int64)
    return np.take_along_axis(cent, ids[..., None].repeat(128, -1), axis=2)
