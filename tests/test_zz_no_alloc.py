"""reskv_decode_recent_noalloc (split-K partials in the library's own device
array) against reskv_decode_recent (partials in a caller workspace), called
through the C ABI: bitwise equal outputs on consecutive calls, the second with
a smaller input, with and without a recent window."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import reskv_oracle as o
from reskv_amd import ResKVKernelConfig, compress
from reskv_amd import _lib
from reskv_amd._extension import _rope, cache_descriptors
from tests.gpu_helpers import ATOL, expected_attention, np_, outlier_kv, theta_freq

pytestmark = pytest.mark.gpu


def _case(device, b, h, t, sparsity, tr, seed):
    k, v, q = outlier_kv(b, h, t, seed=seed)
    cache = compress(k, v, ResKVKernelConfig(sparsity=sparsity, num_clusters=16))
    freq = theta_freq()
    pos = t + tr
    g = torch.Generator().manual_seed(seed + 1)
    kr = (torch.randn(b, h, max(tr, 1), 128, generator=g) * 2).half().to(device)
    vr = torch.randn(b, h, max(tr, 1), 128, generator=g).half().to(device)
    qr = torch.from_numpy(o.rotate(np_(q).astype(np.float64), np.array([pos]), np_(freq))).half().to(device)
    return cache, q, qr, kr, vr, freq, pos


def _call(noalloc, cache, q, qr, kr, vr, freq, pos, tr):
    b, h = cache.key.centroids.shape[:2]
    hq, t = q.shape[1], cache.seq_len
    kd, vd, keep = cache_descriptors(cache)
    f, table = _rope(freq, 500000.0, q.device, t)
    out = torch.full((b * hq, 128), float("nan"), dtype=torch.float16, device=q.device)
    L = _lib.lib()
    stream = torch.cuda.current_stream(q.device).cuda_stream
    args = (q.data_ptr(), ctypes.byref(kd), ctypes.byref(vd), f.data_ptr(), table.data_ptr(), b, hq, h, t, 0, pos,
            128 ** -0.5, 0, qr.data_ptr(), kr.data_ptr(), vr.data_ptr(), tr, kr.shape[2], out.data_ptr())
    if noalloc:
        _lib.check(L.reskv_decode_recent_noalloc(*args, stream), "decode_recent_noalloc")
    else:
        ws = torch.empty(L.reskv_decode_workspace_bytes(b, hq, h, t, 0), dtype=torch.uint8, device=q.device)
        _lib.check(L.reskv_decode_recent(*args, ws.data_ptr(), ws.numel(), stream), "decode_recent")
    torch.cuda.synchronize()
    return out.view(b, hq, 1, 128)


def test_noalloc_equals_workspace_entry_point_on_consecutive_calls(device):
    # first call: B = 4 at 50%, with a recent window; second: smaller, 75%, no window
    for (b, h, t, sp, tr, seed) in ((4, 2, 1536, 0.5, 40, 61), (1, 2, 600, 0.75, 0, 62)):
        cache, q, qr, kr, vr, freq, pos = _case(device, b, h, t, sp, tr, seed)
        ref = _call(False, cache, q, qr, kr, vr, freq, pos, tr)
        got = _call(True, cache, q, qr, kr, vr, freq, pos, tr)
        assert torch.equal(got, ref), (b, t, sp, tr)
        recent = (qr, kr[:, :, :tr], vr[:, :, :tr]) if tr else None
        exp = expected_attention(q, cache, position=pos, inv_freq=freq, recent=recent)
        assert float(np.abs(np_(got).astype(np.float64) - exp).max()) <= ATOL


def test_noalloc_rejects_sizes_beyond_its_scratch(device):
    cache, q, qr, kr, vr, freq, pos = _case(device, 1, 2, 256, 0.5, 0, 63)
    kd, vd, keep = cache_descriptors(cache)
    f, table = _rope(freq, 500000.0, q.device, 256)
    L = _lib.lib()
    # 256 explicit splits: B = 64 batch rows x 8 query heads x 256 splits x 776 B per split record
    # (13 MB) exceed the 8 MiB array
    status = L.reskv_decode_recent_noalloc(q.data_ptr(), ctypes.byref(kd), ctypes.byref(vd), f.data_ptr(),
                                           table.data_ptr(), 64, 8, 2, 256, 0, pos, 0.1, 256, None, None, None, 0,
                                           0, None, None)
    assert status != 0 and b"allocation-free" in L.reskv_last_error()
