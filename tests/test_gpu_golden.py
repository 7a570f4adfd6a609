"""HIP library against the committed golden fixtures (GPU).

Encoders: bit-exact payload, metadata, codes and scales.  Decode: max-abs
<= 2e-3 against the fixture's float64 attention output, with and without a
dense recent window, for every residual format.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from reskv_amd import attention
from reskv_amd._extension import load_extension
from reskv_amd.config import KernelPlan
from reskv_amd.tensors import CompressedKV, CompressedTensor
from tests.gpu_helpers import ATOL, np_

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"

PLANS = {
    "bitmap64": KernelPlan("unstructured", "deferred", 16, 64, 2, 0),
    "bitmap32": KernelPlan("unstructured", "deferred", 16, 32, 2, 0),
    "tiled64": KernelPlan("tiled", "per_token", 16, 64, 4, 0),
    "struct32": KernelPlan("structured", "deferred", 16, 32, 4, 20),
    "sint4": KernelPlan("structured", "deferred", 4, 32, 4, 20),
    "q4n64": KernelPlan("unstructured", "per_token", 4, 64, 16, 0),
    "q2n64": KernelPlan("unstructured", "per_token", 2, 64, 16, 0),
}


@pytest.fixture(scope="module")
def enc():
    with np.load(GOLDEN / "encoders.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture(scope="module")
def dec():
    with np.load(GOLDEN / "decode.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _t(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def _same(got, want):
    got = np_(got)
    assert got.dtype == want.dtype and got.shape == want.shape
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))


@pytest.mark.parametrize("side", ["k", "v"])
def test_encoders_match_fixtures_bit_exactly(device, enc, side):
    ext = load_extension("compression")
    x, c, ids = _t(enc[side], device), _t(enc[side + "c"], device), _t(enc[side + "i"], device)
    for nnz in (64, 32):
        p, m = ext.compress_bitmap(x, c, ids, nnz)
        _same(p, enc[f"{side}_bitmap{nnz}_payload"])
        _same(m, enc[f"{side}_bitmap{nnz}_meta"])
    p, m = ext.compress_fp16(x, c, ids, 64, False)
    _same(p, enc[f"{side}_tiled64_payload"])
    _same(m, enc[f"{side}_tiled64_meta"])
    p, m = ext.compress_fp16(x, c, ids, 32, True)
    _same(p, enc[f"{side}_struct32_payload"])
    _same(m, enc[f"{side}_struct32_meta"])
    p, m, s = ext.compress_structured_int4(x, c, ids)
    _same(p, enc[f"{side}_sint4_payload"])
    _same(m, enc[f"{side}_sint4_meta"])
    _same(s, enc[f"{side}_sint4_scale"])
    for bits in (4, 2):
        for nnz in (64, 32):
            w, s = ext.compress_quantized(x, c, ids, nnz, bits)
            _same(w, enc[f"{side}_q{bits}n{nnz}_payload"])
            _same(s, enc[f"{side}_q{bits}n{nnz}_scale"])


def _cache(enc, key, device):
    plan = PLANS[key]

    def one(side):
        meta = enc.get(f"{side}_{key}_meta")
        scale = enc.get(f"{side}_{key}_scale")
        return CompressedTensor(_t(enc[side + "c"], device), _t(enc[side + "i"], device),
                                _t(enc[f"{side}_{key}_payload"], device),
                                None if meta is None else _t(meta, device),
                                None if scale is None else _t(scale, device), plan)

    return CompressedKV(one("k"), one("v"))


@pytest.mark.parametrize("key", list(PLANS))
def test_decode_matches_fixtures(device, enc, dec, key):
    cache = _cache(enc, key, device)
    q = _t(dec["q"], device)
    freq = (500000.0 ** (-torch.arange(64, device=device).float() / 64)).float()
    pos, start = int(dec["position"]), int(dec["start"])
    out = attention(q, cache, position=pos, start_position=start, inv_freq=freq)
    err = np.abs(np_(out).astype(np.float64) - dec[f"{key}_out"]).max()
    assert err <= ATOL, f"{key}: max-abs {err:.3e}"
    recent = (_t(dec["q_rot"], device), _t(dec["k_recent"], device), _t(dec["v_recent"], device))
    out = attention(q, cache, position=pos, start_position=start, inv_freq=freq, recent=recent)
    err = np.abs(np_(out).astype(np.float64) - dec[f"{key}_out_recent"]).max()
    assert err <= ATOL, f"{key} with recent window: max-abs {err:.3e}"
