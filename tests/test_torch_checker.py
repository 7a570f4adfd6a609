"""The float32 torch checker (oracle/torch_checker.py) against the float64
golden vectors the numpy oracle wrote: every residual format, with and without
a dense recent window.  5e-4 covers float32 RoPE and sums; a wrong bit order,
index or rotation gives errors above 1e-2."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import torch_checker as tc
from reskv_amd.config import KernelPlan
from reskv_amd.tensors import CompressedKV, CompressedTensor

GOLDEN = Path(__file__).resolve().parent / "golden"
PLANS = {"bitmap64": KernelPlan("unstructured", "deferred", 16, 64, 2, 0),
         "bitmap32": KernelPlan("unstructured", "deferred", 16, 32, 2, 0),
         "tiled64": KernelPlan("tiled", "per_token", 16, 64, 4, 0),
         "struct32": KernelPlan("structured", "deferred", 16, 32, 4, 20),
         "sint4": KernelPlan("structured", "deferred", 4, 32, 4, 20),
         "q4n64": KernelPlan("unstructured", "per_token", 4, 64, 16, 0),
         "q2n64": KernelPlan("unstructured", "per_token", 2, 64, 16, 0)}


def _load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _tensor(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def _cache(enc, key):
    def side(s):
        meta, scale = enc.get(f"{s}_{key}_meta"), enc.get(f"{s}_{key}_scale")
        return CompressedTensor(_tensor(enc[s + "c"]), _tensor(enc[s + "i"]), _tensor(enc[f"{s}_{key}_payload"]),
                                None if meta is None else _tensor(meta), None if scale is None else _tensor(scale),
                                PLANS[key])
    return CompressedKV(side("k"), side("v"))


@pytest.mark.parametrize("key", sorted(PLANS))
def test_checker_matches_golden_attention(key):
    enc, dec = _load("encoders.npz"), _load("decode.npz")
    cache = _cache(enc, key)
    freq = (500000.0 ** (-torch.arange(64).float() / 64)).float()
    pos, start = int(dec["position"]), int(dec["start"])
    out = tc.attention(_tensor(dec["q"]), cache, position=pos, start_position=start, inv_freq=freq)
    assert np.abs(out.double().numpy() - dec[f"{key}_out"]).max() <= 5e-4
    recent = (_tensor(dec["q_rot"]), _tensor(dec["k_recent"]), _tensor(dec["v_recent"]))
    out = tc.attention(_tensor(dec["q"]), cache, position=pos, start_position=start, inv_freq=freq, recent=recent)
    assert np.abs(out.double().numpy() - dec[f"{key}_out_recent"]).max() <= 5e-4


@pytest.mark.parametrize("key", sorted(PLANS))
def test_checker_reconstruction_equals_the_oracle(key):
    from oracle import reskv_oracle as o

    enc = _load("encoders.npz")
    cache = _cache(enc, key)
    fmt = {"bitmap64": "bitmap", "bitmap32": "bitmap", "tiled64": "tiled", "struct32": "structured",
           "sint4": "struct_int4", "q4n64": "quant", "q2n64": "quant"}[key]
    bits = PLANS[key].bits
    for ct in (cache.key, cache.value):
        meta = None if ct.metadata is None else ct.metadata.numpy()
        scale = None if ct.scale is None else ct.scale.numpy()
        ref = o.reconstruct(fmt, ct.centroids.numpy(), ct.cluster_ids.numpy().astype(np.int64), ct.payload.numpy(),
                            meta, scale, bits=bits)
        got = tc.reconstruct(ct).double().numpy()
        assert np.abs(got - ref).max() <= 1e-6 * max(1.0, np.abs(ref).max())


# ---------------------------------------------------------------------------
# the torch restatement of compress (used only by bench.py's CPU baseline)
# ---------------------------------------------------------------------------

def _inputs(seed, b=1, h=2, t=300):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(b, h, t, 128, generator=g) * torch.exp(torch.randn(1, h, 1, 128, generator=g))).half()
    c = (torch.randn(b, h, 16, 128, generator=g) * 0.3).half()
    ids = torch.randint(16, (b, h, t), generator=g, dtype=torch.int32)
    return x, c, ids


@pytest.mark.parametrize("nnz", [64, 32])
def test_torch_bitmap_encoder_equals_the_oracle(nnz):
    from oracle import reskv_oracle as o

    x, c, ids = _inputs(1)
    p, m = tc.encode_bitmap(x, c, ids, nnz)
    ep, em = o.encode_bitmap(x.numpy(), c.numpy(), ids.numpy(), nnz)
    assert np.array_equal(p.numpy(), ep) and np.array_equal(m.numpy(), em)


def test_torch_structured_encoder_equals_the_oracle():
    from oracle import reskv_oracle as o

    x, c, ids = _inputs(2)
    p, m = tc.encode_structured(x, c, ids, 32)
    ep, em = o.encode_qtile(x.numpy(), c.numpy(), ids.numpy(), 32, True)
    assert np.array_equal(p.numpy(), ep) and np.array_equal(m.numpy(), em)


@pytest.mark.parametrize("bits", [4, 2])
def test_torch_multibit_encoder_equals_the_oracle(bits):
    from oracle import reskv_oracle as o

    x, c, ids = _inputs(3)
    q, s = tc.encode_multibit(x, c, ids, 64, bits)
    eq, es = o.encode_multibit(x.numpy(), c.numpy(), ids.numpy(), 64, bits)
    assert np.array_equal(s.numpy(), es)
    assert (q.numpy() == eq).mean() > 0.999  # torch.round and numpy rint agree except on fp32 division ties


@pytest.mark.parametrize("value", [False, True])
def test_torch_kmeans_equals_the_oracle(value):
    from oracle import reskv_oracle as o

    x, _, _ = _inputs(4, t=600)
    c, ids = tc.kmeans(x, 16, 3, value=value)
    ec, eids, _ = o.kmeans(x.numpy(), 16, 3, value=value)
    assert (ids.numpy() == eids).mean() > 0.995
    if np.array_equal(ids.numpy(), eids):
        assert np.abs(c.float().numpy() - ec.astype(np.float32)).max() <= 2e-2
