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
