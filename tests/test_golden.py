"""The oracle reproduces the committed golden fixtures exactly (CPU).

The fixtures in tests/golden/ were written by tests/golden/make_fixtures.py
from the oracle; this regression test regenerates them in memory and
requires bit-identical arrays, so a change to the oracle cannot silently move
the targets the GPU parity tests compare against.
"""

import importlib.util
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def _maker():
    spec = importlib.util.spec_from_file_location("make_fixtures", GOLDEN / "make_fixtures.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_encoder_fixtures_are_reproduced_bit_exactly():
    mk = _maker()
    k, v, kc, vc, ki, vi, _ = mk.inputs(2024)
    enc = {}
    mk.encode_all(k, kc, ki, "k", enc)
    mk.encode_all(v, vc, vi, "v", enc)
    with np.load(GOLDEN / "encoders.npz", allow_pickle=False) as ref:
        for name in ("k", "v", "kc", "vc", "ki", "vi"):
            assert np.array_equal(ref[name], {"k": k, "v": v, "kc": kc, "vc": vc, "ki": ki, "vi": vi}[name])
        for key, val in enc.items():
            assert ref[key].dtype == val.dtype and np.array_equal(ref[key].view(np.uint8), val.view(np.uint8)), key


@pytest.mark.parametrize("key,fmt,bits", [f for f in _maker().DECODE_FORMATS])
def test_decode_fixtures_are_reproduced(key, fmt, bits):
    mk = _maker()
    from oracle import reskv_oracle as o

    with np.load(GOLDEN / "encoders.npz", allow_pickle=False) as enc, \
            np.load(GOLDEN / "decode.npz", allow_pickle=False) as dec:
        e = {n: enc[n] for n in enc.files}
        kd = mk.dense_of(e, "k", key, fmt, bits, e["kc"], e["ki"])
        vd = mk.dense_of(e, "v", key, fmt, bits, e["vc"], e["vi"])
        out = o.reference_attention(dec["q"], kd, vd, position=int(dec["position"]),
                                    start_position=int(dec["start"]), freq=o.theta_frequencies(500000.0))
        assert np.array_equal(out, dec[f"{key}_out"])


def test_fixture_residuals_round_trip():
    """Decoded fixtures keep exactly the selected fp16 residuals (closed form)."""
    from oracle import reskv_oracle as o

    with np.load(GOLDEN / "encoders.npz", allow_pickle=False) as e:
        r, key = o.residual_keys(e["k"], e["kc"], e["ki"])
        dense = o.reconstruct("bitmap", e["kc"], e["ki"], e["k_bitmap64_payload"], e["k_bitmap64_meta"])
        cent = o.reconstruct("bitmap", e["kc"], e["ki"], np.zeros_like(e["k_bitmap64_payload"]),
                             np.zeros_like(e["k_bitmap64_meta"]))
        kept = dense - cent
        nz = kept != 0
        assert (nz.sum(-1) <= 64).all()
        assert np.array_equal(kept[nz], o.f16(r)[nz].astype(np.float64))
