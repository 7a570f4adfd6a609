"""Writes the golden fixtures of this directory from the CPU oracle.

Run from the repository root: ``python tests/golden/make_fixtures.py``.
Every fixture is data only (inputs and expected outputs, ``.npz`` without
pickles); the tests load them with ``numpy.load(allow_pickle=False)``.

* ``encoders.npz``: one K-like input (config-0 outlier channels) and one
  V-like input, B=1, H=2, T=64, with centroids and ids, and the oracle's
  payload / metadata / codes / scales for every residual format.
* ``decode.npz``: a compressed cache per format (the encoder outputs above),
  one decode query per query head (GQA 4), RoPE theta 500000 at position 5000
  with start position 4, a dense recent window of 12 rotated tokens, and the
  float64 attention output of the oracle.
"""

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import reskv_oracle as o  # noqa: E402

HERE = Path(__file__).resolve().parent
B, H, T, C, G = 1, 2, 64, 16, 4
POSITION, START, TR = 5000, 4, 12


def inputs(seed):
    rng = np.random.default_rng(seed)
    scale = np.exp(rng.standard_normal((1, H, 1, 128)))
    for h in range(H):
        scale[0, h, 0, rng.permutation(128)[:4]] *= 10.0
    k = (rng.standard_normal((B, H, T, 128)) * scale).astype(np.float16)
    v = rng.standard_normal((B, H, T, 128)).astype(np.float16)
    kc = (rng.standard_normal((B, H, C, 128)) * scale * 0.5).astype(np.float16)
    vc = (rng.standard_normal((B, H, C, 128)) * 0.3).astype(np.float16)
    ki = rng.integers(0, C, (B, H, T)).astype(np.int32)
    vi = rng.integers(0, C, (B, H, T)).astype(np.int32)
    q = rng.standard_normal((B, H * G, 1, 128)).astype(np.float16)
    return k, v, kc, vc, ki, vi, q


def encode_all(x, c, ids, prefix, out):
    for nnz in (64, 32):
        p, m = o.encode_bitmap(x, c, ids, nnz)
        out[f"{prefix}_bitmap{nnz}_payload"], out[f"{prefix}_bitmap{nnz}_meta"] = p, m
    p, m = o.encode_qtile(x, c, ids, 64, struct_index=False)
    out[f"{prefix}_tiled64_payload"], out[f"{prefix}_tiled64_meta"] = p, m
    p, m = o.encode_qtile(x, c, ids, 32, struct_index=True)
    out[f"{prefix}_struct32_payload"], out[f"{prefix}_struct32_meta"] = p, m
    p, m, s = o.encode_struct_int4(x, c, ids)
    out[f"{prefix}_sint4_payload"], out[f"{prefix}_sint4_meta"], out[f"{prefix}_sint4_scale"] = p, m, s
    for bits in (4, 2):
        for nnz in (64, 32):
            w, s = o.encode_multibit(x, c, ids, nnz, bits)
            out[f"{prefix}_q{bits}n{nnz}_payload"], out[f"{prefix}_q{bits}n{nnz}_scale"] = w, s


# (fixture key, oracle reconstruct format, bits)
DECODE_FORMATS = (("bitmap64", "bitmap", 16), ("bitmap32", "bitmap", 16), ("tiled64", "tiled", 16),
                  ("struct32", "structured", 16), ("sint4", "struct_int4", 4), ("q4n64", "quant", 4),
                  ("q2n64", "quant", 2))


def dense_of(enc, prefix, key, fmt, bits, c, ids):
    meta = enc.get(f"{prefix}_{key}_meta")
    scale = enc.get(f"{prefix}_{key}_scale")
    return o.reconstruct(fmt, c, ids, enc[f"{prefix}_{key}_payload"], meta, scale, bits=bits)


def main():
    k, v, kc, vc, ki, vi, q = inputs(2024)
    enc = {"k": k, "v": v, "kc": kc, "vc": vc, "ki": ki, "vi": vi}
    encode_all(k, kc, ki, "k", enc)
    encode_all(v, vc, vi, "v", enc)
    np.savez_compressed(HERE / "encoders.npz", **enc)

    rng = np.random.default_rng(7)
    freq = o.theta_frequencies(500000.0)
    qr = o.rotate(q.astype(np.float64), np.array([POSITION]), freq).astype(np.float16)
    kr = o.rotate(rng.standard_normal((B, H, TR, 128)), np.arange(POSITION - TR, POSITION), freq).astype(np.float16)
    vr = rng.standard_normal((B, H, TR, 128)).astype(np.float16)
    dec = {"q": q, "q_rot": qr, "k_recent": kr, "v_recent": vr,
           "position": np.int64(POSITION), "start": np.int64(START)}
    for key, fmt, bits in DECODE_FORMATS:
        kd = dense_of(enc, "k", key, fmt, bits, kc, ki)
        vd = dense_of(enc, "v", key, fmt, bits, vc, vi)
        dec[f"{key}_out"] = o.reference_attention(q, kd, vd, position=POSITION, start_position=START, freq=freq)
        dec[f"{key}_out_recent"] = o.reference_attention(q, kd, vd, position=POSITION, start_position=START,
                                                         freq=freq, recent=(qr, kr, vr))
    np.savez_compressed(HERE / "decode.npz", **dec)
    print("wrote", HERE / "encoders.npz", HERE / "decode.npz")


if __name__ == "__main__":
    main()
