"""Seeded random sweep of the residual encoders against the oracle, bit for bit.

Each case draws B, KV heads, T (1 to 1000, partial 16-token waves included),
the centroid count (1 to 64), a data kind (Gaussian with out-of-range ids,
coarse-grid ties, all-zero residuals, config-0 outlier channels) and one
encoder with a valid width: the unstructured bitmap (nnz 1..128, also not a
multiple of 8), tiled / 4:16 FP16, structured INT4, INT4 / INT2 top-nnz, and
the one-launch K+V forms of the bitmap and tile encoders with different K and
V centroid counts.
"""

import random

import numpy as np
import pytest

from oracle import reskv_oracle as o
from tests.gpu_helpers import np_
from tests.test_gpu_encode import KINDS, _case

pytestmark = pytest.mark.gpu

ENCODERS = ["bitmap", "tile", "struct4", "sint4", "multibit", "bitmap_kv", "tile_kv"]
CHUNKS, PER_CHUNK = 4, 16


@pytest.fixture(scope="module")
def ext(device):
    from reskv_amd._extension import load_extension

    return load_extension("compression")


def _eq(a, b):
    a = np_(a)
    if a.dtype == np.float16:
        return np.array_equal(a.view(np.uint16), np.asarray(b).view(np.uint16))
    return np.array_equal(a, b)


def _check_bitmap(ext, x, c, ids, nnz):
    p, m = ext.compress_bitmap(x, c, ids, nnz)
    ep, em = o.encode_bitmap(np_(x), np_(c), np_(ids), nnz)
    return _eq(m, em) and _eq(p, ep)


def _check_tile(ext, x, c, ids, nnz, struct):
    p, m = ext.compress_fp16(x, c, ids, nnz, struct)
    ep, em = o.encode_qtile(np_(x), np_(c), np_(ids), nnz, struct)
    return _eq(m, em) and _eq(p, ep)


@pytest.mark.parametrize("chunk", range(CHUNKS))
def test_random_encoder_cases_against_the_oracle(ext, device, chunk):
    for index in range(chunk * PER_CHUNK, (chunk + 1) * PER_CHUNK):
        rnd = random.Random(4099 * index + 11)
        b, h = rnd.choice([1, 2, 3]), rnd.choice([1, 2, 5])
        t = rnd.choice([1, 5, 16, 17, 63, 64, 65, 200, 1000])
        c = rnd.choice([1, 3, 32, 64])
        kind = rnd.choice(KINDS)
        enc = rnd.choice(ENCODERS)
        x, cen, ids = _case(kind, b, h, t, c, 100 + index, device)
        desc = dict(index=index, enc=enc, kind=kind, b=b, h=h, t=t, c=c)
        if enc == "bitmap":
            nnz = rnd.choice([1, 7, 24, 32, 64, 100, 128])
            assert _check_bitmap(ext, x, cen, ids, nnz), (desc, nnz)
        elif enc == "tile":
            nnz = rnd.choice([16, 32, 64, 96, 120])
            assert _check_tile(ext, x, cen, ids, nnz, False), (desc, nnz)
        elif enc == "struct4":
            assert _check_tile(ext, x, cen, ids, 32, True), desc
        elif enc == "sint4":
            qp, qm, qs = ext.compress_structured_int4(x, cen, ids)
            ep, em, es = o.encode_struct_int4(np_(x), np_(cen), np_(ids))
            assert _eq(qm, em) and _eq(qs, es) and _eq(qp, ep), desc
        elif enc == "multibit":
            nnz, bits = rnd.choice([32, 64]), rnd.choice([4, 2])
            qt, qs = ext.compress_quantized(x, cen, ids, nnz, bits)
            et, es = o.encode_multibit(np_(x), np_(cen), np_(ids), nnz, bits)
            assert _eq(qs, es) and _eq(qt, et), (desc, nnz, bits)
        else:
            cv = rnd.choice([1, 3, 32, 64])
            v, vc, vi = _case(rnd.choice(KINDS), b, h, t, cv, 200 + index, device)
            if enc == "bitmap_kv":
                nnz = rnd.choice([8, 24, 32, 64, 96])
                (kp, km), (vp, vm) = ext.compress_bitmap_kv(x, cen, ids, v, vc, vi, nnz)
                ek, ekm = o.encode_bitmap(np_(x), np_(cen), np_(ids), nnz)
                ev, evm = o.encode_bitmap(np_(v), np_(vc), np_(vi), nnz)
            else:
                nnz, struct = rnd.choice([(32, True), (32, False), (64, False)])
                (kp, km), (vp, vm) = ext.compress_fp16_kv(x, cen, ids, v, vc, vi, nnz, struct)
                ek, ekm = o.encode_qtile(np_(x), np_(cen), np_(ids), nnz, struct)
                ev, evm = o.encode_qtile(np_(v), np_(vc), np_(vi), nnz, struct)
            assert _eq(km, ekm) and _eq(kp, ek) and _eq(vm, evm) and _eq(vp, ev), (desc, cv, nnz)
