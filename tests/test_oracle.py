"""Pins the CPU oracle (oracle/reskv_oracle.py) with checks that do not restate it.

Each check is chosen so that a plausible mistake in the restatement (wrong bit
order, wrong tie rule, dropped centroid term, transposed rotation, wrong
rounding point) fails: brute-force selection, hand-computed packed words,
exact round trips, closed-form attention cases, RoPE identities, k-means
fixed-point properties and torch's own linspace.
"""

import itertools

import numpy as np
import pytest

from oracle import reskv_oracle as o


def _inputs(residual, seed=0, c_scale=0.0):
    """x, centroids, ids such that f32(x) - f32(c[id]) == residual exactly (one token row)."""
    r = np.asarray(residual, dtype=np.float16)[None, None, None, :]
    c = np.zeros((1, 1, 1, 128), dtype=np.float16)
    ids = np.zeros((1, 1, 1), dtype=np.int64)
    return r, c, ids


# ---------------------------------------------------------------------------
# selection
# ---------------------------------------------------------------------------

def _brute_force_top(key, k):
    """The unique k-subset S with key_i > key_j or (== and i < j) for i in S, j not in S."""
    n = len(key)
    found = []
    for subset in itertools.combinations(range(n), k):
        s = set(subset)
        ok = all(key[i] > key[j] or (key[i] == key[j] and i < j) for i in s for j in range(n) if j not in s)
        if ok:
            found.append(s)
    assert len(found) == 1
    return found[0]


@pytest.mark.parametrize("k", [1, 2, 4, 8])
def test_top_mask_matches_brute_force_with_ties(k):
    rng = np.random.default_rng(k)
    for _ in range(6):
        key = rng.integers(0, 4, 16).astype(np.float32)  # many ties
        mask = o.top_mask(key[None], k)[0]
        assert set(np.flatnonzero(mask)) == _brute_force_top(key, k)


def test_selection_uses_fp16_rounded_magnitude():
    # 1.0 and 1.0 + 2^-12 tie after fp16 rounding, so the lower channel wins
    res = np.zeros(128, dtype=np.float32)
    res[5] = 1.0
    res[9] = 1.0 + 2.0 ** -12
    x = np.zeros((1, 1, 1, 128), dtype=np.float16)
    c = (-res).astype(np.float16)[None, None, None, :]
    ids = np.zeros((1, 1, 1), dtype=np.int64)
    r, key = o.residual_keys(x, c, ids)
    assert key[0, 0, 0, 5] == key[0, 0, 0, 9]
    _, meta = o.encode_bitmap(x, c, ids, 1)
    assert meta.view(np.uint64)[0, 0, 0, 0] == np.uint64(1) << np.uint64(63 - 5)


def test_cluster_ids_are_clamped():
    x = np.ones((1, 1, 2, 128), dtype=np.float16)
    c = np.stack([np.zeros(128), np.full(128, 0.5)]).astype(np.float16)[None, None]
    r_hi, _ = o.residual_keys(x, c, np.array([[[7, -3]]]))
    assert np.all(r_hi[0, 0, 0] == 0.5) and np.all(r_hi[0, 0, 1] == 1.0)


# ---------------------------------------------------------------------------
# packing known answers
# ---------------------------------------------------------------------------

def test_bitmap_words_are_msb_first():
    res = np.arange(1, 129, dtype=np.float32)  # strictly increasing magnitude
    x, c, ids = _inputs(res)
    payload, meta = o.encode_bitmap(x, c, ids, 64)
    words = meta.view(np.uint64)[0, 0, 0]
    assert words[0] == 0 and words[1] == np.uint64(0xFFFFFFFFFFFFFFFF)
    assert np.array_equal(payload[0, 0, 0].astype(np.float32), res[64:])
    res2 = np.zeros(128, dtype=np.float32)
    res2[[0, 3, 64, 127]] = [4, 3, 2, 1]
    x, c, ids = _inputs(res2)
    payload, meta = o.encode_bitmap(x, c, ids, 4)
    words = meta.view(np.uint64)[0, 0, 0]
    assert words[0] == (np.uint64(1) << np.uint64(63)) | (np.uint64(1) << np.uint64(60))
    assert words[1] == (np.uint64(1) << np.uint64(63)) | np.uint64(1)
    assert payload[0, 0, 0].tolist() == [4, 3, 2, 1]  # ascending channel order


def test_qtile_words_and_tile_major_payload():
    res = np.tile(np.arange(1, 17, dtype=np.float32), 8) * np.repeat(np.arange(1, 9), 16)
    x, c, ids = _inputs(res)
    payload, meta = o.encode_qtile(x, c, ids, 32, struct_index=False)
    w = meta.view(np.uint32)[0, 0, 0]
    assert np.all(w == np.uint32(0xF000F000))  # channels 12..15 of each 16-channel tile
    payload_s, meta_s = o.encode_qtile(x, c, ids, 32, struct_index=True)
    ws = meta_s.view(np.uint32)[0, 0, 0]
    assert np.all(ws == np.uint32(0xFEDCFEDC))  # nibbles 12, 13, 14, 15 ascending
    expected = np.concatenate([res[16 * t + 12: 16 * t + 16] for t in range(8)])
    assert np.array_equal(payload.astype(np.float32)[0, 0, 0], expected)
    assert np.array_equal(payload_s, payload)
    # tile 1 keeps a different set: channels 0, 2 -> mask bits 0 and 2 in the high half
    res3 = np.zeros(128, dtype=np.float32)
    res3[16 + 0], res3[16 + 2] = 5, 6
    x, c, ids = _inputs(res3)
    _, meta3 = o.encode_qtile(x, c, ids, 16, struct_index=False)
    assert meta3.view(np.uint32)[0, 0, 0, 0] >> 16 == 0b101


def test_struct_int4_known_answer():
    res = np.zeros(128, dtype=np.float32)
    res[1] = 7.0           # subgroup 0 keeps channel 1
    res[4 * 17 + 3] = -3.5  # subgroup 17 keeps channel 3
    x, c, ids = _inputs(res)
    qp, qm, qs = o.encode_struct_int4(x, c, ids)
    s = np.float32(7.0) * (np.float32(1) / np.float32(7))
    assert qs[0, 0, 0] == np.float16(s)
    m = qm.view(np.uint32)[0, 0, 0]
    assert m[0] == 1 and m[1] == np.uint32(3 << 2)  # subgroup 17 -> word 1, bits 2..3
    p = qp.view(np.uint32)[0, 0, 0]
    assert p[0] & 0xF == 7
    # -3.5 / 1.0 rounds half to even -> -4 -> nibble 0xC at compact index 17 (word 2, nibble 1)
    assert (p[2] >> 4) & 0xF == 0xC


def test_zero_residual_quantisers():
    x, c, ids = _inputs(np.zeros(128, dtype=np.float32))
    qp, qm, qs = o.encode_struct_int4(x, c, ids)
    assert qs[0, 0, 0] == np.float16(1) and not qp.any() and not qm.any()
    for bits in (2, 4):
        qt, sc = o.encode_multibit(x, c, ids, 64, bits)
        assert sc[0, 0, 0] == np.float16(1) and not qt.any()


@pytest.mark.parametrize("bits", [2, 4])
def test_multibit_codes_and_dequantisation(bits):
    rng = np.random.default_rng(bits)
    x = (rng.standard_normal((1, 2, 32, 128)) * 2).astype(np.float16)
    c = (rng.standard_normal((1, 2, 4, 128)) * 0.2).astype(np.float16)
    ids = rng.integers(0, 4, (1, 2, 32))
    qmax = (1 << (bits - 1)) - 1
    qt, sc = o.encode_multibit(x, c, ids, 64, bits)
    rec = o.reconstruct("quant", c, ids, qt, None, sc, bits=bits)
    r, key = o.residual_keys(x, c, ids)
    mask = o.top_mask(key, 64)
    cent = rec - np.where(mask, 0, 0)  # full reconstruction
    base = np.take_along_axis(c.astype(np.float64), ids[..., None].repeat(128, -1), -2)
    codes = (rec - base) / sc.astype(np.float64)[..., None]
    assert np.allclose(codes, np.rint(codes)) and np.abs(codes).max() <= qmax
    assert np.all(codes[~mask] == 0)
    amax = np.where(mask, np.abs(r), 0).max(-1)
    step = sc.astype(np.float64)
    bound = 0.5 * step + np.maximum(amax - qmax * step, 0)
    err = np.abs((rec - base) - np.where(mask, r, 0)).max(-1)
    assert np.all(err <= bound + 1e-7)
    assert cent.shape == x.shape


def test_multibit_known_answer_uses_the_fp16_scale():
    """Hand-computed INT4 codes (compression.cu:339-360).

    amax = 1.0, so the scale is fp16(1/7) = 0.142822265625 (10-bit mantissa
    146).  Channel 5 holds r = 1.5 * 0.142822265625 = 0.2142333984375 (fp16,
    mantissa 731): divided by the fp16 scale it is exactly 1.5, which rounds
    half-to-even to 2.  Divided by the unrounded fp32 quotient 1/7 it is
    1.4996..., which rounds to 1, so a restatement that skips the fp16
    rounding point fails here.  The second token has amax = 0.875, so its
    scale is exactly 0.125; channel 9 holds 0.3125, 2.5 steps, which
    half-to-even rounds to 2 (half-away-from-zero would give 3).
    """
    res = np.zeros((2, 128), dtype=np.float32)
    res[0, 0] = 1.0
    res[0, 5] = 0.2142333984375
    res[0, 7] = -0.2142333984375
    res[1, 3] = 0.875                      # amax = 7 * 0.125: scale exactly 0.125
    res[1, 9] = 0.3125                     # 2.5 steps
    res[1, 11] = -0.3125
    x = res.astype(np.float16)[None, None]
    c = np.zeros((1, 1, 1, 128), dtype=np.float16)
    ids = np.zeros((1, 1, 2), dtype=np.int64)
    qt, sc = o.encode_multibit(x, c, ids, 64, 4)
    assert sc[0, 0, 0] == np.float16(0.142822265625) and sc[0, 0, 1] == np.float16(0.125)
    assert np.float16(0.142822265625).view(np.uint16) == 0x3092
    words = qt.view(np.uint32)[0, 0]
    nib = lambda t, d: int((words[t, d // 8] >> np.uint32(4 * (d % 8))) & np.uint32(15))
    assert nib(0, 0) == 7 and nib(0, 5) == 2 and nib(0, 7) == (-2 & 15)
    assert nib(1, 3) == 7 and nib(1, 9) == 2 and nib(1, 11) == (-2 & 15)
    # every other channel is 0 (kept zeros and dropped channels alike)
    others = [(t, d) for t in range(2) for d in range(128) if (t, d) not in
              {(0, 0), (0, 5), (0, 7), (1, 3), (1, 9), (1, 11)}]
    assert all(nib(t, d) == 0 for t, d in others)


# ---------------------------------------------------------------------------
# reconstruction round trips
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("fmt,nnz", [("bitmap", 64), ("bitmap", 32), ("tiled", 64), ("structured", 32)])
def test_fp16_round_trip_is_exact(fmt, nnz):
    rng = np.random.default_rng(nnz)
    x = rng.standard_normal((2, 2, 24, 128)).astype(np.float16)
    c = (rng.standard_normal((2, 2, 5, 128)) * 0.3).astype(np.float16)
    ids = rng.integers(0, 5, (2, 2, 24))
    if fmt == "bitmap":
        payload, meta = o.encode_bitmap(x, c, ids, nnz)
    else:
        payload, meta = o.encode_qtile(x, c, ids, nnz, struct_index=(fmt == "structured"))
    rec = o.reconstruct(fmt, c, ids, payload, meta)
    r, key = o.residual_keys(x, c, ids)
    base = np.take_along_axis(c.astype(np.float64), ids[..., None].repeat(128, -1), -2)
    kept = (rec - base) != 0
    assert np.array_equal(rec - base, np.where(kept, o.f16(r).astype(np.float64), 0))
    if fmt == "bitmap":
        assert np.all(kept.sum(-1) <= nnz)
        lo = np.where(kept, key, np.inf).min(-1)
        hi = np.where(kept, -np.inf, key).max(-1)
        assert np.all(lo >= hi)
    else:
        tiles = kept.reshape(*kept.shape[:-1], 8, 16)
        assert np.all(tiles.sum(-1) <= nnz // 8)


def test_struct_int4_round_trip():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((1, 3, 40, 128)).astype(np.float16)
    c = (rng.standard_normal((1, 3, 6, 128)) * 0.3).astype(np.float16)
    ids = rng.integers(0, 6, (1, 3, 40))
    qp, qm, qs = o.encode_struct_int4(x, c, ids)
    rec = o.reconstruct("struct_int4", c, ids, qp, qm, qs)
    base = np.take_along_axis(c.astype(np.float64), ids[..., None].repeat(128, -1), -2)
    res = (rec - base).reshape(1, 3, 40, 32, 4)
    assert np.all((res != 0).sum(-1) <= 1)  # at most one channel per subgroup
    r, key = o.residual_keys(x, c, ids)
    best = key.reshape(1, 3, 40, 32, 4).argmax(-1)
    chosen = np.abs(res).argmax(-1)
    nonzero = (res != 0).any(-1)
    assert np.all(chosen[nonzero] == best[nonzero])


# ---------------------------------------------------------------------------
# RoPE and attention
# ---------------------------------------------------------------------------

def test_rotate_identities():
    rng = np.random.default_rng(1)
    f = o.theta_frequencies(500000.0)
    x = rng.standard_normal((3, 128))
    y = o.rotate(x, np.array([0, 5, 100]), f)
    assert np.allclose(y[0], x[0])
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1))
    assert np.allclose(o.rotate(o.rotate(x, np.array([7, 7, 7]), f), np.array([-7, -7, -7]), f), x)
    # rotate-half pairing: channel d pairs with d + 64 at frequency d
    e = np.zeros(128)
    e[3] = 1.0
    z = o.rotate(e, np.array([1]), f)[0]
    ang = np.float64(np.float32(1.0) * f[3])
    assert np.isclose(z[3], np.cos(ang)) and np.isclose(z[67], np.sin(ang))
    # relative position: <R(a)q, R(b)k> depends on a - b (exact for small integer angles)
    q, k = rng.standard_normal(128), rng.standard_normal(128)
    ones = np.ones(64, dtype=np.float32)
    d1 = o.rotate(q, np.array([3]), ones)[0] @ o.rotate(k, np.array([1]), ones)[0]
    d2 = o.rotate(q, np.array([12]), ones)[0] @ o.rotate(k, np.array([10]), ones)[0]
    assert np.isclose(d1, d2)


def test_theta_frequencies():
    f = o.theta_frequencies(10000.0)
    assert f[0] == 1.0 and np.isclose(f[32], 10000.0 ** -0.5, rtol=1e-6)


def test_attention_closed_forms():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((1, 4, 1, 128))
    v = rng.standard_normal((1, 1, 1, 128))
    k = rng.standard_normal((1, 1, 1, 128))
    out = o.reference_attention(q, k, v, position=5)
    assert np.allclose(out, np.broadcast_to(v, out.shape))
    # identical keys -> uniform weights -> mean of the values, for every head
    k2 = np.repeat(rng.standard_normal((1, 2, 1, 128)), 0, axis=2)
    kk = np.zeros((1, 2, 9, 128))
    vv = rng.standard_normal((1, 2, 9, 128))
    q2 = rng.standard_normal((1, 8, 1, 128))
    out2 = o.reference_attention(q2, kk, vv, position=20)
    assert k2.shape[2] == 0
    assert np.allclose(out2[:, :4, 0], vv[:, 0].mean(1)) and np.allclose(out2[:, 4:, 0], vv[:, 1].mean(1))


def test_attention_matches_explicit_softmax_and_stats():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((2, 8, 1, 128))
    k = rng.standard_normal((2, 2, 17, 128))
    v = rng.standard_normal((2, 2, 17, 128))
    f = o.theta_frequencies(500000.0) / np.linspace(1, 8, 64).astype(np.float32)
    out = o.reference_attention(q, k, v, position=40, start_position=3, freq=f, scaling=0.1)
    qr = o.rotate(q, np.array([40]), f)
    kr = o.rotate(k, np.arange(3, 20), f)
    for b in range(2):
        for h in range(8):
            s = kr[b, h // 4] @ qr[b, h, 0] * 0.1
            p = np.exp(s - s.max())
            p /= p.sum()
            assert np.allclose(out[b, h, 0], p @ v[b, h // 4])
    so, m, l = o.compressed_stats(q, k, v, position=40, start_position=3, freq=f, scaling=0.1)
    assert np.allclose(so, out[:, :, 0])
    s0 = kr[0, 0] @ qr[0, 0, 0] * 0.1
    assert np.isclose(m[0, 0], s0.max()) and np.isclose(l[0, 0], np.exp(s0 - s0.max()).sum())


def test_merge_recent_of_exact_statistics_equals_the_joint_softmax():
    """merge_recent (attention.cu:598-663) restated: joining the unrounded
    compressed (out, m, l) with recent tokens is the softmax over all tokens;
    with no recent token it returns the compressed result."""
    rng = np.random.default_rng(11)
    q = rng.standard_normal((2, 8, 1, 128))
    k = rng.standard_normal((2, 2, 23, 128)) * 2.0
    v = rng.standard_normal((2, 2, 23, 128))
    kr_ = rng.standard_normal((2, 2, 9, 128)) * 3.0
    vr_ = rng.standard_normal((2, 2, 9, 128))
    f = o.theta_frequencies(500000.0)
    qr = o.rotate(q, np.array([40]), f)
    full = o.reference_attention(q, k, v, position=40, start_position=5, freq=f, recent=(qr, kr_, vr_))
    co, m, l = o.compressed_stats(q, k, v, position=40, start_position=5, freq=f)
    krr, vrr = np.repeat(kr_, 4, axis=1), np.repeat(vr_, 4, axis=1)
    scores = (qr @ np.swapaxes(krr, -1, -2))[..., 0, :] * 128 ** -0.5
    got = o.merge_recent(co, m, l, scores, vrr)
    assert np.abs(got - full[:, :, 0]).max() < 1e-12
    assert np.array_equal(o.merge_recent(co, m, l, scores[..., :0], vrr[:, :, :0]), co)


def test_attention_with_recent_equals_concatenation():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, 4, 1, 128))
    k = rng.standard_normal((1, 1, 10, 128))
    v = rng.standard_normal((1, 1, 10, 128))
    kr_ = rng.standard_normal((1, 1, 5, 128))
    vr_ = rng.standard_normal((1, 1, 5, 128))
    f = o.theta_frequencies(500000.0)
    qr = o.rotate(q, np.array([30]), f)
    out = o.reference_attention(q, k, v, position=30, freq=f, recent=(qr, kr_, vr_))
    kall = np.concatenate((o.rotate(k, np.arange(10), f), kr_), axis=2)
    vall = np.concatenate((v, vr_), axis=2)
    s = kall[0, 0] @ qr[0, 2, 0] * 128 ** -0.5
    p = np.exp(s - s.max())
    assert np.allclose(out[0, 2, 0], (p / p.sum()) @ vall[0, 0])


# ---------------------------------------------------------------------------
# k-means
# ---------------------------------------------------------------------------

def test_linspace_indices_match_torch():
    torch = pytest.importorskip("torch")
    for t in (1, 2, 33, 65, 960, 1000, 8192, 16384):
        for c in (1, 7, 31, 32, 64):
            if t >= c:
                assert np.array_equal(o.linspace_indices(t, c), torch.linspace(0, t - 1, c).long().numpy())


@pytest.mark.parametrize("value", [False, True])
def test_kmeans_fixed_point_properties(value):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((1, 2, 200, 128)).astype(np.float16)
    centers, ids, _ = o.kmeans(x, 8, 4, value=value)
    assert centers.shape == (1, 2, 8, 128) and ids.shape == (1, 2, 200)
    # ids are the exact argmin against the pre-update centres: recompute by running one step fewer
    prev_centers, prev_ids, _ = o.kmeans(x, 8, 3, value=value)
    data = x.astype(np.float64).reshape(2, 200, 128)
    # the last assignment is against the centres after 3 updates (kept in fp64 by the oracle)
    assert prev_ids.shape == ids.shape
    # the returned centres are the member means of the returned ids (fp16 rounded)
    for bh in range(2):
        for cidx in range(8):
            members = data[bh][ids.reshape(2, 200)[bh] == cidx]
            if len(members):
                assert np.allclose(centers.reshape(2, 8, 128)[bh, cidx], members.mean(0), atol=2e-3)
            elif value:
                assert not centers.reshape(2, 8, 128)[bh, cidx].any()


@pytest.mark.parametrize("count", [1, 32])
def test_kmeans_constant_data_is_exact(count):
    # known answer of reskv tests/test_cuda.py:161-169
    x = np.full((1, 1, 512, 128), 20.0, dtype=np.float16)
    centers, ids, _ = o.kmeans(x, count, 2, value=True)
    restored = np.take_along_axis(centers, ids[..., None].astype(np.int64).repeat(128, -1), -2)
    assert np.array_equal(restored, x)


def test_kmeans_ids_are_argmin_with_lowest_index_ties():
    data = np.zeros((1, 3, 128))
    data[0, 1, 0] = 1.0
    data[0, 2, 0] = 0.5  # equidistant from centres 0 and 1
    cen = np.zeros((1, 2, 128))
    cen[0, 1, 0] = 1.0
    ids, margin = o.assign(data, cen)
    assert ids.tolist() == [[0, 1, 0]] and margin[0, 2] == 0


def test_incremental_cluster_appends_mean_until_cap():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((1, 1, 16, 128)).astype(np.float16)
    c = rng.standard_normal((1, 1, 3, 128)).astype(np.float16)
    c2, ids, _ = o.incremental_cluster(x, c, max_clusters=4)
    assert c2.shape[2] == 4 and np.allclose(c2[0, 0, 3], x[0, 0].astype(np.float32).mean(0), atol=1e-3)
    c3, _, _ = o.incremental_cluster(x, c2, max_clusters=4)
    assert c3.shape[2] == 4


# ---------------------------------------------------------------------------
# V k-means arithmetic, pinned against CPU torch's own ops
# ---------------------------------------------------------------------------

def _torch():
    return pytest.importorskip("torch")


def test_fp16_sqrt_is_correctly_rounded_for_every_half():
    h = np.arange(0, 0x7C01, dtype=np.uint16).view(np.float16)  # 0 .. +inf
    got = o._fp16_sqrt(h).astype(np.float64)
    exact = np.sqrt(h.astype(np.float64))
    up = np.nextafter(got.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    dn = np.nextafter(got.astype(np.float16), np.float16(0)).astype(np.float64)
    finite = np.isfinite(exact)
    # nearest: the exact root lies within half an ulp on both sides
    with np.errstate(invalid="ignore"):
        assert np.all(np.abs(exact - got)[finite] <= np.maximum(up - got, got - dn)[finite] / 2)
    torch = _torch()
    t = torch.from_numpy(h.copy()).clamp_min(0).sqrt()
    assert np.array_equal(t.numpy().view(np.uint16), got.astype(np.float16).view(np.uint16))


def test_half_norms_match_torch():
    torch = _torch()
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((3, 500, 128)) * rng.lognormal(0, 1, (1, 1, 128))).astype(np.float16)
    ref = torch.from_numpy(x).pow(2).sum(-1).numpy()
    got = o.half_norms(x)
    amb = o._midpoint_distance(o._half_norm_exact(x), 2.0 ** -20)
    assert np.array_equal(got[~amb], ref[~amb]) and amb.mean() < 0.01


@pytest.mark.parametrize("scale", [1.0, 4.0])
def test_value_distances_match_torch_cdist(scale):
    """The restated V distance equals CPU torch's fp16 cdist (mm formulation)
    bit for bit wherever the token is not flagged, and so do the ids; the
    exact-distance rule does not (it differs on ~0.5% of ids)."""
    torch = _torch()
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((4, 2000, 128)) * scale).astype(np.float16)
    c = x[:, o.linspace_indices(2000, 32)]
    ref = torch.cdist(torch.from_numpy(x), torch.from_numpy(c), compute_mode="use_mm_for_euclid_dist")
    s16, _ = o.value_distances(x, c)
    amb = o.value_ambiguous(x, c)
    assert amb.mean() < 0.01
    ref_ids = ref.float().argmin(-1).numpy()
    ids = o.assign_value(x, c)
    assert np.array_equal(ids[~amb], ref_ids[~amb])
    assert (s16 == ref.numpy()).mean() > 0.999
    exact_ids, _ = o.assign(x.astype(np.float64), c.astype(np.float64))
    assert (exact_ids != ref_ids).mean() > 0.001  # the K rule would not pin V


def test_value_ties_take_the_lowest_index():
    """Two different fp16 squared distances with one fp16 root: the lower
    index wins although its squared distance is larger."""
    x = np.zeros((1, 1, 128), dtype=np.float16)
    c = np.zeros((1, 3, 128), dtype=np.float16)
    c[0, 0, 1], c[0, 0, 2] = 16.0, 0.5   # |x - c|^2 = 256.25 -> sqrt 16.0078... rounds to 16
    c[0, 1, 0] = 16.0                    # 256 -> 16
    c[0, 2, 3] = 16.015625               # 256.5 -> 16.0156 (next fp16): farther
    s16, d = o.value_distances(x, c)
    assert d[0, 0, 0] == 256.25 and d[0, 0, 1] == 256.0
    assert s16[0, 0, 0] == s16[0, 0, 1] == np.float16(16)
    assert o.assign_value(x, c)[0, 0] == 0
    exact_ids, _ = o.assign(x.astype(np.float64), c.astype(np.float64))
    assert exact_ids[0, 0] == 1


def test_incremental_value_rule_matches_torch_expression():
    torch = _torch()
    rng = np.random.default_rng(13)
    x = rng.standard_normal((2, 4, 64, 128)).astype(np.float16)
    c = rng.standard_normal((2, 4, 21, 128)).astype(np.float16)
    tx, tc = torch.from_numpy(x), torch.from_numpy(c)
    dist = (tx ** 2).sum(-1, keepdim=True) + (tc ** 2).sum(-1).unsqueeze(2)   # compression.py:63
    dist = dist - 2 * torch.matmul(tx.float(), tc.float().transpose(-2, -1))   # compression.py:64
    d = o.incremental_value_distances(x, c)
    assert np.abs(d - dist.double().numpy()).max() <= 1e-4
    assert np.array_equal(np.argmin(d, -1), dist.argmin(-1).numpy())
    c2, ids, _ = o.incremental_cluster(x, c, 22, value=True)
    assert np.array_equal(c2[:, :, 21], tx.mean(2).numpy())                       # compression.py:60
    d2 = o.incremental_value_distances(x, c2)
    assert np.array_equal(ids, np.argmin(d2, -1))


@pytest.mark.parametrize("value", [False, True])
def test_update_centres_matches_one_hot_product(value):
    torch = _torch()
    rng = np.random.default_rng(14)
    x = rng.standard_normal((2, 300, 128)).astype(np.float16)
    ids = rng.integers(0, 7, (2, 300))       # cluster 7 stays empty
    prev = rng.standard_normal((2, 8, 128))
    got = o.update_centres(x.astype(np.float64), ids, prev, 8, value=value)
    tx = torch.from_numpy(x).float()
    oh = torch.nn.functional.one_hot(torch.from_numpy(ids), 8).float()
    counts = oh.sum(1).unsqueeze(-1)
    sums = torch.bmm(oh.transpose(1, 2), tx)
    if value:
        ref = (sums / counts.clamp_min(1)).half().double().numpy()
        assert np.abs(got - ref).max() <= 2 ** -10 and not got[:, 7].any()
    else:
        ref = torch.where(counts > 0, sums / counts.clamp_min(1), torch.from_numpy(prev).float()).double().numpy()
        assert np.abs(got - ref).max() <= 1e-6 and np.array_equal(got[:, 7], prev[:, 7])
