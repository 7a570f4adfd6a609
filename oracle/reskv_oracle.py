"""CPU oracle for the ResKV compressed-KV hot path.  TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the reference algorithm of every stage the HIP
library implements.  It is imported only by ``tests/``, by
``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of ``bench.py`` --
always as the checker, never as the thing measured or shipped.  The product
path (``reskv_amd``) never imports it and fails loudly without the HIP
library.

Restated functions and the reference lines they follow (under
``/root/reference``):

* ``residual_keys``        -- compression.cu:80-94 (fp32 residual, |fp16(r)| key,
                              ids clamped to [0, C-1])
* ``encode_bitmap``        -- compression.py:75-89 (unstructured FP16; MSB-first
                              int64 bitmaps; payload ascending by channel)
* ``encode_qtile``         -- compression.cu:44-147 (tiled 16-bit masks or 4:16
                              four-nibble index codes, tile-major payload)
* ``encode_struct_int4``   -- compression.cu:153-239 (1-of-4 INT4, 2-bit codes)
* ``encode_multibit``      -- compression.cu:245-383 (top-nnz + symmetric
                              INT4/INT2 with an fp16 per-token scale)
* ``reconstruct``          -- reference.py:12-49
* ``rotate``               -- reference.py:52-56
* ``reference_attention``  -- reference.py:59-91
* ``merge_recent``         -- attention.cu:598-663, cluster_mass.cu:1106-1169
                              (joint softmax of an fp16 compressed result and
                              its (m, l) with recent tokens)
* ``kmeans``               -- compression.py:19-53 (Lloyd: linspace init,
                              assign-then-update, K keeps empty centres, V zeroes
                              them, ids from the last assignment)
* ``value_distances``      -- compression.py:27, 38 (V: fp16 ``cdist`` in the mm
                              formulation -- fp16 norms, one fp16 rounding of
                              the 130-term sum, fp16 sqrt)
* ``update_centres``       -- compression.py:40-52
* ``incremental_cluster``  -- compression.py:56-69 (V: fp16(|x|^2 + |c|^2) - 2 x.c
                              in fp32; group mean in fp16)

How each function is pinned (tests/test_oracle.py):

* selection (all encoders): brute force over every subset on tiny tiles, and
  the lowest-index tie rule on hand-made tie vectors;
* packing: hand-computed words for known masks / codes (bit order MSB-first for
  bitmaps, LSB-first for tile masks, nibble and 2-bit positions);
* quantisation: zero residual -> scale 1, all codes 0; codes bounded by QMAX;
  decode(code) * scale reproduces the kept residual within half a step; a
  hand-computed multibit code that only the fp16-rounded scale gives;
* reconstruct: encode -> reconstruct round trip equals centre + kept residual
  exactly, and the dropped channels are exactly the smallest |fp16(r)|;
* attention: dense softmax closed form (one token -> output equals its value,
  equal scores -> mean), RoPE identities (relative-position invariance, norm
  preservation, inverse rotation); ``merge_recent`` of the unrounded
  compressed statistics equals ``reference_attention`` over the concatenated
  tokens, and with no recent tokens returns the compressed result;
* k-means, K: ids are argmin of exact (float64) distances, centres are member
  means, linspace initial indices, the constant-data known answer of
  tests/test_cuda.py:161-169;
* k-means, V: ``value_distances`` / ``assign_value`` against CPU torch's own
  ``torch.cdist(..., compute_mode="use_mm_for_euclid_dist")`` on fp16 tensors
  (equal fp16 distances and ids away from the tokens ``value_ambiguous``
  flags); ``half_norms`` against ``x.pow(2).sum(-1)``; the incremental rule
  against the reference's expression evaluated by CPU torch; the fp16 square
  root against every fp16 input; ``update_centres`` against a one-hot fp32
  matrix product.

Parity unpinned: exact ``torch.topk`` tie order for unstructured K
(compression.py:82) -- this oracle fixes "lowest index wins" as the CUDA
encoders do.  The reference's fp32 accumulation order inside its GEMMs and
reductions is unknown; where an exact sum lies within fp32 rounding of an fp16
midpoint either rounding is possible, and ``value_ambiguous`` names those
tokens instead of choosing.
"""

import numpy as np

D = 128
HALF = 64


# ---------------------------------------------------------------------------
# shared helpers
# ---------------------------------------------------------------------------

def f16(x):
    """Round-to-nearest-even to fp16 (numpy casts are RNE)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def residual_keys(x, centroids, ids):
    """Residual r = f32(x) - f32(c[id]) and selection key |fp16(r)| (compression.cu:80-94).

    x: fp16 [..., T, 128]; centroids: fp16 [..., C, 128]; ids: int [..., T].
    Returns (r float32 [..., T, 128], key float32 [..., T, 128]).
    """
    x = np.asarray(x, dtype=np.float16)
    c = np.asarray(centroids, dtype=np.float16)
    ids = np.clip(np.asarray(ids).astype(np.int64), 0, c.shape[-2] - 1)
    cent = np.take_along_axis(c, ids[..., None].repeat(D, axis=-1), axis=-2)
    r = x.astype(np.float32) - cent.astype(np.float32)
    key = np.abs(f16(r).astype(np.float32))
    return r, key


def top_mask(key, k):
    """Boolean mask of the k largest keys along the last axis; ties -> lower index.

    A stable sort of -key keeps equal keys in index order, which is exactly the
    comparison ``val > best || (val == best && i < best_i)`` of the reference
    encoders (compression.cu:107-113, 296-298).
    """
    order = np.argsort(-key, axis=-1, kind="stable")[..., :k]
    mask = np.zeros(key.shape, dtype=bool)
    np.put_along_axis(mask, order, True, axis=-1)
    return mask


def _gather_kept(values, mask, count):
    """Values at True positions of mask, ascending by position, as [..., count]."""
    flat_v = values.reshape(-1, values.shape[-1])
    flat_m = mask.reshape(-1, mask.shape[-1])
    out = flat_v[flat_m].reshape(flat_v.shape[0], count)
    return out.reshape(*values.shape[:-1], count)


# ---------------------------------------------------------------------------
# encoders
# ---------------------------------------------------------------------------

def encode_bitmap(x, centroids, ids, nnz):
    """Unstructured FP16 (compression.py:75-89).

    payload fp16 [..., T, nnz]: fp16(r) at the kept channels, ascending.
    meta int64 [..., T, 2]: channel d sets bit (63 - d % 64) of word d // 64.
    """
    r, key = residual_keys(x, centroids, ids)
    mask = top_mask(key, nnz)
    payload = f16(_gather_kept(r, mask, nnz))
    weights = (np.uint64(1) << np.arange(63, -1, -1, dtype=np.uint64))
    words = (mask.reshape(*mask.shape[:-1], 2, 64).astype(np.uint64) * weights).sum(-1, dtype=np.uint64)
    return payload, words.view(np.int64)


def encode_qtile(x, centroids, ids, nnz, struct_index):
    """Tiled / structured-4:16 FP16 (compression.cu:57-147).

    Each 16-channel tile keeps nnz/8 channels; payload fp16 [..., T, nnz] is
    tile-major and ascending inside a tile; meta int32 [..., T, 4] where word w
    holds code(tile 2w) | code(tile 2w+1) << 16.  A code is the 16-bit mask
    (bit i = channel i of the tile) or, with struct_index, the kept channels'
    in-tile indices as four ascending nibbles (rank r at bits 4r).
    """
    per_tile = nnz // 8
    r, key = residual_keys(x, centroids, ids)
    tiles = key.reshape(*key.shape[:-1], 8, 16)
    mask = top_mask(tiles, per_tile)                       # [..., 8, 16]
    flat_mask = mask.reshape(*mask.shape[:-2], D)
    payload = f16(_gather_kept(r, flat_mask, nnz))
    bits = (mask.astype(np.uint32) << np.arange(16, dtype=np.uint32)).sum(-1, dtype=np.uint32)
    if struct_index:
        pos = np.sort(np.argsort(-tiles, axis=-1, kind="stable")[..., :per_tile], axis=-1)
        codes = (pos.astype(np.uint32) << (4 * np.arange(per_tile, dtype=np.uint32))).sum(-1, dtype=np.uint32)
    else:
        codes = bits
    words = codes[..., 0::2] | (codes[..., 1::2] << np.uint32(16))
    return payload, words.astype(np.uint32).view(np.int32)


def encode_struct_int4(x, centroids, ids):
    """Structured 1-of-4 INT4 (compression.cu:153-239).

    Returns qpacked int32 [..., T, 4], qmeta int32 [..., T, 2], qscale fp16 [..., T].
    Subgroup i (channels 4i..4i+3) keeps its largest |fp16(r)| (ties -> lower);
    its 2-bit position goes to bits 2*(i % 16) of meta word i // 16.  The scale
    is s = amax * fl32(1/7) in fp32 (1 when amax == 0), stored as fp16(s); the
    code is rn(r / s) in fp32 clamped to [-7, 7], nibble i % 8 of word i // 8.
    """
    r, key = residual_keys(x, centroids, ids)
    groups = key.reshape(*key.shape[:-1], 32, 4)
    sel = np.argmax(groups, axis=-1)                       # first max -> lower index
    rg = r.reshape(*r.shape[:-1], 32, 4)
    compact = np.take_along_axis(rg, sel[..., None], axis=-1)[..., 0].astype(np.float32)
    meta = np.zeros((*sel.shape[:-1], 2), dtype=np.uint32)
    for i in range(32):
        meta[..., i // 16] |= sel[..., i].astype(np.uint32) << np.uint32(2 * (i % 16))
    amax = np.abs(compact).max(-1)
    inv7 = np.float32(1.0) / np.float32(7.0)
    s = np.where(amax > 0, (amax * inv7).astype(np.float32), np.float32(1.0)).astype(np.float32)
    q = np.rint(compact / s[..., None]).astype(np.int64)
    q = np.clip(q, -7, 7)
    nib = (q & 0xF).astype(np.uint32)
    packed = np.zeros((*q.shape[:-1], 4), dtype=np.uint32)
    for i in range(32):
        packed[..., i // 8] |= nib[..., i] << np.uint32(4 * (i % 8))
    return packed.view(np.int32), meta.view(np.int32), f16(s)


def encode_multibit(x, centroids, ids, nnz, bits):
    """Unstructured top-nnz + symmetric INT4/INT2 (compression.cu:245-383).

    Returns qtiles int32 [..., T, 4*bits] and qscale fp16 [..., T].  The scale
    is fp16(amax / QMAX) (fp16(1) when amax == 0); codes are
    clamp(rint(r / float(scale)), -QMAX, QMAX) for kept channels and 0 for the
    rest; channel d lands in word d // (32/bits) at bit (d % (32/bits)) * bits.
    """
    qmax = (1 << (bits - 1)) - 1
    per_word = 32 // bits
    r, key = residual_keys(x, centroids, ids)
    mask = top_mask(key, nnz)
    amax = np.where(mask, np.abs(r), np.float32(0)).max(-1).astype(np.float32)
    scale = np.where(amax > 0, f16(amax / np.float32(qmax)), np.float16(1.0))
    sf = scale.astype(np.float32)[..., None]
    q = np.clip(np.rint(r / sf), -qmax, qmax).astype(np.int64)
    q = np.where(mask, q, 0)
    code = (q & ((1 << bits) - 1)).astype(np.uint32)
    code = code.reshape(*code.shape[:-1], D // per_word, per_word)
    shifts = (np.arange(per_word, dtype=np.uint32) * np.uint32(bits))
    words = (code << shifts).sum(-1, dtype=np.uint32)
    return words.view(np.int32), scale


# ---------------------------------------------------------------------------
# reconstruction and attention
# ---------------------------------------------------------------------------

def reconstruct(fmt, centroids, ids, payload, meta=None, scale=None, bits=16):
    """Dense float64 K or V from a compressed tensor (reference.py:12-49).

    fmt: 'bitmap' | 'tiled' | 'structured' | 'struct_int4' | 'quant'.
    """
    ids = np.asarray(ids).astype(np.int64)
    cent = np.take_along_axis(
        np.asarray(centroids, dtype=np.float16).astype(np.float64),
        ids[..., None].repeat(D, axis=-1), axis=-2)
    lead = ids.shape
    res = np.zeros((*lead, D), dtype=np.float64)
    if fmt == "quant":
        per_word = 32 // bits
        words = np.asarray(payload).view(np.uint32).astype(np.uint64)
        shifts = np.arange(per_word, dtype=np.uint64) * np.uint64(bits)
        q = ((words[..., None] >> shifts) & np.uint64((1 << bits) - 1)).reshape(*lead, D).astype(np.int64)
        sign = 1 << (bits - 1)
        q = (q ^ sign) - sign
        res = q.astype(np.float64) * np.asarray(scale).astype(np.float64)[..., None]
    elif fmt == "bitmap":
        w = np.asarray(meta).view(np.uint64)
        d = np.arange(D)
        sel = ((w[..., d // 64] >> (np.uint64(63) - (d % 64).astype(np.uint64))) & np.uint64(1)).astype(bool)
        rank = np.cumsum(sel, axis=-1) - 1
        vals = np.take_along_axis(np.asarray(payload).astype(np.float64), np.clip(rank, 0, None), axis=-1)
        res = np.where(sel, vals, 0.0)
    elif fmt == "struct_int4":
        words = np.asarray(payload).view(np.uint32).astype(np.uint64)
        q = ((words[..., None] >> (np.arange(8, dtype=np.uint64) * np.uint64(4))) & np.uint64(15))
        q = q.reshape(*lead, 32).astype(np.int64)
        q = ((q ^ 8) - 8).astype(np.float64) * np.asarray(scale).astype(np.float64)[..., None]
        m = np.asarray(meta).view(np.uint32).astype(np.uint64)
        local = ((m[..., None] >> (np.arange(16, dtype=np.uint64) * np.uint64(2))) & np.uint64(3))
        dims = local.reshape(*lead, 32).astype(np.int64) + np.arange(32) * 4
        np.put_along_axis(res, dims, q, axis=-1)
    elif fmt in ("tiled", "structured"):
        m = np.asarray(meta).view(np.uint32).astype(np.uint64)
        codes = ((m[..., None] >> np.array([0, 16], dtype=np.uint64)) & np.uint64(0xFFFF)).reshape(*lead, 8)
        pay = np.asarray(payload).astype(np.float64)
        if fmt == "structured":
            idx = ((codes[..., None] >> (np.arange(4, dtype=np.uint64) * np.uint64(4))) & np.uint64(15))
            dims = idx.astype(np.int64) + (np.arange(8) * 16)[:, None]
            np.put_along_axis(res, dims.reshape(*lead, 32), pay, axis=-1)
        else:
            bit = ((codes[..., None] >> np.arange(16, dtype=np.uint64)) & np.uint64(1)).astype(bool)
            sel = bit.reshape(*lead, D)
            rank = np.cumsum(sel, axis=-1) - 1
            vals = np.take_along_axis(pay, np.clip(rank, 0, None), axis=-1)
            res = np.where(sel, vals, 0.0)
    else:
        raise ValueError(f"unknown format {fmt}")
    return cent + res


def theta_frequencies(theta):
    """theta ** (-arange(64) / 64) in fp32, as reference.py:73-77 computes it."""
    return (np.float32(theta) ** (-np.arange(64, dtype=np.float32) / np.float32(64))).astype(np.float32)


def rotate(x, positions, freq):
    """Rotate-half RoPE with fp32 angles fl(pos * freq) (reference.py:52-56).

    The angle is formed exactly as the reference does (an fp32 product); its
    cosine and sine are then evaluated in float64, so the oracle carries no
    trigonometric error of its own.
    """
    pos = np.asarray(positions, dtype=np.float32)
    ang = (pos[..., None] * np.asarray(freq, dtype=np.float32)).astype(np.float32).astype(np.float64)
    cos, sin = np.cos(ang), np.sin(ang)
    x = np.asarray(x, dtype=np.float64)
    a, b = x[..., :HALF], x[..., HALF:]
    return np.concatenate((a * cos - b * sin, b * cos + a * sin), axis=-1)


def softmax_stats(scores):
    m = scores.max(-1, keepdims=True)
    e = np.exp(scores - m)
    return m[..., 0], e.sum(-1), e


def reference_attention(q, k_dense, v_dense, *, position, start_position=0, freq=None,
                        rope_theta=500000.0, scaling=None, recent=None):
    """Decode attention of raw q over reconstructed pre-RoPE K and V (reference.py:59-91).

    q: [B, Hq, 1, 128]; k_dense, v_dense: float [B, Hk, T, 128] (pre-RoPE K);
    recent: optional (q_rot [B,Hq,1,128], k_rot [B,Hk,Tr,128], v [B,Hk,Tr,128]).
    Returns float64 [B, Hq, 1, 128].
    """
    b, hk, t, _ = k_dense.shape
    hq = q.shape[1]
    g = hq // hk
    f = theta_frequencies(rope_theta) if freq is None else np.asarray(freq, dtype=np.float32)
    qr = rotate(np.asarray(q, dtype=np.float64), np.array([position]), f)
    kr = rotate(k_dense, np.arange(start_position, start_position + t), f)
    kr = np.repeat(kr, g, axis=1)
    v = np.repeat(np.asarray(v_dense, dtype=np.float64), g, axis=1)
    scale = 128 ** -0.5 if scaling is None else scaling
    scores = np.matmul(qr, np.swapaxes(kr, -1, -2)) * scale
    if recent is not None:
        q_r, k_r, v_r = (np.asarray(z, dtype=np.float64) for z in recent)
        k_r = np.repeat(k_r, g, axis=1)
        scores = np.concatenate((scores, np.matmul(q_r, np.swapaxes(k_r, -1, -2)) * scale), axis=-1)
        v = np.concatenate((v, np.repeat(v_r, g, axis=1)), axis=2)
    scores = scores - scores.max(-1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(-1, keepdims=True)
    return np.matmul(p, v)


def compressed_stats(q, k_dense, v_dense, *, position, start_position=0, freq=None,
                     rope_theta=500000.0, scaling=None):
    """(out, m, l) of the compressed part alone: m = max score, l = sum exp(s - m).

    These are the statistics the decode ops return next to the normalised
    output (cluster_mass.cu:1090-1103, attention.cu:590-595).
    """
    b, hk, t, _ = k_dense.shape
    hq = q.shape[1]
    g = hq // hk
    f = theta_frequencies(rope_theta) if freq is None else np.asarray(freq, dtype=np.float32)
    qr = rotate(np.asarray(q, dtype=np.float64), np.array([position]), f)
    kr = np.repeat(rotate(k_dense, np.arange(start_position, start_position + t), f), g, axis=1)
    v = np.repeat(np.asarray(v_dense, dtype=np.float64), g, axis=1)
    scale = 128 ** -0.5 if scaling is None else scaling
    s = (np.matmul(qr, np.swapaxes(kr, -1, -2)) * scale)[..., 0, :]
    m, l, e = softmax_stats(s)
    out = np.einsum("bht,bhtd->bhd", e, v) / l[..., None]
    return out, m, l


def merge_recent(comp_out, comp_m, comp_l, scores, v_recent):
    """Joint softmax of a compressed result with recent tokens (float64).

    comp_out [B, Hq, 128] (the decode op's normalised output, which the
    reference stores in fp16 before this step), comp_m / comp_l [B, Hq] (max
    score and sum of exp(s - m) of the compressed part), scores [B, Hq, Tr]
    (scaled recent scores), v_recent [B, Hq, Tr, 128] (already repeated over
    the query group).  The reference accumulates comp_out * l and each recent
    token's weighted value with online rescaling and divides by the joint
    normaliser (attention.cu:598-663; the deferred family's merge_recent,
    cluster_mass.cu:1106-1169, takes the same inputs with precomputed scores);
    in exact arithmetic that is
        (comp_out l e^(m - M) + sum_t e^(s_t - M) v_t) / (l e^(m - M) + sum_t e^(s_t - M)),
    M = max(m, max_t s_t), evaluated here directly.
    """
    out = np.asarray(comp_out, dtype=np.float64)
    m = np.asarray(comp_m, dtype=np.float64)
    l = np.asarray(comp_l, dtype=np.float64)
    s = np.asarray(scores, dtype=np.float64)
    if s.shape[-1] == 0:
        return out.copy()
    big = np.maximum(m, s.max(-1))
    wc = l * np.exp(m - big)
    e = np.exp(s - big[..., None])
    num = out * wc[..., None] + np.einsum("bht,bhtd->bhd", e, np.asarray(v_recent, dtype=np.float64))
    return num / (wc + e.sum(-1))[..., None]


# ---------------------------------------------------------------------------
# k-means
# ---------------------------------------------------------------------------

def linspace_indices(t, count):
    """torch.linspace(0, t-1, count).long() evaluated as torch does in fp32.

    torch fills the first half as start + i*step and the second half as
    end - (count-1-i)*step with a fused multiply-add (one fp32 rounding of the
    exact result), step = fl32((end - start) / (count - 1)), then truncates
    toward zero.
    """
    if count == 1:
        return np.zeros(1, dtype=np.int64)
    start, end = np.float32(0), np.float32(t - 1)
    step = np.float64((end - start) / np.float32(count - 1))
    i = np.arange(count)
    half = count // 2
    lo = (np.float64(start) + i * step).astype(np.float32)
    hi = (np.float64(end) - (count - 1 - i) * step).astype(np.float32)
    vals = np.where(i < half, lo, hi)
    return np.trunc(vals).astype(np.int64)


def assign(data, centers):
    """Exact (float64) nearest centre with the lowest index on ties; also the margin.

    This is the K rule: ``cdist`` of fp32 data (compression.py:27, 38-39) whose
    mm formulation accumulates in fp32, so the reference's ids equal the exact
    ones wherever the margin exceeds fp32 rounding.
    Returns (ids [N], margin [N]) where margin = second-best minus best squared
    distance -- a small margin marks an assignment that fp32 rounding may flip.
    """
    x = np.asarray(data, dtype=np.float64)
    c = np.asarray(centers, dtype=np.float64)
    d2 = (x * x).sum(-1)[..., None] - 2.0 * x @ np.swapaxes(c, -1, -2) + (c * c).sum(-1)[..., None, :]
    ids = np.argmin(d2, axis=-1)
    srt = np.sort(d2, axis=-1)
    margin = srt[..., 1] - srt[..., 0] if d2.shape[-1] > 1 else np.full(ids.shape, np.inf)
    return ids, margin


def _half_norm_exact(a):
    """Exact sum of the fp16-rounded squares of fp16 rows (float64; a*a is exact there)."""
    a = np.asarray(a, dtype=np.float16).astype(np.float64)
    return (a * a).astype(np.float16).astype(np.float64).sum(-1)


def half_norms(a):
    """``a.pow(2).sum(-1)`` of fp16 rows as torch evaluates it: each square
    rounded to fp16, the sum accumulated in fp32 and rounded to fp16.  This
    restatement sums exactly and rounds once (the accumulation order only
    matters within fp32 rounding of a rounding midpoint)."""
    return _half_norm_exact(a).astype(np.float16)


def _fp16_sqrt(d16):
    """Correctly rounded fp16 square root of clamped fp16 values (torch's
    ``clamp_min_(0).sqrt_()`` on half; float64 sqrt then one rounding is exact
    here since 53 >= 2*11 + 2)."""
    return np.sqrt(np.maximum(np.asarray(d16, dtype=np.float64), 0.0)).astype(np.float16)


def value_distances(x, centers):
    """fp16 distances of ``torch.cdist(x, c, compute_mode="use_mm_for_euclid_dist")``
    on fp16 data (compression.py:27, 38).

    The mm formulation is one fp16 GEMM of [-2x, |x|^2, 1] against
    [c, 1, |c|^2]: the norms are fp16 (``half_norms``), the 130-term dot
    product accumulates in fp32 and is rounded to fp16, then clamped at zero
    and square-rooted in fp16.  This restatement forms the 130-term sum exactly
    and rounds it once.  Returns (s16 fp16 [..., N, C], exact pre-rounding
    squared distance float64 [..., N, C]).
    """
    x = np.asarray(x, dtype=np.float16)
    c = np.asarray(centers, dtype=np.float16)
    xn = half_norms(x).astype(np.float64)
    cn = half_norms(c).astype(np.float64)
    dot = x.astype(np.float64) @ np.swapaxes(c.astype(np.float64), -1, -2)
    d = xn[..., :, None] + cn[..., None, :] - 2.0 * dot
    with np.errstate(over="ignore"):  # beyond 65504 the fp16 distance is inf, as in torch
        return _fp16_sqrt(d.astype(np.float16)), d


def assign_value(x, centers):
    """V assignment: argmin over the fp16 distances, lowest index on ties
    (``argmin`` returns the first minimum)."""
    s16, _ = value_distances(x, centers)
    return np.argmin(s16.astype(np.float32), axis=-1)


def _midpoint_distance(v, rel):
    """True where an exact value v lies within rel * |v| of an fp16 rounding
    midpoint (so an fp32 accumulation of it may round to either neighbour)."""
    v = np.asarray(v, dtype=np.float64)
    h = v.astype(np.float16)
    up = np.nextafter(h, np.float16(np.inf)).astype(np.float64)
    dn = np.nextafter(h, np.float16(-np.inf)).astype(np.float64)
    hv = h.astype(np.float64)
    mids = np.stack(((hv + up) / 2, (hv + dn) / 2))
    return (np.abs(mids - v) <= rel * np.abs(v) + 1e-30).any(0)


def value_ambiguous(x, centers, rel=2.0 ** -20):
    """Tokens whose V id could differ from ``assign_value`` when the fp32
    accumulations of the reference (or of any other implementation) round
    differently from the exact sums: a 130-term distance or a norm within
    ``rel`` of an fp16 rounding midpoint.  A distance is taken as the interval
    of its two possible fp16 roundings; the token is unambiguous when the
    oracle's winner stays the lowest-indexed minimum over every choice."""
    x = np.asarray(x, dtype=np.float16)
    c = np.asarray(centers, dtype=np.float16)
    s16, d = value_distances(x, c)
    xs, cs = _half_norm_exact(x), _half_norm_exact(c)
    xamb = _midpoint_distance(xs, rel)                         # [..., N]
    camb = _midpoint_distance(cs, rel)                         # [..., C]
    scale = np.abs(x.astype(np.float64)) @ np.swapaxes(np.abs(c.astype(np.float64)), -1, -2)
    width = rel * (xs[..., :, None] + cs[..., None, :] + 2.0 * scale)
    # a norm near a midpoint moves every distance of its row or column by up to one fp16 ulp
    ulp = lambda v: np.abs(np.nextafter(v.astype(np.float16), np.float16(np.inf)).astype(np.float64)
                           - v.astype(np.float16).astype(np.float64))
    width = width + np.where(xamb, ulp(xs), 0.0)[..., :, None] + np.where(camb, ulp(cs), 0.0)[..., None, :]
    with np.errstate(over="ignore"):
        lo = _fp16_sqrt((d - width).astype(np.float16)).astype(np.float64)
        hi = _fp16_sqrt((d + width).astype(np.float16)).astype(np.float64)
    w = np.argmin(s16.astype(np.float32), axis=-1)
    hw = np.take_along_axis(hi, w[..., None], axis=-1)
    idx = np.arange(c.shape[-2])
    before = idx < w[..., None]
    beats = np.where(before, lo <= hw, lo < hw)              # another centre that could win or tie first
    beats &= idx != w[..., None]
    return beats.any(-1)


def incremental_value_distances(x, centers):
    """V distances of the decode-group assignment (compression.py:61-64):
    fp32(fp16(|x|^2 + |c|^2) - 2 * fp32(x . c)), the norms in fp16 (the
    inputs' dtype), their sum rounded to fp16, the product fp32.  Restated with
    an exact dot product, so ids agree with the reference's away from fp32 ties.
    Returns float64 [..., N, C]."""
    x = np.asarray(x, dtype=np.float16)
    c = np.asarray(centers, dtype=np.float16)
    e = (half_norms(x).astype(np.float64)[..., :, None] + half_norms(c).astype(np.float64)[..., None, :])
    e = e.astype(np.float16).astype(np.float64)
    dot = x.astype(np.float64) @ np.swapaxes(c.astype(np.float64), -1, -2)
    return e - 2.0 * dot


def update_centres(data, ids, previous, count, *, value=False):
    """One Lloyd update from given ids (compression.py:40-52).

    Member sums are exact (float64; the reference's fp32 GEMM sums equal them
    within fp32 rounding), counted in fp32, divided in fp32.  K keeps an empty
    cluster's previous centre and stays fp32; V rounds each quotient to fp16
    (``.to(data.dtype)``) and an empty cluster becomes 0 / 1 = 0.
    data float [BH, T, 128], ids int [BH, T], previous [BH, C, 128].
    """
    data = np.asarray(data, dtype=np.float64)
    onehot = np.eye(count)[np.asarray(ids)]                  # [BH, T, C]
    counts = onehot.sum(1)[..., None]
    sums = (np.swapaxes(onehot, 1, 2) @ data).astype(np.float32)
    mean = (sums / np.maximum(counts, 1).astype(np.float32)).astype(np.float32)
    if value:
        return f16(mean).astype(np.float64)
    return np.where(counts > 0, mean.astype(np.float64), np.asarray(previous, dtype=np.float64))


def kmeans(x, count, iterations, *, value=False):
    """Lloyd k-means per (batch, head) (compression.py:19-53).

    x: fp16 [B, H, T, 128].  K (value=False) assigns by exact distances (the
    fp32 rule, ``assign``), keeps an empty cluster's previous centre and
    carries fp32 centres; V (value=True) assigns by the fp16 ``cdist`` rule
    (``assign_value``), zeroes an empty cluster, rounds every updated centre to
    fp16 and uses count = min(count, T).
    Returns (centers fp16 [B,H,C,128], ids int32 [B,H,T], min_margin float) where
    ids come from the last assignment (made against the pre-update centres)
    and centres from the last update.  min_margin is the smallest
    second-minus-best distance (squared for K, fp16 distance for V).  Requires
    T >= count (the reference's random-init branch for T < count is not
    deterministic).
    """
    b, h, t, _ = x.shape
    if value:
        count = min(count, t)
    if t < count:
        raise ValueError("oracle k-means needs T >= count")
    x16 = np.asarray(x, dtype=np.float16).reshape(b * h, t, D)
    data = x16.astype(np.float64)
    idx = linspace_indices(t, count)
    centers = data[:, idx].copy()
    ids = None
    min_margin = np.inf
    for _ in range(iterations):
        if value:
            s16, _ = value_distances(x16, centers.astype(np.float16))
            s = np.sort(s16.astype(np.float64), axis=-1)
            ids = np.argmin(s16.astype(np.float32), axis=-1)
            margin = s[..., 1] - s[..., 0] if count > 1 else np.full(ids.shape, np.inf)
        else:
            ids, margin = assign(data, centers)
        min_margin = min(min_margin, float(margin.min()))
        centers = update_centres(data, ids, centers, count, value=value)
    return f16(centers.reshape(b, h, count, D)), ids.reshape(b, h, t).astype(np.int32), min_margin


def incremental_cluster(x, centers, max_clusters, *, value=False):
    """Append the group mean while under the cap, then assign (compression.py:56-69).

    The appended centre is ``x.mean(2)`` in fp16 (fp32 accumulation, one
    rounding).  K assigns by exact distances (``cdist`` of fp32 data); V by
    ``incremental_value_distances``, lowest index on ties.  Returns (centres
    fp16, ids int32, margin) with margin the smallest second-minus-best distance.
    """
    x = np.asarray(x, dtype=np.float16)
    c = np.asarray(centers, dtype=np.float16)
    if c.shape[2] < max_clusters:
        mean = (x.astype(np.float64).sum(2, keepdims=True) / x.shape[2]).astype(np.float16)
        c = np.concatenate((c, mean), axis=2)
    if value:
        d = incremental_value_distances(x, c)
        ids = np.argmin(d, axis=-1)
        srt = np.sort(d, axis=-1)
        margin = srt[..., 1] - srt[..., 0] if d.shape[-1] > 1 else np.full(ids.shape, np.inf)
    else:
        ids, margin = assign(x.astype(np.float64), c.astype(np.float64))
    return c, ids.astype(np.int32), float(margin.min())
