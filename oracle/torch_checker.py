"""Float32 torch port of ``oracle/reskv_oracle.py``'s reconstruction and
attention.  TEST INFRASTRUCTURE ONLY.

The numpy oracle evaluates in float64 on the CPU, which takes minutes at the
benchmark shapes (config 2 at B = 32, T = 8192; config 3 at T = 16384).  This
port runs the same steps with torch in float32 on whatever device the cache
lives on, so the GPU tests can check those shapes.  It is imported only by
``tests/``; the product package never uses it.

Functions and what they port (numpy oracle function, reference lines it follows):

* ``reconstruct``  -- ``reskv_oracle.reconstruct`` (reference.py:12-49): every
                      residual format decoded to fp32 and added to its centre;
* ``attention``    -- ``reskv_oracle.reference_attention`` (reference.py:52-91):
                      absolute-position rotate-half RoPE with fp32 angles
                      fl32(pos * freq), GQA repeat, one softmax over the
                      compressed tokens followed by the dense recent ones.

Pinned by ``tests/test_torch_checker.py`` against the float64 golden vectors
that the numpy oracle wrote (max-abs 5e-4; a wrong bit order, index or
rotation gives errors above 1e-2).
"""

import torch

D = 128


def _unpack(words: torch.Tensor, field_bits: int, fields_per_word: int) -> torch.Tensor:
    """Unsigned fields of int32 words, LSB-first: [..., W] -> [..., W * fields_per_word] int64."""
    w = words.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(fields_per_word, device=words.device, dtype=torch.int64) * field_bits
    return ((w[..., None] >> shifts) & ((1 << field_bits) - 1)).flatten(-2)


def _signed(code: torch.Tensor, bits: int) -> torch.Tensor:
    sign = 1 << (bits - 1)
    return (code ^ sign) - sign


def _expand_by_mask(mask: torch.Tensor, payload: torch.Tensor) -> torch.Tensor:
    """Dense [..., 128] fp32 placing payload values, in order, on the True channels."""
    rank = mask.to(torch.int64).cumsum(-1) - 1
    vals = payload.float().gather(-1, rank.clamp_min(0))
    return torch.where(mask, vals, torch.zeros((), device=payload.device))


def _residual(ct) -> torch.Tensor:
    plan = ct.plan
    lead = tuple(ct.cluster_ids.shape)
    if plan.bits != 16 and plan.layout != "structured":
        per_word = 32 // plan.bits
        q = _signed(_unpack(ct.payload, plan.bits, per_word), plan.bits)
        return q.float() * ct.scale.float()[..., None]
    if plan.bits == 16 and plan.layout == "unstructured":
        # int64 words, channel d at bit 63 - d % 64 of word d // 64
        w = ct.metadata.to(torch.int64)
        d = torch.arange(D, device=w.device)
        bit = (w[..., d // 64] >> (63 - d % 64)) & 1
        return _expand_by_mask(bit.bool(), ct.payload)
    if plan.bits == 4:
        # structured INT4: nibble i of the packed words, 2-bit slot of subgroup i
        q = _signed(_unpack(ct.payload, 4, 8), 4).float() * ct.scale.float()[..., None]
        slot = _unpack(ct.metadata, 2, 16)                       # [..., 32]
        dims = slot + torch.arange(32, device=slot.device) * 4
        out = torch.zeros(*lead, D, device=q.device)
        return out.scatter(-1, dims, q)
    codes = _unpack(ct.metadata, 16, 2)                          # [..., 8] tile codes
    if plan.layout == "structured":
        idx = _unpack(codes.to(torch.int32), 4, 4).reshape(*lead, 8, 4)[..., :4]
        dims = (idx + torch.arange(8, device=idx.device)[:, None] * 16).reshape(*lead, 32)
        out = torch.zeros(*lead, D, device=codes.device)
        return out.scatter(-1, dims, ct.payload.float())
    mask = ((codes[..., None] >> torch.arange(16, device=codes.device)) & 1).bool().reshape(*lead, D)
    return _expand_by_mask(mask, ct.payload)


def reconstruct(ct) -> torch.Tensor:
    """fp32 [B, H, T, 128]: centre of each token plus its decoded residual."""
    ids = ct.cluster_ids.to(torch.int64)
    centre = ct.centroids.float().gather(2, ids[..., None].expand(*ids.shape, D))
    return centre + _residual(ct)


def _rotate(x: torch.Tensor, positions: torch.Tensor, freq: torch.Tensor) -> torch.Tensor:
    angle = positions.float()[:, None] * freq.float()[None, :]   # one fp32 product per angle
    cos, sin = angle.cos(), angle.sin()
    a, b = x[..., :64], x[..., 64:]
    return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1)


def attention(query, cache, *, position, start_position=0, inv_freq=None, rope_theta=500000.0,
              scaling=None, recent=None) -> torch.Tensor:
    """fp32 [B, Hq, 1, 128] decode attention of raw ``query`` over ``cache``
    (plus the dense ``recent`` = (rotated q, rotated K, V) window)."""
    dev = query.device
    freq = (rope_theta ** (-torch.arange(64, device=dev).float() / 64)).float() if inv_freq is None \
        else inv_freq.float().to(dev)
    k, v = reconstruct(cache.key), reconstruct(cache.value)
    b, hk, t, _ = k.shape
    g = query.shape[1] // hk
    scale = D ** -0.5 if scaling is None else float(scaling)
    q = _rotate(query.float(), torch.tensor([position], device=dev), freq)
    k = _rotate(k, torch.arange(start_position, start_position + t, device=dev), freq)
    k, v = k.repeat_interleave(g, 1), v.repeat_interleave(g, 1)
    scores = torch.matmul(q, k.transpose(-1, -2)) * scale
    if recent is not None:
        qr, kr, vr = (x.float() for x in recent)
        scores = torch.cat((scores, torch.matmul(qr, kr.repeat_interleave(g, 1).transpose(-1, -2)) * scale), -1)
        v = torch.cat((v, vr.repeat_interleave(g, 1)), dim=2)
    return torch.matmul(torch.softmax(scores, dim=-1), v)


# ---------------------------------------------------------------------------
# compress, for the CPU baseline: the numpy oracle's kmeans and encoders on
# torch tensors (any device), so that bench.py can time a multi-threaded CPU
# restatement of compress (reskv/compression.py:19-101).  Pinned against the
# numpy oracle by tests/test_torch_checker.py.
# ---------------------------------------------------------------------------

def _fp16_sqrt(d16):
    return d16.double().clamp_min(0).sqrt().half()


def kmeans(x, count, iterations, *, value=False):
    """Lloyd k-means per (batch, head) on x fp16 [B, H, T, 128] (T >= count).

    K: fp32 data and distances (|x|^2 + |c|^2 - 2 x.c), empty clusters keep
    their centre; V: the fp16 cdist rule (fp16 norms, fp16 distance, fp16
    root, lowest index on ties), fp16 centres, empty -> 0.  Returns (centres
    fp16 [B, H, C, 128], ids int32 [B, H, T]) as reskv_oracle.kmeans.
    """
    b, h, t, _ = x.shape
    count = min(count, t) if value else count
    rows = x.reshape(b * h, t, D)
    idx = torch.linspace(0, t - 1, count).long()
    data = rows.float()
    centres = data[:, idx].clone()
    if value:
        xn = (rows.float() * rows.float()).half().float().sum(-1).half().float()
    for _ in range(iterations):
        if value:
            c16 = centres.half()
            cn = (c16.float() * c16.float()).half().float().sum(-1).half().float()
            dot = torch.bmm(data.double(), c16.double().transpose(1, 2))
            d16 = (xn.double()[..., None] + cn.double()[:, None, :] - 2.0 * dot).half()
            ids = _fp16_sqrt(d16).float().argmin(-1)
        else:
            d = (data * data).sum(-1, keepdim=True) - 2.0 * torch.bmm(data, centres.transpose(1, 2)) \
                + (centres * centres).sum(-1)[:, None, :]
            ids = d.argmin(-1)
        onehot = torch.nn.functional.one_hot(ids, count).float()
        counts = onehot.sum(1)[..., None]
        sums = torch.bmm(onehot.transpose(1, 2), data)
        mean = sums / counts.clamp_min(1)
        centres = mean.half().float() if value else torch.where(counts > 0, mean, centres)
    return centres.reshape(b, h, count, D).half(), ids.reshape(b, h, t).int()


def _residual_and_key(x, centres, ids):
    cent = centres.gather(2, ids.long().clamp(0, centres.shape[2] - 1)[..., None].expand(*ids.shape, D))
    r = x.float() - cent.float()
    return r, r.half().float().abs()


def _top_mask(key, k):
    """k largest keys per row, lowest index on ties (a stable descending sort)."""
    order = torch.sort(key, dim=-1, descending=True, stable=True).indices[..., :k]
    return torch.zeros_like(key, dtype=torch.bool).scatter_(-1, order, True)


def encode_bitmap(x, centres, ids, nnz):
    """Unstructured FP16: payload fp16 [..., nnz] ascending, int64 MSB-first bitmaps [..., 2]."""
    r, key = _residual_and_key(x, centres, ids)
    mask = _top_mask(key, nnz)
    payload = r.half()[mask].reshape(*mask.shape[:-1], nnz)
    bits = mask.reshape(*mask.shape[:-1], 2, 64).long()
    words = (bits << torch.arange(63, -1, -1)).sum(-1)  # int64 wraps like the reference's bit 63
    return payload, words


def encode_structured(x, centres, ids, nnz=32):
    """Tiled / structured 4:16 FP16 with four-nibble codes: payload [..., nnz], int32 words [..., 4]."""
    per_tile = nnz // 8
    r, key = _residual_and_key(x, centres, ids)
    tiles = key.reshape(*key.shape[:-1], 8, 16)
    mask = _top_mask(tiles, per_tile)
    payload = r.half()[mask.reshape(*mask.shape[:-2], D)].reshape(*mask.shape[:-2], nnz)
    pos = torch.sort(torch.sort(tiles, dim=-1, descending=True, stable=True).indices[..., :per_tile], dim=-1).values
    codes = (pos.long() << (4 * torch.arange(per_tile))).sum(-1)
    words = (codes[..., 0::2] | (codes[..., 1::2] << 16)) & 0xFFFFFFFF
    return payload, (words - ((words >> 31) << 32)).to(torch.int32)  # as signed int32 words


def encode_multibit(x, centres, ids, nnz, bits):
    """Top-nnz + symmetric INT4/INT2 codes with an fp16 per-token scale."""
    qmax = (1 << (bits - 1)) - 1
    per_word = 32 // bits
    r, key = _residual_and_key(x, centres, ids)
    mask = _top_mask(key, nnz)
    amax = torch.where(mask, r.abs(), torch.zeros(())).amax(-1)
    scale = torch.where(amax > 0, (amax / qmax).half(), torch.ones((), dtype=torch.float16))
    q = torch.clamp(torch.round(r / scale.float()[..., None]), -qmax, qmax).long()
    q = torch.where(mask, q, torch.zeros((), dtype=torch.long)) & ((1 << bits) - 1)
    q = q.reshape(*q.shape[:-1], D // per_word, per_word)
    words = (q << (torch.arange(per_word) * bits)).sum(-1)
    return (words - ((words >> 31) << 32)).to(torch.int32), scale  # as signed int32 words
