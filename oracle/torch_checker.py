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
