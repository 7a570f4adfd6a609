"""The end-to-end harness's fused steps (include/reskv_llama.h) against the
torch formulas they replace in reskv_amd/llama.py.

- the split / rotation / append: bit for bit (each product and sum is
  rounded to fp32 as torch's separate kernels round them);
- the gated activation: within one fp16 step (torch's and the library's
  ``expf`` come from different device-library builds), equal almost everywhere;
- the RMSNorm: within one fp16 step (the sum of squares is reduced in another
  order), equal almost everywhere, and within 2e-3 relative of float64.
"""

import pytest
import torch
import torch.nn.functional as F

from reskv_amd.llama import _rmsnorm, _rotate, fused_qkv_rope, fused_rmsnorm, fused_silu_mul

pytestmark = pytest.mark.gpu


def _steps_apart(a, b):
    """Distance in fp16 representable steps (same-sign finite values)."""
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    return (ia - ib).abs()


@pytest.mark.parametrize("rows,hidden,scale", [(16, 4096, 1.0), (3, 512, 30.0), (1, 8192, 0.01), (5, 136, 1.0)])
def test_rmsnorm_matches_torch(device, rows, hidden, scale):
    g = torch.Generator(device=device).manual_seed(rows * 7 + hidden)
    x = (torch.randn(rows, hidden, device=device, generator=g) * scale).half()
    w = (1.0 + 0.1 * torch.randn(hidden, device=device, generator=g)).half()
    got = fused_rmsnorm(x, w, 1e-5, torch.empty_like(x))
    ref = _rmsnorm(x, w, 1e-5)
    assert int(_steps_apart(got, ref).max()) <= 1
    assert (got == ref).float().mean().item() > 0.97
    xd = x.double()
    exact = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-5) * w.double()
    assert ((got.double() - exact).abs() <= 2e-3 * exact.abs() + 1e-6).all()


@pytest.mark.parametrize("rows,ffn", [(16, 14336), (2, 1024), (7, 8)])
def test_silu_mul_matches_torch(device, rows, ffn):
    g = torch.Generator(device=device).manual_seed(rows + ffn)
    gu = (torch.randn(rows, 2 * ffn, device=device, generator=g) * 4).half()
    got = fused_silu_mul(gu, torch.empty(rows, ffn, device=device, dtype=torch.float16))
    ref = F.silu(gu[:, :ffn]) * gu[:, ffn:]
    same_sign = (got.view(torch.int16) >= 0) == (ref.view(torch.int16) >= 0)
    zero = (got == 0) & (ref == 0)
    assert (same_sign | zero).all()
    assert int(_steps_apart(got[~zero], ref[~zero]).max()) <= 1
    assert (got == ref).float().mean().item() > 0.99


@pytest.mark.parametrize("dense", [False, True])
def test_qkv_rope_and_append_match_torch_bitwise(device, dense):
    b, hq, hk, cap = 3, 8, 2, 40
    g = torch.Generator(device=device).manual_seed(11 + dense)
    qkv = (torch.randn(b, (hq + 2 * hk) * 128, device=device, generator=g) * 3).half()
    angles = torch.arange(64, device=device).float()[None] * (0.001 + torch.arange(cap, device=device).float()[:, None])
    cos, sin = torch.cos(angles), torch.sin(angles)
    pos = torch.tensor([29], device=device, dtype=torch.int64)
    slot = torch.tensor([17], device=device, dtype=torch.int64)
    q = torch.zeros(b, hq, 128, device=device, dtype=torch.float16)
    qr, k, kr, v = torch.zeros_like(q), *(torch.zeros(b, hk, 128, device=device, dtype=torch.float16) for _ in range(3))
    caches = [torch.full((b, hk, cap, 128), 7.0, device=device, dtype=torch.float16) for _ in range(3)]
    rot, raw, vc = caches
    targets = (None, raw, vc, slot) if dense else (rot, raw, vc, slot)
    fused_qkv_rope(qkv, cos, sin, pos, q, qr, k, kr, v, targets)
    eq, ek, ev = (qkv[:, :hq * 128].view(b, hq, 128), qkv[:, hq * 128:(hq + hk) * 128].view(b, hk, 128),
                  qkv[:, (hq + hk) * 128:].view(b, hk, 128))
    c, s = cos.index_select(0, pos), sin.index_select(0, pos)
    assert torch.equal(q, eq) and torch.equal(k, ek) and torch.equal(v, ev)
    assert torch.equal(qr, _rotate(eq, c, s))
    assert torch.equal(kr, _rotate(ek, c, s))
    assert torch.equal(raw[:, :, 17], ek) and torch.equal(vc[:, :, 17], ev)
    untouched = torch.ones(cap, dtype=torch.bool)
    untouched[17] = False
    for t in caches:
        assert (t[:, :, untouched] == 7.0).all()
    if dense:
        assert (rot == 7.0).all()
    else:
        assert torch.equal(rot[:, :, 17], _rotate(ek, c, s))


def test_strided_append_targets(device):
    """Append into a view whose batch stride is larger than Hk * cap * 128."""
    b, hq, hk, cap = 2, 4, 1, 8
    qkv = torch.randn(b, (hq + 2 * hk) * 128, device=device).half()
    cos = torch.ones(cap, 64, device=device)
    sin = torch.zeros(cap, 64, device=device)
    pos = torch.tensor([3], device=device, dtype=torch.int64)
    slot = torch.tensor([5], device=device, dtype=torch.int64)
    big = torch.zeros(b, 2 * hk, cap, 128, device=device, dtype=torch.float16)
    rot, raw, vc = big[:, :hk], torch.zeros_like(big)[:, :hk], torch.zeros_like(big)[:, :hk]
    q = torch.zeros(b, hq, 128, device=device, dtype=torch.float16)
    qr, k, kr, v = torch.zeros_like(q), *(torch.zeros(b, hk, 128, device=device, dtype=torch.float16) for _ in range(3))
    fused_qkv_rope(qkv, cos, sin, pos, q, qr, k, kr, v, (rot, raw, vc, slot))
    assert torch.equal(rot[:, :, 5], k) and torch.equal(big[:, hk:], torch.zeros_like(big[:, hk:]))
    assert torch.equal(qr, q)  # cos 1, sin 0
