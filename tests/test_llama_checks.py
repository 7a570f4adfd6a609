"""Input checks of the end-to-end harness's fused steps (reskv_amd/llama.py),
on the CPU: every mismatch is refused in Python before a pointer reaches the
library (shape, dtype and layout first, then the device)."""

import pytest
import torch

from reskv_amd.llama import fused_qkv_rope, fused_rmsnorm, fused_silu_mul

f16 = dict(dtype=torch.float16)


def test_rmsnorm_checks():
    x = torch.zeros(4, 64, **f16)
    w = torch.ones(64, **f16)
    with pytest.raises(ValueError, match="out has 3 rows"):
        fused_rmsnorm(x, w, 1e-5, torch.zeros(3, 64, **f16))
    with pytest.raises(ValueError, match="out has 32 columns"):
        fused_rmsnorm(x, w, 1e-5, torch.zeros(4, 32, **f16))
    with pytest.raises(ValueError, match="x must be a contiguous fp16 matrix"):
        fused_rmsnorm(x.float(), w, 1e-5, torch.zeros(4, 64, **f16))
    with pytest.raises(ValueError, match="x must be a contiguous fp16 matrix"):
        fused_rmsnorm(torch.zeros(64, 4, **f16).t(), w, 1e-5, torch.zeros(4, 64, **f16))
    with pytest.raises(ValueError, match="w must be"):
        fused_rmsnorm(x, torch.ones(32, **f16), 1e-5, torch.zeros(4, 64, **f16))
    with pytest.raises(ValueError, match="CUDA"):
        fused_rmsnorm(x, w, 1e-5, torch.zeros(4, 64, **f16))


def test_silu_mul_checks():
    out = torch.zeros(4, 16, **f16)
    with pytest.raises(ValueError, match="gu has 24 columns, expected 32"):
        fused_silu_mul(torch.zeros(4, 24, **f16), out)
    with pytest.raises(ValueError, match="gu has 5 rows"):
        fused_silu_mul(torch.zeros(5, 32, **f16), out)
    with pytest.raises(ValueError, match="gu must be a contiguous fp16 matrix"):
        fused_silu_mul(torch.zeros(4, 32), out)
    with pytest.raises(ValueError, match="CUDA"):
        fused_silu_mul(torch.zeros(4, 32, **f16), out)


def _qkv_args(b=2, hq=4, hk=1, p=8):
    return dict(qkv=torch.zeros(b, (hq + 2 * hk) * 128, **f16), cos=torch.zeros(p, 64), sin=torch.zeros(p, 64),
                pos=torch.zeros(1, dtype=torch.int64), q=torch.zeros(b, hq, 128, **f16),
                qr=torch.zeros(b, hq, 128, **f16), k=torch.zeros(b, hk, 128, **f16),
                kr=torch.zeros(b, hk, 128, **f16), v=torch.zeros(b, hk, 128, **f16))


@pytest.mark.parametrize("field,value,match", [
    ("qkv", torch.zeros(2, 5 * 128, **f16), "qkv has 640 columns, expected 768"),
    ("qkv", torch.zeros(3, 6 * 128, **f16), "qkv has 3 rows"),
    ("qr", torch.zeros(2, 4, 64, **f16), r"qr must be a contiguous fp16 tensor \[2, 4, 128\]"),
    ("kr", torch.zeros(2, 1, 128), r"kr must be a contiguous fp16 tensor"),
    ("v", torch.zeros(2, 2, 128, **f16), r"v must be a contiguous fp16 tensor \[2, 1, 128\]"),
    ("cos", torch.zeros(8, 64, dtype=torch.float16), "cos and sin must be contiguous fp32 tables"),
    ("sin", torch.zeros(4, 64), "cos and sin must be contiguous fp32 tables"),
    ("sin", torch.zeros(64, 8).t(), "cos and sin must be contiguous fp32 tables"),
    ("pos", torch.zeros(1, dtype=torch.int32), "pos must be an int64 tensor"),
])
def test_qkv_rope_checks(field, value, match):
    args = _qkv_args()
    args[field] = value
    with pytest.raises(ValueError, match=match):
        fused_qkv_rope(**args)


def test_qkv_rope_append_target_checks():
    args = _qkv_args()
    slot = torch.zeros(1, dtype=torch.int64)
    cache = torch.zeros(2, 1, 16, 128, **f16)
    with pytest.raises(ValueError, match="slot must be an int64 tensor"):
        fused_qkv_rope(**args, targets=(cache, cache, cache, None))
    with pytest.raises(ValueError, match="one \\[B, Hk, cap, 128\\] layout"):
        fused_qkv_rope(**args, targets=(cache, cache.float(), cache, slot))
    with pytest.raises(ValueError, match="one \\[B, Hk, cap, 128\\] layout"):
        fused_qkv_rope(**args, targets=(torch.zeros(2, 2, 16, 128, **f16), None, None, slot))
    with pytest.raises(ValueError, match="CUDA"):
        fused_qkv_rope(**args, targets=(cache, cache, cache, slot))
