"""The FP16 encoders form residuals with packed fp16 subtraction.  The reference
computes fp16(f32(x) - f32(c)) (reskv/csrc/compression.cu:80-118); for fp16
inputs that equals the correctly rounded fp16 difference, which is what an IEEE
fp16 subtraction returns.  Checked here for every pair of finite fp16 values."""

import numpy as np


def test_fp32_then_fp16_equals_correctly_rounded_fp16_difference():
    every = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    finite = every[np.isfinite(every)]
    c32 = finite.astype(np.float32)[None, :]
    c64 = finite.astype(np.float64)[None, :]
    mismatches = 0
    with np.errstate(over="ignore", invalid="ignore"):
        for start in range(0, finite.size, 64):
            x = finite[start:start + 64, None]
            via_fp32 = (x.astype(np.float32) - c32).astype(np.float16).view(np.uint16)
            exact = (x.astype(np.float64) - c64).astype(np.float16).view(np.uint16)  # float64 holds it exactly
            mismatches += int(np.count_nonzero(via_fp32 != exact))
    assert mismatches == 0
