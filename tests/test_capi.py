"""The C-ABI library: loads on a CPU-only host, exports every declared symbol,
and rejects bad arguments before touching a GPU (no compute calls here)."""

import ctypes
import re
from pathlib import Path

import pytest

from reskv_amd import _lib

INCLUDE = Path(__file__).resolve().parents[1] / "include"
HEADER = INCLUDE / "reskv_hip.h"


def declared_functions(headers=None):
    text = "".join(h.read_text() for h in (headers or sorted(INCLUDE.glob("*.h"))))
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(reskv_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_operator_surface():
    names = declared_functions([HEADER])
    for required in ("reskv_compress_fp16", "reskv_compress_bitmap", "reskv_compress_quantized",
                     "reskv_compress_structured_int4", "reskv_compress_fp16_kv", "reskv_compress_bitmap_kv",
                     "reskv_kmeans", "reskv_kmeans_assign", "reskv_kmeans_kv",
                     "reskv_decode",
                     "reskv_merge_recent_scores", "reskv_merge_recent_qk", "reskv_decode_recent",
                     "reskv_decode_dense"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.reskv_abi_version() == _lib.ABI_VERSION == 7


def test_a_library_of_another_abi_version_is_refused(monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "ABI_VERSION", 5)
    with pytest.raises(RuntimeError, match="ABI version 7, this binding needs 5"):
        _lib.lib()
    assert _lib._lib is None  # nothing half-loaded is kept


def _err(status):
    assert status != 0
    return _lib.lib().reskv_last_error().decode()


def test_null_pointers_are_rejected_without_a_gpu():
    lib = _lib.lib()
    assert "null" in _err(lib.reskv_compress_fp16(None, None, None, None, None, 1, 1, 1, 1, 32, 1, None))
    assert "null" in _err(lib.reskv_compress_bitmap(None, None, None, None, None, 1, 1, 1, 1, 32, None))
    assert "null" in _err(lib.reskv_kmeans(None, None, None, None, 1, 1, 1, 1, 0, None, 0, None))
    p = ctypes.c_void_p(16)
    assert "both initial centre arrays or neither" in _err(lib.reskv_kmeans_kv(p, p, p, None, p, p, p, p, 1, 4, 2, 1,
                                                                                p, 1 << 20, None))
    assert "null" in _err(lib.reskv_kmeans_kv(*([None] * 8), 1, 1, 1, 1, None, 0, None))
    assert "null" in _err(lib.reskv_compress_fp16_kv(*([None] * 10), 1, 1, 1, 4, 4, 32, 1, None))
    assert "null" in _err(lib.reskv_compress_bitmap_kv(*([None] * 10), 1, 1, 1, 4, 4, 32, None))
    assert "null" in _err(lib.reskv_merge_recent_qk(None, None, None, None, None, None, 1, 4, 1, 1, 0, 1.0, None,
                                                    None))
    assert "null" in _err(lib.reskv_decode_recent(None, None, None, None, None, 1, 4, 1, 16, 0, 15, 1.0, 0, None,
                                                  None, None, 1, 0, None, None, 0, None))


@pytest.mark.parametrize(
    "args,message",
    [
        (dict(nnz=30, struct_index=0), "divisible by 8"),
        (dict(nnz=64, struct_index=1), "4:16"),
        (dict(C=65), "centroid count"),
        (dict(T=0), "positive"),
    ],
)
def test_encoder_argument_checks(args, message):
    lib = _lib.lib()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    kw = dict(B=1, H=1, T=4, C=4, nnz=32, struct_index=1)
    kw.update(args)
    st = lib.reskv_compress_fp16(p, p, p, p, p, kw["B"], kw["H"], kw["T"], kw["C"], kw["nnz"],
                                 kw["struct_index"], None)
    assert message in _err(st)


def test_kv_encoder_argument_checks():
    lib = _lib.lib()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    assert "centroid count" in _err(lib.reskv_compress_bitmap_kv(*([p] * 10), 1, 1, 4, 4, 65, 32, None))
    assert "nnz" in _err(lib.reskv_compress_bitmap_kv(*([p] * 10), 1, 1, 4, 4, 4, 0, None))
    assert "positive" in _err(lib.reskv_compress_fp16_kv(*([p] * 10), 1, 0, 4, 4, 4, 32, 1, None))
    assert "divisible by 8" in _err(lib.reskv_compress_fp16_kv(*([p] * 10), 1, 1, 4, 4, 4, 30, 0, None))


def test_linspace_rows_match_torch_and_the_oracle():
    """The library's initial-centre rows equal torch.linspace(0, T-1, C).long()
    (reskv/compression.py:35) and the oracle's restatement."""
    import numpy as np
    import torch

    from oracle import reskv_oracle as o

    lib = _lib.lib()
    for t in (1, 2, 3, 33, 64, 65, 100, 960, 1000, 4095, 8156, 8192, 16384, 65536, 1 << 20):
        for c in (1, 2, 7, 31, 32, 33, 63, 64):
            if t < c:
                continue
            rows = (ctypes.c_int32 * c)()
            assert lib.reskv_linspace_rows(t, c, rows) == 0
            got = np.array(list(rows))
            assert np.array_equal(got, torch.linspace(0, t - 1, c).long().numpy()), (t, c)
            assert np.array_equal(got, o.linspace_indices(t, c)), (t, c)
    rows = (ctypes.c_int32 * 4)()
    assert "T >= C" in _err(lib.reskv_linspace_rows(3, 4, rows))
    assert "T >= C" in _err(lib.reskv_kmeans(ctypes.c_void_p(16), None, ctypes.c_void_p(16), ctypes.c_void_p(16),
                                              1, 3, 4, 1, 0, ctypes.c_void_p(256), 1 << 20, None))


def test_rope_table_needs_whole_blocks_of_positions():
    """The table stores positions in blocks of 16; a count that is not a
    multiple of 16 is refused before any device call."""
    lib = _lib.lib()
    p = ctypes.c_void_p(16)
    assert "null" in _err(lib.reskv_rope_table(None, 16, p, None))
    for count in (0, 20, 1000):
        assert "multiple of 16" in _err(lib.reskv_rope_table(p, count, p, None))


def test_quantiser_argument_checks():
    lib = _lib.lib()
    p = ctypes.c_void_p(16)
    assert "bits" in _err(lib.reskv_compress_quantized(p, p, p, p, p, 1, 1, 4, 4, 64, 3, None))
    assert "nnz" in _err(lib.reskv_compress_quantized(p, p, p, p, p, 1, 1, 4, 4, 48, 4, None))


def test_decode_descriptor_checks():
    lib = _lib.lib()
    p = ctypes.c_void_p(16)
    good = _lib.CTensor(p, p, p, p, None, 32, _lib.FMT_BITMAP, 64, 16)
    bad_fmt = _lib.CTensor(p, p, p, p, None, 32, 9, 64, 16)
    bad_nc = _lib.CTensor(p, p, p, p, None, 65, _lib.FMT_BITMAP, 64, 16)
    bad_quant = _lib.CTensor(p, p, p, None, None, 32, _lib.FMT_QUANT, 16, 4)
    for desc, msg in ((bad_fmt, "unknown residual format"), (bad_nc, "centroid count"), (bad_quant, "quantised")):
        st = lib.reskv_decode(p, ctypes.byref(desc), ctypes.byref(good), p, 1, 32, 8, 16, 0, 16, 0.1, 0, p, None,
                              None, p, 1 << 30, None)
        assert msg in _err(st)
    st = lib.reskv_decode(p, ctypes.byref(good), ctypes.byref(good), p, 1, 24, 8, 16, 0, 16, 0.1, 0, p, None, None,
                          p, 1 << 30, None)
    assert "GQA" in _err(st)
    st = lib.reskv_decode(p, ctypes.byref(good), ctypes.byref(good), p, 1, 32, 8, 16, 0, 16, 0.1, 0, p, None, None,
                          p, 16, None)
    assert "workspace" in _err(st)


def test_split_and_workspace_sizing():
    lib = _lib.lib()
    record = (2 + 128 + 64) * 4  # one split partial per query head: m, l, 128 sums, 64 cluster masses
    # the workspace covers the largest automatic count: ceil(4 * 256 / (B * H)) workgroups per head,
    # capped at T / 128 (two 16-token tiles per wave)
    for b, s in ((1, 64), (4, 32), (8, 16), (16, 8), (32, 4)):
        assert lib.reskv_decode_workspace_bytes(b, 32, 8, 8192, 0) == b * 32 * s * record
    assert lib.reskv_decode_workspace_bytes(1, 32, 8, 256, 0) == 32 * 2 * record
    assert lib.reskv_decode_workspace_bytes(1, 32, 8, 8192, 20) == 32 * 20 * record
    # explicit split counts need no device: capped at T
    p = ctypes.c_void_p(16)
    good = _lib.CTensor(p, p, p, p, None, 32, _lib.FMT_BITMAP, 64, 16)
    assert lib.reskv_decode_splits(ctypes.byref(good), ctypes.byref(good), 1, 1, 32, 8, 5, 20) == 5
    assert lib.reskv_decode_splits(ctypes.byref(good), ctypes.byref(good), 1, 1, 32, 8, 8192, 20) == 20
    assert lib.reskv_decode_splits(ctypes.byref(good), ctypes.byref(good), 1, 1, 30, 8, 8192, 20) == -1
    assert "multiple" in lib.reskv_last_error().decode()
    assert lib.reskv_kmeans_workspace_bytes(16, 8192, 32) > 0


# ---------------------------------------------------------------------------
# merge_recent input checks run before any launch (CPU tensors never reach
# the library: a shape or dtype error is raised first, then the device check)
# ---------------------------------------------------------------------------

def _recent_args(b=2, nh=8, kh=2, tr=5, width=128, m_dtype=None, heads=None):
    import torch

    comp = torch.zeros(b * nh, 128, dtype=torch.float16)
    m = torch.zeros(b * nh, dtype=m_dtype or torch.float32)
    l = torch.zeros(b * nh, dtype=torch.float32)
    v = torch.zeros(b, heads or kh, tr, width, dtype=torch.float16)
    return comp, m, l, v


@pytest.mark.parametrize("bad,match", [
    ({"width": 64}, "v_recent must be"),
    ({"heads": 3}, "v_recent shape mismatch"),
    ({"m_dtype": "f16"}, "comp_m/comp_l must be fp32"),
])
def test_deferred_merge_recent_rejects_bad_shapes(bad, match):
    import torch
    from reskv_amd._extension import load_extension

    if bad.get("m_dtype") == "f16":
        bad = dict(bad, m_dtype=torch.float16)
    comp, m, l, v = _recent_args(**bad)
    scores = torch.zeros(2, 8, v.shape[2], dtype=torch.float32)
    ext = load_extension("cluster_mass")
    with pytest.raises(RuntimeError, match=match):
        ext.merge_recent(comp, m, l, scores, v, 2, 8)


def test_deferred_merge_recent_rejects_score_shape():
    import torch
    from reskv_amd._extension import load_extension

    comp, m, l, v = _recent_args()
    ext = load_extension("cluster_mass")
    with pytest.raises(RuntimeError, match="scores_recent must be"):
        ext.merge_recent(comp, m, l, torch.zeros(2, 8, 4, dtype=torch.float32), v, 2, 8)
    with pytest.raises(RuntimeError, match="Unsupported GQA ratio"):
        ext.merge_recent(comp, m, l, torch.zeros(2, 8, 5, dtype=torch.float32), v, 3, 9)


@pytest.mark.parametrize("bad,match", [
    ({"width": 64}, "v_recent must be"),
    ({"heads": 4}, "v_recent shape mismatch"),
    ({"tr": 0}, "T_recent must be > 0"),
])
def test_per_token_merge_recent_rejects_bad_shapes(bad, match):
    import torch
    from reskv_amd._extension import load_extension

    comp, m, l, v = _recent_args(**bad)
    k = torch.zeros(v.shape, dtype=torch.float16)
    if bad.get("heads"):
        k = torch.zeros(2, 2, v.shape[2], 128, dtype=torch.float16)
    q = torch.zeros(16, 128, dtype=torch.float16)
    ext = load_extension("attention")
    with pytest.raises(RuntimeError, match=match):
        ext.merge_recent(comp, m, l, q, k, v, 2, 8, 0.1)


def test_per_token_merge_recent_rejects_short_key_rows():
    import torch
    from reskv_amd._extension import load_extension

    comp, m, l, v = _recent_args()
    ext = load_extension("attention")
    with pytest.raises(RuntimeError, match="k_recent must be"):
        ext.merge_recent(comp, m, l, torch.zeros(16, 128, dtype=torch.float16),
                         torch.zeros(2, 2, 5, 64, dtype=torch.float16), v, 2, 8, 0.1)
    with pytest.raises(RuntimeError, match="all tensors must be on the same GPU"):
        ext.merge_recent(comp, m, l, torch.zeros(16, 128, dtype=torch.float16),
                         torch.zeros(2, 2, 5, 128, dtype=torch.float16), v, 2, 8, 0.1)


def test_attention_rejects_recent_rows_that_are_not_128_wide():
    import torch
    from reskv_amd._attention import _recent_window

    q = torch.zeros(1, 8, 1, 128, dtype=torch.float16)
    bad = (q, torch.zeros(1, 2, 4, 64, dtype=torch.float16), torch.zeros(1, 2, 4, 64, dtype=torch.float16))
    with pytest.raises(ValueError, match="recent Q/K/V shapes"):
        _recent_window(bad, q, 1, 2)
    empty = (q, torch.zeros(1, 2, 0, 128, dtype=torch.float16), torch.zeros(1, 2, 0, 128, dtype=torch.float16))
    assert _recent_window(empty, q, 1, 2) is None


def test_noalloc_decode_rejects_sizes_beyond_its_scratch_before_any_device_call():
    L = _lib.lib()
    # 64 x 8 rows x 256 splits of 776-byte partial records: far above the 8 MiB array
    status = L.reskv_decode_recent_noalloc(None, None, None, None, None, 64, 8, 2, 256, 0, 300, 0.1, 256,
                                           None, None, None, 0, 0, None, None)
    assert status != 0 and "allocation-free" in L.reskv_last_error().decode()
    assert L.reskv_decode_workspace_bytes(32, 32, 8, 8192, 0) <= 8 << 20


def test_harness_op_argument_checks():
    """The end-to-end harness's fused steps (include/reskv_llama.h) reject bad
    arguments before any launch."""
    lib = _lib.lib()
    a = ctypes.c_void_p(256)  # aligned placeholder address, never dereferenced
    assert "null" in _err(lib.reskv_llama_rmsnorm(None, a, a, 16, 4096, 1e-5, None))
    assert "multiple of 8" in _err(lib.reskv_llama_rmsnorm(a, a, a, 16, 4100, 1e-5, None))
    assert "up to 8192" in _err(lib.reskv_llama_rmsnorm(a, a, a, 16, 8200, 1e-5, None))
    assert "aligned" in _err(lib.reskv_llama_rmsnorm(ctypes.c_void_p(258), a, a, 16, 4096, 1e-5, None))
    assert lib.reskv_llama_rmsnorm(a, a, a, 0, 4096, 1e-5, None) == 0  # no rows: no launch
    assert "multiple of 8" in _err(lib.reskv_llama_silu_mul(a, a, 16, 12, None))
    assert "negative" in _err(lib.reskv_llama_silu_mul(a, a, -1, 16, None))
    args = [a, a, a, a, 2, 32, 8] + [a] * 5
    assert "head counts" in _err(lib.reskv_llama_qkv_rope(a, a, a, a, 2, 32, 7, *[a] * 5, None, None, None, None,
                                                          0, 0, 0, None))
    assert "slot" in _err(lib.reskv_llama_qkv_rope(*args, a, None, None, None, 1, 1, 1, None))
    assert "strides" in _err(lib.reskv_llama_qkv_rope(*args, None, a, a, a, 1, 0, 1, None))
    assert "null" in _err(lib.reskv_llama_qkv_rope(None, *args[1:], None, None, None, None, 0, 0, 0, None))


def test_fixed_shift_statistics_conversion():
    """The fixed-shift plan reports m = 0 and l = sum exp(score): the online
    (m, l) pair converted, overflowing to inf where the unshifted sum does."""
    import torch

    from reskv_amd._extension import _fixed_shift_stats

    out = torch.zeros(3, 128)
    m = torch.tensor([1.5, -20.0, 100.0])
    l = torch.tensor([3.0, 1.0, 2.0])
    o2, m2, l2 = _fixed_shift_stats([out, m, l])
    assert o2 is out and torch.equal(m2, torch.zeros(3))
    assert torch.allclose(l2[:2], l[:2] * torch.exp(m[:2])) and torch.isinf(l2[2])
    assert _fixed_shift_stats([out]) == [out]  # without statistics nothing changes


def test_misaligned_recent_values_are_rejected_before_any_launch():
    """The recent join stages V rows with 16-byte loads: every entry point that
    reads recent V refuses a pointer off a 16-byte boundary (an fp16 tensor at
    an odd storage offset) on the host."""
    lib = _lib.lib()
    p = ctypes.c_void_p(16)
    odd = ctypes.c_void_p(18)
    assert "recent V must be 16-byte aligned" in _err(
        lib.reskv_merge_recent_scores(p, p, p, p, odd, 1, 4, 1, 5, p, None))
    assert "recent K and V must be 16-byte aligned" in _err(
        lib.reskv_merge_recent_qk(p, p, p, p, p, odd, 1, 4, 1, 5, 0, 0.1, p, None))
    assert "recent K and V must be 16-byte aligned" in _err(
        lib.reskv_merge_recent_qk(p, p, p, p, odd, p, 1, 4, 1, 5, 0, 0.1, p, None))
    good = _lib.CTensor(p, p, p, p, None, 32, _lib.FMT_BITMAP, 64, 16)
    assert "recent K and V must be 16-byte aligned" in _err(
        lib.reskv_decode_recent(p, ctypes.byref(good), ctypes.byref(good), p, None, 1, 4, 1, 16, 0, 15, 0.1, 0, p,
                                p, odd, 5, 0, p, p, 1 << 30, None))
