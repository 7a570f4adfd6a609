"""Split-K fused decode (HIP) vs the float64 oracle, through reskv_amd.attention.

The case matrix follows reskv tests/test_cuda.py: every bits x sparsity x
layout x fusion combination with and without a dense recent window, GQA 1/8
with 64 centroids and a start offset, large logits, large finite recent
scores, theta-derived RoPE, non-default streams; plus config-0-distributed K
(outlier channels) at T = 1024 and the split-merge invariance.
Tolerance: max-abs <= 2e-3 on the fp16 output.
"""

import numpy as np
import pytest
import torch

from oracle import reskv_oracle as o
from reskv_amd import ResKVKernelConfig, attention, compress
from tests.gpu_helpers import ATOL, expected_attention, np_, outlier_kv, reference_test_inputs, theta_freq

pytestmark = pytest.mark.gpu

CASES = [
    (16, 0.5, "tiled", "per_token"),
    (16, 0.5, "unstructured", "deferred"),
    (16, 0.75, "unstructured", "deferred"),
    (16, 0.75, "structured", "per_token"),
    (16, 0.75, "structured", "deferred"),
    (4, 0.5, "unstructured", "per_token"),
    (4, 0.75, "unstructured", "per_token"),
    (4, 0.75, "structured", "per_token"),
    (4, 0.75, "structured", "deferred"),
    (2, 0.5, "unstructured", "per_token"),
    (2, 0.75, "unstructured", "per_token"),
]


def _max_err(out, ref):
    return float(np.abs(np_(out).astype(np.float64) - ref).max())


@pytest.mark.parametrize("bits,sparsity,layout,fusion", CASES)
def test_fused_and_mixed_against_oracle(device, bits, sparsity, layout, fusion):
    k, v, q, clustering = reference_test_inputs()
    cfg = ResKVKernelConfig(bits=bits, sparsity=sparsity, layout=layout, centroid_fusion=fusion)
    cache = compress(k, v, cfg, clustering=clustering)
    freq = theta_freq() / torch.linspace(1, 8, 64, device=device)  # catches a hard-coded theta
    out = attention(q, cache, position=288, inv_freq=freq)
    assert _max_err(out, expected_attention(q, cache, position=288, inv_freq=freq)) <= ATOL
    g = torch.Generator().manual_seed(5)
    kr = (torch.randn(1, 1, 32, 128, generator=g) * 0.5).half().to(device)
    vr = (torch.randn(1, 1, 32, 128, generator=g) * 0.5).half().to(device)
    qr = torch.from_numpy(o.rotate(np_(q).astype(np.float64), np.array([288]), np_(freq))).half().to(device)
    mixed = attention(q, cache, position=288, inv_freq=freq, recent=(qr, kr, vr))
    ref = expected_attention(q, cache, position=288, inv_freq=freq, recent=(qr, kr, vr))
    assert _max_err(mixed, ref) <= ATOL


@pytest.mark.parametrize("bits,layout", [(16, "unstructured"), (16, "structured"), (4, "unstructured"),
                                         (4, "structured"), (2, "unstructured")])
def test_current_stream(device, bits, layout):
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        k, v, q, c = reference_test_inputs(t=64)
        cache = compress(k, v, ResKVKernelConfig(bits=bits, sparsity=0.75, layout=layout), clustering=c)
        out = attention(q, cache, position=64)
    stream.synchronize()
    assert _max_err(out, expected_attention(q, cache, position=64)) <= ATOL


@pytest.mark.parametrize("ratio", [1, 8])
@pytest.mark.parametrize("bits,layout", [(16, "unstructured"), (16, "structured"), (4, "structured"),
                                         (2, "unstructured")])
def test_gqa_and_64_centroids(device, ratio, bits, layout):
    k, v, q, _ = reference_test_inputs(t=320)
    q = q[:, :1].repeat(1, ratio, 1, 1)
    centers = k[:, :, :64].contiguous()
    ids = torch.arange(320, device=device, dtype=torch.int32).remainder(64).view(1, 1, -1)
    cfg = ResKVKernelConfig(bits=bits, sparsity=0.75, layout=layout)
    cache = compress(k, v, cfg, clustering=((centers, ids), (centers, ids)))
    out = attention(q, cache, position=330, start_position=10)
    assert _max_err(out, expected_attention(q, cache, position=330, start_position=10)) <= ATOL


@pytest.mark.parametrize("fmt,width", [("bitmap", w) for w in (8, 16, 24, 32, 40, 64, 96, 128)] +
                         [("tiled", w) for w in (8, 16, 32, 48, 64, 96)])
def test_residual_widths_through_family_ops(device, fmt, width):
    """Payload widths across the range the C ABI accepts, not only the plans'
    32 and 64: widths above 64 take the wide decoders (four 16-byte pieces per
    lane), widths 8 and 16 leave most lanes without a piece.  T = 300 leaves a
    partial tile in every wave range."""
    from reskv_amd._extension import load_extension

    b, hk, g, t = 2, 2, 4, 300
    k, v, q, ((kc, ki), (vc, vi)) = reference_test_inputs(b=b, t=t, heads=hk, gqa=g, seed=41)
    comp = load_extension("compression")
    if fmt == "bitmap":
        enc = [comp.compress_bitmap(x, c, i, width) for x, c, i in ((k, kc, ki), (v, vc, vi))]
    else:
        enc = [comp.compress_fp16(x, c, i, width, False) for x, c, i in ((k, kc, ki), (v, vc, vi))]
    (kp, km), (vp, vm) = enc
    flat = lambda x: x.reshape(b * hk, *x.shape[2:]).contiguous()  # noqa: E731
    ids8 = lambda x: flat(x).to(torch.int8)  # noqa: E731
    freq = theta_freq()
    scaling = 128 ** -0.5
    args = (hk, hk * g, 7, 320, 500000.0, scaling)
    Q = q.reshape(b * hk * g, 128).contiguous()
    for splits in (0, 3):
        if fmt == "bitmap":
            out = load_extension("cluster_mass").decode_fp16(
                Q, flat(kc), ids8(ki), flat(kp), flat(km), flat(vc), ids8(vi), flat(vp), flat(vm), *args,
                False, splits, freq)[0]
        else:
            out = load_extension("attention", None).decode_fp16(
                Q, flat(kc), ids8(ki), flat(kp), flat(km), None, flat(vc), ids8(vi), flat(vp), flat(vm), None,
                *args, splits, freq)[0]
        kd = o.reconstruct(fmt, np_(kc), np_(ki), np_(kp), np_(km))
        vd = o.reconstruct(fmt, np_(vc), np_(vi), np_(vp), np_(vm))
        ref = o.reference_attention(np_(q).astype(np.float64), kd, vd, position=320, start_position=7,
                                    freq=np_(freq), scaling=scaling)
        assert _max_err(out.view(b, hk * g, 1, 128), ref) <= ATOL, splits


@pytest.mark.parametrize("bits,sparsity,layout,b,t,inputs",
                         [(16, 0.5, "unstructured", bb, 8192, "sweep") for bb in (1, 4, 8, 16, 32)]
                         + [(16, 0.75, "structured", bb, 8192, "sweep") for bb in (1, 4, 8, 16, 32)]
                         + [(4, 0.5, "unstructured", 8, 16384, "outlier"),
                            (2, 0.5, "unstructured", 8, 16384, "outlier")])
def test_benchmark_shapes_against_fp32_checker(device, bits, sparsity, layout, b, t, inputs):
    """Configs 2 and 3 at their full shapes (Hq = 32, Hk = 8): the split-K decode at the
    automatic split count and at 16 splits against the float32 torch port of the oracle
    (oracle/torch_checker.py, pinned to the oracle's golden vectors on the CPU).  Config 2
    runs at every batch of its sweep (1, 4, 8, 16, 32), so each automatic split count and
    kernel instance the bench times (64 / 16 / 8 / 4 / 2 splits at 50%; the 4:16 instance
    at two and three workgroups per CU) is checked at T = 8192.

    Config 2 uses the timing sweep's inputs (0.5 N(0,1) K and V, 0.1 N(0,1) centres,
    random ids; reskv benchmarks/kernels.py:57-65).  Config 3 uses its own recipe:
    outlier-channel K (N(0,1) x LogNormal(0,1) per channel, 4 channels x 10), N(0,1) V,
    clustered by the device K-means (32 clusters, 10 iterations).  Its "group-64
    asymmetric INT4/INT2 with fp16 scale and zero-point" resolves to the reference
    kernel format, which is what is built and tested here: symmetric codes with one
    fp16 scale per token and no zero-point (reskv/csrc/compression.cu:339-360,
    decoded by reskv/reference.py:17-21); "group 64" is the decode-group token count
    (reskv/config.py:87), not a channel group."""
    from oracle import torch_checker as tc

    if inputs == "sweep":
        g = torch.Generator(device=device).manual_seed(7)
        shape = (b, 8, t, 128)
        k = torch.randn(shape, device=device, dtype=torch.float16, generator=g) * 0.5
        v = torch.randn(shape, device=device, dtype=torch.float16, generator=g) * 0.5
        kc = torch.randn(b, 8, 32, 128, device=device, dtype=torch.float16, generator=g) * 0.1
        vc = torch.randn(b, 8, 32, 128, device=device, dtype=torch.float16, generator=g) * 0.1
        ki = torch.randint(32, shape[:3], device=device, dtype=torch.int32, generator=g)
        vi = torch.randint(32, shape[:3], device=device, dtype=torch.int32, generator=g)
        q = torch.randn(b, 32, 1, 128, device=device, dtype=torch.float16, generator=g)
        cfg = ResKVKernelConfig(bits=bits, sparsity=sparsity, layout=layout)
        cache = compress(k, v, cfg, clustering=((kc, ki), (vc, vi)))
    else:
        k, v, q = outlier_kv(b, 8, t, seed=3)
        cfg = ResKVKernelConfig(bits=bits, sparsity=sparsity, layout=layout, num_clusters=32, kmeans_iterations=10)
        cache = compress(k, v, cfg)
        assert cache.key.scale is not None and cache.key.metadata is None  # symmetric per-token codes
    del k, v
    freq = theta_freq()
    ref = tc.attention(q, cache, position=t, inv_freq=freq)
    for splits in (0, 16):
        out = attention(q, cache, position=t, inv_freq=freq, splits=splits)
        err = (out.float() - ref).abs().max().item()
        assert err <= ATOL, (splits, err)
    del ref
    torch.cuda.empty_cache()


def test_structured_int4_large_logits(device):
    k, v, q, c = reference_test_inputs(t=256)
    k, q = k * 12, q * 12
    cfg = ResKVKernelConfig(bits=4, sparsity=0.75, layout="structured", centroid_fusion="deferred")
    cache = compress(k, v, cfg, clustering=c)
    out = attention(q, cache, position=256)
    assert torch.isfinite(out).all()
    assert _max_err(out, expected_attention(q, cache, position=256)) <= ATOL


def test_invalid_external_cluster_ids_rejected(device):
    k, v, _, c = reference_test_inputs(t=64)
    c[0][1][0, 0, 0] = 32
    with pytest.raises(ValueError, match="out of range"):
        compress(k, v, clustering=c)


def test_theta_rope_with_model_rotated_recent_tokens(device):
    k, v, q, c = reference_test_inputs(t=256)
    cfg = ResKVKernelConfig(bits=4, sparsity=0.75, layout="unstructured", rope_mode="theta")
    cache = compress(k, v, cfg, clustering=c)
    model_freq = theta_freq() / 8
    qr = torch.from_numpy(o.rotate(np_(q).astype(np.float64), np.array([288]), np_(model_freq))).half().to(device)
    recent = (qr, k[:, :, :32].contiguous(), v[:, :, :32].contiguous())
    out = attention(q, cache, position=288, recent=recent)
    assert _max_err(out, expected_attention(q, cache, position=288, recent=recent)) <= ATOL


@pytest.mark.parametrize("sparsity", [0.5, 0.75])
def test_recent_attention_with_large_finite_scores(device, sparsity):
    data = torch.zeros(1, 1, 128, 128, device=device, dtype=torch.float16)
    centers = data[:, :, :1].contiguous()
    ids = torch.zeros(1, 1, 128, device=device, dtype=torch.int32)
    config = ResKVKernelConfig(sparsity=sparsity, centroid_fusion="deferred")
    cache = compress(data, data, config, clustering=((centers, ids), (centers, ids)))
    query = torch.full((1, 4, 1, 128), 100.0, device=device, dtype=torch.float16)
    recent = (query, torch.full_like(data[:, :, :32], 100.0), torch.full_like(data[:, :, :32], 2.0))
    out = attention(query, cache, position=159, recent=recent)
    assert torch.isfinite(out).all()
    ref = expected_attention(query, cache, position=159, recent=recent)
    assert np.allclose(np_(out).astype(np.float64), ref, atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("sparsity,layout", [(0.5, "unstructured"), (0.75, "structured"),
                                             (0.75, "unstructured")])
def test_config0_outlier_keys(device, sparsity, layout):
    """Config 0 shapes and distributions (B=1, 8/32 heads, T=1024, sinks 4, recent 60)."""
    k, v, q = outlier_kv(1, 8, 1024, seed=0)
    freq = theta_freq()
    sink, tc = 4, 960
    cfg = ResKVKernelConfig(sparsity=sparsity, layout=layout, num_clusters=32, kmeans_iterations=15)
    cache = compress(k[:, :, sink:sink + tc].contiguous(), v[:, :, sink:sink + tc].contiguous(), cfg)
    dense_pos = torch.cat((torch.arange(sink), torch.arange(sink + tc, 1024))).numpy()
    k_dense = np_(k)[:, :, dense_pos].astype(np.float64)
    kr = torch.from_numpy(o.rotate(k_dense, dense_pos, np_(freq))).half().to(device)
    vr = v[:, :, dense_pos].contiguous()
    qr = torch.from_numpy(o.rotate(np_(q).astype(np.float64), np.array([1024]), np_(freq))).half().to(device)
    out = attention(q, cache, position=1024, start_position=sink, inv_freq=freq, recent=(qr, kr, vr))
    ref = expected_attention(q, cache, position=1024, start_position=sink, inv_freq=freq, recent=(qr, kr, vr))
    assert _max_err(out, ref) <= ATOL


@pytest.mark.parametrize("layout,sparsity", [("unstructured", 0.5), ("structured", 0.75)])
def test_split_count_invariance_and_stats(device, layout, sparsity):
    from reskv_amd._extension import load_extension

    k, v, q = outlier_kv(2, 2, 700, seed=9, gqa=4)
    cfg = ResKVKernelConfig(sparsity=sparsity, layout=layout, centroid_fusion="deferred", num_clusters=16)
    cache = compress(k, v, cfg)
    ext = load_extension("cluster_mass", cache.key.plan)
    qf = q.reshape(-1, 128).contiguous()
    kc, ki, kp, km, _ = cache.key._native
    vc, vi, vp, vm, _ = cache.value._native
    freq = theta_freq()
    args = (2, 8, 0, 800, 500000.0, 128 ** -0.5, True)
    outs = []
    for splits in (1, 3, 64, 700, 0):
        if layout == "unstructured":
            o_, m_, l_ = ext.decode_fp16(qf, kc, ki, kp, km, vc, vi, vp, vm, *args, splits, freq)
        else:
            e = qf.new_empty(0)
            o_, m_, l_ = ext.decode_structured_fp16(qf, kc, ki, kp, km, e, vc, vi, vp, vm, e, *args, splits, freq)
        outs.append((np_(o_).astype(np.float64), np_(m_), np_(l_)))
    eo, em, el = o.compressed_stats(np_(q).astype(np.float64), _dense(cache.key), _dense(cache.value),
                                    position=800, freq=np_(freq))
    for o_, m_, l_ in outs:
        assert np.abs(o_ - eo.reshape(-1, 128)).max() <= ATOL
        assert np.allclose(m_, em.reshape(-1), atol=1e-3, rtol=1e-4)
        assert np.allclose(l_, el.reshape(-1), rtol=2e-4)


def test_fixed_shift_plan_returns_the_unshifted_statistics(device):
    """Structured INT4 under the fixed-shift plan (cluster_mass.cu:660, 874-888,
    1046-1067): the same output as the online plan, m = 0 and l = sum exp(score)."""
    from reskv_amd._extension import load_extension

    k, v, q = outlier_kv(2, 2, 700, seed=12, gqa=4)
    qf = q.reshape(-1, 128).contiguous()
    freq = theta_freq()
    args = (2, 8, 0, 800, 500000.0, 128 ** -0.5, True, 0, freq)
    res = {}
    for mode in ("online", "fixed_shift"):
        cfg = ResKVKernelConfig(sparsity=0.75, bits=4, layout="structured", centroid_fusion="deferred",
                                num_clusters=16, softmax_mode=mode)
        cache = compress(k, v, cfg)
        assert cache.key.plan.fixed_shift == (mode == "fixed_shift")
        ext = load_extension("cluster_mass", cache.key.plan)
        kc, ki, kp, km, ks = cache.key._native
        vc, vi, vp, vm, vs = cache.value._native
        res[mode] = [np_(t).astype(np.float64) for t in
                     ext.decode_structured_int4(qf, kc, ki, kp, km, ks, vc, vi, vp, vm, vs, *args)]
    eo, em, el = o.compressed_stats(np_(q).astype(np.float64), _dense(cache.key), _dense(cache.value),
                                    position=800, freq=np_(freq))
    (o_on, m_on, l_on), (o_fs, m_fs, l_fs) = res["online"], res["fixed_shift"]
    assert np.array_equal(o_on, o_fs)
    assert np.abs(o_fs - eo.reshape(-1, 128)).max() <= ATOL
    assert (m_fs == 0).all()
    assert np.allclose(l_fs, (el * np.exp(em)).reshape(-1), rtol=5e-4)
    assert np.allclose(m_on, em.reshape(-1), atol=1e-3, rtol=1e-4)


def _dense(ct):
    from tests.gpu_helpers import dense

    return dense(ct)


def test_dense_baseline_decode(device):
    from reskv_amd._extension import dense_decode

    k, v, q = outlier_kv(2, 4, 513, seed=4, gqa=8)
    freq = theta_freq()
    out = dense_decode(q, k, v, freq, position=600, start_position=3)
    ref = o.reference_attention(np_(q).astype(np.float64), np_(k).astype(np.float64), np_(v).astype(np.float64),
                                position=600, start_position=3, freq=np_(freq))
    assert _max_err(out, ref) <= ATOL


def test_dense_baseline_decode_reads_cache_prefix(device):
    """A token prefix of a preallocated [B, H, Tmax, 128] cache equals the same tokens packed."""
    from reskv_amd._extension import dense_decode

    k, v, q = outlier_kv(2, 8, 300, seed=5, gqa=4)
    freq = theta_freq()
    kbuf = torch.zeros(2, 8, 512, 128, dtype=torch.float16, device=k.device)
    vbuf = torch.zeros_like(kbuf)
    kbuf[:, :, :300] = k
    vbuf[:, :, :300] = v
    out = dense_decode(q, kbuf[:, :, :300], vbuf[:, :, :300], freq, position=310)
    ref = dense_decode(q, k, v, freq, position=310)
    assert torch.equal(out, ref)


def test_query_position_before_cache_rejected(device):
    k, v, q, c = reference_test_inputs(t=64)
    cache = compress(k, v, clustering=c)
    with pytest.raises(ValueError, match="precedes"):
        attention(q, cache, position=10)


@pytest.mark.parametrize("sparsity,layout", [(0.5, "unstructured"), (0.75, "structured")])
def test_deferred_merge_recent_with_fp32_scores(device, sparsity, layout):
    """The deferred family's merge_recent(comp_out, m, l, scores, v_recent)
    (cluster_mass.cu:1461-1508) fed as reskv/_attention.py:135-143 feeds it:
    fp32 scores q_rot . k_rot * scale, against the oracle's joint softmax."""
    from reskv_amd._extension import load_extension

    k, v, q = outlier_kv(2, 2, 640, seed=33)
    cfg = ResKVKernelConfig(sparsity=sparsity, layout=layout, centroid_fusion="deferred", num_clusters=16)
    cache = compress(k, v, cfg)
    ext = load_extension("cluster_mass", cache.key.plan)
    freq = theta_freq()
    pos, tr, scale = 700, 57, 128 ** -0.5
    g = torch.Generator().manual_seed(34)
    kr = (torch.randn(2, 2, tr, 128, generator=g) * 2).half().to(device)
    vr = torch.randn(2, 2, tr, 128, generator=g).half().to(device)
    qr = torch.from_numpy(o.rotate(np_(q).astype(np.float64), np.array([pos]), np_(freq))).half().to(device)
    qf = q.reshape(-1, 128).contiguous()
    kc, ki, kp, km, _ = cache.key._native
    vc, vi, vp, vm, _ = cache.value._native
    args = (2, 8, 0, pos, 500000.0, scale, True, 0, freq)
    if layout == "unstructured":
        out, m, l = ext.decode_fp16(qf, kc, ki, kp, km, vc, vi, vp, vm, *args)
    else:
        e = qf.new_empty(0)
        out, m, l = ext.decode_structured_fp16(qf, kc, ki, kp, km, e, vc, vi, vp, vm, e, *args)
    scores = torch.matmul(qr.float().reshape(2, 2, 4, 128), kr.float().transpose(-1, -2)) * scale
    merged = ext.merge_recent(out, m, l, scores.reshape(2, 8, tr).contiguous(), vr, 2, 8)
    ref = expected_attention(q, cache, position=pos, inv_freq=freq, recent=(qr, kr, vr))
    assert _max_err(merged.reshape(2, 8, 1, 128), ref) <= ATOL
    # the same joint softmax as the in-kernel-score path
    fused = attention(q, cache, position=pos, inv_freq=freq, recent=(qr, kr, vr))
    assert _max_err(merged.reshape(2, 8, 1, 128), np_(fused).astype(np.float64)) <= 1e-3


@pytest.mark.parametrize("tr", [129, 300])
def test_recent_window_longer_than_one_chunk(device, tr):
    """Recent windows above 128 tokens take the merge's multi-chunk online
    rescale (the model reaches them with recent_size >= 128)."""
    k, v, q = outlier_kv(2, 2, 512, seed=35)
    cache = compress(k, v, ResKVKernelConfig(sparsity=0.5, num_clusters=16))
    freq = theta_freq()
    pos = 512 + tr
    g = torch.Generator().manual_seed(36)
    kr = (torch.randn(2, 2, tr, 128, generator=g) * 2).half().to(device)
    vr = torch.randn(2, 2, tr, 128, generator=g).half().to(device)
    # a late token with a large score moves the running maximum in the last chunk
    kr[:, :, tr - 3] = 8.0
    qr = torch.from_numpy(o.rotate(np_(q).astype(np.float64), np.array([pos]), np_(freq))).half().to(device)
    out = attention(q, cache, position=pos, inv_freq=freq, recent=(qr, kr, vr))
    ref = expected_attention(q, cache, position=pos, inv_freq=freq, recent=(qr, kr, vr))
    assert _max_err(out, ref) <= ATOL


@pytest.mark.parametrize("sparsity,layout", [(0.5, "unstructured"), (0.75, "structured")])
def test_rope_table_growth_across_calls(device, sparsity, layout):
    """One frequency set decoded at compressed positions that cross the RoPE
    table's growth points (1,024 -> 2,048 -> 4,096 positions), then back down:
    every call reads the table rows of its own positions, the grown table
    replaces the old one and the old one stays alive, and each output matches
    the float64 oracle at those positions."""
    import reskv_amd._extension as ext

    k, v, q = outlier_kv(1, 2, 700, seed=21, gqa=4)
    cache = compress(k, v, ResKVKernelConfig(sparsity=sparsity, layout=layout, num_clusters=16))
    # a frequency set no other test (or case) uses, so its table starts at
    # 1,024 positions: the cache is per process
    freq = theta_freq(123457.0 if sparsity == 0.5 else 223457.0)
    before = len(ext._RETIRED)
    sizes = []
    for start in (300, 330, 1400, 3300, 20):
        position = start + 700 + 3
        out = attention(q, cache, position=position, start_position=start, inv_freq=freq)
        ref = expected_attention(q, cache, position=position, start_position=start, inv_freq=freq)
        assert float(np.abs(np_(out).astype(np.float64) - ref).max()) <= ATOL, start
        key = ext._content_key(freq, freq.device)
        sizes.append(ext._ROPE_TABLES[key][0].shape[0])
    assert sizes == [1024, 2048, 4096, 4096, 4096]
    assert len(ext._RETIRED) - before == 2
