"""Native operator families behind the reference's loader interface.

``load_extension(family, plan=None, device_index=0)`` keeps the signature,
caching and family names of ``reskv/_extension.py:14-61`` and returns a
namespace whose attributes are the same operators with the same argument
order (``reskv/csrc/compression.cu:508-512``, ``attention.cu:1350-1355``,
``cluster_mass.cu:1511-1516``).  Behind them is the prebuilt gfx950 library
``libreskv_hip.so`` (C ABI, ``include/reskv_hip.h``) instead of a JIT-built
CUDA extension; plan fields select formats at run time instead of ``-D``
rebuilds.

Each operator validates like the reference's ``TORCH_CHECK`` (raising
``RuntimeError``), allocates its outputs and split-K scratch with torch on
the input's device, and enqueues the kernels on torch's current stream of
that device without synchronising.
"""

import ctypes
import weakref
from functools import lru_cache
from types import SimpleNamespace

import torch

from . import _lib
from .config import KernelPlan

FAMILIES = ("compression", "attention", "cluster_mass")


# ---------------------------------------------------------------------------
# small helpers
# ---------------------------------------------------------------------------

def _require(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _ptr(t):
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _dev_check(*tensors, contiguous=True):
    dev = tensors[0].device
    for t in tensors:
        if t is not None and t.numel() > 0:
            _require(t.is_cuda and t.device == dev, "all tensors must be on the same GPU")
            if contiguous:
                _require(t.is_contiguous(), "tensors must be contiguous")
    return dev


def _row_stride(t, width):
    """Rows of a [BH, T(, width)] view: unit-stride within a token, token rows
    `width` apart; returns the token stride between (batch, head) blocks."""
    if t.dim() == 2:
        _require(t.stride(1) == 1 or t.shape[1] == 1, "cache rows must be unit-stride")
        return t.stride(0) if t.shape[0] > 1 else t.shape[1]
    _require(t.stride(2) == 1 and (t.stride(1) == width or t.shape[1] == 1), "cache rows must be dense")
    if t.shape[0] == 1:
        return t.shape[1]
    _require(t.stride(0) % width == 0, "cache blocks must start on a token row")
    return t.stride(0) // width


def _empty(shape, dtype, device):
    return torch.empty(shape, dtype=dtype, device=device)


def _workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# RoPE tables, one per frequency set, keyed by the 64 fp32 frequency values
# (content), or by theta for the theta-derived set.  Compressed tokens keep
# their positions, so one table serves every layer and decode step.
#
# A caller's inv_freq tensor is matched to its content key through
# _BY_TENSOR (storage address, offset and dtype; the version counter detects
# in-place updates, except for inference tensors, which have none), whose
# entry is dropped by a finalizer when that tensor is collected, so a reused address never maps to
# a stale key; a tensor not seen before costs one 256-byte device-to-host copy
# of its values.  Fresh tensors with equal values (a per-call `.float()` of an
# fp16 buffer, a `.to(device)` copy) therefore share one table.
#
# At most _MAX_FREQ_SETS frequency sets are kept (least recently used
# evicted; an evicted table is released to torch's allocator, whose reuse is
# ordered on the current stream).  A table that grows is replaced, and the
# replaced one stays alive in _RETIRED, because a captured HIP graph or work
# queued on another stream may still hold its address; growth is geometric
# (powers of two), so the retired tables add at most the size of the live one.
# Graph capture: make one eager call with the same inv_freq tensor (or theta)
# at the largest position first, so that nothing is copied or allocated while
# capturing, and keep the captured sets within _MAX_FREQ_SETS.
_MAX_FREQ_SETS = 8
_ROPE_TABLES = {}  # content key -> (table fp32 [P, 128], frequencies fp32 [64]), in LRU order
_BY_TENSOR = {}    # (device, storage address, offset, dtype) -> (version, content key)
_RETIRED = []


def _build_table(freq, count):
    table = torch.empty((count, 128), dtype=torch.float32, device=freq.device)
    with torch.cuda.device(freq.device):
        _lib.check(_lib.lib().reskv_rope_table(freq.data_ptr(), count, table.data_ptr(), _stream(freq.device)),
                   "rope_table")
    return table


def _table_for(key, freq, positions):
    """(frequencies, fp32 [P, 128] table covering [0, positions)), P a power of two >= 1024."""
    entry = _ROPE_TABLES.pop(key, None)
    if entry is not None:
        freq = entry[1]
        if entry[0].shape[0] < positions:
            _RETIRED.append(entry[0])
            entry = None
    if entry is None:
        count = 1 << max(10, (int(positions) - 1).bit_length())
        entry = (_build_table(freq, count), freq)
    _ROPE_TABLES[key] = entry  # most recently used last
    while len(_ROPE_TABLES) > _MAX_FREQ_SETS:
        _ROPE_TABLES.pop(next(iter(_ROPE_TABLES)))
    return entry[1], entry[0]


def _content_key(inv_freq, dev):
    ident = (dev, inv_freq.untyped_storage().data_ptr(), inv_freq.storage_offset(), inv_freq.dtype)
    # inference tensors carry no version counter: an in-place update of one is
    # not seen (pass a new tensor instead)
    version = -1 if inv_freq.is_inference() else inv_freq._version
    seen = _BY_TENSOR.get(ident)
    if seen is not None and seen[0] == version:
        return seen[1]
    values = inv_freq.detach().reshape(64).to(device="cpu", dtype=torch.float32)
    key = (dev, "freq", values.numpy().tobytes())
    _BY_TENSOR[ident] = (version, key)  # an in-place update replaces the entry
    if seen is None:
        weakref.finalize(inv_freq, _BY_TENSOR.pop, ident, None)
    return key


def _rope(inv_freq, rope_base, dev, positions):
    """(fp32 frequencies, table) for the caller's inv_freq [64] (any float
    dtype, converted to fp32 as the reference's kernels read it) or the
    theta-derived set."""
    if inv_freq is not None and inv_freq.numel():
        _require(inv_freq.numel() == 64 and inv_freq.is_floating_point(), "inv_freq must be fp32 [64]")
        key = _content_key(inv_freq, dev)
        freq = None
        if key not in _ROPE_TABLES:
            freq = _frequencies(inv_freq.detach().reshape(64).float(), rope_base, dev)
        return _table_for(key, freq, positions)
    key = (dev, "theta", float(rope_base))
    freq = None if key in _ROPE_TABLES else _frequencies(None, rope_base, dev)
    return _table_for(key, freq, positions)


def _frequencies(inv_freq, rope_base, device):
    """The 64 RoPE frequencies: the caller's, or theta-derived (reskv/reference.py:73-77)."""
    if inv_freq is not None and inv_freq.numel():
        _require(inv_freq.numel() == 64 and inv_freq.dtype == torch.float32, "inv_freq must be fp32 [64]")
        return inv_freq.to(device).contiguous()
    idx = torch.arange(64, device=device).float()
    return (float(rope_base) ** (-idx / 64)).float().contiguous()


# ---------------------------------------------------------------------------
# compression family
# ---------------------------------------------------------------------------

def _check_encoder_inputs(keys, centroids, cluster_ids):
    _require(keys.is_cuda and centroids.is_cuda and cluster_ids.is_cuda, "inputs must be CUDA tensors")
    _require(keys.dtype == torch.float16 and centroids.dtype == torch.float16, "keys and centroids must be float16")
    _require(cluster_ids.dtype == torch.int32, "cluster_ids must be int32")
    _require(keys.dim() == 4 and centroids.dim() == 4 and cluster_ids.dim() == 3,
             "expected keys[B,nh,T,D], centroids[B,nh,C,D], cluster_ids[B,nh,T]")
    _require(keys.shape[3] == 128 and centroids.shape[3] == 128, "Only D=128 is supported")
    _require(tuple(cluster_ids.shape) == tuple(keys.shape[:3]) and centroids.shape[:2] == keys.shape[:2],
             "keys, centroids and cluster_ids disagree in [B, nh, T]")
    _dev_check(keys, centroids, cluster_ids)
    b, h, t, _ = keys.shape
    return b, h, t, centroids.shape[2]


def compress_fp16(keys, centroids, cluster_ids, nnz_per_token, use_4x16_struct_index):
    """Tiled / structured-4:16 FP16 encoder (reskv/csrc/compression.cu:423-473)."""
    b, h, t, c = _check_encoder_inputs(keys, centroids, cluster_ids)
    nnz = int(nnz_per_token)
    dev = keys.device
    payload = _empty((b, h, t, nnz), torch.float16, dev)
    meta = _empty((b, h, t, 4), torch.int32, dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().reskv_compress_fp16(
            keys.data_ptr(), centroids.data_ptr(), cluster_ids.data_ptr(), payload.data_ptr(), meta.data_ptr(),
            b, h, t, c, nnz, int(bool(use_4x16_struct_index)), _stream(dev)), "compress_fp16")
    return [payload, meta]


def compress_bitmap(keys, centroids, cluster_ids, nnz_per_token):
    """Unstructured FP16 encoder with MSB-first int64 bitmaps (reskv/compression.py:75-89)."""
    b, h, t, c = _check_encoder_inputs(keys, centroids, cluster_ids)
    nnz = int(nnz_per_token)
    dev = keys.device
    payload = _empty((b, h, t, nnz), torch.float16, dev)
    meta = _empty((b, h, t, 2), torch.int64, dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().reskv_compress_bitmap(
            keys.data_ptr(), centroids.data_ptr(), cluster_ids.data_ptr(), payload.data_ptr(), meta.data_ptr(),
            b, h, t, c, nnz, _stream(dev)), "compress_bitmap")
    return [payload, meta]


def _check_pair(k, kc, ki, v, vc, vi):
    b, h, t, ck = _check_encoder_inputs(k, kc, ki)
    cv = _check_encoder_inputs(v, vc, vi)[3]
    _require(tuple(v.shape) == tuple(k.shape) and v.device == k.device, "K and V must have identical shapes and devices")
    return b, h, t, ck, cv


def compress_fp16_kv(k, k_centroids, k_ids, v, v_centroids, v_ids, nnz_per_token, use_4x16_struct_index):
    """``compress_fp16`` of a layer's K and of its V in one launch
    (reskv/compression.py:166-167).  Returns ((payload, meta) of K, of V)."""
    b, h, t, ck, cv = _check_pair(k, k_centroids, k_ids, v, v_centroids, v_ids)
    nnz, dev = int(nnz_per_token), k.device
    out = [(_empty((b, h, t, nnz), torch.float16, dev), _empty((b, h, t, 4), torch.int32, dev)) for _ in range(2)]
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().reskv_compress_fp16_kv(
            k.data_ptr(), v.data_ptr(), k_centroids.data_ptr(), v_centroids.data_ptr(), k_ids.data_ptr(),
            v_ids.data_ptr(), out[0][0].data_ptr(), out[1][0].data_ptr(), out[0][1].data_ptr(), out[1][1].data_ptr(),
            b, h, t, ck, cv, nnz, int(bool(use_4x16_struct_index)), _stream(dev)), "compress_fp16_kv")
    return out


def compress_bitmap_kv(k, k_centroids, k_ids, v, v_centroids, v_ids, nnz_per_token):
    """``compress_bitmap`` of a layer's K and of its V in one launch
    (reskv/compression.py:166-167).  Returns ((payload, meta) of K, of V)."""
    b, h, t, ck, cv = _check_pair(k, k_centroids, k_ids, v, v_centroids, v_ids)
    nnz, dev = int(nnz_per_token), k.device
    out = [(_empty((b, h, t, nnz), torch.float16, dev), _empty((b, h, t, 2), torch.int64, dev)) for _ in range(2)]
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().reskv_compress_bitmap_kv(
            k.data_ptr(), v.data_ptr(), k_centroids.data_ptr(), v_centroids.data_ptr(), k_ids.data_ptr(),
            v_ids.data_ptr(), out[0][0].data_ptr(), out[1][0].data_ptr(), out[0][1].data_ptr(), out[1][1].data_ptr(),
            b, h, t, ck, cv, nnz, _stream(dev)), "compress_bitmap_kv")
    return out


def compress_quantized(keys, centroids, cluster_ids, nnz_per_token, bitwidth):
    """Unstructured top-nnz + signed INT4/INT2 (reskv/csrc/compression.cu:392-421)."""
    b, h, t, c = _check_encoder_inputs(keys, centroids, cluster_ids)
    bits = int(bitwidth)
    dev = keys.device
    qtiles = _empty((b, h, t, 4 * bits), torch.int32, dev)
    qscale = _empty((b, h, t), torch.float16, dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().reskv_compress_quantized(
            keys.data_ptr(), centroids.data_ptr(), cluster_ids.data_ptr(), qtiles.data_ptr(), qscale.data_ptr(),
            b, h, t, c, int(nnz_per_token), bits, _stream(dev)), "compress_quantized")
    return [qtiles, qscale]


def compress_structured_int4(keys, centroids, cluster_ids):
    """Structured 1-of-4 INT4 encoder (reskv/csrc/compression.cu:475-504)."""
    b, h, t, c = _check_encoder_inputs(keys, centroids, cluster_ids)
    dev = keys.device
    qpacked = _empty((b, h, t, 4), torch.int32, dev)
    qmeta = _empty((b, h, t, 2), torch.int32, dev)
    qscale = _empty((b, h, t), torch.float16, dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().reskv_compress_structured_int4(
            keys.data_ptr(), centroids.data_ptr(), cluster_ids.data_ptr(), qpacked.data_ptr(), qmeta.data_ptr(),
            qscale.data_ptr(), b, h, t, c, _stream(dev)), "compress_structured_int4")
    return [qpacked, qmeta, qscale]


def _init_count(inits, count, t):
    """The centroid count: from the given initial centres, or ``count`` for the
    linspace tokens (reskv/compression.py:34-36), which need T >= count."""
    given = [c for c in inits if c is not None]
    _require(len(given) in (0, len(inits)), "give every initial centre array or none")
    for c in given:
        _require(c.dtype == torch.float32 and c.dim() == 3, "centres must be fp32 [BH,C,128]")
    if given:
        return given[0].shape[1]
    _require(count is not None and 1 <= int(count) <= t, "linspace initial centres need 1 <= count <= T")
    return int(count)


def linspace_rows(t, count):
    """Initial-centre token rows, torch.linspace(0, T-1, count).long() evaluated in fp32 (host list)."""
    rows = (ctypes.c_int32 * int(count))()
    _lib.check(_lib.lib().reskv_linspace_rows(int(t), int(count), rows), "linspace_rows")
    return list(rows)


def kmeans(x, centers_init, iterations, value, count=None):
    """Lloyd k-means (reskv/compression.py:37-53).

    x fp16 [BH, T, 128]; centers_init fp32 [BH, C, 128], or None for the
    tokens at linspace(0, T-1, count) of each row (gathered on the device).
    Returns (centres fp16 [BH, C, 128], ids int32 [BH, T]).
    """
    _require(x.dtype == torch.float16 and x.dim() == 3 and x.shape[2] == 128, "x must be fp16 [BH,T,128]")
    bh, t, _ = x.shape
    c = _init_count((centers_init,), count, t)
    dev = _dev_check(x, *(() if centers_init is None else (centers_init,)))
    out = _empty((bh, c, 128), torch.float16, dev)
    ids = _empty((bh, t), torch.int32, dev)
    L = _lib.lib()
    ws = _workspace(L.reskv_kmeans_workspace_bytes(bh, t, c), dev)
    with torch.cuda.device(dev):
        _lib.check(L.reskv_kmeans(x.data_ptr(), _ptr(centers_init), out.data_ptr(), ids.data_ptr(), bh, t, c,
                                  int(iterations), int(bool(value)), ws.data_ptr(), ws.numel(), _stream(dev)),
                   "kmeans")
    return out, ids


def kmeans_kv(k, v, init_k, init_v, iterations, count=None):
    """A layer's K and V clustered in one launch sequence (reskv/compression.py:164-165).

    k, v fp16 [BH, T, 128]; init_k, init_v fp32 [BH, C, 128], or both None for
    the linspace tokens (``count`` of them).  Returns ((centres_k, ids_k),
    (centres_v, ids_v)), each equal to ``kmeans`` with value=False for K and
    value=True for V.
    """
    for x in (k, v):
        _require(x.dtype == torch.float16 and x.dim() == 3 and x.shape[2] == 128, "x must be fp16 [BH,T,128]")
    bh, t, _ = k.shape
    c = _init_count((init_k, init_v), count, t)
    _require(k.shape == v.shape and (init_k is None or (init_k.shape == init_v.shape and init_k.shape[0] == bh)),
             "K and V must share [BH, T] and the centroid count")
    dev = _dev_check(k, v, *(() if init_k is None else (init_k, init_v)))
    outs = [_empty((bh, c, 128), torch.float16, dev) for _ in range(2)]
    ids = [_empty((bh, t), torch.int32, dev) for _ in range(2)]
    L = _lib.lib()
    ws = _workspace(L.reskv_kmeans_workspace_bytes(2 * bh, t, c), dev)
    with torch.cuda.device(dev):
        _lib.check(L.reskv_kmeans_kv(k.data_ptr(), v.data_ptr(), _ptr(init_k), _ptr(init_v),
                                     outs[0].data_ptr(), outs[1].data_ptr(), ids[0].data_ptr(), ids[1].data_ptr(),
                                     bh, t, c, int(iterations), ws.data_ptr(), ws.numel(), _stream(dev)), "kmeans_kv")
    return (outs[0], ids[0]), (outs[1], ids[1])


def kmeans_assign(x, centers, value=False):
    """Nearest-centre ids, lowest index on ties. x fp16 [BH,T,128]; centres fp32 [BH,C,128].

    value=False: fp32 distances (K); value=True: the decode-group V rule,
    fp32(fp16(|x|^2 + |c|^2) - 2 x.c) with fp16 norms.
    """
    _require(x.dtype == torch.float16 and x.dim() == 3 and x.shape[2] == 128, "x must be fp16 [BH,T,128]")
    _require(centers.dtype == torch.float32 and centers.dim() == 3 and centers.shape[2] == 128,
             "centres must be fp32 [BH,C,128]")
    _require(centers.shape[0] == x.shape[0], "x and centres must have the same leading dimension")
    dev = _dev_check(x, centers)
    bh, t, _ = x.shape
    c = centers.shape[1]
    ids = _empty((bh, t), torch.int32, dev)
    L = _lib.lib()
    ws = _workspace(L.reskv_kmeans_workspace_bytes(bh, t, c), dev)
    with torch.cuda.device(dev):
        _lib.check(L.reskv_kmeans_assign(x.data_ptr(), centers.data_ptr(), ids.data_ptr(), bh, t, c, int(bool(value)),
                                         ws.data_ptr(), ws.numel(), _stream(dev)), "kmeans_assign")
    return ids


# ---------------------------------------------------------------------------
# decode families
# ---------------------------------------------------------------------------

def _ctensor(cent, ids, payload, meta, scale, fmt, bits):
    """Descriptor of one compressed tensor; the tensors may be views into
    larger capacity buffers (rows of each (batch, head) block evenly strided)."""
    _require(cent.dtype == torch.float16 and cent.dim() == 3 and cent.shape[2] == 128,
             "centroids must be fp16 [B*nh_kv, nc, 128]")
    _require(ids.dtype == torch.int8 and ids.dim() == 2, "cluster ids must be int8 [B*nh_kv, T]")
    _require(payload.dim() == 3 and payload.shape[:2] == ids.shape, "payload must be [B*nh_kv, T, width]")
    _require(cent.shape[0] == ids.shape[0], "centroid batch-head mismatch")
    ts = _row_stride(ids, 1)
    _require(_row_stride(payload, payload.shape[2]) == ts, "payload and ids row strides differ")
    if meta is not None and meta.numel():
        _require(meta.dim() == 3 and meta.shape[:2] == ids.shape, "metadata shape mismatch")
        _require(_row_stride(meta, meta.shape[2]) == ts, "metadata and ids row strides differ")
    if scale is not None and scale.numel():
        _require(scale.dtype == torch.float16 and tuple(scale.shape) == tuple(ids.shape), "scale shape mismatch")
        _require(_row_stride(scale, 1) == ts, "scale and ids row strides differ")
    cs = _row_stride(cent, 128)
    return _lib.CTensor(_ptr(cent), _ptr(ids), _ptr(payload), _ptr(meta), _ptr(scale), int(cent.shape[1]),
                        int(fmt), int(payload.shape[2]), int(bits), int(ts), int(cs))


def _decode(Q, kdesc, vdesc, keep, nh_kv, nh, start_pos, pos_q, rope_base, scaling, splits, inv_freq,
            return_stats=True):
    _require(Q.is_cuda and Q.dtype == torch.float16, "Q must be fp16 CUDA")
    _require(Q.dim() == 2 and Q.shape[1] == 128, "Q must be [B*nh, 128]")
    _require(Q.is_contiguous(), "Q must be contiguous")
    _dev_check(Q, *keep, contiguous=False)
    nh_kv, nh = int(nh_kv), int(nh)
    _require(nh % nh_kv == 0, "num_q_heads must be divisible by num_kv_heads")
    _require(nh // nh_kv in (1, 2, 4, 8), "supported GQA ratios are 1, 2, 4 and 8")
    bnh = Q.shape[0]
    _require(bnh % nh == 0, "Q rows must be a multiple of num_q_heads")
    b = bnh // nh
    ids = keep[1]
    _require(ids.shape[0] == b * nh_kv, "cache batch-head count does not match Q")
    t = ids.shape[1]
    dev = Q.device
    freq, table = _rope(inv_freq, rope_base, dev, int(start_pos) + t)
    L = _lib.lib()
    out = _empty((bnh, 128), torch.float16, dev)
    m = _empty((bnh,), torch.float32, dev)
    l = _empty((bnh,), torch.float32, dev)
    ws = _workspace(L.reskv_decode_workspace_bytes(b, nh, nh_kv, t, int(splits)), dev)
    with torch.cuda.device(dev):
        _lib.check(L.reskv_decode_rope(Q.data_ptr(), kdesc, vdesc, freq.data_ptr(), table.data_ptr(), b, nh, nh_kv,
                                       t, int(start_pos), int(pos_q), float(scaling), int(splits), out.data_ptr(),
                                       m.data_ptr(), l.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev)),
                   "decode")
    return [out, m, l] if return_stats else [out]


def cache_descriptors(cache):
    """C descriptors of a CompressedKV's key and value tensors (the format the
    family ops derive from the plan) and the tensors they point into."""
    plan = cache.key.plan
    out, keep = [], []
    for t in (cache.key, cache.value):
        c, i, p, m, sc = t._native
        if plan.bits == 16 and plan.layout == "unstructured":
            fmt, bits, sc = _lib.FMT_BITMAP, 16, None
        elif plan.bits == 16:
            fmt, bits, sc = (_lib.FMT_STRUCT16 if plan.layout == "structured" else _lib.FMT_TILED), 16, None
        elif plan.layout == "structured":
            fmt, bits = _lib.FMT_STRUCT_INT4, 4
        else:
            fmt, bits, m = _lib.FMT_QUANT, int(plan.bits), None
        out.append(_ctensor(c, i, p, m, sc, fmt, bits))
        keep.extend(x for x in (c, i, p, m, sc) if x is not None)
    return out[0], out[1], tuple(keep)


def decode_splits(cache, num_q_heads, splits=0, rope_table=True):
    """Split count a decode of ``cache`` with ``num_q_heads`` query heads makes
    (``splits`` = 0: automatic, from the format kernel's per-CU occupancy)."""
    kdesc, vdesc, _keep = cache_descriptors(cache)
    b, kh = cache.key.centroids.shape[:2]
    n = _lib.lib().reskv_decode_splits(kdesc, vdesc, int(bool(rope_table)), b, int(num_q_heads), kh, cache.seq_len,
                                       int(splits))
    _lib.check(0 if n > 0 else 1, "decode_splits")
    return n


class StepDecoder:
    """Repeated decode steps of one layer against a fixed compressed history and
    a dense ring of recent tokens, without per-call validation or allocation.

    Descriptors, the RoPE table, the split workspace and the outputs are made
    once for a CompressedKV; each ``run`` issues the fused decode and the
    in-place ring merge (rows of ``ring_stride`` tokens) as two kernels
    (``reskv_decode_recent``).  The result equals ``attention(query, cache,
    position=..., recent=(...))``."""

    def __init__(self, cache, num_q_heads, scaling, inv_freq=None, rope_theta=500000.0, splits=0):
        self.cache = cache
        self.kdesc, self.vdesc, self.keep = cache_descriptors(cache)
        dev = cache.key.payload.device
        self.dev = dev
        self.b, self.kh = cache.key.centroids.shape[:2]
        self.nh = int(num_q_heads)
        self.t = cache.seq_len
        self.scaling = float(scaling)
        self.freq, self.table = _rope(inv_freq, rope_theta, dev, self.t)
        L = _lib.lib()
        self.splits = int(splits)
        self.ws = _workspace(L.reskv_decode_workspace_bytes(self.b, self.nh, self.kh, self.t, self.splits), dev)
        rows = self.b * self.nh
        self.out = torch.empty((rows, 128), dtype=torch.float16, device=dev)
        self.m = torch.empty((rows,), dtype=torch.float32, device=dev)
        self.l = torch.empty((rows,), dtype=torch.float32, device=dev)
        self.merged = torch.empty((rows, 128), dtype=torch.float16, device=dev)

    def run(self, query, position, query_rot=None, ring_k=None, ring_v=None, ring_len=0, ring_stride=0, out=None):
        """query fp16 [B, Hq, 1, 128] pre-RoPE (contiguous); ring_k/ring_v fp16
        [B, Hk, ring_stride, 128] buffers whose first ring_len tokens are the
        recent window (rotated K, V); query_rot its rotated query.  Returns
        fp16 [B, Hq, 1, 128]: ``out`` (contiguous fp16 with B * Hq * 128
        elements) when given, else a buffer reused by the next call.  With a
        recent window the split merge joins it in the same launch
        (``reskv_decode_recent``)."""
        L = _lib.lib()
        stream = _stream(self.dev)
        if out is not None:
            _require(out.dtype == torch.float16 and out.is_contiguous() and out.numel() == self.b * self.nh * 128
                     and out.device == self.dev, "out must be contiguous fp16 with B * Hq * 128 elements")
        if ring_len <= 0:
            dst = self.out if out is None else out
            _lib.check(L.reskv_decode_rope(query.data_ptr(), self.kdesc, self.vdesc, self.freq.data_ptr(),
                                           self.table.data_ptr(), self.b, self.nh, self.kh, self.t, 0, int(position),
                                           self.scaling, self.splits, dst.data_ptr(), self.m.data_ptr(),
                                           self.l.data_ptr(), self.ws.data_ptr(), self.ws.numel(), stream), "decode")
            return dst.view(self.b, self.nh, 1, 128)
        dst = self.merged if out is None else out
        _lib.check(L.reskv_decode_recent(query.data_ptr(), self.kdesc, self.vdesc, self.freq.data_ptr(),
                                         self.table.data_ptr(), self.b, self.nh, self.kh, self.t, 0, int(position),
                                         self.scaling, self.splits, query_rot.data_ptr(), ring_k.data_ptr(),
                                         ring_v.data_ptr(), int(ring_len), int(ring_stride), dst.data_ptr(),
                                         self.ws.data_ptr(), self.ws.numel(), stream), "decode")
        return dst.view(self.b, self.nh, 1, 128)


def decode_step(query2d, cache, num_q_heads, *, position, start_position, scaling, inv_freq, rope_theta,
                splits=0, recent=None):
    """One decode call over a CompressedKV: fp16 [B*Hq, 128].

    query2d fp16 [B*Hq, 128] pre-RoPE, contiguous.  ``recent`` is None or
    (rotated query fp16 [B*Hq, 128], rotated K and V fp16 [B, Hk, Tr, 128],
    contiguous); the split merge then joins the window before it writes the
    output (``reskv_decode_recent``), so a step is two kernel launches.
    """
    kdesc, vdesc, keep = cache_descriptors(cache)
    dev = query2d.device
    _dev_check(query2d, *keep, contiguous=False)
    b, kh = cache.key.centroids.shape[:2]
    nh, t = int(num_q_heads), cache.seq_len
    freq, table = _rope(inv_freq, rope_theta, dev, int(start_position) + t)
    L = _lib.lib()
    out = _empty((b * nh, 128), torch.float16, dev)
    ws = _workspace(L.reskv_decode_workspace_bytes(b, nh, kh, t, int(splits)), dev)
    common = (query2d.data_ptr(), kdesc, vdesc, freq.data_ptr(), table.data_ptr(), b, nh, kh, t,
              int(start_position), int(position), float(scaling), int(splits))
    with torch.cuda.device(dev):
        if recent is None:
            _lib.check(L.reskv_decode_rope(*common, out.data_ptr(), None, None, ws.data_ptr(), ws.numel(),
                                           _stream(dev)), "decode")
        else:
            q_rot, k_rec, v_rec = recent
            _dev_check(q_rot, k_rec, v_rec)
            tr = int(k_rec.shape[2])
            _lib.check(L.reskv_decode_recent(*common, q_rot.data_ptr(), k_rec.data_ptr(), v_rec.data_ptr(), tr, tr,
                                             out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev)), "decode")
    return out


def _check_recent_inputs(comp_out, comp_m, comp_l, v_recent, nh_kv, nh):
    """Shape and dtype checks shared by both merge_recent ops
    (reskv/csrc/attention.cu:850-868, cluster_mass.cu:1469-1476); returns (B, Tr)."""
    _require(comp_out.dim() == 2 and comp_out.shape[1] == 128, "comp_out must be [B*nh, 128]")
    _require(comp_out.dtype == torch.float16, "comp_out must be fp16")
    _require(comp_m.dim() == 1 and comp_l.dim() == 1, "comp_m/comp_l must be [B*nh]")
    _require(comp_m.dtype == torch.float32 and comp_l.dtype == torch.float32, "comp_m/comp_l must be fp32")
    _require(nh_kv > 0 and nh % nh_kv == 0, "num_q_heads must be divisible by num_kv_heads")
    _require(nh // nh_kv in (1, 2, 4, 8), f"Unsupported GQA ratio: {nh // max(nh_kv, 1)}")
    _require(comp_out.shape[0] % nh == 0, "Q/comp_out batch-head mismatch")
    b = comp_out.shape[0] // nh
    _require(comp_m.shape[0] == b * nh and comp_l.shape[0] == b * nh, "comp_m/comp_l must be [B*nh]")
    _require(v_recent.dim() == 4 and v_recent.shape[3] == 128, "v_recent must be [B, nh_kv, T, 128]")
    _require(v_recent.dtype == torch.float16, "v_recent must be fp16")
    _require(v_recent.shape[0] == b and v_recent.shape[1] == nh_kv, "v_recent shape mismatch")
    return b, int(v_recent.shape[2])


def _fixed_shift_stats(res):
    """The fixed-shift softmax's statistics (cluster_mass.cu:660, 874-888,
    1046-1067): the reference sums exp(score) with the shift held at 0, so it
    returns m = 0 and l = sum exp(score).  The online sum gives the same
    normaliser as l * exp(m), which overflows to inf where the reference's
    unshifted sum does (scores above about 88).  The output is the online
    one: where the reference's sums overflow, its output divides overflowed
    sums (inf / inf = NaN, or 0 for a channel whose weighted sum stayed
    finite), while this output stays the finite softmax average.  That
    overflow case is parity unpinned; wherever the unshifted sums are finite
    the outputs agree within the decode tolerance."""
    if len(res) == 3:
        out, m, l = res
        res = [out, torch.zeros_like(m), l * torch.exp(m)]
    return res


def _make_cluster_mass(plan=None):
    fixed_shift = bool(plan is not None and plan.fixed_shift)

    def decode_fp16(Q, kc, ki, kp, kbitmap, vc, vi, vp, vbitmap, nh_kv, nh, start_pos, pos_q, rope_base,
                    scaling, return_stats, splits, inv_freq):
        """Deferred unstructured FP16 decode (reskv/csrc/cluster_mass.cu:1177-1296)."""
        for t, name in ((kp, "k_sparse"), (vp, "v_sparse")):
            _require(t.dtype == torch.float16, f"cmass fp16 sparse-only: {name} must be fp16")
        for t in (kbitmap, vbitmap):
            _require(t.dtype == torch.int64 and t.shape[-1] == 2, "bitmaps must be int64 [B*nh_kv, T, 2]")
        kd = _ctensor(kc, ki, kp, kbitmap, None, _lib.FMT_BITMAP, 16)
        vd = _ctensor(vc, vi, vp, vbitmap, None, _lib.FMT_BITMAP, 16)
        return _decode(Q, kd, vd, (kc, ki, kp, kbitmap, vc, vi, vp, vbitmap), nh_kv, nh, start_pos, pos_q,
                       rope_base, scaling, splits, inv_freq, bool(return_stats))

    def _structured(int4):
        def op(Q, kc, ki, kqv, kmeta, kscale, vc, vi, vqv, vmeta, vscale, nh_kv, nh, start_pos, pos_q, rope_base,
               scaling, return_stats, splits, inv_freq):
            want = torch.int32 if int4 else torch.float16
            _require(kqv.dtype == want and vqv.dtype == want, "structured payload dtype mismatch")
            _require(kmeta.dtype == torch.int32 and vmeta.dtype == torch.int32, "structured metadata must be int32")
            _require(kmeta.shape[-1] == (2 if int4 else 4) and vmeta.shape[-1] == (2 if int4 else 4),
                     "structured metadata width mismatch")
            _require(kqv.shape[-1] == (4 if int4 else 32) and vqv.shape[-1] == (4 if int4 else 32),
                     "4:16 structured payload width mismatch")
            fmt = _lib.FMT_STRUCT_INT4 if int4 else _lib.FMT_STRUCT16
            bits = 4 if int4 else 16
            ks = kscale if int4 else None
            vs = vscale if int4 else None
            if int4:
                _require(ks is not None and ks.numel() and vs is not None and vs.numel(),
                         "INT4 structured scales must be fp16")
            kd = _ctensor(kc, ki, kqv, kmeta, ks, fmt, bits)
            vd = _ctensor(vc, vi, vqv, vmeta, vs, fmt, bits)
            keep = (kc, ki, kqv, kmeta, vc, vi, vqv, vmeta) + ((ks, vs) if int4 else ())
            res = _decode(Q, kd, vd, keep, nh_kv, nh, start_pos, pos_q, rope_base, scaling, splits, inv_freq,
                          bool(return_stats))
            # the reference compiles the fixed shift into its structured INT4 kernel only
            return _fixed_shift_stats(res) if int4 and fixed_shift else res

        op.__doc__ = ("Deferred structured %s decode (reskv/csrc/cluster_mass.cu:1298-1459)."
                      % ("INT4" if int4 else "FP16"))
        return op

    def merge_recent(comp_out, comp_m, comp_l, scores_recent, v_recent, nh_kv, nh):
        """Joint softmax with precomputed fp32 recent scores (reskv/csrc/cluster_mass.cu:1461-1508)."""
        nh_kv, nh = int(nh_kv), int(nh)
        b, tr = _check_recent_inputs(comp_out, comp_m, comp_l, v_recent, nh_kv, nh)
        _require(scores_recent.dtype == torch.float32 and scores_recent.dim() == 3, "scores must be fp32 [B,nh,Tr]")
        _require(tuple(scores_recent.shape) == (b, nh, tr), "scores_recent must be [B, nh, T_recent]")
        dev = _dev_check(comp_out, comp_m, comp_l, scores_recent, v_recent)
        out = torch.empty_like(comp_out)
        with torch.cuda.device(dev):
            _lib.check(_lib.lib().reskv_merge_recent_scores(
                comp_out.data_ptr(), comp_m.data_ptr(), comp_l.data_ptr(), _ptr(scores_recent), _ptr(v_recent),
                b, nh, nh_kv, tr, out.data_ptr(), _stream(dev)), "merge_recent")
        return out

    return SimpleNamespace(decode_fp16=decode_fp16, decode_structured_fp16=_structured(False),
                           decode_structured_int4=_structured(True), merge_recent=merge_recent)


def _make_attention(plan):
    struct_index = plan is not None and plan.layout == "structured"

    def _per_token(int4):
        def op(Q, kc, ki, kp, km, ks, vc, vi, vp, vm, vs, nh_kv, nh, start_pos, pos_q, rope_base, scaling, splits,
               inv_freq):
            want = torch.int32 if int4 else torch.float16
            _require(kp.dtype == want and vp.dtype == want, "payload dtype mismatch")
            _require(km.dtype == torch.int32 and vm.dtype == torch.int32, "k_qmeta/v_qmeta must be int32")
            if int4:
                fmt, bits = _lib.FMT_STRUCT_INT4, 4
                _require(ks is not None and ks.numel() and vs is not None and vs.numel(), "INT4 scales must be fp16")
            else:
                fmt = _lib.FMT_STRUCT16 if struct_index else _lib.FMT_TILED
                bits, ks, vs = 16, None, None
            kd = _ctensor(kc, ki, kp, km, ks, fmt, bits)
            vd = _ctensor(vc, vi, vp, vm, vs, fmt, bits)
            keep = (kc, ki, kp, km, vc, vi, vp, vm) + ((ks, vs) if int4 else ())
            return _decode(Q, kd, vd, keep, nh_kv, nh, start_pos, pos_q, rope_base, scaling, splits, inv_freq)

        op.__doc__ = "Per-token %s decode (reskv/csrc/attention.cu:665-835)." % ("INT4" if int4 else "FP16")
        return op

    def decode_quantized(Q, kc, ki, kp, ks, vc, vi, vp, vs, nh_kv, nh, start_pos, pos_q, rope_base, scaling,
                         k_bits, v_bits, splits, inv_freq):
        """Per-token unstructured INT4/INT2 decode (reskv/csrc/attention.cu:1296-1348)."""
        _require(kp.dtype == torch.int32 and vp.dtype == torch.int32, "quantized payloads must be int32")
        _require(int(k_bits) in (2, 4) and int(v_bits) in (2, 4), "bit widths must be 2 or 4")
        kd = _ctensor(kc, ki, kp, None, ks, _lib.FMT_QUANT, int(k_bits))
        vd = _ctensor(vc, vi, vp, None, vs, _lib.FMT_QUANT, int(v_bits))
        return _decode(Q, kd, vd, (kc, ki, kp, ks, vc, vi, vp, vs), nh_kv, nh, start_pos, pos_q, rope_base,
                       scaling, splits, inv_freq)

    def merge_recent(comp_out, comp_m, comp_l, Q_rope, k_recent, v_recent, nh_kv, nh, scaling):
        """Joint softmax with dense rotated recent tokens (reskv/csrc/attention.cu:839-906)."""
        nh_kv, nh = int(nh_kv), int(nh)
        b, tr = _check_recent_inputs(comp_out, comp_m, comp_l, v_recent, nh_kv, nh)
        _require(Q_rope.dim() == 2 and Q_rope.shape[1] == 128, "Q_rope must be [B*nh, 128]")
        _require(Q_rope.dtype == torch.float16, "Q_rope must be fp16")
        _require(Q_rope.shape[0] == comp_out.shape[0], "Q/comp_out batch-head mismatch")
        _require(k_recent.dim() == 4 and k_recent.shape[3] == 128, "k_recent must be [B, nh_kv, T, 128]")
        _require(k_recent.dtype == torch.float16, "k_recent must be fp16")
        _require(k_recent.shape == v_recent.shape, "v_recent shape mismatch")
        _require(tr > 0, "T_recent must be > 0")
        dev = _dev_check(comp_out, comp_m, comp_l, Q_rope, k_recent, v_recent)
        out = torch.empty_like(comp_out)
        with torch.cuda.device(dev):
            _lib.check(_lib.lib().reskv_merge_recent_qk(
                comp_out.data_ptr(), comp_m.data_ptr(), comp_l.data_ptr(), _ptr(Q_rope), _ptr(k_recent),
                _ptr(v_recent), b, nh, nh_kv, tr, tr, float(scaling), out.data_ptr(), _stream(dev)), "merge_recent")
        return out

    return SimpleNamespace(decode_fp16=_per_token(False), decode_int4=_per_token(True),
                           decode_quantized=decode_quantized, merge_recent=merge_recent)


def _make_compression():
    return SimpleNamespace(compress_fp16=compress_fp16, compress_quantized=compress_quantized,
                           compress_structured_int4=compress_structured_int4, compress_bitmap=compress_bitmap,
                           compress_fp16_kv=compress_fp16_kv, compress_bitmap_kv=compress_bitmap_kv,
                           kmeans=kmeans, kmeans_kv=kmeans_kv, kmeans_assign=kmeans_assign)


@lru_cache(maxsize=32)
def load_extension(family: str, plan: KernelPlan | None = None, device_index: int = 0):
    """Operator namespace for ``family`` (reskv/_extension.py:14-61).

    Raises ValueError for an unknown family and RuntimeError when the HIP
    library is unavailable; there is no CPU fallback.
    """
    if family not in FAMILIES:
        raise ValueError(f"unknown native family: {family}")
    _lib.lib()
    if family == "compression":
        return _make_compression()
    if family == "attention":
        return _make_attention(plan)
    return _make_cluster_mass(plan)


def dense_decode(q, k, v, inv_freq, *, position, start_position=0, scaling=None, splits=0, out=None):
    """Dense fp16 decode attention baseline on the same split-K engine.

    q fp16 [B, Hq, 1, 128] pre-RoPE; k, v fp16 [B, H, T, 128] (k pre-RoPE),
    contiguous or the first T tokens of a preallocated [B, H, Tmax, 128] cache.
    Returns fp16 [B, Hq, 1, 128], written to ``out`` (contiguous fp16 with
    B * Hq * 128 elements) when given.
    """
    _require(q.dtype == torch.float16 and k.dtype == torch.float16 and v.dtype == torch.float16, "fp16 inputs")
    dev = _dev_check(q, contiguous=True)
    _dev_check(q, k, v, contiguous=False)
    b, hq = q.shape[:2]
    h, t = k.shape[1], k.shape[2]
    _require(v.shape == k.shape and k.dim() == 4 and k.shape[3] == 128, "K and V must be [B, H, T, 128]")
    ts = k.stride(1) // 128
    for x in (k, v):
        _require(x.stride(3) == 1 and x.stride(2) == 128 and x.stride(1) == ts * 128
                 and (x.shape[0] == 1 or x.stride(0) == h * x.stride(1)),
                 "K/V must be contiguous or a token prefix of a [B, H, Tmax, 128] buffer")
    scale = 128 ** -0.5 if scaling is None else float(scaling)
    # sin/cos evaluated in-kernel (no table): the dense stream leaves VALU time to
    # spare, while table reads would compete with it for the caches
    freq = _frequencies(inv_freq, 500000.0, dev)
    L = _lib.lib()
    if out is None:
        out = _empty((b * hq, 128), torch.float16, dev)
    else:
        _require(out.dtype == torch.float16 and out.is_contiguous() and out.numel() == b * hq * 128
                 and out.device == dev, "out must be contiguous fp16 with B * Hq * 128 elements")
    ws = _workspace(L.reskv_decode_workspace_bytes(b, hq, h, t, int(splits)), dev)
    with torch.cuda.device(dev):
        _lib.check(L.reskv_decode_dense(q.data_ptr(), k.data_ptr(), v.data_ptr(), freq.data_ptr(), None,
                                        b, hq, h, t, ts, int(start_position), int(position), scale, int(splits),
                                        out.data_ptr(), None, None, ws.data_ptr(), ws.numel(), _stream(dev)),
                   "decode_dense")
    return out.reshape(b, hq, 1, 128)
