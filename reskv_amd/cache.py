"""Two-segment decode cache: compressed history plus a bounded dense ring.

Behaviour follows ``reskv/cache.py:11-122`` (``ResKVLayerCache``,
``ResKVCache``):

* At prefill, the first ``floor(max(0, T - recent) / group) * group`` tokens are
  compressed. The rest (rotated K, pre-RoPE K and V) go into a dense ring of
  ``recent_size + group_size`` slots.
* Each decode step appends one token to the ring.
* When the ring is full, its oldest ``group_size`` tokens are compressed
  against the shared centroid tables (``previous=``) and dropped from the ring.

The compressed history lives in device buffers with preallocated capacity,
instead of being re-concatenated (``torch.cat``) at every group. Capacity
doubles when it runs out. ``compressed`` is a ``CompressedKV`` of views into
those buffers; the decode kernels read the views in place through their row
strides. When transformers is importable the classes derive from its
``CacheLayerMixin`` / ``Cache`` (as the reference's do), so ``generate`` and the
mask builders accept them; without it they are the same methods duck-typed.
"""

import torch

try:
    from transformers.cache_utils import Cache as _CacheBase, CacheLayerMixin as _LayerBase
except ImportError:  # the kernels and the harness do not need transformers
    _CacheBase = _LayerBase = object

from ._extension import StepDecoder
from .compression import _compress_group, compress
from .config import ResKVKernelConfig
from .tensors import CompressedKV, CompressedTensor


class _Store:
    """Capacity buffers for one compressed tensor (K or V) of one layer."""

    def __init__(self, ct: CompressedTensor, max_clusters: int, capacity: int):
        b, h, t = ct.cluster_ids.shape
        dev = ct.payload.device
        self.plan = ct.plan
        self.max_clusters = max_clusters
        self.cent = torch.zeros(b, h, max_clusters, 128, dtype=torch.float16, device=dev)
        self.nc = 0
        cap = max(capacity, t)
        self.ids = torch.empty(b, h, cap, dtype=torch.int8, device=dev)
        self.payload = torch.empty(b, h, cap, ct.payload.shape[-1], dtype=ct.payload.dtype, device=dev)
        self.meta = None if ct.metadata is None else torch.empty(
            b, h, cap, ct.metadata.shape[-1], dtype=ct.metadata.dtype, device=dev)
        self.scale = None if ct.scale is None else torch.empty(b, h, cap, dtype=ct.scale.dtype, device=dev)
        self.n = 0
        self.append(ct)

    @property
    def capacity(self) -> int:
        return self.ids.shape[2]

    def _grow(self, need: int):
        cap = self.capacity
        while cap < need:
            cap *= 2

        def regrow(buf):
            if buf is None:
                return None
            new = torch.empty((*buf.shape[:2], cap, *buf.shape[3:]), dtype=buf.dtype, device=buf.device)
            new[:, :, : self.n].copy_(buf[:, :, : self.n])
            return new

        self.ids, self.payload = regrow(self.ids), regrow(self.payload)
        self.meta, self.scale = regrow(self.meta), regrow(self.scale)

    def append(self, ct: CompressedTensor):
        """Copy ct's tokens after the stored ones and adopt its centroid table."""
        t = ct.cluster_ids.shape[2]
        nc = ct.centroids.shape[2]
        if nc > self.max_clusters:
            raise ValueError("centroid table exceeds the configured limit")
        if self.n + t > self.capacity:
            self._grow(self.n + t)
        end = self.n + t
        self.cent[:, :, :nc].copy_(ct.centroids)
        self.nc = nc
        self.ids[:, :, self.n:end].copy_(ct.cluster_ids)
        self.payload[:, :, self.n:end].copy_(ct.payload)
        if self.meta is not None:
            self.meta[:, :, self.n:end].copy_(ct.metadata)
        if self.scale is not None:
            self.scale[:, :, self.n:end].copy_(ct.scale)
        self.n = end

    def view(self) -> CompressedTensor:
        n = self.n
        return CompressedTensor(
            self.cent[:, :, : self.nc], self.ids[:, :, :n], self.payload[:, :, :n],
            None if self.meta is None else self.meta[:, :, :n],
            None if self.scale is None else self.scale[:, :, :n], self.plan)

    def select(self, index: torch.Tensor):
        """Keep the batch rows in ``index`` (beam reordering)."""
        for name in ("cent", "ids", "payload", "meta", "scale"):
            buf = getattr(self, name)
            if buf is not None:
                setattr(self, name, buf.index_select(0, index.to(buf.device)))


class ResKVLayerCache(_LayerBase):
    """One layer's cache (reskv/cache.py:11-103)."""

    is_sliding = False
    is_compileable = False

    def __init__(self, config: ResKVKernelConfig, capacity: int | None = None):
        self.config = config
        self.capacity_hint = capacity
        self.keys = self.values = self.raw_keys = None
        self.length = 0
        self.live = 0
        self.plan = None
        self.is_initialized = False
        self._k = self._v = None
        self._view = None
        self._stepper = None

    # -- state ---------------------------------------------------------------
    @property
    def compressed(self) -> CompressedKV | None:
        """The compressed history as views into the capacity buffers, or None."""
        if self._k is None:
            return None
        if self._view is None:
            self._view = CompressedKV(self._k.view(), self._v.view())
        return self._view

    def lazy_initialization(self, key_states, value_states=None):
        b, h, _, d = key_states.shape
        shape = (b, h, self.config.recent_size + self.config.group_size, d)
        self.keys = torch.empty(shape, device=key_states.device, dtype=key_states.dtype)
        self.raw_keys = torch.empty_like(self.keys)
        self.values = torch.empty_like(self.keys)
        self.plan = self.config.resolve(b)
        self.is_initialized = True

    def _store(self, ckv: CompressedKV, extra: int):
        cap = self.capacity_hint if self.capacity_hint is not None else ckv.seq_len + extra
        self._k = _Store(ckv.key, self.config.max_clusters, cap)
        self._v = _Store(ckv.value, self.config.max_clusters, cap)
        self._view = None

    # -- update (reskv/cache.py:32-77) ---------------------------------------
    def update(self, key_states, value_states, cache_kwargs=None):
        """Add rotated K, V (and ``cache_kwargs["raw_keys"]``, pre-RoPE K); return the dense ring."""
        raw = (cache_kwargs or {}).get("raw_keys")
        if raw is None:
            raise ValueError("ResKV cache update requires pre-RoPE raw_keys")
        q_len = key_states.shape[2]
        if not self.is_initialized:
            self.lazy_initialization(key_states)
        group, recent = self.config.group_size, self.config.recent_size
        if self.length == 0:
            compressed_len = max(0, q_len - recent) // group * group
            if compressed_len:
                ckv = compress(raw[:, :, :compressed_len].contiguous(),
                               value_states[:, :, :compressed_len].contiguous(), self.config, plan=self.plan)
                self._store(ckv, extra=16 * group)
            self.live = q_len - compressed_len
            self.keys[:, :, : self.live].copy_(key_states[:, :, compressed_len:])
            self.raw_keys[:, :, : self.live].copy_(raw[:, :, compressed_len:])
            self.values[:, :, : self.live].copy_(value_states[:, :, compressed_len:])
        else:
            if q_len != 1:
                raise ValueError("ResKV continuation supports one token per step; chunked prefill is unsupported")
            self.keys[:, :, self.live: self.live + 1].copy_(key_states)
            self.raw_keys[:, :, self.live: self.live + 1].copy_(raw)
            self.values[:, :, self.live: self.live + 1].copy_(value_states)
            self._take_token()
            return self.keys[:, :, : self.live], self.values[:, :, : self.live]
        self.length += q_len
        return self.keys[:, :, : self.live], self.values[:, :, : self.live]

    def advance(self):
        """Accounts for one decode token that the caller has already written into
        ring slot ``live`` of ``keys`` (rotated K), ``raw_keys`` (pre-RoPE K)
        and ``values``, e.g. from a captured graph; otherwise the same as
        ``update`` with that token (the ring is compressed by a group when full)."""
        if not self.is_initialized or self.length == 0:
            raise ValueError("advance() continues a prefilled cache")
        self._take_token()

    def _take_token(self):
        """One more token in the ring; a full ring gives its oldest group to the compressed history."""
        group = self.config.group_size
        self.live += 1
        self.length += 1
        if self.live < self.keys.shape[2]:
            return
        k_grp = self.raw_keys[:, :, :group].contiguous()
        v_grp = self.values[:, :, :group].contiguous()
        if self._k is None:
            self._store(compress(k_grp, v_grp, self.config, plan=self.plan), extra=16 * group)
        else:
            k, v = _compress_group(k_grp, v_grp, self.config, self.compressed, self.plan)
            self._k.append(k)
            self._v.append(v)
            self._view = None
        remain = self.live - group
        for buf in (self.keys, self.raw_keys, self.values):
            buf[:, :, :remain].copy_(buf[:, :, group: self.live].clone())
        self.live = remain

    # -- decode attention (reskv/models/llama.py:45-60) ------------------------
    def attend(self, query, query_rot, *, scaling, inv_freq=None, rope_theta=500000.0, out=None):
        """Attention of the newest token (after ``update``) over the compressed
        history and the dense ring, as the model patch computes it with
        ``attention(query, self.compressed, position=self.length - 1,
        recent=(query_rot, ring K, ring V))``.  Repeated steps reuse the
        descriptors, RoPE table and buffers until a group compression changes
        the history; the ring is read in place.  query / query_rot fp16
        [B, Hq, 1, 128] (pre-RoPE / rotated, contiguous).  The result goes to
        ``out`` (contiguous fp16, B * Hq * 128 elements) when given; otherwise
        the returned tensor is reused by the next call."""
        cv = self.compressed
        if cv is None:
            raise ValueError("no compressed history yet; attend over the ring densely")
        if self._stepper is None or self._stepper.cache is not cv:
            self._stepper = StepDecoder(cv, query.shape[1], scaling, inv_freq, rope_theta)
        return self._stepper.run(query, self.length - 1, query_rot, self.keys, self.values, self.live,
                                 self.keys.shape[2], out=out)

    # -- queries -------------------------------------------------------------
    def get_seq_length(self, *_):
        return self.length

    def get_mask_sizes(self, query, *_):
        """(kv length, offset) for the next query; ``query`` is its cache_position (or its length)."""
        q = query if isinstance(query, int) else query.shape[0]
        return self.length + q, 0

    def get_max_cache_shape(self):
        return -1

    def get_max_length(self):
        return -1

    def reset(self):
        self.keys = self.values = self.raw_keys = None
        self._k = self._v = self._view = None
        self._stepper = None
        self.length = self.live = 0
        self.plan = None
        self.is_initialized = False

    def reorder_cache(self, beam_idx):
        if self.is_initialized:
            index = beam_idx.to(self.keys.device)
            self.keys = self.keys.index_select(0, index)
            self.raw_keys = self.raw_keys.index_select(0, index)
            self.values = self.values.index_select(0, index)
            if self._k is not None:
                self._k.select(index)
                self._v.select(index)
                self._view = None


class ResKVCache(_CacheBase):
    """Per-layer ResKV caches for a decoder stack (reskv/cache.py:106-122)."""

    def __init__(self, config: ResKVKernelConfig, num_layers: int, capacity: int | None = None):
        layers = [ResKVLayerCache(config, capacity) for _ in range(num_layers)]
        if _CacheBase is object:
            self.layers = layers
        else:
            super().__init__(layers=layers)
        self.config = config

    def __len__(self):
        return len(self.layers)

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        return self.layers[layer_idx].update(key_states, value_states, cache_kwargs)

    def get_seq_length(self, layer_idx=0):
        return self.layers[layer_idx].get_seq_length()

    def get_mask_sizes(self, query_length, layer_idx=0):
        return self.layers[layer_idx].get_mask_sizes(query_length)

    def crop(self, max_length):
        raise NotImplementedError("ResKV does not support speculative cache rollback")

    def reorder_cache(self, beam_idx):
        for layer in self.layers:
            layer.reorder_cache(beam_idx)

    def batch_repeat_interleave(self, repeats):
        for layer in self.layers:
            if layer.is_initialized:
                indices = torch.arange(layer.keys.shape[0], device=layer.keys.device).repeat_interleave(repeats)
                layer.reorder_cache(indices)

    def batch_select_indices(self, indices):
        self.reorder_cache(indices)
