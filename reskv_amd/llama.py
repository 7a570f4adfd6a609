"""Random-init Llama-3.1-8B-shaped decoder for the end-to-end decode benchmark.

The decode branch follows the reference model patch
(reskv/models/llama.py:36-72): each layer adds the new token's rotated K, V
and pre-RoPE ("raw") K to its ``ResKVLayerCache`` and attends with the
pre-RoPE query against the compressed history, merging the dense ring
(rotated Q/K and V) as the recent window.  The token is written into the ring
by the layer's captured graph (slot from device memory) and the cache then
accounts for it (``advance``), which is ``update`` without its copies.  The
dense baseline keeps pre-RoPE K and V in a preallocated fp16 cache, appended
the same way, and runs the same split-K engine over it
(``reskv_decode_dense``, which rotates K in-kernel like the compressed path).
Both write the attention output straight into the buffer the next graph reads.

No checkpoint can be fetched, so the weights are random (N(0, 0.02), unit
RMSNorm gains).  Around attention the work has fixed shapes -- RMSNorm, the
fused QKV projection and RoPE of the new token, the output projection and the
gated MLP, the LM head with greedy argmax and the next token's embedding --
and runs as HIP graphs, one before and one after each layer's attention.
Inside them the RMSNorms, the split / rotation / append of the new token's
Q, K and V, and the gated activation are single fused launches
(``include/reskv_llama.h``), and the residual adds ride in the projection
GEMMs (``addmm_``), so a layer's graphs hold eight kernels instead of about
fifty.  Attention and the cache bookkeeping, whose sizes change from step to
step, run eagerly through the library.
"""

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import _lib
from ._extension import dense_decode
from .cache import ResKVLayerCache
from .config import ResKVKernelConfig


@dataclass(frozen=True)
class LlamaShape:
    layers: int = 32
    hidden: int = 4096
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 14336
    vocab: int = 128256
    rope_theta: float = 500000.0
    rms_eps: float = 1e-5
    # llama3 rotary scaling (Llama-3.1): factor, low/high frequency factors, original context
    rope_factor: float = 8.0
    low_freq_factor: float = 1.0
    high_freq_factor: float = 4.0
    original_context: int = 8192


def llama3_inv_freq(shape: LlamaShape) -> torch.Tensor:
    """theta^(-2i/d) with the llama3 wavelength-dependent scaling of Llama-3.1."""
    inv = 1.0 / (shape.rope_theta ** (torch.arange(0, shape.head_dim, 2, dtype=torch.int64).float() / shape.head_dim))
    if shape.rope_factor == 1.0:
        return inv.float()
    low_wl = shape.original_context / shape.low_freq_factor
    high_wl = shape.original_context / shape.high_freq_factor
    wl = 2 * math.pi / inv
    scaled = torch.where(wl > low_wl, inv / shape.rope_factor, inv)
    smooth = (shape.original_context / wl - shape.low_freq_factor) / (shape.high_freq_factor - shape.low_freq_factor)
    smoothed = (1 - smooth) * scaled / shape.rope_factor + smooth * scaled
    medium = (wl >= high_wl) & (wl <= low_wl)
    return torch.where(medium, smoothed, scaled).float()


def _rmsnorm(x, w, eps):
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w).to(x.dtype)


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _need(cond, msg):
    if not cond:
        raise ValueError(msg)


def _fp16_rows(name, t, rows=None, width=None):
    """t must be a contiguous fp16 CUDA matrix (of the given rows / width)."""
    _need(t.dtype == torch.float16 and t.dim() == 2 and t.is_contiguous(), f"{name} must be a contiguous fp16 matrix")
    _need(rows is None or t.shape[0] == rows, f"{name} has {t.shape[0]} rows, expected {rows}")
    _need(width is None or t.shape[1] == width, f"{name} has {t.shape[1]} columns, expected {width}")


def _fp16_heads(name, t, b, heads):
    _need(t.dtype == torch.float16 and t.is_contiguous() and tuple(t.shape) == (b, heads, 128),
          f"{name} must be a contiguous fp16 tensor [{b}, {heads}, 128]")


def _on_gpu(*tensors):
    """Checked last, after every shape, dtype and layout check."""
    _need(all(t is None or t.is_cuda for t in tensors), "every tensor must be a CUDA tensor")


def fused_rmsnorm(x, w, eps, out):
    """``_rmsnorm`` of fp16 rows x [R, hidden] into out, one launch."""
    _fp16_rows("x", x)
    _fp16_rows("out", out, x.shape[0], x.shape[1])
    _need(w.dtype == torch.float16 and w.is_contiguous() and w.numel() == x.shape[1],
          "w must be a contiguous fp16 vector of the hidden size")
    _on_gpu(x, w, out)
    _lib.check(_lib.lib().reskv_llama_rmsnorm(x.data_ptr(), w.data_ptr(), out.data_ptr(), x.shape[0], x.shape[1],
                                              eps, _stream(x)), "reskv_llama_rmsnorm")
    return out


def fused_silu_mul(gu, out):
    """``silu(gu[:, :F]) * gu[:, F:]`` (fp16, as torch rounds it) into out [R, F], one launch."""
    _fp16_rows("out", out)
    _fp16_rows("gu", gu, out.shape[0], 2 * out.shape[1])
    _on_gpu(gu, out)
    _lib.check(_lib.lib().reskv_llama_silu_mul(gu.data_ptr(), out.data_ptr(), gu.shape[0], out.shape[1],
                                               _stream(gu)), "reskv_llama_silu_mul")
    return out


def fused_qkv_rope(qkv, cos, sin, pos, q, qr, k, kr, v, targets=None):
    """Splits qkv [B, (Hq + 2 Hk) * 128] into q, k, v, writes ``_rotate`` of q and k
    at position ``pos[0]`` (device) into qr, kr and, with ``targets = (rot, raw,
    v_cache, slot)`` ([B, Hk, cap, 128] tensors, any of the three None; slot a
    device int64), appends kr, k and v at token ``slot[0]``, one launch."""
    _need(q.dim() == 3 and k.dim() == 3, "q must be [B, Hq, 128] and k [B, Hk, 128]")
    b, hq, hk = q.shape[0], q.shape[1], k.shape[1]
    _fp16_rows("qkv", qkv, b, (hq + 2 * hk) * 128)
    for name, t, heads in (("q", q, hq), ("qr", qr, hq), ("k", k, hk), ("kr", kr, hk), ("v", v, hk)):
        _fp16_heads(name, t, b, heads)
    _need(all(t.dtype == torch.float32 and t.dim() == 2 and t.shape[1] == 64 and t.is_contiguous()
              for t in (cos, sin)) and cos.shape == sin.shape,
          "cos and sin must be contiguous fp32 tables [P, 64] of one shape")
    _need(pos.dtype == torch.int64 and pos.numel() >= 1, "pos must be an int64 tensor")
    rot = raw = vc = slot = None
    strides = (0, 0, 0)
    if targets is not None:
        rot, raw, vc, slot = targets
        _need(slot is not None and slot.dtype == torch.int64 and slot.numel() >= 1, "slot must be an int64 tensor")
        ref = next(t for t in (rot, raw, vc) if t is not None)
        for t in (rot, raw, vc):
            if t is not None and (t.dtype != torch.float16 or t.dim() != 4 or t.shape[3] != 128
                                  or t.stride() != ref.stride() or t.stride(3) != 1 or t.shape[:2] != (b, hk)):
                raise ValueError("cache append targets must share one [B, Hk, cap, 128] layout")
        strides = ref.stride()[:3]

    _on_gpu(qkv, cos, sin, pos, q, qr, k, kr, v, rot, raw, vc, slot)
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    _lib.check(_lib.lib().reskv_llama_qkv_rope(
        qkv.data_ptr(), cos.data_ptr(), sin.data_ptr(), pos.data_ptr(), b, hq, hk, q.data_ptr(), qr.data_ptr(),
        k.data_ptr(), kr.data_ptr(), v.data_ptr(), ptr(rot), ptr(raw), ptr(vc), ptr(slot), *strides,
        _stream(qkv)), "reskv_llama_qkv_rope")


def _rotate(x, cos, sin):
    """Rotate-half RoPE in fp32; x [..., 128], cos/sin broadcastable to [..., 64]."""
    xf = x.float()
    a, b = xf[..., :64], xf[..., 64:]
    return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1).to(x.dtype)


class RandomLlama:
    """fp16 weights of the Llama shape; QKV and gate/up projections fused."""

    def __init__(self, shape: LlamaShape = LlamaShape(), device="cuda", seed=0, std=0.02):
        self.shape = s = shape
        dev = torch.device(device)
        self.device = dev
        g = torch.Generator(device=dev)
        g.manual_seed(seed)

        def w(*size):
            return torch.randn(*size, generator=g, device=dev, dtype=torch.float16) * std

        kvd = s.kv_heads * s.head_dim
        self.embed = w(s.vocab, s.hidden)
        self.layers = []
        for _ in range(s.layers):
            self.layers.append({
                "wqkv": w(s.hidden + 2 * kvd, s.hidden), "wo": w(s.hidden, s.hidden),
                "wgu": w(2 * s.ffn, s.hidden), "wd": w(s.hidden, s.ffn),
                "n1": torch.ones(s.hidden, device=dev, dtype=torch.float16),
                "n2": torch.ones(s.hidden, device=dev, dtype=torch.float16),
            })
        self.norm = torch.ones(s.hidden, device=dev, dtype=torch.float16)
        self.lm_head = w(s.vocab, s.hidden)
        self.inv_freq = llama3_inv_freq(s).to(dev)
        self.scaling = s.head_dim ** -0.5

    def rope_tables(self, positions: int):
        """cos/sin fp32 [positions, 64] of the angles fl32(p * inv_freq)."""
        ang = torch.arange(positions, device=self.device, dtype=torch.float32)[:, None] * self.inv_freq[None, :]
        return torch.cos(ang), torch.sin(ang)

    def _split(self, qkv):
        s = self.shape
        kvd = s.kv_heads * s.head_dim
        q = qkv[..., : s.hidden].unflatten(-1, (s.heads, s.head_dim))
        k = qkv[..., s.hidden: s.hidden + kvd].unflatten(-1, (s.kv_heads, s.head_dim))
        v = qkv[..., s.hidden + kvd:].unflatten(-1, (s.kv_heads, s.head_dim))
        return q, k, v

    def _mlp(self, x, p, rows=16384):
        s = self.shape
        flat = x.view(-1, s.hidden)
        for r0 in range(0, flat.shape[0], rows):
            h = _rmsnorm(flat[r0: r0 + rows], p["n2"], s.rms_eps)
            gu = F.linear(h, p["wgu"])
            act = F.silu(gu[:, : s.ffn])
            act.mul_(gu[:, s.ffn:])
            flat[r0: r0 + rows] += F.linear(act, p["wd"])

    @torch.no_grad()
    def prefill(self, ids, sink, q_rows=2048, logits=False):
        """Causal forward of the prompt ids [B, T]; ``sink(layer, raw_k, rot_k, v)``
        receives each layer's keys and values as [B, Hk, T, 128].  Returns the
        greedy next token per sequence [B] (or, with ``logits``, the last
        position's logits [B, vocab])."""
        s = self.shape
        b, t = ids.shape
        cos, sin = self.rope_tables(t)
        x = self.embed[ids]  # [B, T, hidden]
        rep = s.heads // s.kv_heads
        causal = torch.ones(q_rows, t, dtype=torch.bool, device=self.device)
        for li, p in enumerate(self.layers):
            h = _rmsnorm(x, p["n1"], s.rms_eps)
            q, k, v = self._split(F.linear(h, p["wqkv"]))
            del h
            q = q.transpose(1, 2)
            k = k.transpose(1, 2).contiguous()
            v = v.transpose(1, 2).contiguous()
            qr = _rotate(q, cos, sin)
            kr = _rotate(k, cos, sin)
            sink(li, k, kr, v)
            attn = torch.empty(b, t, s.heads, s.head_dim, dtype=torch.float16, device=self.device)
            for bi in range(b):
                kt = kr[bi].repeat_interleave(rep, dim=0).transpose(1, 2).contiguous()  # [H, 128, T]
                vv = v[bi].repeat_interleave(rep, dim=0).contiguous()  # [H, T, 128]
                for r0 in range(0, t, q_rows):
                    r1 = min(t, r0 + q_rows)
                    sc = torch.matmul(qr[bi, :, r0:r1].contiguous(), kt).float() * self.scaling
                    mask = torch.triu(causal[: r1 - r0], diagonal=r0 + 1)
                    sc.masked_fill_(mask[None], float("-inf"))
                    pr = torch.softmax(sc, dim=-1).half()
                    attn[bi, r0:r1] = torch.matmul(pr, vv).transpose(0, 1)
            del q, k, v, qr, kr
            x += F.linear(attn.view(b, t, s.hidden), p["wo"])
            del attn
            self._mlp(x, p)
        last = _rmsnorm(x[:, -1], self.norm, s.rms_eps)
        out = F.linear(last, self.lm_head)
        return out if logits else torch.argmax(out, dim=-1)


class GreedyDecoder:
    """Batch greedy decoding, one token per sequence per step, over ResKV
    (``mode="reskv"``) or dense fp16 (``mode="dense"``) KV caches."""

    def __init__(self, model: RandomLlama, batch: int, prompt_len: int, max_new: int, mode: str,
                 kernel_config: ResKVKernelConfig | None = None):
        if mode not in ("reskv", "dense"):
            raise ValueError("mode must be 'reskv' or 'dense'")
        s = model.shape
        dev = model.device
        self.model, self.mode, self.batch = model, mode, batch
        self.pos = prompt_len
        self.max_pos = prompt_len + max_new
        self.cos, self.sin = model.rope_tables(self.max_pos)
        f16 = dict(dtype=torch.float16, device=dev)
        self.x = torch.zeros(batch, s.hidden, **f16)
        self.q = torch.zeros(batch, s.heads, s.head_dim, **f16)
        self.qr = torch.zeros_like(self.q)
        self.k = torch.zeros(batch, s.kv_heads, s.head_dim, **f16)
        self.kr = torch.zeros_like(self.k)
        self.v = torch.zeros_like(self.k)
        self.attn = torch.zeros(batch, s.heads, s.head_dim, **f16)
        self.h = torch.zeros(batch, s.hidden, **f16)  # RMSNorm output
        self.act = torch.zeros(batch, s.ffn, **f16)  # gated activation
        self.tok = torch.zeros(batch, dtype=torch.int64, device=dev)
        self.pos_buf = torch.zeros(1, dtype=torch.int64, device=dev)
        self.slot_buf = torch.zeros(1, dtype=torch.int64, device=dev)  # ring slot of the new token
        if mode == "reskv":
            cfg = kernel_config or ResKVKernelConfig(sparsity=0.75)
            self.caches = [ResKVLayerCache(cfg) for _ in range(s.layers)]
        else:
            shape = (batch, s.kv_heads, self.max_pos, s.head_dim)
            self.kc = [torch.zeros(shape, **f16) for _ in range(s.layers)]
            self.vc = [torch.zeros(shape, **f16) for _ in range(s.layers)]
        self.graphs = None

    # -- prefill hand-off ----------------------------------------------------
    def absorb(self, layer, raw_k, rot_k, v):
        """Takes one layer's prompt keys/values (the prefill sink)."""
        t = raw_k.shape[2]
        if self.mode == "reskv":
            self.caches[layer].update(rot_k, v, {"raw_keys": raw_k})
        else:
            self.kc[layer][:, :, :t].copy_(raw_k)
            self.vc[layer][:, :, :t].copy_(v)

    def start(self, first_token):
        self.tok.copy_(first_token)
        self.x.copy_(self.model.embed[self.tok])

    # -- fixed-shape parts as graphs -----------------------------------------
    def _pre(self, li, p):
        s = self.model.shape
        fused_rmsnorm(self.x, p["n1"], s.rms_eps, self.h)
        qkv = F.linear(self.h, p["wqkv"])
        fused_qkv_rope(qkv, self.cos, self.sin, self.pos_buf, self.q, self.qr, self.k, self.kr, self.v,
                       self._append_targets(li))

    def _append_targets(self, li):
        """Where the pre graph appends the new token's K/V in layer li's cache: ring
        slot ``live`` (ResKV: rotated K, pre-RoPE K, V) or position ``pos`` (dense:
        pre-RoPE K, V), read from device memory when the graph runs."""
        if self.mode == "reskv":
            layer = self.caches[li]
            return layer.keys, layer.raw_keys, layer.values, self.slot_buf
        return None, self.kc[li], self.vc[li], self.pos_buf

    def _set_slots(self):
        """Device copies of this step's position and ring slot (the layers' rings fill in step)."""
        self.pos_buf.fill_(self.pos)
        if self.mode == "reskv":
            self.slot_buf.fill_(self.caches[0].live)

    def _post(self, p):
        s = self.model.shape
        # residual adds in the GEMM epilogue: x = x + attn @ wo^T (one rounding)
        self.x.addmm_(self.attn.view(self.batch, s.hidden), p["wo"].t())
        fused_rmsnorm(self.x, p["n2"], s.rms_eps, self.h)
        fused_silu_mul(F.linear(self.h, p["wgu"]), self.act)
        self.x.addmm_(self.act, p["wd"].t())

    def _head(self):
        s = self.model.shape
        logits = F.linear(fused_rmsnorm(self.x, self.model.norm, s.rms_eps, self.h), self.model.lm_head)
        self.tok.copy_(torch.argmax(logits, dim=-1))
        self.x.copy_(self.model.embed.index_select(0, self.tok))

    def capture(self):
        """Records the fixed-shape parts once (after a warm-up on a side stream).
        The warm-up appends layer 0's token at this step's slot, which the
        step's own append then overwrites with the same values."""
        self._set_slots()
        x0, tok0 = self.x.clone(), self.tok.clone()
        side = torch.cuda.Stream(device=self.model.device)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for p in self.model.layers[:1]:
                self._pre(0, p)
                self._post(p)
            self._head()
        torch.cuda.current_stream().wait_stream(side)
        pool = torch.cuda.graph_pool_handle()
        pre, post = [], []
        for li, p in enumerate(self.model.layers):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                self._pre(li, p)
            pre.append(g)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                self._post(p)
            post.append(g)
        head = torch.cuda.CUDAGraph()
        with torch.cuda.graph(head, pool=pool):
            self._head()
        self.graphs = (pre, post, head)
        self.x.copy_(x0)
        self.tok.copy_(tok0)

    # -- attention ---------------------------------------------------------------
    def _attend(self, li):
        # the pre graph has already written the token's K/V into the cache
        if self.mode == "reskv":
            layer = self.caches[li]
            layer.advance()
            layer.attend(self.q[:, :, None], self.qr[:, :, None], scaling=self.model.scaling,
                         inv_freq=self.model.inv_freq, out=self.attn)
        else:
            t = self.pos + 1
            dense_decode(self.q[:, :, None], self.kc[li][:, :, :t], self.vc[li][:, :, :t], self.model.inv_freq,
                         position=self.pos, scaling=self.model.scaling, out=self.attn)

    def step(self, events=None):
        """One decode step for every sequence; returns the new tokens [B] (device).
        ``events`` (list) collects (before, after) CUDA events around each attention."""
        if self.pos >= self.max_pos:
            raise RuntimeError("decoder capacity exhausted")
        if self.graphs is None:
            self.capture()
        self._set_slots()
        pre, post, head = self.graphs
        for li in range(len(pre)):
            pre[li].replay()
            if events is not None:
                e0 = torch.cuda.Event(enable_timing=True)
                e0.record()
            self._attend(li)
            if events is not None:
                e1 = torch.cuda.Event(enable_timing=True)
                e1.record()
                events.append((e0, e1))
            post[li].replay()
        head.replay()
        self.pos += 1
        return self.tok
