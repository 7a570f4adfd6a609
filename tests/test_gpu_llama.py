"""End-to-end decode harness (random-init Llama shape) at a tiny size."""

import pytest
import torch

from reskv_amd import ResKVKernelConfig
from reskv_amd._extension import dense_decode
from reskv_amd.llama import GreedyDecoder, LlamaShape, RandomLlama, llama3_inv_freq

TINY = LlamaShape(layers=2, hidden=512, heads=4, kv_heads=1, ffn=1024, vocab=1000)


class _EagerAppend(GreedyDecoder):
    """The harness with the K/V append outside the graphs, through the cache's own
    ``update`` (ResKV) or slice copies (dense), and the output copied."""

    def _append_targets(self, li):
        return None

    def _attend(self, li):
        if self.mode == "reskv":
            layer = self.caches[li]
            layer.update(self.kr[:, :, None], self.v[:, :, None], {"raw_keys": self.k[:, :, None]})
            out = layer.attend(self.q[:, :, None], self.qr[:, :, None], scaling=self.model.scaling,
                               inv_freq=self.model.inv_freq)
        else:
            t = self.pos + 1
            self.kc[li][:, :, self.pos].copy_(self.k)
            self.vc[li][:, :, self.pos].copy_(self.v)
            out = dense_decode(self.q[:, :, None], self.kc[li][:, :, :t], self.vc[li][:, :, :t],
                               self.model.inv_freq, position=self.pos, scaling=self.model.scaling)
        self.attn.copy_(out.view(self.batch, -1, self.model.shape.head_dim))


def _run(mode, steps=70, prompt=256, batch=2, cls=GreedyDecoder):
    model = RandomLlama(TINY, "cuda", seed=1)
    ids = torch.randint(128, TINY.vocab, (batch, prompt), generator=torch.Generator().manual_seed(3)).cuda()
    cfg = ResKVKernelConfig(sparsity=0.75, num_clusters=8, kmeans_iterations=4)
    dec = cls(model, batch, prompt, steps, mode, cfg)
    keep = {}

    def sink(layer, raw_k, rot_k, v):
        keep[layer] = (raw_k.clone(), v.clone())
        dec.absorb(layer, raw_k, rot_k, v)

    first = model.prefill(ids, sink, q_rows=64)
    dec.start(first)
    toks = [dec.step().clone() for _ in range(steps)]
    torch.cuda.synchronize()
    return model, dec, keep, torch.stack(toks)


def test_llama3_frequencies_match_closed_form():
    inv = llama3_inv_freq(LlamaShape())
    base = 1.0 / (500000.0 ** (torch.arange(0, 128, 2).float() / 128))
    assert torch.allclose(inv[:8], base[:8])  # short wavelengths untouched
    assert torch.allclose(inv[-4:], base[-4:] / 8.0)  # long wavelengths divided by the factor


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["reskv", "dense"])
def test_decode_runs_and_keeps_cache_consistent(device, mode):
    model, dec, _, toks = _run(mode)
    assert toks.shape == (70, 2)
    assert int(toks.min()) >= 0 and int(toks.max()) < TINY.vocab
    assert torch.isfinite(dec.x.float()).all()
    if mode == "reskv":
        for layer in dec.caches:
            assert layer.get_seq_length() == 256 + 70
            assert layer.compressed.seq_len + layer.live == layer.get_seq_length()
            assert layer.live <= 96


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["reskv", "dense"])
def test_in_graph_append_equals_eager_update(device, mode):
    """Appending inside the captured graphs (slot from device memory) and writing the
    attention into the graph's buffer give bitwise the decode of the eager path, across
    a group compression (the 96-slot ring, 64 tokens after the prompt, fills at step 32)."""
    _, dec, _, toks = _run(mode)
    _, ref, _, ref_toks = _run(mode, cls=_EagerAppend)
    assert torch.equal(toks, ref_toks)
    assert torch.equal(dec.x, ref.x)
    if mode == "reskv":
        for a, b in zip(dec.caches, ref.caches):
            assert a.live == b.live and a.length == b.length
            assert torch.equal(a.keys[:, :, :a.live], b.keys[:, :, :b.live])
            assert torch.equal(a.values[:, :, :a.live], b.values[:, :, :b.live])
            assert torch.equal(a.compressed.key.payload, b.compressed.key.payload)


@pytest.mark.gpu
def test_dense_first_step_attention_matches_fp32(device):
    """The harness's dense attention (strided cache, in-kernel RoPE) against fp32 attention."""
    model = RandomLlama(TINY, "cuda", seed=2)
    ids = torch.randint(128, TINY.vocab, (2, 128), generator=torch.Generator().manual_seed(4)).cuda()
    dec = GreedyDecoder(model, 2, 128, 4, "dense")
    first = model.prefill(ids, dec.absorb, q_rows=64)
    dec.start(first)
    dec.capture()
    dec.graphs[0][0].replay()
    dec._attend(0)
    t = dec.pos + 1
    cos, sin = model.rope_tables(t)
    k = dec.kc[0][:, :, :t].float()
    kr = torch.cat((k[..., :64] * cos - k[..., 64:] * sin, k[..., 64:] * cos + k[..., :64] * sin), -1)
    v = dec.vc[0][:, :, :t].float()
    q = dec.qr.float()  # [B, Hq, 128] rotated at the step's position
    kr = kr.repeat_interleave(4, dim=1)
    v = v.repeat_interleave(4, dim=1)
    w = torch.softmax(torch.einsum("bhd,bhtd->bht", q, kr) * model.scaling, -1)
    ref = torch.einsum("bht,bhtd->bhd", w, v)
    assert (dec.attn.float() - ref).abs().max().item() <= 2e-3


@pytest.mark.gpu
def test_fused_decode_step_equals_the_torch_forward(device):
    """One graph-replayed decode step of the harness (fused RMSNorm, QKV split and
    rotation, gated activation, residual adds in the GEMMs, dense attention) gives
    the logits of the plain torch forward over the prompt plus that token."""
    model = RandomLlama(TINY, "cuda", seed=5)
    ids = torch.randint(128, TINY.vocab, (2, 96), generator=torch.Generator().manual_seed(6)).cuda()
    dec = GreedyDecoder(model, 2, 96, 4, "dense")
    first = model.prefill(ids, dec.absorb, q_rows=64)
    dec.start(first)
    dec.step()
    got = torch.nn.functional.linear(dec.h, model.lm_head).float()  # the head graph's normed hidden
    ref = model.prefill(torch.cat((ids, first[:, None]), 1), lambda *a: None, q_rows=64, logits=True).float()
    scale = ref.abs().max().item()
    assert (got - ref).abs().max().item() <= 2e-2 * scale
    assert torch.equal(dec.tok, ref.argmax(-1))
