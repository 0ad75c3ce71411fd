"""The model-level decode runtime on the CPU (float32, a tiny Llama shape).

* causal_attention equals a direct softmax(QK^T/sqrt(d) + causal mask) V;
* a cached decode step (cache write at pos, attention over 0..pos through the
  adapter contract) gives the same logits as recomputing the whole prefix;
* the exact decode backend equals torch SDPA on the CPU.
"""
import math

import torch
import torch.nn.functional as F

from santa_amd.runtime import (ExactDecodeBackend, LlamaShape, NHDCache, RandomLlama, causal_attention,
                               decode_deviation, greedy_decode)

TINY = LlamaShape(hidden=128, intermediate=256, heads=8, kv_heads=2, layers=2, vocab=97)


def test_causal_attention_matches_direct_softmax():
    g = torch.Generator().manual_seed(0)
    B, P, H, KVH, D = 2, 37, 8, 2, 16
    q, k, v = (torch.randn(B, P, n, D, generator=g) for n in (H, KVH, KVH))
    out = causal_attention(q, k, v, chunk=8)
    ke, ve = k.repeat_interleave(H // KVH, dim=2), v.repeat_interleave(H // KVH, dim=2)
    sc = torch.einsum("bphd,bshd->bhps", q, ke) / math.sqrt(D)
    sc = sc.masked_fill(torch.triu(torch.ones(P, P, dtype=torch.bool), 1), float("-inf"))
    ref = torch.einsum("bhps,bshd->bphd", sc.softmax(-1), ve)
    assert (out - ref).abs().max() < 1e-5


def test_exact_decode_backend_matches_sdpa():
    g = torch.Generator().manual_seed(1)
    q = torch.randn(3, 8, 16, generator=g)
    k = torch.randn(3, 50, 2, 16, generator=g)
    v = torch.randn(3, 50, 2, 16, generator=g)
    out = ExactDecodeBackend().decode(q, k, v, 41)
    ref = F.scaled_dot_product_attention(q.unsqueeze(2), k[:, :41].transpose(1, 2), v[:, :41].transpose(1, 2),
                                         enable_gqa=True)[:, :, 0]
    assert (out - ref).abs().max() < 1e-5


def test_cached_decode_equals_recomputation():
    torch.manual_seed(2)
    model = RandomLlama(TINY, seed=3, std=0.05, dtype=torch.float32, device="cpu")
    toks = torch.randint(0, TINY.vocab, (2, 20))
    cache = NHDCache(TINY, 2, 40, torch.float32, "cpu")
    logits = model.prefill(toks[:, :12], cache, attn_chunk=5)
    res = greedy_decode(model, logits, 12, cache, ExactDecodeBackend(), 8, forced=toks[:, 12:20])
    assert res["tokens"].shape == (2, 8) and res["logits"].shape == (8, 2, TINY.vocab)
    for j in range(8):
        ref = model.prefill(toks[:, :12 + j], NHDCache(TINY, 2, 40, torch.float32, "cpu"), attn_chunk=7)
        assert (res["logits"][j] - ref).abs().max() < 1e-5, j
    # the cache holds the fed tokens' K/V at positions 12..18 (step 7's token is not fed)
    assert cache.k[0][:, 12:19].abs().sum() > 0 and cache.k[0][:, 19:].abs().sum() == 0


def test_greedy_decode_and_deviation():
    model = RandomLlama(TINY, seed=4, std=0.05, dtype=torch.float32, device="cpu")
    toks = torch.randint(0, TINY.vocab, (2, 10), generator=torch.Generator().manual_seed(5))
    cache = NHDCache(TINY, 2, 20, torch.float32, "cpu")
    logits = model.prefill(toks, cache)
    a = greedy_decode(model, logits, 10, cache.clone(), ExactDecodeBackend(), 5)
    b = greedy_decode(model, logits, 10, cache.clone(), ExactDecodeBackend(), 5, forced=a["tokens"])
    assert torch.equal(a["tokens"], b["tokens"])
    dev = decode_deviation(a["logits"], b["logits"])
    assert max(dev["max_abs"]) == 0.0 and min(dev["top1_agree"]) == 1.0


def test_rms_norm_matches_llama_rms_norm():
    """_rms_norm has LlamaRMSNorm's roundings (the reference model's norm,
    runtime_common.py:536): the normalised row is rounded to the input dtype
    before the weight multiply, in bf16 and in float32."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    from santa_amd.runtime import _rms_norm

    g = torch.Generator().manual_seed(5)
    for dtype in (torch.bfloat16, torch.float32):
        x = (3.0 * torch.randn(4, 4096, generator=g)).to(dtype)
        w = (1.0 + 0.3 * torch.randn(4096, generator=g)).to(dtype)
        ref = LlamaRMSNorm(4096, eps=1e-5).to(dtype)
        with torch.no_grad():
            ref.weight.copy_(w)
            want = ref(x)
        got = _rms_norm(x, w, 1e-5)
        assert got.dtype == want.dtype
        assert torch.equal(got.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                           want.view(torch.int16 if dtype == torch.bfloat16 else torch.int32))
