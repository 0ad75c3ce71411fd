"""GPU checks of the fused decode-step kernels (santa_rt_* in santa_amd.h)
against the torch expressions of santa_amd/runtime.py they replace.

* RoPE with the cache write: bit-exact (each product and the sum are one
  IEEE float operation rounded to bf16, as in torch's bf16 arithmetic);
  rows of the caches other than the written position are untouched.
* add + RMSNorm: the residual sum bit-exact; the norm to two bf16 units in
  the last place (the float32 sum of squares is reduced in another order, so
  the normalised row can round to a neighbouring bf16 value, which the weight
  multiply scales by up to 1.3 before the second rounding).
* SwiGLU: to one bf16 unit in the last place (exp is this library's).
* The few-row weight product (santa_rt_linear) against the float64 product
  of the same bf16 operands: at least 99.9 % of the outputs are that value
  rounded to bf16 (float32 accumulation changes the rounding only next to a
  rounding boundary) and every output is within 2^-7 relative plus 2^-20 of
  sum |x| |w|.  With the SwiGLU epilogue: bit for bit silu_mul of the
  plain product (same sums, silu_mul's roundings), and at least 99.9 % equal
  to silu_mul of the float64 product's bf16 roundings.  Shapes cover every
  row padding (1, 2, 4, 8 staged rows), odd N, K not a multiple of the
  2048-column chunk, the largest staged K, and more row pairs than resident
  waves.  With the RoPE epilogue: bit for bit rope_write of the plain
  product (q, the cache rows at pos), the caches' other rows untouched.
* The greedy step's argmax: equal to torch.argmax on random rows, rows
  with the maximum planted at several positions (first index wins), a NaN
  row (NaN counts as the maximum), an all -inf row, and a width that is not
  a multiple of 4 (the scalar path).

Every case prints its name and shape before touching the GPU.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from santa_amd.runtime import NHDCache, LlamaShape, _FusedOps, _apply_rope, _rms_norm, _rope_cos_sin

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _ulp_close(got: torch.Tensor, ref: torch.Tensor, ulps: int = 1):
    a = got.view(torch.int16).cpu().numpy().astype(np.int32)
    b = ref.view(torch.int16).cpu().numpy().astype(np.int32)
    # bf16 bit patterns of same-sign values are ordered like the values
    assert np.abs(a - b).max() <= ulps, np.abs(a - b).max()


@pytest.mark.parametrize("rows,hidden", [(1, 4096), (4, 4096), (3, 1000), (2, 14336), (2, 8192), (2, 1004)])
def test_add_rms_norm(rows, hidden):
    print(f"\n[case] add_rms_norm rows={rows} hidden={hidden}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows * 7 + hidden)
    h = torch.randn(rows, hidden, device=DEV, generator=g).to(torch.bfloat16)
    a = torch.randn(rows, hidden, device=DEV, generator=g).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn(hidden, device=DEV, generator=g)).to(torch.bfloat16)
    ref_h = h + a
    ref_x = _rms_norm(ref_h, w, 1e-5)
    h2 = h.clone()
    x = _FusedOps.add_rms_norm(h2, a, w, 1e-5)
    x0 = _FusedOps.add_rms_norm(h.clone(), None, w, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(h2.view(torch.int16), ref_h.view(torch.int16))
    _ulp_close(x, ref_x, 2)
    _ulp_close(x0, _rms_norm(h, w, 1e-5), 2)


@pytest.mark.parametrize("B,H,KVH,pos", [(4, 32, 8, 37), (2, 64, 8, 0), (1, 16, 2, 99)])
def test_rope_write(B, H, KVH, pos):
    D = 128
    print(f"\n[case] rope_write B={B} H={H} KVH={KVH} pos={pos}", flush=True)
    shape = LlamaShape(hidden=H * D, intermediate=256, heads=H, kv_heads=KVH, layers=1, vocab=16)
    cache = NHDCache(shape, B, 128, torch.bfloat16, DEV)
    g = torch.Generator(device=DEV).manual_seed(B * 100 + pos)
    for t in (cache.k[0], cache.v[0]):
        t.copy_(torch.randn(t.shape, device=DEV, generator=g).to(torch.bfloat16))
    k_before, v_before = cache.k[0].clone(), cache.v[0].clone()
    qkv = torch.randn(B, (H + 2 * KVH) * D, device=DEV, generator=g).to(torch.bfloat16)
    cos, sin = _rope_cos_sin(torch.tensor([pos], device=DEV), D, 500000.0, torch.bfloat16)
    q = _FusedOps.rope_write(qkv, cos.reshape(D).contiguous(), sin.reshape(D).contiguous(), cache, 0, pos, H, KVH, D)
    torch.cuda.synchronize()
    q_ref, k_ref, v_ref = qkv.split([H * D, KVH * D, KVH * D], dim=-1)
    q_ref = _apply_rope(q_ref.view(B, H, D), cos, sin)
    k_ref = _apply_rope(k_ref.view(B, KVH, D), cos, sin)
    assert torch.equal(q.view(torch.int16), q_ref.view(torch.int16))
    assert torch.equal(cache.k[0][:, pos].view(torch.int16), k_ref.view(torch.int16))
    assert torch.equal(cache.v[0][:, pos].view(torch.int16), v_ref.reshape(B, KVH, D).view(torch.int16))
    mask = torch.ones(128, dtype=torch.bool)
    mask[pos] = False
    assert torch.equal(cache.k[0][:, mask], k_before[:, mask]) and torch.equal(cache.v[0][:, mask], v_before[:, mask])


@pytest.mark.parametrize("rows,inter", [(4, 14336), (1, 300)])
def test_silu_mul(rows, inter):
    print(f"\n[case] silu_mul rows={rows} inter={inter}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows + inter)
    gu = (3.0 * torch.randn(rows, 2 * inter, device=DEV, generator=g)).to(torch.bfloat16)
    out = _FusedOps.silu_mul(gu)
    gate, up = gu.chunk(2, dim=-1)
    ref = F.silu(gate) * up
    torch.cuda.synchronize()
    _ulp_close(out, ref)


def _bf16_bits_diff(got: torch.Tensor, ref: torch.Tensor) -> np.ndarray:
    a = got.contiguous().view(torch.int16).cpu().numpy().astype(np.int32)
    b = ref.contiguous().view(torch.int16).cpu().numpy().astype(np.int32)
    return np.abs(a - b)


@pytest.mark.parametrize("M,N,K", [(4, 6144, 4096), (4, 4096, 14336), (1, 1000, 512), (3, 777, 1000),
                                   (8, 1030, 8192), (2, 129, 2056), (5, 64, 8), (4, 128256, 4096)])
def test_linear(M, N, K):
    print(f"\n[case] linear M={M} N={N} K={K}", flush=True)
    assert _FusedOps.linear_fits(M, K)
    g = torch.Generator(device=DEV).manual_seed(M * 7919 + N + K)
    x = torch.randn(M, K, device=DEV, generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn(N, K, device=DEV, generator=g)).to(torch.bfloat16)
    y = _FusedOps.linear(x, w)
    ref = x.double() @ w.double().t()
    bound = ref.abs() * 2.0 ** -7 + (x.double().abs() @ w.double().abs().t()) * 2.0 ** -20
    torch.cuda.synchronize()
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    assert ((y.double() - ref).abs() <= bound).all()
    exact = (_bf16_bits_diff(y, ref.to(torch.bfloat16)) == 0).mean()
    assert exact >= 0.999, exact


@pytest.mark.parametrize("M,inter,K", [(4, 14336, 4096), (3, 1000, 1000), (1, 33, 2048), (8, 256, 8192)])
def test_linear_swiglu(M, inter, K):
    print(f"\n[case] linear swiglu M={M} inter={inter} K={K}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(M * 104729 + inter + K)
    x = torch.randn(M, K, device=DEV, generator=g).to(torch.bfloat16)
    w = (0.05 * torch.randn(2 * inter, K, device=DEV, generator=g)).to(torch.bfloat16)
    out = _FusedOps.linear(x, w, swiglu=True)
    # each row's sum takes the same path through the lanes wherever it sits
    # in the wave's pair of rows, so the epilogue sees the plain product's
    # values and applies silu_mul's roundings to them
    two = _FusedOps.silu_mul(_FusedOps.linear(x, w))
    gu = (x.double() @ w.double().t()).to(torch.bfloat16)
    gate, up = gu.chunk(2, dim=-1)
    ref = F.silu(gate) * up
    torch.cuda.synchronize()
    assert out.shape == (M, inter)
    assert torch.equal(out.view(torch.int16), two.view(torch.int16))
    exact = (out.view(torch.int16) == ref.view(torch.int16)).float().mean().item()
    assert exact >= 0.999, exact


@pytest.mark.parametrize("B,H,KVH,D,K,pos", [(4, 32, 8, 128, 4096, 37), (2, 4, 1, 128, 512, 0), (3, 16, 2, 64, 1000, 99)])
def test_linear_rope(B, H, KVH, D, K, pos):
    print(f"\n[case] linear_rope B={B} H={H} KVH={KVH} D={D} K={K} pos={pos}", flush=True)
    shape = LlamaShape(hidden=H * D, intermediate=8, heads=H, kv_heads=KVH, layers=1, vocab=8)  # head_dim D
    g = torch.Generator(device=DEV).manual_seed(B * 31 + H + D + K + pos)
    x = torch.randn(B, K, device=DEV, generator=g).to(torch.bfloat16)
    w = (0.05 * torch.randn((H + 2 * KVH) * D, K, device=DEV, generator=g)).to(torch.bfloat16)
    cos, sin = _rope_cos_sin(torch.tensor([pos], device=DEV), D, 5e5, torch.bfloat16)
    cos, sin = cos.reshape(D).contiguous(), sin.reshape(D).contiguous()
    fused = NHDCache(shape, B, pos + 5, torch.bfloat16, DEV)
    for t in (fused.k[0], fused.v[0]):
        t.copy_(torch.randn(t.shape, device=DEV, generator=g).to(torch.bfloat16))
    two = fused.clone()
    q = _FusedOps.linear_rope(x, w, cos, sin, fused, 0, pos, H, KVH, D)
    q2 = _FusedOps.rope_write(_FusedOps.linear(x, w), cos, sin, two, 0, pos, H, KVH, D)
    torch.cuda.synchronize()
    assert torch.equal(q.view(torch.int16), q2.view(torch.int16))
    assert torch.equal(fused.k[0].view(torch.int16), two.k[0].view(torch.int16))
    assert torch.equal(fused.v[0].view(torch.int16), two.v[0].view(torch.int16))


@pytest.mark.parametrize("rows,n", [(4, 128256), (3, 1001), (1, 7)])
def test_argmax(rows, n):
    print(f"\n[case] argmax rows={rows} n={n}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows * 13 + n)
    x = torch.randn(rows, n, device=DEV, generator=g)
    got = _FusedOps.argmax(x)
    assert torch.equal(got, torch.argmax(x, dim=-1))
    # ties: the row maximum planted at several positions
    y = x.clone()
    for r in range(rows):
        cols = torch.randint(0, n, (3,), generator=torch.Generator().manual_seed(r + n)).tolist()
        y[r, cols] = 10.0
    assert torch.equal(_FusedOps.argmax(y), torch.argmax(y, dim=-1))
    # NaN above any number; an all -inf row
    z = x.clone()
    z[0, n // 2] = float("nan")
    z[-1] = float("-inf")
    torch.cuda.synchronize()
    assert torch.equal(_FusedOps.argmax(z), torch.argmax(z, dim=-1))
