"""Vectorized PyTorch CPU restatement of santa_flash decode (the CPU baseline).

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` and the ``cpu_baseline``
leg of ``bench.py`` -- never by the product package or the extension
modules.  It is the reference algorithm's PyTorch CPU path: whole tiles
batched into torch matmuls, then per-tile max, exp and mass, the 16-bit u,
the seeded systematic counts, the sampled V gather and the split-KV merge
(flash/santa_cuda.cpp:174-343, flash/santa_cuda_kernel.cu:161-470).

It follows the reference's steps but not its association: the scores are a
torch matmul and the count scan a torch cumsum, so m_t, ell_t and, at
rounding edges, a count can differ from the bit-exact C oracle
(santa_oracle.c); tests/test_torch_ref.py bounds the difference.
"""
from __future__ import annotations

import math

import numpy as np
import torch

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def u01(seed: int, key: np.ndarray, t: np.ndarray) -> np.ndarray:
    """SplitMix64 of seed ^ ((key << 32) ^ t), top 53 bits scaled to [0, 1)
    and rounded to float32 (flash/santa_cuda_kernel.cu:74-87), vectorized."""
    with np.errstate(over="ignore"):
        x = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) ^ ((key.astype(np.uint64) << np.uint64(32)) ^ t.astype(np.uint64))
        z = x + _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return ((z >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)).astype(np.float32)


def flash_decode(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, S: int, seed: int = 42,
                 block_n: int = 256, return_counts: bool = False):
    """q [B,H,D], K,V [B,L,KVH,D] (bf16 or f16, CPU) -> (out [B,H,D] in q's
    dtype, m_star [B,H] f32), the estimator of decode_systematic_batched on
    the whole cache; with return_counts also the counts [B,H,T_c,block_n]."""
    B, H, D = q.shape
    L, KVH = K.shape[1], K.shape[2]
    GH = H // KVH
    BN = block_n
    T_c = (L + BN - 1) // BN
    S_pt = max(1, S // T_c) if S > 0 else 0
    Lp = T_c * BN
    qs = (q.float() * (1.0 / math.sqrt(D))).view(B, KVH, GH, D)
    Kf = K.float().permute(0, 2, 1, 3)                                  # [B, KVH, L, D]
    s = torch.matmul(Kf, qs.transpose(-1, -2))                          # [B, KVH, L, GH]
    del Kf
    if Lp != L:
        s = torch.cat([s, s.new_full((B, KVH, Lp - L, GH), -math.inf)], dim=2)
    s = s.view(B, KVH, T_c, BN, GH)
    m_t = s.amax(dim=3)                                                 # [B, KVH, T_c, GH]
    u = torch.exp(s - m_t.unsqueeze(3))
    ell = u.sum(dim=3)
    u16 = u.to(q.dtype).float()
    invdel = torch.where(ell > 1e-20, S_pt / ell, torch.zeros_like(ell)) if S_pt > 0 else torch.zeros_like(ell)
    x = u16 * invdel.unsqueeze(3)
    cum = torch.cumsum(x, dim=3)
    key = (np.arange(B)[:, None, None, None] * H + np.arange(KVH)[None, :, None, None] * GH
           + np.arange(GH)[None, None, None, :])
    tt = np.arange(T_c)[None, None, :, None]
    a0 = torch.from_numpy(u01(seed, np.broadcast_to(key, (B, KVH, T_c, GH)),
                              np.broadcast_to(tt, (B, KVH, T_c, GH))).copy()).unsqueeze(3)
    prev = torch.cat([torch.zeros_like(cum[:, :, :, :1]), cum[:, :, :, :-1]], dim=3)
    c = (torch.floor(a0 + cum) - torch.floor(a0 + prev)).clamp_(0, 32767)  # [B, KVH, T_c, BN, GH]
    # merge weights w_t = exp(m_t - m*) ell_t, Z = sum_t w_t
    m_star = m_t.amax(dim=2, keepdim=True)                              # [B, KVH, 1, GH]
    w = torch.exp(m_t - m_star) * ell
    Z = w.sum(dim=2)                                                    # [B, KVH, GH]
    coef = (c * w.unsqueeze(3)).view(B, KVH, Lp, GH)[:, :, :L]          # [B, KVH, L, GH]
    # the sampled rows only: gather them and sum count-weighted V rows
    rows = coef.gt(0).any(dim=3).nonzero(as_tuple=True)                 # (b, kv, n)
    vsel = V[rows[0], rows[2], rows[1]].float()                         # [N, D]
    csel = coef[rows[0], rows[1], rows[2]]                              # [N, GH]
    num = torch.zeros(B * KVH, GH, D)
    num.index_add_(0, rows[0] * KVH + rows[1], csel.unsqueeze(2) * vsel.unsqueeze(1))
    num = num.view(B, KVH, GH, D)
    scale = torch.where(Z > 0, 1.0 / (Z * S_pt), torch.zeros_like(Z)) if S_pt > 0 else torch.zeros_like(Z)
    out = (num * scale.unsqueeze(3)).reshape(B, H, D)
    if return_counts:
        counts = c.permute(0, 1, 4, 2, 3).reshape(B, H, T_c, BN).to(torch.int16)
        return out.to(q.dtype), m_star.view(B, KVH, GH).reshape(B, H), counts
    return out.to(q.dtype), m_star.view(B, KVH, GH).reshape(B, H)
