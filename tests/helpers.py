"""Shared input recipes and comparison helpers for the test suite."""
from __future__ import annotations

import hashlib
import math

import numpy as np
import torch

SEED = 1690


def gen_qkv(B, H, KVH, L, D=128, seed=SEED, dtype=torch.bfloat16, lowrank=0.0, single=False):
    """q [B,H,D], K,V [B,L,KVH,D] ~ N(0,1) from a CPU generator (f32, then cast).

    lowrank > 0 adds the per-head rank-4 key bias of the headline config:
    K += lowrank * sqrt(D) * (C @ U_kv), C ~ N(0,1)[B,L,KVH,4],
    U_kv ~ N(0,1)[KVH,4,D] / sqrt(D)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, D, generator=g, dtype=torch.float32)
    K = torch.randn(B, L, KVH, D, generator=g, dtype=torch.float32)
    V = torch.randn(B, L, KVH, D, generator=g, dtype=torch.float32)
    if lowrank:
        C = torch.randn(B, L, KVH, 4, generator=g, dtype=torch.float32)
        U = torch.randn(KVH, 4, D, generator=g, dtype=torch.float32) / math.sqrt(D)
        K = K + lowrank * math.sqrt(D) * torch.einsum("blkr,krd->blkd", C, U)
    q, K, V = q.to(dtype), K.to(dtype), V.to(dtype)
    if single:
        return q[0].contiguous(), K[0].contiguous(), V[0].contiguous()
    return q, K, V


def tensor_digest(*ts) -> str:
    h = hashlib.sha256()
    for t in ts:
        h.update(t.detach().cpu().contiguous().view(torch.int16).numpy().tobytes())
    return h.hexdigest()[:16]


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def h16_to_f32(bits: np.ndarray, is_bf16=True) -> np.ndarray:
    if is_bf16:
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float16).astype(np.float32)


def tol_check(got: np.ndarray, ref: np.ndarray, max_abs=2e-2, mean_rel=1e-3):
    """bf16 tolerance of the north star: max |got-ref| <= 2e-2 and
    mean relative error sum|got-ref| / sum|ref| <= 1e-3 (both in the output dtype)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    mabs = float(err.max()) if err.size else 0.0
    mrel = float(err.sum() / max(np.abs(ref).sum(), 1e-30)) if err.size else 0.0
    return mabs <= max_abs and mrel <= mean_rel, mabs, mrel


def flash_oracle_sequence(q, K, V, b, Lb, S, bn, seed=SEED, is_bf16=True):
    """The oracle of sequence b of a ragged flash batch on its own (CPU
    tensors): its first Lb tokens, S_per_tile from its own tile count, RNG
    key b*H + h -- what the ragged call does for that sequence."""
    import oracle

    return oracle.flash_decode(q[b:b + 1], K[b:b + 1, :Lb], V[b:b + 1, :Lb], S, seed=seed, block_n=bn,
                               is_bf16=is_bf16, debug=True, b_offset=b)


def seeded_lens(B, lo, hi, seed):
    """B lengths drawn uniformly from [lo, hi] by a seeded CPU generator."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (B,), generator=g).tolist()
