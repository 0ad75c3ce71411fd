"""The vectorized PyTorch CPU restatement (oracle/torch_ref.py, the bench's CPU
baseline) computes the same estimator as the bit-exact C oracle.

It keeps the reference's steps with torch's own association (a matmul for
the scores, a cumsum for the count scan), so it is pinned where the
association cannot matter and bounded where it can:
- q = 0 makes every tile uniform (u = 1, ell = len, x = S_pt / len, sums of
  powers of two): every count and the output equal the oracle's;
- on peaky random inputs m* agrees to float32 rounding and the counts differ
  only at rounding edges (a sample moved to a neighbouring row), in well
  under 0.5 % of the sampled (row, head) entries;
- with a budget that samples every row many times the estimator converges:
  both outputs equal exact softmax attention to the bf16 tolerance;
- its SplitMix64 / u01 equals the oracle's on random keys.
"""
import math

import numpy as np
import torch

import oracle
from helpers import SEED, bits16, gen_qkv, h16_to_f32, tol_check
from oracle import torch_ref


def test_u01_matches_oracle():
    rng = np.random.default_rng(5)
    key = rng.integers(0, 1 << 20, 2000)
    t = rng.integers(0, 1 << 16, 2000)
    for seed in (0, 1690, 2 ** 64 - 1):
        got = torch_ref.u01(seed, key, t)
        exp = np.array([oracle.u01(seed, int(k), int(tt)) for k, tt in zip(key, t)], np.float32)
        np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_uniform_tiles_equal_the_oracle():
    B, H, KVH, L, S = 2, 32, 8, 3000, 256
    _, K, V = gen_qkv(B, H, KVH, L, seed=SEED + 1)
    q = torch.zeros(B, H, 128, dtype=torch.bfloat16)
    out, ms, cnt = torch_ref.flash_decode(q, K, V, S, seed=SEED, return_counts=True)
    exp = oracle.flash_decode(q, K, V, S, seed=SEED, block_n=256, debug=True)
    np.testing.assert_array_equal(cnt.numpy(), exp["counts"])
    np.testing.assert_array_equal(ms.numpy().view(np.uint32), exp["m_star"].view(np.uint32))
    ok, mabs, mrel = tol_check(h16_to_f32(bits16(out)), h16_to_f32(exp["out16"]))
    assert ok, (mabs, mrel)


def test_peaky_inputs_counts_differ_only_at_rounding_edges():
    for (B, H, L, S) in ((2, 32, 5000, 256), (2, 64, 3000, 512)):
        q, K, V = gen_qkv(B, H, 8, L, seed=SEED + L, lowrank=0.5)
        out, ms, cnt = torch_ref.flash_decode(q, K, V, S, seed=SEED, return_counts=True)
        exp = oracle.flash_decode(q, K, V, S, seed=SEED, block_n=256, debug=True)
        np.testing.assert_allclose(ms.numpy(), exp["m_star"], rtol=1e-5, atol=1e-5)
        c = cnt.numpy().astype(np.int64)
        ce = exp["counts"].astype(np.int64)
        sampled = np.count_nonzero(ce)
        assert np.count_nonzero(c != ce) <= 0.005 * sampled, (np.count_nonzero(c != ce), sampled)
        # a moved sample keeps the tile's total (or changes it by one at an edge)
        assert np.abs(c.sum(axis=3) - ce.sum(axis=3)).max() <= 1


def test_large_budget_converges_to_exact_attention():
    B, H, KVH, L = 1, 32, 8, 700
    q, K, V = gen_qkv(B, H, KVH, L, seed=SEED + 3)
    S = 16384 * 3  # 3 tiles of 256 rows: S_per_tile = 16384
    out, _ = torch_ref.flash_decode(q, K, V, S, seed=SEED)
    qf = q.float().view(B, KVH, H // KVH, 128)
    s = torch.einsum("bkgd,blkd->bkgl", qf, K.float()) / math.sqrt(128)
    ref = torch.einsum("bkgl,blkd->bkgd", torch.softmax(s, dim=-1), V.float()).reshape(B, H, 128)
    exp = oracle.flash_decode(q, K, V, S, seed=SEED, block_n=256)
    for got in (h16_to_f32(bits16(out)), h16_to_f32(exp["out16"])):
        ok, mabs, mrel = tol_check(got, ref.to(torch.bfloat16).float().numpy(), max_abs=2e-2, mean_rel=1e-2)
        assert ok, (mabs, mrel)
