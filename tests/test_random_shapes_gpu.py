"""Seeded random shapes: santa_flash and santa_prop against the CPU oracle.

Twenty-four flash, sixteen prop and fourteen generic-shape prop
configurations drawn once from fixed seeds (the draw is part of the test, so
every run checks the same cases):
group sizes 4 and 8 with 1-8 KV heads, 1-3 sequences, lengths from one token to
20k (so every block size, partial tiles and one-tile sequences occur),
budgets from 0 to several per row, explicit and automatic block_n, and a
valid_len below the storage length.  Each case checks, bit for bit, the
flash production kernel's tile statistics and counts (block_n 256) or the
tile kernel's (block_n 32/64), m* and vrows, and the output to the bf16
tolerance; for prop, m*, vrows and the output per sequence.  These are the
plans and grids (chunk sizes, the rows and four-wave layouts, ragged last
chunks) that hand-picked cases leave out.  The generic-shape prop cases
(`santa_prop_gen.hip`: group sizes other than 4 and 8, head dims 16-256,
block_n 16-512, bf16 and f16) run the batched, ragged call and check each
sequence against the oracle's per-sequence call: m* and vrows exact, the
output to the bf16 tolerance.

Every case prints its name, shape and seed before touching the GPU.
"""
import random

import numpy as np
import pytest
import torch

import oracle
from helpers import bits16, gen_qkv, h16_to_f32, tol_check

pytestmark = pytest.mark.gpu


def _flash_cases():
    rng = random.Random(20261201)
    cases = []
    for i in range(24):
        GH = rng.choice([4, 4, 8])
        KVH = rng.choice([1, 2, 4, 8, 8])
        H = GH * KVH
        B = rng.choice([1, 2, 3])
        L = rng.choice([1, 7, 255, 256, 257, 1000, 1536, 1537, 3072, 3073, 5000, 9999, 20000])
        S = rng.choice([0, 1, 13, 256, 1000, 20000])
        block_n = rng.choice([0, 0, 32, 64, 256])
        valid_len = rng.choice([-1, -1, max(1, L - rng.randrange(0, max(1, L // 2)))])
        cases.append((i, B, H, KVH, L, S, block_n, valid_len))
    return cases


def _prop_cases():
    rng = random.Random(20261202)
    cases = []
    for i in range(16):
        KVH = rng.choice([2, 4, 8])
        GH = rng.choice([4, 4, 8])
        H = GH * KVH
        L = rng.choice([1, 100, 300, 2000, 4097, 12000])
        S = rng.choice([0, 1, 50, 1000, 5000])
        block_n = rng.choice([0, 32, 64, 256])
        cases.append((i, H, KVH, L, S, block_n))
    return cases


def _prop_generic_cases():
    rng = random.Random(20261203)
    cases = []
    for i in range(14):
        GH = rng.choice([1, 2, 3, 5, 6, 12, 16])
        KVH = rng.choice([1, 2, 4]) if GH > 4 else rng.choice([1, 2, 4, 8])
        D = rng.choice([16, 32, 64, 64, 96, 128, 128, 256, 256])
        B = rng.choice([1, 2, 3])
        L = rng.choice([200, 1000, 4097, 9000])
        lens = [L] + [rng.randint(1, L) for _ in range(B - 1)]
        Ss = [rng.choice([0, 1, 40, 40, 700, 700]) for _ in range(B)]
        block_n = rng.choice([16, 48, 256, 256, 512])
        f16 = rng.random() < 0.25
        cases.append((i, GH * KVH, KVH, D, lens, Ss, block_n, f16))
    return cases


@pytest.mark.parametrize("case", _flash_cases(), ids=lambda c: f"flash{c[0]}")
def test_flash_random_shape(case):
    import santa_flash_batch_cuda as m

    i, B, H, KVH, L, S, block_n, valid_len = case
    seed = 7000 + i
    print(f"\n[case] flash random #{i} B={B} H={H} KVH={KVH} L={L} S={S} block_n={block_n} valid_len={valid_len} "
          f"seed={seed}", flush=True)
    q, K, V = gen_qkv(B, H, KVH, L, seed=seed, lowrank=0.5)
    dev = torch.device("cuda:0")
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    bn_eff = oracle.auto_block_n(valid_len if valid_len > 0 else L) if block_n <= 0 else block_n
    if bn_eff == 256:
        mt, lt, cnt = m._debug_wave(qd, Kd, Vd, S, seed=seed, valid_len=valid_len)
    else:
        mt, lt, cnt, _, _ = m._debug_tiles(qd, Kd, Vd, S, seed=seed, block_n=block_n, valid_len=valid_len)
    out, ms, vr = m.decode_systematic_batched(qd, Kd, Vd, S, seed=seed, block_n=block_n, want_vrows=True,
                                              valid_len=valid_len)
    torch.cuda.synchronize()
    exp = oracle.flash_decode(q, K, V, S, seed=seed, block_n=block_n, valid_len=valid_len, debug=True)
    np.testing.assert_array_equal(mt.cpu().numpy().view(np.uint32), exp["m_tiles"].view(np.uint32), err_msg="m_tiles")
    np.testing.assert_array_equal(lt.cpu().numpy().view(np.uint32), exp["ell_tiles"].view(np.uint32),
                                  err_msg="ell_tiles")
    c_gpu = cnt.cpu().numpy()
    assert np.array_equal(c_gpu, exp["counts"]), f"counts differ at {np.argwhere(c_gpu != exp['counts'])[:8]}"
    np.testing.assert_array_equal(ms.cpu().numpy().view(np.uint32), exp["m_star"].view(np.uint32), err_msg="m_star")
    np.testing.assert_array_equal(vr.cpu().numpy(), exp["vrows"], err_msg="vrows")
    ok, mabs, mrel = tol_check(h16_to_f32(bits16(out)), h16_to_f32(exp["out16"]))
    assert ok, ("vs oracle", mabs, mrel)


@pytest.mark.parametrize("case", _prop_cases(), ids=lambda c: f"prop{c[0]}")
def test_prop_random_shape(case, monkeypatch):
    import santa_prop_batch_cuda as m

    monkeypatch.delenv("SANTA_PASS1", raising=False)
    i, H, KVH, L, S, block_n = case
    seed = 8000 + i
    print(f"\n[case] prop random #{i} H={H} KVH={KVH} L={L} S={S} block_n={block_n} seed={seed}", flush=True)
    q, K, V = gen_qkv(1, H, KVH, L, seed=seed, lowrank=0.5, single=True)
    dev = torch.device("cuda:0")
    out, ms, vr = m.decode_systematic_scalar(q.to(dev), K.to(dev), V.to(dev), S, seed=seed, block_n=block_n,
                                             want_vrows=True)
    torch.cuda.synchronize()
    exp = oracle.prop_decode(q, K, V, S, seed=seed, block_n=block_n, debug=True)
    np.testing.assert_array_equal(ms.cpu().numpy().view(np.uint32), exp["m_star"].view(np.uint32), err_msg="m_star")
    np.testing.assert_array_equal(vr.cpu().numpy(), exp["vrows"], err_msg="vrows")
    ok, mabs, mrel = tol_check(h16_to_f32(bits16(out)), h16_to_f32(exp["out16"]))
    assert ok, ("vs oracle", mabs, mrel)


@pytest.mark.parametrize("case", _prop_generic_cases(), ids=lambda c: f"propgen{c[0]}")
def test_prop_generic_random_shape(case, monkeypatch):
    import santa_prop_batch_cuda as m

    monkeypatch.delenv("SANTA_PASS1", raising=False)
    i, H, KVH, D, lens, Ss, block_n, f16 = case
    seed = 9000 + i
    dtype = torch.float16 if f16 else torch.bfloat16
    print(f"\n[case] prop generic random #{i} H={H} KVH={KVH} D={D} lens={lens} S={Ss} block_n={block_n} "
          f"dtype={'f16' if f16 else 'bf16'} seed={seed}", flush=True)
    q, K, V = gen_qkv(len(lens), H, KVH, max(lens), D=D, seed=seed, dtype=dtype, lowrank=0.5)
    dev = torch.device("cuda:0")
    out, ms, vr = m.decode_systematic_batched(q.to(dev), K.to(dev), V.to(dev), Ss, seed=seed, block_n=block_n,
                                              want_vrows=True, valid_len=lens)
    torch.cuda.synchronize()
    for b, (Lb, Sb) in enumerate(zip(lens, Ss)):
        exp = oracle.prop_decode(q[b], K[b, :Lb], V[b, :Lb], Sb, seed=seed, block_n=block_n, is_bf16=not f16,
                                 debug=True)
        assert exp["pass1_mode"] == 1
        np.testing.assert_array_equal(ms[b].cpu().numpy().view(np.uint32), exp["m_star"].view(np.uint32),
                                      err_msg=f"m_star b={b}")
        np.testing.assert_array_equal(vr[b].cpu().numpy(), exp["vrows"], err_msg=f"vrows b={b}")
        ok, mabs, mrel = tol_check(h16_to_f32(bits16(out[b]), f16), h16_to_f32(exp["out16"], f16))
        assert ok, (f"b={b} vs oracle", mabs, mrel)
