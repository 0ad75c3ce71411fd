"""GPU parity of ragged santa_flash (one valid_len per sequence).

The ragged call plans block_n from the longest sequence (or takes it as
given) and decodes sequence b on its first valid_len[b] tokens with
S_per_tile from its own tile count and RNG key b*H + h -- what the uniform
batched call does for sequence b when every length equals valid_len[b].  So
sequence b is checked against row b of that uniform call (itself bit-exact to
the oracle, tests/test_flash_gpu.py): m* bit-exact, vrows exact, output to
the north-star bf16 tolerance (the output sum is merged in another chunking),
and against the oracle directly on one case.

Every case prints its name, shape and seed before touching the GPU.
"""
import numpy as np
import pytest
import torch

from helpers import SEED, bits16, flash_oracle_sequence, gen_qkv, h16_to_f32, seeded_lens, tol_check

pytestmark = pytest.mark.gpu


def _mod():
    import santa_flash_batch_cuda as m

    return m


def _run(H, KVH, lens, S, block_n, dtype=torch.bfloat16, L_st=None, as_tensor=False, oracle_check=False):
    m = _mod()
    B = len(lens)
    L_st = L_st or max(lens)
    print(f"\n[case] flash ragged H={H} KVH={KVH} L_storage={L_st} lens={lens} S={S} block_n={block_n} {dtype} "
          f"seed={SEED}", flush=True)
    q, K, V = gen_qkv(B, H, KVH, L_st, seed=SEED + 31 * B + L_st, dtype=dtype, lowrank=0.5)
    dev = torch.device("cuda:0")
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    vl = torch.tensor(lens, dtype=torch.int32) if as_tensor else list(lens)
    out, ms, vr = m.decode_systematic_batched(qd, Kd, Vd, S, seed=SEED, block_n=block_n, want_vrows=True,
                                              valid_len=vl)
    out2, ms2, vr2 = m.decode_systematic_batched(qd, Kd, Vd, S, seed=SEED, block_n=block_n, valid_len=vl)
    torch.cuda.synchronize()
    assert out.shape == (B, H, 128) and ms.shape == (B, H) and vr.shape == (B, KVH) and vr2.numel() == 0
    np.testing.assert_array_equal(bits16(out), bits16(out2), err_msg="repeat call")
    bn = block_n if block_n > 0 else (32 if max(lens) <= 1536 else 64 if max(lens) <= 3072 else 256)
    is_bf16 = dtype == torch.bfloat16
    for b, Lb in enumerate(lens):
        ref, ms_r, vr_r = m.decode_systematic_batched(qd, Kd, Vd, S, seed=SEED, block_n=bn, want_vrows=True,
                                                      valid_len=Lb)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ms[b].cpu().numpy().view(np.uint32), ms_r[b].cpu().numpy().view(np.uint32),
                                      err_msg=f"m_star b={b}")
        np.testing.assert_array_equal(vr[b].cpu().numpy(), vr_r[b].cpu().numpy(), err_msg=f"vrows b={b}")
        got = h16_to_f32(bits16(out[b]), is_bf16)
        ok, mabs, mrel = tol_check(got, h16_to_f32(bits16(ref[b]), is_bf16))
        assert ok, (f"b={b} vs uniform call", mabs, mrel)
        if S <= 0:
            assert not got.any(), f"b={b}: S <= 0 must give a zero output"
        if oracle_check:
            exp = flash_oracle_sequence(q, K, V, b, Lb, S, bn, is_bf16=is_bf16)
            np.testing.assert_array_equal(ms[b].cpu().numpy().view(np.uint32), exp["m_star"][0].view(np.uint32))
            np.testing.assert_array_equal(vr[b].cpu().numpy(), exp["vrows"][0])
            ok, mabs, mrel = tol_check(got, h16_to_f32(exp["out16"][0], is_bf16))
            assert ok, (f"b={b} vs oracle", mabs, mrel)


@pytest.mark.parametrize(
    "H,KVH,lens,S,block_n",
    [
        (32, 8, [9000, 3100, 5000, 4097], 256, 0),   # block_n 256, few tiles: tile kernel, ragged grid
        (32, 8, [9000, 1, 257, 8999, 6000], 300, 0),  # one-token and one-row tiles
        (64, 8, [5000, 300, 7000], 512, 256),       # GH=8 (tile kernel)
        (32, 8, [1000, 200, 33, 1500], 64, 0),      # block_n 32 (tile kernel, ragged grid)
        (32, 8, [2000, 3000, 1700], 96, 0),         # block_n 64
        (32, 8, [6000, 4000], 0, 0),                # S = 0
    ],
)
def test_flash_ragged_parity(H, KVH, lens, S, block_n):
    _run(H, KVH, lens, S, block_n)


def test_flash_ragged_against_oracle():
    _run(32, 8, [4096, 3500, 300], 128, 256, L_st=4096, as_tensor=True, oracle_check=True)


@pytest.mark.parametrize("H,S", [(32, 256), (64, 512)])
def test_flash_ragged_wave_kernel_against_oracle(H, S):
    """The production ragged wave kernel (GH 4 and GH 8): every sequence's m*
    and vrows exact against the oracle, the output within the bf16
    tolerance, and against the uniform call per sequence."""
    # lengths in [9000, 40000]: more (kv, tile) items than one resident
    # round, so the ragged grid runs the production wave kernel (rows
    # layout, ragged chunk plan)
    lens = seeded_lens(8, 9000, 40000, SEED + H)
    assert sum((l + 255) // 256 for l in lens) * 8 > 2048
    _run(H, 8, lens, S, 0, oracle_check=True)


def test_flash_ragged_f16():
    _run(32, 8, [6000, 2500, 4100], 256, 0, dtype=torch.float16)


def test_flash_equal_lengths_take_the_uniform_path():
    m = _mod()
    print("\n[case] flash valid_len list of equal lengths B=3 L=5000 valid_len=4500", flush=True)
    q, K, V = gen_qkv(3, 32, 8, 5000, seed=SEED + 5)
    dev = torch.device("cuda:0")
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    a = m.decode_systematic_batched(qd, Kd, Vd, 256, seed=SEED, valid_len=4500, want_vrows=True)
    b = m.decode_systematic_batched(qd, Kd, Vd, 256, seed=SEED, valid_len=[4500] * 3, want_vrows=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(a[0]), bits16(b[0]))
    for x, y in zip(a[1:], b[1:]):
        np.testing.assert_array_equal(x.cpu().numpy(), y.cpu().numpy())


def test_flash_ragged_errors():
    m = _mod()
    print("\n[case] flash ragged argument errors", flush=True)
    dev = torch.device("cuda:0")
    q, K, V = gen_qkv(2, 32, 8, 512)
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    with pytest.raises(RuntimeError, match="one entry per sequence"):
        m.decode_systematic_batched(qd, Kd, Vd, 10, valid_len=[100, 200, 300])
    with pytest.raises(RuntimeError, match="valid_len exceeds storage length"):
        m.decode_systematic_batched(qd, Kd, Vd, 10, valid_len=[100, 513])
    with pytest.raises(RuntimeError, match="batched form"):
        m.decode_systematic_scalar(qd[0].contiguous(), Kd[0].contiguous(), Vd[0].contiguous(), 10, valid_len=[100])
