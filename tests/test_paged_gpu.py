"""GPU parity of the paged-KV entry points (decode_systematic_paged).

A paged call reads a page pool [num_pages, page_size, KVH, D] through an
int32 block table.  It runs the same kernels, chunk plan and merge as the
contiguous call on the same tokens (ragged flash, batched prop); only the
row addressing differs.  So its results must be bit-identical to that call,
which is itself pinned to the oracle (tests/test_flash_ragged_gpu.py,
tests/test_prop_batched_gpu.py); the production-sized cases are also
compared with the oracle directly, sequence by sequence.  The one exception is a prop batch whose
sequences plan to different block sizes: it is decoded one paged launch per
sequence, while the contiguous call runs the scalar path per sequence.
There m* and vrows must be identical, and the output must agree to the
north-star bf16 tolerance (the same terms summed in another chunking).

The pool holds the sequences' pages in a seeded random order among spare
pages filled with NaN.  Every page's rows past its sequence's length are NaN
too, and unused table entries point at a NaN page.  A read of anything but
the valid rows would therefore show up in the output.

Every case prints its name, shape and seed before touching the GPU.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import SEED, bits16, flash_oracle_sequence, gen_qkv, h16_to_f32, seeded_lens, tol_check

pytestmark = pytest.mark.gpu


def make_pool(K, V, lens, page_size, seed, spare=3):
    """Scatter K, V [B, L_storage, KVH, D] (CPU) into a page pool; returns
    (K_pages, V_pages, block_table [B, stride] int32)."""
    B, _, KVH, D = K.shape
    npp = [(l + page_size - 1) // page_size for l in lens]
    stride = max(npp) + 1  # one column more than any sequence needs
    total = sum(npp) + spare
    perm = torch.randperm(total, generator=torch.Generator().manual_seed(seed)).tolist()
    Kp = torch.full((total, page_size, KVH, D), float("nan"), dtype=K.dtype)
    Vp = torch.full((total, page_size, KVH, D), float("nan"), dtype=V.dtype)
    nan_page = perm[-1]  # a spare page
    table = torch.full((B, stride), nan_page, dtype=torch.int32)
    i = 0
    for b in range(B):
        for j in range(npp[b]):
            pid = perm[i]
            i += 1
            table[b, j] = pid
            r0, r1 = j * page_size, min((j + 1) * page_size, lens[b])
            Kp[pid, : r1 - r0] = K[b, r0:r1]
            Vp[pid, : r1 - r0] = V[b, r0:r1]
    return Kp, Vp, table


def _check(got, ref, exact, is_bf16, what):
    out, ms, vr = got
    out_r, ms_r, vr_r = ref
    np.testing.assert_array_equal(ms.cpu().numpy().view(np.uint32), ms_r.cpu().numpy().view(np.uint32),
                                  err_msg=f"{what}: m_star")
    np.testing.assert_array_equal(vr.cpu().numpy(), vr_r.cpu().numpy(), err_msg=f"{what}: vrows")
    if exact:
        np.testing.assert_array_equal(bits16(out), bits16(out_r), err_msg=f"{what}: out")
    else:
        ok, mabs, mrel = tol_check(h16_to_f32(bits16(out), is_bf16), h16_to_f32(bits16(out_r), is_bf16))
        assert ok, (what, mabs, mrel)
    assert torch.isfinite(out.float()).all(), f"{what}: non-finite output (a NaN row was read)"


def _inputs(B, H, KVH, lens, page_size, dtype, seed):
    L_st = max(lens)
    q, K, V = gen_qkv(B, H, KVH, L_st, seed=seed, dtype=dtype, lowrank=0.5)
    Kp, Vp, table = make_pool(K, V, lens, page_size, seed)
    dev = torch.device("cuda:0")
    return [t.to(dev) for t in (q, K, V, Kp, Vp, table)]


@pytest.mark.parametrize(
    "H,KVH,lens,S,page_size,block_n,dtype",
    [
        (32, 8, [9000, 3100, 5000, 4097], 256, 16, 0, torch.bfloat16),  # few tiles: tile kernel, 16-token pages
        (32, 8, [9000, 1, 257, 8999], 300, 8, 0, torch.bfloat16),       # 8-token pages, a one-token sequence
        (32, 8, [7000, 6000, 5000], 256, 256, 0, torch.bfloat16),       # one page per tile
        (32, 8, [7000, 6000], 256, 1024, 0, torch.bfloat16),            # tiles inside pages
        (64, 8, [5000, 300, 7000], 512, 64, 256, torch.bfloat16),       # GH 8
        (32, 8, [1000, 200, 33, 1500], 64, 16, 0, torch.bfloat16),      # block_n 32 (tile kernel)
        (32, 8, [2000, 3000, 1700], 96, 32, 0, torch.bfloat16),         # block_n 64
        (32, 8, [6000, 4000], 0, 16, 0, torch.bfloat16),                # S = 0
        (32, 8, [6000, 2500, 4100], 256, 16, 0, torch.float16),         # f16
    ],
)
def test_flash_paged_matches_contiguous(H, KVH, lens, S, page_size, block_n, dtype):
    import santa_flash_batch_cuda as m

    seed = SEED + 7 * len(lens) + page_size
    print(f"\n[case] flash paged H={H} KVH={KVH} lens={lens} S={S} page_size={page_size} block_n={block_n} {dtype} "
          f"seed={seed}", flush=True)
    q, K, V, Kp, Vp, table = _inputs(len(lens), H, KVH, lens, page_size, dtype, seed)
    got = m.decode_systematic_paged(q, Kp, Vp, table, lens, S, seed=SEED, block_n=block_n, want_vrows=True)
    ref = m.decode_systematic_batched(q, K, V, S, seed=SEED, block_n=block_n, want_vrows=True, valid_len=lens)
    again = m.decode_systematic_paged(q, Kp, Vp, table, torch.tensor(lens), S, seed=SEED, block_n=block_n,
                                      want_vrows=True)
    torch.cuda.synchronize()
    _check(got, ref, True, dtype == torch.bfloat16, "paged vs contiguous")
    _check(again, got, True, dtype == torch.bfloat16, "repeat call, lengths as a tensor")


@pytest.mark.parametrize(
    "H,KVH,lens,Ss,page_size,block_n,env,exact",
    [
        (32, 8, [12000, 3100, 7777, 4096], [256, 64, 300, 1], 16, 0, None, True),  # vec pass 1 (wave kernel)
        (32, 8, [12000, 3100, 7777, 4096], [256, 64, 300, 1], 16, 0, "gqa", True),  # general pass 1
        (16, 2, [1, 33, 500, 1000], [7, 40, 256, 1000], 8, 32, None, True),        # block_n 32, GH 8
        (32, 8, [5000, 9000], [100, 0], 512, 0, None, True),                       # S = 0 for one sequence
        (32, 8, [1000, 8000, 2000], [256, 256, 256], 64, 0, None, False),          # mixed block sizes
    ],
)
def test_prop_paged_matches_contiguous(H, KVH, lens, Ss, page_size, block_n, env, exact, monkeypatch):
    import santa_prop_batch_cuda as m

    if env is None:
        monkeypatch.delenv("SANTA_PASS1", raising=False)
    else:
        monkeypatch.setenv("SANTA_PASS1", env)
    seed = SEED + 11 * len(lens) + page_size
    print(f"\n[case] prop paged H={H} KVH={KVH} lens={lens} S={Ss} page_size={page_size} block_n={block_n} "
          f"env={env} seed={seed}", flush=True)
    q, K, V, Kp, Vp, table = _inputs(len(lens), H, KVH, lens, page_size, torch.bfloat16, seed)
    got = m.decode_systematic_paged(q, Kp, Vp, table, lens, Ss, seed=SEED, block_n=block_n, want_vrows=True)
    ref = m.decode_systematic_batched(q, K, V, Ss, seed=SEED, block_n=block_n, want_vrows=True, valid_len=lens)
    torch.cuda.synchronize()
    _check(got, ref, exact, True, "paged vs contiguous")


def _oracle_checks(got, q, K, V, lens, what, oracle_of):
    """Per sequence: m* bit-exact and vrows exact against the oracle, the
    output within the bf16 tolerance."""
    out, ms, vr = (t.cpu() for t in got)
    qc, Kc, Vc = q.cpu(), K.cpu(), V.cpu()
    for b, Lb in enumerate(lens):
        exp = oracle_of(qc, Kc, Vc, b, Lb)
        np.testing.assert_array_equal(ms[b].numpy().view(np.uint32), exp["m_star"].reshape(-1).view(np.uint32),
                                      err_msg=f"{what}: m_star b={b}")
        np.testing.assert_array_equal(vr[b].numpy(), exp["vrows"].reshape(-1), err_msg=f"{what}: vrows b={b}")
        ok, mabs, mrel = tol_check(h16_to_f32(bits16(out[b])), h16_to_f32(exp["out16"].reshape(out[b].shape)))
        assert ok, (f"{what}: b={b} vs oracle", mabs, mrel)


@pytest.mark.parametrize("H,S,page_size", [(32, 256, 16), (32, 256, 256), (64, 512, 16), (64, 512, 256)])
def test_flash_paged_wave_kernel_against_oracle(H, S, page_size):
    """The production paged wave kernel (lengths in [9000, 40000]: more
    (kv, tile) items than one resident round; GH 4 and 8; pages of 16 and
    256 tokens): bit-identical to the contiguous ragged call, and every
    sequence's m* and vrows exact against the oracle, its output within the
    bf16 tolerance."""
    import santa_flash_batch_cuda as m

    lens = seeded_lens(8, 9000, 40000, SEED + H + page_size)
    assert sum((l + 255) // 256 for l in lens) * 8 > 2048
    seed = SEED + 13 * H + page_size
    print(f"\n[case] flash paged wave kernel vs oracle H={H} lens={lens} S={S} page_size={page_size} seed={seed}",
          flush=True)
    q, K, V, Kp, Vp, table = _inputs(len(lens), H, 8, lens, page_size, torch.bfloat16, seed)
    got = m.decode_systematic_paged(q, Kp, Vp, table, lens, S, seed=SEED, want_vrows=True)
    ref = m.decode_systematic_batched(q, K, V, S, seed=SEED, want_vrows=True, valid_len=lens)
    torch.cuda.synchronize()
    _check(got, ref, True, True, "paged vs contiguous")
    _oracle_checks(got, q, K, V, lens, "flash paged",
                   lambda qc, Kc, Vc, b, Lb: flash_oracle_sequence(qc, Kc, Vc, b, Lb, S, 256))


@pytest.mark.parametrize("H,page_size", [(32, 16), (64, 256)])
def test_flash_paged_full_lists_against_oracle(H, page_size):
    """The paged wave kernel with a budget that fills the per-head sample lists
    within every tile (64 samples per tile and head over lengths in
    [16384, 32768]): the lists are gathered through the page table mid-chunk
    and at the chunk's end.  Bit-identical to the contiguous ragged call;
    every sequence's m* and vrows exact against the oracle, its output within
    the bf16 tolerance."""
    import santa_flash_batch_cuda as m

    lens = seeded_lens(4, 16384, 32768, SEED + 7 * H + page_size)
    assert sum((l + 255) // 256 for l in lens) * 8 > 2048
    S = 64 * max((l + 255) // 256 for l in lens)
    seed = SEED + 17 * H + page_size
    print(f"\n[case] flash paged full lists vs oracle H={H} lens={lens} S={S} page_size={page_size} seed={seed}",
          flush=True)
    q, K, V, Kp, Vp, table = _inputs(len(lens), H, 8, lens, page_size, torch.bfloat16, seed)
    got = m.decode_systematic_paged(q, Kp, Vp, table, lens, S, seed=SEED, want_vrows=True)
    ref = m.decode_systematic_batched(q, K, V, S, seed=SEED, want_vrows=True, valid_len=lens)
    torch.cuda.synchronize()
    _check(got, ref, True, True, "paged vs contiguous")
    _oracle_checks(got, q, K, V, lens, "flash paged",
                   lambda qc, Kc, Vc, b, Lb: flash_oracle_sequence(qc, Kc, Vc, b, Lb, S, 256))


@pytest.mark.parametrize("H,page_size", [(32, 16), (64, 256)])
def test_prop_paged_against_oracle(H, page_size, monkeypatch):
    """Paged batched santa_prop on lengths in [9000, 40000] with S_b = L_b // 64
    (GH 4: the vec pass 1 on the wave kernel; GH 8: the general pass 1):
    every sequence's m* and vrows exact against the oracle of the
    per-sequence call, its output within the bf16 tolerance."""
    import santa_prop_batch_cuda as m

    monkeypatch.delenv("SANTA_PASS1", raising=False)
    lens = seeded_lens(6, 9000, 40000, SEED + 2 * H + page_size)
    Ss = [l // 64 for l in lens]
    seed = SEED + 17 * H + page_size
    print(f"\n[case] prop paged vs oracle H={H} lens={lens} S={Ss} page_size={page_size} seed={seed}", flush=True)
    q, K, V, Kp, Vp, table = _inputs(len(lens), H, 8, lens, page_size, torch.bfloat16, seed)
    got = m.decode_systematic_paged(q, Kp, Vp, table, lens, Ss, seed=SEED, want_vrows=True)
    torch.cuda.synchronize()
    _oracle_checks(got, q, K, V, lens, "prop paged",
                   lambda qc, Kc, Vc, b, Lb: oracle.prop_decode(qc[b], Kc[b, :Lb], Vc[b, :Lb], Ss[b], seed=SEED,
                                                                debug=True))


def test_paged_argument_errors():
    import santa_flash_batch_cuda as flash
    import santa_prop_batch_cuda as prop

    print("\n[case] paged argument errors", flush=True)
    dev = torch.device("cuda:0")
    q = torch.zeros(2, 32, 128, dtype=torch.bfloat16, device=dev)
    Kp = torch.zeros(6, 16, 8, 128, dtype=torch.bfloat16, device=dev)
    table = torch.zeros(2, 3, dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="capacity"):
        flash.decode_systematic_paged(q, Kp, Kp, table, [48, 49], 16)
    with pytest.raises(RuntimeError, match="one entry per sequence"):
        flash.decode_systematic_paged(q, Kp, Kp, table, [10, 20, 30], 16)
    with pytest.raises(RuntimeError, match="int32"):
        flash.decode_systematic_paged(q, Kp, Kp, table.long(), [10, 20], 16)
    with pytest.raises(RuntimeError, match="power of two"):
        Kbad = torch.zeros(6, 12, 8, 128, dtype=torch.bfloat16, device=dev)
        flash.decode_systematic_paged(q, Kbad, Kbad, table, [10, 20], 16)
    with pytest.raises(RuntimeError, match="capacity"):
        prop.decode_systematic_paged(q, Kp, Kp, table, [48, 49], 16)
    with pytest.raises(RuntimeError, match="one row per sequence"):
        prop.decode_systematic_paged(q, Kp, Kp, table[:1].contiguous(), [10, 20], 16)


def test_adapters_decode_paged():
    from santa_amd import attention_backends as ab
    import santa_flash_batch_cuda as flash

    lens = [5000, 3000, 4097]
    seed = SEED + 99
    print(f"\n[case] adapters decode_paged lens={lens} page_size=16 seed={seed}", flush=True)
    q, K, V, Kp, Vp, table = _inputs(len(lens), 32, 8, lens, 16, torch.bfloat16, seed)
    fb = ab.SantaFlashBackend(S=256, seed=SEED, block_n=None)
    out = fb.decode_paged(q, Kp, Vp, table, lens)
    ref = flash.decode_systematic_batched(q, K, V, 256, seed=SEED, valid_len=lens)[0]
    pb = ab.SantaPropBackend(S=300, seed=SEED, block_n=None)
    out_p = pb.decode_paged(q, Kp, Vp, table, lens)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(out), bits16(ref))
    assert fb.info()["actual_mode"] == "paged" and pb.info()["actual_mode"] == "paged"
    assert out_p.shape == (3, 32, 128) and torch.isfinite(out_p.float()).all()
