"""GPU parity of the batched, ragged santa_prop entry point.

Sequence b of a batched call must be decoded exactly as the per-sequence
call on K[b, :valid_len[b]] with budget S[b]: m* bit-exact and vrows exact
against that call (whose every intermediate is bit-exact to the CPU oracle,
tests/test_prop_gpu.py) and against the oracle itself on the smaller cases.
The output sums the same count-weighted rows in another chunking, so it is
checked to the north-star bf16 tolerance (max abs <= 2e-2, mean rel <= 1e-3)
against the per-sequence output and against a torch fp32 restatement of the
estimator given the per-sequence counts.

Every case prints its name, shape and seed before touching the GPU.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import SEED, bits16, gen_qkv, h16_to_f32, tol_check
from test_prop_gpu import prop_estimator_given_counts

pytestmark = pytest.mark.gpu


def _run(H, KVH, lens, Ss, block_n, env, monkeypatch, seed, L_st=None, oracle_check=False, as_tensor=False):
    import santa_prop_batch_cuda as m

    if env is None:
        monkeypatch.delenv("SANTA_PASS1", raising=False)
    else:
        monkeypatch.setenv("SANTA_PASS1", env)
    B = len(lens)
    L_st = L_st or max(lens)
    print(f"\n[case] prop batched H={H} KVH={KVH} L_storage={L_st} lens={lens} S={Ss} block_n={block_n} "
          f"env={env} seed={seed}", flush=True)
    q, K, V = gen_qkv(B, H, KVH, L_st, seed=seed + B, lowrank=0.5)
    dev = torch.device("cuda:0")
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    vl = torch.tensor(lens, dtype=torch.int32) if as_tensor else list(lens)
    out, ms, vr = m.decode_systematic_batched(qd, Kd, Vd, list(Ss), seed=seed, block_n=block_n, want_vrows=True,
                                              valid_len=vl)
    out2, ms2, vr2 = m.decode_systematic_batched(qd, Kd, Vd, list(Ss), seed=seed, block_n=block_n, valid_len=vl)
    torch.cuda.synchronize()
    assert out.shape == (B, H, 128) and ms.shape == (B, H) and vr.shape == (B, KVH) and vr2.numel() == 0
    np.testing.assert_array_equal(bits16(out), bits16(out2), err_msg="repeat call")
    np.testing.assert_array_equal(ms.cpu().numpy().view(np.uint32), ms2.cpu().numpy().view(np.uint32))
    for b, (Lb, Sb) in enumerate(zip(lens, Ss)):
        qb = qd[b].contiguous()
        Kb, Vb = Kd[b, :Lb].contiguous(), Vd[b, :Lb].contiguous()
        ref, ms_r, vr_r = m.decode_systematic_scalar(qb, Kb, Vb, Sb, seed=seed, block_n=block_n, want_vrows=True)
        dbg = m._debug_pass(qb, Kb, Vb, Sb, seed=seed, block_n=block_n)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ms[b].cpu().numpy().view(np.uint32), ms_r.cpu().numpy().view(np.uint32),
                                      err_msg=f"m_star b={b}")
        np.testing.assert_array_equal(vr[b].cpu().numpy(), vr_r.cpu().numpy(), err_msg=f"vrows b={b}")
        got = h16_to_f32(bits16(out[b]))
        ok, mabs, mrel = tol_check(got, h16_to_f32(bits16(ref)))
        assert ok, (f"b={b} vs per-sequence", mabs, mrel)
        est = prop_estimator_given_counts(dbg[7].cpu(), V[b, :Lb], Sb).to(q.dtype).float().numpy()
        ok, mabs, mrel = tol_check(got, est)
        assert ok, (f"b={b} vs torch estimator", mabs, mrel)
        if Sb <= 0:
            assert not got.any(), f"b={b}: S <= 0 must give a zero output"
        if oracle_check:
            exp = oracle.prop_decode(q[b], K[b, :Lb].contiguous(), V[b, :Lb].contiguous(), Sb, seed=seed,
                                     block_n=block_n, is_bf16=True, debug=True)
            np.testing.assert_array_equal(ms[b].cpu().numpy().view(np.uint32), exp["m_star"].view(np.uint32))
            np.testing.assert_array_equal(vr[b].cpu().numpy(), exp["vrows"])
            ok, mabs, mrel = tol_check(got, h16_to_f32(exp["out16"]))
            assert ok, (f"b={b} vs oracle", mabs, mrel)


@pytest.mark.parametrize(
    "H,KVH,lens,Ss,block_n,env",
    [
        # ragged, one block size (256) for every sequence: the single ragged grid
        (32, 8, [12000, 3100, 7777, 4096, 11999], [256, 64, 300, 1, 0], 0, None),
        (32, 8, [12000, 3100, 7777, 4096, 11999], [256, 64, 300, 1, 0], 0, "vec"),
        (32, 8, [12000, 3100, 7777, 4096, 11999], [256, 64, 300, 1, 0], 0, "gqa"),
        # forced small tiles, GH=8, lengths down to one token
        (16, 2, [1, 33, 500, 1000], [7, 40, 256, 1000], 32, None),
        (16, 2, [64, 65, 130, 2000], [3, 64, 129, 500], 64, None),
        # block sizes differ between sequences: one launch sequence each
        (32, 8, [1000, 8000, 2000], [256, 256, 256], 0, None),
    ],
)
def test_prop_batched_parity(H, KVH, lens, Ss, block_n, env, monkeypatch):
    _run(H, KVH, lens, Ss, block_n, env, monkeypatch, SEED)


def test_prop_batched_against_oracle(monkeypatch):
    _run(32, 8, [4000, 3500, 4096], [256, 100, 17], 256, None, monkeypatch, SEED + 3, L_st=4096,
         oracle_check=True, as_tensor=True)


def test_prop_batched_uniform_int_arguments(monkeypatch):
    import santa_prop_batch_cuda as m

    monkeypatch.delenv("SANTA_PASS1", raising=False)
    print("\n[case] prop batched int S / int valid_len B=3 L=5000 valid_len=4500", flush=True)
    q, K, V = gen_qkv(3, 32, 8, 5000, seed=SEED + 9)
    dev = torch.device("cuda:0")
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    a = m.decode_systematic_batched(qd, Kd, Vd, 256, seed=SEED, valid_len=4500, want_vrows=True)
    b = m.decode_systematic_batched(qd, Kd, Vd, [256] * 3, seed=SEED, valid_len=[4500] * 3, want_vrows=True)
    c = m.decode_systematic_batched(qd, Kd[:, :4500].contiguous(), Vd[:, :4500].contiguous(), 256, seed=SEED,
                                    want_vrows=True)
    torch.cuda.synchronize()
    for x, y in ((a, b), (a, c)):
        np.testing.assert_array_equal(bits16(x[0]), bits16(y[0]))
        np.testing.assert_array_equal(x[1].cpu().numpy(), y[1].cpu().numpy())
        np.testing.assert_array_equal(x[2].cpu().numpy(), y[2].cpu().numpy())


def test_prop_batched_errors(monkeypatch):
    import santa_prop_batch_cuda as m

    monkeypatch.delenv("SANTA_PASS1", raising=False)
    print("\n[case] prop batched argument errors", flush=True)
    dev = torch.device("cuda:0")
    q, K, V = gen_qkv(2, 32, 8, 512)
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    with pytest.raises(RuntimeError, match="one entry per sequence"):
        m.decode_systematic_batched(qd, Kd, Vd, [10, 20, 30])
    with pytest.raises(RuntimeError, match="one entry per sequence"):
        m.decode_systematic_batched(qd, Kd, Vd, 10, valid_len=[100])
    with pytest.raises(RuntimeError, match="valid_len exceeds storage length"):
        m.decode_systematic_batched(qd, Kd, Vd, 10, valid_len=[100, 513])
    with pytest.raises(RuntimeError, match="Batch mismatch"):
        m.decode_systematic_batched(qd[:1], Kd, Vd, 10)
    with pytest.raises(RuntimeError, match=r"\[B, L, KVH, D\]"):
        nc = Kd.transpose(0, 1).contiguous().transpose(0, 1)
        m.decode_systematic_batched(qd, nc, nc, 10)


def test_cfg3_workload_parity():
    """The benchmark's batched ragged workload at full size (bench.py
    --workload cfg3: B=16, 32q/8kv, L_b seeded in [8192, 131072], S_b = L_b //
    64, inputs drawn on the device by bench.device_inputs): every sequence's
    m* and vrows exact against the CPU oracle of the per-sequence call, the
    output within the bf16 tolerance (max abs 2e-2, mean rel 1e-3)."""
    import bench
    import santa_prop_batch_cuda as m

    B, H, KVH, D = 16, 32, 8, 128
    gl = torch.Generator().manual_seed(SEED)
    lens = torch.randint(8192, 131072 + 1, (B,), generator=gl).tolist()
    Ss = [l // 64 for l in lens]
    print(f"\n[case] prop cfg3 workload B={B} lens={lens} S={Ss} seed={SEED}", flush=True)
    dev = torch.device("cuda:0")
    q, K, V = bench.device_inputs(B, max(lens), H, KVH, D, SEED, dev)
    out, ms, vr = m.decode_systematic_batched(q, K, V, Ss, seed=SEED, want_vrows=True, valid_len=lens)
    torch.cuda.synchronize()
    qc, Kc, Vc = q.cpu(), K.cpu(), V.cpu()
    del K, V
    for b, (Lb, Sb) in enumerate(zip(lens, Ss)):
        exp = oracle.prop_decode(qc[b], Kc[b, :Lb], Vc[b, :Lb], Sb, seed=SEED, debug=True)
        np.testing.assert_array_equal(ms[b].cpu().numpy().view(np.uint32), exp["m_star"].view(np.uint32),
                                      err_msg=f"m_star b={b}")
        np.testing.assert_array_equal(vr[b].cpu().numpy(), exp["vrows"], err_msg=f"vrows b={b}")
        ok, mabs, mrel = tol_check(h16_to_f32(bits16(out[b])), h16_to_f32(exp["out16"]))
        assert ok, (f"b={b} vs oracle", mabs, mrel)


def test_cfg5_prop_leg_parity():
    """cfg5's santa_prop leg (bench.py --workload cfg5p): 64q/8kv (GH 8, the
    general pass 1), L=131072, Student-t(3) keys with planted needles, S=512
    per sequence (the flash leg's budget), on 2 sequences of the batched call:
    m* and vrows exact against the oracle, the output within the bf16
    tolerance; for sequence 0 also the stage outputs -- tile max and mass, the
    u stash, the budgets S_t, invdelta_t, a0_t and every sampled count --
    bit-exact."""
    import bench
    import santa_prop_batch_cuda as m

    B, H, KVH, L, S = 2, 64, 8, 131072, 512
    print(f"\n[case] prop cfg5 leg B={B} H={H} KVH={KVH} L={L} S={S} needles seed={SEED}", flush=True)
    dev = torch.device("cuda:0")
    q, K, V = bench.device_inputs(B, L, H, KVH, 128, SEED, dev, keys="needles")
    out, ms, vr = m.decode_systematic_batched(q, K, V, S, seed=SEED, want_vrows=True)
    dbg = m._debug_pass(q[0].contiguous(), K[0].contiguous(), V[0].contiguous(), S, seed=SEED)
    torch.cuda.synchronize()
    mt, lt, mstar, St, inv, a0, stash, cnt, out_d, vr_d = [t.cpu() for t in dbg]
    qc, Kc, Vc = q.cpu(), K.cpu(), V.cpu()
    del K, V
    for b in range(B):
        exp = oracle.prop_decode(qc[b], Kc[b], Vc[b], S, seed=SEED, debug=True)
        assert exp["pass1_mode"] == 1 and exp["T_c"] == 512
        np.testing.assert_array_equal(ms[b].cpu().numpy().view(np.uint32), exp["m_star"].view(np.uint32),
                                      err_msg=f"m_star b={b}")
        np.testing.assert_array_equal(vr[b].cpu().numpy(), exp["vrows"], err_msg=f"vrows b={b}")
        ok, mabs, mrel = tol_check(h16_to_f32(bits16(out[b])), h16_to_f32(exp["out16"]))
        assert ok, (f"b={b} vs oracle", mabs, mrel)
        if b == 0:
            for name, got in (("m_tiles", mt), ("ell_tiles", lt), ("invdelta", inv), ("a0", a0)):
                np.testing.assert_array_equal(got.numpy().view(np.uint32), exp[name].view(np.uint32), err_msg=name)
            np.testing.assert_array_equal(St.numpy(), exp["S_tiles"], err_msg="S_tiles")
            assert (St.sum(dim=1) == S).all()
            np.testing.assert_array_equal(bits16(stash), exp["u_stash"], err_msg="u_stash")
            assert np.array_equal(cnt.numpy(), exp["counts"]), "counts"
            np.testing.assert_array_equal(vr_d.numpy(), exp["vrows"], err_msg="vrows (stages)")


@pytest.mark.parametrize("H,KVH,D,lens,Ss,block_n,page_size", [
    (16, 8, 64, [3000, 1700, 2500], [100, 40, 77], 48, 16),
    (32, 2, 128, [900, 2048, 1333, 64], [30, 64, 0, 5], 32, 256),
    (8, 8, 128, [5000, 3300, 700], [80, 60, 10], 256, 16),     # MHA on the fast generic pass 1, ragged
    (24, 8, 256, [4100, 2600], [70, 33], 256, 64),             # GH 3, D 256, fast generic pass 1
    (28, 4, 128, [70000, 50000, 30000], [800, 600, 100], 256, 64),  # GH 7, 2,352 items: the GH 8 wave kernel's pass 1
    (48, 8, 128, [40000, 40000], [300, 500], 256, 256),        # GH 6, 2,504 items, equal lengths: the uniform plan
    (64, 4, 128, [50000, 30000, 20000], [600, 300, 90], 256, 64),  # GH 16 on virtual KV heads, ragged and paged
])
def test_prop_general_batched_and_paged(H, KVH, D, lens, Ss, block_n, page_size, monkeypatch):
    """The generic kernels in the batched, ragged call (one launch sequence over
    the batch) and the paged one: every sequence's m* and vrows exact against
    the oracle of the per-sequence call, the output within the bf16 tolerance,
    and the paged call bit-identical to the contiguous one."""
    import santa_prop_batch_cuda as m
    from test_paged_gpu import make_pool

    monkeypatch.delenv("SANTA_PASS1", raising=False)
    B, L = len(lens), max(lens)
    print(f"\n[case] prop general batched H={H} KVH={KVH} D={D} lens={lens} S={Ss} bn={block_n} page={page_size}",
          flush=True)
    g = torch.Generator().manual_seed(SEED + D)
    q = torch.randn(B, H, D, generator=g).bfloat16()
    K = torch.randn(B, L, KVH, D, generator=g).bfloat16()
    V = torch.randn(B, L, KVH, D, generator=g).bfloat16()
    Kp, Vp, table = make_pool(K, V, lens, page_size, SEED + 1)
    dev = torch.device("cuda:0")
    qd, Kd, Vd, Kpd, Vpd, td = (t.to(dev) for t in (q, K, V, Kp, Vp, table))
    out, ms, vr = m.decode_systematic_batched(qd, Kd, Vd, Ss, seed=SEED, block_n=block_n, want_vrows=True,
                                              valid_len=lens)
    po, pm, pv = m.decode_systematic_paged(qd, Kpd, Vpd, td, lens, Ss, seed=SEED, block_n=block_n, want_vrows=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(po), bits16(out), err_msg="paged vs contiguous: out")
    np.testing.assert_array_equal(pm.cpu().numpy().view(np.uint32), ms.cpu().numpy().view(np.uint32))
    np.testing.assert_array_equal(pv.cpu().numpy(), vr.cpu().numpy())
    for b, (Lb, Sb) in enumerate(zip(lens, Ss)):
        exp = oracle.prop_decode(q[b], K[b, :Lb], V[b, :Lb], Sb, seed=SEED, block_n=block_n, debug=True)
        np.testing.assert_array_equal(ms[b].cpu().numpy().view(np.uint32), exp["m_star"].view(np.uint32),
                                      err_msg=f"m_star b={b}")
        np.testing.assert_array_equal(vr[b].cpu().numpy(), exp["vrows"], err_msg=f"vrows b={b}")
        ok, mabs, mrel = tol_check(h16_to_f32(bits16(out[b])), h16_to_f32(exp["out16"]))
        assert ok, (f"b={b} vs oracle", mabs, mrel)
