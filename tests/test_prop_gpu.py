"""GPU parity of santa_prop against the CPU oracle.

Bit-exact: per-tile max and mass, the u stash, m*, the largest-remainder
budgets S_t, invdelta_t, a0_t and every sampled count; vrows exact.  The
output is summed in a different (fixed) order than the oracle's, so it is
checked to the north-star bf16 tolerance against the oracle and against an
independent torch fp32 restatement of the estimator given the GPU's counts.

Every case prints its name, shape and seed before touching the GPU.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import SEED, bits16, gen_qkv, h16_to_f32, tol_check

pytestmark = pytest.mark.gpu


def _mod():
    import santa_prop_batch_cuda as m

    return m


def _announce(msg):
    print(f"\n[case] {msg}", flush=True)


def prop_estimator_given_counts(counts, V, S):
    """fp32 torch: out[h] = sum_t sum_r c[h,t,r] v[t*BN+r, kv(h)] / S (0 if S <= 0)."""
    H, T_c, BN = counts.shape
    L, KVH, D = V.shape
    GH = H // KVH
    c = counts.float().cpu().reshape(H, T_c * BN)[:, :L].reshape(KVH, GH, L)
    y = torch.einsum("kgl,lkd->kgd", c, V.float().cpu()).reshape(H, D)
    return y / S if S > 0 else torch.zeros_like(y)


def _check(q, K, V, S, seed, block_n=0, pass1_env=None, is_bf16=True, monkeypatch=None):
    m = _mod()
    if pass1_env is None:
        monkeypatch.delenv("SANTA_PASS1", raising=False)
    else:
        monkeypatch.setenv("SANTA_PASS1", pass1_env)
    dev = torch.device("cuda:0")
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    dbg = m._debug_pass(qd, Kd, Vd, S, seed=seed, block_n=block_n)
    out, ms, vr = m.decode_systematic_scalar(qd, Kd, Vd, S, seed=seed, block_n=block_n, want_vrows=True)
    out2, ms2, vr2 = m.decode_systematic_scalar(qd, Kd, Vd, S, seed=seed, block_n=block_n)
    torch.cuda.synchronize()
    mt, lt, mstar, St, inv, a0, stash, cnt, out_d, vr_d = [t.cpu() for t in dbg]
    exp = oracle.prop_decode(q, K, V, S, seed=seed, block_n=block_n, is_bf16=is_bf16, debug=True)
    for name, got in (("m_tiles", mt), ("ell_tiles", lt), ("invdelta", inv), ("a0", a0)):
        np.testing.assert_array_equal(got.numpy().view(np.uint32), exp[name].view(np.uint32), err_msg=name)
    np.testing.assert_array_equal(St.numpy(), exp["S_tiles"], err_msg="S_tiles")
    np.testing.assert_array_equal(bits16(stash), exp["u_stash"], err_msg="u_stash")
    c_gpu = cnt.numpy()
    assert np.array_equal(c_gpu, exp["counts"]), f"counts differ at {np.argwhere(c_gpu != exp['counts'])[:8]}"
    for got in (mstar, ms.cpu()):
        np.testing.assert_array_equal(got.numpy().view(np.uint32), exp["m_star"].view(np.uint32), err_msg="m_star")
    np.testing.assert_array_equal(vr.cpu().numpy(), exp["vrows"], err_msg="vrows")
    np.testing.assert_array_equal(vr_d.numpy(), exp["vrows"], err_msg="vrows (stages)")
    assert vr2.numel() == 0
    # the three stage entry points and the fused decode give the same bits
    np.testing.assert_array_equal(bits16(out), bits16(out_d), err_msg="decode vs stages")
    np.testing.assert_array_equal(bits16(out), bits16(out2), err_msg="repeat call")
    T_c = St.shape[1]
    if S > 0 and T_c & (T_c - 1) == 0:
        # the budgets sum to S when the bitonic network is a full power of two;
        # padded to one, the reference's network can drop candidates
        # (prop/santa_cuda_kernel.cu:686-707), which the oracle reproduces
        assert (St.sum(dim=1) == S).all(), "budgets must sum to S per head"
    got = h16_to_f32(bits16(out), is_bf16)
    ok, mabs, mrel = tol_check(got, h16_to_f32(exp["out16"], is_bf16))
    assert ok, ("vs oracle", mabs, mrel)
    ref = prop_estimator_given_counts(cnt, V, S).to(q.dtype).float().numpy()
    ok, mabs, mrel = tol_check(got, ref)
    assert ok, ("vs torch estimator", mabs, mrel)
    return exp


@pytest.mark.parametrize(
    "H,KVH,L,S,block_n,env",
    [
        (32, 8, 5000, 5000 // 64, 0, None),     # vec path, BN 256, ragged last tile
        (32, 8, 32768, 512, 0, None),           # vec path, 128 tiles
        (32, 8, 1000, 40, 0, None),             # general path, BN 32
        (32, 8, 2000, 64, 0, None),             # general path, BN 64
        (32, 8, 4096, 64, 0, "gqa"),            # general path forced at BN 256
        (32, 8, 3000, 300, 0, "vec"),           # vec forced: BN 256 chosen by the env
        (64, 8, 3000, 100, 0, None),            # GH 8 (general path), BN 64
        (64, 8, 9000, 150, 0, None),            # GH 8 (general path), BN 256
        (32, 8, 700, 0, 256, None),             # S = 0 -> zeros
        (32, 8, 2048, 100000, 256, None),       # S far above the tile count
        (32, 8, 33, 3, 32, None),               # two tiles, one of one row
    ],
)
def test_prop_parity(H, KVH, L, S, block_n, env, monkeypatch):
    _announce(f"prop H={H} KVH={KVH} L={L} S={S} bn={block_n} SANTA_PASS1={env}")
    q, K, V = gen_qkv(1, H, KVH, L, seed=SEED + L + H, single=True)
    exp = _check(q, K, V, S, SEED, block_n=block_n, pass1_env=env, monkeypatch=monkeypatch)
    if S == 0:
        assert not exp["out16"].any()


def test_prop_f16_and_peaky(monkeypatch):
    _announce("prop f16 L=6000 S=100 and bf16 low-rank keys L=20000 S=312")
    q, K, V = gen_qkv(1, 32, 8, 6000, seed=SEED, dtype=torch.float16, single=True)
    _check(q, K, V, 100, SEED, is_bf16=False, monkeypatch=monkeypatch)
    q, K, V = gen_qkv(1, 32, 8, 20000, seed=SEED + 7, lowrank=0.5, single=True)
    _check(q, K, V, 312, 1690, monkeypatch=monkeypatch)


def test_prop_errors(monkeypatch):
    _announce("prop input errors")
    m = _mod()
    dev = torch.device("cuda:0")
    q, K, V = gen_qkv(1, 32, 8, 512, single=True)
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    with pytest.raises(RuntimeError, match="bad ranks"):
        m.decode_systematic_scalar(qd[None], Kd, Vd, 8)
    Kn = Kd.transpose(1, 2).contiguous().transpose(1, 2)  # [L, KVH, D], not contiguous
    with pytest.raises(RuntimeError, match=r"K_g/V_g must be contiguous with layout \[L, KVH, D\] \(NHD\)"):
        m.decode_systematic_scalar(qd, Kn, Vd, 8)
    monkeypatch.setenv("SANTA_PASS1", "vec")
    with pytest.raises(RuntimeError, match="SANTA_PASS1=vec requires GH=4, D=128, block_n=256"):
        m.decode_systematic_scalar(qd, Kd, Vd, 8, block_n=64)
    monkeypatch.delenv("SANTA_PASS1")
    with pytest.raises(TypeError):
        m.decode_systematic_scalar(qd, Kd, Vd, 8, valid_len=3)


def _general_inputs(H, KVH, D, L, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(H, D, generator=g)
    K = torch.randn(L, KVH, D, generator=g)
    V = torch.randn(L, KVH, D, generator=g)
    return q.to(dtype), K.to(dtype), V.to(dtype)


@pytest.mark.parametrize(
    "H,KVH,D,L,S,block_n",
    [
        (8, 8, 128, 3000, 200, 0),     # GH 1 (auto block_n 64)
        (16, 8, 64, 5000, 300, 0),     # GH 2, D 64 (block_n 256)
        (32, 2, 128, 2000, 150, 48),   # GH 16, block_n 48
        (12, 4, 80, 1000, 90, 16),     # GH 3, D 80, block_n 16
        (32, 8, 128, 4000, 250, 128),  # GH 4 at block_n 128
        (16, 1, 256, 900, 64, 512),    # GH 16, D 256, block_n 512
        (4, 4, 16, 700, 40, 32),       # GH 1, D 16
        (32, 8, 48, 2500, 100, 0),     # GH 4, D 48
    ],
)
def test_prop_general_shapes(H, KVH, D, L, S, block_n, monkeypatch):
    """Shapes outside the tuned kernels (the reference's general path takes
    any GH, D % 16 == 0 and block_n % 16 == 0, prop/santa_cuda.cpp:212-259):
    tile max and mass, the stash, the budgets and every count bit-exact to the
    oracle, m* and vrows exact, the output within the bf16 tolerance."""
    _announce(f"prop general shape H={H} KVH={KVH} D={D} L={L} S={S} bn={block_n}")
    q, K, V = _general_inputs(H, KVH, D, L, SEED + 3 * D + H)
    exp = _check(q, K, V, S, SEED, block_n=block_n, monkeypatch=monkeypatch)
    assert exp["pass1_mode"] == 1


@pytest.mark.parametrize(
    "H,KVH,D,L,S",
    [
        (8, 8, 128, 5000, 300),    # MHA (GH 1: one head block, three of its heads unused)
        (16, 8, 256, 4000, 200),   # GH 2, D 256
        (32, 2, 128, 3000, 150),   # GH 16: four head blocks
        (12, 4, 64, 3500, 100),    # GH 3 (odd: 16-bit stash stores), D 64
        (64, 8, 256, 2600, 90),    # GH 8, D 256: two head blocks
        (48, 4, 64, 6000, 256),    # GH 12, D 64 (a padded fourth block)
    ],
)
def test_prop_fast_generic_pass1(H, KVH, D, L, S, monkeypatch):
    """block_n 256 on shapes outside the tuned kernels runs the MFMA generic
    pass 1 (K by 16-byte loads into swizzled LDS, broadcast 4x4x1 MFMA
    chains in the general association): tile max and mass, the stash, the
    budgets and every count bit-exact to the oracle, m* and vrows exact, the
    output within the bf16 tolerance.  The last tile is partial in each."""
    _announce(f"prop fast generic pass 1 H={H} KVH={KVH} D={D} L={L} S={S} bn=256")
    q, K, V = _general_inputs(H, KVH, D, L, SEED + 7 * D + H)
    exp = _check(q, K, V, S, SEED, block_n=256, monkeypatch=monkeypatch)
    assert exp["pass1_mode"] == 1 and exp["T_c"] == (L + 255) // 256


@pytest.mark.parametrize("H,KVH,D,L,S", [
    (32, 32, 128, 32700, 512),   # MHA: chunks of 8 tiles per workgroup, the next tile's rows in registers
    (32, 4, 64, 40000, 600),     # GH 8 at D 64 (two head blocks, registers): chunks of 2 tiles
    (8, 2, 256, 40000, 300),     # GH 4 at D 256 (one workgroup per CU): chunks of 2 tiles
    (28, 4, 128, 140000, 512),   # GH 7 at D 128, 2,188 items: santa_flash's GH 8 pass-1 wave kernel, four-wave layout
    (40, 8, 128, 70000, 300),    # GH 5, 2,192 items: the GH 8 wave kernel in its rows layout
    (28, 4, 128, 32700, 512),    # GH 7 below 2,048 items: the generic kernel
    (64, 4, 128, 70000, 512),    # GH 16: two virtual KV heads of 8 per cache KV head, rows layout
    (128, 8, 128, 40000, 512),   # GH 16 at 128q/8kv (Llama-3.1-405B's heads): 16 virtual KV heads, four-wave layout
    (48, 4, 128, 70000, 300),    # GH 12: virtual groups of 6
])
def test_prop_fast_generic_streaming(H, KVH, D, L, S, monkeypatch):
    """The generic pass 1 streaming a chunk of tiles per workgroup (one
    resident round of (KV head, chunk) items, the next tile's rows loaded
    while the current one is scored) and the tile-major stash of the fused
    decode: every stage bit-exact to the oracle, the fused decode equal to the
    stage entry points bit for bit.  The last tile is partial in each."""
    _announce(f"prop fast generic streaming H={H} KVH={KVH} D={D} L={L} S={S} bn=256")
    q, K, V = _general_inputs(H, KVH, D, L, SEED + 11 * D + H)
    exp = _check(q, K, V, S, SEED, block_n=256, monkeypatch=monkeypatch)
    assert exp["pass1_mode"] == 1 and exp["T_c"] == (L + 255) // 256


@pytest.mark.parametrize("H,KVH,D,L,S,block_n", [(8, 4, 512, 1500, 60, 64), (4, 2, 1024, 900, 40, 32),
                                                  (4, 4, 512, 3100, 50, 256)])
def test_prop_head_dim_above_256(H, KVH, D, L, S, block_n, monkeypatch):
    """Head dims above 256 (the reference's general path takes any D % 16 ==
    0, prop/santa_cuda.cpp:212-215): every stage bit-exact to the oracle, the
    output within the bf16 tolerance."""
    _announce(f"prop D > 256 H={H} KVH={KVH} D={D} L={L} S={S} bn={block_n}")
    q, K, V = _general_inputs(H, KVH, D, L, SEED + D)
    exp = _check(q, K, V, S, SEED, block_n=block_n, monkeypatch=monkeypatch)
    assert exp["pass1_mode"] == 1


@pytest.mark.parametrize("H,KVH,L,S", [(28, 4, 140000, 512), (64, 4, 70000, 300)])
def test_prop_gh8_route_f16(H, KVH, L, S, monkeypatch):
    """f16 through santa_flash's GH 8 pass-1 wave kernel on santa_prop's
    generic shapes (GH 7 with each group's eighth head zero; GH 16 over two
    virtual KV heads per cache KV head), above the 2,048-item threshold: every
    stage bit-exact to the oracle, the fused decode equal to the stages."""
    _announce(f"prop GH 8 route f16 H={H} KVH={KVH} L={L} S={S} bn=256")
    q, K, V = _general_inputs(H, KVH, 128, L, SEED + 17 + H, dtype=torch.float16)
    exp = _check(q, K, V, S, SEED, block_n=256, is_bf16=False, monkeypatch=monkeypatch)
    assert exp["pass1_mode"] == 1


def test_prop_fast_generic_f16(monkeypatch):
    _announce("prop fast generic pass 1 f16 H=16 KVH=8 D=64 L=3300 S=90 bn=256")
    q, K, V = _general_inputs(16, 8, 64, 3300, SEED + 9, dtype=torch.float16)
    _check(q, K, V, 90, SEED, block_n=256, is_bf16=False, monkeypatch=monkeypatch)


@pytest.mark.parametrize("H,KVH,L,S", [(32, 8, 20000, 300), (64, 8, 20000, 300)])
def test_prop_wave_pass1_f16(H, KVH, L, S, monkeypatch):
    """f16 through the wave-kernel pass 1 (GH 4 vec path, GH 8 general path)
    above the small pass, with the tile-major stash of the fused decode: every
    stage bit-exact to the oracle, the fused decode equal to the stages."""
    _announce(f"prop wave pass 1 f16 H={H} KVH={KVH} L={L} S={S} bn=256")
    q, K, V = _general_inputs(H, KVH, 128, L, SEED + 13 + H, dtype=torch.float16)
    _check(q, K, V, S, SEED, block_n=256, is_bf16=False, monkeypatch=monkeypatch)


def test_prop_general_f16(monkeypatch):
    _announce("prop general shape f16 H=16 KVH=8 D=96 L=1500 S=70 bn=32")
    q, K, V = _general_inputs(16, 8, 96, 1500, SEED + 5, dtype=torch.float16)
    _check(q, K, V, 70, SEED, block_n=32, is_bf16=False, monkeypatch=monkeypatch)


@pytest.mark.parametrize("H,KVH,D,L,block_n", [(32, 8, 128, 140000, 32), (8, 4, 64, 70000, 16)])
def test_prop_more_than_4096_tiles(H, KVH, D, L, block_n, monkeypatch):
    """4375 tiles per head: beyond the register network's 4096, the budgets
    run their network in memory (for the tuned GH 4 / D 128 passes at block_n
    32 and for a generic shape alike); every stage bit-exact to the oracle."""
    _announce(f"prop T_c > 4096 H={H} KVH={KVH} D={D} L={L} bn={block_n}")
    q, K, V = _general_inputs(H, KVH, D, L, SEED + L)
    exp = _check(q, K, V, L // 50, SEED, block_n=block_n, monkeypatch=monkeypatch)
    assert exp["T_c"] == 4375


def test_prop_unbiased_given_budgets_at_full_size():
    """santa_prop on one sequence of 32768 tokens (32q/8kv, S = L / 64 = 512,
    the rank-4 key bias recipe) through the production call.  Its output is
    sum_r c_r v_r / S with integer tile budgets S_t from the largest-remainder
    allocation, so it estimates sum_t (S_t / S) o_t rather than exact
    attention; given the budgets, the systematic sampler's expected count of
    row r is x_r = f32(u16_r) * invdelta_t.  The output averaged over 2048
    seeds agrees with sum_r x_r v_r / S (budgets and u16 from the debug call)
    within 6 standard errors of the mean in every element (plus 0.4 % of the
    value for the bf16 rounding of each output), and the same criterion
    rejects that expectation scaled by 1.1."""
    import santa_prop_batch_cuda as m

    H, KVH, L, D, BN = 32, 8, 32768, 128, 256
    S = L // 64
    n = 2048
    print(f"\n[case] prop unbiased given budgets over {n} seeds H={H} KVH={KVH} L={L} S={S}", flush=True)
    q, K, V = gen_qkv(1, H, KVH, L, seed=SEED + 23, lowrank=0.5)
    dev = torch.device("cuda:0")
    qd, Kd, Vd = q[0].to(dev), K[0].to(dev), V[0].to(dev)
    dbg = m._debug_pass(qd, Kd, Vd, S, seed=0)
    invdelta, stash = dbg[4], dbg[6]  # [H, T_c], [L, H]
    x = stash.float().t() * invdelta.repeat_interleave(BN, dim=1)[:, :L]  # [H, L]
    GH = H // KVH
    Vf = Vd.float()  # [L, KVH, D]
    expected = torch.stack([x[h] @ Vf[:, h // GH, :] for h in range(H)]) / S  # [H, D]
    acc = torch.zeros(H, D, dtype=torch.float64, device=dev)
    acc2 = torch.zeros(H, D, dtype=torch.float64, device=dev)
    for sd in range(n):
        out, _, _ = m.decode_systematic_scalar(qd, Kd, Vd, S, seed=sd)
        o = out.double()
        acc += o
        acc2 += o * o
    mean = acc / n
    se = ((acc2 / n - mean * mean).clamp_min(0.0) / n).sqrt()
    ex = expected.double()
    floor = 4e-3 * ex.abs() + 1e-6
    zs = {f: ((mean - (1.0 + f) * ex).abs() / (se + floor)).max().item() for f in (0.0, 0.02, 0.05, 0.1, 0.2)}
    print("[case] z for a scale error of " + ", ".join(f"{f:.0%}: {v:.2f}" for f, v in zs.items()), flush=True)
    assert zs[0.0] < 6.0, zs
    assert zs[0.1] > 6.0, zs
