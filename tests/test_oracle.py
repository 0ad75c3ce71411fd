"""Pins for the CPU oracle (oracle/santa_oracle.c), which the GPU parity
tests trust.  Every check here comes from outside the oracle's own formula:
published known answers (SplitMix64), the anchors derived from the
reference's RNG, closed forms (uniform tile, one-hot tile, planning),
float64 brute force on small inputs, library conversions (torch / numpy
round-to-nearest-even), and statistical properties of the estimator
(unbiasedness, convergence to exact softmax attention as S grows).  Each is
chosen so that a plausible slip -- a dropped term, a swapped index, an
inclusive/exclusive scan mix-up, a missing normalization -- fails it.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from helpers import SEED, gen_qkv, h16_to_f32, tol_check

F32_MAX_EXP = 88.72283935546875


# ------------------------------------------------------------------ RNG
def test_splitmix64_known_answer():
    # first output of Vigna's SplitMix64 seeded with 0
    assert oracle.splitmix64(0) == 0xE220A8397B1DCDAF


@pytest.mark.parametrize(
    "seed,key,t,want",
    [(1690, 0, 0, 0.407740563), (1690, 1, 0, 0.717892289), (1690, 0, 1, 0.164398178), (42, 0, 0, 0.74156487),
     (1690, 31, 127, 0.114427596)],
)
def test_u01_anchors(seed, key, t, want):
    # anchors derived from the reference's u01_from_seed
    # (flash/santa_cuda_kernel.cu:74-87), printed to 9 digits
    assert abs(oracle.u01(seed, key, t) - want) < 1e-9


def test_u01_range_and_packing():
    keys = np.arange(-4, 300, dtype=np.int32).repeat(3)
    ts = np.tile(np.array([0, 1, 4095], np.int32), keys.size // 3)
    u = oracle.u01_array(SEED, keys, ts)
    assert (u >= 0).all() and (u < 1).all()
    # key and t occupy different halves of the 64-bit word: swapping them
    # changes the draw
    assert oracle.u01(SEED, 3, 5) != oracle.u01(SEED, 5, 3)
    # 64-bit seeds are used whole
    assert oracle.u01(SEED + (1 << 40), 0, 0) != oracle.u01(SEED, 0, 0)


# ------------------------------------------------------------------ EXP
def _ulp_err(y, x):
    ref = np.exp(x.astype(np.float64))
    y64 = y.astype(np.float64)
    ulp = 2.0 ** (np.floor(np.log2(ref)) - 23)  # binary32 ulp at the true value (normal range)
    return np.abs(y64 - ref) / ulp


def test_expf_accuracy_normal_range():
    rng = np.random.default_rng(0)
    x = np.concatenate([np.linspace(-87.3, 88.7228, 2_000_001, dtype=np.float32),
                        rng.uniform(-30, 0, 1_000_000).astype(np.float32),
                        rng.uniform(-1e-3, 1e-3, 100_000).astype(np.float32)])
    y = oracle.expf(x)
    assert _ulp_err(y, x).max() <= 2.0
    assert oracle.expf(np.array([0.0], np.float32))[0] == 1.0
    assert oracle.expf(np.array([-0.0], np.float32))[0] == 1.0


def test_expf_subnormal_and_special():
    x = np.linspace(-103.9, -87.4, 200_001, dtype=np.float32)
    y = oracle.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.maximum(2.0 ** (np.floor(np.log2(ref)) - 23), 2.0 ** -149)
    assert (np.abs(y - ref) <= 2 * ulp).all()
    sp = oracle.expf(np.array([np.inf, -np.inf, np.nan, 89.0, -104.0, 88.7228, -200.0, F32_MAX_EXP], np.float32))
    assert sp[0] == np.inf and sp[1] == 0.0 and np.isnan(sp[2]) and sp[3] == np.inf and sp[4] == 0.0
    assert np.isfinite(sp[5]) and sp[6] == 0.0
    # exp(88.72283935546875) exceeds FLT_MAX by more than half an ulp
    assert sp[7] == np.inf


# ------------------------------------------------------------------ conversions
def _conversion_inputs():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    # exact ties for bf16 (low 16 bits = 0x8000) and for f16, subnormals, specials
    ties = (rng.integers(0, 2 ** 16, 5000, dtype=np.uint32) << 16 | 0x8000).astype(np.uint32).view(np.float32)
    f16_ties = (np.arange(1, 5000, dtype=np.float32) + 0.5) / 1024.0
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65520.0, 65519.99, 6e-8, 3e-8, 2.9e-8, 1e-45,
                        3.4e38, -3.4e38, 1.0, -1.0], np.float32)
    return np.concatenate([x, ties, f16_ties, special])


def test_bf16_round_to_nearest_even_matches_torch():
    x = _conversion_inputs()
    got = oracle.f32_to_h16(x, True)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert ((got[nan] & 0x7F80) == 0x7F80).all() and ((got[nan] & 0x7F) != 0).all()
    back = oracle.h16_to_f32(want[~nan], True)
    assert np.array_equal(back, torch.from_numpy(want[~nan].view(np.int16)).view(torch.bfloat16).float().numpy())


def test_f16_round_to_nearest_even_matches_numpy():
    x = _conversion_inputs()
    got = oracle.f32_to_h16(x, False)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert ((got[nan] & 0x7C00) == 0x7C00).all() and ((got[nan] & 0x3FF) != 0).all()
    assert np.array_equal(oracle.h16_to_f32(want[~nan], False), want[~nan].view(np.float16).astype(np.float32))


# ------------------------------------------------------------------ planning
def test_planning_closed_forms():
    # flash/santa_cuda.cpp:36-44
    assert [oracle.auto_block_n(L) for L in (1, 1536, 1537, 3072, 3073, 131072)] == [32, 32, 64, 64, 256, 256]
    # S_per_tile = S > 0 ? max(1, S / T_c) : 0 (flash/santa_cuda.cpp:202-208)
    assert oracle.flash_s_per_tile(0, 16) == 0
    assert oracle.flash_s_per_tile(-5, 16) == 0
    assert oracle.flash_s_per_tile(32, 16) == 2
    assert oracle.flash_s_per_tile(5, 16) == 1
    assert oracle.flash_s_per_tile(256, 128) == 2
    assert oracle.flash_s_per_tile(256, 129) == 1
    assert oracle.flash_s_per_tile(512, 512) == 1


# ------------------------------------------------------------------ flash closed forms
def test_uniform_tile_sampler_known_answer():
    """q = 0: every score is 0, u = 1, ell = 256, x = S_pt / 256 per row, so
    head h of tile t samples rows ceil((k - a0) * 256 / S_pt) - 1, k = 1..S_pt
    with a0 = u01(seed, b*H + h, t).  Seed 1690, b = h = t = 0: rows 75, 203."""
    q, K, V = gen_qkv(1, 32, 8, 4096)
    q = torch.zeros_like(q)
    r = oracle.flash_decode(q, K, V, 32, seed=SEED, debug=True)
    assert r["S_per_tile"] == 2 and r["block_n"] == 256
    c = r["counts"][0]
    assert sorted(np.nonzero(c[0, 0])[0].tolist()) == [75, 203]
    assert (r["m_tiles"] == 0).all() and (r["ell_tiles"] == 256.0).all()
    for h in range(32):
        for t in range(16):
            a0 = oracle.u01(SEED, h, t)
            rows = [math.ceil((k - a0) * 128) - 1 for k in (1, 2)]
            want = np.zeros(256, np.int16)
            want[rows] = 1
            assert np.array_equal(c[h, t], want), (h, t)


def test_uniform_tile_sampler_known_answer_batch_key():
    """The same closed form at B = 2: sequence b draws with RNG key b*H + h
    (flash/santa_cuda_kernel.cu:281), so sequence 1's rows come from
    u01(seed, H + h, t).  A key slip (b*KVH + h, or h alone) moves them."""
    H = 32
    q, K, V = gen_qkv(2, H, 8, 4096)
    q = torch.zeros_like(q)
    r = oracle.flash_decode(q, K, V, 32, seed=SEED, debug=True)
    c = r["counts"]
    for b in range(2):
        for h in range(H):
            for t in range(16):
                a0 = oracle.u01(SEED, b * H + h, t)
                want = np.zeros(256, np.int16)
                want[[math.ceil((k - a0) * 128) - 1 for k in (1, 2)]] = 1
                assert np.array_equal(c[b, h, t], want), (b, h, t)
    # the key slips would pick other rows for sequence 1 somewhere
    slip = [oracle.u01(SEED, 8 + h, t) for h in range(H) for t in range(16)]
    true = [oracle.u01(SEED, H + h, t) for h in range(H) for t in range(16)]
    assert slip != true


def test_b_offset_equals_the_batched_sequence():
    """flash_decode(q[b:b+1], ..., b_offset=b) is sequence b of the batched
    call: same counts, statistics, m*, vrows and output bits."""
    q, K, V = gen_qkv(3, 16, 4, 1000, seed=SEED + 11)
    full = oracle.flash_decode(q, K, V, 24, seed=SEED, debug=True)
    for b in range(3):
        one = oracle.flash_decode(q[b:b + 1], K[b:b + 1], V[b:b + 1], 24, seed=SEED, debug=True, b_offset=b)
        for key in ("counts", "m_tiles", "ell_tiles", "m_star", "vrows", "out"):
            got, want = np.asarray(one[key])[0], np.asarray(full[key])[b]
            assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), (b, key)
        if b > 0:
            zero = oracle.flash_decode(q[b:b + 1], K[b:b + 1], V[b:b + 1], 24, seed=SEED, debug=True)
            assert not np.array_equal(zero["counts"][0], full["counts"][b])


def test_one_hot_tile_takes_every_sample():
    """One key row aligned with the group's query (score ~ 45 nats above the
    rest) receives all S_pt samples of its tile for every head."""
    q, K, V = gen_qkv(1, 4, 1, 512, seed=SEED + 3)
    q[0] = q[0, 0:1].expand(4, 128)
    star = 300
    K[0, star, 0] = (q[0, 0].float() * 4).to(K.dtype)
    r = oracle.flash_decode(q, K, V, 16, seed=SEED, block_n=256, debug=True)
    S_pt = r["S_per_tile"]
    c = r["counts"][0]
    t, rr = divmod(star, 256)
    for h in range(4):
        assert c[h, t, rr] == S_pt and c[h, t].sum() == S_pt


# ------------------------------------------------------------------ flash brute force
def _scores64(q, K):
    """float64 scaled scores [B,H,L] with f32 (q * q_scale) as the kernels use."""
    B, H, D = q.shape
    KVH = K.shape[2]
    GH = H // KVH
    scale = np.float32(1.0) / np.sqrt(np.float32(D))
    qf = (q.float().numpy() * scale).astype(np.float32).astype(np.float64)
    Kf = K.float().numpy().astype(np.float64)
    s = np.empty((B, H, K.shape[1]))
    for h in range(H):
        s[:, h] = np.einsum("bd,bld->bl", qf[:, h], Kf[:, :, h // GH])
    return s


@pytest.mark.parametrize("L,bn,S", [(300, 0, 40), (777, 64, 100), (1000, 256, 9)])
def test_flash_tile_statistics_bruteforce(L, bn, S):
    q, K, V = gen_qkv(2, 8, 2, L, seed=SEED + L)
    r = oracle.flash_decode(q, K, V, S, seed=SEED, block_n=bn, debug=True)
    BN, T_c = r["block_n"], r["T_c"]
    s = _scores64(q, K)
    for t in range(T_c):
        st = s[:, :, t * BN:(t + 1) * BN]
        m64 = st.max(axis=2)
        assert np.allclose(r["m_tiles"][:, :, t], m64, rtol=1e-5, atol=1e-5)
        ell64 = np.exp(st - r["m_tiles"][:, :, t, None].astype(np.float64)).sum(axis=2)
        assert np.allclose(r["ell_tiles"][:, :, t], ell64, rtol=2e-6 * BN ** 0.5 + 1e-6)
    assert np.array_equal(r["m_star"], r["m_tiles"].max(axis=2))


@pytest.mark.parametrize("L,bn,S", [(300, 0, 40), (2500, 0, 1000), (5000, 256, 64)])
def test_flash_count_invariants(L, bn, S):
    """Per (b, h, t): total = S_pt or S_pt +- 1 (x sums to S_pt up to the
    16-bit rounding of u); every count is floor(x_r) or ceil(x_r) with x_r
    from float64 scores; vrows = |union of sampled rows| per group."""
    q, K, V = gen_qkv(1, 8, 2, L, seed=SEED + 2 * L)
    r = oracle.flash_decode(q, K, V, S, seed=SEED, block_n=bn, debug=True)
    BN, T_c, S_pt = r["block_n"], r["T_c"], r["S_per_tile"]
    c = r["counts"][0].astype(np.int64)
    tot = c.sum(axis=2)
    assert (np.abs(tot - S_pt) <= 1).all()
    s = _scores64(q, K)[0]
    for t in range(T_c):
        st = s[:, t * BN:(t + 1) * BN]
        x = S_pt * np.exp(st - st.max(axis=1, keepdims=True))
        x /= np.exp(st - st.max(axis=1, keepdims=True)).sum(axis=1, keepdims=True)
        ct = c[:, t, :st.shape[1]]
        # allow the 16-bit rounding of u (relative 2^-8) near integer edges
        lo = np.floor(x * (1 - 2 ** -7) - 1e-6)
        hi = np.ceil(x * (1 + 2 ** -7) + 1e-6)
        assert ((ct >= lo) & (ct <= hi)).all(), t
    union = (r["counts"][0].reshape(2, 4, T_c * BN)[:, :, :L] > 0).any(axis=1).sum(axis=1)
    assert np.array_equal(r["vrows"][0], union)


def test_systematic_counts_float64_model():
    """so_counts_1d (the 32-lane scan with carries, A.7) against float64
    systematic sampling: c_r = floor(a0 + C_r) - floor(a0 + C_{r-1}) with
    C the running sum, away from integer edges."""
    rng = np.random.default_rng(7)
    for trial in range(200):
        n = int(rng.integers(1, 257))
        u = rng.random(n).astype(np.float32) ** 3
        ub = oracle.f32_to_h16(u, True)
        uf = oracle.h16_to_f32(ub, True).astype(np.float64)
        S_pt = int(rng.integers(1, 40))
        ell = np.float32(uf.sum())
        invdel = np.float32(S_pt) / ell
        a0 = float(rng.random())
        c = oracle.counts_1d(ub, float(invdel), a0).astype(np.int64)
        x = uf * float(invdel)
        C = np.concatenate([[0.0], np.cumsum(x)])
        want = np.floor(a0 + C[1:]) - np.floor(a0 + C[:-1])
        frac_hi = np.abs((a0 + C[1:]) - np.round(a0 + C[1:]))
        frac_lo = np.abs((a0 + C[:-1]) - np.round(a0 + C[:-1]))
        safe = (frac_hi > 1e-4) & (frac_lo > 1e-4)
        assert np.array_equal(c[safe], want[safe]), trial
        assert abs(int(c.sum()) - (math.floor(a0 + C[-1]) - math.floor(a0))) <= 1


def test_flash_output_given_counts_float64():
    """y[h] = sum_t w_t sum_r c_r v_r / (Z S_pt), w_t = exp(m_t - m*) ell_t,
    recomputed in float64 from the oracle's own statistics and counts."""
    q, K, V = gen_qkv(2, 8, 2, 1500, seed=SEED + 11)
    r = oracle.flash_decode(q, K, V, 48, seed=SEED, block_n=64, debug=True)
    BN, T_c, S_pt = r["block_n"], r["T_c"], r["S_per_tile"]
    m = r["m_tiles"].astype(np.float64)
    w = np.exp(m - m.max(axis=2, keepdims=True)) * r["ell_tiles"]
    Z = w.sum(axis=2)
    Vf = V.float().numpy().astype(np.float64)
    L = K.shape[1]
    y = np.zeros((2, 8, 128))
    for b in range(2):
        for h in range(8):
            cw = (r["counts"][b, h].astype(np.float64) * w[b, h, :, None]).reshape(-1)[:L]
            y[b, h] = cw @ Vf[b, :, h // 4] / (Z[b, h] * S_pt)
    assert np.allclose(r["out"], y, rtol=1e-4, atol=2e-5)


def _exact_attention(q, K, V):
    B, H, D = q.shape
    KVH = K.shape[2]
    s = _scores64(q, K)
    p = np.exp(s - s.max(axis=2, keepdims=True))
    p /= p.sum(axis=2, keepdims=True)
    Vf = V.float().numpy().astype(np.float64)
    out = np.empty((B, H, D))
    for h in range(H):
        out[:, h] = np.einsum("bl,bld->bd", p[:, h], Vf[:, :, h // (H // KVH)])
    return out


def test_flash_converges_to_exact_attention():
    """With S_pt = 16384 samples per 256-row tile the estimator is exact
    softmax attention up to count rounding (<= 1 per row) and the 16-bit
    rounding of u; checked in float64 with the bf16 tolerance."""
    q, K, V = gen_qkv(1, 8, 2, 1024, seed=SEED + 5, lowrank=0.5)
    T_c = 4
    r = oracle.flash_decode(q, K, V, 16384 * T_c, seed=SEED, block_n=256)
    exact = _exact_attention(q, K, V)
    ok, mabs, mrel = tol_check(r["out"], exact, max_abs=2e-2, mean_rel=5e-3)
    assert ok, (mabs, mrel)


def test_flash_unbiased_over_seeds():
    """The sampled estimate averaged over seeds converges to exact attention
    (error shrinking like 1/sqrt(n)); a missing tile weight or normalization
    would leave a bias far above the standard error."""
    q, K, V = gen_qkv(1, 4, 1, 64, seed=SEED + 9, lowrank=0.5)
    qb, Kb, Vb = oracle.as_bits(q), oracle.as_bits(K), oracle.as_bits(V)
    n = 3000
    outs = np.stack([oracle.flash_decode(qb, Kb, Vb, 4, seed=sd, block_n=32)["out"] for sd in range(n)])
    mean = outs.mean(axis=0)
    se = outs.std(axis=0) / math.sqrt(n)
    exact = _exact_attention(q, K, V)
    z = np.abs(mean - exact) / (se + 1e-3)
    assert z.max() < 6.0, z.max()


# ------------------------------------------------------------------ prop
def _bitonic_model(frac, T_c):
    """Brute-force model of the reference's budget sort
    (prop/santa_cuda_kernel.cu:686-707): a bitonic network over the next
    power of two, descending, where positions past T_c read as (-inf, -1)
    and are never stored."""
    N = 1
    while N < T_c:
        N *= 2
    a = list(frac) + [-math.inf] * (N - T_c)
    ix = list(range(T_c)) + [-1] * (N - T_c)
    k = 2
    while k <= N:
        j = k // 2
        while j > 0:
            new_a, new_ix = a[:], ix[:]
            for i in range(N):
                p = i ^ j
                if p > i:
                    up = (i & k) != 0
                    ai, aj, ii, ij = a[i], a[p], ix[i], ix[p]
                    if (ai > aj) == up:
                        ai, aj, ii, ij = aj, ai, ij, ii
                    new_a[i], new_ix[i], new_a[p], new_ix[p] = ai, ii, aj, ij
            for i in range(T_c, N):
                new_a[i], new_ix[i] = -math.inf, -1
            a, ix = new_a, new_ix
            j //= 2
        k *= 2
    return ix


@pytest.mark.parametrize("T_c", [1, 2, 5, 8, 20, 64, 100, 128, 333])
def test_prop_budgets_properties(T_c):
    rng = np.random.default_rng(T_c)
    m = rng.normal(0, 3, T_c).astype(np.float32)
    ell = rng.uniform(1, 256, T_c).astype(np.float32)
    for S in (1, 7, T_c, 4 * T_c + 3, 1000):
        res = oracle.prop_budgets(m, ell, S, SEED, h=3)
        St = res["S_tiles"]
        assert res["m_star"] == m.max()
        # float64 view of the split: every tile gets floor(q_t) or floor(q_t)+1
        W = np.exp(m.astype(np.float64) - m.max()) * ell
        qt = S * W / W.sum()
        assert ((St >= np.floor(qt - 1e-4)) & (St <= np.floor(qt + 1e-4) + 1)).all()
        assert St.sum() <= S
        # the network is a true sort when T_c is a power of two: the +1 go to
        # the largest jittered remainders, and the budgets add up to S
        if T_c & (T_c - 1) == 0:
            assert St.sum() == S
            base = np.floor(qt).astype(np.int64)
            plus = np.nonzero(St - base == 1)[0]
            fr = qt - base + 1e-7 * oracle.u01_array(SEED, np.full(T_c, 3, np.int32), np.arange(T_c, dtype=np.int32))
            order = np.argsort(-fr, kind="stable")
            gap = np.sort(fr)[::-1]
            rem = len(plus)
            if 0 < rem < T_c and gap[rem - 1] - gap[rem] > 1e-5:
                assert set(plus.tolist()) == set(order[:rem].tolist())
        # which tiles may receive +1: the model of the padded network
        fr32 = []
        for t in range(T_c):
            q32 = np.float32(S) * (np.float32(W[t] / W.sum()))
            fr32.append(float(q32 - np.floor(q32)))
        ix = _bitonic_model(fr32, T_c)
        rem = S - int(np.floor(qt).sum())
        allowed = {i for i in ix[:max(0, min(rem + 1, T_c))] if i >= 0}
        plus = set(np.nonzero(St > np.floor(qt + 1e-4))[0].tolist())
        assert plus <= allowed | set(np.nonzero(np.abs(qt - np.round(qt)) < 1e-4)[0].tolist())
        inv_ok = np.where(St > 0, St / ell.astype(np.float64), 0.0)
        assert np.allclose(res["invdelta"], inv_ok, rtol=1e-6)
        assert np.array_equal(res["a0"], oracle.u01_array(SEED, np.full(T_c, 3, np.int32), np.arange(T_c, dtype=np.int32)))


def test_prop_budgets_uniform_and_degenerate():
    T_c = 12
    m = np.zeros(T_c, np.float32)
    ell = np.full(T_c, 256.0, np.float32)
    assert (oracle.prop_budgets(m, ell, 36, SEED, 0)["S_tiles"] == 3).all()
    zero = oracle.prop_budgets(m, ell, 0, SEED, 0)
    assert (zero["S_tiles"] == 0).all() and (zero["invdelta"] == 0).all()
    dead = oracle.prop_budgets(m, np.zeros(T_c, np.float32), 36, SEED, 0)
    assert (dead["S_tiles"] == 0).all()


def test_prop_vec_pass1_equals_flash_tile_statistics():
    """The vec pass 1 runs the flash tile arithmetic (prop/santa_cuda_kernel.cu
    :278-441 vs flash/santa_cuda_kernel.cu:161-273)."""
    q, K, V = gen_qkv(1, 32, 8, 3000, seed=SEED + 1, single=True)
    p = oracle.prop_decode(q, K, V, 50, seed=SEED, block_n=256, pass1_mode=0, debug=True)
    f = oracle.flash_decode(q, K, V, 50, seed=SEED, block_n=256, debug=True)
    assert np.array_equal(p["m_tiles"].view(np.uint32), f["m_tiles"].view(np.uint32))
    assert np.array_equal(p["ell_tiles"].view(np.uint32), f["ell_tiles"].view(np.uint32))


def test_prop_general_pass1_bruteforce():
    """General path: scores from q rounded to bf16 after scaling, checked in
    float64; ell from the 16-row slabs."""
    q, K, V = gen_qkv(1, 64, 8, 700, seed=SEED + 2, single=True)
    p = oracle.prop_decode(q, K, V, 30, seed=SEED, block_n=64, pass1_mode=1, debug=True)
    scale = np.float32(1.0) / np.sqrt(np.float32(128))
    qr = torch.from_numpy(q.float().numpy() * scale).to(torch.bfloat16).double().numpy()
    Kf = K.double().numpy()
    s = np.einsum("hd,lhd->hl", qr, np.repeat(Kf, 8, axis=1))
    for t in range(p["T_c"]):
        st = s[:, t * 64:(t + 1) * 64]
        assert np.allclose(p["m_tiles"][:, t], st.max(axis=1), rtol=1e-5, atol=1e-5)
        ell64 = np.exp(st - p["m_tiles"][:, t, None].astype(np.float64)).sum(axis=1)
        assert np.allclose(p["ell_tiles"][:, t], ell64, rtol=2e-5)


def test_prop_output_given_counts_and_convergence():
    q, K, V = gen_qkv(1, 32, 8, 2000, seed=SEED + 4, single=True, lowrank=0.5)
    S = 80
    p = oracle.prop_decode(q, K, V, S, seed=SEED, debug=True)
    L = 2000
    cnt = p["counts"].reshape(32, -1)[:, :L].astype(np.float64)
    Vf = V.double().numpy()
    y = np.stack([cnt[h] @ Vf[:, h // 4] for h in range(32)]) / S
    assert np.allclose(p["out"], y, rtol=1e-4, atol=2e-5)
    assert (p["S_tiles"].sum(axis=1) == S).all()
    # a budget far above L makes every tile's share near-exact (kept below
    # the per-row count ceiling of 32767)
    big = oracle.prop_decode(q, K, V, 200_000, seed=SEED, block_n=256)
    assert oracle.prop_decode(q, K, V, 200_000, seed=SEED, block_n=256, debug=True)["counts"].max() < 32767
    exact = _exact_attention(q[None], K[None], V[None])[0]
    ok, mabs, mrel = tol_check(big["out"], exact, max_abs=2e-2, mean_rel=5e-3)
    assert ok, (mabs, mrel)


# ---------------------------------------------------- prop: general shapes
def _general_case(H, KVH, D, L, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(H, D, generator=g).bfloat16()
    K = torch.randn(L, KVH, D, generator=g).bfloat16()
    V = torch.randn(L, KVH, D, generator=g).bfloat16()
    return q, K, V


@pytest.mark.parametrize("H,KVH,D,BN,L", [
    (8, 8, 128, 48, 500),     # GH 1, the vec score association (D = 128)
    (8, 4, 64, 16, 300),      # GH 2
    (32, 2, 80, 512, 1100),   # GH 16, block_n 512
    (6, 2, 256, 128, 600),    # GH 3, D 256
    (32, 8, 48, 256, 800),    # GH 4, D 48
])
def test_prop_general_shapes_bruteforce(H, KVH, D, BN, L):
    """The general pass 1 on shapes outside D = 128 / GH 4, 8 / block_n 32, 64,
    256: tile max and mass against float64 scores of q rounded to bf16 after
    scaling by 1/sqrt(D); the stash against exp(s - m_t) to bf16 rounding;
    the counts sum per tile to the systematic sampler's total, sampled rows
    are where the counts are, and the output is the float64 estimator given
    the counts."""
    q, K, V = _general_case(H, KVH, D, L, SEED + D + H)
    GH = H // KVH
    S = 3 * (L // 16)
    p = oracle.prop_decode(q, K, V, S, seed=SEED, block_n=BN, pass1_mode=1, debug=True)
    assert p["T_c"] == (L + BN - 1) // BN
    scale = np.float32(1.0) / np.sqrt(np.float32(D))
    qr = torch.from_numpy(q.float().numpy() * scale).to(torch.bfloat16).double().numpy()
    s = np.einsum("hd,lhd->hl", qr, np.repeat(K.double().numpy(), GH, axis=1))
    u16 = h16_to_f32(p["u_stash"]).astype(np.float64)  # [L, H]
    for t in range(p["T_c"]):
        st = s[:, t * BN:(t + 1) * BN]
        assert np.allclose(p["m_tiles"][:, t], st.max(axis=1), rtol=1e-5, atol=1e-5)
        e = np.exp(st - p["m_tiles"][:, t, None].astype(np.float64))
        assert np.allclose(p["ell_tiles"][:, t], e.sum(axis=1), rtol=2e-5)
        assert np.allclose(u16[t * BN:(t + 1) * BN].T, e, rtol=2 ** -8, atol=1e-6)
    assert (p["S_tiles"].sum(axis=1) == S).all()
    cnt = p["counts"].reshape(H, -1)[:, :L].astype(np.float64)
    # per tile: sum of counts = floor(a0 + X) - floor(a0), X ~ S_t (float32 sums)
    for t in range(p["T_c"]):
        tot = cnt[:, t * BN:(t + 1) * BN].sum(axis=1)
        assert (np.abs(tot - p["S_tiles"][:, t]) <= 1).all()
    rows = (cnt.reshape(KVH, GH, L) > 0).any(axis=1)
    assert np.array_equal(p["vrows"], rows.sum(axis=1))
    y = np.stack([cnt[h] @ V.double().numpy()[:, h // GH] for h in range(H)]) / S
    assert np.allclose(p["out"], y, rtol=1e-4, atol=2e-5)


def test_prop_general_score_exact_on_integer_inputs():
    """D = 48 with small-integer K and q' a power of two times small integers:
    every fma of the chain is exact, so the tile max equals the exact integer
    dot product scaled -- whatever the association (a dropped or repeated term
    would not)."""
    H, KVH, D, L = 4, 2, 48, 40
    rng = np.random.default_rng(7)
    qi = rng.integers(-3, 4, (H, D))
    ki = rng.integers(-3, 4, (L, KVH, D))
    # q' = bf16(q * 1/sqrt(48)); pick q so that q' is exactly qi / 8: q = qi/8 * sqrt(48)
    scale = np.float32(1.0) / np.sqrt(np.float32(D))
    qf = (qi / 8.0 / float(scale)).astype(np.float32)
    q = torch.from_numpy(qf).bfloat16()
    qr = torch.from_numpy(q.float().numpy() * scale).to(torch.bfloat16).float().numpy()
    K = torch.from_numpy(ki.astype(np.float32)).bfloat16()
    p = oracle.prop_decode(q, K, K, 10, seed=SEED, block_n=16, pass1_mode=1, debug=True)
    # the exact dot products of the rounded q' (small dyadic numbers: exact in float32)
    s = np.einsum("hd,lhd->hl", qr.astype(np.float64), np.repeat(ki.astype(np.float64), H // KVH, axis=1))
    for t in range(p["T_c"]):
        assert np.array_equal(p["m_tiles"][:, t].astype(np.float64), s[:, t * 16:(t + 1) * 16].max(axis=1))


@pytest.mark.parametrize("T_c", [4100, 8192])
def test_prop_budgets_beyond_4096_tiles(T_c):
    """More tiles than the register network holds: the same invariants (every
    tile floor(q_t) or floor(q_t) + 1, the budgets add up to S when T_c is a
    power of two, the +1 on the largest jittered remainders) and, for one
    budget, the brute-force model of the padded network."""
    rng = np.random.default_rng(T_c)
    m = rng.normal(0, 3, T_c).astype(np.float32)
    ell = rng.uniform(1, 256, T_c).astype(np.float32)
    W = np.exp(m.astype(np.float64) - m.max()) * ell
    for S in (T_c // 3, 5 * T_c + 17):
        res = oracle.prop_budgets(m, ell, S, SEED, h=5)
        St = res["S_tiles"]
        qt = S * W / W.sum()
        assert ((St >= np.floor(qt - 1e-4)) & (St <= np.floor(qt + 1e-4) + 1)).all()
        assert St.sum() <= S
        if T_c & (T_c - 1) == 0:
            assert St.sum() == S
    S = T_c // 3
    res = oracle.prop_budgets(m, ell, S, SEED, h=5)
    fr32 = []
    for t in range(T_c):
        q32 = np.float32(S) * np.float32(W[t] / W.sum())
        fr32.append(float(q32 - np.floor(q32)))
    ix = _bitonic_model(fr32, T_c)
    rem = S - int(np.floor(S * W / W.sum()).sum())
    allowed = {i for i in ix[:max(0, min(rem + 1, T_c))] if i >= 0}
    plus = set(np.nonzero(res["S_tiles"] > np.floor(S * W / W.sum() + 1e-4))[0].tolist())
    assert plus <= allowed | set(np.nonzero(np.abs(S * W / W.sum() - np.round(S * W / W.sum())) < 1e-4)[0].tolist())


def test_prop_general_shape_converges_to_exact_attention():
    H, KVH, D, L = 8, 4, 64, 600
    q, K, V = _general_case(H, KVH, D, L, SEED + 99)
    big = oracle.prop_decode(q, K, V, 200_000, seed=SEED, block_n=48, pass1_mode=1)
    qf = q.double().numpy() / math.sqrt(D)
    s = np.einsum("hd,lhd->hl", qf, np.repeat(K.double().numpy(), H // KVH, axis=1))
    w = np.exp(s - s.max(axis=1, keepdims=True))
    w /= w.sum(axis=1, keepdims=True)
    exact = np.einsum("hl,lhd->hd", w, np.repeat(V.double().numpy(), H // KVH, axis=1))
    ok, mabs, mrel = tol_check(big["out"], exact, max_abs=2e-2, mean_rel=1e-2)
    assert ok, (mabs, mrel)
