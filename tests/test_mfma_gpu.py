"""The score path's K=1 MFMA is fmaf, bit for bit, on edge operands.

Every score the kernels compute is a chain of v_mfma_f32_4x4x1f32 with the A
operand (q, scaled) broadcast from one 4-lane block and the lane's own K
element as B -- the reference's per-virtual-lane fmaf chain
(flash/santa_cuda_kernel.cu:183-211).  The sampled indices are bit-exact only
if each such MFMA rounds exactly as one fmaf does.  N(0,1) inputs never reach
the corners, so this test drives the same instruction form (the library's
test hook runs every broadcast block J = 0..15) with signed zeros,
subnormal operands and results, the smallest normal, products that overflow,
infinities, NaN and random values over the whole exponent range, and
compares each result with fmaf on the same operands: equal bits, or NaN for
NaN (the payload is not part of IEEE-754's contract).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SPECIALS = np.array([
    0.0, -0.0, 1.0, -1.0, 0.5, 3.0,
    1e-40, -1e-40, 1.4e-45, -1.4e-45, 5.877e-39, 1.1754942e-38,  # subnormals, largest subnormal
    1.17549435e-38, -1.17549435e-38,                            # smallest normal
    1e-20, -1e-20, 3e-23, 1e20, -1e20, 3.4e38, -3.4e38,         # subnormal / overflowing products
    np.inf, -np.inf, np.nan,
], np.float32)


@np.errstate(all="ignore")
def _operands(n_waves, seed):
    rng = np.random.default_rng(seed)

    def draw(n):
        x = np.empty(n, np.float32)
        pick = rng.random(n)
        sp = pick < 0.45
        x[sp] = rng.choice(SPECIALS, sp.sum())
        wide = (pick >= 0.45) & (pick < 0.8)  # any exponent, both signs
        bits = rng.integers(0, 2 ** 32, wide.sum(), dtype=np.uint64).astype(np.uint32)
        x[wide] = bits.view(np.float32)
        rest = pick >= 0.8
        x[rest] = rng.standard_normal(rest.sum()).astype(np.float32)
        return x

    a = draw(n_waves * 64).reshape(n_waves, 64)
    b = draw(n_waves * 64).reshape(n_waves, 64)
    c = draw(n_waves * 64 * 4).reshape(n_waves, 64, 4)
    # exact cancellation: c = -(a_J,i * b_l) for a few lanes of each wave
    for w in range(n_waves):
        for l in range(0, 64, 7):
            j = int(rng.integers(0, 16))
            c[w, l, :] = -(a[w, 4 * j:4 * j + 4].astype(np.float64) * b[w, l]).astype(np.float32)
    return a, b, c


@np.errstate(all="ignore")
def test_broadcast_mfma_equals_fmaf():
    import santa_flash_batch_cuda as m

    n_waves = 96
    print(f"\n[case] broadcast v_mfma_f32_4x4x1f32 vs fmaf, {n_waves} waves x 16 blocks x 64 lanes x 4", flush=True)
    a, b, c = _operands(n_waves, 2026)
    dev = torch.device("cuda:0")
    mo, fo = m._mfma_fma_check(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), torch.from_numpy(c).to(dev))
    torch.cuda.synchronize()
    mo, fo = mo.cpu().numpy(), fo.cpu().numpy()
    # the fmaf leg against numpy's correctly rounded reference (float64 product
    # and sum round once when the float32 operands' exact result fits; checked
    # only where it does: no overflow, no NaN, and a result that is normal)
    a_bc = a.reshape(n_waves, 16, 4)[:, :, None, :]              # [w, J, 1, i]
    exact = a_bc.astype(np.float64) * b[:, None, :, None] + c[:, None, :, :]
    ref = exact.astype(np.float32)
    ok_ref = np.isfinite(exact) & (np.abs(exact) >= 2.0 ** -126) & (np.abs(exact) < 2.0 ** 100)
    assert ok_ref.sum() > 10000
    # float64 holds a float32 product exactly and its sum with c to within
    # 2^-53 relative; a double rounding differs only at exact ties, which the
    # check below tolerates by one ulp
    d_ulps = np.abs(fo.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert (d_ulps[ok_ref] <= 1).all(), "the fmaf leg is not a fused multiply-add"
    nan_m, nan_f = np.isnan(mo), np.isnan(fo)
    assert np.array_equal(nan_m, nan_f), (
        f"NaN-ness differs at {np.argwhere(nan_m != nan_f)[:5].tolist()}")
    same = mo.view(np.uint32) == fo.view(np.uint32)
    bad = ~nan_f & ~same
    if bad.any():
        idx = np.argwhere(bad)[:8]
        rows = []
        for w, j, l, i in idx:
            rows.append((float(a[w, 4 * j + i]), float(b[w, l]), float(c[w, l, i]), float(mo[w, j, l, i]),
                         float(fo[w, j, l, i])))
        raise AssertionError(f"{int(bad.sum())} MFMA results differ from fmaf (a, b, c, mfma, fmaf): {rows}")
    # the corners were exercised
    sub = (np.abs(fo) < 2.0 ** -126) & (fo != 0)
    assert sub.sum() > 100, "no subnormal results were exercised"
    assert np.isinf(fo).sum() > 100 and nan_f.sum() > 100
    assert (fo == 0).sum() > 100 and (np.signbit(fo) & (fo == 0)).sum() > 10
