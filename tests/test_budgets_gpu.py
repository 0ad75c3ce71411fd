"""GPU parity of the santa_prop tile budgets (santa_prop_tile_budgets, C-ABI).

The budget kernel runs the reference's largest-remainder split
(prop/santa_cuda_kernel.cu:577-726): m*, W_t, Z, integer bases, jittered
remainders, the bitonic network over the next power of two with its
padding semantics (reads past T_c see (-inf, -1), writes there are dropped)
and the +1 for the top `rem`.  Its output must equal the C oracle's bit for
bit -- S_t, invdelta_t, a0_t and m* -- including where remainders tie, since
ties are resolved by the network's exact sequence of compare-exchange steps.

The tile counts cover every (waves, registers) form of the kernel: one wave
with one or two registers, 2 to 16 waves with two, 16 waves with four, and
counts just below and above powers of two.  Per count, four heads:
  0  random m_t and ell_t;
  1  every tile identical (every remainder equal before the jitter, which
     at remainders near 0.5 only moves them by a unit or two in the last
     place, so most of them tie exactly);
  2  equal m_t, ell_t from three values (three tied classes);
  3  random, with a quarter of the tiles at ell_t = 0 (zero weight).
Every case prints its name before touching the GPU.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "santa_amd", "libsanta_amd.so")
SEED = 1690


def _lib():
    if not os.path.exists(LIB):
        pytest.fail("libsanta_amd.so not built (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB)
    L.santa_last_error.restype = ctypes.c_char_p
    return L


def _inputs(T_c, seed):
    rng = np.random.default_rng(seed)
    H = 4
    m = np.empty((H, T_c), np.float32)
    ell = np.empty((H, T_c), np.float32)
    m[0] = rng.normal(0.0, 2.0, T_c)
    ell[0] = rng.uniform(1.0, 200.0, T_c)
    m[1] = 1.25
    ell[1] = 37.5
    m[2] = -0.5
    ell[2] = rng.choice(np.array([10.0, 20.0, 40.0], np.float32), T_c)
    m[3] = rng.normal(0.0, 1.0, T_c)
    ell[3] = rng.uniform(0.5, 50.0, T_c)
    ell[3][rng.random(T_c) < 0.25] = 0.0
    return m, ell


@pytest.mark.parametrize("T_c", [1, 5, 33, 64, 65, 100, 128, 129, 255, 256, 300, 482, 512, 700, 1024, 1500, 2048,
                                 3000, 4096])
@pytest.mark.parametrize("S_kind", ["many", "few"])
def test_budgets_match_oracle(T_c, S_kind):
    L = _lib()
    S = 3 * T_c + 7 if S_kind == "many" else max(1, T_c // 2)
    print(f"\n[case] tile budgets T_c={T_c} S={S} seed={SEED + T_c}", flush=True)
    m, ell = _inputs(T_c, SEED + T_c)
    H = m.shape[0]
    dev = torch.device("cuda:0")
    mt = torch.from_numpy(m).to(dev)
    lt = torch.from_numpy(ell).to(dev)
    ms = torch.empty(H, dtype=torch.float32, device=dev)
    St = torch.empty(H, T_c, dtype=torch.int32, device=dev)
    inv = torch.empty(H, T_c, dtype=torch.float32, device=dev)
    a0 = torch.empty(H, T_c, dtype=torch.float32, device=dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.santa_prop_tile_budgets(P(mt), P(lt), H, T_c, S, ctypes.c_uint64(SEED), P(ms), P(St), P(inv), P(a0),
                                   stream)
    assert rc == 0, L.santa_last_error()
    torch.cuda.synchronize()
    for h in range(H):
        ref = oracle.prop_budgets(m[h], ell[h], S, SEED, h)
        assert np.float32(ms[h].item()).view(np.uint32) == np.float32(ref["m_star"]).view(np.uint32), (T_c, h)
        np.testing.assert_array_equal(St[h].cpu().numpy(), ref["S_tiles"], err_msg=f"S_t T_c={T_c} head {h}")
        np.testing.assert_array_equal(inv[h].cpu().numpy().view(np.uint32), ref["invdelta"].view(np.uint32),
                                      err_msg=f"invdelta T_c={T_c} head {h}")
        np.testing.assert_array_equal(a0[h].cpu().numpy().view(np.uint32), ref["a0"].view(np.uint32),
                                      err_msg=f"a0 T_c={T_c} head {h}")
        assert int(St[h].sum().item()) == S, (T_c, h)
