"""santa_flash_decode_noalloc (the entry point that allocates nothing) gives
santa_flash_decode's results, called through the C ABI.

The allocation-free entry point keeps its workspace in a static device array
that every call on the device shares.  Two calls in a row, the second on a
smaller input, must each match santa_flash_decode with a caller workspace
bit for bit (out, m*, vrows): same kernels, same plan.  The array keeps the
first call's contents, so the second call also shows that nothing it reads
depends on what an earlier call left there.  (The rejection of shapes beyond
the array's 16 MiB is checked on the CPU, tests/test_library.py.)
"""
import ctypes
import os

import numpy as np
import pytest
import torch

from helpers import SEED, bits16, gen_qkv

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
P, I, U64, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_size_t


def _lib():
    import santa_flash_batch_cuda  # noqa: F401  (torch's HIP runtime first)

    lib = ctypes.CDLL(os.path.join(REPO, "santa_amd", "libsanta_amd.so"))
    lib.santa_last_error.restype = ctypes.c_char_p
    lib.santa_flash_workspace_size.restype = SZ
    lib.santa_flash_workspace_size.argtypes = [I] * 5
    lib.santa_flash_plan.argtypes = [ctypes.c_int64] * 4 + [ctypes.POINTER(I)] * 4
    lib.santa_flash_decode.argtypes = [P, P, P] + [I] * 9 + [U64, P, P, P, P, SZ, P]
    lib.santa_flash_decode_noalloc.argtypes = [P, P, P] + [I] * 9 + [U64, P, P, P, P]
    return lib


def _decode(lib, q, K, V, S, valid_len, noalloc):
    B, H, D = q.shape
    L_st, KVH = K.shape[1], K.shape[2]
    L, bn, T_c, spt = (I() for _ in range(4))
    assert lib.santa_flash_plan(L_st, valid_len, 0, S, *(ctypes.byref(x) for x in (L, bn, T_c, spt))) == 0
    out = torch.empty_like(q)
    m_star = torch.empty(B, H, device=q.device)
    vrows = torch.empty(B, KVH, dtype=torch.int32, device=q.device)
    stream = torch.cuda.current_stream().cuda_stream
    args = (q.data_ptr(), K.data_ptr(), V.data_ptr(), 0 if q.dtype == torch.bfloat16 else 1, B, H, KVH, D, L.value,
            L_st, bn.value, spt.value, SEED, out.data_ptr(), m_star.data_ptr(), vrows.data_ptr())
    if noalloc:
        rc = lib.santa_flash_decode_noalloc(*args, stream)
    else:
        n = lib.santa_flash_workspace_size(B, H, KVH, D, T_c.value)
        ws = torch.empty(n, dtype=torch.uint8, device=q.device)
        rc = lib.santa_flash_decode(*args, ws.data_ptr(), n, stream)
    assert rc == 0, lib.santa_last_error().decode()
    return out, m_star, vrows


@pytest.mark.parametrize("first,second", [
    ((8, 32, 32768, 256, -1), (2, 32, 5000, 256, -1)),    # headline shape, then a smaller GH 4 call
    ((4, 64, 20000, 512, -1), (1, 64, 3000, 300, 2900)),  # GH 8, then a smaller one with valid_len
])
def test_noalloc_matches_decode(first, second):
    lib = _lib()
    dev = torch.device("cuda:0")
    for i, (B, H, L, S, vl) in enumerate((first, second)):
        print(f"\n[case] santa_flash_decode_noalloc call {i + 1}: B={B} H={H} KVH=8 L={L} S={S} valid_len={vl}",
              flush=True)
        q, K, V = gen_qkv(B, H, 8, L, seed=SEED + 3 * L + H, lowrank=0.5)
        qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
        got = _decode(lib, qd, Kd, Vd, S, vl, noalloc=True)
        ref = _decode(lib, qd, Kd, Vd, S, vl, noalloc=False)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits16(got[0]), bits16(ref[0]), err_msg=f"call {i + 1}: out")
        np.testing.assert_array_equal(got[1].cpu().numpy().view(np.uint32), ref[1].cpu().numpy().view(np.uint32),
                                      err_msg=f"call {i + 1}: m_star")
        np.testing.assert_array_equal(got[2].cpu().numpy(), ref[2].cpu().numpy(), err_msg=f"call {i + 1}: vrows")
        assert torch.isfinite(got[0].float()).all()


def test_noalloc_under_graph_capture():
    """A santa_flash_decode_noalloc call captured into a HIP graph (after one
    uncaptured call on the device, which takes the scratch array's address)
    replays with santa_flash_decode's results: three replays, with eager
    calls on other inputs between them (which leave other contents in the
    shared scratch), each bit-equal to the direct call."""
    lib = _lib()
    dev = torch.device("cuda:0")
    B, H, L, S = 4, 32, 16384, 256
    print(f"\n[case] santa_flash_decode_noalloc under graph capture: B={B} H={H} KVH=8 L={L} S={S}", flush=True)
    q, K, V = gen_qkv(B, H, 8, L, seed=SEED + 77, lowrank=0.5)
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    ref = _decode(lib, qd, Kd, Vd, S, -1, noalloc=False)
    _decode(lib, qd, Kd, Vd, S, -1, noalloc=True)  # the uncaptured first call on the device
    torch.cuda.synchronize()
    L_, bn, T_c, spt = (I() for _ in range(4))
    assert lib.santa_flash_plan(L, -1, 0, S, *(ctypes.byref(x) for x in (L_, bn, T_c, spt))) == 0
    out = torch.empty_like(qd)
    m_star = torch.empty(B, H, device=dev)
    vrows = torch.empty(B, 8, dtype=torch.int32, device=dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = lib.santa_flash_decode_noalloc(qd.data_ptr(), Kd.data_ptr(), Vd.data_ptr(), 0, B, H, 8, 128, L_.value, L,
                                            bn.value, spt.value, SEED, out.data_ptr(), m_star.data_ptr(),
                                            vrows.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.santa_last_error().decode()
    q2, K2, V2 = gen_qkv(2, H, 8, 5000, seed=SEED + 78, lowrank=0.5)
    q2, K2, V2 = q2.to(dev), K2.to(dev), V2.to(dev)
    for rep in range(3):
        out.zero_()
        m_star.zero_()
        vrows.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits16(out), bits16(ref[0]), err_msg=f"replay {rep}: out")
        np.testing.assert_array_equal(m_star.cpu().numpy().view(np.uint32), ref[1].cpu().numpy().view(np.uint32),
                                      err_msg=f"replay {rep}: m_star")
        np.testing.assert_array_equal(vrows.cpu().numpy(), ref[2].cpu().numpy(), err_msg=f"replay {rep}: vrows")
        _decode(lib, q2, K2, V2, 200, -1, noalloc=True)  # eager work between replays
        torch.cuda.synchronize()
