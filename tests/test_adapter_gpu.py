"""The backend adapters on the real extension modules (MI355X).

* SantaFlashBackend takes the batched path and returns exactly the module's
  output; with a budget of 64 x block_n samples per tile it agrees with
  exact softmax attention (float64 on the CPU) to the bf16 tolerance.
* SantaPropBackend takes the prop module's batched entry (an addition over
  the reference, whose prop module has none) and each sequence agrees with a
  direct per-sequence call on K[b, :valid_len] to the bf16 tolerance.
"""
import numpy as np
import pytest
import torch

from helpers import SEED, bits16, gen_qkv, tol_check
from santa_amd import attention_backends as ab

pytestmark = pytest.mark.gpu


def _exact64(q, K, V, valid_len):
    qd = q.double().cpu().numpy()
    Kd = K.double().cpu().numpy()[:, :valid_len]
    Vd = V.double().cpu().numpy()[:, :valid_len]
    B, H, D = qd.shape
    GH = H // Kd.shape[2]
    out = np.empty((B, H, D))
    for b in range(B):
        for h in range(H):
            s = Kd[b, :, h // GH] @ qd[b, h] / np.sqrt(D)
            p = np.exp(s - s.max())
            out[b, h] = (p / p.sum()) @ Vd[b, :, h // GH]
    return out


def test_flash_backend_batched_and_exact_limit():
    print("\n[case] adapter santa_flash B=3 L=3000 valid_len=2500", flush=True)
    import santa_flash_batch_cuda as flash

    dev = torch.device("cuda:0")
    q, K, V = gen_qkv(3, 32, 8, 3000, seed=SEED + 21)
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    be = ab.build_backends(["santa_flash"], santa_s=64, santa_seed=SEED, santa_block_n=None, flashinfer_mode="auto",
                           flashinfer_use_tensor_cores=False)[0]
    out = be.decode(qd, Kd, Vd, 2500)
    ref, _, _ = flash.decode_systematic_batched(qd, Kd, Vd, 64, seed=SEED, valid_len=2500)
    torch.cuda.synchronize()
    assert be.info()["actual_mode"] == "batch" and be.supports_true_batch_decode
    assert np.array_equal(bits16(out), bits16(ref))
    big = ab.SantaFlashBackend(S=64 * 256 * 10, seed=SEED, block_n=256)
    out = big.decode(qd, Kd, Vd, 2500)
    torch.cuda.synchronize()
    ok, mabs, mrel = tol_check(out.float().cpu().numpy(), _exact64(q, K, V, 2500), max_abs=2e-2, mean_rel=5e-3)
    assert ok, (mabs, mrel)


def test_prop_backend_batched(monkeypatch):
    print("\n[case] adapter santa_prop B=2 L=4096 valid_len=3000", flush=True)
    monkeypatch.delenv("SANTA_PASS1", raising=False)
    import santa_prop_batch_cuda as prop

    dev = torch.device("cuda:0")
    q, K, V = gen_qkv(2, 32, 8, 4096, seed=SEED + 22)
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    be = ab.SantaPropBackend(S=47, seed=SEED, block_n=None)
    assert be.supports_true_batch_decode
    out = be.decode(qd, Kd, Vd, 3000)
    ref_b, _, _ = prop.decode_systematic_batched(qd, Kd, Vd, 47, seed=SEED, valid_len=3000)
    torch.cuda.synchronize()
    assert be.actual_mode == "batch"
    assert np.array_equal(bits16(out), bits16(ref_b))
    for b in range(2):
        ref, _, _ = prop.decode_systematic_scalar(qd[b].contiguous(), Kd[b, :3000].contiguous(),
                                                  Vd[b, :3000].contiguous(), 47, seed=SEED)
        torch.cuda.synchronize()
        ok, mabs, mrel = tol_check(out[b].float().cpu().numpy(), ref.float().cpu().numpy())
        assert ok, (b, mabs, mrel)
