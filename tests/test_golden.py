"""Committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the pinned CPU oracle).

CPU: the inputs regenerate to the recorded digest and the oracle still
reproduces every fixture bit for bit (a regression pin on the oracle).
GPU: the HIP path reproduces the fixtures' tile statistics, m* and every
sampled (head, tile, row, count) bit for bit, and the output within the
bf16 tolerance (bit for bit through the reference-order merge)."""
import glob
import json
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden  # noqa: E402
from helpers import bits16, h16_to_f32, tensor_digest, tol_check  # noqa: E402

FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    d["spec"] = json.loads(str(d["spec"]))
    return d


def test_fixture_set_is_complete():
    names = {os.path.basename(p)[:-4] for p in FIXTURES}
    assert names == set(make_golden.CASES)


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p))
def test_oracle_reproduces_fixture(path):
    fx = _load(path)
    spec = fx["spec"]
    q, K, V = make_golden.inputs(spec)
    assert tensor_digest(q, K, V) == str(fx["digest"]), "input generator drifted"
    got = make_golden.compute(spec)
    for k in ("m_star", "m_tiles", "ell_tiles", "samples", "out16") + (("S_tiles",) if spec["kind"] == "prop" else ()):
        assert np.array_equal(got[k], fx[k]), k


def _samples(counts):
    nz = np.argwhere(counts > 0)
    return np.concatenate([nz, counts[tuple(nz.T)][:, None]], axis=1).astype(np.int32)


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p))
def test_gpu_reproduces_fixture(path, monkeypatch):
    fx = _load(path)
    spec = fx["spec"]
    print(f"\n[case] golden {os.path.basename(path)} {spec}", flush=True)
    q, K, V = make_golden.inputs(spec)
    dev = torch.device("cuda:0")
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    if spec["kind"] == "flash":
        import santa_flash_batch_cuda as m

        kw = dict(seed=spec["seed"], block_n=spec["block_n"], valid_len=spec["valid_len"])
        mt, lt, cnt, _, _ = m._debug_tiles(qd, Kd, Vd, spec["S"], **kw)
        out_r, _, _ = m._decode_reference_order(qd, Kd, Vd, spec["S"], **kw)
        out, ms, _ = m.decode_systematic_batched(qd, Kd, Vd, spec["S"], **kw)
        c = cnt.cpu().numpy()
        B, H, T_c, BN = c.shape
        samples = _samples(c.reshape(B * H, T_c, BN))
        assert np.array_equal(bits16(out_r), fx["out16"])
    else:
        import santa_prop_batch_cuda as m

        monkeypatch.delenv("SANTA_PASS1", raising=False)
        mt, lt, ms, St, _, _, _, cnt, _, _ = m._debug_pass(qd, Kd, Vd, spec["S"], seed=spec["seed"],
                                                           block_n=spec["block_n"])
        out, _, _ = m.decode_systematic_scalar(qd, Kd, Vd, spec["S"], seed=spec["seed"], block_n=spec["block_n"])
        samples = _samples(cnt.cpu().numpy())
        assert np.array_equal(St.cpu().numpy(), fx["S_tiles"])
    torch.cuda.synchronize()
    assert np.array_equal(mt.cpu().numpy().view(np.uint32), fx["m_tiles"])
    assert np.array_equal(lt.cpu().numpy().view(np.uint32), fx["ell_tiles"])
    assert np.array_equal(ms.cpu().numpy().view(np.uint32), fx["m_star"])
    assert np.array_equal(samples, fx["samples"])
    ok, mabs, mrel = tol_check(h16_to_f32(bits16(out)), h16_to_f32(fx["out16"]))
    assert ok, (mabs, mrel)
