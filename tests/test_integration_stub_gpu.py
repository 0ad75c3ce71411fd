"""The ctypes binding of santa_flash_decode that the repository's integration
notes give a maintainer runs as written and gives the extension module's
results.

The test reads the stub's code block from the notes themselves (the one
python block that loads the library with ctypes and calls
santa_flash_decode), so the document and the tested code cannot drift apart,
executes it from the repository root (its library path is relative), and
compares its decode_systematic_batched with santa_flash_batch_cuda's on the
same inputs: out, m* and vrows bit-identical (the same launches through the
C ABI).
"""
import os
import re

import numpy as np
import pytest
import torch

from helpers import SEED, bits16, gen_qkv

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _stub_source():
    with open(os.path.join(REPO, "INTEGRATION.md")) as f:
        text = f.read()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    stubs = [b for b in blocks if "ctypes.CDLL" in b and "santa_flash_decode" in b]
    assert len(stubs) == 1, "the integration notes must hold exactly one ctypes stub of santa_flash_decode"
    return stubs[0]


@pytest.mark.parametrize("B,L,S,valid_len", [(2, 5000, 256, -1), (8, 32768, 256, -1), (3, 4096, 100, 3001)])
def test_ctypes_stub_matches_extension(B, L, S, valid_len, monkeypatch):
    import santa_flash_batch_cuda as flash

    print(f"\n[case] integration-notes ctypes stub B={B} L={L} S={S} valid_len={valid_len}", flush=True)
    monkeypatch.chdir(REPO)
    ns = {}
    exec(compile(_stub_source(), "INTEGRATION.md", "exec"), ns)
    q, K, V = gen_qkv(B, 32, 8, L, seed=SEED + L, lowrank=0.5)
    dev = torch.device("cuda:0")
    qd, Kd, Vd = q.to(dev), K.to(dev), V.to(dev)
    got = ns["decode_systematic_batched"](qd, Kd, Vd, S, seed=SEED, want_vrows=True, valid_len=valid_len)
    ref = flash.decode_systematic_batched(qd, Kd, Vd, S, seed=SEED, want_vrows=True, valid_len=valid_len)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(got[0]), bits16(ref[0]), err_msg="out")
    np.testing.assert_array_equal(got[1].cpu().numpy().view(np.uint32), ref[1].cpu().numpy().view(np.uint32),
                                  err_msg="m_star")
    np.testing.assert_array_equal(got[2].cpu().numpy(), ref[2].cpu().numpy(), err_msg="vrows")
    with pytest.raises(RuntimeError, match="block_n must be 0"):
        ns["decode_systematic_batched"](qd, Kd, Vd, S, block_n=100)
