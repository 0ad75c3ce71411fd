"""Host logic of the backend adapters (santa_amd/attention_backends.py) on
the CPU, with stand-in extension modules that record their calls: module
lookup order, the batched call, the message-driven per-sequence fallback,
actual_mode, info() keys and the factory's names and error policy
(tutorial_code/attention_backends.py:420-621).  The SDPA comparator runs on
the CPU in float32 against a float64 softmax-attention restatement."""
import sys
import types

import numpy as np
import pytest
import torch

from santa_amd import attention_backends as ab

INFO_KEYS = {"backend", "paper_role", "exact_attention", "supports_true_batch_decode", "module", "requested_S",
             "seed", "block_n", "actual_mode"}


def _fake_module(name, batched=True, batch_error=None):
    mod = types.ModuleType(name)
    mod.calls = []

    def decode(q, K, V, S, seed=42, block_n=0, want_vrows=False, **kw):
        mod.calls.append({"q": tuple(q.shape), "K": tuple(K.shape), "S": S, "seed": seed, "block_n": block_n,
                          "want_vrows": want_vrows, **kw})
        if q.dim() == 3 and batch_error is not None:
            raise RuntimeError(batch_error)
        if "valid_len" in kw and not batched:
            raise TypeError("decode_systematic_scalar(): incompatible function arguments ... valid_len=5")
        out = q.float().sum(dim=-1, keepdim=True).expand_as(q).to(q.dtype) + K.shape[-3]
        return out, torch.zeros(q.shape[:-1]), torch.zeros(0, dtype=torch.int32)

    mod.decode_systematic_scalar = decode
    if batched:
        mod.decode_systematic_batched = decode
    return mod


@pytest.fixture
def fake_modules(monkeypatch):
    flash = _fake_module("santa_flash_batch_cuda", batched=True)
    prop = _fake_module("santa_prop_batch_cuda", batched=False)
    monkeypatch.setitem(sys.modules, "santa_flash_batch_cuda", flash)
    monkeypatch.setitem(sys.modules, "santa_prop_batch_cuda", prop)
    return flash, prop


def _inputs(B=3, H=8, KVH=2, T=40, D=16, dtype=torch.float32):
    g = torch.Generator().manual_seed(0)
    return (torch.randn(B, H, D, generator=g).to(dtype), torch.randn(B, T, KVH, D, generator=g).to(dtype),
            torch.randn(B, T, KVH, D, generator=g).to(dtype))


def test_flash_backend_batched_call(fake_modules):
    flash, _ = fake_modules
    be = ab.SantaFlashBackend(S=256, seed=1690, block_n=None)
    assert be.supports_true_batch_decode and be.module_name == "santa_flash_batch_cuda"
    assert be.info()["actual_mode"] == "unknown"
    q, K, V = _inputs()
    out = be.decode(q, K, V, 30)
    assert out.shape == q.shape and out.is_contiguous()
    assert len(flash.calls) == 1
    c = flash.calls[0]
    assert c["valid_len"] == 30 and c["seed"] == 1690 and c["S"] == 256 and c["want_vrows"] is False
    assert c["block_n"] == 0  # block_n=None is not passed: the module default applies
    info = be.info()
    assert set(info) == INFO_KEYS and info["actual_mode"] == "batch" and info["requested_S"] == 256


def test_block_n_is_forwarded(fake_modules):
    flash, _ = fake_modules
    be = ab.SantaFlashBackend(S=8, seed=1, block_n=64)
    q, K, V = _inputs()
    be.decode(q, K, V, 40)
    assert flash.calls[-1]["block_n"] == 64


def test_prop_backend_falls_back_per_sequence(fake_modules):
    _, prop = fake_modules
    be = ab.SantaPropBackend(S=32, seed=7, block_n=None)
    assert not be.supports_true_batch_decode
    q, K, V = _inputs(B=3, T=40)
    out = be.decode(q, K, V, 25)
    assert be.actual_mode == "single_loop_fallback"
    # the first call carried valid_len and failed; then one call per sequence on K[b, :valid_len]
    assert len(prop.calls) == 1 + 3
    for c in prop.calls[1:]:
        assert c["q"] == (8, 16) and c["K"] == (25, 2, 16) and "valid_len" not in c
    assert out.shape == q.shape
    assert torch.allclose(out[:, 0, 0], q.float().sum(-1)[:, 0] + 25)


@pytest.mark.parametrize("msg", ["Expected q_h [H,D]", "Expected q_h [H, D]", "bad ranks",
                                 "Single-request shape mismatch", "valid_len is not supported"])
def test_fallback_markers(monkeypatch, msg):
    mod = _fake_module("santa_flash_batch_cuda", batched=True, batch_error=msg)
    monkeypatch.setitem(sys.modules, "santa_flash_batch_cuda", mod)
    be = ab.SantaFlashBackend(S=4, seed=0, block_n=None)
    q, K, V = _inputs(B=2)
    be.decode(q, K, V, 10)
    assert be.actual_mode == "single_loop_fallback"


def test_other_errors_propagate(monkeypatch):
    mod = _fake_module("santa_flash_batch_cuda", batched=True, batch_error="HIP error: out of memory")
    monkeypatch.setitem(sys.modules, "santa_flash_batch_cuda", mod)
    be = ab.SantaFlashBackend(S=4, seed=0, block_n=None)
    q, K, V = _inputs(B=2)
    with pytest.raises(RuntimeError, match="out of memory"):
        be.decode(q, K, V, 10)
    assert be.actual_mode == "unknown"


def test_module_candidates_and_import_failure(monkeypatch):
    monkeypatch.setitem(sys.modules, "santa_flash_batch_cuda", None)  # import raises
    alt = _fake_module("santa_cuda", batched=False)
    monkeypatch.setitem(sys.modules, "santa_cuda", alt)
    be = ab.SantaFlashBackend(S=4, seed=0, block_n=None)
    assert be.module_name == "santa_cuda"
    monkeypatch.setitem(sys.modules, "santa_prop_batch_cuda", None)
    with pytest.raises(ab.BackendError, match="Could not import any santa_prop extension module") as ei:
        ab.SantaPropBackend(S=4, seed=0, block_n=None)
    assert "santa_prop_batch_cuda" in ei.value.details


def test_factory_names_and_policy(fake_modules):
    kw = dict(santa_s=16, santa_seed=3, santa_block_n=None, flashinfer_mode="auto", flashinfer_use_tensor_cores=False)
    bes = ab.build_backends(["SDPA", " santa ", "santa_flash", "santa_prop"], **kw)
    assert [type(b).__name__ for b in bes] == ["SDPABackend", "SantaFlashBackend", "SantaFlashBackend",
                                               "SantaPropBackend"]
    with pytest.raises(ValueError, match="Unsupported backend name"):
        ab.build_backends(["nope"], **kw)
    with pytest.raises(ab.BackendError):
        ab.build_backends(["fa2"], **kw)
    got, errors = ab.build_backends(["fa2", "flashinfer", "sdpa", "bogus"], skip_init_failures=True, **kw)
    assert [type(b).__name__ for b in got] == ["SDPABackend"]
    assert [e["backend"] for e in errors] == ["fa2", "flashinfer", "bogus"]
    assert errors[2]["error_type"] == "ValueError"
    got, errors = ab.build_backends(["sdpa"], skip_init_failures=False, **kw)
    assert len(got) == 1 and errors == []


def test_sdpa_backend_matches_float64_attention():
    q, K, V = _inputs(B=2, H=8, KVH=2, T=50, D=16)
    be = ab.SDPABackend()
    out = be.decode(q, K, V, 37)
    qd, Kd, Vd = q.double().numpy(), K.double().numpy()[:, :37], V.double().numpy()[:, :37]
    ref = np.empty(qd.shape)
    for b in range(2):
        for h in range(8):
            s = Kd[b, :, h // 4] @ qd[b, h] / np.sqrt(16)
            p = np.exp(s - s.max())
            ref[b, h] = (p / p.sum()) @ Vd[b, :, h // 4]
    assert np.allclose(out.numpy(), ref, atol=1e-5)
    rep = be.smoke_test(device=torch.device("cpu"), dtype=torch.float32, num_heads=8, num_kv_heads=2, head_dim=16,
                        valid_len=12)
    assert rep["output_shape"] == [2, 8, 16] and rep["exact_attention"] is True
