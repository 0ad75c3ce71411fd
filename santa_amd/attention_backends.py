"""Decode-attention backend adapters: the drop-in counterpart of the
reference's adapter layer (tutorial_code/attention_backends.py:18-89,
420-621), with the same classes, constructor arguments, factory names,
``info()`` keys and fallback rules, so a runtime written against the
reference's adapters runs unchanged on MI355X.

Contract (tutorial_code/attention_backends.py:30,462-500):
``decode(q_bhd [B,H,D], k_nhd [B,T_storage,KVH,D], v_nhd, valid_len) ->
[B,H,D]`` contiguous, in q's dtype.  The sparse backends import their
extension module by name (``santa_flash_batch_cuda`` / ``santa_prop_batch_cuda``
here, both built from this package's HIP library) and call its batched
entry point once; if the module rejects the batched form (message mentioning
"Expected q_h [H,D]", "valid_len", "rank" or "shape") they fall back to one
call per sequence on ``k_nhd[b, :valid_len]``.  ``actual_mode`` records which
happened: ``"batch"``, ``"single_loop_fallback"`` or ``"unknown"`` before the
first call.

The exact dense comparators of the reference that have no ROCm build here
(flash-attn 2.7.4.post1, FlashInfer 0.6.6) are named by the factory but raise
``BackendError``; ``SDPABackend`` (torch scaled_dot_product_attention with
GQA) is the exact comparator on this platform.
"""
from __future__ import annotations

import importlib
from typing import Any, Dict, Iterable, List, Optional, Sequence, Tuple, Union

import torch
import torch.nn.functional as F

FA2_PAPER_TARGET_VERSION = "2.7.4.post1"
FLASHINFER_PAPER_TARGET_VERSION = "0.6.6"

# Substrings of a batched-call failure that mean "this module only takes one
# sequence": tutorial_code/attention_backends.py:477-489.
_FALLBACK_MARKERS = ("Expected q_h [H,D]", "Expected q_h [H, D]", "valid_len", "rank", "shape")


class BackendError(RuntimeError):
    """A backend could not be built or run; ``details`` carries the causes."""

    def __init__(self, message: str, *, details: Optional[str] = None) -> None:
        super().__init__(message)
        self.details = details


class DecodeAttentionBackend:
    """One attention call per layer per decode step (tutorial_code/attention_backends.py:24-67)."""

    name: str = "backend"
    paper_role: str = "auxiliary"
    exact_attention: Optional[bool] = None
    supports_true_batch_decode: Optional[bool] = None

    def decode(self, q_bhd: torch.Tensor, k_nhd: torch.Tensor, v_nhd: torch.Tensor, valid_len: int) -> torch.Tensor:
        raise NotImplementedError

    def info(self) -> Dict[str, Any]:
        return {
            "backend": self.name,
            "paper_role": self.paper_role,
            "exact_attention": self.exact_attention,
            "supports_true_batch_decode": self.supports_true_batch_decode,
        }

    def smoke_test(self, *, device: torch.device, dtype: torch.dtype, num_heads: int, num_kv_heads: int,
                   head_dim: int, valid_len: int) -> Dict[str, Any]:
        """Batch of 2 random sequences through decode(); checks the output shape."""
        batch_size = 2
        q = torch.randn(batch_size, num_heads, head_dim, device=device, dtype=dtype)
        k = torch.randn(batch_size, valid_len, num_kv_heads, head_dim, device=device, dtype=dtype)
        v = torch.randn(batch_size, valid_len, num_kv_heads, head_dim, device=device, dtype=dtype)
        out = self.decode(q, k, v, valid_len)
        expected = (batch_size, num_heads, head_dim)
        if tuple(out.shape) != expected:
            raise BackendError(
                f"Smoke test returned wrong shape for {self.name}: got {tuple(out.shape)}, expected {expected}")
        return {"backend": self.name, "batch_size": batch_size, "valid_len": int(valid_len),
                "output_shape": list(out.shape), **self.info()}


class SDPABackend(DecodeAttentionBackend):
    """Exact dense decode with torch SDPA and GQA (tutorial_code/attention_backends.py:70-89)."""

    name = "sdpa"
    paper_role = "debug_exact_reference"
    exact_attention = True
    supports_true_batch_decode = True

    def decode(self, q_bhd: torch.Tensor, k_nhd: torch.Tensor, v_nhd: torch.Tensor, valid_len: int) -> torch.Tensor:
        q = q_bhd.unsqueeze(2)                                  # [B,H,1,D]
        k = k_nhd[:, :valid_len].permute(0, 2, 1, 3)            # [B,KVH,L,D]
        v = v_nhd[:, :valid_len].permute(0, 2, 1, 3)
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=None, dropout_p=0.0, is_causal=False,
                                             enable_gqa=(q.shape[1] != k.shape[1]))
        return out[:, :, 0, :].contiguous()


class _UnavailableExactBackend(DecodeAttentionBackend):
    """A reference comparator with no ROCm build in this environment."""

    paper_role = "main_exact_dense_batched_baseline"
    exact_attention = True
    package = ""
    version = ""

    def __init__(self, **_: Any) -> None:
        raise BackendError(
            f"{self.name} ({self.package} {self.version}) is not available on ROCm in this build; "
            f"use 'sdpa' as the exact comparator")


class FA2Backend(_UnavailableExactBackend):
    name = "fa2"
    package = "flash-attn"
    version = FA2_PAPER_TARGET_VERSION


class FlashInferBackend(_UnavailableExactBackend):
    name = "flashinfer"
    package = "flashinfer-python"
    version = FLASHINFER_PAPER_TARGET_VERSION


class _SantaBaseBackend(DecodeAttentionBackend):
    """Sampled decode through an S^2ANTA extension module
    (tutorial_code/attention_backends.py:420-510)."""

    module_candidates: Sequence[str] = ()
    name = "santa"
    paper_role = "main_batched_sparse_baseline"
    exact_attention = False

    def __init__(self, *, S: int, seed: int, block_n: Optional[int]) -> None:
        self.S = int(S)
        self.seed = int(seed)
        self.block_n = None if block_n is None else int(block_n)
        self.actual_mode = "unknown"
        self.module = None
        self.module_name = None
        self.supports_true_batch_decode = False
        errors: List[str] = []
        for candidate in self.module_candidates:
            try:
                self.module = importlib.import_module(candidate)
                self.module_name = candidate
                break
            except Exception as exc:  # noqa: BLE001 -- every import failure is reported
                errors.append(f"{candidate}: {exc}")
        if self.module is None:
            raise BackendError(
                f"Could not import any {self.name} extension module. Tried: {', '.join(self.module_candidates)}.",
                details=" | ".join(errors))
        self.supports_true_batch_decode = hasattr(self.module, "decode_systematic_batched")

    @staticmethod
    def _unwrap_tensor_out(x: Any) -> torch.Tensor:
        return x[0] if isinstance(x, (tuple, list)) else x

    def _get_decode_fn(self):
        for attr in ("decode_systematic_batched", "decode_systematic_scalar"):
            if hasattr(self.module, attr):
                return getattr(self.module, attr)
        raise BackendError(f"Module {self.module_name} does not expose a decode entry point.")

    def decode(self, q_bhd: torch.Tensor, k_nhd: torch.Tensor, v_nhd: torch.Tensor, valid_len: int) -> torch.Tensor:
        fn = self._get_decode_fn()
        kwargs: Dict[str, Any] = {"seed": self.seed, "want_vrows": False, "valid_len": int(valid_len)}
        if self.block_n is not None:
            kwargs["block_n"] = int(self.block_n)
        try:
            out = fn(q_bhd.contiguous(), k_nhd, v_nhd, self.S, **kwargs)
            self.actual_mode = "batch"
            return self._unwrap_tensor_out(out).contiguous()
        except Exception as exc:  # noqa: BLE001 -- re-raised unless it is the single-sequence signal
            msg = str(exc)
            if not (q_bhd.dim() == 3 and any(m in msg for m in _FALLBACK_MARKERS)):
                raise
        kwargs.pop("valid_len", None)
        self.actual_mode = "single_loop_fallback"
        outputs = []
        for b in range(int(q_bhd.shape[0])):
            k_b = k_nhd[b, :valid_len].contiguous()
            v_b = v_nhd[b, :valid_len].contiguous()
            outputs.append(self._unwrap_tensor_out(fn(q_bhd[b].contiguous(), k_b, v_b, self.S, **kwargs)))
        return torch.stack(outputs, dim=0).contiguous()

    def decode_paged(self, q_bhd: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                     block_table: torch.Tensor, seq_lens) -> torch.Tensor:
        """Decode over a paged cache (not in the reference's adapters, whose
        caches are contiguous): k_pages / v_pages [num_pages, page_size, KVH, D],
        block_table int32 [B, pages per sequence], seq_lens an int or one
        length per sequence.  Same S, seed and block_n as decode()."""
        fn = getattr(self.module, "decode_systematic_paged", None)
        if fn is None:
            raise BackendError(f"Module {self.module_name} does not expose a paged decode entry point.")
        kwargs: Dict[str, Any] = {"seed": self.seed, "want_vrows": False}
        if self.block_n is not None:
            kwargs["block_n"] = int(self.block_n)
        out = fn(q_bhd.contiguous(), k_pages, v_pages, block_table, seq_lens, self.S, **kwargs)
        self.actual_mode = "paged"
        return self._unwrap_tensor_out(out).contiguous()

    def info(self) -> Dict[str, Any]:
        return {**super().info(), "module": self.module_name, "requested_S": self.S, "seed": self.seed,
                "block_n": self.block_n, "actual_mode": self.actual_mode}


class SantaFlashBackend(_SantaBaseBackend):
    name = "santa_flash"
    module_candidates = ("santa_flash_batch_cuda", "santa_cuda")


class SantaPropBackend(_SantaBaseBackend):
    name = "santa_prop"
    module_candidates = ("santa_prop_batch_cuda",)


def _make_one_backend(raw_name: str, *, fa2_expected_version: str, fa2_version_policy: str, santa_s: int,
                      santa_seed: int, santa_block_n: Optional[int], flashinfer_mode: str,
                      flashinfer_use_tensor_cores: bool, flashinfer_expected_version: str,
                      flashinfer_version_policy: str, flashinfer_jit_mode: str,
                      flashinfer_preload_libstdcpp: str) -> DecodeAttentionBackend:
    """Name -> backend (tutorial_code/attention_backends.py:523-566)."""
    name = raw_name.lower().strip()
    if name == "sdpa":
        return SDPABackend()
    if name in ("fa2", "flashattn2", "flash_attention_2", "flash_attn"):
        return FA2Backend(expected_version=fa2_expected_version, version_policy=fa2_version_policy)
    if name == "flashinfer":
        return FlashInferBackend(mode=flashinfer_mode, use_tensor_cores=flashinfer_use_tensor_cores,
                                 expected_version=flashinfer_expected_version,
                                 version_policy=flashinfer_version_policy, jit_mode=flashinfer_jit_mode,
                                 preload_libstdcpp=flashinfer_preload_libstdcpp)
    if name in ("santa", "santa_flash"):
        return SantaFlashBackend(S=santa_s, seed=santa_seed, block_n=santa_block_n)
    if name == "santa_prop":
        return SantaPropBackend(S=santa_s, seed=santa_seed, block_n=santa_block_n)
    raise ValueError(f"Unsupported backend name: {raw_name}")


def build_backends(
    backend_names: Iterable[str],
    *,
    fa2_expected_version: str = FA2_PAPER_TARGET_VERSION,
    fa2_version_policy: str = "warn",
    santa_s: int,
    santa_seed: int,
    santa_block_n: Optional[int],
    flashinfer_mode: str,
    flashinfer_use_tensor_cores: bool,
    flashinfer_expected_version: str = FLASHINFER_PAPER_TARGET_VERSION,
    flashinfer_version_policy: str = "warn",
    flashinfer_jit_mode: str = "auto",
    flashinfer_preload_libstdcpp: str = "auto",
    skip_init_failures: Optional[bool] = None,
) -> Union[List[DecodeAttentionBackend], Tuple[List[DecodeAttentionBackend], List[Dict[str, Any]]]]:
    """Backends by name (tutorial_code/attention_backends.py:569-621).  With
    skip_init_failures=None a failure raises and the list is returned; with
    True/False the result is (backends, init_errors) and True records each
    failure instead of raising."""
    backends: List[DecodeAttentionBackend] = []
    init_errors: List[Dict[str, Any]] = []
    for raw_name in backend_names:
        try:
            backends.append(_make_one_backend(
                raw_name, fa2_expected_version=fa2_expected_version, fa2_version_policy=fa2_version_policy,
                santa_s=santa_s, santa_seed=santa_seed, santa_block_n=santa_block_n,
                flashinfer_mode=flashinfer_mode, flashinfer_use_tensor_cores=flashinfer_use_tensor_cores,
                flashinfer_expected_version=flashinfer_expected_version,
                flashinfer_version_policy=flashinfer_version_policy, flashinfer_jit_mode=flashinfer_jit_mode,
                flashinfer_preload_libstdcpp=flashinfer_preload_libstdcpp))
        except Exception as exc:  # noqa: BLE001 -- recorded or re-raised per skip_init_failures
            if skip_init_failures:
                init_errors.append({"backend": str(raw_name), "error_type": type(exc).__name__, "error": str(exc),
                                    "details": getattr(exc, "details", None)})
                continue
            raise
    if skip_init_failures is None:
        return backends
    return backends, init_errors
