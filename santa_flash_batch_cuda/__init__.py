"""S^2ANTA-Flash sampled-attention decode on MI355X -- drop-in for the
reference's `santa_flash_batch_cuda` extension module
(flash_style_fused_santa_fixed_tile_budgets/santa_cuda.cpp:346-359).

    decode_systematic_scalar(q_h, K_g, V_g, S, seed=42, block_n=0,
                             want_vrows=False, valid_len=-1) -> (out, m_star, vrows)
    decode_systematic_batched(...)   # the same function

torch is imported first so that the native module binds to torch's HIP runtime.
"""
import torch  # noqa: F401  (must precede the native module)

from ._C import (  # noqa: F401
    _debug_tiles,
    _debug_wave,
    _decode_reference_order,
    _decode_tiles_only,
    _device_expf,
    _library_version,
    _workspace_bytes,
    decode_systematic_batched,
    decode_systematic_scalar,
)
