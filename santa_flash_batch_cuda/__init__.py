"""S^2ANTA-Flash sampled-attention decode on MI355X -- drop-in for the
reference's `santa_flash_batch_cuda` extension module
(flash_style_fused_santa_fixed_tile_budgets/santa_cuda.cpp:346-359).

    decode_systematic_scalar(q_h, K_g, V_g, S, seed=42, block_n=0,
                             want_vrows=False, valid_len=-1) -> (out, m_star, vrows)
    decode_systematic_batched(...)   # the same function
    decode_systematic_paged(q_h, K_pages, V_pages, block_table, seq_lens, S,
                            seed=42, block_n=0, want_vrows=False) -> (out, m_star, vrows)

decode_systematic_paged (an addition over the reference, which reads
contiguous caches only) takes a page pool K_pages / V_pages
[num_pages, page_size, KVH, D] and an int32 block table [B, pages per
sequence]: token n of sequence b is row n % page_size of page
block_table[b, n // page_size].  page_size is a power of two >= 8.

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
    _mfma_fma_check,
    _tile_pass_kernel,
    _workspace_bytes,
    decode_systematic_batched,
    decode_systematic_paged,
    decode_systematic_scalar,
)
