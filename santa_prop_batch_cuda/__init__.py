"""S^2ANTA-Prop sampled-attention decode on MI355X -- drop-in for the
reference's `santa_prop_batch_cuda` extension module
(santa_fused_proportional_tile_budgets/santa_cuda.cpp:354-358).

    decode_systematic_scalar(q_h, K_g, V_g, S, seed=42, block_n=0,
                             want_vrows=False) -> (out, m_star, vrows)
    decode_systematic_batched(q_h, K_g, V_g, S, seed=42, block_n=0,
                              want_vrows=False, valid_len=-1) -> (out, m_star, vrows)
    decode_systematic_paged(q_h, K_pages, V_pages, block_table, seq_lens, S,
                            seed=42, block_n=0, want_vrows=False) -> (out, m_star, vrows)

Single sequence: q_h [H, D], K_g / V_g [L, KVH, D].  Batched (an addition
over the reference, whose adapter loops over sequences): q_h [B, H, D],
K_g / V_g [B, L_storage, KVH, D]; S and valid_len are ints or one value per
sequence, and sequence b is decoded exactly as the scalar call on
K_g[b, :valid_len[b]] with budget S[b].  The environment variable
SANTA_PASS1 (auto / gqa / vec) selects the pass-1 numerics on every call, as
in the reference.  Paged (also an addition): a page pool K_pages / V_pages
[num_pages, page_size, KVH, D] and an int32 block table [B, pages per
sequence]; token n of sequence b is row n % page_size of page
block_table[b, n // page_size], page_size a power of two >= 8.

torch is imported first so that the native module binds to torch's HIP runtime.
"""
import torch  # noqa: F401  (must precede the native module)

from ._C import (  # noqa: F401
    _debug_pass,
    _library_version,
    decode_systematic_batched,
    decode_systematic_paged,
    decode_systematic_scalar,
)
