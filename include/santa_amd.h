/*
 * santa_amd.h -- C ABI of the MI355X (gfx950) S^2ANTA sampled-attention
 * decode library (libsanta_amd.so).
 *
 * Plain pointers, sizes and a hipStream_t; no torch types.  All device
 * pointers are device memory on the current HIP device; every launch is
 * asynchronous on `stream` and nothing here synchronizes the device or reads
 * device memory on the host.  Inputs are never written.
 *
 * Reference interfaces replaced (upstream paths, with
 *   flash/ = flash_style_fused_santa_fixed_tile_budgets/,
 *   prop/  = santa_fused_proportional_tile_budgets/):
 *   santa_flash_plan          <- flash/santa_cuda.cpp:36-44,188-210 (block_n, T_c, S_per_tile)
 *   santa_flash_fused_tiles   <- launch_fused_tiles_vec_gqa_gh4_d128_bn{32,64,256}_{bf16,f16}
 *                                flash/santa_cuda.cpp:56-96, flash/santa_cuda_kernel.cu:514-626
 *   santa_flash_finalize      <- launch_finalize_weighted_{bf16,f16} + launch_reduce_vrows
 *                                flash/santa_cuda.cpp:98-120, flash/santa_cuda_kernel.cu:628-681
 *   santa_flash_decode        <- the launch sequence of decode_systematic_scalar,
 *   (+ _decode_tiles/_merge)     flash/santa_cuda.cpp:174-343 (minus the torch allocations)
 *   santa_prop_plan           <- prop/santa_cuda.cpp:39-77,188-229 (block_n, T_c, pass-1 path)
 *   santa_prop_pass1          <- launch_pass1_tiles_{vec,wmma}_gqa_{bf16,f16}
 *                                prop/santa_cuda.cpp:81-101, prop/santa_cuda_kernel.cu:445-519
 *   santa_prop_tile_budgets   <- launch_tile_budgets, prop/santa_cuda.cpp:108-112,
 *                                prop/santa_cuda_kernel.cu:904-915
 *   santa_prop_pass2          <- launch_pass2_grouped_fused_atomic_{bf16,f16} +
 *                                launch_cast_scale_out_{bf16,f16} + launch_reduce_vrows,
 *                                prop/santa_cuda.cpp:114-138, prop/santa_cuda_kernel.cu:917-1005
 *   santa_prop_decode         <- the launch sequence of decode_systematic_scalar,
 *                                prop/santa_cuda.cpp:270-352
 *
 * The stage entry points keep the reference launchers' split of the work and
 * their argument meaning, with these deviations:
 *   - no q_scale / scale argument (santa_flash_fused_tiles, santa_prop_pass1):
 *     the scale is computed inside from D exactly as the reference's host
 *     computes the value it passes, 1.0f / sqrtf((float)D) (flash: D = 128,
 *     bits 0x3DB504F3, flash/santa_cuda.cpp:210; prop/santa_cuda.cpp:208);
 *   - santa_flash_fused_tiles writes emit_cnt [B,KVH,T_c] (rows emitted per
 *     tile) where launch_fused_tiles_* writes rowmask [B,KVH,L]
 *     (flash/santa_cuda_kernel.cu:514-519), and santa_flash_finalize derives
 *     vrows from it (the reference's launch_reduce_vrows sums the rowmask);
 *   - one entry point per stage takes dtype, block_n and the pass-1 path as
 *     arguments where the reference has one launcher per (dtype, block_n,
 *     path) instantiation;
 *   - santa_prop_pass2 also casts and scales the output (the reference's
 *     launch_cast_scale_out_* is a separate launcher).
 *
 * Layouts (row-major, contiguous):
 *   q   [B, H, D]            (B = 1 for the single-request form [H, D])
 *   K,V [B, L_storage, KVH, D]  (NHD cache; prop: [L, KVH, D])
 *   out [B, H, D] in the input dtype, m_star [B, H] f32, vrows [B, KVH] i32.
 */
#ifndef SANTA_AMD_H_
#define SANTA_AMD_H_

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of q, K, V and out (the reference accepts bf16 or f16,
 * flash/santa_cuda.cpp:128-133). */
enum santa_dtype { SANTA_BF16 = 0, SANTA_F16 = 1 };

/* Return codes.  On failure santa_last_error() holds a message whose text
 * follows the reference's TORCH_CHECK messages where one exists. */
enum santa_status {
  SANTA_OK = 0,
  SANTA_ERR_INVALID = 1,     /* bad shape / argument */
  SANTA_ERR_UNSUPPORTED = 2, /* shape outside what the kernels implement */
  SANTA_ERR_WORKSPACE = 3,   /* workspace too small */
  SANTA_ERR_HIP = 4          /* a HIP launch failed */
};

/* Message of the last failure on the calling thread ("" if none). */
const char* santa_last_error(void);

/* Library version string. */
const char* santa_version(void);

/* ------------------------------------------------------------- flash */

/* Host planning.  L = valid_len > 0 ? valid_len : L_storage; block_n <= 0
 * selects 32 (L <= 1536), 64 (L <= 3072) or 256; T_c = ceil(L / block_n);
 * S_per_tile = S > 0 ? max(1, S / T_c) : 0. */
int santa_flash_plan(int64_t L_storage, int64_t valid_len, int64_t block_n, int64_t S, int* L_out,
                     int* block_n_out, int* T_c_out, int* S_per_tile_out);

/* One fused pass over every (b, kv, tile): scores, tile max / mass, seeded
 * systematic counts, emission compaction and the count-weighted V sum.
 * Outputs (device): m_tiles, ell_tiles [B,H,T_c] f32; out_tiles [B,H,T_c,D]
 * f32; emit_cnt [B,KVH,T_c] i32 (rows emitted per tile; replaces the
 * reference's rowmask); counts [B,H,T_c,block_n] i16 (may be NULL). */
int santa_flash_fused_tiles(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH,
                            int D, int L_valid, int L_storage, int block_n, int S_per_tile, uint64_t seed,
                            float* m_tiles, float* ell_tiles, float* out_tiles, int* emit_cnt, int16_t* counts,
                            hipStream_t stream);

/* Split-KV merge across tiles: m* = max_t m_t, w_t = exp(m_t - m*) ell_t,
 * out = (sum_t w_t out_t) / (Z S_per_tile) cast to dtype; vrows (may be
 * NULL) = distinct sampled rows per (b, kv). */
int santa_flash_finalize(const float* m_tiles, const float* ell_tiles, const float* out_tiles,
                         const int* emit_cnt, int dtype, int B, int H, int KVH, int D, int T_c, int S_per_tile,
                         void* out, float* m_star, int* vrows, hipStream_t stream);

/* Bytes of device workspace santa_flash_decode needs for this shape on the
 * current device (it depends on the device's compute-unit count). */
size_t santa_flash_workspace_size(int B, int H, int KVH, int D, int T_c);

/* Whole decode step (the production path).  Same results as
 * santa_flash_fused_tiles + santa_flash_finalize for m_star, vrows and every
 * sampled count; the output sum is merged per chunk of tiles with a running
 * max, so `out` agrees with the reference-order merge to rounding.
 * workspace >= santa_flash_workspace_size bytes, 256-B aligned; its contents
 * need no initialization. */
int santa_flash_decode(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH, int D,
                       int L_valid, int L_storage, int block_n, int S_per_tile, uint64_t seed, void* out,
                       float* m_star, int* vrows, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* The two launches of santa_flash_decode, for callers that schedule them
 * separately: the tile pass writes chunk partials into the workspace, the
 * merge pass reads them. */
int santa_flash_decode_tiles(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH, int D,
                             int L_valid, int L_storage, int block_n, int S_per_tile, uint64_t seed, void* workspace,
                             size_t workspace_bytes, hipStream_t stream);
int santa_flash_decode_merge(const void* workspace, size_t workspace_bytes, int dtype, int B, int H, int KVH, int D,
                             int T_c, int S_per_tile, void* out, float* m_star, int* vrows, hipStream_t stream);

/* santa_flash_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The workspace lives in a static device array of 16 MiB (16,777,216
 * bytes) that each device holds until the process ends; shapes whose
 * santa_flash_workspace_size exceeds it are rejected with
 * SANTA_ERR_WORKSPACE before anything is launched.  The call makes no hipMalloc / hipFree or other allocation.
 * The array needs no initialisation (every kernel writes what a later one
 * reads).  Every call on a device shares that device's array: calls that
 * overlap on one device (different streams, or host threads) race and must
 * be ordered by the caller.  Results are bit-identical to santa_flash_decode
 * on the same arguments.  Under HIP graph capture: make one uncaptured call
 * on each device first (it takes the scratch array's device address with
 * hipGetSymbolAddress); captured calls then record kernel launches only (no
 * memset or copy nodes), and their replays give the direct call's bits. */
int santa_flash_decode_noalloc(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH, int D,
                               int L_valid, int L_storage, int block_n, int S_per_tile, uint64_t seed, void* out,
                               float* m_star, int* vrows, hipStream_t stream);

/* Ragged flash (no counterpart in the reference, whose batched call takes
 * one valid_len for every sequence, flash/santa_cuda.cpp:188): sequence b of
 * a [B, L_storage, KVH, D] cache is decoded on its first seq_lens[b] tokens
 * with S_per_tile = S > 0 ? max(1, S / ceil(seq_lens[b] / block_n)) : 0 and
 * RNG key b*H + h -- exactly what the uniform call does when every length
 * equals seq_lens[b].  seq_lens: device int array [B]; max_len = max
 * seq_lens (<= L_storage) and total_tiles = sum over b of
 * ceil(seq_lens[b] / block_n), from the host; one block_n (32, 64 or 256)
 * for every sequence.  out [B,H,D], m_star [B,H], vrows [B,KVH] (may be
 * NULL).  Lengths are clamped on the device to [1, max_len].  Workspace:
 * santa_flash_ragged_workspace_size with max_tiles = ceil(max_len / block_n). */
size_t santa_flash_ragged_workspace_size(int B, int H, int KVH, int D, int max_tiles, long long total_tiles);
int santa_flash_decode_ragged(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH, int D,
                              int L_storage, const int* seq_lens, int max_len, long long total_tiles, int block_n,
                              int64_t S, uint64_t seed, void* out, float* m_star, int* vrows, void* workspace,
                              size_t workspace_bytes, hipStream_t stream);

/* Paged flash (no counterpart in the reference, which reads contiguous NHD
 * caches only, README.md:257 and tutorial_code/runtime_common.py:340-397):
 * santa_flash_decode_ragged over a page pool K_pages / V_pages
 * [num_pages, page_size, KVH, D] in place of the contiguous cache.  Token n
 * of sequence b is row n % page_size of page
 * block_table[b * table_stride + n / page_size]; block_table is a device int
 * array [B, table_stride] with table_stride >= ceil(max_len / page_size).
 * page_size is a power of two in [8, 2^20].  Page ids are clamped to
 * [0, num_pages) on the device.  Results are bit-identical to the ragged call
 * on the same tokens stored contiguously.  Workspace:
 * santa_flash_ragged_workspace_size(B, H, KVH, D, ceil(max_len / block_n),
 * total_tiles). */
int santa_flash_decode_paged(const void* q, const void* K_pages, const void* V_pages, int dtype, int B, int H, int KVH,
                             int D, int num_pages, int page_size, const int* block_table, int table_stride,
                             const int* seq_lens, int max_len, long long total_tiles, int block_n, int64_t S,
                             uint64_t seed, void* out, float* m_star, int* vrows, void* workspace,
                             size_t workspace_bytes, hipStream_t stream);

/* -------------------------------------------------------------- prop */

/* Host planning.  block_n <= 0 selects 256 when pass1_env is "vec"/"gqa_vec",
 * else the flash heuristic; pass1_path_out = 0 (exact vec path: GH=4, D=128,
 * block_n=256) or 1 (general MFMA path).  pass1_env may be NULL. */
int santa_prop_plan(int L, int H, int KVH, int D, int64_t block_n, const char* pass1_env, int* block_n_out,
                    int* T_c_out, int* pass1_path_out);

/* Pass 1 for one sequence: per-tile max / mass and the u stash [L, H]
 * (16-bit, index n*H + h).  m_tiles, ell_tiles [H, T_c] f32. */
int santa_prop_pass1(const void* q, const void* K, int dtype, int H, int KVH, int D, int L, int block_n,
                     int pass1_path, float* m_tiles, float* ell_tiles, void* u_stash, hipStream_t stream);

/* Largest-remainder tile budgets per head (deterministic Z order):
 * m_star [H]; S_tiles [H,T_c] i32; invdelta, a0 [H,T_c] f32. */
int santa_prop_tile_budgets(const float* m_tiles, const float* ell_tiles, int H, int T_c, int S, uint64_t seed,
                            float* m_star, int* S_tiles, float* invdelta, float* a0, hipStream_t stream);

/* Pass 2 + cast: counts from the stash, count-weighted V sums summed per
 * chunk of tiles in a fixed order (deterministic), out = dtype(sum / S)
 * (0 when S <= 0).  counts [H,T_c,block_n] i16 and vrows [KVH] may be NULL.
 * workspace >= santa_prop_workspace_size bytes (its chunk-partial region is
 * used; contents need no initialization). */
int santa_prop_pass2(const void* V, const void* u_stash, int dtype, int H, int KVH, int D, int L, int block_n,
                     int S, const float* invdelta, const float* a0, int16_t* counts, void* out, int* vrows,
                     void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Bytes of device workspace santa_prop_decode / santa_prop_pass2 need on the
 * current device (m, ell, budgets, the u stash and chunk partials). */
size_t santa_prop_workspace_size(int H, int KVH, int D, int L, int T_c);

/* Whole single-sequence prop decode with the caller's workspace. */
int santa_prop_decode(const void* q, const void* K, const void* V, int dtype, int H, int KVH, int D, int L,
                      int block_n, int pass1_path, int S, uint64_t seed, void* out, float* m_star, int* vrows,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Batched, ragged santa_prop (no counterpart in the reference, whose adapter
 * loops over sequences, tutorial_code/attention_backends.py:491-500): B
 * sequences of a [B, L_storage, KVH, D] cache, sequence b decoded exactly as
 * santa_prop_decode on its first seq_lens[b] tokens with budget seq_S[b]
 * (RNG key h, as in the per-sequence calls).  seq_lens, seq_S: device int
 * arrays [B]; max_len = max seq_lens; total_tiles = sum over b of
 * ceil(seq_lens[b] / block_n); every sequence uses the same block_n and
 * pass-1 path.  out [B,H,D], m_star [B,H], vrows [B,KVH] (may be NULL). */
size_t santa_prop_batched_workspace_size(int B, int H, int KVH, int D, int L_storage, int max_tiles,
                                         long long total_tiles);
int santa_prop_decode_batched(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH, int D,
                              int L_storage, const int* seq_lens, const int* seq_S, int max_len, long long total_tiles,
                              int block_n, int pass1_path, uint64_t seed, void* out, float* m_star, int* vrows,
                              void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Paged santa_prop (no counterpart in the reference, which reads contiguous
 * NHD caches only, README.md:257): santa_prop_decode_batched over a page
 * pool K_pages / V_pages [num_pages, page_size, KVH, D], with the block table
 * and page geometry of santa_flash_decode_paged.  Results are bit-identical
 * to the batched call on the same tokens stored contiguously.  Workspace:
 * santa_prop_batched_workspace_size(B, H, KVH, D, max_len, ceil(max_len /
 * block_n), total_tiles). */
int santa_prop_decode_paged(const void* q, const void* K_pages, const void* V_pages, int dtype, int B, int H, int KVH,
                            int D, int num_pages, int page_size, const int* block_table, int table_stride,
                            const int* seq_lens, const int* seq_S, int max_len, long long total_tiles, int block_n,
                            int pass1_path, uint64_t seed, void* out, float* m_star, int* vrows, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------- model-level decode */

/* Fused elementwise steps of the model-level decode loop
 * (santa_amd/runtime.py); the reference runs them as separate torch
 * kernels inside the HF decoder layer (tutorial_code/runtime_common.py:
 * 501-571).  bf16 tensors, rows contiguous.
 *
 * santa_rt_add_rms_norm: per row of h [rows, hidden], h = bf16(h + a) when a
 * is not null, then x = bf16(float(h) * rsqrt(mean(float(h)^2) + eps) *
 * float(w)).
 * santa_rt_rope_write: qkv [B, H + 2 KVH, D] (the fused projection's
 * output); q heads rotated into q_out [B, H, D], k heads rotated into
 * k_cache[b, pos] and v heads copied into v_cache[b, pos] of caches
 * [B, storage, KVH, D]; RoPE in the rotate-half convention with cos, sin
 * [D] and bf16 rounding of each product and of the sum.
 * santa_rt_silu_mul: out [rows, inter] = bf16(bf16(silu(gate)) * up), gate
 * and up the two halves of gu [rows, 2 inter].
 * santa_rt_linear: the decode step's weight products (the HF layers'
 * nn.Linear, bf16, no bias): y [M, N] = bf16(x [M, K] . w [N, K]^T),
 * float32 accumulation, for 1 <= M <= 8, K a multiple of 8, M rounded up to
 * 1, 2, 4 or 8 times K rounded up to 2048 at most 65536, x and w 16-byte
 * aligned.  swiglu != 0: w is [2N, K] (gate rows, then up rows) and
 * y [M, N] = bf16(bf16(silu(bf16(g))) * bf16(u)), silu_mul of the product.
 * The weights are read once at the HBM bound.
 * santa_rt_linear_rope: the fused q/k/v projection of rows x [M, K] by
 * w [(H + 2 KVH) D, K] (head by head) with santa_rt_rope_write's epilogue
 * applied to the bf16 products: q heads rotated into q_out [M, H, D], k heads
 * rotated into k_cache[b, pos], v heads into v_cache[b, pos] (caches
 * [M, storage, KVH, D]); bit for bit santa_rt_rope_write of santa_rt_linear's
 * output, without writing that output.  D even; the santa_rt_linear limits
 * on M and K.
 * santa_rt_argmax: out[r] (int64) = the index of the maximum of row r of
 * x [rows, n] (float32), torch.argmax's choice: NaN above any number, the
 * first index among equal values; the greedy step's token choice
 * (tutorial_code/runtime_common.py:574-675). */
int santa_rt_add_rms_norm(void* h, const void* a, const void* w, void* x, int rows, int hidden, float eps,
                          hipStream_t stream);
int santa_rt_rope_write(const void* qkv, const void* cos_, const void* sin_, void* q_out, void* k_cache, void* v_cache,
                        int B, int H, int KVH, int D, long long storage, int pos, hipStream_t stream);
int santa_rt_silu_mul(const void* gu, void* out, int rows, int inter, hipStream_t stream);
int santa_rt_linear(const void* x, const void* w, void* y, int M, int N, int K, int swiglu, hipStream_t stream);
int santa_rt_linear_rope(const void* x, const void* w, int M, int K, const void* cos_, const void* sin_, void* q_out,
                         void* k_cache, void* v_cache, int H, int KVH, int D, long long storage, int pos,
                         hipStream_t stream);
int santa_rt_argmax(const float* x, int rows, int n, long long* out, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SANTA_AMD_H_ */
