// santa_internal.h -- host-side helpers shared by the C-ABI translation units.
#pragma once

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

namespace santa {

// Paged KV cache: a pool of pages [num_pages, 1 << shift, KVH, D]; token n of
// sequence b is row n & ((1 << shift) - 1) of page
// table[b * stride + (n >> shift)].  table == nullptr selects the contiguous
// [B, L_storage, KVH, D] layout.  shift >= 3, so an 8-row aligned block of
// tokens never straddles two pages.
struct PageTable {
  const int* table;
  int stride;  // table entries per sequence
  int shift;   // log2 of the page size
  int num_pages;
};

// Records a printf-style message as the calling thread's last error and
// returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the calling thread's last error and returns SANTA_OK.
int clear_error();
// Checks a paged cache's geometry (page_size a power of two in [8, 2^20],
// num_pages > 0, table_stride >= ceil(max_len / page_size)) and fills pt.
int check_page_table(const int* table, int num_pages, int page_size, int table_stride, int max_len, PageTable* pt);

constexpr size_t kWsAlign = 256;
inline size_t align_up(size_t x) { return (x + kWsAlign - 1) & ~(kWsAlign - 1); }

namespace flash {
// santa_prop pass 1 on the flash tile kernel: per-tile m, ell [B, H, T_c] and
// the 16-bit u stash [B, L_storage, H].  path 0 = vec numerics (GH 4,
// block_n 256), 1 = general numerics.  Shapes are checked by the caller.
// Ragged form: seq_lens (device, [B]) holds each sequence's length, L the
// longest (it sets the tile stride of m/ell), cs tiles per chunk and n_wg
// workgroups (any workgroup past the last sequence exits at once).
// stash_ld > 0 (vec path only): the stash is tile-major [B, stash_ld / 256, H, 256],
// whole 256-row tiles, 0 past each sequence's length.
// kv_div > 1: KVH counts virtual KV heads, kv_div per KV head of the cache,
// each with H / KVH (5-8) query heads (the general path at block_n 256 with
// the tile-major stash only).
hipError_t launch_prop_pass1(const void* q, const void* K, int dtype, int B, int H, int KVH, int L, int L_storage,
                             int block_n, int path, float* m_tiles, float* ell_tiles, uint16_t* u_stash,
                             const int* seq_lens, int cs, int n_wg, int stash_ld, hipStream_t stream,
                             PageTable pt = PageTable{nullptr, 0, 3, 1}, long long total_tiles = -1,
                             int kv_div = 1);
// Chunking of a ragged batch with total_tiles tiles, the longest sequence
// having max_tiles: cs tiles per chunk and an upper bound n_wg on the
// workgroups of the ragged grid.
// per_round: work items per resident round (0: one per 4-wave workgroup
// slot); granule: cs is a multiple of it for uneven lengths; rounds: about
// how many resident rounds the chunks of uneven lengths make.
void plan_ragged(int B, int KVH, long long total_tiles, int max_tiles, int* cs, int* n_wg, int per_round = 0,
                 int granule = 4, int rounds = 8);
// The flash tile pass's layout: one wave per KV head (ROWS) for KVH = 8, its
// chunks planned for rows_per_round() items per round.
bool rows_layout(int KVH);
// A tile pass with at most one resident round of (kv, tile) items (a quarter of
// one at GH 8) runs four waves per tile (tile_kernel) rather than one
// (wave_kernel).
bool small_pass(long long kv_tiles, int GH);
// Uniform (one length) flash calls keep the tile kernel up to one and a half
// resident rounds (a quarter of one at GH 8); the launch, the workspace plan and
// the bench label all decide with this one function.
bool uniform_small_pass(int B, int KVH, int T_c, int GH);
bool small_prop_pass(long long kv_tiles);
// santa_prop's pass 1 on the wave kernel (block_n 256: the vec path at GH 4,
// the general path at GH 8); it writes the tile-major stash when given a
// stash_ld, which pass 2 then reads.
bool prop_wave_pass1(int path, int GH, int block_n);
int rows_per_round();
// The block_n = 256 online tile pass (the wave kernel) with its per-tile
// statistics m, ell [B, H, T_c] and counts [B, H, T_c, 256] written out
// (test hook; the chunk partials go to the santa_flash_decode workspace).
hipError_t launch_wave_debug(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH,
                             int L_valid, int L_storage, int S_pt, uint64_t seed, void* workspace, float* m_tiles,
                             float* ell_tiles, int16_t* counts, hipStream_t stream);
// y[i] = santa_expf(x[i]) on the device (test hook for the exponential).
hipError_t launch_expf(const float* x, float* y, size_t n, hipStream_t stream);
// The score path's broadcast K=1 MFMA and fmaf on the same operands (test
// hook): n_waves waves; a, b [64 n_waves], c [4 * 64 n_waves]; outputs
// [n_waves, 16 blocks, 64 lanes, 4].
hipError_t launch_mfma_check(const float* a, const float* b, const float* c, float* mfma_out, float* fma_out,
                             int n_waves, hipStream_t stream);
// Chunks of cs tiles per workgroup, cpg chunks per (b, kv) group, sized to
// about one resident round of 256-thread workgroups on the current device.
void plan_chunks(int B, int KVH, int T_c, int* cs, int* cpg, int per_round = 0);
}  // namespace flash

namespace propgen {
// santa_prop's shapes outside the tuned kernels (santa_prop_gen.hip): any
// GH <= 16, D a multiple of 16 up to 1024, block_n a multiple of 16 up to 512.
// generic_shape: the shape is not one the tuned kernels take (D = 128, GH 4
// or 8, block_n 32 / 64 / 256); shape_supported: the generic kernels take it.
bool generic_shape(int GH, int D, int block_n);
bool shape_supported(int GH, int D, int block_n);
// Pass 1 (general numerics): m, ell [B, H, T_c] and the stash [B, L_storage,
// H], or tile-major [B, stash_ld / 256, H, 256] when stash_ld > 0 (only for
// fast_pass1_shape); ragged with seq_lens (L the longest) over total_tiles
// tiles.
bool fast_pass1_shape(int GH, int D, int block_n);
hipError_t launch_pass1(const void* q, const void* K, int dtype, int B, int H, int KVH, int D, int L, int L_storage,
                        int BN, float* m_tiles, float* ell_tiles, uint16_t* u_stash, const int* seq_lens,
                        long long total_tiles, PageTable pt, hipStream_t stream, int stash_ld = 0);
// The budgets for any tile count (one workgroup per (b, h), BH of them).
hipError_t launch_budgets_big(const float* m_tiles, const float* ell_tiles, int BH, int H, int T_c, int S,
                              uint64_t seed, float* m_star, int* S_tiles, float* invdelta, float* a0,
                              const int* seq_lens, const int* seq_S, int BN, hipStream_t stream);
// Pass 2 over the [B, L_storage, H] stash into per-chunk partials
// [chunks, GH, D] (the chunk grid of flash::plan_chunks / plan_ragged), and
// the finalize that sums them.
hipError_t launch_pass2(const void* V, const uint16_t* u_stash, int dtype, int B, int H, int KVH, int D, int L,
                        int L_storage, int BN, int T_c, int cs, int cpg, int n_wg, const float* invdelta,
                        const float* a0, int16_t* counts, float* part, int* part_emit, int want_emit,
                        const int* seq_lens, PageTable pt, hipStream_t stream, int stash_ld = 0);
// Waves per generic pass-2 workgroup (one per head, up to four); the chunk
// plan counts min(GH, 4)-wave workgroups for GH < 4.
int pass2_waves(int GH);
// Generic pass-2 workgroups resident on the current device at once (its
// registers and LDS allow), for the chunk plan; 0 if the runtime cannot say.
int pass2_resident(int GH, int D);
hipError_t launch_finalize(const float* part, const int* part_emit, int dtype, int B, int H, int KVH, int D, int cpg,
                           float scale_out, void* out, int* vrows, const int* seq_lens, const int* seq_S, int BN,
                           int cs, int max_rows, int n_wg, hipStream_t stream);
}  // namespace propgen

}  // namespace santa
