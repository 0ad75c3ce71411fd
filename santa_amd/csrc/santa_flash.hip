// santa_flash.hip -- santa_flash (fixed tile budget) decode kernels for gfx950.
//
// Decomposition.  A KV tile is block_n consecutive tokens of one (b, kv)
// group.  The tiles of a group are split into contiguous chunks, one chunk
// per 256-thread workgroup (4 wave64), sized so that the grid is about one
// resident round on the device.  A workgroup walks its chunk tile by tile and
// prefetches the next tile's K rows (non-temporal loads) before it runs the
// current tile's softmax statistics, sampler and V gather, so the HBM stream
// never waits for that serial tail.
//
// Per tile:
//  A  scores.  Lane i of wave w owns K row 64w+i.  The wave stages its 64
//     rows in LDS (coalesced non-temporal 16-B loads, 16 lanes per row,
//     XOR-swizzled 16-B slots) and reads back its own row.  The reference's
//     per-virtual-lane fma chains (4 dims each) run on the matrix pipe as
//     v_mfma_f32_4x4x1f32 with the A operand broadcast (CBSZ=4, ABID=dim%16):
//     q for 16 dims x 4 heads sits in one VGPR (lane 4j+i: head i, dim 16m+j),
//     k of the lane's own row is the B operand, and each lane accumulates its
//     row's 4 heads in place.  A K=1 MFMA is one fused multiply-add with a
//     single rounding, bit-identical to fmaf (checked by a GPU test).  The
//     reference's 32-lane tree (flash/santa_cuda_kernel.cu:183-211) becomes
//     in-register adds over the virtual lanes in the same pairing.
//  B  tile max per head: wave maxima, one LDS exchange (exact in any order).
//  C  u = exp(s - m), the 16-bit u and ell with the reference's per-thread /
//     32-lane-tree / per-warp association (:243-273), the 32-lane trees as
//     in-wave butterflies.
//  D  systematic counts (:275-311): each wave owns one head (two for GH=8)
//     and scans the tile two rows per lane (systematic_counts), the
//     reference's sequential cross-chunk carries as wave-uniform scalars, so
//     no workgroup barrier is needed.
//  E  the head's sampled rows, in ascending order (ballot prefix counts),
//     go to a wave-private LDS list: the reference's emission list with zero
//     counts skipped (:314-379).  The count-weighted V sum gathers the
//     listed rows, fma per element in ascending row order.
//  Two workgroup barriers per tile.
//
// The same kernel runs santa_prop's pass 1 (modes kPass1Vec / kPass1Gen):
// phases A-C, then the tile's m, ell and the 16-bit u stash [L, H]
// (prop/santa_cuda_kernel.cu:87-267, 278-441).
//
// Outputs.  Mode kOnline merges the chunk's tiles on the fly (running max
// and rescaled mass / numerator per head) into a chunk partial; a small
// kernel merges the chunk partials of each (b, h).  Mode kPerTile writes the
// reference's per-tile m, ell and count-weighted sums (plus, on request, the
// counts) and finalize_kernel merges them with the reference's association.
#include "santa_device.h"
#include "santa_amd.h"
#include "santa_internal.h"

#include <algorithm>
#include <type_traits>
#include <utility>
#include <atomic>
#include <mutex>

namespace santa {
namespace flash {

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kPartStride = kD + 2;  // chunk partial: M, Z, num[128]
constexpr int kListCap = 128;        // sampled rows buffered per head before a gather (>= 2 x 64)
// Buffer descriptor word 3 for raw (untyped) loads on gfx9-family parts, and
// the cache-policy bits of a non-temporal load (the "nt" bit).
constexpr int kBufferWord3 = 0x00020000;
constexpr int kBufferNontemporal = 2;
// kPerTile / kOnline: santa_flash.  kPass1Vec: santa_prop pass 1 with the
// vec kernel's numerics (= the flash tile statistics).  kPass1Gen: santa_prop
// pass 1 of the general path: q rounded to the 16-bit type after scaling and
// ell summed per 16-row slab, then over slabs (the reference's WMMA kernel,
// prop/santa_cuda_kernel.cu:121-140,225-262); scores keep the vec
// association, one fixed order for what the reference leaves to its MMA.
enum Mode : int { kPerTile = 0, kOnline = 1, kPass1Vec = 2, kPass1Gen = 3 };

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// K=1 MFMA with the A operand of block J broadcast to all 16 blocks:
// d[i] at lane l = a(lane 4J+i) * b(lane l) + c[i], one rounding per element.
template <int J>
__device__ __forceinline__ f32x4 mfma_bcast(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, J, 0);
}

// The fma chains of virtual lanes 2C (dims 8C..8C+3) and 2C+1 (8C+4..8C+7)
// for this lane's K row (chunk C of its LDS slot) and every head block.
template <bool BF16, int NHB, int C>
__device__ __forceinline__ void score_chunk(const u32x4* wk, int row, const float (&qa)[NHB][8], f32x4 (&pe)[NHB],
                                            f32x4 (&po)[NHB]) {
  const u32x4 kc = wk[row * 16 + (C ^ (row & 15))];
  const float k0 = lo16_to_f32<BF16>(kc.x), k1 = hi16_to_f32<BF16>(kc.x);
  const float k2 = lo16_to_f32<BF16>(kc.y), k3 = hi16_to_f32<BF16>(kc.y);
  const float k4 = lo16_to_f32<BF16>(kc.z), k5 = hi16_to_f32<BF16>(kc.z);
  const float k6 = lo16_to_f32<BF16>(kc.w), k7 = hi16_to_f32<BF16>(kc.w);
  constexpr int M = C / 2;          // q register: dims 16M .. 16M+15
  constexpr int J = 8 * (C % 2);    // block of dim 8C inside it
  const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb) {
    const float qv = qa[hb][M];
    f32x4 de = mfma_bcast<J + 0>(qv, k0, z);
    f32x4 dd = mfma_bcast<J + 4>(qv, k4, z);
    de = mfma_bcast<J + 1>(qv, k1, de);
    dd = mfma_bcast<J + 5>(qv, k5, dd);
    de = mfma_bcast<J + 2>(qv, k2, de);
    dd = mfma_bcast<J + 6>(qv, k6, dd);
    de = mfma_bcast<J + 3>(qv, k3, de);
    dd = mfma_bcast<J + 7>(qv, k7, dd);
    pe[hb] = de;
    po[hb] = dd;
  }
}

// B(C) of the reference tree for even and odd virtual lanes: chunks C, C+8
// (level off16), C+4, C+12 (level off8); four independent chunks so eight
// MFMA chains overlap.
template <bool BF16, int NHB, int C>
__device__ __forceinline__ void score_group(const u32x4* wk, int row, const float (&qa)[NHB][8], f32x4 (&be)[NHB],
                                            f32x4 (&bo)[NHB]) {
  f32x4 e0[NHB], o0[NHB], e8[NHB], o8[NHB], e4[NHB], o4[NHB], e12[NHB], o12[NHB];
  score_chunk<BF16, NHB, C>(wk, row, qa, e0, o0);
  score_chunk<BF16, NHB, C + 8>(wk, row, qa, e8, o8);
  score_chunk<BF16, NHB, C + 4>(wk, row, qa, e4, o4);
  score_chunk<BF16, NHB, C + 12>(wk, row, qa, e12, o12);
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb) {
    be[hb] = (e0[hb] + e8[hb]) + (e4[hb] + e12[hb]);
    bo[hb] = (o0[hb] + o8[hb]) + (o4[hb] + o12[hb]);
  }
}

// Materializes v here: an empty asm that reads and writes it, so the
// compiler cannot sink the arithmetic that produces v to its later uses
// (which would keep every partial of a tile's scores live at once).
__device__ __forceinline__ void pin(f32x4& v) { asm volatile("" : "+v"(v)); }

// score_chunk / score_group for one head block (q registers qv[8]).
template <bool BF16, int C>
__device__ __forceinline__ void score_chunk1(const u32x4* wk, int row, const float (&qv)[8], f32x4& pe, f32x4& po) {
  const u32x4 kc = wk[row * 16 + (C ^ (row & 15))];
  const float k0 = lo16_to_f32<BF16>(kc.x), k1 = hi16_to_f32<BF16>(kc.x);
  const float k2 = lo16_to_f32<BF16>(kc.y), k3 = hi16_to_f32<BF16>(kc.y);
  const float k4 = lo16_to_f32<BF16>(kc.z), k5 = hi16_to_f32<BF16>(kc.z);
  const float k6 = lo16_to_f32<BF16>(kc.w), k7 = hi16_to_f32<BF16>(kc.w);
  constexpr int M = C / 2;
  constexpr int J = 8 * (C % 2);
  const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
  const float q = qv[M];
  f32x4 de = mfma_bcast<J + 0>(q, k0, z);
  f32x4 dd = mfma_bcast<J + 4>(q, k4, z);
  de = mfma_bcast<J + 1>(q, k1, de);
  dd = mfma_bcast<J + 5>(q, k5, dd);
  de = mfma_bcast<J + 2>(q, k2, de);
  dd = mfma_bcast<J + 6>(q, k6, dd);
  de = mfma_bcast<J + 3>(q, k3, de);
  dd = mfma_bcast<J + 7>(q, k7, dd);
  pe = de;
  po = dd;
}
template <bool BF16, int C>
__device__ __forceinline__ void score_group1(const u32x4* wk, int row, const float (&qv)[8], f32x4& be, f32x4& bo) {
  // a scheduling fence after each chunk pair keeps only two chunks'
  // accumulators live
  f32x4 e0, o0, e8, o8, e4, o4, e12, o12;
  score_chunk1<BF16, C>(wk, row, qv, e0, o0);
  score_chunk1<BF16, C + 8>(wk, row, qv, e8, o8);
  const f32x4 ae = e0 + e8, ao = o0 + o8;
  __builtin_amdgcn_sched_barrier(0);
  score_chunk1<BF16, C + 4>(wk, row, qv, e4, o4);
  score_chunk1<BF16, C + 12>(wk, row, qv, e12, o12);
  be = ae + (e4 + e12);
  bo = ao + (o4 + o12);
  __builtin_amdgcn_sched_barrier(0);
}

// Number of rows of a tile sampled by any head of the group: the union of
// the per-head nonzero-count masks (one 64-row block per lane < NBLK).
template <int GH, int NBLK>
__device__ __forceinline__ int union_rows(const uint64_t* s_mask, int lane) {
  int e = 0;
  if (lane < NBLK) {
    uint64_t u = 0;
#pragma unroll
    for (int g = 0; g < GH; ++g) u |= s_mask[g * NBLK + lane];
    e = __popcll(u);
  }
#pragma unroll
  for (int m = 1; m < NBLK; m <<= 1) e += __shfl_xor(e, m, 64);
  return e;
}

// Tile max of head g from the four waves' order-key maxima.
template <int GH>
__device__ __forceinline__ float tile_max_of(const int* s_wmax, int g) {
  return from_order_key(max(max(s_wmax[g], s_wmax[GH + g]), max(s_wmax[2 * GH + g], s_wmax[3 * GH + g])));
}

template <bool BF16, int GH, int BN, int MODE, bool PAGED = false>
__global__ __launch_bounds__(kThreads, 2) void tile_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V, int H, int KVH,
    int L_valid, int L_storage, int T_c, int cs, int cpg, float q_scale, int S_pt, uint64_t seed,
    float* __restrict__ m_tiles, float* __restrict__ ell_tiles, float* __restrict__ out_tiles,
    int* __restrict__ emit_cnt, int16_t* __restrict__ dbg_counts, float* __restrict__ part,
    int* __restrict__ part_emit, uint16_t* __restrict__ u_stash, const int* __restrict__ seq_lens, int B,
    long long S_total, PageTable pt) {
  static_assert(BN == 32 || BN == 64 || BN == 256, "block_n");
  static_assert(!PAGED || MODE != kPerTile, "the reference-structured per-tile mode reads contiguous caches only");
  static_assert(GH == 4 || GH == 8, "group size");
  constexpr int NT_REF = (BN == 256) ? 256 : 128;  // reference block size (launchers :521,:559)
  constexpr int NW_REF = NT_REF / 32;
  constexpr int HPW = GH / 4;                      // heads per wave in phases D-E
  constexpr int NCH = BN / 32;                     // 32-row scan chunks
  constexpr int NPAIR = (NCH + 3) / 4;             // two-rows-per-lane scan registers
  constexpr int KC = BN * GH / NT_REF;             // (row, head) items per reference thread
  constexpr bool PASS1 = (MODE == kPass1Vec || MODE == kPass1Gen);
  constexpr int NSLAB = BN / 16;                   // 16-row slabs of the general pass 1
  constexpr int NWS = (MODE == kPass1Gen) ? NSLAB : NW_REF;  // ell partials per head
  constexpr int LCAP = (MODE == kOnline) ? kListCap : (PASS1 ? 1 : BN);  // sampled rows buffered per head

  const int wg = static_cast<int>(blockIdx.x);
  // The KV heads of one chunk of tokens are neighbours in launch order, so
  // they run together and read whole token rows (KVH x 256 B) of the NHD
  // cache at about the same time.  T_c is the tile stride of the per-tile
  // outputs (the longest sequence's tile count in the ragged form).
  const GridPos gp = grid_pos(wg, seq_lens, B, KVH, BN, L_valid, T_c, cs, cpg);
  const int kv = gp.kv;
  const int chunk = gp.chunk;
  const int b = gp.b < 0 ? 0 : gp.b;
  const int bk = b * KVH + kv;
  const int h0 = kv * GH;
  L_valid = gp.len;  // this sequence's valid length from here on
  const int t_begin = chunk * cs;
  const int t_end = (gp.b < 0) ? t_begin : min(gp.n_tiles, t_begin + cs);
  // ragged flash: S_per_tile from this sequence's tile count (flash/santa_cuda.cpp:204-208)
  if (seq_lens && MODE == kOnline)
    S_pt = (S_total > 0) ? static_cast<int>(max(1LL, S_total / static_cast<long long>(max(gp.n_tiles, 1)))) : 0;

  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform for the compiler

  __shared__ float s_sc[BN * GH];          // scores, [row][head]
  __shared__ uint16_t s_ub[GH * BN];       // 16-bit u, [head][row]
  // wave maxima as order keys, double-buffered by tile parity: a wave may
  // write the next tile's maxima (phase B, before that tile's first barrier)
  // while another still reads this tile's (phases C-D, after its last one)
  __shared__ int s_wmax2[2][4 * GH];
  __shared__ float s_W[NWS * GH];
  __shared__ uint64_t s_mask[GH * NPAIR * 2];

  // Addresses: a wave-uniform 64-bit base (SGPRs) plus a 32-bit per-lane byte
  // offset, so loads take the scalar-base form and need no 64-bit VALU math.
  // Paged: the base is the pool's (plus this KV head), rows go through pt.
  const size_t row_stride = static_cast<size_t>(KVH) * kD;
  const uint32_t row_bytes = static_cast<uint32_t>(KVH) * kD * 2u;
  const size_t seq_off = PAGED ? 0 : static_cast<size_t>(b) * L_storage * row_stride;
  const char* Kg = reinterpret_cast<const char*>(K + seq_off + static_cast<size_t>(kv) * kD);
  const char* Vg = reinterpret_cast<const char*>(V + seq_off + static_cast<size_t>(kv) * kD);
  const uint32_t v_lane_off = 4u * static_cast<uint32_t>(lane);  // dims 2*lane, 2*lane+1

  // Online-merge state: per head owned by this wave, running max M, mass Z
  // and this lane's two numerator dims.
  float runM[HPW], runZ[HPW], num0[HPW], num1[HPW];
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    runM[k] = -__builtin_inff();
    runZ[k] = 0.0f;
    num0[k] = 0.0f;
    num1[k] = 0.0f;
  }
  int emit_total = 0;

  if (t_begin >= t_end) {
    if constexpr (MODE == kOnline) {
#pragma unroll
      for (int k = 0; k < HPW; ++k) {
        float* pp = part + (static_cast<size_t>(wg) * GH + wave + 4 * k) * kPartStride;
        if (lane == 0) {
          pp[0] = -__builtin_inff();
          pp[1] = 0.0f;
        }
        pp[2 + 2 * lane] = 0.0f;
        pp[3 + 2 * lane] = 0.0f;
      }
      if (tid == 0) part_emit[wg] = 0;
    }
    return;
  }

  // ---- q of the group, scaled once (A.1): qa[hb][m] at lane 4j+i holds head
  // 4hb+i, dim 16m+j -- the broadcast A operand of the score MFMAs.
  constexpr int NHB = GH / 4;
  float qa[NHB][8];
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb) {
    const uint16_t* qh = Q + (static_cast<size_t>(b) * H + h0 + 4 * hb + (lane & 3)) * kD + (lane >> 2);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      qa[hb][m] = h16_to_f32<BF16>(qh[16 * m]) * q_scale;
      if constexpr (MODE == kPass1Gen) qa[hb][m] = h16_to_f32<BF16>(f32_to_h16<BF16>(qa[hb][m]));
    }
  }
  // K staging: wave w's 64 rows, row r chunk c (16 B) at slot r*16 + (c ^ (r & 15)).
  __shared__ u32x4 s_k[4 * 64 * 16];
  u32x4* const wk = s_k + wave * 64 * 16;
  __syncthreads();

  // Per-head sample lists: each wave owns its heads' lists, so appending and
  // gathering need no workgroup barrier.  Per-tile mode: (row, count) of the
  // current tile.  Online mode: (row, count * ell_t, m_t) until a flush.
  __shared__ float s_lm[(MODE == kOnline) ? GH * LCAP : 1];
  __shared__ float s_lcw[GH * LCAP];
  __shared__ int s_lrow[GH * LCAP];
  int lcnt[HPW];
  float numM[HPW];
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    lcnt[k] = 0;
    numM[k] = -__builtin_inff();
  }
  // num = sum over listed samples of count * ell_t * exp(m_t - M) * v_row,
  // with M the running max at flush time; earlier flushes are rescaled.
  auto flush = [&](int k, int g) {
    if (lcnt[k] == 0) return;
    const float Mf = runM[k];
    const float rs = santa_expf(numM[k] - Mf);
    num0[k] *= rs;
    num1[k] *= rs;
    numM[k] = Mf;
    for (int base = 0; base < lcnt[k]; base += 64) {
      // lane i prepares element base+i; the gather then walks the elements in
      // order with the row and coefficient broadcast from their lane
      const int i = base + lane;
      const bool ok = i < lcnt[k];
      const int rowv = ok ? s_lrow[g * LCAP + i] : 0;
      const float coefv = ok ? s_lcw[g * LCAP + i] * santa_expf(s_lm[g * LCAP + i] - Mf) : 0.0f;
      const int pgv = PAGED ? page_of_row(pt, b, rowv, ok) : 0;
      const int nb = min(64, lcnt[k] - base);
      for (int q0 = 0; q0 < nb; q0 += 16) {
        float coef[16];
        uint32_t vw[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int j = min(q0 + q, nb - 1);
          const int row = __builtin_amdgcn_readlane(rowv, j);
          coef[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(coefv), j));
          const size_t off = PAGED ? paged_row(pt, __builtin_amdgcn_readlane(pgv, j), row, row_bytes)
                                   : static_cast<size_t>(row) * row_bytes;
          vw[q] = *reinterpret_cast<const uint32_t*>(Vg + off + v_lane_off);
        }
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          if (q0 + q < nb) {
            num0[k] = fmaf(coef[q], lo16_to_f32<BF16>(vw[q]), num0[k]);
            num1[k] = fmaf(coef[q], hi16_to_f32<BF16>(vw[q]), num1[k]);
          }
        }
      }
    }
    lcnt[k] = 0;
  };

  // This wave's 64 rows of a tile: 16 buffer loads of 16 B per lane, 4 rows
  // each.  Load c reads rows 64w+4c .. 64w+4c+3 through its own descriptor
  // (base and record count in SGPRs); every lane's offset inside the 4-row
  // group is the same constant VGPR.  Rows at or past the tile's end are out
  // of the descriptor's range: they read as zero and cost no memory traffic,
  // so one unconditional call site covers short tiles, waves without rows and
  // the missing successor of a chunk's last tile (no branches, so the loaded
  // registers are never copied and no wait lands before the scores).
  // Paged: pv holds the pages of the wave's 64 rows of the tile (one per
  // lane), loaded a tile ahead; a 4-row group never straddles two pages.
  u32x4 kw[16];
  const int k_lane_off = static_cast<int>((lane >> 4) * row_bytes + 16u * (lane & 15));
  auto load_k = [&](int t, int pv) {
    const int n0 = t * BN;
    const int len = (t < t_end) ? min(BN, L_valid - n0) : 0;
    const char* kt = Kg + static_cast<size_t>(n0 + 64 * wave) * row_bytes;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      // wave-uniform; readfirstlane keeps the descriptor in SGPRs
      const int nvalid = __builtin_amdgcn_readfirstlane(min(max(len - 64 * wave - 4 * c, 0), 4));
      const char* gb;
      if constexpr (PAGED) {
        const int n = n0 + 64 * wave + 4 * c;
        const int page = __builtin_amdgcn_readlane(pv, (n >> pt.shift) - ((n0 + 64 * wave) >> pt.shift));
        gb = Kg + paged_row(pt, page, n, row_bytes);
      } else {
        gb = kt + static_cast<size_t>(4 * c) * row_bytes;
      }
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<char*>(gb), static_cast<short>(0), nvalid * static_cast<int>(row_bytes), kBufferWord3);
      kw[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, k_lane_off, 0, kBufferNontemporal));
    }
  };
  auto wave_pages = [&](int t) -> int {
    return PAGED ? pages_of_rows(pt, b, t * BN + 64 * wave, 64, L_valid, lane) : 0;
  };
  load_k(t_begin, wave_pages(t_begin));
  int pv_next = wave_pages(t_begin + 1);

  for (int t = t_begin; t < t_end; ++t) {
    const int n0 = t * BN;
    const int len = min(BN, L_valid - n0);
    int* const s_wmax = s_wmax2[(t - t_begin) & 1];

    // ---- A: scores -----------------------------------------------------------
    float lmax[GH];
#pragma unroll
    for (int g = 0; g < GH; ++g) lmax[g] = -__builtin_inff();
    const bool has_rows = 64 * wave < len;
    if (has_rows) {
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const int r = 4 * c + (lane >> 4);
        wk[r * 16 + ((lane & 15) ^ (r & 15))] = kw[c];
      }
    }
    // the next tile's rows stream in through this tile's scores and tail
    load_k(t + 1, pv_next);
    if constexpr (PAGED) pv_next = wave_pages(t + 2);
    // LDS operations of one wave complete in order; the barrier only keeps
    // the compiler from moving the reads above the writes
    __builtin_amdgcn_wave_barrier();
    if (has_rows) {
      // score = D_even + D_odd with C(c) = B(c) + B(c+2), D = C(0) + C(1)
      const int row = lane;
      f32x4 be0[NHB], bo0[NHB], be2[NHB], bo2[NHB], be1[NHB], bo1[NHB], be3[NHB], bo3[NHB];
      score_group<BF16, NHB, 0>(wk, row, qa, be0, bo0);
      score_group<BF16, NHB, 2>(wk, row, qa, be2, bo2);
      score_group<BF16, NHB, 1>(wk, row, qa, be1, bo1);
      score_group<BF16, NHB, 3>(wk, row, qa, be3, bo3);
      const int r = 64 * wave + row;
#pragma unroll
      for (int hb = 0; hb < NHB; ++hb) {
        const f32x4 de = (be0[hb] + be2[hb]) + (be1[hb] + be3[hb]);
        const f32x4 dd = (bo0[hb] + bo2[hb]) + (bo1[hb] + bo3[hb]);
        f32x4 sc = de + dd;  // heads 4hb .. 4hb+3 of row r
        if (BN == 256 || r < BN) reinterpret_cast<f32x4*>(s_sc + r * GH)[hb] = sc;
        // rows past len read as zero: they take no part in the max
        if (r >= len) sc = f32x4{-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
#pragma unroll
        for (int i = 0; i < 4; ++i) lmax[4 * hb + i] = sc[i];
      }
    }

    // ---- B: tile max per head (A.3) ------------------------------------------
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      const int mk = wave_max_key_lane63(order_key(lmax[g]));
      if (lane == 63) s_wmax[wave * GH + g] = mk;
    }
    __syncthreads();  // (1) scores and wave maxima visible
    if constexpr (MODE == kOnline) {
      // union of the previous tile's sampled rows: its masks were published
      // before barrier (1) and are rewritten only after barrier (2).
      if (wave == 0 && t > t_begin) emit_total += union_rows<GH, 2 * NPAIR>(s_mask, lane);
    }

    // ---- C: u, 16-bit u and ell partials (A.4) ---------------------------------
    if constexpr (MODE == kPass1Gen) {
      // thread (slab w, head g): the slab's 16 rows in order
      if (tid < NSLAB * GH) {
        const int g = tid % GH;
        const int w = tid / GH;
        const float mg = tile_max_of<GH>(s_wmax, g);
        float part_ell = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int r = 16 * w + j;
          if (r < len) {
            const float u = santa_expf(s_sc[r * GH + g] - mg);
            part_ell += u;
            s_ub[g * BN + r] = f32_to_h16<BF16>(u);
          }
        }
        s_W[w * GH + g] = part_ell;
      }
    } else if (tid < NT_REF) {
      // Thread tid plays the reference's thread tid: items idx = tid + NT_REF k,
      // valid while idx < len * GH (a prefix in k).  Invalid items add +0.
      const int g = tid % GH;
      const float mg = tile_max_of<GH>(s_wmax, g);
      float sv[KC];
#pragma unroll
      for (int k = 0; k < KC; ++k) sv[k] = s_sc[tid + NT_REF * k];
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        const int idx = tid + NT_REF * k;
        const float u = santa_expf(sv[k] - mg);
        acc += (idx < len * GH) ? u : 0.0f;
        s_ub[g * BN + idx / GH] = f32_to_h16<BF16>(u);
      }
      // the reference's 32-lane __shfl_down tree for lane g: pairs at lane
      // distance 16, 8, ... GH (the remaining levels only add +0).  Distance
      // 16 crosses 16-lane rows (permlane16 swap); 8 and 4 stay inside.
      {
        const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc), __float_as_uint(acc), false, false);
        acc = acc + __uint_as_float(sw[1]);  // lanes of rows 0 and 2 (the ones used)
      }
      if constexpr (GH <= 8) acc = acc + dpp_shl_zero<8>(acc);
      if constexpr (GH <= 4) acc = acc + dpp_shl_zero<4>(acc);
      if ((tid & 31) < GH) s_W[(tid >> 5) * GH + (tid & 31)] = acc;
    }
    __syncthreads();  // (2) 16-bit u and warp masses visible

    if constexpr (PASS1) {
      // tile statistics and the 16-bit u of every (row, head) of the group
#pragma unroll
      for (int k = 0; k < HPW; ++k) {
        const int g = wave + 4 * k;
        const float mg = tile_max_of<GH>(s_wmax, g);
        float ell = 0.0f;
#pragma unroll
        for (int w = 0; w < NWS; ++w) ell += s_W[w * GH + g];
        if (lane == 0) {
          const size_t mt = (static_cast<size_t>(b) * H + h0 + g) * T_c + t;
          m_tiles[mt] = mg;
          ell_tiles[mt] = ell;
        }
      }
      if (tid < len) {
        uint16_t* dst = u_stash + (static_cast<size_t>(b) * L_storage + n0 + tid) * H + h0;
        if constexpr (GH == 4) {
          uint2 w;
          w.x = s_ub[0 * BN + tid] | (static_cast<uint32_t>(s_ub[1 * BN + tid]) << 16);
          w.y = s_ub[2 * BN + tid] | (static_cast<uint32_t>(s_ub[3 * BN + tid]) << 16);
          *reinterpret_cast<uint2*>(dst) = w;
        } else {
          uint4 w;
          w.x = s_ub[0 * BN + tid] | (static_cast<uint32_t>(s_ub[1 * BN + tid]) << 16);
          w.y = s_ub[2 * BN + tid] | (static_cast<uint32_t>(s_ub[3 * BN + tid]) << 16);
          w.z = s_ub[4 * BN + tid] | (static_cast<uint32_t>(s_ub[5 * BN + tid]) << 16);
          w.w = s_ub[6 * BN + tid] | (static_cast<uint32_t>(s_ub[7 * BN + tid]) << 16);
          *reinterpret_cast<uint4*>(dst) = w;
        }
      }
      continue;
    }

    // ---- D/E: per-head counts, sample lists -------------------------------------
#pragma unroll
    for (int k = 0; k < HPW; ++k) {
      const int g = wave + 4 * k;
      const int h = h0 + g;
      const float mg = tile_max_of<GH>(s_wmax, g);
      float ell = 0.0f;
#pragma unroll
      for (int w = 0; w < NW_REF; ++w) ell += s_W[w * GH + g];
      const float invdel = (S_pt > 0 && ell > 1e-20f) ? (static_cast<float>(S_pt) / ell) : 0.0f;
      const float a0 = u01(seed, b * H + h, t);

      // rows two per lane, in the layout systematic_counts takes
      const int jrow = lane >> 4;
      const int qq = lane & 15;
      float x0[NPAIR], x1[NPAIR];
#pragma unroll
      for (int pp = 0; pp < NPAIR; ++pp) {
        const int row = 32 * (4 * pp + jrow) + 2 * qq;
        const uint32_t w2 = (BN >= 128 || row < BN) ? *reinterpret_cast<const uint32_t*>(s_ub + g * BN + row) : 0u;
        x0[pp] = (row < len && invdel > 0.0f) ? lo16_to_f32<BF16>(w2) * invdel : 0.0f;
        x1[pp] = (row + 1 < len && invdel > 0.0f) ? hi16_to_f32<BF16>(w2) * invdel : 0.0f;
      }
      int c0[NPAIR], c1[NPAIR];
      systematic_counts<NCH>(x0, x1, len, a0, lane, c0, c1);
      uint64_t nz0[NPAIR], nz1[NPAIR];
#pragma unroll
      for (int pp = 0; pp < NPAIR; ++pp) {
        const int row = 32 * (4 * pp + jrow) + 2 * qq;
        nz0[pp] = __ballot(c0[pp] != 0);
        nz1[pp] = __ballot(c1[pp] != 0);
        if (lane == 0) {
          s_mask[(g * NPAIR + pp) * 2 + 0] = nz0[pp];
          s_mask[(g * NPAIR + pp) * 2 + 1] = nz1[pp];
        }
        if constexpr (MODE == kPerTile) {
          if (dbg_counts && row < BN) {
            int16_t* dc = dbg_counts + ((static_cast<size_t>(b) * H + h) * T_c + t) * BN + row;
            dc[0] = static_cast<int16_t>(c0[pp]);
            dc[1] = static_cast<int16_t>(c1[pp]);
          }
        }
      }

      if constexpr (MODE == kOnline) {
        // running max and mass of the chunk
        if (mg > runM[k]) {
          runZ[k] = fmaf(runZ[k], santa_expf(runM[k] - mg), ell);
          runM[k] = mg;
        } else {
          runZ[k] = fmaf(santa_expf(mg - runM[k]), ell, runZ[k]);
        }
      }
      // Append the head's sampled rows in ascending order: (row, count[*ell_t], m_t).
      const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
      for (int pp = 0; pp < NPAIR; ++pp) {
        const int row = 32 * (4 * pp + jrow) + 2 * qq;
        if constexpr (MODE == kOnline) {
          // at most 128 new rows per register pair; the list holds that many
          if (lcnt[k] + __popcll(nz0[pp]) + __popcll(nz1[pp]) > LCAP) flush(k, g);
        }
        const int pos0 = lcnt[k] + __popcll(nz0[pp] & below) + __popcll(nz1[pp] & below);
        const int pos1 = pos0 + (c0[pp] != 0 ? 1 : 0);
        if (c0[pp] != 0) {
          s_lrow[g * LCAP + pos0] = n0 + row;
          s_lcw[g * LCAP + pos0] = (MODE == kOnline) ? static_cast<float>(c0[pp]) * ell : static_cast<float>(c0[pp]);
          if constexpr (MODE == kOnline) s_lm[g * LCAP + pos0] = mg;
        }
        if (c1[pp] != 0) {
          s_lrow[g * LCAP + pos1] = n0 + row + 1;
          s_lcw[g * LCAP + pos1] = (MODE == kOnline) ? static_cast<float>(c1[pp]) * ell : static_cast<float>(c1[pp]);
          if constexpr (MODE == kOnline) s_lm[g * LCAP + pos1] = mg;
        }
        lcnt[k] += __popcll(nz0[pp]) + __popcll(nz1[pp]);
      }

      if constexpr (MODE == kPerTile) {
        // count-weighted V sum over the head's sampled rows, ascending, one fma
        // per element (flash/santa_cuda_kernel.cu:347-379)
        float acc0 = 0.0f, acc1 = 0.0f;
        for (int base = 0; base < lcnt[k]; base += 8) {
          float cf[8];
          uint32_t vw[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const int i = min(base + q, lcnt[k] - 1);
            const int rr = __builtin_amdgcn_readfirstlane(s_lrow[g * LCAP + i]);
            cf[q] = s_lcw[g * LCAP + i];
            vw[q] = *reinterpret_cast<const uint32_t*>(Vg + static_cast<size_t>(rr) * row_bytes + v_lane_off);
          }
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            if (base + q < lcnt[k]) {
              acc0 = fmaf(cf[q], lo16_to_f32<BF16>(vw[q]), acc0);
              acc1 = fmaf(cf[q], hi16_to_f32<BF16>(vw[q]), acc1);
            }
          }
        }
        lcnt[k] = 0;
        const size_t mt = (static_cast<size_t>(b) * H + h) * T_c + t;
        if (lane == 0) {
          m_tiles[mt] = mg;
          ell_tiles[mt] = ell;
        }
        reinterpret_cast<float2*>(out_tiles + mt * kD)[lane] = make_float2(acc0, acc1);
      }
    }

    if constexpr (MODE == kPerTile) {
      // rows sampled by any head of the group -> emit_cnt
      __syncthreads();
      if (wave == 0) {
        const int e = union_rows<GH, 2 * NPAIR>(s_mask, lane);
        if (lane == 0) emit_cnt[static_cast<size_t>(bk) * T_c + t] = e;
      }
    }
  }

  if constexpr (MODE == kOnline) {
    __syncthreads();  // last tile's masks visible
    if (wave == 0) emit_total += union_rows<GH, 2 * NPAIR>(s_mask, lane);
#pragma unroll
    for (int k = 0; k < HPW; ++k) flush(k, wave + 4 * k);
#pragma unroll
    for (int k = 0; k < HPW; ++k) {
      float* pp = part + (static_cast<size_t>(wg) * GH + wave + 4 * k) * kPartStride;
      if (lane == 0) {
        pp[0] = runM[k];
        pp[1] = runZ[k];
      }
      pp[2 + 2 * lane] = num0[k];
      pp[3 + 2 * lane] = num1[k];
    }
    if (tid == 0) part_emit[wg] = emit_total;
  }
}

// ------------------------------------------------------------- wave kernel
// santa_flash tiles of block_n = 256, online mode, with each wave64 owning
// whole tiles: wave w of a workgroup takes tiles t_begin + w, t_begin + w + 4,
// ... of the chunk, so the four waves never wait for one another until the
// chunk ends.  A tile is scored in four 64-row sub-blocks (hh, e) = (0,0),
// (0,1), (1,0), (1,1); lane 16j+q of sub-block (hh, e) owns row
// 128hh + 32j + 2q + e.  That is the two-rows-per-lane layout of
// systematic_counts (register pair hh, element e), so scores, u, the 16-bit
// u, x and the counts never leave registers; only the sub-block staging of K
// (the row-per-lane transpose for the MFMA operand) and the sampled-row
// lists use LDS.  Each sub-block load takes 4 rows of stride 2 (16 lanes x
// 16 B per row, still 256 contiguous bytes per row); the loads of the next
// sub-block are issued before the current one is scored.
//
// Statistics are bit-identical to tile_kernel's (the reference's): the tile
// max is exact in any order, and ell keeps the reference thread / 32-lane
// tree / warp association (flash/santa_cuda_kernel.cu:243-273), rebuilt from
// this layout with cross-row swaps and DPP.  The output merge differs only
// in rounding: a sampled row's coefficient c * ell_t * exp(m_t - M) is formed
// when the row is listed, relative to the wave's running max M, and listed
// coefficients are rescaled in place when M grows.  The four waves' partials
// are merged in wave order at the end of the chunk.
constexpr int kWaveListCap = 64;  // listed rows per head (one per lane)

// The value of lane i + 16 in the even 16-lane rows (rows 0, 2; the odd rows
// get their own value back): the second result of the row swap of v with
// itself.  The callers read it in the even rows only.
template <int N>
__device__ __forceinline__ float xrow16(float v) {
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(s[1]);
}
// The value of lane i + 32 in lanes 0..31 (lanes 32..63 get their own value
// back): the second result of the half-wave swap of v with itself.  The
// callers read it in lanes 0..31 only.
__device__ __forceinline__ float xhalf32(float v) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(s[1]);
}

// ell of one head from its u values (u[hh][e] at this lane; 0 past len),
// with the reference's association for block_n = 256 (256 reference
// threads; thread tau = GH * rho + g sums rows rho + (256 / GH) k in order k,
// then per 32-thread warp a shfl_down tree of distances 16, 8, ... GH, then
// the warps in order).
template <int GH>
__device__ __forceinline__ float wave_ell(const float (&u)[2][2]) {
  float A[2];
  if constexpr (GH == 4) {
    // rows rho' + 64 k: k = 0..3 -> (hh 0, row block j), (hh 0, j + 2),
    // (hh 1, j), (hh 1, j + 2); valid in lanes 0..31
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      float a = u[0][e] + xhalf32(u[0][e]);
      a = a + u[1][e];
      A[e] = a + xhalf32(u[1][e]);
    }
    // warp w = lanes 4w .. 4w+3: ((A0 + A4) + (A2 + A6)) + ((A1 + A5) + (A3 + A7)),
    // A_m = A[m % 2] at lane 4w + m / 2
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      A[e] = A[e] + dpp_shl_zero<2>(A[e]);
      A[e] = A[e] + dpp_shl_zero<1>(A[e]);
    }
    const float W = A[0] + A[1];
    float ell = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(W), 0));
#pragma unroll
    for (int w = 1; w < 8; ++w) ell = ell + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(W), 4 * w));
    return ell;
  } else {
    // rows rho'' + 32 k: k = 0..7 -> (hh 0, j = 0..3), (hh 1, j = 0..3); lanes 0..15
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      float a = 0.0f;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const float v = u[hh][e];
        const float v16 = xrow16<0>(v);
        a = (hh == 0) ? v : a + v;
        a = a + v16;
        a = a + xhalf32(v);
        a = a + xhalf32(v16);
      }
      A[e] = a;
    }
    // warp w = lanes 2w, 2w+1: (A0 + A2) + (A1 + A3), A_m = A[m % 2] at lane 2w + m / 2
#pragma unroll
    for (int e = 0; e < 2; ++e) A[e] = A[e] + dpp_shl_zero<1>(A[e]);
    const float W = A[0] + A[1];
    float ell = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(W), 0));
#pragma unroll
    for (int w = 1; w < 8; ++w) ell = ell + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(W), 2 * w));
    return ell;
  }
}

// ell of four heads with the general path's association: the reference's
// WMMA pass 1 sums each head's u over a 16-row slab in row order, then the
// slabs in order (prop/santa_cuda_kernel.cu:225-262).  In the wave layout a
// slab is 8 consecutive lanes of one register pair, so the u values go
// through LDS (two regions of this wave's sample-list area, which pass 1
// leaves unused): head k's 256 values at fa_k[row], fa_k = (k < 2 ? fa01 :
// fa23) + 256 (k & 1).  Then lane 16k + w sums slab w of head k in row
// order, and lane k sums head k's 16 slab sums in slab order.  Rows past the
// tile's end hold u = 0, which adds exactly.
__device__ __forceinline__ void slab_ell4(const float (&u)[4][2][2], float* fa01, float* fa23, int lane,
                                          float (&ell)[4]) {
  const int jrow = lane >> 4, qq = lane & 15;
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
      *reinterpret_cast<float2*>((k < 2 ? fa01 : fa23) + 256 * (k & 1) + 128 * hh + 32 * jrow + 2 * qq) =
          make_float2(u[k][hh][0], u[k][hh][1]);
  __builtin_amdgcn_wave_barrier();
  const int ks = lane >> 4;
  const float4* src = reinterpret_cast<const float4*>((ks < 2 ? fa01 : fa23) + 256 * (ks & 1) + 16 * (lane & 15));
  const float4 a = src[0], b = src[1], c = src[2], d = src[3];
  float p = a.x;
  p = p + a.y;
  p = p + a.z;
  p = p + a.w;
  p = p + b.x;
  p = p + b.y;
  p = p + b.z;
  p = p + b.w;
  p = p + c.x;
  p = p + c.y;
  p = p + c.z;
  p = p + c.w;
  p = p + d.x;
  p = p + d.y;
  p = p + d.z;
  p = p + d.w;
  // every lane's reads have returned (p needs all of them), so the slab sums
  // may overwrite the start of head 0's values
  __builtin_amdgcn_wave_barrier();
  fa01[lane] = p;
  __builtin_amdgcn_wave_barrier();
  const float4* s2 = reinterpret_cast<const float4*>(fa01 + 16 * (lane & 3));
  const float4 e0 = s2[0], e1 = s2[1], e2 = s2[2], e3 = s2[3];
  float e = e0.x;
  e = e + e0.y;
  e = e + e0.z;
  e = e + e0.w;
  e = e + e1.x;
  e = e + e1.y;
  e = e + e1.z;
  e = e + e1.w;
  e = e + e2.x;
  e = e + e2.y;
  e = e + e2.z;
  e = e + e2.w;
  e = e + e3.x;
  e = e + e3.y;
  e = e + e3.z;
  e = e + e3.w;
#pragma unroll
  for (int k = 0; k < 4; ++k) ell[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), k));
  __builtin_amdgcn_wave_barrier();
}

// P1: santa_prop pass 1 -- for GH 4 with the vec path's numerics (the flash
// tile statistics), for GH 8 with the general path's (q rounded after
// scaling, ell per 16-row slab): per tile and head m and ell into dbg_m /
// dbg_ell ([B, H, T_c])
// and the 16-bit u into u_stash ([B, L_storage, H]); no sampling, no partials.
// ROWS: a workgroup of KVH waves (KVH <= 8), wave kv taking KV head kv over
// every tile of the workgroup's chunk, so the KV heads of a token chunk are
// read together, row by row, by one CU; each wave writes its own chunk
// partial.  Otherwise four waves share one KV head, taking every fourth
// tile, and merge their partials at the end of the chunk.
template <bool BF16, int GH, bool DBG, bool P1 = false, bool PAGED = false, bool ROWS = false>
__global__ __launch_bounds__(ROWS ? 512 : kThreads, ROWS ? 1 : 2) void wave_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V, int H, int KVH,
    int L_valid, int L_storage, int T_c, int cs, int cpg, float q_scale, int S_pt, uint64_t seed,
    float* __restrict__ part, int* __restrict__ part_emit, const int* __restrict__ seq_lens, int B, long long S_total,
    float* __restrict__ dbg_m, float* __restrict__ dbg_ell, int16_t* __restrict__ dbg_counts,
    uint16_t* __restrict__ u_stash, int stash_ld, PageTable pt, int stash_nt, int kv_div) {
  constexpr int BN = 256;
  constexpr int NHB = GH / 4;
  constexpr int LCAP = kWaveListCap;
  const int wg = static_cast<int>(blockIdx.x);
  // uniform grid, or the ragged one (seq_lens: per-sequence lengths, L_valid
  // the longest; workgroups past the last sequence only write an empty
  // partial)
  constexpr int NWV = ROWS ? 8 : 4;  // waves per workgroup (at most)
  constexpr int TS = ROWS ? 1 : 4;    // tile stride of a wave
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // ROWS workgroups enumerate (sequence, chunk) items (grid_pos with one
  // "head"); the KV head is the wave
  const GridPos gp = grid_pos(wg, seq_lens, B, ROWS ? 1 : KVH, BN, L_valid, T_c, cs, cpg);
  const int kv = ROWS ? wave : gp.kv;
  const int b = gp.b < 0 ? 0 : gp.b;
  // heads per KV head: GH, except that santa_prop's pass 1 at GH 8 also takes
  // groups of 5-7 heads (santa_prop's generic shapes at D = 128), the second
  // head block's last heads then zero and never written (tile-major stash only)
  const int gsz = (P1 && GH == 8) ? H / KVH : GH;
  const int h0 = kv * gsz;
  L_valid = gp.len;
  const int t_begin = gp.chunk * cs;
  const int t_end = (gp.b < 0) ? t_begin : min(gp.n_tiles, t_begin + cs);
  if (seq_lens)  // S_per_tile from this sequence's tile count (flash/santa_cuda.cpp:204-208)
    S_pt = (S_total > 0) ? static_cast<int>(max(1LL, S_total / static_cast<long long>(max(gp.n_tiles, 1)))) : 0;
  const int t_first = ROWS ? t_begin : t_begin + wave;

  __shared__ u32x4 s_k[NWV * 64 * 16];  // per wave: 64 rows x 256 B staging; the chunk merge reuses it
  __shared__ int2 s_list[NWV * GH * LCAP];  // (row, coefficient bits) per listed row
  u32x4* const wk = s_k + wave * 64 * 16;
  int2* const list = s_list + wave * GH * LCAP;

  // Paged: the base is the pool's (plus this KV head), rows go through pt.
  // kv_div > 1 (santa_prop's pass 1 at GH 10-16): KVH counts virtual KV heads,
  // kv_div of them per cache KV head, each taking 8 of its query heads; wave
  // kv reads the rows of cache KV head kv / kv_div (1 everywhere else).
  const int kvc = kv / kv_div;
  const size_t row_stride = static_cast<size_t>(KVH / kv_div) * kD;
  const uint32_t row_bytes = static_cast<uint32_t>(KVH / kv_div) * kD * 2u;
  const size_t seq_off = PAGED ? 0 : static_cast<size_t>(b) * L_storage * row_stride;
  const char* Kg = reinterpret_cast<const char*>(K + seq_off + static_cast<size_t>(kvc) * kD);
  const char* Vg = reinterpret_cast<const char*>(V + seq_off + static_cast<size_t>(kvc) * kD);
  const uint32_t v_lane_off = 4u * static_cast<uint32_t>(lane);

  float qa[NHB][8];
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb) {
    const int gq = 4 * hb + (lane & 3);
    const uint16_t* qh = Q + (static_cast<size_t>(b) * H + h0 + min(gq, gsz - 1)) * kD + (lane >> 2);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      qa[hb][m] = (gq < gsz) ? h16_to_f32<BF16>(qh[16 * m]) * q_scale : 0.0f;
      // pass 1 of GH 8 is santa_prop's general path: q rounded to the 16-bit
      // type after scaling (prop/santa_cuda_kernel.cu:121-140)
      if constexpr (P1 && GH == 8) qa[hb][m] = h16_to_f32<BF16>(f32_to_h16<BF16>(qa[hb][m]));
    }
  }

  float runM[GH], runZ[GH], num0[GH], num1[GH];
  int lcnt[GH];
#pragma unroll
  for (int g = 0; g < GH; ++g) {
    runM[g] = -__builtin_inff();
    runZ[g] = 0.0f;
    num0[g] = 0.0f;
    num1[g] = 0.0f;
    lcnt[g] = 0;
  }
  int emit_total = 0;

  // Gathers of listed rows: lane i holds the V row address of list entry i
  // (computed for all entries at once), and entry j's row is loaded through
  // that address read back as a scalar base, the lane's 4 B at v_lane_off.
  auto v_addr = [&](int rowv, bool ok) -> uint64_t {
    if constexpr (PAGED) {
      return reinterpret_cast<uint64_t>(Vg + paged_row(pt, page_of_row(pt, b, rowv, ok), rowv, row_bytes));
    } else {
      return reinterpret_cast<uint64_t>(Vg + static_cast<size_t>(rowv) * row_bytes);
    }
  };
  auto v_load = [&](uint64_t av, int j) -> uint32_t {
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(av), j);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(av >> 32), j);
    typedef const __attribute__((address_space(1))) char* gbytes;
    const gbytes row = reinterpret_cast<gbytes>((static_cast<uint64_t>(hi) << 32) | lo);
    return *reinterpret_cast<const __attribute__((address_space(1))) uint32_t*>(row + v_lane_off);
  };
  // entry q0 + q of a list of n into the numerator (a selected update, so the
  // loads past n -- repeats of entry n - 1 -- are consumed but change nothing)
  auto accumulate = [&](int g, float coefv, const uint32_t (&vw)[16], int q0, int n) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(coefv), min(q0 + q, n - 1)));
      const float a0 = fmaf(c, lo16_to_f32<BF16>(vw[q]), num0[g]);
      const float a1 = fmaf(c, hi16_to_f32<BF16>(vw[q]), num1[g]);
      const bool ok = q0 + q < n;
      num0[g] = ok ? a0 : num0[g];
      num1[g] = ok ? a1 : num1[g];
    }
  };

  // the listed rows of head g, in list order, into the numerator
  auto flush = [&](int g) {
    const int n = lcnt[g];
    if (n <= 0) return;
    const int2 ent = (lane < n) ? list[g * LCAP + lane] : make_int2(0, 0);
    const uint64_t av = v_addr(ent.x, lane < n);
    const float coefv = __int_as_float(ent.y);
    int q0 = 0;
    do {
      uint32_t vw[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) vw[q] = v_load(av, min(q0 + q, n - 1));
      accumulate(g, coefv, vw, q0, n);
      q0 += 16;
    } while (q0 < n);
    lcnt[g] = 0;
  };

  // Sub-block sb = 2 hh + e of tile t: 16 loads of 4 rows (stride 2), one
  // descriptor each; rows at or past the tile's end (and every row of a tile
  // at or past t_end) read as zero and cost no traffic.  A load's rows lie in
  // one 8-row aligned block, so in a paged cache in one page: pv holds the
  // tile's pages, one per lane.
  u32x4 kw[16];
  const int k_lane_off = static_cast<int>((lane >> 4) * 2u * row_bytes + 16u * (lane & 15));
  auto group_base = [&](int t, int r, int pv) -> const char* {  // row t*BN + r, first of its load group
    const int n = t * BN + r;
    if constexpr (PAGED) {
      const int page = __builtin_amdgcn_readlane(pv, (n >> pt.shift) - ((t * BN) >> pt.shift));
      return Kg + paged_row(pt, page, n, row_bytes);
    } else {
      return Kg + static_cast<size_t>(n) * row_bytes;
    }
  };
  auto tile_pages = [&](int t) -> int {
    return PAGED ? pages_of_rows(pt, b, t * BN, BN, L_valid, lane) : 0;
  };
  auto load_k = [&](int t, int sb, int pv) {
    const uint32_t rb = row_bytes;
    const int len = (t < t_end) ? min(BN, L_valid - t * BN) : 0;
    const int r0 = 128 * (sb >> 1) + (sb & 1);
    const char* kt = Kg + static_cast<size_t>(t * BN + r0) * rb;
    // rows of the sub-block's stride-2 run still valid, wave-uniform (one
    // readfirstlane, then scalar arithmetic per load)
    const int rem = __builtin_amdgcn_readfirstlane(len - r0);
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const int nvalid = min(max(rem - 8 * c, 0), 8);
      const char* gb = PAGED ? group_base(t, r0 + 8 * c, pv) : kt + static_cast<size_t>(8 * c) * rb;
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<char*>(gb), static_cast<short>(0), nvalid * static_cast<int>(rb), kBufferWord3);
      kw[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, k_lane_off, 0, kBufferNontemporal));
    }
  };
  // Sub-block 0 of tile t straight into the staging area (buffer loads to LDS;
  // no registers held while in flight), in the staged layout: the load of
  // rows 4c .. 4c+3 fills slots 64c .. 64c+63 in lane order, so lane 16j + p
  // fetches the 16-B piece p ^ ((4c + j) & 15) of row 4c + j.  The caller
  // waits (vmcnt) before reading the rows and issues it only once the area's
  // previous rows have been read.
  uint32_t k_dma_off[4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
    k_dma_off[m] = (lane >> 4) * 2u * row_bytes + 16u * static_cast<uint32_t>((lane & 15) ^ (4 * m + (lane >> 4)));
  auto dma_k = [&](int t, int pv) {
    const uint32_t rb = row_bytes;
    const int len = min(BN, L_valid - t * BN);
    const char* kt = Kg + static_cast<size_t>(t * BN) * rb;
    const int rem = __builtin_amdgcn_readfirstlane(len);
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const int nvalid = min(max(rem - 8 * c, 0), 8);
      const char* gb = PAGED ? group_base(t, 8 * c, pv) : kt + static_cast<size_t>(8 * c) * rb;
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<char*>(gb), static_cast<short>(0), nvalid * static_cast<int>(rb), kBufferWord3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(wk + 64 * c), 16,
                                               k_dma_off[c & 3], 0, 0, kBufferNontemporal);
    }
  };
  // pv: pages of the current tile; pv_next: of the wave's next tile (loaded
  // while the current one is scored)
  int pv = tile_pages(t_first);
  int pv_next = 0;
  if (t_first < t_end) dma_k(t_first, pv);
  load_k(t_first, 1, pv);

  const int jrow = lane >> 4;
  const int qq = lane & 15;
  // ROWS: waves w and w ^ 4 share a SIMD and walk the same tiles.  Left to
  // the oldest-first issue order, waves 0-3 would end their loops about
  // 14 us (at 32k tokens, 4 tiles per wave) before waves 4-7 and leave half
  // of each SIMD idle meanwhile.  Each wave publishes a checkpoint count
  // three times per tile (tile start, sub-block 2, scores done) and the one
  // behind takes the higher issue priority.  (More checkpoints cost more in
  // LDS waits than they balance.)  GH 8 has no LDS left for the counts and
  // alternates the favour by tile parity (below).
  constexpr bool PRIO = ROWS && GH == 4;
  __shared__ int s_prog[PRIO ? 8 : 1];
  if constexpr (PRIO) {
    if (lane == 0) s_prog[wave] = 0;
    __syncthreads();
  }
  auto balance = [&](int c) {
    if constexpr (PRIO) {
      if (lane == 0) s_prog[wave] = c;
      const int pc = __builtin_amdgcn_readfirstlane(s_prog[wave ^ 4]);
      if (c < pc) {
        __builtin_amdgcn_s_setprio(2);
      } else {
        __builtin_amdgcn_s_setprio(0);
      }
    }
  };
  for (int t = t_first; t < t_end; t += TS) {
    const int n0 = t * BN;
    const int len = min(BN, L_valid - n0);
    if constexpr (ROWS && GH == 8) {
      // no LDS for the checkpoint counts: the favour alternates by tile
      // parity instead (waves 4-7 on even tiles, 0-3 on odd ones), so that
      // neither SIMD partner keeps the lead the issue order gives it
      if ((t + (wave >> 2)) & 1) {
        __builtin_amdgcn_s_setprio(1);
      } else {
        __builtin_amdgcn_s_setprio(0);
      }
    }
    balance(3 * (t - t_first));

    // ---- scores of the four sub-blocks -------------------------------------
    f32x4 sc[2][2][NHB];
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      if (sb == 0) {
        // sub-block 0 came by DMA; for GH 8 the 16 register loads of
        // sub-block 1 were issued after it (and may still be in flight)
        if constexpr (GH == 4) {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } else {
          asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        }
        if constexpr (PAGED) pv_next = tile_pages(t + TS);
      } else {
#pragma unroll
        for (int c = 0; c < 16; ++c) {
          const int r = 4 * c + (lane >> 4);
          wk[r * 16 + ((lane & 15) ^ (r & 15))] = kw[c];
        }
        // sub-blocks 2, 3, then the next tile's sub-block 1 (GH 4; GH 8 loads
        // it after the next tile's DMA, below)
        if (sb < 3) {
          load_k(t, sb + 1, pv);
        } else if constexpr (GH == 4) {
          load_k(t + TS, 1, pv_next);
        }
        if (sb == 2) balance(3 * (t - t_first) + 1);
      }
      __builtin_amdgcn_wave_barrier();
      const int row = lane;
      if constexpr (NHB == 1) {
        f32x4 be0[NHB], bo0[NHB], be2[NHB], bo2[NHB], be1[NHB], bo1[NHB], be3[NHB], bo3[NHB];
        score_group<BF16, NHB, 0>(wk, row, qa, be0, bo0);
        score_group<BF16, NHB, 2>(wk, row, qa, be2, bo2);
        score_group<BF16, NHB, 1>(wk, row, qa, be1, bo1);
        score_group<BF16, NHB, 3>(wk, row, qa, be3, bo3);
        const f32x4 de = (be0[0] + be2[0]) + (be1[0] + be3[0]);
        const f32x4 dd = (bo0[0] + bo2[0]) + (bo1[0] + bo3[0]);
        sc[sb >> 1][sb & 1][0] = de + dd;
        pin(sc[sb >> 1][sb & 1][0]);
      } else {
        // one head block at a time: the staged rows are read once per block
        // rather than holding every block's accumulators
#pragma unroll
        for (int hb = 0; hb < NHB; ++hb) {
          f32x4 be0, bo0, be2, bo2, be1, bo1, be3, bo3;
          score_group1<BF16, 0>(wk, row, qa[hb], be0, bo0);
          score_group1<BF16, 2>(wk, row, qa[hb], be2, bo2);
          score_group1<BF16, 1>(wk, row, qa[hb], be1, bo1);
          score_group1<BF16, 3>(wk, row, qa[hb], be3, bo3);
          sc[sb >> 1][sb & 1][hb] = ((be0 + be2) + (be1 + be3)) + ((bo0 + bo2) + (bo1 + bo3));
          pin(sc[sb >> 1][sb & 1][hb]);
        }
      }
    }

    // every row of the staging area has been read: the next tile's sub-block 0
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (t + TS < t_end) dma_k(t + TS, pv_next);
    // GH 8: the next tile's sub-block 1 too, so that 32 KiB per wave are in
    // flight during the tail as for GH 4 (its registers fit beside the tail's)
    if constexpr (GH == 8) load_k(t + TS, 1, pv_next);
    balance(3 * (t - t_first) + 2);

    // ---- tile max per head (exact in any order) --------------------------------
    bool valid[2][2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int e = 0; e < 2; ++e) valid[hh][e] = 128 * hh + 32 * jrow + 2 * qq + e < len;
    float mg[GH];
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      int k = -2147483647 - 1;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int e = 0; e < 2; ++e)
          if (valid[hh][e]) k = max(k, order_key(sc[hh][e][g >> 2][g & 3]));
      k = wave_max_key_lane63(k);
      mg[g] = from_order_key(__builtin_amdgcn_readlane(k, 63));
    }

    // ---- per block of four heads: u, ell, counts, running max, sampled rows -----
    // Each step runs for the block's four heads side by side with no branch, so
    // their dependency chains interleave; only the list appends are sequential.
    uint64_t uni[2][2] = {{0, 0}, {0, 0}};
    uint32_t ubits[P1 ? GH : 1][2][2];  // pass 1: the 16-bit u of this lane's rows
    // (a lambda per block index, so both blocks of GH 8 are emitted unrolled:
    // the per-head state stays in registers)
    auto head_block = [&](auto hbc) {
      constexpr int hb = decltype(hbc)::value;
      float u[4][2][2], ub[4][2][2];
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            // s - m <= 0 for the rows that take part (inputs are finite);
            // rows past len take 0 in place of s - m and give u = 0
            const float d = sc[hh][e][hb][k] - mg[4 * hb + k];
            const float ex = santa_expf_nonpos(valid[hh][e] ? d : 0.0f);
            u[k][hh][e] = valid[hh][e] ? ex : 0.0f;
            ub[k][hh][e] = round16_nonneg<BF16>(u[k][hh][e]);
          }
      float ell[4];
      if constexpr (P1 && GH == 8) {
        slab_ell4(u, reinterpret_cast<float*>(list), reinterpret_cast<float*>(list) + GH * LCAP, lane, ell);
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) ell[k] = wave_ell<GH>(u[k]);
      }
      if constexpr (P1) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const size_t mt = (static_cast<size_t>(b) * H + h0 + 4 * hb + k) * T_c + t;
          if (lane == 0 && 4 * hb + k < gsz) {
            dbg_m[mt] = mg[4 * hb + k];
            dbg_ell[mt] = ell[k];
          }
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int e = 0; e < 2; ++e)
              ubits[4 * hb + k][hh][e] =
                  BF16 ? (__float_as_uint(ub[k][hh][e]) >> 16) : static_cast<uint32_t>(f32_to_h16<false>(u[k][hh][e]));
        }
        return;
      }
      // u (so the 16-bit u) is 0 past len and invdel is finite and >= 0, so
      // x = ub * invdel is the reference's 0 there without a select
      float x0[4][2], x1[4][2], a0[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float invdel = (S_pt > 0 && ell[k] > 1e-20f) ? (static_cast<float>(S_pt) / ell[k]) : 0.0f;
        a0[k] = u01(seed, b * H + h0 + 4 * hb + k, t);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          x0[k][hh] = ub[k][hh][0] * invdel;
          x1[k][hh] = ub[k][hh][1] * invdel;
        }
      }
      // cnt[k][0] / cnt[k][1] are the e = 0 / e = 1 rows of register pairs hh = 0, 1
      int cnt[4][2][2];
      if (len == BN) {
#pragma unroll
        for (int k = 0; k < 4; ++k) systematic_counts_full<8>(x0[k], x1[k], a0[k], lane, cnt[k][0], cnt[k][1]);
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) systematic_counts<8>(x0[k], x1[k], len, a0[k], lane, cnt[k][0], cnt[k][1]);
      }
      if constexpr (DBG) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const size_t mt = (static_cast<size_t>(b) * H + h0 + 4 * hb + k) * T_c + t;
          if (lane == 0) {
            dbg_m[mt] = mg[4 * hb + k];
            dbg_ell[mt] = ell[k];
          }
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            int16_t* dc = dbg_counts + mt * BN + 128 * hh + 32 * jrow + 2 * qq;
            dc[0] = static_cast<int16_t>(cnt[k][0][hh]);
            dc[1] = static_cast<int16_t>(cnt[k][1][hh]);
          }
        }
      }

      // running max and mass; a sampled row's coefficient is c * f, relative to
      // the running max.  When the max grows, the numerator and the listed
      // coefficients are rescaled by exp(old - new).
      float f[4], rsc[4];
      bool grow[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int g = 4 * hb + k;
        grow[k] = mg[g] > runM[g];
        const float ex = santa_expf(grow[k] ? runM[g] - mg[g] : mg[g] - runM[g]);
        runZ[g] = grow[k] ? fmaf(runZ[g], ex, ell[k]) : fmaf(ex, ell[k], runZ[g]);
        num0[g] = grow[k] ? num0[g] * ex : num0[g];
        num1[g] = grow[k] ? num1[g] * ex : num1[g];
        f[k] = grow[k] ? ell[k] : ell[k] * ex;
        rsc[k] = ex;
        runM[g] = grow[k] ? mg[g] : runM[g];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int g = 4 * hb + k;
        if (grow[k] && lane < lcnt[g]) {
          int* const cw = &list[g * LCAP + lane].y;
          *cw = __float_as_int(__int_as_float(*cw) * rsc[k]);
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int c = cnt[k][e][hh];
            const uint64_t nz = __ballot(c != 0);
            uni[hh][e] |= nz;
            const int nn = __popcll(nz);
            if (nn) {
              // a full list is rare (about once per chunk and head at
              // S_per_tile = 1): the gather is laid out off the hot path, so
              // the loop's hot code stays contiguous in the instruction cache
              if (__builtin_expect(lcnt[g] + nn > LCAP, 0)) flush(g);
              if (c != 0) {
                const int pos = lcnt[g] + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                              static_cast<uint32_t>(nz >> 32),
                                              __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(nz), 0u)));
                list[g * LCAP + pos] =
                    make_int2(n0 + 128 * hh + 32 * jrow + 2 * qq + e, __float_as_int(static_cast<float>(c) * f[k]));
              }
              lcnt[g] += nn;
            }
          }
      }
    };
    head_block(std::integral_constant<int, 0>{});
    if constexpr (NHB == 2) head_block(std::integral_constant<int, 1>{});
    if (P1 && stash_ld > 0) {
      // tile-major stash [B, T, H, 256] (T = stash_ld / 256): per head and
      // register pair, the lane's two rows as one 4-B store (whole tiles, 0
      // past len).  The KV heads of a tile write one contiguous block (GH 8:
      // the cfg5-shaped prop step 2058 -> 1983 us against the head-major
      // [B, H, stash_ld], whose per-head rows lie stash_ld * 2 bytes apart)
      if (stash_nt) {
        // non-temporal: buffer stores with the nt bit through one descriptor
        // over this sequence's stash (a separate instruction form, so the two
        // branches cannot be merged into one store that drops the hint)
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            u_stash + static_cast<size_t>(b) * H * stash_ld, static_cast<short>(0), H * stash_ld * 2, kBufferWord3);
#pragma unroll
        for (int g = 0; g < GH; ++g)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
            if (g < gsz)
              __builtin_amdgcn_raw_buffer_store_b32(
                  ubits[g][hh][0] | (ubits[g][hh][1] << 16), rs,
                  2 * (((t * H + h0 + g) * BN) + 128 * hh + 32 * jrow + 2 * qq), 0, kBufferNontemporal);
      } else {
#pragma unroll
        for (int g = 0; g < GH; ++g)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
            if (g < gsz)
              *reinterpret_cast<uint32_t*>(u_stash + static_cast<size_t>(b) * H * stash_ld +
                                           (static_cast<size_t>(t) * H + h0 + g) * BN + 128 * hh + 32 * jrow +
                                           2 * qq) = ubits[g][hh][0] | (ubits[g][hh][1] << 16);
      }
    } else if constexpr (P1) {
      // the stash row [n, h0 .. h0+GH) of each valid row: one 8-B (GH 4) or
      // 16-B (GH 8) store (whole groups only: the launcher takes groups of 5-7
      // heads with the tile-major stash alone)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          if (valid[hh][e]) {
            uint16_t* dst = u_stash + (static_cast<size_t>(b) * L_storage + n0 + 128 * hh + 32 * jrow + 2 * qq + e) * H + h0;
            if constexpr (GH == 4) {
              *reinterpret_cast<uint2*>(dst) = make_uint2(ubits[0][hh][e] | (ubits[1][hh][e] << 16),
                                                          ubits[2][hh][e] | (ubits[3][hh][e] << 16));
            } else {
              *reinterpret_cast<uint4*>(dst) = make_uint4(ubits[0][hh][e] | (ubits[1][hh][e] << 16),
                                                          ubits[2][hh][e] | (ubits[3][hh][e] << 16),
                                                          ubits[4][hh][e] | (ubits[5][hh][e] << 16),
                                                          ubits[6][hh][e] | (ubits[7][hh][e] << 16));
            }
          }
        }
    }
    emit_total += __popcll(uni[0][0]) + __popcll(uni[0][1]) + __popcll(uni[1][0]) + __popcll(uni[1][1]);
    pv = pv_next;
  }
  // no load to LDS outstanding past here (the staging area is reused below)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (P1) return;  // pass 1 writes no partials
  // The chunk's remaining listed rows: the loads of up to 16 rows of every
  // head are issued together (one memory round trip per 16 rows, not one per
  // head), then accumulated head by head in list order, as flush() does.
  {
    int nmax = 0;
#pragma unroll
    for (int g = 0; g < GH; ++g) nmax = max(nmax, lcnt[g]);
    // Non-paged V with 32-bit offsets: the entries are read two at a time as
    // one LDS broadcast and each row loads through one descriptor; slots past
    // a list's end take an offset past the descriptor's range (no traffic,
    // zero) and are not accumulated.
    const bool v32 = !PAGED && static_cast<uint64_t>(L_valid) * row_bytes <= 0xffffffffull;
    if (v32 && nmax > 0) {
      const __amdgpu_buffer_rsrc_t rs_v = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<char*>(Vg), static_cast<short>(0), static_cast<int>(static_cast<uint32_t>(L_valid) * row_bytes),
          kBufferWord3);
      // four heads at a time (GH 8: two such blocks, so that the 16 rows and
      // coefficients in flight per head fit the registers)
      for (int q0 = 0; q0 < nmax; q0 += 16) {
#pragma unroll
        for (int hb = 0; hb < NHB; ++hb) {
          uint32_t vw[4][16];
          float cw[4][16];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int g = 4 * hb + k;
            if (lcnt[g] > q0) {
#pragma unroll
              for (int p = 0; p < 8; ++p) {
                const int4 e2 = *reinterpret_cast<const int4*>(&list[g * LCAP + q0 + 2 * p]);
                cw[k][2 * p] = __int_as_float(e2.y);
                cw[k][2 * p + 1] = __int_as_float(e2.w);
                const uint32_t o0 = (q0 + 2 * p < lcnt[g])
                                        ? __umul24(static_cast<uint32_t>(e2.x), row_bytes) + v_lane_off
                                        : 0xffffffffu;
                const uint32_t o1 = (q0 + 2 * p + 1 < lcnt[g])
                                        ? __umul24(static_cast<uint32_t>(e2.z), row_bytes) + v_lane_off
                                        : 0xffffffffu;
                vw[k][2 * p] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(rs_v, o0, 0, 0));
                vw[k][2 * p + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(rs_v, o1, 0, 0));
              }
            }
          }
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int g = 4 * hb + k;
            if (lcnt[g] > q0) {
#pragma unroll
              for (int q = 0; q < 16; ++q) {
                if (q0 + q < lcnt[g]) {
                  num0[g] = fmaf(cw[k][q], lo16_to_f32<BF16>(vw[k][q]), num0[g]);
                  num1[g] = fmaf(cw[k][q], hi16_to_f32<BF16>(vw[k][q]), num1[g]);
                }
              }
            }
          }
        }
      }
      nmax = 0;
    }
    uint64_t av[GH];
    float coefv[GH];
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      const int2 ent = (lane < lcnt[g]) ? list[g * LCAP + lane] : make_int2(0, 0);
      av[g] = v_addr(ent.x, lane < lcnt[g]);
      coefv[g] = __int_as_float(ent.y);
    }
    for (int q0 = 0; q0 < nmax; q0 += 16) {
      uint32_t vw[GH][16];
#pragma unroll
      for (int g = 0; g < GH; ++g) {
        if (lcnt[g] > q0) {
#pragma unroll
          for (int q = 0; q < 16; ++q) vw[g][q] = v_load(av[g], min(q0 + q, lcnt[g] - 1));
        }
      }
#pragma unroll
      for (int g = 0; g < GH; ++g) {
        if (lcnt[g] > q0) accumulate(g, coefv[g], vw[g], q0, lcnt[g]);
      }
    }
#pragma unroll
    for (int g = 0; g < GH; ++g) lcnt[g] = 0;
  }

  if constexpr (ROWS) {
    // this wave's partial is the (b, kv, chunk) partial
    const size_t slot = static_cast<size_t>(wg) * KVH + wave;
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      float* pp = part + (slot * GH + g) * kPartStride;
      if (lane == 0) {
        pp[0] = runM[g];
        pp[1] = runZ[g];
      }
      pp[2 + 2 * lane] = num0[g];
      pp[3 + 2 * lane] = num1[g];
    }
    if (lane == 0) part_emit[slot] = emit_total;
    return;
  }

  // ---- the four waves' partials, merged in wave order -----------------------------
  __syncthreads();  // every wave is done with its staging area
  float* sp = reinterpret_cast<float*>(s_k);  // [wave][g][kPartStride], then the wave emit counts
  int* s_emit = reinterpret_cast<int*>(sp + 4 * GH * kPartStride);
#pragma unroll
  for (int g = 0; g < GH; ++g) {
    float* p = sp + (wave * GH + g) * kPartStride;
    if (lane == 0) {
      p[0] = runM[g];
      p[1] = runZ[g];
    }
    p[2 + 2 * lane] = num0[g];
    p[3 + 2 * lane] = num1[g];
  }
  if (lane == 0) s_emit[wave] = emit_total;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < NHB; ++k) {
    const int g = wave + 4 * k;
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sp[(w * GH + g) * kPartStride]);
    float Z = 0.0f, n0v = 0.0f, n1v = 0.0f;
    if (M != -__builtin_inff()) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float* p = sp + (w * GH + g) * kPartStride;
        const float r = santa_expf(p[0] - M);
        Z = fmaf(p[1], r, Z);
        n0v = fmaf(p[2 + 2 * lane], r, n0v);
        n1v = fmaf(p[3 + 2 * lane], r, n1v);
      }
    }
    float* pp = part + (static_cast<size_t>(wg) * GH + g) * kPartStride;
    if (lane == 0) {
      pp[0] = M;
      pp[1] = Z;
    }
    pp[2 + 2 * lane] = n0v;
    pp[3 + 2 * lane] = n1v;
  }
  if (tid == 0) part_emit[wg] = (s_emit[0] + s_emit[1]) + (s_emit[2] + s_emit[3]);
}

// Split-KV merge of per-tile partials (flash/santa_cuda_kernel.cu:386-470):
// one workgroup per (b, h); max and Z trees with the reference's pairing
// (strides 128 .. 1), numerator accumulated over tiles in ascending order
// with fma.
template <bool BF16>
__global__ __launch_bounds__(kThreads) void finalize_kernel(const float* __restrict__ m_tiles,
                                                            const float* __restrict__ ell_tiles,
                                                            const float* __restrict__ out_tiles,
                                                            const int* __restrict__ emit_cnt, int H, int KVH,
                                                            int T_c, int S_pt, uint16_t* __restrict__ out,
                                                            float* __restrict__ m_star, int* __restrict__ vrows) {
  extern __shared__ float smem[];
  float* w_s = smem;
  float* red = smem + T_c;
  const int bh = static_cast<int>(blockIdx.x);
  const int tid = static_cast<int>(threadIdx.x);
  const float* mt = m_tiles + static_cast<size_t>(bh) * T_c;
  const float* lt = ell_tiles + static_cast<size_t>(bh) * T_c;

  float lm = -__builtin_inff();
  for (int t = tid; t < T_c; t += kThreads) lm = fmaxf(lm, mt[t]);
  red[tid] = lm;
  __syncthreads();
  for (int s = kThreads >> 1; s > 0; s >>= 1) {
    if (tid < s) red[tid] = fmaxf(red[tid], red[tid + s]);
    __syncthreads();
  }
  const float ms = red[0];
  __syncthreads();
  if (tid == 0 && m_star) m_star[bh] = ms;

  float z = 0.0f;
  for (int t = tid; t < T_c; t += kThreads) {
    const float wt = santa_expf(mt[t] - ms) * lt[t];
    w_s[t] = wt;
    z += wt;
  }
  red[tid] = z;
  __syncthreads();
  for (int s = kThreads >> 1; s > 0; s >>= 1) {
    if (tid < s) red[tid] = red[tid] + red[tid + s];
    __syncthreads();
  }
  const float Z = red[0];
  const float inv_norm = (S_pt > 0 && Z > 0.0f) ? (1.0f / (Z * static_cast<float>(S_pt))) : 0.0f;

  if (tid < kD) {
    const float* ot = out_tiles + static_cast<size_t>(bh) * T_c * kD + tid;
    float num = 0.0f;
#pragma unroll 8
    for (int t = 0; t < T_c; ++t) num = fmaf(w_s[t], ot[static_cast<size_t>(t) * kD], num);
    out[static_cast<size_t>(bh) * kD + tid] = f32_to_h16<BF16>(num * inv_norm);
  }

  const int GH = H / KVH;
  const int h = bh % H;
  if (vrows && (h % GH) == 0) {
    __syncthreads();
    const int b = bh / H;
    const int kv = h / GH;
    const int* ec = emit_cnt + (static_cast<size_t>(b) * KVH + kv) * T_c;
    int cnt = 0;
    for (int t = tid; t < T_c; t += kThreads) cnt += ec[t];
    int* ired = reinterpret_cast<int*>(red);
    ired[tid] = cnt;
    __syncthreads();
    for (int s = kThreads >> 1; s > 0; s >>= 1) {
      if (tid < s) ired[tid] += ired[tid + s];
      __syncthreads();
    }
    if (tid == 0) vrows[static_cast<size_t>(b) * KVH + kv] = ired[0];
  }
}

// Merge of the chunk partials of one (b, h): m* = max_c M_c,
// w_c = exp(M_c - m*), out = (sum_c w_c num_c) / ((sum_c w_c Z_c) S_pt).
template <bool BF16, int GH>
__global__ __launch_bounds__(1024) void merge_kernel(const float* __restrict__ part, const int* __restrict__ part_emit,
                                                     int H, int KVH, int cpg, int S_pt, uint16_t* __restrict__ out,
                                                     float* __restrict__ m_star, int* __restrict__ vrows,
                                                     const int* __restrict__ seq_lens, int BN, int cs, int max_len,
                                                     int n_wg, long long S_total) {
  const int bh = static_cast<int>(blockIdx.x);
  const int b = bh / H;
  const int h = bh % H;
  const int kv = h / GH;
  const int g = h % GH;
  const int bk = b * KVH + kv;
  const int d = static_cast<int>(threadIdx.x) & (kD - 1);
  const int grp = static_cast<int>(threadIdx.x) / kD;   // thread group: a range of chunks
  const int ngrp = static_cast<int>(blockDim.x) / kD;
  // chunk c of (b, kv) was workgroup base_b + c * KVH + kv
  int base = b * cpg * KVH;
  if (seq_lens) {
    base = 0;
    for (int bb = 0; bb < b; ++bb) base += KVH * (((ragged_len(seq_lens, bb, max_len) + BN - 1) / BN + cs - 1) / cs);
    const int tiles = (ragged_len(seq_lens, b, max_len) + BN - 1) / BN;
    cpg = (tiles + cs - 1) / cs;
    cpg = max(0, min(cpg, (n_wg - base - kv + KVH - 1) / KVH));  // only launched workgroups wrote partials
    S_pt = (S_total > 0) ? static_cast<int>(max(1LL, S_total / static_cast<long long>(tiles))) : 0;
  }
  const float* pb = part + ((static_cast<size_t>(base) + kv) * GH + g) * kPartStride;
  const size_t cstride = static_cast<size_t>(KVH) * GH * kPartStride;
  // Each thread group merges a contiguous range of chunks, with the loads of
  // a batch of up to 16 chunks issued before the first use (one memory round
  // trip per batch, usually the only one); max and sums keep the ascending
  // chunk order inside a range, and the ranges are combined in group order.
  constexpr int kBatch = 16;
  const int per = (cpg + ngrp - 1) / ngrp;
  const int c0 = min(cpg, grp * per);
  const int n = min(cpg, c0 + per) - c0;
  float ms = -__builtin_inff();
  float Z = 0.0f, num = 0.0f;
  int e = 0;
  if (n <= kBatch) {
    float mc[kBatch], zc[kBatch], nc[kBatch];
    int ec[kBatch];
#pragma unroll
    for (int c = 0; c < kBatch; ++c) {
      const int cc = c0 + (c < n ? c : 0);
      const float* pc = pb + static_cast<size_t>(cc) * cstride;
      mc[c] = pc[0];
      zc[c] = pc[1];
      nc[c] = pc[2 + d];
      ec[c] = (vrows && d == 0) ? part_emit[static_cast<size_t>(base) + cc * KVH + kv] : 0;
    }
    if (n > 0) {
#pragma unroll
      for (int c = 0; c < kBatch; ++c)
        if (c < n) ms = fmaxf(ms, mc[c]);
#pragma unroll
      for (int c = 0; c < kBatch; ++c) {
        if (c < n) {
          const float w = santa_expf(mc[c] - ms);
          Z = fmaf(w, zc[c], Z);
          num = fmaf(w, nc[c], num);
          e += ec[c];
        }
      }
    }
  } else {
    for (int c = c0; c < c0 + n; ++c) ms = fmaxf(ms, pb[c * cstride]);
    for (int c = c0; c < c0 + n; ++c) {
      const float* pc = pb + c * cstride;
      const float w = santa_expf(pc[0] - ms);
      Z = fmaf(w, pc[1], Z);
      num = fmaf(w, pc[2 + d], num);
      if (vrows && d == 0) e += part_emit[static_cast<size_t>(base) + c * KVH + kv];
    }
  }
  if (ngrp > 1) {
    __shared__ float s_m[8], s_z[8], s_n[8][kD];
    __shared__ int s_e[8];
    if (d == 0) {
      s_m[grp] = ms;
      s_z[grp] = Z;
      s_e[grp] = e;
    }
    s_n[grp][d] = num;
    __syncthreads();
    if (grp != 0) return;
    ms = -__builtin_inff();
    for (int j = 0; j < ngrp; ++j) ms = fmaxf(ms, s_m[j]);
    Z = 0.0f;
    num = 0.0f;
    e = 0;
    if (ms != -__builtin_inff()) {
      for (int j = 0; j < ngrp; ++j) {
        const float w = santa_expf(s_m[j] - ms);
        Z = fmaf(w, s_z[j], Z);
        num = fmaf(w, s_n[j][d], num);
      }
    }
    for (int j = 0; j < ngrp; ++j) e += s_e[j];
  }
  const float inv_norm = (S_pt > 0 && Z > 0.0f) ? (1.0f / (Z * static_cast<float>(S_pt))) : 0.0f;
  out[static_cast<size_t>(bh) * kD + d] = f32_to_h16<BF16>(num * inv_norm);
  if (d == 0 && m_star) m_star[bh] = ms;
  if (vrows && g == 0 && d == 0) vrows[bk] = e;
}

// The same merge for at most NB chunks per (b, h), one wave per (b, h): lane
// c reads chunk c's M, Z (and emitted-row count), lane l the numerator pair
// (2l, 2l + 1) of every chunk, all loads issued before the first use; w_c =
// exp(M_c - m*) is computed once, by lane c; Z and the numerator are summed
// over c in ascending order.  One memory round trip, no LDS, no barrier.
template <bool BF16, int GH, int NB>
__global__ __launch_bounds__(64) void merge_wave_kernel(const float* __restrict__ part,
                                                        const int* __restrict__ part_emit, int H, int KVH, int cpg,
                                                        int S_pt, uint16_t* __restrict__ out,
                                                        float* __restrict__ m_star, int* __restrict__ vrows,
                                                        const int* __restrict__ seq_lens, int BN, int cs,
                                                        int max_len, int n_wg, long long S_total) {
  const int bh = static_cast<int>(blockIdx.x);
  const int b = bh / H;
  const int h = bh % H;
  const int kv = h / GH;
  const int g = h % GH;
  const int lane = static_cast<int>(threadIdx.x);
  // chunk c of (b, kv) was workgroup base_b + c * KVH + kv
  int base = b * cpg * KVH;
  if (seq_lens) {
    base = 0;
    for (int bb = 0; bb < b; ++bb) base += KVH * (((ragged_len(seq_lens, bb, max_len) + BN - 1) / BN + cs - 1) / cs);
    const int tiles = (ragged_len(seq_lens, b, max_len) + BN - 1) / BN;
    cpg = (tiles + cs - 1) / cs;
    cpg = max(0, min(cpg, (n_wg - base - kv + KVH - 1) / KVH));  // only launched workgroups wrote partials
    S_pt = (S_total > 0) ? static_cast<int>(max(1LL, S_total / static_cast<long long>(tiles))) : 0;
  }
  const int n = min(cpg, NB);
  const float* pb = part + ((static_cast<size_t>(base) + kv) * GH + g) * kPartStride;
  const size_t cstride = static_cast<size_t>(KVH) * GH * kPartStride;
  float Mc = -__builtin_inff(), Zc = 0.0f;
  int ec = 0;
  if (lane < n) {
    Mc = pb[lane * cstride];
    Zc = pb[lane * cstride + 1];
    if (vrows && g == 0) ec = part_emit[static_cast<size_t>(base) + lane * KVH + kv];
  }
  float2 nv[NB];
  if (n > 0) {
#pragma unroll
    for (int c = 0; c < NB; ++c) {
      const int cc = min(c, n - 1);  // past n: chunk n - 1 again, weighted by 0
      nv[c] = *reinterpret_cast<const float2*>(pb + cc * cstride + 2 + 2 * lane);
    }
  } else {
#pragma unroll
    for (int c = 0; c < NB; ++c) nv[c] = make_float2(0.0f, 0.0f);
  }
  const float ms = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_max_lane63(Mc + 0.0f)), 63));
  const float w = (lane < n && ms != -__builtin_inff()) ? santa_expf(Mc - ms) : 0.0f;
  float Z = 0.0f, num0 = 0.0f, num1 = 0.0f;
#pragma unroll
  for (int c = 0; c < NB; ++c) {
    const float wc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), c));
    const float zc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(Zc), c));
    Z = fmaf(wc, zc, Z);
    num0 = fmaf(wc, nv[c].x, num0);
    num1 = fmaf(wc, nv[c].y, num1);
  }
  const float inv_norm = (S_pt > 0 && Z > 0.0f) ? (1.0f / (Z * static_cast<float>(S_pt))) : 0.0f;
  *reinterpret_cast<uint32_t*>(out + static_cast<size_t>(bh) * kD + 2 * lane) =
      static_cast<uint32_t>(f32_to_h16<BF16>(num0 * inv_norm)) |
      (static_cast<uint32_t>(f32_to_h16<BF16>(num1 * inv_norm)) << 16);
  if (lane == 0 && m_star) m_star[bh] = ms;
  if (vrows && g == 0) {
    const int e = wave_sum_int(ec);
    if (lane == 0) vrows[static_cast<size_t>(b) * KVH + kv] = e;
  }
}

// The merge split over NW waves of one workgroup per (b, h), wave s taking
// chunks 16s .. 16s+15: each wave finds its chunks' maximum, the workgroup's
// maximum m* goes through LDS, each wave sums its chunks' Z and numerator
// (ascending) with weights exp(M_c - m*), and wave 0 adds the waves' sums in
// wave order.
template <bool BF16, int GH, int NW>
__global__ __launch_bounds__(64 * NW) void merge_split_kernel(const float* __restrict__ part,
                                                              const int* __restrict__ part_emit, int H, int KVH,
                                                              int cpg, int S_pt, uint16_t* __restrict__ out,
                                                              float* __restrict__ m_star, int* __restrict__ vrows,
                                                              const int* __restrict__ seq_lens, int BN, int cs,
                                                              int max_len, int n_wg, long long S_total) {
  constexpr int NB = 16;
  __shared__ float s_m[NW];
  __shared__ float s_z[NW];
  __shared__ int s_e[NW];
  __shared__ float2 s_n[NW][64];
  const int bh = static_cast<int>(blockIdx.x);
  const int b = bh / H;
  const int h = bh % H;
  const int kv = h / GH;
  const int g = h % GH;
  const int lane = static_cast<int>(threadIdx.x) & 63;
  const int wv = static_cast<int>(threadIdx.x) >> 6;
  int base = b * cpg * KVH;
  if (seq_lens) {
    base = 0;
    for (int bb = 0; bb < b; ++bb) base += KVH * (((ragged_len(seq_lens, bb, max_len) + BN - 1) / BN + cs - 1) / cs);
    const int tiles = (ragged_len(seq_lens, b, max_len) + BN - 1) / BN;
    cpg = (tiles + cs - 1) / cs;
    cpg = max(0, min(cpg, (n_wg - base - kv + KVH - 1) / KVH));
    S_pt = (S_total > 0) ? static_cast<int>(max(1LL, S_total / static_cast<long long>(tiles))) : 0;
  }
  const int n = min(cpg, NB * NW);
  const int c0 = NB * wv;
  const int nw = max(0, min(n - c0, NB));  // chunks of this wave
  const size_t cstride = static_cast<size_t>(KVH) * GH * kPartStride;
  const float* pb = part + ((static_cast<size_t>(base) + kv) * GH + g) * kPartStride + c0 * cstride;
  float Mc = -__builtin_inff(), Zc = 0.0f;
  int ec = 0;
  if (lane < nw) {
    Mc = pb[lane * cstride];
    Zc = pb[lane * cstride + 1];
    if (vrows && g == 0) ec = part_emit[static_cast<size_t>(base) + (c0 + lane) * KVH + kv];
  }
  float2 nv[NB];
  if (nw > 0) {
#pragma unroll
    for (int c = 0; c < NB; ++c) {
      const int cc = min(c, nw - 1);  // past nw: chunk nw - 1 again, weighted by 0
      nv[c] = *reinterpret_cast<const float2*>(pb + cc * cstride + 2 + 2 * lane);
    }
  } else {
#pragma unroll
    for (int c = 0; c < NB; ++c) nv[c] = make_float2(0.0f, 0.0f);
  }
  const float ml = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_max_lane63(Mc + 0.0f)), 63));
  if (lane == 0) s_m[wv] = ml;
  __syncthreads();
  float ms = s_m[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) ms = fmaxf(ms, s_m[i]);
  const float w = (lane < nw && ms != -__builtin_inff()) ? santa_expf(Mc - ms) : 0.0f;
  float Z = 0.0f, num0 = 0.0f, num1 = 0.0f;
#pragma unroll
  for (int c = 0; c < NB; ++c) {
    const float wc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), c));
    const float zc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(Zc), c));
    Z = fmaf(wc, zc, Z);
    num0 = fmaf(wc, nv[c].x, num0);
    num1 = fmaf(wc, nv[c].y, num1);
  }
  const int e = (vrows && g == 0) ? wave_sum_int(ec) : 0;
  if (lane == 0) {
    s_z[wv] = Z;
    s_e[wv] = e;
  }
  s_n[wv][lane] = make_float2(num0, num1);
  __syncthreads();
  if (wv != 0) return;
#pragma unroll
  for (int i = 1; i < NW; ++i) {
    Z = Z + s_z[i];
    num0 = num0 + s_n[i][lane].x;
    num1 = num1 + s_n[i][lane].y;
  }
  const float inv_norm = (S_pt > 0 && Z > 0.0f) ? (1.0f / (Z * static_cast<float>(S_pt))) : 0.0f;
  *reinterpret_cast<uint32_t*>(out + static_cast<size_t>(bh) * kD + 2 * lane) =
      static_cast<uint32_t>(f32_to_h16<BF16>(num0 * inv_norm)) |
      (static_cast<uint32_t>(f32_to_h16<BF16>(num1 * inv_norm)) << 16);
  if (lane == 0 && m_star) m_star[bh] = ms;
  if (vrows && g == 0 && lane == 0) {
    int et = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) et += s_e[i];
    vrows[static_cast<size_t>(b) * KVH + kv] = et;
  }
}

struct Args {
  const void* q;
  const void* K;
  const void* V;
  int B, H, KVH, L_valid, L_storage, T_c, S_pt;
  uint64_t seed;
  float *m_tiles, *ell_tiles, *out_tiles;
  int* emit_cnt;
  int16_t* counts;
  float* part;
  int* part_emit;
  int cs, cpg;
  uint16_t* u_stash;
  const int* seq_lens;  // ragged form (prop pass 1, ragged flash) or nullptr
  int n_wg;             // grid size of the ragged form
  long long S_total;    // ragged flash: S, for each sequence's S_per_tile
  PageTable pt;         // paged K/V (pt.table set) or contiguous
};

template <bool BF16, int GH, int BN, int MODE, bool PAGED>
static hipError_t launch_tk(const Args& a, hipStream_t stream) {
  const float q_scale = 1.0f / sqrtf(static_cast<float>(kD));
  const unsigned grid = a.seq_lens ? static_cast<unsigned>(a.n_wg)
                                   : static_cast<unsigned>(a.B) * static_cast<unsigned>(a.KVH) * static_cast<unsigned>(a.cpg);
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL((tile_kernel<BF16, GH, BN, MODE, PAGED>), dim3(grid), dim3(kThreads), 0, stream,
                     static_cast<const uint16_t*>(a.q), static_cast<const uint16_t*>(a.K),
                     static_cast<const uint16_t*>(a.V), a.H, a.KVH, a.L_valid, a.L_storage, a.T_c, a.cs, a.cpg,
                     q_scale, a.S_pt, a.seed, a.m_tiles, a.ell_tiles, a.out_tiles, a.emit_cnt, a.counts, a.part,
                     a.part_emit, a.u_stash, a.seq_lens, a.B, a.S_total, a.pt);
  return hipGetLastError();
}

// Paged caches go through the online mode at block_n 32/64 (block_n 256 is
// the wave kernel's) and the general pass 1.
template <bool BF16, int GH, int BN, int MODE>
static hipError_t launch_t(const Args& a, hipStream_t stream) {
  if (a.pt.table) {
    if constexpr (MODE == kOnline || MODE == kPass1Gen) return launch_tk<BF16, GH, BN, MODE, true>(a, stream);
    return hipErrorInvalidValue;
  }
  return launch_tk<BF16, GH, BN, MODE, false>(a, stream);
}

template <bool BF16, int GH, int MODE>
static hipError_t launch_bn(int bn, const Args& a, hipStream_t stream) {
  switch (bn) {
    case 32:
      return launch_t<BF16, GH, 32, MODE>(a, stream);
    case 64:
      return launch_t<BF16, GH, 64, MODE>(a, stream);
    default:
      return launch_t<BF16, GH, 256, MODE>(a, stream);
  }
}

template <bool BF16, int GH>
static hipError_t launch_wave_t(const Args& a, float* dbg_m, float* dbg_ell, int16_t* dbg_counts,
                                hipStream_t stream) {
  const float q_scale = 1.0f / sqrtf(static_cast<float>(kD));
  const unsigned grid = a.seq_lens ? static_cast<unsigned>(a.n_wg)
                                   : static_cast<unsigned>(a.B) * static_cast<unsigned>(a.KVH) * static_cast<unsigned>(a.cpg);
  if (grid == 0) return hipSuccess;
  if (dbg_counts) {
    if (a.pt.table) return hipErrorInvalidValue;  // the statistics check reads contiguous caches
    if (rows_layout(a.KVH)) {  // the production layout, with the statistics written out
      hipLaunchKernelGGL((wave_kernel<BF16, GH, true, false, false, true>), dim3(grid / static_cast<unsigned>(a.KVH)),
                         dim3(static_cast<unsigned>(64 * a.KVH)), 0, stream, static_cast<const uint16_t*>(a.q),
                         static_cast<const uint16_t*>(a.K), static_cast<const uint16_t*>(a.V), a.H, a.KVH, a.L_valid,
                         a.L_storage, a.T_c, a.cs, a.cpg, q_scale, a.S_pt, a.seed, a.part, a.part_emit, a.seq_lens,
                         a.B, a.S_total, dbg_m, dbg_ell, dbg_counts, nullptr, 0, a.pt, 0, 1);
      return hipGetLastError();
    }
    hipLaunchKernelGGL((wave_kernel<BF16, GH, true>), dim3(grid), dim3(kThreads), 0, stream,
                       static_cast<const uint16_t*>(a.q), static_cast<const uint16_t*>(a.K),
                       static_cast<const uint16_t*>(a.V), a.H, a.KVH, a.L_valid, a.L_storage, a.T_c, a.cs, a.cpg,
                       q_scale, a.S_pt, a.seed, a.part, a.part_emit, a.seq_lens, a.B, a.S_total, dbg_m, dbg_ell,
                       dbg_counts, nullptr, 0, a.pt, 0, 1);
  } else if (rows_layout(a.KVH)) {
    // one workgroup of KVH waves per (sequence, chunk) item
    const unsigned rgrid = grid / static_cast<unsigned>(a.KVH);
    const dim3 block(static_cast<unsigned>(64 * a.KVH));
    if (a.pt.table)
      hipLaunchKernelGGL((wave_kernel<BF16, GH, false, false, true, true>), dim3(rgrid), block, 0, stream,
                         static_cast<const uint16_t*>(a.q), static_cast<const uint16_t*>(a.K),
                         static_cast<const uint16_t*>(a.V), a.H, a.KVH, a.L_valid, a.L_storage, a.T_c, a.cs, a.cpg,
                         q_scale, a.S_pt, a.seed, a.part, a.part_emit, a.seq_lens, a.B, a.S_total, nullptr,
                         nullptr, nullptr, nullptr, 0, a.pt, 0, 1);
    else
      hipLaunchKernelGGL((wave_kernel<BF16, GH, false, false, false, true>), dim3(rgrid), block, 0, stream,
                         static_cast<const uint16_t*>(a.q), static_cast<const uint16_t*>(a.K),
                         static_cast<const uint16_t*>(a.V), a.H, a.KVH, a.L_valid, a.L_storage, a.T_c, a.cs, a.cpg,
                         q_scale, a.S_pt, a.seed, a.part, a.part_emit, a.seq_lens, a.B, a.S_total, nullptr,
                         nullptr, nullptr, nullptr, 0, a.pt, 0, 1);
  } else if (a.pt.table) {
    hipLaunchKernelGGL((wave_kernel<BF16, GH, false, false, true>), dim3(grid), dim3(kThreads), 0, stream,
                       static_cast<const uint16_t*>(a.q), static_cast<const uint16_t*>(a.K),
                       static_cast<const uint16_t*>(a.V), a.H, a.KVH, a.L_valid, a.L_storage, a.T_c, a.cs, a.cpg,
                       q_scale, a.S_pt, a.seed, a.part, a.part_emit, a.seq_lens, a.B, a.S_total, nullptr,
                       nullptr, nullptr, nullptr, 0, a.pt, 0, 1);
  } else {
    hipLaunchKernelGGL((wave_kernel<BF16, GH, false>), dim3(grid), dim3(kThreads), 0, stream,
                       static_cast<const uint16_t*>(a.q), static_cast<const uint16_t*>(a.K),
                       static_cast<const uint16_t*>(a.V), a.H, a.KVH, a.L_valid, a.L_storage, a.T_c, a.cs, a.cpg,
                       q_scale, a.S_pt, a.seed, a.part, a.part_emit, a.seq_lens, a.B, a.S_total, nullptr,
                       nullptr, nullptr, nullptr, 0, a.pt, 0, 1);
  }
  return hipGetLastError();
}

// The online tile pass of block_n = 256 on the wave kernel (debug outputs
// may be null).
static hipError_t launch_wave(int dtype, int GH, const Args& a, float* dbg_m, float* dbg_ell, int16_t* dbg_counts,
                              hipStream_t stream) {
  if (dtype == SANTA_BF16)
    return (GH == 4) ? launch_wave_t<true, 4>(a, dbg_m, dbg_ell, dbg_counts, stream)
                     : launch_wave_t<true, 8>(a, dbg_m, dbg_ell, dbg_counts, stream);
  return (GH == 4) ? launch_wave_t<false, 4>(a, dbg_m, dbg_ell, dbg_counts, stream)
                   : launch_wave_t<false, 8>(a, dbg_m, dbg_ell, dbg_counts, stream);
}

// The chunk-partial merge, one workgroup per (b, h); seq_lens selects the
// ragged chunk layout (then bn, cs, max_len, n_wg and S_total describe it).
static hipError_t launch_merge(const float* part, const int* pe, int dtype, int B, int H, int KVH, int cpg, int S_pt,
                               void* out, float* m_star, int* vrows, const int* seq_lens, int bn, int cs,
                               int max_len, int n_wg, long long S_total, hipStream_t stream) {
  const int GH = H / KVH;
  const unsigned grid = static_cast<unsigned>(B) * static_cast<unsigned>(H);
  uint16_t* o = static_cast<uint16_t*>(out);
  const int max_chunks = seq_lens ? ((max_len + bn - 1) / bn + cs - 1) / cs : cpg;
  if (max_chunks <= 256) {
    // one wave per (b, h) up to 32 chunks, else 4, 8 or 16 waves of 16
    // chunks each, every load in one round trip (B = 1 at 32k, 64 chunks:
    // step 24.7 -> 23.6 us; beyond 64 chunks the thread-group merge below
    // took 20-26 us per call at B = 1, GH 8, 64k-96k tokens)
#define SANTA_MERGE_WAVE(BF, G, NBC)                                                                          \
  hipLaunchKernelGGL((merge_wave_kernel<BF, G, NBC>), dim3(grid), dim3(64), 0, stream, part, pe, H, KVH, cpg, \
                     S_pt, o, m_star, vrows, seq_lens, bn, cs, max_len, n_wg, S_total)
#define SANTA_MERGE_SPLIT(BF, G, NWC)                                                                       \
  hipLaunchKernelGGL((merge_split_kernel<BF, G, NWC>), dim3(grid), dim3(64 * NWC), 0, stream, part, pe, H, KVH, cpg, \
                     S_pt, o, m_star, vrows, seq_lens, bn, cs, max_len, n_wg, S_total)
#define SANTA_MERGE_NB(BF, G)           \
  if (max_chunks <= 16)                 \
    SANTA_MERGE_WAVE(BF, G, 16);        \
  else if (max_chunks <= 32)            \
    SANTA_MERGE_WAVE(BF, G, 32);        \
  else if (max_chunks <= 64)            \
    SANTA_MERGE_SPLIT(BF, G, 4);        \
  else if (max_chunks <= 128)           \
    SANTA_MERGE_SPLIT(BF, G, 8);        \
  else                                  \
    SANTA_MERGE_SPLIT(BF, G, 16)
    if (dtype == SANTA_BF16) {
      if (GH == 4) { SANTA_MERGE_NB(true, 4); } else { SANTA_MERGE_NB(true, 8); }
    } else {
      if (GH == 4) { SANTA_MERGE_NB(false, 4); } else { SANTA_MERGE_NB(false, 8); }
    }
#undef SANTA_MERGE_NB
#undef SANTA_MERGE_WAVE
#undef SANTA_MERGE_SPLIT
    return hipGetLastError();
  }
  // thread groups of 128: enough that each merges at most 16 chunks (up to 8)
  const int ngrp = std::min(8, std::max(1, (max_chunks + 15) / 16));
  const dim3 block(static_cast<unsigned>(kD * ngrp));
  if (dtype == SANTA_BF16) {
    if (GH == 4)
      hipLaunchKernelGGL((merge_kernel<true, 4>), dim3(grid), block, 0, stream, part, pe, H, KVH, cpg, S_pt, o,
                         m_star, vrows, seq_lens, bn, cs, max_len, n_wg, S_total);
    else
      hipLaunchKernelGGL((merge_kernel<true, 8>), dim3(grid), block, 0, stream, part, pe, H, KVH, cpg, S_pt, o,
                         m_star, vrows, seq_lens, bn, cs, max_len, n_wg, S_total);
  } else {
    if (GH == 4)
      hipLaunchKernelGGL((merge_kernel<false, 4>), dim3(grid), block, 0, stream, part, pe, H, KVH, cpg, S_pt, o,
                         m_star, vrows, seq_lens, bn, cs, max_len, n_wg, S_total);
    else
      hipLaunchKernelGGL((merge_kernel<false, 8>), dim3(grid), block, 0, stream, part, pe, H, KVH, cpg, S_pt, o,
                         m_star, vrows, seq_lens, bn, cs, max_len, n_wg, S_total);
  }
  return hipGetLastError();
}

template <int MODE>
static hipError_t launch_tiles(int dtype, int GH, int bn, const Args& a, hipStream_t stream) {
  if (dtype == SANTA_BF16)
    return (GH == 4) ? launch_bn<true, 4, MODE>(bn, a, stream) : launch_bn<true, 8, MODE>(bn, a, stream);
  return (GH == 4) ? launch_bn<false, 4, MODE>(bn, a, stream) : launch_bn<false, 8, MODE>(bn, a, stream);
}

// Workgroups resident per device: CUs x 2 (two 256-thread workgroups per CU
// at the tile kernel's register budget), cached per device in atomics (host
// threads on different devices each see their own count; two threads filling
// the same entry store the same value).
static int resident_workgroups() {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cached[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 512;
  if (dev >= 0 && dev < kMaxDev) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (dev >= 0 && dev < kMaxDev) cached[dev].store(2 * cus, std::memory_order_relaxed);
  return 2 * cus;
}

// Chunking of each group's T_c tiles so that B*KVH*cpg is about one resident
// round of per_round items (0: resident_workgroups(), one 4-wave workgroup
// per item): cpg chunks of cs tiles (the last may be shorter).  The chunk
// count per group is rounded to the nearest, unless that puts more than one
// round of items in the grid; then it is the count that fits one round.  The
// few items of a second round would each walk a whole chunk after the rest:
// in the flash rows layout (one workgroup per CU) B = 6, 10, 20, 24, ... at
// 32k tokens had planned 258-264 workgroups, and one round took B = 6 from
// 116.7 to 85.6 us per step, B = 10 194.1 -> 123.4, B = 20 341.1 -> 224.7,
// B = 24 380.7 -> 262.1 (GH 8: B = 6 191.7 -> 129.2, B = 10 295.1 -> 187.2).
// Chunks whose lengths differ by one tile, so that every CU holds one,
// measured slower (B = 6 at 32k 92.7 us; B = 4 at T_c = 129, 43 chunks of
// three tiles, 71.8 against 66.8 us): the pass is bandwidth-bound there, and
// the longer chunks run on alone after the others.
static void chunk_plan(int B, int KVH, int T_c, int* cs, int* cpg, int per_round = 0) {
  const long long groups = static_cast<long long>(B) * KVH;
  const long long round = per_round > 0 ? per_round : resident_workgroups();
  long long want = (round + groups / 2) / groups;
  if (want < 1) want = 1;
  if (want > T_c) want = T_c;
  int c = static_cast<int>((T_c + want - 1) / want);
  if (groups * ((T_c + c - 1) / c) > round && round / groups >= 1) {
    want = round / groups;  // one round
    c = static_cast<int>((T_c + want - 1) / want);
  }
  *cs = c;
  *cpg = (T_c + c - 1) / c;
}

// The device exponential on an array (test hook, declared in santa_internal.h).
__global__ void expf_kernel(const float* __restrict__ x, float* __restrict__ y, size_t n) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    y[i] = santa_expf(x[i]);
}
hipError_t launch_expf(const float* x, float* y, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const size_t blocks = (n + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(expf_kernel, dim3(static_cast<unsigned>(blocks < 65536 ? blocks : 65536)), dim3(kThreads), 0,
                     stream, x, y, n);
  return hipGetLastError();
}

// The score path's K=1 MFMA against fmaf on the same operands (test hook,
// declared in santa_internal.h).  Wave n reads a[64n + l], b[64n + l] and
// c[4(64n + l) + i] at lane l; for every broadcast block J it writes
// mfma_out / fma_out[((16n + J) * 64 + l) * 4 + i] =
// a[64n + 4J + i] * b[64n + l] + c[4(64n + l) + i], once through
// v_mfma_f32_4x4x1f32 with the A operand of block J broadcast (the form
// score_chunk issues) and once through fmaf.
template <int J>
__device__ __forceinline__ void mfma_fma_block(float a, float b, f32x4 c, int lane, size_t base, float* mo,
                                               float* fo) {
  const f32x4 d = mfma_bcast<J>(a, b, c);
  const size_t o = (base + static_cast<size_t>(J) * 64 + lane) * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float ai = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 4 * J + i));
    mo[o + i] = d[i];
    fo[o + i] = fmaf(ai, b, c[i]);
  }
}
template <int... J>
__device__ __forceinline__ void mfma_fma_blocks(std::integer_sequence<int, J...>, float a, float b, f32x4 c,
                                                int lane, size_t base, float* mo, float* fo) {
  (mfma_fma_block<J>(a, b, c, lane, base, mo, fo), ...);
}
__global__ __launch_bounds__(64) void mfma_fma_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                      const float* __restrict__ c, float* __restrict__ mo,
                                                      float* __restrict__ fo) {
  const int lane = static_cast<int>(threadIdx.x);
  const size_t n = blockIdx.x;
  const size_t i = n * 64 + lane;
  const f32x4 cv = {c[4 * i], c[4 * i + 1], c[4 * i + 2], c[4 * i + 3]};
  mfma_fma_blocks(std::make_integer_sequence<int, 16>{}, a[i], b[i], cv, lane, n * 16 * 64, mo, fo);
}
hipError_t launch_mfma_check(const float* a, const float* b, const float* c, float* mfma_out, float* fma_out,
                             int n_waves, hipStream_t stream) {
  if (n_waves <= 0) return hipSuccess;
  hipLaunchKernelGGL(mfma_fma_kernel, dim3(static_cast<unsigned>(n_waves)), dim3(64), 0, stream, a, b, c, mfma_out,
                     fma_out);
  return hipGetLastError();
}

// santa_prop pass 1 on the tile kernel (declared in santa_internal.h).
hipError_t launch_prop_pass1(const void* q, const void* K, int dtype, int B, int H, int KVH, int L, int L_storage,
                             int block_n, int path, float* m_tiles, float* ell_tiles, uint16_t* u_stash,
                             const int* seq_lens, int cs, int n_wg, int stash_ld, hipStream_t stream,
                             PageTable pt, long long total_tiles, int kv_div) {
  Args a{q, K, nullptr, B, H, KVH, L, L_storage, (L + block_n - 1) / block_n, 0, 0, m_tiles, ell_tiles, nullptr,
         nullptr, nullptr, nullptr, nullptr, 0, 0, u_stash, seq_lens};
  a.pt = pt;
  if (seq_lens) {
    // ragged: L is the longest sequence; n_wg workgroups of cs tiles
    a.cs = cs;
    a.cpg = 0;
    a.n_wg = n_wg;
  } else {
    chunk_plan(B, KVH, a.T_c, &a.cs, &a.cpg);
  }
  const int GH = H / KVH;
  // groups of 5-7 heads with the tile-major stash: the GH 8 kernel, the last
  // heads of each group zero (santa_prop's generic shapes at D = 128)
  const bool pad8 = path == 1 && block_n == 256 && GH >= 5 && GH <= 7 && stash_ld > 0;
  if (kv_div != 1 && !(path == 1 && block_n == 256 && GH >= 5 && GH <= 8 && stash_ld > 0 && KVH % kv_div == 0))
    return hipErrorInvalidValue;  // virtual KV heads: the GH 8 wave kernel with the tile-major stash only
  if (prop_wave_pass1(path, GH, block_n) || pad8) {
    // block_n 256 on the wave kernel -- GH 4 with the vec path's numerics,
    // GH 8 with the general path's; for KVH = 8 in its rows form, with a
    // plan of its own (pass 1 writes no chunk partials, so it need not share
    // pass 2's chunking)
    const float q_scale = 1.0f / sqrtf(static_cast<float>(kD));
    // little K to read and the [L, H] stash: four waves per tile, as for flash
    const long long kv_tiles = (a.seq_lens ? total_tiles : static_cast<long long>(a.B) * a.T_c) * a.KVH;
    if (stash_ld == 0 && !a.pt.table && (!a.seq_lens || total_tiles >= 0) && small_prop_pass(kv_tiles)) {
      if (GH == 4)
        return (dtype == SANTA_BF16) ? launch_bn<true, 4, kPass1Vec>(256, a, stream)
                                     : launch_bn<false, 4, kPass1Vec>(256, a, stream);
      return (dtype == SANTA_BF16) ? launch_bn<true, 8, kPass1Gen>(256, a, stream)
                                   : launch_bn<false, 8, kPass1Gen>(256, a, stream);
    }
    const bool rows = rows_layout(a.KVH) && (!a.seq_lens || total_tiles >= 0);
    if (rows) {
      if (a.seq_lens) {
        // one round of chunks up to 32 sequences (B * KVH at most an eighth
        // of the round), as flash's ragged plan: B = 8 at 16k-64k 172.4 ->
        // 149.7 us per step, B = 4 at 32k-128k 206.6 -> 182.7, B = 12 at
        // 1k-128k 362.8 -> 351.3, cfg3 516.8 -> 514.4 (the same bits); pass 1
        // gathers nothing, so a short sequence's chunk is no heavier than
        // its tiles
        plan_ragged(a.B, a.KVH, total_tiles, a.T_c, &a.cs, &a.n_wg, rows_per_round(), 1,
                    (8LL * a.B * a.KVH <= rows_per_round()) ? 1 : 8);
      } else {
        chunk_plan(a.B, a.KVH, a.T_c, &a.cs, &a.cpg, rows_per_round());
      }
    }
    unsigned grid = a.seq_lens ? static_cast<unsigned>(a.n_wg)
                               : static_cast<unsigned>(a.B) * static_cast<unsigned>(a.KVH) * static_cast<unsigned>(a.cpg);
    if (rows) grid /= static_cast<unsigned>(a.KVH);
    // A tile-major stash larger than half the 256 MiB last-level cache is
    // written with non-temporal stores: cached, it would only evict itself
    // before pass 2 reads it (cfg5-shaped prop step, a 1 GiB stash: 1961 ->
    // 1896 us), while a smaller one is read back from the cache (B = 32 at 32k
    // tokens, 64 MiB: 507 us cached against 525 us non-temporal)
    // (the non-temporal stores address one sequence's stash through a
    // buffer descriptor, whose range and offsets are 32-bit)
    const size_t seq_stash_bytes = static_cast<size_t>(stash_ld) * a.H * sizeof(uint16_t);
    const int stash_nt = (stash_ld > 0 && a.B * seq_stash_bytes > (static_cast<size_t>(128) << 20) &&
                          seq_stash_bytes < (static_cast<size_t>(1) << 31))
                             ? 1
                             : 0;
    if (grid == 0) return hipSuccess;
    const dim3 block(rows ? static_cast<unsigned>(64 * a.KVH) : static_cast<unsigned>(kThreads));
#define SANTA_P1_LAUNCH(BF, G, PG, RW)                                                                            \
  hipLaunchKernelGGL((wave_kernel<BF, G, false, true, PG, RW>), dim3(grid), block, 0, stream,                     \
                     static_cast<const uint16_t*>(a.q), static_cast<const uint16_t*>(a.K), nullptr, a.H, a.KVH,     \
                     a.L_valid, a.L_storage, a.T_c, a.cs, a.cpg, q_scale, 0, 0ULL, nullptr, nullptr, a.seq_lens,   \
                     a.B, 0LL, m_tiles, ell_tiles, nullptr, u_stash, stash_ld, a.pt, stash_nt, kv_div)
#define SANTA_P1_GH(BF, PG, RW)    \
  do {                             \
    if (GH == 4)                   \
      SANTA_P1_LAUNCH(BF, 4, PG, RW); \
    else                           \
      SANTA_P1_LAUNCH(BF, 8, PG, RW); \
  } while (0)
    if (dtype == SANTA_BF16) {
      if (rows) {
        if (a.pt.table) SANTA_P1_GH(true, true, true); else SANTA_P1_GH(true, false, true);
      } else {
        if (a.pt.table) SANTA_P1_GH(true, true, false); else SANTA_P1_GH(true, false, false);
      }
    } else {
      if (rows) {
        if (a.pt.table) SANTA_P1_GH(false, true, true); else SANTA_P1_GH(false, false, true);
      } else {
        if (a.pt.table) SANTA_P1_GH(false, true, false); else SANTA_P1_GH(false, false, false);
      }
    }
#undef SANTA_P1_GH
#undef SANTA_P1_LAUNCH
    return hipGetLastError();
  }
  if (dtype == SANTA_BF16)
    return (GH == 4) ? launch_bn<true, 4, kPass1Gen>(block_n, a, stream)
                     : launch_bn<true, 8, kPass1Gen>(block_n, a, stream);
  return (GH == 4) ? launch_bn<false, 4, kPass1Gen>(block_n, a, stream)
                   : launch_bn<false, 8, kPass1Gen>(block_n, a, stream);
}

// Tile chunking shared with santa_prop's pass 2.
void plan_chunks(int B, int KVH, int T_c, int* cs, int* cpg, int per_round) {
  chunk_plan(B, KVH, T_c, cs, cpg, per_round);
}

// The flash tile pass runs its ROWS form (one wave per KV head) for KVH = 8
// (its LDS is sized for eight waves); its chunks are then planned for one
// resident round of single-wave items (four per 4-wave workgroup slot).
bool rows_layout(int KVH) { return KVH == 8; }
int rows_per_round() { return 4 * resident_workgroups(); }

// Little K to read (at most one resident round of single-wave items: B = 1
// up to 64k tokens, B = 8 up to 8k; uniform batches take one and a half,
// see the overload below): the block_n = 256 tile pass runs on the
// tile kernel, four waves per tile, whose per-tile latency chain is a
// quarter of a wave's (B = 1, 4k tokens: 13.0 against 31.2 us per step; B =
// 1, 32k: 26.5 against 36.2 us).  Above it the wave kernel is faster (B = 4,
// 32k: 60.9 against 63.9 us).  At GH 8 the tile kernel holds one workgroup
// per CU (its registers), one wave per SIMD, and keeps the tile pass only up
// to 1 / kGh8SmallDiv of a round of (kv, tile) items, uniform or ragged.
constexpr int kGh8SmallDiv = 4;
static long long gh8_small_items() { return rows_per_round() / kGh8SmallDiv; }
bool small_pass(long long kv_tiles, int GH) {
  return kv_tiles <= (GH == 8 ? gh8_small_items() : static_cast<long long>(rows_per_round()));
}
// santa_prop's vec pass 1 takes the tile kernel below a quarter of that: the
// [L, H] stash it writes costs pass 2 four 2-byte loads per lane and row pair
// where the tile-major one costs one, which outweighs the shorter pass 1 from
// about 32k tokens of one sequence (per call: 4k 30.8 -> 19.7 us, 16k 38.5 ->
// 31.3 us; 32k 44.0 -> 45.8 us, 64k 54.3 -> 64.5 us).
bool small_prop_pass(long long kv_tiles) { return kv_tiles <= rows_per_round() / 4; }
// santa_prop's pass 1 runs on the wave kernel at block_n 256 for the vec
// path (GH 4) and for the general path at GH 8.
bool prop_wave_pass1(int path, int GH, int block_n) {
  return block_n == 256 && ((path == 0 && GH == 4) || (path == 1 && GH == 8));
}
// Uniform batches keep the tile kernel up to one and a half rounds: at 32k
// tokens it measures 41.3 us for B = 2 just past 2,048 items (T_c = 129)
// against 50.8 us for the rows layout, and the two meet near 4,096 items
// (B = 4: 66.4 against 67.2 us at T_c = 129; B = 8 is 10 % faster on the rows
// layout).  Ragged grids keep the one-round threshold.
bool uniform_small_pass(int B, int KVH, int T_c, int GH) {
  const long long items = static_cast<long long>(B) * KVH * T_c;
  return items <= (GH == 8 ? gh8_small_items() : static_cast<long long>(rows_per_round()) * 3 / 2);
}

// Ragged batches: chunks small enough for about `rounds` resident rounds over
// all (kv, tile) items, so the hardware's workgroup dispatch evens out the
// uneven chunks (each sequence adds at most one partial chunk per KV head;
// B * KVH slots of each round are counted for those).  Eight rounds measured
// best for santa_prop on 16 sequences of 8k-128k tokens (one round: 824 us,
// four: 795, eight: 745, sixteen: 750).
void plan_ragged(int B, int KVH, long long total_tiles, int max_tiles, int* cs, int* n_wg, int per_round,
                 int granule, int rounds) {
  if (max_tiles > 0 && total_tiles == static_cast<long long>(B) * max_tiles) {
    // every sequence has the same tile count: the uniform plan (one resident
    // round), whose workgroups the ragged grid enumerates in the same order
    int cpg = 1;
    chunk_plan(B, KVH, max_tiles, cs, &cpg, per_round);
    *n_wg = B * KVH * cpg;
    return;
  }
  // uneven lengths: chunks for about eight resident rounds, so that the
  // hardware dispatcher balances the sequences' partial chunks; a multiple of
  // `granule` tiles (4: one per wave of the 4-wave block_n = 256 kernel)
  const long long items = total_tiles * KVH;
  const long long resident = per_round > 0 ? per_round : resident_workgroups();
  const long long slack = static_cast<long long>(B) * KVH;
  const long long want = rounds * ((resident > 2 * slack) ? resident - slack : (resident + 1) / 2);
  long long c = (items + want - 1) / want;
  c = (c + granule - 1) / granule * granule;
  *cs = static_cast<int>(c);
  *n_wg = static_cast<int>(KVH * ((total_tiles + c - 1) / c + B));
}

}  // namespace flash
}  // namespace santa

using namespace santa;

extern "C" int santa_flash_plan(int64_t L_storage, int64_t valid_len, int64_t block_n, int64_t S, int* L_out,
                                int* block_n_out, int* T_c_out, int* S_per_tile_out) {
  const int64_t L = (valid_len > 0) ? valid_len : L_storage;
  if (L <= 0) return set_error(SANTA_ERR_INVALID, "valid_len must be > 0; got %lld", static_cast<long long>(L));
  if (L > L_storage)
    return set_error(SANTA_ERR_INVALID, "valid_len exceeds storage length: valid_len=%lld storage=%lld",
                     static_cast<long long>(L), static_cast<long long>(L_storage));
  int64_t bn = block_n;
  if (bn <= 0) bn = (L <= 1536) ? 32 : ((L <= 3072) ? 64 : 256);
  if (!(bn == 32 || bn == 64 || bn == 256))
    return set_error(SANTA_ERR_INVALID, "block_n must be 0 (auto) or one of {32,64,256}. Got block_n=%lld",
                     static_cast<long long>(bn));
  const int64_t T_c = (L + bn - 1) / bn;
  int64_t spt = 0;
  if (S > 0) {
    spt = S / T_c;
    if (spt < 1) spt = 1;
  }
  if (L_out) *L_out = static_cast<int>(L);
  if (block_n_out) *block_n_out = static_cast<int>(bn);
  if (T_c_out) *T_c_out = static_cast<int>(T_c);
  if (S_per_tile_out) *S_per_tile_out = static_cast<int>(spt);
  return clear_error();
}

static int check_flash_shape(int dtype, int B, int H, int KVH, int D, int L_valid, int L_storage, int block_n) {
  if (dtype != SANTA_BF16 && dtype != SANTA_F16) return set_error(SANTA_ERR_INVALID, "q_h must be bf16 or f16");
  if (B <= 0 || H <= 0 || KVH <= 0) return set_error(SANTA_ERR_INVALID, "empty batch/head dimension");
  if (L_valid <= 0) return set_error(SANTA_ERR_INVALID, "valid_len must be > 0; got %d", L_valid);
  if (L_valid > L_storage)
    return set_error(SANTA_ERR_INVALID, "valid_len exceeds storage length: valid_len=%d storage=%d", L_valid,
                     L_storage);
  if (D != 128) return set_error(SANTA_ERR_UNSUPPORTED, "This build supports only D=128. Got D=%d", D);
  if (H % KVH != 0) return set_error(SANTA_ERR_INVALID, "H must be divisible by KVH. Got H=%d KVH=%d", H, KVH);
  const int GH = H / KVH;
  if (GH != 4 && GH != 8)
    return set_error(SANTA_ERR_UNSUPPORTED, "This build supports only GH=4 or GH=8 (H/KVH). Got GH=%d (H=%d KVH=%d)",
                     GH, H, KVH);
  if (!(block_n == 32 || block_n == 64 || block_n == 256))
    return set_error(SANTA_ERR_INVALID, "block_n must be 0 (auto) or one of {32,64,256}. Got block_n=%d", block_n);
  const long long items = static_cast<long long>(B) * KVH * ((L_valid + block_n - 1) / block_n);
  if (items > 0x7fffffffLL) return set_error(SANTA_ERR_UNSUPPORTED, "too many tiles for one launch");
  return SANTA_OK;
}

extern "C" int santa_flash_fused_tiles(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH,
                                       int D, int L_valid, int L_storage, int block_n, int S_per_tile, uint64_t seed,
                                       float* m_tiles, float* ell_tiles, float* out_tiles, int* emit_cnt,
                                       int16_t* counts, hipStream_t stream) {
  int st = check_flash_shape(dtype, B, H, KVH, D, L_valid, L_storage, block_n);
  if (st != SANTA_OK) return st;
  if (!q || !K || !V || !m_tiles || !ell_tiles || !out_tiles || !emit_cnt)
    return set_error(SANTA_ERR_INVALID, "null pointer argument");
  flash::Args a{q, K, V, B, H, KVH, L_valid, L_storage, (L_valid + block_n - 1) / block_n, S_per_tile, seed,
                m_tiles, ell_tiles, out_tiles, emit_cnt, counts, nullptr, nullptr, 0, 0, nullptr};
  flash::chunk_plan(B, KVH, a.T_c, &a.cs, &a.cpg);
  hipError_t e = flash::launch_tiles<flash::kPerTile>(dtype, H / KVH, block_n, a, stream);
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "fused tile launch failed: %s", hipGetErrorString(e));
  return clear_error();
}

extern "C" int santa_flash_finalize(const float* m_tiles, const float* ell_tiles, const float* out_tiles,
                                    const int* emit_cnt, int dtype, int B, int H, int KVH, int D, int T_c,
                                    int S_per_tile, void* out, float* m_star, int* vrows, hipStream_t stream) {
  if (D != 128) return set_error(SANTA_ERR_UNSUPPORTED, "This build supports only D=128. Got D=%d", D);
  if (B <= 0 || H <= 0 || KVH <= 0 || H % KVH != 0 || T_c <= 0)
    return set_error(SANTA_ERR_INVALID, "bad finalize shape");
  if (!m_tiles || !ell_tiles || !out_tiles || !out || (vrows && !emit_cnt))
    return set_error(SANTA_ERR_INVALID, "null pointer argument");
  const size_t shmem = static_cast<size_t>(T_c + flash::kThreads) * sizeof(float);
  if (shmem > 64 * 1024) return set_error(SANTA_ERR_UNSUPPORTED, "T_c too large for the finalize kernel");
  const unsigned grid = static_cast<unsigned>(B) * static_cast<unsigned>(H);
  if (dtype == SANTA_BF16)
    hipLaunchKernelGGL(flash::finalize_kernel<true>, dim3(grid), dim3(flash::kThreads), shmem, stream, m_tiles,
                       ell_tiles, out_tiles, emit_cnt, H, KVH, T_c, S_per_tile, static_cast<uint16_t*>(out), m_star,
                       vrows);
  else
    hipLaunchKernelGGL(flash::finalize_kernel<false>, dim3(grid), dim3(flash::kThreads), shmem, stream, m_tiles,
                       ell_tiles, out_tiles, emit_cnt, H, KVH, T_c, S_per_tile, static_cast<uint16_t*>(out), m_star,
                       vrows);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "finalize launch failed: %s", hipGetErrorString(e));
  return clear_error();
}

namespace {
struct FlashWs {
  size_t part, emit, total;
  int cs, cpg;
};
FlashWs flash_ws_layout(int B, int H, int KVH, int T_c) {
  FlashWs w{};
  const bool rows = flash::rows_layout(KVH) && !flash::uniform_small_pass(B, KVH, T_c, H / KVH);
  flash::chunk_plan(B, KVH, T_c, &w.cs, &w.cpg, rows ? flash::rows_per_round() : 0);
  const size_t chunks = static_cast<size_t>(B) * KVH * w.cpg;
  const int GH = H / KVH;
  size_t off = 0;
  w.part = off;
  off = santa::align_up(off + chunks * GH * flash::kPartStride * sizeof(float));
  w.emit = off;
  off = santa::align_up(off + chunks * sizeof(int));
  w.total = off;
  return w;
}
}  // namespace

namespace santa {
namespace flash {
// Declared in santa_internal.h.
hipError_t launch_wave_debug(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH,
                             int L_valid, int L_storage, int S_pt, uint64_t seed, void* workspace, float* m_tiles,
                             float* ell_tiles, int16_t* counts, hipStream_t stream) {
  const int T_c = (L_valid + 255) / 256;
  const FlashWs w = flash_ws_layout(B, H, KVH, T_c);
  char* base = static_cast<char*>(workspace);
  Args a{q, K, V, B, H, KVH, L_valid, L_storage, T_c, S_pt, seed, nullptr, nullptr, nullptr, nullptr, nullptr,
         reinterpret_cast<float*>(base + w.part), reinterpret_cast<int*>(base + w.emit), w.cs, w.cpg, nullptr};
  return launch_wave(dtype, H / KVH, a, m_tiles, ell_tiles, counts, stream);
}
}  // namespace flash
}  // namespace santa

extern "C" size_t santa_flash_workspace_size(int B, int H, int KVH, int D, int T_c) {
  (void)D;
  if (B <= 0 || H <= 0 || KVH <= 0 || T_c <= 0 || H % KVH != 0) return 0;
  return flash_ws_layout(B, H, KVH, T_c).total;
}

static int flash_ws_check(int B, int H, int KVH, int T_c, void* workspace, size_t workspace_bytes, FlashWs* w) {
  *w = flash_ws_layout(B, H, KVH, T_c);
  if (!workspace || workspace_bytes < w->total)
    return set_error(SANTA_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", w->total, workspace_bytes);
  return SANTA_OK;
}

extern "C" int santa_flash_decode_tiles(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH,
                                        int D, int L_valid, int L_storage, int block_n, int S_per_tile, uint64_t seed,
                                        void* workspace, size_t workspace_bytes, hipStream_t stream) {
  int st = check_flash_shape(dtype, B, H, KVH, D, L_valid, L_storage, block_n);
  if (st != SANTA_OK) return st;
  if (!q || !K || !V) return set_error(SANTA_ERR_INVALID, "null pointer argument");
  const int T_c = (L_valid + block_n - 1) / block_n;
  FlashWs w;
  if ((st = flash_ws_check(B, H, KVH, T_c, workspace, workspace_bytes, &w)) != SANTA_OK) return st;
  char* base = static_cast<char*>(workspace);
  flash::Args a{q, K, V, B, H, KVH, L_valid, L_storage, T_c, S_per_tile, seed, nullptr, nullptr, nullptr, nullptr,
                nullptr, reinterpret_cast<float*>(base + w.part), reinterpret_cast<int*>(base + w.emit), w.cs, w.cpg,
                nullptr};
  const bool wave = block_n == 256 && !flash::uniform_small_pass(B, KVH, T_c, H / KVH);
  const hipError_t e = wave ? flash::launch_wave(dtype, H / KVH, a, nullptr, nullptr, nullptr, stream)
                            : flash::launch_tiles<flash::kOnline>(dtype, H / KVH, block_n, a, stream);
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "tile launch failed: %s", hipGetErrorString(e));
  return clear_error();
}

extern "C" int santa_flash_decode_merge(const void* workspace, size_t workspace_bytes, int dtype, int B, int H,
                                        int KVH, int D, int T_c, int S_per_tile, void* out, float* m_star, int* vrows,
                                        hipStream_t stream) {
  if (D != 128) return set_error(SANTA_ERR_UNSUPPORTED, "This build supports only D=128. Got D=%d", D);
  if (B <= 0 || H <= 0 || KVH <= 0 || H % KVH != 0 || T_c <= 0 || (H / KVH != 4 && H / KVH != 8))
    return set_error(SANTA_ERR_INVALID, "bad merge shape");
  if (!out) return set_error(SANTA_ERR_INVALID, "null pointer argument");
  FlashWs w;
  int st = flash_ws_check(B, H, KVH, T_c, const_cast<void*>(workspace), workspace_bytes, &w);
  if (st != SANTA_OK) return st;
  const char* base = static_cast<const char*>(workspace);
  const float* part = reinterpret_cast<const float*>(base + w.part);
  const int* pe = reinterpret_cast<const int*>(base + w.emit);
  const hipError_t e = flash::launch_merge(part, pe, dtype, B, H, KVH, w.cpg, S_per_tile, out, m_star, vrows, nullptr,
                                           0, 0, 0, 0, 0, stream);
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "merge launch failed: %s", hipGetErrorString(e));
  return clear_error();
}

extern "C" int santa_flash_decode(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH,
                                  int D, int L_valid, int L_storage, int block_n, int S_per_tile, uint64_t seed,
                                  void* out, float* m_star, int* vrows, void* workspace, size_t workspace_bytes,
                                  hipStream_t stream) {
  const int st = santa_flash_decode_tiles(q, K, V, dtype, B, H, KVH, D, L_valid, L_storage, block_n, S_per_tile, seed,
                                          workspace, workspace_bytes, stream);
  if (st != SANTA_OK) return st;
  return santa_flash_decode_merge(workspace, workspace_bytes, dtype, B, H, KVH, D, (L_valid + block_n - 1) / block_n,
                                  S_per_tile, out, m_star, vrows, stream);
}

// ------------------------------------------------- allocation-free decode
// santa_flash_decode with its workspace (the chunk partials and per-chunk
// emitted-row counts) in this file-scope device array instead of caller or
// allocator memory.  Each device holds its own copy for the life of the
// process.  Host code never passes the array's name to a kernel or a copy:
// the name is a host-side stand-in, not a device address.  Its address on a
// device comes from hipGetSymbolAddress, taken once per device with that
// device current and kept in s_scratch_ptr.
namespace {
constexpr size_t kScratchBytes = size_t{16} << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
std::mutex s_scratch_mu;
void* s_scratch_ptr[kMaxDevices];

// The scratch array's address on the current device (nullptr and the
// error recorded on failure).
void* scratch_on_current_device(int* status) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *status = set_error(SANTA_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *status = set_error(SANTA_ERR_UNSUPPORTED, "device %d: at most %d devices are supported", dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(s_scratch_mu);
  if (!s_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *status = set_error(SANTA_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                          hipGetErrorString(e));
      return nullptr;
    }
    s_scratch_ptr[dev] = p;
  }
  *status = SANTA_OK;
  return s_scratch_ptr[dev];
}
}  // namespace

extern "C" int santa_flash_decode_noalloc(const void* q, const void* K, const void* V, int dtype, int B, int H,
                                          int KVH, int D, int L_valid, int L_storage, int block_n, int S_per_tile,
                                          uint64_t seed, void* out, float* m_star, int* vrows, hipStream_t stream) {
  int st = check_flash_shape(dtype, B, H, KVH, D, L_valid, L_storage, block_n);
  if (st != SANTA_OK) return st;
  if (!q || !K || !V || !out) return set_error(SANTA_ERR_INVALID, "null pointer argument");
  const int T_c = (L_valid + block_n - 1) / block_n;
  // checked before any HIP call: a shape beyond the scratch array launches nothing
  const size_t need = flash_ws_layout(B, H, KVH, T_c).total;
  if (need > kScratchBytes)
    return set_error(SANTA_ERR_WORKSPACE,
                     "santa_flash_decode_noalloc: this shape needs %zu bytes of scratch; the static scratch holds "
                     "%zu (use santa_flash_decode with a workspace)",
                     need, kScratchBytes);
  void* ws = scratch_on_current_device(&st);
  if (!ws) return st;
  return santa_flash_decode(q, K, V, dtype, B, H, KVH, D, L_valid, L_storage, block_n, S_per_tile, seed, out, m_star,
                            vrows, ws, kScratchBytes, stream);
}

// ------------------------------------------------------------ ragged flash
namespace {
struct RaggedWs {
  size_t part, emit, total;
  int cs, n_wg;
};
// small: the tile kernel takes the pass (flash::small_pass), with the
// four-wave plan
RaggedWs ragged_ws_layout(int B, int H, int KVH, long long total_tiles, int max_tiles, bool small = false) {
  RaggedWs w{};
  const bool rows = flash::rows_layout(KVH) && !small;
  // The rows layout takes one round where the sequences' partial chunks
  // (B * KVH items at most) hold no more than an eighth of it (B <= 32 at KVH
  // 8), eight otherwise.  Each chunk costs its workgroup a start and an end
  // (first K after about 8 us, the V gathers and partial write after the
  // loop), which eight rounds of two- or three-tile chunks pay several times
  // per CU.  One round, against eight: cfg3's 16 lengths (8k-128k) 441.6 ->
  // 384.5 us per step, B = 8 at 16k-64k 172.3 -> 116.2, B = 4 at 32k-128k
  // 240.4 -> 131.8, B = 2 at 64k-128k 173.7 -> 89.4, B = 32 at 8k-32k 285.3
  // -> 247.4; but B = 12 at 1k-128k 325.2 -> 353.6, and at B = 40, 48 and 64
  // (a quarter of the round and more in partial chunks) 3-10 % slower.  The
  // loss at B = 12 (GH 8: 450.1 -> 589.6 us) is a sequence shorter than one
  // chunk (4 tiles against 12): it is one chunk, and S_per_tile = S / 4 puts
  // all its S samples per head, S * GH row gathers per wave in dependent
  // batches of 16, on one CU, where eight rounds split it in two.  The host
  // does not know the shortest length (the call carries total_tiles and
  // max_len), so the rule stands on the batches measured above.
  const int rounds = (rows && 8LL * B * KVH <= flash::rows_per_round()) ? 1 : 8;
  flash::plan_ragged(B, KVH, total_tiles, max_tiles, &w.cs, &w.n_wg, rows ? flash::rows_per_round() : 0,
                     rows ? 1 : 4, rounds);
  const size_t chunks = static_cast<size_t>(w.n_wg);
  size_t off = 0;
  w.part = off;
  off = santa::align_up(off + chunks * (H / KVH) * flash::kPartStride * sizeof(float));
  w.emit = off;
  off = santa::align_up(off + chunks * sizeof(int));
  w.total = off;
  return w;
}
}  // namespace

extern "C" size_t santa_flash_ragged_workspace_size(int B, int H, int KVH, int D, int max_tiles,
                                                    long long total_tiles) {
  (void)D;
  if (B <= 0 || H <= 0 || KVH <= 0 || H % KVH != 0 || max_tiles <= 0 || total_tiles < 0) return 0;
  // both plans a call may take (the small one only at block_n 256, which
  // this size does not know about)
  size_t bytes = ragged_ws_layout(B, H, KVH, total_tiles, max_tiles).total;
  if (flash::small_pass(total_tiles * KVH, H / KVH))
    bytes = std::max(bytes, ragged_ws_layout(B, H, KVH, total_tiles, max_tiles, true).total);
  return bytes;
}

// The ragged decode over a contiguous [B, L_storage, KVH, D] cache or, with
// pt.table set, a paged one (L_storage is then only checked against max_len).
static int flash_decode_ragged(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH, int D,
                               int L_storage, const int* seq_lens, int max_len, long long total_tiles, int block_n,
                               int64_t S, uint64_t seed, void* out, float* m_star, int* vrows, void* workspace,
                               size_t workspace_bytes, hipStream_t stream, const PageTable& pt) {
  int st = check_flash_shape(dtype, B, H, KVH, D, max_len, L_storage, block_n);
  if (st != SANTA_OK) return st;
  if (!q || !K || !V || !out || !seq_lens) return set_error(SANTA_ERR_INVALID, "null pointer argument");
  const int T_c = (max_len + block_n - 1) / block_n;
  if (total_tiles < 0 || total_tiles > static_cast<long long>(B) * T_c)
    return set_error(SANTA_ERR_INVALID, "total_tiles out of range");
  // little K: the tile kernel, for contiguous and paged caches alike (so that
  // the two stay bit-identical)
  const bool small = block_n == 256 && flash::small_pass(total_tiles * KVH, H / KVH);
  const RaggedWs w = ragged_ws_layout(B, H, KVH, total_tiles, T_c, small);
  if (!workspace || workspace_bytes < w.total)
    return set_error(SANTA_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", w.total, workspace_bytes);
  char* base = static_cast<char*>(workspace);
  float* part = reinterpret_cast<float*>(base + w.part);
  int* pe = reinterpret_cast<int*>(base + w.emit);
  flash::Args a{q, K, V, B, H, KVH, max_len, L_storage, T_c, 0, seed, nullptr, nullptr, nullptr, nullptr, nullptr,
                part, pe, w.cs, 0, nullptr, seq_lens, w.n_wg, static_cast<long long>(S), pt};
  hipError_t e = (block_n == 256 && !small) ? flash::launch_wave(dtype, H / KVH, a, nullptr, nullptr, nullptr, stream)
                                            : flash::launch_tiles<flash::kOnline>(dtype, H / KVH, block_n, a, stream);
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "tile launch failed: %s", hipGetErrorString(e));
  e = flash::launch_merge(part, pe, dtype, B, H, KVH, 0, 0, out, m_star, vrows, seq_lens, block_n, w.cs, max_len,
                          w.n_wg, static_cast<long long>(S), stream);
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "merge launch failed: %s", hipGetErrorString(e));
  return clear_error();
}

extern "C" int santa_flash_decode_ragged(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH,
                                         int D, int L_storage, const int* seq_lens, int max_len, long long total_tiles,
                                         int block_n, int64_t S, uint64_t seed, void* out, float* m_star, int* vrows,
                                         void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return flash_decode_ragged(q, K, V, dtype, B, H, KVH, D, L_storage, seq_lens, max_len, total_tiles, block_n, S, seed,
                             out, m_star, vrows, workspace, workspace_bytes, stream, PageTable{nullptr, 0, 3, 1});
}

extern "C" int santa_flash_decode_paged(const void* q, const void* K_pages, const void* V_pages, int dtype, int B,
                                        int H, int KVH, int D, int num_pages, int page_size, const int* block_table,
                                        int table_stride, const int* seq_lens, int max_len, long long total_tiles,
                                        int block_n, int64_t S, uint64_t seed, void* out, float* m_star, int* vrows,
                                        void* workspace, size_t workspace_bytes, hipStream_t stream) {
  PageTable pt{};
  const int st = check_page_table(block_table, num_pages, page_size, table_stride, max_len, &pt);
  if (st != SANTA_OK) return st;
  return flash_decode_ragged(q, K_pages, V_pages, dtype, B, H, KVH, D, max_len, seq_lens, max_len, total_tiles,
                             block_n, S, seed, out, m_star, vrows, workspace, workspace_bytes, stream, pt);
}
