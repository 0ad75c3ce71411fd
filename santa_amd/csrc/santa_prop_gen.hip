// santa_prop_gen.hip -- santa_prop on the shapes the tuned kernels of
// santa_flash.hip / santa_prop.hip do not take: any query-group size GH up to
// 16, head_dim D any multiple of 16 up to 1024, block_n any multiple of 16 up
// to 512 (the reference's general pass 1 takes D % 16 == 0 and
// block_n % 16 == 0, prop/santa_cuda.cpp:212-259; its pass 2 launches
// (128, GH) threads, prop/santa_cuda_kernel.cu:917-946), and more than 4096
// tiles per head in the budgets (the reference sizes that kernel's shared
// memory at T_c * 8 bytes, prop/santa_cuda_kernel.cu:904-915).
//
// Pass 1 rounds q after scaling, q' = TK(f32(q) * scale)
// (prop/santa_cuda_kernel.cu:121-140), and sums ell as the reference's WMMA
// kernel does: per 16-row slab in row order, then the slabs in order
// (:225-262).  The scores take one fixed association for what the reference
// leaves to its 16x16x16 MMA, the same for every D: virtual lanes of 4 dims
// chained with fma, then the shfl_down tree over the D / 4 lanes (for D = 128
// the vec path's association).
//
// Kernels (one decode step, as in santa_prop.hip):
//  * pass1_fast_kernel (block_n 256, D 64 / 128 / 256): four waves per tile,
//    a row per lane, K staged in swizzled LDS by 16-byte loads and scored on
//    the matrix pipe (broadcast 4x4x1 MFMA chains); for one head block a
//    workgroup streams a chunk of tiles, the next tile's rows in registers.
//    m_t, ell_t and the 16-bit u stash ([B, L_storage, H], or tile-major
//    [B, T, H, 256] inside the fused decode).
//  * pass1_kernel (every other D and block_n): one workgroup per (sequence,
//    KV head, tile), scalar fma chains read from LDS.
//  * budgets_big_kernel: the largest-remainder budgets of santa_prop.hip's
//    budgets_kernel (same m*, Z association, bases, jitter and bitonic
//    network, :577-726) with the network's keys in global memory (the
//    head's invdelta and a0 rows until their final values), for any number
//    of tiles.
//  * pass2_kernel: per (sequence, KV head, chunk of tiles), one wave per head
//    (up to four heads a wave): each head's systematic counts from the stash
//    (at block_n 256 the two-rows-per-lane DPP scan, otherwise 32-row chunks
//    with the reference's Hillis-Steele scan and sequential carry, :771-807),
//    its sampled rows ascending, and their count-weighted V rows summed with
//    fma (:843-857).
//  * finalize_kernel: out = dtype(sum over chunks * (1/S)) and vrows.
#include "santa_device.h"
#include "santa_amd.h"
#include "santa_internal.h"

#include <algorithm>
#include <atomic>
#include <type_traits>
#include <cfloat>

namespace santa {
namespace propgen {

constexpr int kThreads = 256;
constexpr int kMaxD = 1024;
constexpr int kMaxGH = 16;
constexpr int kMaxBN = 512;
constexpr int kStageElems = 64 * 256;  // 16-bit K elements staged in LDS at a time (64 rows at D <= 256)

bool generic_shape(int GH, int D, int block_n) {
  return !(D == 128 && (GH == 4 || GH == 8) && (block_n == 32 || block_n == 64 || block_n == 256));
}

bool shape_supported(int GH, int D, int block_n) {
  return GH >= 1 && GH <= kMaxGH && D >= 16 && D <= kMaxD && D % 16 == 0 && block_n >= 16 &&
         block_n <= kMaxBN && block_n % 16 == 0;
}

// Score of one (row, head) from the rounded q' (floats) and the 16-bit K row,
// in this build's general association: virtual lane v of P = D / 4 chains
// dims 4v .. 4v+3 with fma, then the shfl_down tree over the P lanes (at
// offsets N/2, ..., 1, N the next power of two >= P, lane l adds lane l + off
// when that lane holds a value).  The tree is summed depth first over the
// lanes in bit-reversed order -- its first pairs are lanes l and l + N/2 --
// so only log2(N) partial sums are live; float addition commutes, so each
// pair's sum is the tree's.  For D = 128 this is the vec path's association.
template <bool BF16>
__device__ __forceinline__ float score(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, int D) {
  const int P = D / 4;
  int lg = 0;
  while ((1 << lg) < P) ++lg;
  const int N = 1 << lg;
  float st[12];
  int lv[12];
  bool pr[12];
  int sp = 0;
  for (int i = 0; i < N; ++i) {
    const int v = lg > 0 ? static_cast<int>(__builtin_bitreverse32(static_cast<uint32_t>(i)) >> (32 - lg)) : 0;
    bool cp = v < P;
    float cur = 0.0f;
    if (cp) {
      cur = fmaf(h16_to_f32<BF16>(q[4 * v]), h16_to_f32<BF16>(k[4 * v]), 0.0f);
      cur = fmaf(h16_to_f32<BF16>(q[4 * v + 1]), h16_to_f32<BF16>(k[4 * v + 1]), cur);
      cur = fmaf(h16_to_f32<BF16>(q[4 * v + 2]), h16_to_f32<BF16>(k[4 * v + 2]), cur);
      cur = fmaf(h16_to_f32<BF16>(q[4 * v + 3]), h16_to_f32<BF16>(k[4 * v + 3]), cur);
    }
    int lvl = 0;
    while (sp > 0 && lv[sp - 1] == lvl) {
      --sp;
      if (pr[sp] && cp) {
        cur = st[sp] + cur;
      } else if (pr[sp]) {
        cur = st[sp];
      }
      cp = cp || pr[sp];
      ++lvl;
    }
    st[sp] = cur;
    lv[sp] = lvl;
    pr[sp] = cp;
    ++sp;
  }
  return st[0];
}

// Element offset of token n of sequence b, KV head kv (contiguous or paged).
template <bool PAGED>
__device__ __forceinline__ size_t row_offset(const PageTable& pt, int b, int n, int kv, int KVH, int D,
                                             int L_storage) {
  if constexpr (PAGED) {
    const int page = page_of_row(pt, b, n, true);
    return ((static_cast<size_t>(page) << pt.shift) + static_cast<size_t>(n & ((1 << pt.shift) - 1))) * KVH * D +
           static_cast<size_t>(kv) * D;
  } else {
    return (static_cast<size_t>(b) * L_storage + n) * KVH * D + static_cast<size_t>(kv) * D;
  }
}

// ------------------------------------------------------------------ pass 1
template <bool BF16, bool PAGED>
__global__ __launch_bounds__(kThreads) void pass1_kernel(const uint16_t* __restrict__ Q,
                                                         const uint16_t* __restrict__ K, int H, int KVH, int D,
                                                         int BN, int L_valid, int L_storage, int T_c, float q_scale,
                                                         float* __restrict__ m_tiles, float* __restrict__ ell_tiles,
                                                         uint16_t* __restrict__ u_stash,
                                                         const int* __restrict__ seq_lens, int B, PageTable pt) {
  const int GH = H / KVH;
  const GridPos gp = grid_pos(static_cast<int>(blockIdx.x), seq_lens, B, KVH, BN, L_valid, T_c, 1, T_c);
  if (gp.b < 0) return;
  const int b = gp.b, kv = gp.kv, t = gp.chunk;
  const int n0 = t * BN;
  const int len = min(BN, gp.len - n0);
  const int h0 = kv * GH;
  const int tid = static_cast<int>(threadIdx.x);

  __shared__ uint16_t s_q[kMaxGH * kMaxD];  // q' (already a 16-bit value)
  __shared__ uint16_t s_k[kStageElems];
  __shared__ float s_sc[kMaxBN * kMaxGH];
  __shared__ int s_mk[kMaxGH * 16];
  __shared__ float s_m[kMaxGH];
  __shared__ float s_part[kMaxGH * (kMaxBN / 16)];

  for (int i = tid; i < GH * D; i += kThreads) {
    const int g = i / D, d = i - (i / D) * D;
    const float qv = h16_to_f32<BF16>(Q[(static_cast<size_t>(b) * H + h0 + g) * D + d]) * q_scale;
    s_q[i] = f32_to_h16<BF16>(qv);
  }
  const int hw = D / 2;  // 4-byte words per row
  const int row_chunk = kStageElems / D;  // K rows staged at a time
  for (int r0 = 0; r0 < len; r0 += row_chunk) {
    const int nr = min(row_chunk, len - r0);
    __syncthreads();  // q' written; the previous chunk's rows read
    for (int i = tid; i < nr * hw; i += kThreads) {
      const int r = i / hw, w = i - (i / hw) * hw;
      const uint32_t* src =
          reinterpret_cast<const uint32_t*>(K + row_offset<PAGED>(pt, b, n0 + r0 + r, kv, KVH, D, L_storage));
      reinterpret_cast<uint32_t*>(s_k)[r * hw + w] = src[w];
    }
    __syncthreads();
    for (int i = tid; i < nr * GH; i += kThreads) {
      const int r = i / GH, g = i - (i / GH) * GH;
      s_sc[(r0 + r) * GH + g] = score<BF16>(s_q + g * D, s_k + r * D, D);
    }
  }
  __syncthreads();
  // tile max per head (order keys: exact in any order)
  if (tid < GH * 16) {
    const int g = tid / 16, p = tid % 16;
    int k = -2147483647 - 1;
    for (int r = p; r < len; r += 16) k = max(k, order_key(s_sc[r * GH + g]));
    s_mk[g * 16 + p] = k;
  }
  __syncthreads();
  if (tid < GH) {
    int k = s_mk[tid * 16];
    for (int p = 1; p < 16; ++p) k = max(k, s_mk[tid * 16 + p]);
    s_m[tid] = from_order_key(k);
  }
  __syncthreads();
  // u, the 16-bit stash and the slab partials of ell
  const int nslab = BN / 16;
  for (int i = tid; i < GH * nslab; i += kThreads) {
    const int g = i / nslab, w = i - (i / nslab) * nslab;
    const float mg = s_m[g];
    float part = 0.0f;
    for (int j = 0; j < 16; ++j) {
      const int r = 16 * w + j;
      if (r < len) {
        const float u = santa_expf(s_sc[r * GH + g] - mg);
        part += u;
        u_stash[(static_cast<size_t>(b) * L_storage + n0 + r) * H + h0 + g] = f32_to_h16<BF16>(u);
      }
    }
    s_part[g * nslab + w] = part;
  }
  __syncthreads();
  if (tid < GH) {
    float ell = 0.0f;
    for (int w = 0; w < nslab; ++w) ell += s_part[tid * nslab + w];
    const size_t mt = (static_cast<size_t>(b) * H + h0 + tid) * T_c + t;
    m_tiles[mt] = s_m[tid];
    ell_tiles[mt] = ell;
  }
}

// ------------------------------------------------------------ fast pass 1
// block_n 256 with D 64, 128 or 256 and any GH up to 16: one workgroup of
// four waves per (sequence, KV head, tile), wave w owning rows 64w .. 64w+63,
// one per lane.  The wave's rows come by 16-byte buffer loads straight into
// LDS, each lane fetching the piece that lands in the XOR-swizzled slot of its
// lane index (rows past the tile's end read as zero, with no traffic).  The
// scores run on the matrix pipe: for 8 dims at a time, v_mfma_f32_4x4x1f32
// with the A operand broadcast (q of four heads, one dim) and k of the lane's
// row as B, so each lane accumulates its row's four heads in place; a K=1
// MFMA is one fused multiply-add.  The chunk results are combined in the
// general association (virtual lanes of 4 dims, then the shfl_down tree over
// the D/4 lanes: its even lanes are chunk c's first half and its odd lanes
// the second, and over chunks the tree pairs c with c + D/16 first).  Then
// the tile max per head (one LDS exchange), u = exp(s - m), the 16-bit stash
// [B, L_storage, H] and ell: per 16-row slab in row order (a DPP chain inside
// each 16-lane row), then over the 16 slabs in order.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kBufWord3 = 0x00020000;  // raw buffer descriptor word 3 (gfx9 family)
constexpr int kBufNontemporal = 2;

template <int J>
__device__ __forceinline__ f32x4 mfma_bc(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, J, 0);
}

// Chunk C (dims 8C .. 8C+7) of this lane's row: the fma chains of virtual
// lanes 2C (e) and 2C+1 (o) for the head block whose broadcast q is qa
// (register m: dims 16m .. 16m+15, lane 4j+i: head i, dim 16m+j).
template <bool BF16, int NS, int C>
__device__ __forceinline__ void fast_leaf(const u32x4* wk, int row, const float* qa, f32x4& e, f32x4& o) {
  const u32x4 kc = wk[row * NS + (C ^ (row & (NS - 1)))];
  const float k0 = lo16_to_f32<BF16>(kc.x), k1 = hi16_to_f32<BF16>(kc.x);
  const float k2 = lo16_to_f32<BF16>(kc.y), k3 = hi16_to_f32<BF16>(kc.y);
  const float k4 = lo16_to_f32<BF16>(kc.z), k5 = hi16_to_f32<BF16>(kc.z);
  const float k6 = lo16_to_f32<BF16>(kc.w), k7 = hi16_to_f32<BF16>(kc.w);
  constexpr int M = C / 2;
  constexpr int J = 8 * (C % 2);
  const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
  const float q = qa[M];
  f32x4 de = mfma_bc<J + 0>(q, k0, z);
  f32x4 dd = mfma_bc<J + 4>(q, k4, z);
  de = mfma_bc<J + 1>(q, k1, de);
  dd = mfma_bc<J + 5>(q, k5, dd);
  de = mfma_bc<J + 2>(q, k2, de);
  dd = mfma_bc<J + 6>(q, k6, dd);
  de = mfma_bc<J + 3>(q, k3, de);
  dd = mfma_bc<J + 7>(q, k7, dd);
  e = de;
  o = dd;
}

// The shfl_down tree over the chunks {R, R + S, R + 2S, ...} below NS: the
// trees over {R, R + 2S, ...} and {R + S, R + 3S, ...} summed (the leaves R
// and R + NS/2 form the first pairs).
template <bool BF16, int NS, int R, int S>
__device__ __forceinline__ void fast_tree(const u32x4* wk, int row, const float* qa, f32x4& e, f32x4& o) {
  if constexpr (S == NS) {
    fast_leaf<BF16, NS, R>(wk, row, qa, e, o);
  } else {
    f32x4 e1, o1, e2, o2;
    fast_tree<BF16, NS, R, 2 * S>(wk, row, qa, e1, o1);
    fast_tree<BF16, NS, R + S, 2 * S>(wk, row, qa, e2, o2);
    e = e1 + e2;
    o = o1 + o2;
    // a scheduling fence after each subtree of four leaves keeps eight MFMA
    // chains in flight rather than every leaf's accumulators live at once
    if constexpr (4 * S == NS) __builtin_amdgcn_sched_barrier(0);
  }
}

bool fast_pass1_shape(int GH, int D, int block_n) {
  return block_n == 256 && (D == 64 || D == 128 || D == 256) && GH >= 1 && GH <= kMaxGH;
}

// Workgroups per CU of pass1_fast_kernel: its LDS staging (64 rows of D
// 16-bit values per wave) allows two at D = 128 and four at D = 64, where one
// head block fits 128 registers (B = 8, 32k tokens, GQA 4: 95.1 -> 91.1 us per
// step against two); D = 256, and four head blocks (whose scores, exps and
// the next tile's rows need more than half the registers), take one.
template <int D, int NHB>
constexpr int fast_occupancy() {
  return (D == 256 || (D == 128 && NHB == 4)) ? 1 : ((D == 64 && NHB == 1) ? 4 : 2);
}
static int fast_occupancy(int D, int nhb) {
  return (D == 256 || (D == 128 && nhb == 4)) ? 1 : ((D == 64 && nhb == 1) ? 4 : 2);
}
// Whether the next tile's rows are held in registers while a tile is scored
// (D / 2 registers); the wider shapes load each tile straight into the
// staging instead, and rely on the other resident workgroup to cover the wait.
template <int D, int NHB>
constexpr bool fast_prefetch() {
  return NHB == 1 || (D == 64 && NHB == 2);
}

template <bool BF16, int D, int NHB, bool PAGED>
__global__ __launch_bounds__(kThreads, (fast_occupancy<D, NHB>())) void pass1_fast_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, int H, int KVH, int L_valid, int L_storage,
    int T_c, int cs, int cpg, float q_scale, float* __restrict__ m_tiles, float* __restrict__ ell_tiles,
    uint16_t* __restrict__ u_stash, const int* __restrict__ seq_lens, int B, PageTable pt, int stash_ld) {
  constexpr int BN = 256;
  constexpr int NS = D / 8;     // 16-byte slots (8-dim chunks) per K row
  constexpr int RPL = 64 / NS;  // rows per 64-lane load
  constexpr int NQ = D / 16;    // broadcast q registers per head block
  const int GH = H / KVH;
  // one (sequence, KV head, chunk of cs tiles) per workgroup
  const GridPos gp = grid_pos(static_cast<int>(blockIdx.x), seq_lens, B, KVH, BN, L_valid, T_c, cs, cpg);
  if (gp.b < 0) return;
  const int b = gp.b, kv = gp.kv;
  const int t_begin = gp.chunk * cs;
  const int t_end = min(gp.n_tiles, t_begin + cs);
  const int h0 = kv * GH;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  __shared__ u32x4 s_k[4 * 64 * NS];
  __shared__ int s_wmax[2][4][4 * NHB];      // by tile parity: the next tile's writes
  __shared__ float s_slab[2][4 * NHB][16];   // never meet this tile's late reads
  u32x4* const wk = s_k + wave * 64 * NS;

  // This wave's rows n0 + 64 wave .. + 63 of a tile, register form: load i
  // holds rows RPL i .. RPL i + RPL - 1, lane l the piece (l % NS) ^ (row &
  // (NS - 1)) of row RPL i + l / NS, which is the staging slot 64 i + l
  // (rows past the tile's end read as zero, with no traffic).  The next
  // tile's loads are in flight while this one is scored.
  const uint32_t row_bytes = static_cast<uint32_t>(KVH) * D * 2u;
  const int wrow0 = 64 * wave;
  constexpr bool PF = fast_prefetch<D, NHB>();
  u32x4 kw[PF ? NS : 1];
  // one load of this wave's rows of tile t: to registers (PF) or straight
  // into the staging
  auto load_rows = [&](int t) {
    // the lane index through an empty asm, so that the per-load offsets are
    // recomputed at each tile rather than held in registers across the loop
    int l = lane;
    asm volatile("" : "+v"(l));
    const int rl = l / NS, sl = l % NS;
    const int n0 = t * BN;
    const int nrows = min(max(min(BN, gp.len - n0) - wrow0, 0), 64);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int nvalid = __builtin_amdgcn_readfirstlane(min(max(nrows - i * RPL, 0), RPL));
      const int n = n0 + wrow0 + i * RPL;  // first token of the load (RPL tokens lie in one page)
      size_t base;
      if constexpr (PAGED) {
        const int page = __builtin_amdgcn_readfirstlane(page_of_row(pt, b, n, nvalid > 0));
        base = ((static_cast<size_t>(page) << pt.shift) + static_cast<size_t>(n & ((1 << pt.shift) - 1))) * KVH * D +
               static_cast<size_t>(kv) * D;
      } else {
        base = (static_cast<size_t>(b) * L_storage + n) * KVH * D + static_cast<size_t>(kv) * D;
      }
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(K + base), static_cast<short>(0), nvalid * static_cast<int>(row_bytes), kBufWord3);
      const uint32_t voff = static_cast<uint32_t>(rl) * row_bytes +
                            16u * static_cast<uint32_t>(sl ^ ((i * RPL + rl) & (NS - 1)));
      if constexpr (PF) {
        kw[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 0, kBufNontemporal));
      } else {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(wk + 64 * i), 16, voff,
                                                 0, 0, kBufNontemporal);
      }
    }
  };
  if constexpr (PF) {
    load_rows(t_begin);
  } else {
    load_rows(t_begin);  // one tile per workgroup: its rows first, then q
  }

  // q' = TK(f32(q) * scale) of each head block, broadcast layout (heads past
  // GH are 0 and their results unused)
  float qa[NHB][NQ];
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb) {
    const int g = 4 * hb + (lane & 3);
#pragma unroll
    for (int m = 0; m < NQ; ++m) {
      float v = 0.0f;
      if (g < GH) {
        const float qv = h16_to_f32<BF16>(Q[(static_cast<size_t>(b) * H + h0 + g) * D + 16 * m + (lane >> 2)]) * q_scale;
        v = h16_to_f32<BF16>(f32_to_h16<BF16>(qv));
      }
      qa[hb][m] = v;
    }
  }

  const int slab = 4 * wave + (lane >> 4);
  auto tile = [&](int t) {
    const int par = (t - t_begin) & 1;
    const int n0 = t * BN;
    const int len = min(BN, gp.len - n0);
    if constexpr (PF) {
      // the tile's rows into this wave's staging (its previous reads are
      // done: LDS accesses of one wave complete in order), then the next
      // tile's loads
#pragma unroll
      for (int i = 0; i < NS; ++i) wk[64 * i + lane] = kw[i];
      if (t + 1 < t_end) load_rows(t + 1);
    } else {
      // (the loads to LDS are not ordered before LDS reads by the compiler)
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __builtin_amdgcn_wave_barrier();

    // (the row through an empty asm: the staging addresses are recomputed at
    // each tile rather than held in registers across the loop)
    int row = lane;
    asm volatile("" : "+v"(row));
    f32x4 sc[NHB];
#pragma unroll
    for (int hb = 0; hb < NHB; ++hb) {
      f32x4 e, o;
      fast_tree<BF16, NS, 0, 1>(wk, row, qa[hb], e, o);
      sc[hb] = e + o;
      __builtin_amdgcn_sched_barrier(0);
    }

    // tile max per head (order keys: exact in any order)
    const bool valid = wrow0 + lane < len;
#pragma unroll
    for (int hb = 0; hb < NHB; ++hb)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        int key = valid ? order_key(sc[hb][k]) : (-2147483647 - 1);
        key = wave_max_key_lane63(key);
        const int wm = __builtin_amdgcn_readlane(key, 63);
        if (lane == 0) s_wmax[par][wave][4 * hb + k] = wm;
      }
    __syncthreads();

    uint32_t bits[NHB][4];
#pragma unroll
    for (int hb = 0; hb < NHB; ++hb)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int g = 4 * hb + k;
        const float mg = from_order_key(max(max(s_wmax[par][0][g], s_wmax[par][1][g]),
                                            max(s_wmax[par][2][g], s_wmax[par][3][g])));
        const float u = valid ? santa_expf_nonpos(sc[hb][k] - mg) : 0.0f;
        bits[hb][k] = BF16 ? (__float_as_uint(round16_nonneg<true>(u)) >> 16)
                           : static_cast<uint32_t>(f32_to_h16<false>(u));
        // the slab's sum in row order at its last lane: ((u0 + u1) + u2) + ...
        float a = u;
#pragma unroll
        for (int j = 1; j < 16; ++j) a = dpp_shr_zero<1>(a) + u;
        if ((lane & 15) == 15) s_slab[par][g][slab] = a;
      }
    if (stash_ld > 0) {
      // tile-major [B, T, H, 256]: per head the wave's 64 rows as one 128-B
      // run (0 past len), where [L, H] would scatter 2-B pieces H * 2 B apart
      uint16_t* dst = u_stash + static_cast<size_t>(b) * H * stash_ld + (static_cast<size_t>(t) * H + h0) * BN +
                      wrow0 + lane;
#pragma unroll
      for (int hb = 0; hb < NHB; ++hb)
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (4 * hb + k < GH) dst[(4 * hb + k) * BN] = static_cast<uint16_t>(bits[hb][k]);
    } else if (valid) {
      uint16_t* dst = u_stash + (static_cast<size_t>(b) * L_storage + n0 + wrow0 + lane) * H + h0;
#pragma unroll
      for (int hb = 0; hb < NHB; ++hb)
#pragma unroll
        for (int k = 0; k < 4; k += 2) {
          const int g = 4 * hb + k;
          if (GH % 2 == 0) {
            if (g < GH) *reinterpret_cast<uint32_t*>(dst + g) = bits[hb][k] | (bits[hb][k + 1] << 16);
          } else {
            if (g < GH) dst[g] = static_cast<uint16_t>(bits[hb][k]);
            if (g + 1 < GH) dst[g + 1] = static_cast<uint16_t>(bits[hb][k + 1]);
          }
        }
    }
    __syncthreads();
    if (tid < GH) {
      float ell = 0.0f;
#pragma unroll
      for (int w = 0; w < 16; ++w) ell += s_slab[par][tid][w];
      const size_t mt = (static_cast<size_t>(b) * H + h0 + tid) * T_c + t;
      m_tiles[mt] = from_order_key(max(max(s_wmax[par][0][tid], s_wmax[par][1][tid]),
                                       max(s_wmax[par][2][tid], s_wmax[par][3][tid])));
      ell_tiles[mt] = ell;
    }
  };
  if constexpr (PF) {
    for (int t = t_begin; t < t_end; ++t) tile(t);
  } else {
    tile(t_begin);
  }
}

// ----------------------------------------------------------------- budgets
// One workgroup per (sequence, head).  The network only reads and writes
// positions below the tile count (the rest read as (-inf, -1)), so its
// (key, index) pairs live in this head's rows of invdelta and a0 (as int
// bits) until the last phase writes their final values.
constexpr int kBudgetThreads = 1024;

__global__ __launch_bounds__(kBudgetThreads) void budgets_big_kernel(
    const float* __restrict__ m_tiles, const float* __restrict__ ell_tiles, int H, int T_c, int S, uint64_t seed,
    float* __restrict__ m_star, int* __restrict__ S_tiles, float* __restrict__ invdelta, float* __restrict__ a0_tile,
    const int* __restrict__ seq_lens, const int* __restrict__ seq_S, int BN) {
  __shared__ float s_red[kBudgetThreads / 64];
  __shared__ long long s_lred[kBudgetThreads / 64];
  __shared__ float s_z[128];
  const int bh = static_cast<int>(blockIdx.x);
  const int h = bh % H;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63, wv = tid >> 6;
  const size_t off = static_cast<size_t>(bh) * T_c;
  int T = T_c;
  if (seq_lens) T = (ragged_len(seq_lens, bh / H, T_c * BN) + BN - 1) / BN;
  if (seq_S) S = seq_S[bh / H];
  const float* mt = m_tiles + off;
  const float* lt = ell_tiles + off;
  float* f = invdelta + off;
  int* ix = reinterpret_cast<int*>(a0_tile + off);

  // m* = max_t m_t (exact in any order), from -FLT_MAX as in :597
  float ms = -FLT_MAX;
  for (int t = tid; t < T; t += kBudgetThreads) ms = fmaxf(ms, mt[t]);
  for (int s = 32; s > 0; s >>= 1) ms = fmaxf(ms, __shfl_xor(ms, s, 64));
  if (lane == 0) s_red[wv] = ms;
  __syncthreads();
  ms = s_red[0];
  for (int i = 1; i < kBudgetThreads / 64; ++i) ms = fmaxf(ms, s_red[i]);
  if (tid == 0 && m_star) m_star[bh] = ms;
  // W_t, then Z: 128 partials over tiles tau, tau + 128, ... ascending, then
  // the pairwise tree red[i] += red[i + s], s = 64 .. 1
  for (int t = tid; t < T; t += kBudgetThreads) f[t] = santa_expf(mt[t] - ms) * lt[t];
  __syncthreads();
  if (tid < 128) {
    float z = 0.0f;
    for (int t = tid; t < T; t += 128) z += f[t];
    s_z[tid] = z;
  }
  __syncthreads();
  for (int s = 64; s > 0; s >>= 1) {
    if (tid < s) s_z[tid] = s_z[tid] + s_z[tid + s];
    __syncthreads();
  }
  const float Z = s_z[0];
  if (S <= 0 || !(Z > 0.0f)) {
    for (int t = tid; t < T; t += kBudgetThreads) {
      S_tiles[off + t] = 0;
      invdelta[off + t] = 0.0f;
      a0_tile[off + t] = u01(seed, h, t);
    }
    return;
  }
  // integer bases and jittered fractional parts (:662-678)
  long long base = 0;
  for (int t = tid; t < T; t += kBudgetThreads) {
    const float q = static_cast<float>(S) * (f[t] / Z);
    const float fq = floorf(q);
    const int bt = (fq != fq) ? 0 : (fq >= 2147483648.0f ? 2147483647 : static_cast<int>(fq));
    S_tiles[off + t] = bt;
    base += bt;
    f[t] = (q - static_cast<float>(bt)) + 1.0e-7f * u01(seed, h, t);
    ix[t] = t;
  }
  for (int s = 32; s > 0; s >>= 1) base += __shfl_xor(base, s, 64);
  if (lane == 0) s_lred[wv] = base;
  __syncthreads();
  base = 0;
  for (int i = 0; i < kBudgetThreads / 64; ++i) base += s_lred[i];
  long long rem = static_cast<long long>(S) - base;
  if (rem < 0) rem = 0;
  if (rem > T) rem = T;
  // the bitonic network over N = next power of two >= T (:686-707): the pair
  // (i, i ^ j) with i the lower position swaps when (a_i > a_j) == (i & k);
  // positions >= T read as (-inf, -1) and are never written
  int N = 1;
  while (N < T) N <<= 1;
  for (int k = 2; k <= N; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int p = tid; p < N / 2; p += kBudgetThreads) {
        const int i = (p / j) * 2 * j + (p % j);
        const int ixj = i + j;
        const bool up = (i & k) != 0;
        float ai = (i < T) ? f[i] : -__builtin_inff();
        float aj = (ixj < T) ? f[ixj] : -__builtin_inff();
        int ii = (i < T) ? ix[i] : -1;
        int ij = (ixj < T) ? ix[ixj] : -1;
        if ((ai > aj) == up) {
          const float tf = ai;
          ai = aj;
          aj = tf;
          const int ti = ii;
          ii = ij;
          ij = ti;
        }
        if (i < T) {
          f[i] = ai;
          ix[i] = ii;
        }
        if (ixj < T) {
          f[ixj] = aj;
          ix[ixj] = ij;
        }
      }
      __syncthreads();
    }
  }
  // +1 to the top `rem` (distinct tiles, :710-716)
  for (int r = tid; r < rem; r += kBudgetThreads) {
    const int best = ix[r];
    if (best >= 0) S_tiles[off + best] += 1;
  }
  __syncthreads();
  __syncthreads();  // the pairs' last reads are done before they are overwritten
  for (int t = tid; t < T; t += kBudgetThreads) {
    const int s_t = S_tiles[off + t];
    const float ell = lt[t];
    invdelta[off + t] = (s_t > 0 && ell > 1e-20f) ? (static_cast<float>(s_t) / ell) : 0.0f;
    a0_tile[off + t] = u01(seed, h, t);
  }
}

// ------------------------------------------------------------------ pass 2
// One workgroup of NWV = min(GH, 4) waves per (sequence, KV head, chunk of
// tiles); wave w takes heads w, w + NWV, ... over every tile of the chunk (so
// no wave idles when GH < 4; the chunk plan then counts the smaller
// workgroups).  Per (head, tile): x_r = f32(u16 stash) * invdelta_t, the
// systematic counts (at block_n 256 two rows per lane with the DPP scan of
// santa_device.h, else 32-row pieces with the lane scan; both the
// reference's 32-lane Hillis-Steele scan with a sequential carry,
// :771-807), the sampled rows ascending, and their count-weighted V rows
// added with one fma per element in row order (:843-857), up to 16 rows'
// loads in flight at a time.  Lane l holds dims DPL l .. DPL l + DPL - 1.
constexpr int kGatherRows = 16;
constexpr int kMaxHeadsPerWave = kMaxGH / 4;

template <int DPL>
__device__ __forceinline__ void load_dims(const uint16_t* p, uint16_t (&v)[DPL]) {
  if constexpr (DPL == 1) {
    v[0] = p[0];
  } else if constexpr (DPL == 2) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    v[0] = static_cast<uint16_t>(w & 0xffffu);
    v[1] = static_cast<uint16_t>(w >> 16);
  } else {
#pragma unroll
    for (int c = 0; c < DPL / 4; ++c) {
      const uint2 w = reinterpret_cast<const uint2*>(p)[c];
      v[4 * c] = static_cast<uint16_t>(w.x & 0xffffu);
      v[4 * c + 1] = static_cast<uint16_t>(w.x >> 16);
      v[4 * c + 2] = static_cast<uint16_t>(w.y & 0xffffu);
      v[4 * c + 3] = static_cast<uint16_t>(w.y >> 16);
    }
  }
}

// T256: block_n is 256 (the two-rows-per-lane path only; compiled apart so
// that the other path's per-piece bounds are not computed for it).  NK: the
// most heads a wave takes (1 for GH <= 4, 2 for GH <= 8, else
// kMaxHeadsPerWave), which sizes the unrolled per-head state.
template <bool BF16, bool PAGED, int DPL, bool T256, int NK>
__global__ __launch_bounds__(kThreads) void pass2_kernel(const uint16_t* __restrict__ V,
                                                         const uint16_t* __restrict__ u_stash, int H, int KVH, int D,
                                                         int BN_arg, int L, int L_storage, int T_c, int cs, int cpg,
                                                         const float* __restrict__ invdelta,
                                                         const float* __restrict__ a0_tile,
                                                         int16_t* __restrict__ dbg_counts, float* __restrict__ part,
                                                         int* __restrict__ part_emit, int want_emit,
                                                         const int* __restrict__ seq_lens, int B, PageTable pt,
                                                         int stash_ld) {
  const int BN = T256 ? 256 : BN_arg;
  const int GH = H / KVH;
  const int wg = static_cast<int>(blockIdx.x);
  const GridPos gp = grid_pos(wg, seq_lens, B, KVH, BN, L, T_c, cs, cpg);
  const int b = gp.b < 0 ? 0 : gp.b;
  const int kv = gp.kv;
  const int h0 = kv * GH;
  L = gp.len;
  const int t_begin = gp.chunk * cs;
  const int t_end = (gp.b < 0) ? t_begin : min(gp.n_tiles, t_begin + cs);
  const int tid = static_cast<int>(threadIdx.x);
  const int nthreads = static_cast<int>(blockDim.x);
  const int nwv = nthreads >> 6;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int jrow = lane >> 4;
  const int qq = lane & 15;

  // LDS sized by the launch (pass2_lds_bytes): per wave and head k (block_n
  // 256; one list otherwise) BN listed rows and their counts, then BN
  // emitted-row flags and the tile's emitted total
  constexpr int NL = T256 ? NK : 1;  // lists per wave
  extern __shared__ int s_p2[];
  int* const s_lrow = s_p2 + wave * NL * BN;
  float* const s_lc = reinterpret_cast<float*>(s_p2 + nwv * NL * BN) + wave * NL * BN;
  int* const s_flag = s_p2 + 2 * nwv * NL * BN;
  int* const s_nemit = s_flag + BN;

  static_assert(NK == 1 || NK == 2 || NK == kMaxHeadsPerWave, "heads per wave");
  float acc[NK][DPL];
  int lcnt[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    lcnt[k] = 0;
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[k][j] = 0.0f;
  }
  int emit_total = 0;
  const uint16_t* ub = u_stash + static_cast<size_t>(b) * L_storage * H;
  const int d0 = DPL * lane;  // this lane's first dim

  // Head k's listed rows, in list order, into its numerator: count-weighted
  // V rows, one fma per element, in batches of 16 rows whose loads go out
  // before the first is used, then what is left in batches of 4.  At block_n
  // 256 a head's list collects the rows of consecutive tiles and is gathered
  // when the next tile's rows would not fit and at the end of the chunk (the
  // same ascending (tile, row) fma order as a gather per tile, so the same
  // bits, with fewer memory round trips); otherwise after every tile.
  auto flush = [&](int k) {
    const int n = lcnt[k];
    int* const lrow = s_lrow + (T256 ? k : 0) * BN;
    float* const lcw = s_lc + (T256 ? k : 0) * BN;
    auto gather = [&](auto nb, int i0) {
      constexpr int NB = decltype(nb)::value;
      uint16_t vv[NB][DPL];
      float cf[NB];
#pragma unroll
      for (int q = 0; q < NB; ++q) {
        const int i = min(i0 + q, n - 1);
        const int row = __builtin_amdgcn_readfirstlane(lrow[i]);
        cf[q] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(lcw[i])));
        if (d0 < D) {
          load_dims<DPL>(V + row_offset<PAGED>(pt, b, row, kv, KVH, D, L_storage) + d0, vv[q]);
        } else {
#pragma unroll
          for (int j = 0; j < DPL; ++j) vv[q][j] = 0;
        }
      }
#pragma unroll
      for (int q = 0; q < NB; ++q) {
        if (i0 + q < n) {
#pragma unroll
          for (int j = 0; j < DPL; ++j) acc[k][j] = fmaf(cf[q], h16_to_f32<BF16>(vv[q][j]), acc[k][j]);
        }
      }
    };
    int i0 = 0;
    for (; i0 + kGatherRows <= n; i0 += kGatherRows) gather(std::integral_constant<int, kGatherRows>{}, i0);
    for (; i0 < n; i0 += 4) gather(std::integral_constant<int, 4>{}, i0);
    lcnt[k] = 0;
    __builtin_amdgcn_wave_barrier();
  };

  for (int t = t_begin; t < t_end; ++t) {
    const int n0 = t * BN;
    const int len = min(BN, L - n0);
    if (want_emit) {
      for (int r = tid; r < BN; r += nthreads) s_flag[r] = 0;
      __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      const int g = wave + nwv * k;
      if (g >= GH) break;
      const int h = h0 + g;
      const size_t ht = (static_cast<size_t>(b) * H + h) * T_c + t;
      const float inv = invdelta[ht];
      const float a0 = a0_tile[ht];
      if (!(inv > 0.0f)) {
        // a zero budget on this tile: every count is 0, nothing is listed
        if (dbg_counts)
          for (int r = lane; r < BN; r += 64) dbg_counts[ht * BN + r] = 0;
        continue;
      }
      if constexpr (T256) {
        // two rows per lane: rows 32 (4p + j) + 2q (x0) and + 1 (x1) at lane 16j + q
        float x0[2], x1[2];
        if (stash_ld > 0) {
          // tile-major stash (whole tiles): the lane's two rows as one 4-B load
          const uint16_t* ut = u_stash + static_cast<size_t>(b) * H * stash_ld + (static_cast<size_t>(t) * H + h) * BN;
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            const int row = 32 * (4 * p + jrow) + 2 * qq;
            const uint32_t w2 = *reinterpret_cast<const uint32_t*>(ut + row);
            x0[p] = (row < len) ? h16_to_f32<BF16>(static_cast<uint16_t>(w2 & 0xffffu)) * inv : 0.0f;
            x1[p] = (row + 1 < len) ? h16_to_f32<BF16>(static_cast<uint16_t>(w2 >> 16)) * inv : 0.0f;
          }
        } else {
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            const int row = 32 * (4 * p + jrow) + 2 * qq;
            x0[p] = (row < len) ? h16_to_f32<BF16>(ub[static_cast<size_t>(n0 + row) * H + h]) * inv : 0.0f;
            x1[p] = (row + 1 < len) ? h16_to_f32<BF16>(ub[static_cast<size_t>(n0 + row + 1) * H + h]) * inv : 0.0f;
          }
        }
        int c0[2], c1[2];
        systematic_counts<8>(x0, x1, len, a0, lane, c0, c1);
        const uint64_t below = (1ull << lane) - 1ull;
        uint64_t nz0[2], nz1[2];
        int cnt = 0;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          nz0[p] = __ballot(c0[p] != 0);
          nz1[p] = __ballot(c1[p] != 0);
          cnt += __popcll(nz0[p]) + __popcll(nz1[p]);
        }
        if (lcnt[k] + cnt > BN) flush(k);
        int* const lrow = s_lrow + k * BN;
        float* const lcw = s_lc + k * BN;
        int lc = lcnt[k];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int row = 32 * (4 * p + jrow) + 2 * qq;
          if (dbg_counts) {
            dbg_counts[ht * BN + row] = static_cast<int16_t>(c0[p]);
            dbg_counts[ht * BN + row + 1] = static_cast<int16_t>(c1[p]);
          }
          const int pos0 = lc + __popcll(nz0[p] & below) + __popcll(nz1[p] & below);
          const int pos1 = pos0 + (c0[p] != 0 ? 1 : 0);
          if (c0[p] != 0) {
            lrow[pos0] = n0 + row;
            lcw[pos0] = static_cast<float>(c0[p]);
            if (want_emit) s_flag[row] = 1;
          }
          if (c1[p] != 0) {
            lrow[pos1] = n0 + row + 1;
            lcw[pos1] = static_cast<float>(c1[p]);
            if (want_emit) s_flag[row + 1] = 1;
          }
          lc += __popcll(nz0[p]) + __popcll(nz1[p]);
        }
        lcnt[k] = lc;
        __builtin_amdgcn_wave_barrier();
      } else {
        int lc = 0;
        float carry = 0.0f;
        for (int base = 0; base < len; base += 32) {
          const int r = base + lane;
          const bool in = lane < 32 && r < len;
          const float x = in ? h16_to_f32<BF16>(ub[static_cast<size_t>(n0 + r) * H + h]) * inv : 0.0f;
          // Hillis-Steele inclusive scan over 32 lanes, then res - x
          // (flash/santa_cuda_kernel.cu:60-69)
          float res = x;
#pragma unroll
          for (int off = 1; off < 32; off <<= 1) {
            const float o = __shfl_up(res, off, 32);
            res = ((lane & 31) >= off) ? res + o : res;
          }
          const float pre = res - x;
          const float pre_g = carry + pre;
          const float cum_g = pre_g + x;
          const int c = in ? count_from_floors(a0, pre_g, cum_g) : 0;
          const int last = min(31, len - base - 1);
          const float chunk_total = __shfl(pre + x, last, 64);
          carry = carry + chunk_total;
          if (dbg_counts && lane < 32 && r < BN) dbg_counts[ht * BN + r] = static_cast<int16_t>(c);
          const uint64_t nz = __ballot(c != 0);
          if (c != 0) {
            const int pos = lc + __popcll(nz & ((1ull << lane) - 1ull));
            s_lrow[pos] = n0 + r;
            s_lc[pos] = static_cast<float>(c);
            if (want_emit) s_flag[r] = 1;
          }
          lc += __popcll(nz);
        }
        if (dbg_counts)
          for (int r = ((len + 31) / 32) * 32 + lane; r < BN; r += 64) dbg_counts[ht * BN + r] = 0;
        __builtin_amdgcn_wave_barrier();
        lcnt[k] = lc;
        flush(k);
      }
    }
    if (want_emit) {
      __syncthreads();
      if (wave == 0) {
        int e = 0;
        for (int r = lane; r < BN; r += 64) e += s_flag[r];
        for (int s = 32; s > 0; s >>= 1) e += __shfl_xor(e, s, 64);
        if (lane == 0) *s_nemit = e;
      }
      __syncthreads();
      emit_total += *s_nemit;
    }
  }
  if constexpr (T256) {
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      if (wave + nwv * k >= GH) break;
      flush(k);
    }
  }
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int g = wave + nwv * k;
    if (g >= GH) break;
    if (d0 < D) {
#pragma unroll
      for (int j = 0; j < DPL; ++j) part[(static_cast<size_t>(wg) * GH + g) * D + d0 + j] = acc[k][j];
    }
  }
  if (tid == 0) part_emit[wg] = emit_total;
}

// Waves per pass-2 workgroup: one per head up to four.
int pass2_waves(int GH) { return GH < 4 ? GH : 4; }

// Pass 2's dynamic LDS: per wave and list (one per head it holds at block_n
// 256, one otherwise) BN row indices and BN counts, then BN flags and one
// total.
static size_t pass2_lds_bytes(int nw, int BN, int lists) {
  return (static_cast<size_t>(2 * nw * lists + 1) * BN + 1) * sizeof(int);
}
static int pass2_heads_per_wave(int GH) { return GH <= 4 ? 1 : (GH <= 8 ? 2 : kMaxHeadsPerWave); }

static int pass2_dpl(int D) { return D <= 64 ? 1 : (D <= 128 ? 2 : (D <= 256 ? 4 : (D <= 512 ? 8 : 16))); }

// The fewest workgroups per CU over the instantiations of one DPL and head
// bound NK (bf16 / f16, contiguous / paged, block_n 256 or not): their
// registers differ (f16 takes more).
template <int DPL, int NK>
static int pass2_blocks_per_cu(int threads, size_t lds) {
  const void* fns[8] = {reinterpret_cast<const void*>(&pass2_kernel<true, false, DPL, true, NK>),
                        reinterpret_cast<const void*>(&pass2_kernel<true, true, DPL, true, NK>),
                        reinterpret_cast<const void*>(&pass2_kernel<false, false, DPL, true, NK>),
                        reinterpret_cast<const void*>(&pass2_kernel<false, true, DPL, true, NK>),
                        reinterpret_cast<const void*>(&pass2_kernel<true, false, DPL, false, NK>),
                        reinterpret_cast<const void*>(&pass2_kernel<true, true, DPL, false, NK>),
                        reinterpret_cast<const void*>(&pass2_kernel<false, false, DPL, false, NK>),
                        reinterpret_cast<const void*>(&pass2_kernel<false, true, DPL, false, NK>)};
  int best = 0;
  for (int i = 0; i < 8; ++i) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fns[i], threads, lds) != hipSuccess) {
      (void)hipGetLastError();
      return 0;
    }
    best = (i == 0 || n < best) ? n : best;
  }
  return best;
}

template <int NK>
static int pass2_blocks_per_cu_dpl(int dpl, int threads, size_t lds) {
  switch (dpl) {
    case 1: return pass2_blocks_per_cu<1, NK>(threads, lds);
    case 2: return pass2_blocks_per_cu<2, NK>(threads, lds);
    case 4: return pass2_blocks_per_cu<4, NK>(threads, lds);
    case 8: return pass2_blocks_per_cu<8, NK>(threads, lds);
    default: return pass2_blocks_per_cu<16, NK>(threads, lds);
  }
}

// Pass-2 workgroups resident on the current device at once for this shape,
// from the compiled kernel's registers and the most LDS a launch takes (one
// list at block_n 512, or a list per head at block_n 256); 0 where the runtime
// cannot say (no device).
// Cached per (device, D class, waves per workgroup and heads per wave).
int pass2_resident(int GH, int D) {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cached[kMaxDev][5][6];  // [dev][DPL class][waves - 1; 4 for GH 5-8, 5 above]
  const int nw = pass2_waves(GH);
  const int wi = GH > 8 ? 5 : (GH > 4 ? 4 : nw - 1);
  const int dpl = pass2_dpl(D);
  const int di = dpl == 1 ? 0 : (dpl == 2 ? 1 : (dpl == 4 ? 2 : (dpl == 8 ? 3 : 4)));
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  const bool slot = dev >= 0 && dev < kMaxDev;
  if (slot) {
    const int c = cached[dev][di][wi].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();
    return 0;
  }
  const int threads = 64 * nw;
  const size_t lds = std::max(pass2_lds_bytes(nw, kMaxBN, 1), pass2_lds_bytes(nw, 256, pass2_heads_per_wave(GH)));
  const int per_cu = GH <= 4 ? pass2_blocks_per_cu_dpl<1>(dpl, threads, lds)
                             : (GH <= 8 ? pass2_blocks_per_cu_dpl<2>(dpl, threads, lds)
                                        : pass2_blocks_per_cu_dpl<kMaxHeadsPerWave>(dpl, threads, lds));
  if (per_cu <= 0) return 0;
  const int r = per_cu * cus;
  if (slot) cached[dev][di][wi].store(r, std::memory_order_relaxed);
  return r;
}

// ---------------------------------------------------------------- finalize
template <bool BF16>
__global__ __launch_bounds__(kMaxD) void finalize_kernel(const float* __restrict__ part,
                                                         const int* __restrict__ part_emit, int H, int KVH, int D,
                                                         int cpg, float scale_out, uint16_t* __restrict__ out,
                                                         int* __restrict__ vrows, const int* __restrict__ seq_lens,
                                                         const int* __restrict__ seq_S, int BN, int cs, int max_rows,
                                                         int n_wg) {
  const int GH = H / KVH;
  const int bh = static_cast<int>(blockIdx.x);
  const int b = bh / H, h = bh % H;
  const int kv = h / GH, g = h % GH;
  const int d = static_cast<int>(threadIdx.x);
  // chunk c of (b, kv) was workgroup base_b + c * KVH + kv
  int base = b * cpg * KVH;
  int nch = cpg;
  if (seq_lens) {
    base = 0;
    for (int bb = 0; bb < b; ++bb) base += KVH * (((ragged_len(seq_lens, bb, max_rows) + BN - 1) / BN + cs - 1) / cs);
    nch = ((ragged_len(seq_lens, b, max_rows) + BN - 1) / BN + cs - 1) / cs;
    nch = max(0, min(nch, (n_wg - base - kv + KVH - 1) / KVH));
  }
  if (seq_S) scale_out = (seq_S[b] > 0) ? (1.0f / static_cast<float>(seq_S[b])) : 0.0f;
  // the chunks' partials summed in chunk order, up to 32 chunks' loads per
  // memory round trip
  const bool lead = vrows && g == 0 && d == 0;
  float s = 0.0f;
  int e = 0;
  sum_chunks(
      nch,
      [&](int c) {
        const size_t slot = static_cast<size_t>(base) + static_cast<size_t>(c) * KVH + kv;
        return (d < D) ? part[(slot * GH + g) * D + d] : 0.0f;
      },
      [&](int c) { return part_emit[static_cast<size_t>(base) + static_cast<size_t>(c) * KVH + kv]; }, lead, s, e);
  if (d < D) out[static_cast<size_t>(bh) * D + d] = f32_to_h16<BF16>(s * scale_out);
  if (vrows && g == 0 && d == 0) vrows[static_cast<size_t>(b) * KVH + kv] = e;
}

// ---------------------------------------------------------------- launchers
// (kv, tile) items from which GH 5-7 at D = 128 take santa_flash's GH 8 pass 1
// (one resident round of single-wave items; at 1,024 the two measured level)
constexpr long long kPad8Items = 2048;

hipError_t launch_pass1(const void* q, const void* K, int dtype, int B, int H, int KVH, int D, int L, int L_storage,
                        int BN, float* m_tiles, float* ell_tiles, uint16_t* u_stash, const int* seq_lens,
                        long long total_tiles, PageTable pt, hipStream_t stream, int stash_ld) {
  const int T_c = (L + BN - 1) / BN;
  long long grid = seq_lens ? total_tiles * KVH : static_cast<long long>(B) * KVH * T_c;
  if (grid <= 0) return hipSuccess;
  const float q_scale = 1.0f / sqrtf(static_cast<float>(D));
  const uint16_t* Qh = static_cast<const uint16_t*>(q);
  const uint16_t* Kh = static_cast<const uint16_t*>(K);
  const int GH = H / KVH;
  // GH 10, 12, 14, 16: two virtual KV heads per cache KV head, each with half
  // its query heads (5-8), on the same kernel; each cache row is read by the
  // two virtual heads' waves at about the same time
  const int kvd = (GH >= 10 && GH <= 16 && GH % 2 == 0) ? 2 : 1;
  const int ghv = GH / kvd;
  const long long items = (seq_lens ? total_tiles : static_cast<long long>(B) * T_c) * KVH * kvd;
  if (D == 128 && BN == 256 && ghv >= 5 && ghv <= (kvd == 2 ? 8 : 7) && stash_ld > 0 && items >= kPad8Items) {
    // two or more head blocks at D = 128 with the tile-major stash and at
    // least one resident round of items: santa_flash's GH 8 pass-1 wave
    // kernel, the last heads of each (virtual) group zero (the same general
    // numerics, so the same bits; 28q/4kv at 32k tokens: B = 8 step 140.6 ->
    // 99.3 us, B = 4 82.9 -> 64.2; 40q/8kv, B = 8: 245.1 -> 152.5 us; 64q/4kv
    // 353.6 -> 156.0 us; 128q/8kv 658.5 -> 305.2 us).  With fewer items the
    // generic kernel stays (28q/4kv, B = 1: 43.3 against 49.0 us)
    int cs = 0, n_wg = 0;
    if (seq_lens) flash::plan_ragged(B, KVH * kvd, total_tiles, T_c, &cs, &n_wg);
    return flash::launch_prop_pass1(q, K, dtype, B, H, KVH * kvd, L, L_storage, BN, 1, m_tiles, ell_tiles, u_stash,
                                    seq_lens, cs, n_wg, stash_ld, stream, pt, total_tiles, kvd);
  }
  if (fast_pass1_shape(GH, D, BN)) {
    // head blocks of four: GH 1-4 -> 1, 5-8 -> 2, 9-16 -> 4
    const int nhb = GH <= 4 ? 1 : (GH <= 8 ? 2 : 4);
    const bool bf = dtype == SANTA_BF16, pg = pt.table != nullptr;
    // chunks of tiles for about one resident round of workgroups (uniform),
    // or about eight over the sequences' tiles (ragged)
    const int occ = fast_occupancy(D, nhb);
    const int per_round = flash::rows_per_round() / 8 * occ;
    const bool stream_tiles = nhb == 1 || (D == 64 && nhb == 2);  // fast_prefetch<D, NHB>()
    int cs = 1, cpg = T_c, n_wg = 0;
    if (!stream_tiles) {
      // one tile per workgroup (grid as computed above)
    } else if (seq_lens) {
      flash::plan_ragged(B, KVH, total_tiles, T_c, &cs, &n_wg, per_round, 1);
      cpg = 0;
      grid = n_wg;
    } else {
      flash::plan_chunks(B, KVH, T_c, &cs, &cpg, per_round);
      grid = static_cast<long long>(B) * KVH * cpg;
    }
#define SANTA_GF1(BF, DD, NB, PG)                                                                                  \
  hipLaunchKernelGGL((pass1_fast_kernel<BF, DD, NB, PG>), dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0,    \
                     stream, Qh, Kh, H, KVH, L, L_storage, T_c, cs, cpg, q_scale, m_tiles, ell_tiles, u_stash,      \
                     seq_lens, B, pt, stash_ld)
#define SANTA_GF1_NB(BF, DD, PG) \
  do {                           \
    if (nhb == 1)                \
      SANTA_GF1(BF, DD, 1, PG);  \
    else if (nhb == 2)           \
      SANTA_GF1(BF, DD, 2, PG);  \
    else                         \
      SANTA_GF1(BF, DD, 4, PG);  \
  } while (0)
#define SANTA_GF1_D(BF, PG)        \
  do {                             \
    if (D == 64)                   \
      SANTA_GF1_NB(BF, 64, PG);    \
    else if (D == 128)             \
      SANTA_GF1_NB(BF, 128, PG);   \
    else                           \
      SANTA_GF1_NB(BF, 256, PG);   \
  } while (0)
    if (bf) {
      if (pg) SANTA_GF1_D(true, true); else SANTA_GF1_D(true, false);
    } else {
      if (pg) SANTA_GF1_D(false, true); else SANTA_GF1_D(false, false);
    }
#undef SANTA_GF1_D
#undef SANTA_GF1_NB
#undef SANTA_GF1
    return hipGetLastError();
  }
#define SANTA_GP1(BF, PG)                                                                                          \
  hipLaunchKernelGGL((pass1_kernel<BF, PG>), dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, stream, Qh, Kh, \
                     H, KVH, D, BN, L, L_storage, T_c, q_scale, m_tiles, ell_tiles, u_stash, seq_lens, B, pt)
  const bool bf = dtype == SANTA_BF16, pg = pt.table != nullptr;
  if (bf) {
    if (pg) SANTA_GP1(true, true); else SANTA_GP1(true, false);
  } else {
    if (pg) SANTA_GP1(false, true); else SANTA_GP1(false, false);
  }
#undef SANTA_GP1
  return hipGetLastError();
}

hipError_t launch_budgets_big(const float* m_tiles, const float* ell_tiles, int BH, int H, int T_c, int S,
                              uint64_t seed, float* m_star, int* S_tiles, float* invdelta, float* a0,
                              const int* seq_lens, const int* seq_S, int BN, hipStream_t stream) {
  if (BH <= 0) return hipSuccess;
  hipLaunchKernelGGL(budgets_big_kernel, dim3(static_cast<unsigned>(BH)), dim3(kBudgetThreads), 0, stream, m_tiles,
                     ell_tiles, H, T_c, S, seed, m_star, S_tiles, invdelta, a0, seq_lens, seq_S, BN);
  return hipGetLastError();
}

hipError_t launch_pass2(const void* V, const uint16_t* u_stash, int dtype, int B, int H, int KVH, int D, int L,
                        int L_storage, int BN, int T_c, int cs, int cpg, int n_wg, const float* invdelta,
                        const float* a0, int16_t* counts, float* part, int* part_emit, int want_emit,
                        const int* seq_lens, PageTable pt, hipStream_t stream, int stash_ld) {
  const long long grid = seq_lens ? n_wg : static_cast<long long>(B) * KVH * cpg;
  if (grid <= 0) return hipSuccess;
  const uint16_t* Vh = static_cast<const uint16_t*>(V);
  const int nw = pass2_waves(H / KVH);
  const unsigned threads = static_cast<unsigned>(64 * nw);
  const int dpl = pass2_dpl(D);
  const size_t lds = pass2_lds_bytes(nw, BN, BN == 256 ? pass2_heads_per_wave(H / KVH) : 1);
#define SANTA_GP2_K(BF, PG, DP, T2, NK)                                                                              \
  hipLaunchKernelGGL((pass2_kernel<BF, PG, DP, T2, NK>), dim3(static_cast<unsigned>(grid)), dim3(threads), lds,      \
                     stream, Vh, u_stash, H, KVH, D, BN, L, L_storage, T_c, cs, cpg, invdelta, a0, counts, part,     \
                     part_emit, want_emit, seq_lens, B, pt, stash_ld)
#define SANTA_GP2(BF, PG, DP)                                 \
  do {                                                        \
    if (H / KVH <= 4) {                                       \
      if (BN == 256)                                          \
        SANTA_GP2_K(BF, PG, DP, true, 1);                     \
      else                                                    \
        SANTA_GP2_K(BF, PG, DP, false, 1);                    \
    } else if (H / KVH <= 8) {                                \
      if (BN == 256)                                          \
        SANTA_GP2_K(BF, PG, DP, true, 2);                     \
      else                                                    \
        SANTA_GP2_K(BF, PG, DP, false, 2);                    \
    } else {                                                  \
      if (BN == 256)                                          \
        SANTA_GP2_K(BF, PG, DP, true, kMaxHeadsPerWave);      \
      else                                                    \
        SANTA_GP2_K(BF, PG, DP, false, kMaxHeadsPerWave);     \
    }                                                         \
  } while (0)
#define SANTA_GP2_D(BF, PG)      \
  do {                           \
    if (dpl == 1)                \
      SANTA_GP2(BF, PG, 1);      \
    else if (dpl == 2)           \
      SANTA_GP2(BF, PG, 2);      \
    else if (dpl == 4)           \
      SANTA_GP2(BF, PG, 4);      \
    else if (dpl == 8)           \
      SANTA_GP2(BF, PG, 8);      \
    else                         \
      SANTA_GP2(BF, PG, 16);     \
  } while (0)
  if (dtype == SANTA_BF16) {
    if (pt.table) SANTA_GP2_D(true, true); else SANTA_GP2_D(true, false);
  } else {
    if (pt.table) SANTA_GP2_D(false, true); else SANTA_GP2_D(false, false);
  }
#undef SANTA_GP2_D
#undef SANTA_GP2
#undef SANTA_GP2_K
  return hipGetLastError();
}

hipError_t launch_finalize(const float* part, const int* part_emit, int dtype, int B, int H, int KVH, int D, int cpg,
                           float scale_out, void* out, int* vrows, const int* seq_lens, const int* seq_S, int BN,
                           int cs, int max_rows, int n_wg, hipStream_t stream) {
  const unsigned grid = static_cast<unsigned>(B) * static_cast<unsigned>(H);
  if (grid == 0) return hipSuccess;
  const unsigned threads = static_cast<unsigned>((D + 63) / 64 * 64);
  uint16_t* o = static_cast<uint16_t*>(out);
  if (dtype == SANTA_BF16)
    hipLaunchKernelGGL(finalize_kernel<true>, dim3(grid), dim3(threads), 0, stream, part, part_emit, H, KVH, D, cpg,
                       scale_out, o, vrows, seq_lens, seq_S, BN, cs, max_rows, n_wg);
  else
    hipLaunchKernelGGL(finalize_kernel<false>, dim3(grid), dim3(threads), 0, stream, part, part_emit, H, KVH, D, cpg,
                       scale_out, o, vrows, seq_lens, seq_S, BN, cs, max_rows, n_wg);
  return hipGetLastError();
}

}  // namespace propgen
}  // namespace santa
