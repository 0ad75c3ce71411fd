// santa_prop.hip -- santa_prop (proportional tile budgets) decode kernels for
// gfx950, after prop/santa_cuda_kernel.cu and prop/santa_cuda.cpp:270-352.
//
// One decode step of one sequence (or of B sequences in the batched form)
// is four launches on one stream:
//  1. pass 1 (the flash tile kernel in a pass-1 mode, santa_flash.hip): per
//     (kv, tile) scores, tile max m_t and mass ell_t per head, and the 16-bit
//     u = exp(s - m_t) stashed as [L, H] -- all of K is read once here;
//  2. budgets_kernel: per head, m* = max m_t, W_t = exp(m_t - m*) ell_t and
//     the largest-remainder split of S over the tiles (the reference's
//     bitonic network), invdelta_t = S_t / ell_t and a0_t = u01(seed, h, t);
//  3. pass2_kernel: per (kv, chunk of tiles) workgroup, the systematic counts
//     of every head from the stash, the sampled rows' count-weighted V sums
//     accumulated over the chunk (rows ascending, tiles ascending);
//  4. finalize_kernel: out = dtype(sum over chunks * (1/S)), vrows.
//
// Determinism.  The reference sums Z and out with float atomics (order
// unspecified).  Here Z is 128 per-thread partials (tiles tid, tid+128, ...
// in order) reduced by a pairwise tree with strides 64 .. 1, and out is a
// fixed chunk order, so repeated calls give identical bits.  The sampled
// counts depend only on (m_t, ell_t, u stash), which are bit-exact to the
// restatement of the reference algorithm.
#include "santa_device.h"
#include "santa_amd.h"
#include "santa_internal.h"

#include <algorithm>
#include <cctype>
#include <cfloat>
#include <cstring>

namespace santa {
namespace prop {

constexpr int kD = 128;
constexpr int kThreads = 256;
constexpr int kMaxTiles = 4096;  // budgets: 16 waves x 4 registers x 64 lanes

// ---------------------------------------------------------------- budgets
// prop/santa_cuda_kernel.cu:577-726, one workgroup of NW waves per (b, h);
// the RNG key is h (the reference's per-sequence call).  Tile (and network
// position) p = NT r + tid lives in register r of thread tid (NT = 64 NW
// threads, R registers: every tile of the launch's longest sequence).
//  * m* = max_t m_t: exact in any order.
//  * Z keeps the association of 128 partial sums (partial i over tiles i,
//    i + 128, ... ascending, read back from LDS), then a pairwise tree
//    red[i] += red[i + s] for s = 64 .. 1 (s = 64 through LDS, the rest as
//    lane shifts of wave 0).
//  * The bitonic network (:686-707) runs as the reference's sequence of
//    compare-exchange steps over N = next power of two >= T_c; each element
//    takes its own side of every exchange (the pair's lower index decides
//    the swap), elements at positions >= T_c stay (-inf, -1), which is the
//    reference's "reads past T_c see (-inf, -1), writes are dropped".
//    Exchanges at distance < 64 are between lanes of a wave (DPP within
//    16-lane rows, LDS permutes across them), at distance < NT between
//    waves (through LDS, between two barriers), and at larger distances
//    between registers of one thread.

// Butterfly reductions over the wave through lane_xor (every lane gets the
// result): maximum of floats, sum of ints (both exact in any order).
__device__ __forceinline__ float wave_max_xor(float v, int lane) {
  v = fmaxf(v, __int_as_float(lane_xor<32>(__float_as_int(v), lane)));
  v = fmaxf(v, __int_as_float(lane_xor<16>(__float_as_int(v), lane)));
  v = fmaxf(v, __int_as_float(lane_xor<8>(__float_as_int(v), lane)));
  v = fmaxf(v, __int_as_float(lane_xor<4>(__float_as_int(v), lane)));
  v = fmaxf(v, __int_as_float(lane_xor<2>(__float_as_int(v), lane)));
  return fmaxf(v, __int_as_float(lane_xor<1>(__float_as_int(v), lane)));
}
__device__ __forceinline__ int wave_sum_xor(int v, int lane) {
  v += lane_xor<32>(v, lane);
  v += lane_xor<16>(v, lane);
  v += lane_xor<8>(v, lane);
  v += lane_xor<4>(v, lane);
  v += lane_xor<2>(v, lane);
  return v + lane_xor<1>(v, lane);
}

// One compare-exchange step given each element's partner value (of, oi):
// the pair's lower position decides, with up = (position & k) != 0.
template <int NT, int R>
__device__ __forceinline__ void bitonic_apply(float (&f)[R], int (&id)[R], const float (&of)[R], const int (&oi)[R],
                                              int j, int k, int T_c, int tid) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int p = NT * r + tid;
    const bool lo = (p & j) == 0;
    const bool up = (p & k) != 0;
    const float alo = lo ? f[r] : of[r];
    const float ahi = lo ? of[r] : f[r];
    const bool sw = (p < T_c) && ((alo > ahi) == up);
    f[r] = sw ? of[r] : f[r];
    id[r] = sw ? oi[r] : id[r];
  }
}

template <int NT, int R, int J>
__device__ __forceinline__ void bitonic_lanes(float (&f)[R], int (&id)[R], int k, int T_c, int tid) {
  // every exchange of the step is issued before the first is used
  float of[R];
  int oi[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    of[r] = __int_as_float(lane_xor<J>(__float_as_int(f[r]), tid & 63));
    oi[r] = lane_xor<J>(id[r], tid & 63);
  }
  bitonic_apply<NT, R>(f, id, of, oi, J, k, T_c, tid);
}

template <int NT, int R, int JR>
__device__ __forceinline__ void bitonic_regs(float (&f)[R], int (&id)[R], int k, int T_c, int tid) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r & JR) continue;
    const int rh = r | JR;
    const int plo = NT * r + tid;
    const int phi = NT * rh + tid;
    const bool up = (plo & k) != 0;
    const float alo = f[r], ahi = f[rh];
    const int ilo = id[r], ihi = id[rh];
    const bool sw = (alo > ahi) == up;
    const bool wlo = plo < T_c && sw;
    const bool whi = phi < T_c && sw;
    f[r] = wlo ? ahi : alo;
    id[r] = wlo ? ihi : ilo;
    f[rh] = whi ? alo : ahi;
    id[rh] = whi ? ilo : ihi;
  }
}

template <int NW, int R>
__device__ __forceinline__ void bitonic_desc(float (&f)[R], int (&id)[R], int T_c, int tid, float* s_f, int* s_i) {
  constexpr int NT = 64 * NW;
  int N = 1;
  while (N < T_c) N <<= 1;
  for (int k = 2; k <= N; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j < 64) {
        switch (j) {
          case 1: bitonic_lanes<NT, R, 1>(f, id, k, T_c, tid); break;
          case 2: bitonic_lanes<NT, R, 2>(f, id, k, T_c, tid); break;
          case 4: bitonic_lanes<NT, R, 4>(f, id, k, T_c, tid); break;
          case 8: bitonic_lanes<NT, R, 8>(f, id, k, T_c, tid); break;
          case 16: bitonic_lanes<NT, R, 16>(f, id, k, T_c, tid); break;
          default: bitonic_lanes<NT, R, 32>(f, id, k, T_c, tid); break;
        }
      } else if (j < NT) {
        if constexpr (NW > 1) {
          __syncthreads();  // the previous exchange's reads are done
#pragma unroll
          for (int r = 0; r < R; ++r) {
            s_f[NT * r + tid] = f[r];
            s_i[NT * r + tid] = id[r];
          }
          __syncthreads();
          float of[R];
          int oi[R];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            of[r] = s_f[(NT * r + tid) ^ j];
            oi[r] = s_i[(NT * r + tid) ^ j];
          }
          bitonic_apply<NT, R>(f, id, of, oi, j, k, T_c, tid);
        }
      } else {
        const int jr = j / NT;
        if constexpr (R > 1) if (jr == 1) bitonic_regs<NT, R, 1>(f, id, k, T_c, tid);
        if constexpr (R > 2) if (jr == 2) bitonic_regs<NT, R, 2>(f, id, k, T_c, tid);
        if constexpr (R > 4) if (jr == 4) bitonic_regs<NT, R, 4>(f, id, k, T_c, tid);
      }
    }
  }
}

template <int NW, int R>
__global__ __launch_bounds__(64 * NW) void budgets_kernel(const float* __restrict__ m_tiles,
                                                          const float* __restrict__ ell_tiles, int H, int T_c, int S,
                                                          uint64_t seed, float* __restrict__ m_star,
                                                          int* __restrict__ S_tiles, float* __restrict__ invdelta,
                                                          float* __restrict__ a0_tile, const int* __restrict__ seq_lens,
                                                          const int* __restrict__ seq_S, int BN) {
  constexpr int NT = 64 * NW;
  __shared__ float s_f[NT * R];  // W_t, then the network's exchanges
  __shared__ int s_i[NT * R];    // the network's exchanges, then the +1 flags
  __shared__ float s_z[128];
  __shared__ float s_red[NW];
  __shared__ int s_ired[NW];
  const int bh = static_cast<int>(blockIdx.x);
  const int h = bh % H;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const size_t off = static_cast<size_t>(bh) * T_c;  // T_c: tile stride of the [B, H, T_c] arrays
  // ragged batches: this sequence's tile count and budget
  if (seq_lens) T_c = (ragged_len(seq_lens, bh / H, T_c * BN) + BN - 1) / BN;
  if (seq_S) S = seq_S[bh / H];
  const float* mt = m_tiles + off;
  const float* lt = ell_tiles + off;

  float mv[R], lv[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int t = NT * r + tid;
    mv[r] = (t < T_c) ? mt[t] : 0.0f;
    lv[r] = (t < T_c) ? lt[t] : 0.0f;
  }
  // m* = max_t m_t (exact in any order); -FLT_MAX start as in :597
  float ms = -FLT_MAX;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (NT * r + tid < T_c) ms = fmaxf(ms, mv[r]);
  ms = wave_max_xor(ms, lane);
  if (lane == 0) s_red[wv] = ms;
  __syncthreads();
  ms = s_red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) ms = fmaxf(ms, s_red[i]);
  if (tid == 0 && m_star) m_star[bh] = ms;

  // W_t, then Z in the fixed order
  float w[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int t = NT * r + tid;
    w[r] = 0.0f;
    if (t < T_c) {
      w[r] = santa_expf(mv[r] - ms) * lv[r];
      s_f[t] = w[r];
    }
  }
  __syncthreads();
  for (int tau = tid; tau < 128; tau += NT) {
    float z = 0.0f;
    for (int t = tau; t < T_c; t += 128) z += s_f[t];
    s_z[tau] = z;
  }
  __syncthreads();
  if (wv == 0) {
    float z = s_z[lane] + s_z[lane + 64];
    // the tree z[i] += z[i + s] for s = 32 .. 1: for the lanes below s that
    // it reads, lane ^ s is lane + s, so lane 0 ends with the same sum
    z = z + __int_as_float(lane_xor<32>(__float_as_int(z), lane));
    z = z + __int_as_float(lane_xor<16>(__float_as_int(z), lane));
    z = z + __int_as_float(lane_xor<8>(__float_as_int(z), lane));
    z = z + __int_as_float(lane_xor<4>(__float_as_int(z), lane));
    z = z + __int_as_float(lane_xor<2>(__float_as_int(z), lane));
    z = z + __int_as_float(lane_xor<1>(__float_as_int(z), lane));
    if (lane == 0) s_z[0] = z;
  }
  __syncthreads();
  const float Z = s_z[0];

  if (S <= 0 || !(Z > 0.0f)) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int t = NT * r + tid;
      if (t < T_c) {
        S_tiles[off + t] = 0;
        invdelta[off + t] = 0.0f;
        a0_tile[off + t] = u01(seed, h, t);
      }
    }
    return;
  }

  // integer bases and jittered fractional parts (:662-678); u01(seed, h, t)
  // is both the jitter's draw and the tile's a0
  int bt[R], id[R];
  float f[R], ut[R];
  int base = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int t = NT * r + tid;
    bt[r] = 0;
    f[r] = -__builtin_inff();
    id[r] = -1;
    ut[r] = 0.0f;
    if (t < T_c) {
      ut[r] = u01(seed, h, t);
      const float q = static_cast<float>(S) * (w[r] / Z);
      const float fq = floorf(q);
      bt[r] = (fq != fq) ? 0 : (fq >= 2147483648.0f ? 2147483647 : static_cast<int>(fq));
      base += bt[r];
      const float ft = q - static_cast<float>(bt[r]);
      const float jitter = 1.0e-7f * ut[r];
      f[r] = ft + jitter;
      id[r] = t;
    }
  }
  base = wave_sum_xor(base, lane);
  if (lane == 0) s_ired[wv] = base;
  __syncthreads();
  base = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) base += s_ired[i];
  int rem = S - base;
  if (rem < 0) rem = 0;
  if (rem > T_c) rem = T_c;

  bitonic_desc<NW, R>(f, id, T_c, tid, s_f, s_i);

  // +1 to the top `rem` (distinct tiles, :710-716)
  __syncthreads();  // the network's last reads of s_i are done
#pragma unroll
  for (int r = 0; r < R; ++r) s_i[NT * r + tid] = 0;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (NT * r + tid < rem && id[r] >= 0) s_i[id[r]] = 1;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int t = NT * r + tid;
    if (t < T_c) {
      const int s_t = bt[r] + s_i[t];
      S_tiles[off + t] = s_t;
      invdelta[off + t] = (s_t > 0 && lv[r] > 1e-20f) ? (static_cast<float>(s_t) / lv[r]) : 0.0f;
      a0_tile[off + t] = ut[r];
    }
  }
}

// Number of rows of a tile sampled by any head of the group (union of the
// per-head nonzero masks, one 64-bit mask per lane < NM).
template <int GH, int NM>
__device__ __forceinline__ int union_rows(const uint64_t* s_mask, int lane) {
  int e = 0;
  if (lane < NM) {
    uint64_t u = 0;
#pragma unroll
    for (int g = 0; g < GH; ++g) u |= s_mask[g * NM + lane];
    e = __popcll(u);
  }
#pragma unroll
  for (int m = 1; m < NM; m <<= 1) e += __shfl_xor(e, m, 64);
  return e;
}

// ---------------------------------------------------------------- pass 2
// prop/santa_cuda_kernel.cu:734-864.  Workgroup = (b, kv, chunk of cs
// tiles); wave w owns heads w and w+4.  Per tile and head: x_r = f32(u16
// stash) * invdelta_t, counts by systematic_counts (the reference's 32-lane
// scan with carry), the sampled rows in ascending order in a wave-private
// LDS list, then the count-weighted V rows (fma per element) added to the
// head's running sum.  The next tile's stash entries are loaded before the
// current tile's V gather.
// HM: the stash is tile-major [B, T, H, 256], T = stash_ld / 256 (the fused decode's layout
// for the vec path: a lane reads its row pair with one 4-B load); otherwise
// the reference's [B, L_storage, H].
// PAGED: V is a page pool read through pt (the stash is indexed by token).
// The kernel is bound by the latency of its per-tile chains (stash load,
// scan, carries, list appends) and of the V gathers, so it is compiled for
// as many resident waves as fit without spilling: six per SIMD (80 VGPRs)
// for one head per wave at block_n 256, four (128) otherwise; the V gathers
// go out 16 rows at a time (cfg3 step 542 -> 518 us).
template <bool BF16, int GH, int BN, bool HM, bool PAGED = false>
__global__ __launch_bounds__(kThreads, (GH == 4 && BN == 256 && !PAGED) ? 6 : 4) void pass2_kernel(const uint16_t* __restrict__ V,
                                                         const uint16_t* __restrict__ u_stash, int H, int KVH,
                                                         int L, int L_storage, int T_c, int cs, int cpg,
                                                         const float* __restrict__ invdelta,
                                                         const float* __restrict__ a0_tile,
                                                         int16_t* __restrict__ dbg_counts, float* __restrict__ part,
                                                         int* __restrict__ part_emit, int want_emit,
                                                         const int* __restrict__ seq_lens, int B, int stash_ld,
                                                         PageTable pt) {
  constexpr int NCH = BN / 32;
  constexpr int NPAIR = (NCH + 3) / 4;
  constexpr int HPW = GH / 4;
  constexpr int NM = 2 * NPAIR;  // 64-bit row masks per head and tile

  const int wg = static_cast<int>(blockIdx.x);
  // The KV heads of one chunk of tokens are neighbours in launch order;
  // T_c is the tile stride of the [B, H, T_c] budget arrays.
  const GridPos gp = grid_pos(wg, seq_lens, B, KVH, BN, L, T_c, cs, cpg);
  const int kv = gp.kv;
  const int chunk = gp.chunk;
  const int b = gp.b < 0 ? 0 : gp.b;
  const int h0 = kv * GH;
  L = gp.len;  // this sequence's length from here on
  const int t_begin = chunk * cs;
  const int t_end = (gp.b < 0) ? t_begin : min(gp.n_tiles, t_begin + cs);
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform for the compiler
  const int jrow = lane >> 4;
  const int qq = lane & 15;

  __shared__ uint64_t s_mask[2][GH * NM];
  __shared__ float s_lcw[GH * BN];
  __shared__ int s_lrow[GH * BN];

  const size_t row_stride = static_cast<size_t>(KVH) * kD;
  const uint32_t row_bytes = static_cast<uint32_t>(KVH) * kD * 2u;
  // wave-uniform 64-bit base + 32-bit lane offset (scalar-base loads)
  const size_t seq_off = PAGED ? 0 : static_cast<size_t>(b) * L_storage * row_stride;
  const char* Vg = reinterpret_cast<const char*>(V + seq_off + static_cast<size_t>(kv) * kD);
  const uint32_t v_lane_off = 4u * static_cast<uint32_t>(lane);
  const uint16_t* ub = u_stash + static_cast<size_t>(b) * (HM ? static_cast<size_t>(H) * stash_ld
                                                              : static_cast<size_t>(L_storage) * H);

  float acc0[HPW], acc1[HPW];
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    acc0[k] = 0.0f;
    acc1[k] = 0.0f;
  }
  int emit_total = 0;

  // Count-weighted V rows of the listed samples, in list (ascending) order,
  // one fma per element (prop/santa_cuda_kernel.cu:843-857); up to FB row
  // loads are in flight before the first is used.
  int lc[HPW];
#pragma unroll
  for (int k = 0; k < HPW; ++k) lc[k] = 0;
  constexpr int FB = 16;
  auto flush = [&](int k, int g) {
    for (int base = 0; base < lc[k]; base += FB) {
      float cf[FB];
      uint32_t vw[FB];
      // paged: lane q looks up the page of the batch's q-th row
      int pgv = 0;
      if constexpr (PAGED) {
        const int iq = min(base + (lane & (FB - 1)), lc[k] - 1);
        pgv = page_of_row(pt, b, s_lrow[g * BN + iq], true);
      }
#pragma unroll
      for (int q = 0; q < FB; ++q) {
        const int i = min(base + q, lc[k] - 1);
        const int rr = __builtin_amdgcn_readfirstlane(s_lrow[g * BN + i]);
        cf[q] = s_lcw[g * BN + i];
        const size_t off = PAGED ? paged_row(pt, __builtin_amdgcn_readlane(pgv, q), rr, row_bytes)
                                 : static_cast<size_t>(rr) * row_bytes;
        vw[q] = *reinterpret_cast<const uint32_t*>(Vg + off + v_lane_off);
      }
#pragma unroll
      for (int q = 0; q < FB; ++q) {
        if (base + q < lc[k]) {
          acc0[k] = fmaf(cf[q], lo16_to_f32<BF16>(vw[q]), acc0[k]);
          acc1[k] = fmaf(cf[q], hi16_to_f32<BF16>(vw[q]), acc1[k]);
        }
      }
    }
    lc[k] = 0;
  };

  // stash entries of tile t for this lane's rows: u[k][p][0/1]; heads whose
  // bit in `heads` is clear (a zero budget on that tile) are not loaded
  using UBuf = uint16_t[HPW][NPAIR];
  auto load_u = [&](int t, UBuf& un0, UBuf& un1, unsigned heads) {
    const int n0 = t * BN;
    const int len = min(BN, L - n0);
#pragma unroll
    for (int k = 0; k < HPW; ++k) {
      const int h = h0 + wave + 4 * k;
      if (!((heads >> k) & 1u)) continue;
#pragma unroll
      for (int p = 0; p < NPAIR; ++p) {
        const int row = 32 * (4 * p + jrow) + 2 * qq;
        if constexpr (HM) {
          // whole padded tiles are in the stash (0 past len)
          const uint32_t w = *reinterpret_cast<const uint32_t*>(ub + (static_cast<size_t>(t) * H + h) * BN + row);
          un0[k][p] = static_cast<uint16_t>(w & 0xffffu);
          un1[k][p] = static_cast<uint16_t>(w >> 16);
        } else {
          un0[k][p] = (row < len) ? ub[static_cast<size_t>(n0 + row) * H + h] : static_cast<uint16_t>(0);
          un1[k][p] = (row + 1 < len) ? ub[static_cast<size_t>(n0 + row + 1) * H + h] : static_cast<uint16_t>(0);
        }
      }
    }
  };
  // The chunk's per-tile terms invdelta_t and a0_t, one tile per lane (64
  // tiles at a time), so that no tile waits on a load of its own.
  float inv_l[HPW], a0_l[HPW];
  auto load_terms = [&](int t0) {
    const int tt = min(t0 + lane, t_end - 1);
#pragma unroll
    for (int k = 0; k < HPW; ++k) {
      const size_t ht = (static_cast<size_t>(b) * H + h0 + wave + 4 * k) * T_c + tt;
      inv_l[k] = invdelta[ht];
      a0_l[k] = a0_tile[ht];
    }
  };
  // heads of this wave with a nonzero budget on tile t of the current window
  // (which starts at t0)
  auto active_heads = [&](int t, int t0) -> unsigned {
    unsigned m = 0;
#pragma unroll
    for (int k = 0; k < HPW; ++k)
      if (__int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv_l[k]), t - t0)) > 0.0f) m |= 1u << k;
    return m;
  };
  // Tiles where every head of the group has a zero budget list nothing and
  // add nothing (every count is floor(a0) - floor(a0) = 0), so each window of
  // 64 tiles is walked over the tiles where some head of the group has a
  // budget, in ascending order; every wave walks the same tiles, so the
  // emit barriers match.  The debug path (counts written out) walks them all.
  auto window_mask = [&](int t0) -> uint64_t {
    const int tt = t0 + lane;
    bool act = tt < t_end;
    if (act && !dbg_counts) {
      bool any = false;
#pragma unroll
      for (int g = 0; g < GH; ++g) any = any || invdelta[(static_cast<size_t>(b) * H + h0 + g) * T_c + tt] > 0.0f;
      act = any;
    }
    return __ballot(act);
  };
  auto pop_tile = [](uint64_t& m, int t0) -> int {
    if (m == 0) return -1;
    const int i = __builtin_ctzll(m);
    m &= m - 1;
    return t0 + i;
  };

  int processed = 0;  // tiles walked so far (parity of the emit masks)
  auto tile_step = [&](int t, int t0, UBuf& un0, UBuf& un1) {
    const int n0 = t * BN;
    const int len = min(BN, L - n0);
    const int par = processed & 1;
    const int li = t - t0;
    float x0[HPW][NPAIR], x1[HPW][NPAIR], inv[HPW], a0v[HPW];
#pragma unroll
    for (int k = 0; k < HPW; ++k) {
      inv[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv_l[k]), li));
      a0v[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a0_l[k]), li));
#pragma unroll
      for (int p = 0; p < NPAIR; ++p) {
        x0[k][p] = (inv[k] > 0.0f) ? h16_to_f32<BF16>(un0[k][p]) * inv[k] : 0.0f;
        x1[k][p] = (inv[k] > 0.0f) ? h16_to_f32<BF16>(un1[k][p]) * inv[k] : 0.0f;
      }
    }
#pragma unroll
    for (int k = 0; k < HPW; ++k) {
      const int g = wave + 4 * k;
      const int h = h0 + g;
      if (!(inv[k] > 0.0f)) {
        // a zero budget on this tile: x = 0 on every row, so every count is 0
        // (floor(a0) - floor(a0)) and nothing is listed
        if (lane == 0)
#pragma unroll
          for (int m = 0; m < NM; ++m) s_mask[par][g * NM + m] = 0;
        if (dbg_counts)
          for (int r = lane; r < BN; r += 64)
            dbg_counts[((static_cast<size_t>(b) * H + h) * T_c + t) * BN + r] = 0;
        continue;
      }
      int c0[NPAIR], c1[NPAIR];
      systematic_counts<NCH>(x0[k], x1[k], len, a0v[k], lane, c0, c1);
      const uint64_t below = (1ull << lane) - 1ull;
      uint64_t nz0[NPAIR], nz1[NPAIR];
      int cnt = 0;
#pragma unroll
      for (int p = 0; p < NPAIR; ++p) {
        nz0[p] = __ballot(c0[p] != 0);
        nz1[p] = __ballot(c1[p] != 0);
        cnt += __popcll(nz0[p]) + __popcll(nz1[p]);
      }
      // the list keeps the head's sampled rows across tiles; it is gathered
      // when this tile's rows would not fit (and at the end of the chunk)
      if (lc[k] + cnt > BN) flush(k, g);
      int pos = lc[k];
#pragma unroll
      for (int p = 0; p < NPAIR; ++p) {
        const int row = 32 * (4 * p + jrow) + 2 * qq;
        if (lane == 0) {
          s_mask[par][g * NM + 2 * p + 0] = nz0[p];
          s_mask[par][g * NM + 2 * p + 1] = nz1[p];
        }
        if (dbg_counts && row < BN) {
          int16_t* dc = dbg_counts + ((static_cast<size_t>(b) * H + h) * T_c + t) * BN + row;
          dc[0] = static_cast<int16_t>(c0[p]);
          dc[1] = static_cast<int16_t>(c1[p]);
        }
        const int pos0 = pos + __popcll(nz0[p] & below) + __popcll(nz1[p] & below);
        const int pos1 = pos0 + (c0[p] != 0 ? 1 : 0);
        if (c0[p] != 0) {
          s_lrow[g * BN + pos0] = n0 + row;
          s_lcw[g * BN + pos0] = static_cast<float>(c0[p]);
        }
        if (c1[p] != 0) {
          s_lrow[g * BN + pos1] = n0 + row + 1;
          s_lcw[g * BN + pos1] = static_cast<float>(c1[p]);
        }
        pos += __popcll(nz0[p]) + __popcll(nz1[p]);
      }
      lc[k] = pos;
    }
    if (want_emit) {
      // masks double-buffered by tile parity: one barrier per tile
      __syncthreads();
      if (wave == 0) emit_total += union_rows<GH, NM>(s_mask[par], lane);
    }
    ++processed;
  };
  // stash entries two walked tiles ahead: the walked tiles alternate between
  // two register buffers, each refilled as soon as its tile has been read
  UBuf ua0, ua1, ub0, ub1;
  for (int t0 = t_begin; t0 < t_end; t0 += 64) {
    load_terms(t0);
    uint64_t m = window_mask(t0);
    int tA = pop_tile(m, t0), tB = pop_tile(m, t0);
    if (tA >= 0) load_u(tA, ua0, ua1, active_heads(tA, t0));
    if (tB >= 0) load_u(tB, ub0, ub1, active_heads(tB, t0));
    while (tA >= 0) {
      const int tC = pop_tile(m, t0);
      tile_step(tA, t0, ua0, ua1);
      if (tC >= 0) load_u(tC, ua0, ua1, active_heads(tC, t0));
      if (tB < 0) break;
      const int tD = pop_tile(m, t0);
      tile_step(tB, t0, ub0, ub1);
      if (tD >= 0) load_u(tD, ub0, ub1, active_heads(tD, t0));
      tA = tC;
      tB = tD;
    }
  }

#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    flush(k, wave + 4 * k);
    float* pp = part + (static_cast<size_t>(wg) * GH + wave + 4 * k) * kD;
    reinterpret_cast<float2*>(pp)[lane] = make_float2(acc0[k], acc1[k]);
  }
  if (tid == 0) part_emit[wg] = emit_total;
}

// ---------------------------------------------------------------- finalize
// out[b, h, :] = dtype((sum over the chunks of (b, kv), ascending) * scale_out)
// (prop/santa_cuda_kernel.cu:976-985 with the chunk sums in place of the
// atomics); vrows[b, kv] = rows emitted by any head of the group.
template <bool BF16, int GH>
__global__ __launch_bounds__(kD) void finalize_kernel(const float* __restrict__ part,
                                                      const int* __restrict__ part_emit, int H, int KVH, int cpg,
                                                      float scale_out, uint16_t* __restrict__ out,
                                                      int* __restrict__ vrows, const int* __restrict__ seq_lens,
                                                      const int* __restrict__ seq_S, int BN, int cs,
                                                      int max_rows, int n_wg) {
  const int bh = static_cast<int>(blockIdx.x);
  const int b = bh / H;
  const int h = bh % H;
  const int kv = h / GH;
  const int g = h % GH;
  const int bk = b * KVH + kv;
  const int d = static_cast<int>(threadIdx.x);
  // chunk c of (b, kv) was workgroup base_b + c * KVH + kv
  int base = b * cpg * KVH;
  int nch = cpg;
  if (seq_lens) {
    base = 0;
    for (int bb = 0; bb < b; ++bb) base += KVH * (((ragged_len(seq_lens, bb, max_rows) + BN - 1) / BN + cs - 1) / cs);
    nch = ((ragged_len(seq_lens, b, max_rows) + BN - 1) / BN + cs - 1) / cs;
    // only the n_wg launched workgroups wrote partials
    nch = max(0, min(nch, (n_wg - base - kv + KVH - 1) / KVH));
  }
  if (seq_S) scale_out = (seq_S[b] > 0) ? (1.0f / static_cast<float>(seq_S[b])) : 0.0f;
  const float* pb = part + ((static_cast<size_t>(base) + kv) * GH + g) * kD + d;
  const size_t cstride = static_cast<size_t>(KVH) * GH * kD;
  // chunks in ascending order, up to 32 chunks' loads per memory round trip
  const bool emit = vrows && g == 0 && d == 0;
  float s = 0.0f;
  int e = 0;
  sum_chunks(
      nch, [&](int c) { return pb[static_cast<size_t>(c) * cstride]; },
      [&](int c) { return part_emit[static_cast<size_t>(base) + c * KVH + kv]; }, emit, s, e);
  out[static_cast<size_t>(bh) * kD + d] = f32_to_h16<BF16>(s * scale_out);
  if (emit) vrows[bk] = e;
}

// Grid: B * KVH * cpg workgroups (uniform) or n_wg (ragged, seq_lens set).
struct Pass2Grid {
  const int* seq_lens;
  int n_wg;
  int stash_ld;  // > 0: tile-major stash [B, stash_ld / 256, H, 256] (block_n 256 only)
  PageTable pt;  // paged V (pt.table set) or contiguous
};

template <bool BF16, int GH, int BN>
static hipError_t launch_pass2_t(const uint16_t* V, const uint16_t* u_stash, int B, int H, int KVH, int L,
                                 int L_storage, int T_c, int cs, int cpg, const float* invdelta, const float* a0,
                                 int16_t* counts, float* part, int* part_emit, int want_emit, Pass2Grid rg,
                                 hipStream_t stream) {
  const unsigned grid = rg.seq_lens ? static_cast<unsigned>(rg.n_wg)
                                    : static_cast<unsigned>(B) * static_cast<unsigned>(KVH) * static_cast<unsigned>(cpg);
  if (grid == 0) return hipSuccess;
#define SANTA_P2_LAUNCH(HM, PG, SLD)                                                                               \
  hipLaunchKernelGGL((pass2_kernel<BF16, GH, BN, HM, PG>), dim3(grid), dim3(kThreads), 0, stream, V, u_stash, H, KVH, \
                     L, L_storage, T_c, cs, cpg, invdelta, a0, counts, part, part_emit, want_emit, rg.seq_lens, B,    \
                     SLD, rg.pt)
  const bool hm = BN == 256 && rg.stash_ld > 0;
  if (rg.pt.table) {
    if (hm) SANTA_P2_LAUNCH(true, true, rg.stash_ld); else SANTA_P2_LAUNCH(false, true, 0);
  } else {
    if (hm) SANTA_P2_LAUNCH(true, false, rg.stash_ld); else SANTA_P2_LAUNCH(false, false, 0);
  }
#undef SANTA_P2_LAUNCH
  return hipGetLastError();
}

template <bool BF16, int GH>
static hipError_t launch_pass2_bn(int bn, const uint16_t* V, const uint16_t* u_stash, int B, int H, int KVH, int L,
                                  int L_storage, int T_c, int cs, int cpg, const float* invdelta, const float* a0,
                                  int16_t* counts, float* part, int* part_emit, int want_emit, Pass2Grid rg,
                                  hipStream_t stream) {
  switch (bn) {
    case 32:
      return launch_pass2_t<BF16, GH, 32>(V, u_stash, B, H, KVH, L, L_storage, T_c, cs, cpg, invdelta, a0, counts,
                                          part, part_emit, want_emit, rg, stream);
    case 64:
      return launch_pass2_t<BF16, GH, 64>(V, u_stash, B, H, KVH, L, L_storage, T_c, cs, cpg, invdelta, a0, counts,
                                          part, part_emit, want_emit, rg, stream);
    default:
      return launch_pass2_t<BF16, GH, 256>(V, u_stash, B, H, KVH, L, L_storage, T_c, cs, cpg, invdelta, a0, counts,
                                           part, part_emit, want_emit, rg, stream);
  }
}

// Rows per (sequence, head) of the tile-major stash: whole 256-row tiles.
static int stash_ld(int L_storage) { return (L_storage + 255) / 256 * 256; }

// Workspace of one decode call (offsets 256-B aligned).
// T_c is the tile stride of the [B, H, T_c] arrays (the longest sequence's
// tile count); total_tiles >= 0 selects the ragged grid over that many tiles.
struct PropWs {
  size_t m, ell, st, inv, a0, stash, part, emit, total;
  int cs, cpg, n_wg;
};
static PropWs prop_ws_layout(int B, int H, int KVH, int D, int L_storage, int T_c, long long total_tiles = -1) {
  PropWs w{};
  size_t chunks;
  // Shapes that only the generic pass 2 takes: chunks for one round of as many
  // of its workgroups as the device holds at once (the runtime's occupancy
  // for the compiled kernels), since each wave walks its tiles one dependent
  // round trip after another; with no device to ask, for as many GH-wave workgroups as
  // four-wave ones leave room for.  D = 128 at GH 4 or 8 (the tuned kernels):
  // uniform lengths over at least 32 (sequence, KV head) groups plan one round
  // of four 4-wave workgroups per CU, the four waves per SIMD every tuned pass
  // 2 holds (six at GH 4, block_n 256), where two per CU left two thirds of
  // them idle (B = 32, 32k tokens, GH 4: step 510.2 -> 476.7 us; cfg5p 1897
  // -> 1871 us; same bits).  Fewer groups keep two per CU: their chunks are
  // already short, and more of them only lengthen the finalize (B = 1, 32k:
  // 43.7 against 47.2 us).  Ragged lengths keep about eight rounds of two per
  // CU (four per CU measured 531.9 against 515.8 us on cfg3).
  const int GH = H / KVH;
  const int nw = propgen::pass2_waves(GH);
  const bool tuned = D == 128 && (GH == 4 || GH == 8);
  const bool uniform = total_tiles < 0 || total_tiles == static_cast<long long>(B) * T_c;
  int per_round = (!tuned && nw < 4) ? flash::rows_per_round() / nw : 0;
  if (tuned && uniform && static_cast<long long>(B) * KVH >= 32) per_round = flash::rows_per_round() / 4 * 2;
  if (!tuned) {
    const int r = propgen::pass2_resident(GH, D);
    if (r > 0) per_round = r;
  }
  if (total_tiles >= 0) {
    flash::plan_ragged(B, KVH, total_tiles, T_c, &w.cs, &w.n_wg, per_round);
    w.cpg = 0;
    chunks = static_cast<size_t>(w.n_wg);
  } else {
    flash::plan_chunks(B, KVH, T_c, &w.cs, &w.cpg, per_round);
    chunks = static_cast<size_t>(B) * KVH * w.cpg;
  }
  const size_t bht = static_cast<size_t>(B) * H * T_c;
  size_t off = 0;
  w.m = off;
  off = align_up(off + bht * sizeof(float));
  w.ell = off;
  off = align_up(off + bht * sizeof(float));
  w.st = off;
  off = align_up(off + bht * sizeof(int));
  w.inv = off;
  off = align_up(off + bht * sizeof(float));
  w.a0 = off;
  off = align_up(off + bht * sizeof(float));
  w.stash = off;  // [B, L_storage, H] or tile-major [B, stash_ld(L_storage) / 256, H, 256]
  off = align_up(off + static_cast<size_t>(B) * stash_ld(L_storage) * H * sizeof(uint16_t));
  w.part = off;  // [chunks, GH, D]
  off = align_up(off + chunks * (H / KVH) * static_cast<size_t>(D) * sizeof(float));
  w.emit = off;
  off = align_up(off + chunks * sizeof(int));
  w.total = off;
  return w;
}

// SANTA_PASS1 as the reference reads it (prop/santa_cuda.cpp:39-51):
// 0 auto, 1 force the general path, 2 force the vec path.
static int pass1_mode(const char* env) {
  if (!env) return 0;
  char s[32];
  size_t n = 0;
  for (; env[n] && n + 1 < sizeof(s); ++n) s[n] = static_cast<char>(std::tolower(static_cast<unsigned char>(env[n])));
  s[n] = 0;
  if (env[n] != 0) return 0;
  if (!std::strcmp(s, "gqa") || !std::strcmp(s, "perhead")) return 1;
  if (!std::strcmp(s, "vec") || !std::strcmp(s, "gqa_vec")) return 2;
  return 0;
}

// D = 128 with GH 4 or 8 runs the tuned kernels at block_n 32 / 64 / 256;
// every other shape with D a multiple of 16 up to 1024, GH up to 16 and
// block_n a multiple of 16 up to 512 runs the generic ones
// (santa_prop_gen.hip).
static int check_common(int dtype, int H, int KVH, int D) {
  if (dtype != SANTA_BF16 && dtype != SANTA_F16) return set_error(SANTA_ERR_INVALID, "q_h must be bf16 or f16");
  if (H <= 0 || KVH <= 0) return set_error(SANTA_ERR_INVALID, "empty head dimension");
  if (H % KVH != 0)
    return set_error(SANTA_ERR_INVALID, "H must be divisible by KVH (expected KVH == K_g.size(1) for NHD)");
  if (D < 16 || D > 1024 || D % 16 != 0)
    return set_error(SANTA_ERR_UNSUPPORTED, "This build supports D a multiple of 16 up to 1024 for santa_prop. Got D=%d",
                     D);
  const int GH = H / KVH;
  if (GH > 16)
    return set_error(SANTA_ERR_UNSUPPORTED, "This build supports GH (H/KVH) up to 16 for santa_prop. Got GH=%d (H=%d KVH=%d)",
                     GH, H, KVH);
  return SANTA_OK;
}

static int check_bn(int block_n, int GH, int D) {
  if (!propgen::shape_supported(GH, D, block_n))
    return set_error(SANTA_ERR_UNSUPPORTED,
                     "This build supports block_n a multiple of 16 up to 512 for santa_prop. Got block_n=%d", block_n);
  return SANTA_OK;
}

}  // namespace prop
}  // namespace santa

using namespace santa;

extern "C" int santa_prop_plan(int L, int H, int KVH, int D, int64_t block_n, const char* pass1_env,
                               int* block_n_out, int* T_c_out, int* pass1_path_out) {
  const int mode = prop::pass1_mode(pass1_env);
  int64_t bn = block_n;
  if (bn <= 0) bn = (mode == 2) ? 256 : ((L <= 1536) ? 32 : ((L <= 3072) ? 64 : 256));
  if (L <= 0) return set_error(SANTA_ERR_INVALID, "empty KV cache: L=%d", L);
  if (KVH <= 0 || H % KVH != 0) return set_error(SANTA_ERR_INVALID, "H must be divisible by KVH");
  const int GH = H / KVH;
  const bool can_vec = GH == 4 && D == 128 && bn == 256;
  if (mode == 2 && !can_vec)
    return set_error(SANTA_ERR_INVALID, "SANTA_PASS1=vec requires GH=4, D=128, block_n=256. Got GH=%d D=%d block_n=%lld",
                     GH, D, static_cast<long long>(bn));
  const bool use_vec = (mode == 0 && can_vec) || mode == 2;
  if (!use_vec && (((D & 15) != 0) || ((bn & 15) != 0)))
    return set_error(SANTA_ERR_INVALID, "Pass-1 WMMA-GQA requires D %% 16 == 0 and block_n %% 16 == 0. Got D=%d block_n=%lld",
                     D, static_cast<long long>(bn));
  const int64_t T_c = (L + bn - 1) / bn;
  if (block_n_out) *block_n_out = static_cast<int>(bn);
  if (T_c_out) *T_c_out = static_cast<int>(T_c);
  if (pass1_path_out) *pass1_path_out = use_vec ? 0 : 1;
  return clear_error();
}

extern "C" int santa_prop_pass1(const void* q, const void* K, int dtype, int H, int KVH, int D, int L, int block_n,
                                int pass1_path, float* m_tiles, float* ell_tiles, void* u_stash, hipStream_t stream) {
  int st = prop::check_common(dtype, H, KVH, D);
  if (st != SANTA_OK) return st;
  if (L <= 0) return set_error(SANTA_ERR_INVALID, "empty KV cache: L=%d", L);
  if ((st = prop::check_bn(block_n, H / KVH, D)) != SANTA_OK) return st;
  if (pass1_path == 0 && !(H / KVH == 4 && D == 128 && block_n == 256))
    return set_error(SANTA_ERR_INVALID, "SANTA_PASS1=vec requires GH=4, D=128, block_n=256. Got GH=%d D=%d block_n=%d",
                     H / KVH, D, block_n);
  if (!q || !K || !m_tiles || !ell_tiles || !u_stash) return set_error(SANTA_ERR_INVALID, "null pointer argument");
  const hipError_t e =
      propgen::generic_shape(H / KVH, D, block_n)
          ? propgen::launch_pass1(q, K, dtype, 1, H, KVH, D, L, L, block_n, m_tiles, ell_tiles,
                                  static_cast<uint16_t*>(u_stash), nullptr, -1, PageTable{nullptr, 0, 3, 1}, stream)
          : flash::launch_prop_pass1(q, K, dtype, 1, H, KVH, L, L, block_n, pass1_path, m_tiles, ell_tiles,
                                     static_cast<uint16_t*>(u_stash), nullptr, 0, 0, 0, stream);
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "pass-1 launch failed: %s", hipGetErrorString(e));
  return clear_error();
}

static int prop_budgets_launch(const float* m_tiles, const float* ell_tiles, int BH, int H, int T_c, int S,
                               uint64_t seed, float* m_star, int* S_tiles, float* invdelta, float* a0,
                               hipStream_t stream, const int* seq_lens = nullptr, const int* seq_S = nullptr,
                               int block_n = 0) {
  if (T_c > prop::kMaxTiles) {
    // more tiles than the register network holds: the network in memory
    const hipError_t e = propgen::launch_budgets_big(m_tiles, ell_tiles, BH, H, T_c, S, seed, m_star, S_tiles,
                                                     invdelta, a0, seq_lens, seq_S, block_n, stream);
    if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "budget launch failed: %s", hipGetErrorString(e));
    return SANTA_OK;
  }
  // waves per (b, h) and registers per thread for every tile of the longest
  // sequence (T_c <= kMaxTiles): two registers a thread, up to 16 waves
  // (up to 256 tiles one per thread: B = 1 at 32k tokens 42.4 -> 40.7 us per
  // step, at 64k 51.6 -> 49.9 us; MHA at B = 8 419.4 -> 417.8 us; at 512
  // tiles two per thread stay ahead on cfg5p)
  int N = 1;
  while (N < T_c) N <<= 1;
  const int NW = N <= 256 ? std::max(1, N / 64) : std::min(16, N / 128);
  const int R = std::max(1, N / (64 * NW));
#define SANTA_BUDGETS(W, RR)                                                                                      \
  hipLaunchKernelGGL((prop::budgets_kernel<W, RR>), dim3(BH), dim3(64 * W), 0, stream, m_tiles, ell_tiles, H, T_c, \
                     S, seed, m_star, S_tiles, invdelta, a0, seq_lens, seq_S, block_n)
  if (NW == 1 && R == 1) SANTA_BUDGETS(1, 1);
  else if (NW == 2 && R == 1) SANTA_BUDGETS(2, 1);
  else if (NW == 4 && R == 1) SANTA_BUDGETS(4, 1);
  else if (NW == 1 && R == 2) SANTA_BUDGETS(1, 2);
  else if (NW == 2 && R == 2) SANTA_BUDGETS(2, 2);
  else if (NW == 4 && R == 2) SANTA_BUDGETS(4, 2);
  else if (NW == 8 && R == 2) SANTA_BUDGETS(8, 2);
  else if (NW == 16 && R == 2) SANTA_BUDGETS(16, 2);
  else SANTA_BUDGETS(16, 4);
#undef SANTA_BUDGETS
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "budget launch failed: %s", hipGetErrorString(e));
  return SANTA_OK;
}

extern "C" int santa_prop_tile_budgets(const float* m_tiles, const float* ell_tiles, int H, int T_c, int S,
                                       uint64_t seed, float* m_star, int* S_tiles, float* invdelta, float* a0,
                                       hipStream_t stream) {
  if (H <= 0 || T_c <= 0) return set_error(SANTA_ERR_INVALID, "bad budget shape: H=%d T_c=%d", H, T_c);
  if (!m_tiles || !ell_tiles || !S_tiles || !invdelta || !a0)
    return set_error(SANTA_ERR_INVALID, "null pointer argument");
  const int st = prop_budgets_launch(m_tiles, ell_tiles, H, H, T_c, S, seed, m_star, S_tiles, invdelta, a0, stream);
  if (st != SANTA_OK) return st;
  return clear_error();
}

static int prop_pass2_launch(const void* V, const uint16_t* u_stash, int dtype, int B, int H, int KVH, int D, int L,
                             int L_storage, int block_n, int T_c, int S, const float* invdelta, const float* a0,
                             int16_t* counts, void* out, int* vrows, const prop::PropWs& w, char* base,
                             hipStream_t stream, const int* seq_lens = nullptr, const int* seq_S = nullptr,
                             int stash_ld = 0, PageTable pt = PageTable{nullptr, 0, 3, 1}) {
  float* part = reinterpret_cast<float*>(base + w.part);
  int* pe = reinterpret_cast<int*>(base + w.emit);
  const int GH = H / KVH;
  const int want_emit = vrows ? 1 : 0;
  const float scale_out = (S > 0) ? (1.0f / static_cast<float>(S)) : 0.0f;
  hipError_t e;
  if (propgen::generic_shape(GH, D, block_n)) {
    e = propgen::launch_pass2(V, u_stash, dtype, B, H, KVH, D, L, L_storage, block_n, T_c, w.cs, w.cpg, w.n_wg,
                              invdelta, a0, counts, part, pe, want_emit, seq_lens, pt, stream, stash_ld);
    if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "pass-2 launch failed: %s", hipGetErrorString(e));
    e = propgen::launch_finalize(part, pe, dtype, B, H, KVH, D, w.cpg, scale_out, out, vrows, seq_lens, seq_S,
                                 block_n, w.cs, L, w.n_wg, stream);
    if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "finalize launch failed: %s", hipGetErrorString(e));
    return SANTA_OK;
  }
  const prop::Pass2Grid rg{seq_lens, w.n_wg, stash_ld, pt};
  const uint16_t* Vh = static_cast<const uint16_t*>(V);
  if (dtype == SANTA_BF16)
    e = (GH == 4) ? prop::launch_pass2_bn<true, 4>(block_n, Vh, u_stash, B, H, KVH, L, L_storage, T_c, w.cs, w.cpg,
                                                   invdelta, a0, counts, part, pe, want_emit, rg, stream)
                  : prop::launch_pass2_bn<true, 8>(block_n, Vh, u_stash, B, H, KVH, L, L_storage, T_c, w.cs, w.cpg,
                                                   invdelta, a0, counts, part, pe, want_emit, rg, stream);
  else
    e = (GH == 4) ? prop::launch_pass2_bn<false, 4>(block_n, Vh, u_stash, B, H, KVH, L, L_storage, T_c, w.cs, w.cpg,
                                                    invdelta, a0, counts, part, pe, want_emit, rg, stream)
                  : prop::launch_pass2_bn<false, 8>(block_n, Vh, u_stash, B, H, KVH, L, L_storage, T_c, w.cs, w.cpg,
                                                    invdelta, a0, counts, part, pe, want_emit, rg, stream);
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "pass-2 launch failed: %s", hipGetErrorString(e));
  const unsigned grid = static_cast<unsigned>(B) * static_cast<unsigned>(H);
  uint16_t* o = static_cast<uint16_t*>(out);
  if (dtype == SANTA_BF16) {
    if (GH == 4)
      hipLaunchKernelGGL((prop::finalize_kernel<true, 4>), dim3(grid), dim3(prop::kD), 0, stream, part, pe, H, KVH,
                         w.cpg, scale_out, o, vrows, seq_lens, seq_S, block_n, w.cs, L, w.n_wg);
    else
      hipLaunchKernelGGL((prop::finalize_kernel<true, 8>), dim3(grid), dim3(prop::kD), 0, stream, part, pe, H, KVH,
                         w.cpg, scale_out, o, vrows, seq_lens, seq_S, block_n, w.cs, L, w.n_wg);
  } else {
    if (GH == 4)
      hipLaunchKernelGGL((prop::finalize_kernel<false, 4>), dim3(grid), dim3(prop::kD), 0, stream, part, pe, H, KVH,
                         w.cpg, scale_out, o, vrows, seq_lens, seq_S, block_n, w.cs, L, w.n_wg);
    else
      hipLaunchKernelGGL((prop::finalize_kernel<false, 8>), dim3(grid), dim3(prop::kD), 0, stream, part, pe, H, KVH,
                         w.cpg, scale_out, o, vrows, seq_lens, seq_S, block_n, w.cs, L, w.n_wg);
  }
  e = hipGetLastError();
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "finalize launch failed: %s", hipGetErrorString(e));
  return SANTA_OK;
}

extern "C" size_t santa_prop_workspace_size(int H, int KVH, int D, int L, int T_c) {
  if (H <= 0 || KVH <= 0 || H % KVH != 0 || D <= 0 || L <= 0 || T_c <= 0) return 0;
  return prop::prop_ws_layout(1, H, KVH, D, L, T_c).total;
}

extern "C" int santa_prop_pass2(const void* V, const void* u_stash, int dtype, int H, int KVH, int D, int L,
                                int block_n, int S, const float* invdelta, const float* a0, int16_t* counts,
                                void* out, int* vrows, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  int st = prop::check_common(dtype, H, KVH, D);
  if (st != SANTA_OK) return st;
  if (L <= 0) return set_error(SANTA_ERR_INVALID, "empty KV cache: L=%d", L);
  const int T_c = (L + block_n - 1) / block_n;
  if ((st = prop::check_bn(block_n, H / KVH, D)) != SANTA_OK) return st;
  if (!V || !u_stash || !invdelta || !a0 || !out) return set_error(SANTA_ERR_INVALID, "null pointer argument");
  const prop::PropWs w = prop::prop_ws_layout(1, H, KVH, D, L, T_c);
  if (!workspace || workspace_bytes < w.total)
    return set_error(SANTA_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", w.total, workspace_bytes);
  st = prop_pass2_launch(V, static_cast<const uint16_t*>(u_stash), dtype, 1, H, KVH, D, L, L, block_n, T_c, S,
                         invdelta, a0, counts, out, vrows, w, static_cast<char*>(workspace), stream);
  if (st != SANTA_OK) return st;
  return clear_error();
}

extern "C" int santa_prop_decode(const void* q, const void* K, const void* V, int dtype, int H, int KVH, int D, int L,
                                 int block_n, int pass1_path, int S, uint64_t seed, void* out, float* m_star,
                                 int* vrows, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  int st = prop::check_common(dtype, H, KVH, D);
  if (st != SANTA_OK) return st;
  if (L <= 0) return set_error(SANTA_ERR_INVALID, "empty KV cache: L=%d", L);
  const int T_c = (L + block_n - 1) / block_n;
  if ((st = prop::check_bn(block_n, H / KVH, D)) != SANTA_OK) return st;
  if (pass1_path == 0 && !(H / KVH == 4 && D == 128 && block_n == 256))
    return set_error(SANTA_ERR_INVALID, "SANTA_PASS1=vec requires GH=4, D=128, block_n=256. Got GH=%d D=%d block_n=%d",
                     H / KVH, D, block_n);
  if (!q || !K || !V || !out) return set_error(SANTA_ERR_INVALID, "null pointer argument");
  const prop::PropWs w = prop::prop_ws_layout(1, H, KVH, D, L, T_c);
  if (!workspace || workspace_bytes < w.total)
    return set_error(SANTA_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", w.total, workspace_bytes);
  char* base = static_cast<char*>(workspace);
  float* m_tiles = reinterpret_cast<float*>(base + w.m);
  float* ell_tiles = reinterpret_cast<float*>(base + w.ell);
  int* S_tiles = reinterpret_cast<int*>(base + w.st);
  float* inv = reinterpret_cast<float*>(base + w.inv);
  float* a0 = reinterpret_cast<float*>(base + w.a0);
  uint16_t* stash = reinterpret_cast<uint16_t*>(base + w.stash);
  const bool gen = propgen::generic_shape(H / KVH, D, block_n);
  // a pass 1 on the wave kernel (the vec path, the general path at GH 8)
  // keeps the stash tile-major between the two passes, except for a small
  // pass, which runs four waves per tile with the [L, H] stash
  // (the generic path keeps it tile-major too wherever its fast pass 1 runs)
  const bool small = flash::small_prop_pass(static_cast<long long>(T_c) * KVH);
  const int sld = gen ? (propgen::fast_pass1_shape(H / KVH, D, block_n) ? prop::stash_ld(L) : 0)
                      : ((flash::prop_wave_pass1(pass1_path, H / KVH, block_n) && !small) ? prop::stash_ld(L) : 0);
  hipError_t e = gen ? propgen::launch_pass1(q, K, dtype, 1, H, KVH, D, L, L, block_n, m_tiles, ell_tiles, stash,
                                             nullptr, -1, PageTable{nullptr, 0, 3, 1}, stream, sld)
                     : flash::launch_prop_pass1(q, K, dtype, 1, H, KVH, L, L, block_n, pass1_path, m_tiles, ell_tiles,
                                                stash, nullptr, 0, 0, sld, stream);
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "pass-1 launch failed: %s", hipGetErrorString(e));
  if ((st = prop_budgets_launch(m_tiles, ell_tiles, H, H, T_c, S, seed, m_star, S_tiles, inv, a0, stream)) != SANTA_OK)
    return st;
  if ((st = prop_pass2_launch(V, stash, dtype, 1, H, KVH, D, L, L, block_n, T_c, S, inv, a0, nullptr, out, vrows, w,
                              base, stream, nullptr, nullptr, sld)) != SANTA_OK)
    return st;
  return clear_error();
}

extern "C" size_t santa_prop_batched_workspace_size(int B, int H, int KVH, int D, int L_storage, int max_tiles,
                                                    long long total_tiles) {
  if (B <= 0 || H <= 0 || KVH <= 0 || H % KVH != 0 || D <= 0 || L_storage <= 0 || max_tiles <= 0 || total_tiles < 0)
    return 0;
  return prop::prop_ws_layout(B, H, KVH, D, L_storage, max_tiles, total_tiles).total;
}

// The batched decode over a contiguous [B, L_storage, KVH, D] cache or, with
// pt.table set, a paged one (L_storage then only sizes the stash).
static int prop_decode_batched(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH, int D,
                               int L_storage, const int* seq_lens, const int* seq_S, int max_len,
                               long long total_tiles, int block_n, int pass1_path, uint64_t seed, void* out,
                               float* m_star, int* vrows, void* workspace, size_t workspace_bytes, hipStream_t stream,
                               const PageTable& pt) {
  int st = prop::check_common(dtype, H, KVH, D);
  if (st != SANTA_OK) return st;
  if (B <= 0) return set_error(SANTA_ERR_INVALID, "empty batch");
  if (max_len <= 0 || max_len > L_storage)
    return set_error(SANTA_ERR_INVALID, "max_len must be in [1, L_storage]: max_len=%d L_storage=%d", max_len, L_storage);
  const int T_c = (max_len + block_n - 1) / block_n;
  if ((st = prop::check_bn(block_n, H / KVH, D)) != SANTA_OK) return st;
  if (total_tiles < 0 || total_tiles > static_cast<long long>(B) * T_c)
    return set_error(SANTA_ERR_INVALID, "total_tiles out of range");
  if (pass1_path == 0 && !(H / KVH == 4 && D == 128 && block_n == 256))
    return set_error(SANTA_ERR_INVALID, "SANTA_PASS1=vec requires GH=4, D=128, block_n=256. Got GH=%d D=%d block_n=%d",
                     H / KVH, D, block_n);
  if (!q || !K || !V || !out || !seq_lens || !seq_S) return set_error(SANTA_ERR_INVALID, "null pointer argument");
  const prop::PropWs w = prop::prop_ws_layout(B, H, KVH, D, L_storage, T_c, total_tiles);
  if (!workspace || workspace_bytes < w.total)
    return set_error(SANTA_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", w.total, workspace_bytes);
  char* base = static_cast<char*>(workspace);
  float* m_tiles = reinterpret_cast<float*>(base + w.m);
  float* ell_tiles = reinterpret_cast<float*>(base + w.ell);
  int* S_tiles = reinterpret_cast<int*>(base + w.st);
  float* inv = reinterpret_cast<float*>(base + w.inv);
  float* a0 = reinterpret_cast<float*>(base + w.a0);
  uint16_t* stash = reinterpret_cast<uint16_t*>(base + w.stash);
  const bool gen = propgen::generic_shape(H / KVH, D, block_n);
  const bool small = !pt.table && flash::small_prop_pass(total_tiles * KVH);  // as in the scalar call
  const int sld =
      gen ? (propgen::fast_pass1_shape(H / KVH, D, block_n) ? prop::stash_ld(L_storage) : 0)
          : ((flash::prop_wave_pass1(pass1_path, H / KVH, block_n) && !small) ? prop::stash_ld(L_storage) : 0);
  hipError_t e = gen ? propgen::launch_pass1(q, K, dtype, B, H, KVH, D, max_len, L_storage, block_n, m_tiles,
                                             ell_tiles, stash, seq_lens, total_tiles, pt, stream, sld)
                     : flash::launch_prop_pass1(q, K, dtype, B, H, KVH, max_len, L_storage, block_n, pass1_path,
                                                m_tiles, ell_tiles, stash, seq_lens, w.cs, w.n_wg, sld, stream, pt,
                                                total_tiles);
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "pass-1 launch failed: %s", hipGetErrorString(e));
  if ((st = prop_budgets_launch(m_tiles, ell_tiles, B * H, H, T_c, 0, seed, m_star, S_tiles, inv, a0, stream, seq_lens,
                                seq_S, block_n)) != SANTA_OK)
    return st;
  if ((st = prop_pass2_launch(V, stash, dtype, B, H, KVH, D, max_len, L_storage, block_n, T_c, 0, inv, a0, nullptr,
                              out, vrows, w, base, stream, seq_lens, seq_S, sld, pt)) != SANTA_OK)
    return st;
  return clear_error();
}

extern "C" int santa_prop_decode_batched(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH,
                                         int D, int L_storage, const int* seq_lens, const int* seq_S, int max_len,
                                         long long total_tiles, int block_n, int pass1_path, uint64_t seed, void* out,
                                         float* m_star, int* vrows, void* workspace, size_t workspace_bytes,
                                         hipStream_t stream) {
  return prop_decode_batched(q, K, V, dtype, B, H, KVH, D, L_storage, seq_lens, seq_S, max_len, total_tiles, block_n,
                             pass1_path, seed, out, m_star, vrows, workspace, workspace_bytes, stream,
                             PageTable{nullptr, 0, 3, 1});
}

extern "C" int santa_prop_decode_paged(const void* q, const void* K_pages, const void* V_pages, int dtype, int B, int H,
                                       int KVH, int D, int num_pages, int page_size, const int* block_table,
                                       int table_stride, const int* seq_lens, const int* seq_S, int max_len,
                                       long long total_tiles, int block_n, int pass1_path, uint64_t seed, void* out,
                                       float* m_star, int* vrows, void* workspace, size_t workspace_bytes,
                                       hipStream_t stream) {
  PageTable pt{};
  const int st = check_page_table(block_table, num_pages, page_size, table_stride, max_len, &pt);
  if (st != SANTA_OK) return st;
  return prop_decode_batched(q, K_pages, V_pages, dtype, B, H, KVH, D, max_len, seq_lens, seq_S, max_len, total_tiles,
                             block_n, pass1_path, seed, out, m_star, vrows, workspace, workspace_bytes, stream, pt);
}
