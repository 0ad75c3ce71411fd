// santa_device.h -- gfx950 device numerics and wave64 primitives shared by
// the santa_flash and santa_prop kernels.
//
// Every routine here is IEEE binary32 with round-to-nearest-even.  The
// translation units are compiled with -ffp-contract=off so that a*b+c is
// never fused unless written as fmaf(); the bit patterns the kernels produce
// (scores, tile softmax statistics, sampled counts) therefore depend only on
// the association order spelled out in the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "santa_internal.h"  // PageTable

namespace santa {

// ---------------------------------------------------------------- 16-bit I/O
// bf16 -> f32 is a 16-bit shift (flash/santa_cuda_kernel.cu:33-36); f16 -> f32
// is the exact hardware conversion.  Both are exact.
template <bool BF16>
__device__ __forceinline__ float lo16_to_f32(uint32_t w) {
  if constexpr (BF16) {
    return __uint_as_float(w << 16);
  } else {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
  }
}
template <bool BF16>
__device__ __forceinline__ float hi16_to_f32(uint32_t w) {
  if constexpr (BF16) {
    return __uint_as_float(w & 0xffff0000u);
  } else {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
  }
}
template <bool BF16>
__device__ __forceinline__ float h16_to_f32(uint16_t h) {
  return lo16_to_f32<BF16>(static_cast<uint32_t>(h));
}

// f32 -> bf16 / f16, round to nearest even (the reference's __float2bfloat16 /
// __float2half_rn, flash/santa_cuda_kernel.cu:53-55).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t qnan = (u >> 16) | 0x0040u;
  return static_cast<uint16_t>(((u & 0x7fffffffu) > 0x7f800000u) ? qnan : rne);
}
// f32 -> f16 in integer arithmetic.  A plain (_Float16) cast lets the
// backend fold a preceding f32 multiply into v_fma_mixlo_f16, which rounds
// once instead of twice; the integer form keeps the two IEEE roundings.
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  const uint32_t x = __float_as_uint(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return static_cast<uint16_t>(sign | 0x7c00u | (ax > 0x7f800000u ? 0x0200u : 0u));
  if (ax >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // rounds to infinity
  if (ax < 0x38800000u) {                                                 // f16 subnormal or zero
    const uint32_t e = ax >> 23;
    if (e < 101u) return static_cast<uint16_t>(sign);
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;  // 14 .. 25
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return static_cast<uint16_t>(sign | q);
  }
  const uint32_t r = ax + 0x0fffu + ((ax >> 13) & 1u);
  return static_cast<uint16_t>(sign | ((r - 0x38000000u) >> 13));
}
template <bool BF16>
__device__ __forceinline__ uint16_t f32_to_h16(float f) {
  if constexpr (BF16) {
    return f32_to_bf16_rne(f);
  } else {
    return f32_to_f16_rne(f);
  }
}

// ---------------------------------------------------------------- RNG
// SplitMix64 (Vigna) and the per-(key, tile) uniform offset of the
// systematic sampler, flash/santa_cuda_kernel.cu:74-87.
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ULL;
  uint64_t z = x;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}
__device__ __forceinline__ float u01(uint64_t seed, int key, int t) {
  const uint64_t x = seed ^ ((static_cast<uint64_t>(static_cast<int64_t>(key)) << 32) ^
                             static_cast<uint64_t>(static_cast<int64_t>(t)));
  const uint64_t r = splitmix64(x);
  const double u = static_cast<double>(r >> 11) * (1.0 / 9007199254740992.0);
  return static_cast<float>(u);
}

// ---------------------------------------------------------------- EXP
// This project's binary32 exponential: Cody-Waite reduction with ln2 split
// hi/lo, degree-7 Taylor polynomial in Horner form with explicit fma, and
// scaling by 2^n as two exact power-of-two multiplies (one rounding for
// subnormal results).  exp(0) == 1 exactly; <= 2 ulp from the true value.
__device__ __forceinline__ float santa_expf(float x) {
  // Branch-free: the argument is clamped to [-104, 89] (outside it the
  // result is 0 or inf either way) and 2^n is applied by one v_ldexp_f32,
  // which rounds p * 2^n once -- the same value as the two exact
  // power-of-two multiplies of the restatement.  NaN passes through.
  const float xc = fminf(fmaxf(x, -104.0f), 89.0f);
  const float n = __builtin_rintf(xc * 1.44269502162933349609375f);
  float r = fmaf(n, -0.693145751953125f, xc);
  r = fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.984126984126984e-4f;
  p = fmaf(p, r, 1.3888888888888889e-3f);
  p = fmaf(p, r, 8.3333333333333333e-3f);
  p = fmaf(p, r, 4.1666666666666667e-2f);
  p = fmaf(p, r, 1.6666666666666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const float res = __builtin_amdgcn_ldexpf(p, static_cast<int>(n));
  return (x != x) ? x : res;
}

// santa_expf for x <= 0 that is not NaN (the softmax weights exp(s - m)):
// the same value with the upper clamp and the NaN select left out.
__device__ __forceinline__ float santa_expf_nonpos(float x) {
  const float xc = fmaxf(x, -104.0f);
  const float n = __builtin_rintf(xc * 1.44269502162933349609375f);
  float r = fmaf(n, -0.693145751953125f, xc);
  r = fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.984126984126984e-4f;
  p = fmaf(p, r, 1.3888888888888889e-3f);
  p = fmaf(p, r, 8.3333333333333333e-3f);
  p = fmaf(p, r, 4.1666666666666667e-2f);
  p = fmaf(p, r, 1.6666666666666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return __builtin_amdgcn_ldexpf(p, static_cast<int>(n));
}

// f32 -> 16-bit (RNE) -> f32 for a finite, non-negative value: for bf16 the
// rounding is done in place on the bit pattern (no NaN case to handle).
template <bool BF16>
__device__ __forceinline__ float round16_nonneg(float f) {
  if constexpr (BF16) {
    const uint32_t u = __float_as_uint(f);
    return __uint_as_float((u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u);
  } else {
    return h16_to_f32<false>(f32_to_f16_rne(f));
  }
}

// float -> int as the reference's (int)(f_curr - f_prev) sees it for the
// finite, small differences that occur; NaN maps to 0 (then clamped).
// Clamping the float difference to [0, 32767] before the conversion is the
// same as clamping the integer (and fmaxf maps NaN to 0).
__device__ __forceinline__ int count_from_floors(float a0, float pg, float cum) {
  const float d = floorf(a0 + cum) - floorf(a0 + pg);
  return static_cast<int>(fminf(fmaxf(d, 0.0f), 32767.0f));
}

// ---------------------------------------------------------------- grids
// Position of workgroup wg in a persistent chunked grid.  Uniform form: every
// sequence has T_c tiles in cpg chunks of cs tiles, wg = (b * cpg + chunk) *
// KVH + kv.  Ragged form (seq_lens != nullptr): sequence b has
// T_b = ceil(seq_lens[b] / BN) tiles in ceil(T_b / cs) chunks, and its
// workgroups follow those of sequences 0 .. b-1 (kv fastest); workgroups past
// the last sequence get an empty tile range (b = -1).
// Length of sequence b of a ragged batch, clamped to [1, max_rows] so that a
// malformed length can only give wrong numbers, never an access outside the
// [B, L_storage] cache or the [B, H, T_c] tile arrays.
__device__ __forceinline__ int ragged_len(const int* seq_lens, int b, int max_rows) {
  return min(max(seq_lens[b], 1), max_rows);
}

struct GridPos {
  int b, kv, chunk, len, n_tiles, wg_base;
};
__device__ __forceinline__ GridPos grid_pos(int wg, const int* seq_lens, int B, int KVH, int BN, int L_valid, int T_c,
                                            int cs, int cpg) {
  GridPos p;
  if (!seq_lens) {
    p.kv = wg % KVH;
    p.chunk = (wg / KVH) % cpg;
    p.b = wg / (KVH * cpg);
    p.len = L_valid;
    p.n_tiles = T_c;
    p.wg_base = p.b * cpg * KVH;
    return p;
  }
  int base = 0;
  p.b = -1;
  p.kv = 0;
  p.chunk = 0;
  p.len = 0;
  p.n_tiles = 0;
  p.wg_base = 0;
  for (int bb = 0; bb < B; ++bb) {
    const int len = ragged_len(seq_lens, bb, L_valid);
    const int tiles = (len + BN - 1) / BN;
    const int n = KVH * ((tiles + cs - 1) / cs);
    if (wg < base + n) {
      const int local = wg - base;
      p.b = bb;
      p.kv = local % KVH;
      p.chunk = local / KVH;
      p.len = len;
      p.n_tiles = tiles;
      p.wg_base = base;
      break;
    }
    base += n;
  }
  return p;
}

// ---------------------------------------------------------------- paged KV
// Paged caches (PageTable): page ids are clamped to [0, num_pages), so a
// malformed table gives wrong numbers, never an access outside the pool.

// The pages of rows [n0, n0 + rows) of sequence b that lie below len, one per
// lane: lane i holds the page of row block (n0 >> shift) + i; lanes past the
// last such page (all lanes when n0 >= len) hold page 0.
__device__ __forceinline__ int pages_of_rows(const PageTable& pt, int b, int n0, int rows, int len, int lane) {
  const int last = min(n0 + rows, len) - 1;
  const int p0 = n0 >> pt.shift;
  const int np = (last >= n0) ? (last >> pt.shift) - p0 + 1 : 0;
  int v = 0;
  if (lane < np) v = pt.table[static_cast<size_t>(b) * pt.stride + p0 + lane];
  return min(max(v, 0), pt.num_pages - 1);
}

// Per lane: the page of token `row` of sequence b (page 0 where !ok).
__device__ __forceinline__ int page_of_row(const PageTable& pt, int b, int row, bool ok) {
  const int v = ok ? pt.table[static_cast<size_t>(b) * pt.stride + (row >> pt.shift)] : 0;
  return min(max(v, 0), pt.num_pages - 1);
}

// Byte offset from the pool base of token n, which lies in page `page`.
__device__ __forceinline__ size_t paged_row(const PageTable& pt, int page, int n, uint32_t row_bytes) {
  return ((static_cast<size_t>(page) << pt.shift) + static_cast<size_t>(n & ((1 << pt.shift) - 1))) * row_bytes;
}

// ---------------------------------------------------------------- DPP
// gfx9 DPP controls used by the 8-lane score tree.
enum : int {
  kDppQuadXor1 = 0xB1,      // quad_perm [1,0,3,2]
  kDppQuadXor2 = 0x4E,      // quad_perm [2,3,0,1]
  kDppRowHalfMirror = 0x141, // lane i <-> 7-i within each 8 lanes
  kDppRowMirror = 0x140,     // lane i <-> 15-i within each 16 lanes
  kDppRowBcast15 = 0x142,    // lane 15 of each row to the next row
  kDppRowBcast31 = 0x143     // lane 31 to rows 2 and 3
};
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// v from lane (i + N) of the same 16-lane row, 0 where that lane is outside it.
template <int N>
__device__ __forceinline__ float dpp_shl_zero(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + N, 0xF, 0xF, true));
}

// dpp<CTRL>(v) + 0.0f: the same value (scores and sums are never -0.0 here)
// but a floating-point result, so a following fmaxf needs no NaN
// canonicalisation of its operands and compiles to one v_max_f32.
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false)) + 0.0f;
}

// v from lane (i - N) of the same 16-lane row, 0 where that lane is outside it.
template <int N>
__device__ __forceinline__ float dpp_shr_zero(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x110 + N, 0xF, 0xF, true));
}

// Order keys: a monotone bijection float <-> int32 (flip the magnitude bits
// of negative values), so a float maximum is an integer maximum -- which
// needs no NaN canonicalisation and fuses with DPP.  Exact for every
// non-NaN input (-0.0 orders below +0.0).
__device__ __forceinline__ int order_key(float f) {
  const int b = __float_as_int(f);
  return b ^ static_cast<int>(static_cast<unsigned>(b >> 31) >> 1);
}
__device__ __forceinline__ float from_order_key(int k) {
  return __int_as_float(k ^ static_cast<int>(static_cast<unsigned>(k >> 31) >> 1));
}

// Maximum of order keys over the 64 lanes of a wave, valid in lane 63:
// DPP inside each 16-lane row, then the row broadcasts 15 and 31 (rows left
// out by a broadcast see INT_MIN, the identity).
__device__ __forceinline__ int wave_max_key_lane63(int k) {
  k = max(k, __builtin_amdgcn_update_dpp(0, k, kDppQuadXor1, 0xF, 0xF, false));
  k = max(k, __builtin_amdgcn_update_dpp(0, k, kDppQuadXor2, 0xF, 0xF, false));
  k = max(k, __builtin_amdgcn_update_dpp(0, k, kDppRowHalfMirror, 0xF, 0xF, false));
  k = max(k, __builtin_amdgcn_update_dpp(0, k, kDppRowMirror, 0xF, 0xF, false));
  k = max(k, __builtin_amdgcn_update_dpp(-2147483647 - 1, k, kDppRowBcast15, 0xA, 0xF, false));
  k = max(k, __builtin_amdgcn_update_dpp(-2147483647 - 1, k, kDppRowBcast31, 0xC, 0xF, false));
  return k;
}

// Max over the 64 lanes of a wave (exact in any order), valid in lane 63:
// DPP inside each 16-lane row, then the row broadcasts 15 and 31.  v must be
// the result of floating-point arithmetic (or a constant).
__device__ __forceinline__ float wave_max_lane63(float v) {
  v = fmaxf(v, dppf<kDppQuadXor1>(v));
  v = fmaxf(v, dppf<kDppQuadXor2>(v));
  v = fmaxf(v, dppf<kDppRowHalfMirror>(v));
  v = fmaxf(v, dppf<kDppRowMirror>(v));
  // rows 1, 3 take lane 15 / 47; then rows 2, 3 take lane 31
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), kDppRowBcast15, 0xA,
                                                          0xF, false)) + 0.0f);
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), kDppRowBcast31, 0xC,
                                                          0xF, false)) + 0.0f);
  return v;
}

// ------------------------------------------------------ systematic counts
// Counts of one head over one tile of len <= 32 * NCH rows (A.5-A.7 of the
// sampler, flash/santa_cuda_kernel.cu:275-311; prop/santa_cuda_kernel.cu:
// 771-807).  Rows are held two per lane: lane 16j+q of register pair p holds
// rows 32(4p+j)+2q (x0) and 32(4p+j)+2q+1 (x1), so every step of the 32-row
// Hillis-Steele scan (offsets 1, 2, 4, 8, 16) stays inside one 16-lane DPP
// row and pairs the same elements as the reference's 32-lane scan
// (flash/santa_cuda_kernel.cu:60-69).  x = f32(u16) * invdel, 0 past len.
// The 32-row chunk totals (pre + x at the chunk's last row) are carried
// sequentially; c = floor(a0 + pre + x) - floor(a0 + pre) clamped to
// [0, 32767].
// In-row inclusive scan of the register pairs; pre0 / pre1 are the exclusive
// prefixes of x0 / x1 inside each 32-row chunk.
template <int NP>
__device__ __forceinline__ void scan_pairs(const float (&x0)[NP], const float (&x1)[NP], float (&pre0)[NP],
                                           float (&pre1)[NP]) {
  float r0[NP], r1[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    r1[p] = x1[p] + x0[p];
    r0[p] = x0[p] + dpp_shr_zero<1>(x1[p]);
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    r0[p] = r0[p] + dpp_shr_zero<1>(r0[p]);
    r1[p] = r1[p] + dpp_shr_zero<1>(r1[p]);
    r0[p] = r0[p] + dpp_shr_zero<2>(r0[p]);
    r1[p] = r1[p] + dpp_shr_zero<2>(r1[p]);
    r0[p] = r0[p] + dpp_shr_zero<4>(r0[p]);
    r1[p] = r1[p] + dpp_shr_zero<4>(r1[p]);
    r0[p] = r0[p] + dpp_shr_zero<8>(r0[p]);
    r1[p] = r1[p] + dpp_shr_zero<8>(r1[p]);
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    pre0[p] = r0[p] - x0[p];
    pre1[p] = r1[p] - x1[p];
  }
}

// The counts of a full tile (len = 32 * NCH): every chunk ends at its row's
// lane 15, odd element.  No branch, so the callers can interleave heads.
template <int NCH, int NP = (NCH + 3) / 4>
__device__ __forceinline__ void systematic_counts_full(const float (&x0)[NP], const float (&x1)[NP], float a0,
                                                       int lane, int (&c0)[NP], int (&c1)[NP]) {
  const int jrow = lane >> 4;
  float pre0[NP], pre1[NP], car[NP];
  scan_pairs<NP>(x0, x1, pre0, pre1);
  float carry = 0.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const float tot1 = pre1[p] + x1[p];
    float cj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      cj[j] = carry;
      if (4 * p + j < NCH) carry = carry + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tot1), 16 * j + 15));
    }
    car[p] = (jrow == 0) ? cj[0] : (jrow == 1) ? cj[1] : (jrow == 2) ? cj[2] : cj[3];
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const float pg0 = car[p] + pre0[p];
    const float pg1 = car[p] + pre1[p];
    c0[p] = count_from_floors(a0, pg0, pg0 + x0[p]);
    c1[p] = count_from_floors(a0, pg1, pg1 + x1[p]);
    if (32 * (4 * p + jrow) >= 32 * NCH) {  // rows past BN (BN < 128)
      c0[p] = 0;
      c1[p] = 0;
    }
  }
}

template <int NCH, int NP = (NCH + 3) / 4>
__device__ __forceinline__ void systematic_counts(const float (&x0)[NP], const float (&x1)[NP], int len, float a0,
                                                  int lane, int (&c0)[NP], int (&c1)[NP]) {
  if (len >= 32 * NCH) {
    systematic_counts_full<NCH>(x0, x1, a0, lane, c0, c1);
    return;
  }
  const int jrow = lane >> 4;
  const int qq = lane & 15;
  float pre0[NP], pre1[NP], car[NP];
  scan_pairs<NP>(x0, x1, pre0, pre1);
  float carry = 0.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const float tot0 = pre0[p] + x0[p];
    const float tot1 = pre1[p] + x1[p];
    float cj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rem = len - 32 * (4 * p + j);
      cj[j] = carry;
      if (4 * p + j < NCH && rem > 0) {
        const int last = min(31, rem - 1);
        const int src = 16 * j + (last >> 1);
        const float tot = (last & 1) ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tot1), src))
                                     : __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tot0), src));
        carry = carry + tot;
      }
    }
    car[p] = (jrow == 0) ? cj[0] : (jrow == 1) ? cj[1] : (jrow == 2) ? cj[2] : cj[3];
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int row = 32 * (4 * p + jrow) + 2 * qq;
    const float pg0 = car[p] + pre0[p];
    const float pg1 = car[p] + pre1[p];
    c0[p] = (row < len) ? count_from_floors(a0, pg0, pg0 + x0[p]) : 0;
    c1[p] = (row + 1 < len) ? count_from_floors(a0, pg1, pg1 + x1[p]) : 0;
  }
}

// Max over the 64 lanes of a wave (exact in any order).
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Lane 0 of the reference's 32-lane __shfl_down tree (off 16,8,4,2,1) over
// 32 values held in registers: the classic pairwise tree.
__device__ __forceinline__ float tree32(float* v) {
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) {
#pragma unroll
    for (int l = 0; l < off; ++l) v[l] = v[l] + v[l + off];
  }
  return v[0];
}

// The value of lane (lane ^ J): DPP inside 16-lane rows (quad permutes for
// 1 and 2; row shifts up or down for 4 and 8, picked by the lane's bit J),
// the row and half-wave swaps for 16 and 32 (no LDS round trip).
template <int J>
__device__ __forceinline__ int lane_xor(int v, int lane) {
  if constexpr (J == 1) {
    return __builtin_amdgcn_update_dpp(0, v, kDppQuadXor1, 0xF, 0xF, false);
  } else if constexpr (J == 2) {
    return __builtin_amdgcn_update_dpp(0, v, kDppQuadXor2, 0xF, 0xF, false);
  } else if constexpr (J == 4 || J == 8) {
    const int from_above = __builtin_amdgcn_update_dpp(0, v, 0x100 + J, 0xF, 0xF, true);  // lane + J
    const int from_below = __builtin_amdgcn_update_dpp(0, v, 0x110 + J, 0xF, 0xF, true);  // lane - J
    return (lane & J) ? from_below : from_above;
  } else if constexpr (J == 16) {
    // the swap of the odd rows of its first operand with the even rows of its
    // second (both v) leaves rows (0, 0, 2, 2) in the first result and
    // (1, 1, 3, 3) in the second: even rows take the second, odd the first
    const auto s = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false, false);
    return static_cast<int>((lane & 16) ? s[0] : s[1]);
  } else {
    static_assert(J == 32, "lane_xor: J is a power of two below 64");
    // the swap of the upper half of its first operand with the lower half of
    // its second (both v) leaves (lo, lo) in the first result and (hi, hi) in
    // the second: the lower half takes the second, the upper the first
    const auto s = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false, false);
    return static_cast<int>((lane & 32) ? s[0] : s[1]);
  }
}

// Chunk sums of the finalize kernels: s += fv(c) and e += fe(c) (fe only
// where with_e) over chunks c = 0 .. n - 1 in ascending order, the loads of up
// to 32 chunks issued before the first add: full batches of 32, then one batch
// of 8, 16 or 32 for what is left (loads past n repeat chunk n - 1 and are
// not added).
template <int NB, class FV, class FE>
__device__ __forceinline__ void chunk_batch(int c0, int n, FV fv, FE fe, bool with_e, float& s, int& e) {
  float v[NB];
  int ev[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int c = min(c0 + i, n - 1);
    v[i] = fv(c);
    ev[i] = with_e ? fe(c) : 0;
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    if (c0 + i < n) {
      s += v[i];
      e += ev[i];
    }
  }
}
template <class FV, class FE>
__device__ __forceinline__ void sum_chunks(int n, FV fv, FE fe, bool with_e, float& s, int& e) {
  int c0 = 0;
  for (; c0 + 32 <= n; c0 += 32) chunk_batch<32>(c0, n, fv, fe, with_e, s, e);
  const int r = n - c0;
  if (r > 16) {
    chunk_batch<32>(c0, n, fv, fe, with_e, s, e);
  } else if (r > 8) {
    chunk_batch<16>(c0, n, fv, fe, with_e, s, e);
  } else if (r > 0) {
    chunk_batch<8>(c0, n, fv, fe, with_e, s, e);
  }
}

}  // namespace santa
