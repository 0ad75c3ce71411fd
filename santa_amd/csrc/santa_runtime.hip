// santa_runtime.hip -- fused elementwise kernels of the model-level decode
// step (santa_amd/runtime.py): the residual add with the RMSNorm that
// follows it, RoPE of q and k with the step's cache write, and the SwiGLU
// product.  Each replaces a chain of small torch kernels (about 26 per layer
// and step) with one launch and keeps torch's bf16 semantics: values are
// rounded to bf16 where the torch expression rounds them, and the norm is
// computed in float32 as in the torch expression.  The counterpart in the
// reference is the HF model's own decoder layer
// (tutorial_code/runtime_common.py:501-571), which runs them as separate
// torch kernels too.
#include "santa_device.h"
#include "santa_amd.h"
#include "santa_internal.h"

namespace santa {
namespace rt {

__device__ __forceinline__ float bf(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }
__device__ __forceinline__ uint16_t to_bf(float f) { return f32_to_h16<true>(f); }

constexpr int kNormThreads = 256;

// One workgroup per row: h = bf16(h + a) when add, then
// x = bf16(float(w) * float(bf16(float(h) * rsqrt(mean(float(h)^2) + eps)))),
// the roundings of LlamaRMSNorm: the normalised row is rounded to bf16
// before the weight multiply.
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(uint16_t* __restrict__ h,
                                                                    const uint16_t* __restrict__ a,
                                                                    const uint16_t* __restrict__ w,
                                                                    uint16_t* __restrict__ x, int hidden, float eps,
                                                                    int add) {
  __shared__ float s_part[kNormThreads / 64];
  const size_t row = blockIdx.x;
  uint16_t* hr = h + row * hidden;
  const uint16_t* ar = a ? a + row * hidden : nullptr;
  uint16_t* xr = x + row * hidden;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < hidden; i += kNormThreads) {
    float v = bf(hr[i]);
    if (add) {
      const uint16_t s = to_bf(v + bf(ar[i]));
      hr[i] = s;
      v = bf(s);
    }
    ss = fmaf(v, v, ss);
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) ss += __shfl_xor(ss, m, 64);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += s_part[i];
  const float r = 1.0f / sqrtf(tot / static_cast<float>(hidden) + eps);
  for (int i = threadIdx.x; i < hidden; i += kNormThreads) xr[i] = to_bf(bf(w[i]) * bf(to_bf(bf(hr[i]) * r)));
}

// The same computation for rows of 16-byte-aligned vectors of 8 values
// (hidden a multiple of 8, at most 512 x 8 x R): 512 threads, thread t
// holding vectors t, t + 512, ... of h, a and w in registers, all loaded
// before any is used, so a row costs one memory round trip, one reduction
// and one store instead of a dependent loop.  Same roundings; only the order
// of the float32 sum of squares differs.
constexpr int kNormVecThreads = 512;
template <int R>
__global__ __launch_bounds__(kNormVecThreads) void add_rms_norm_vec_kernel(uint16_t* __restrict__ h,
                                                                           const uint16_t* __restrict__ a,
                                                                           const uint16_t* __restrict__ w,
                                                                           uint16_t* __restrict__ x, int hidden,
                                                                           float eps, int add) {
  __shared__ float s_part[kNormVecThreads / 64];
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  const size_t row = blockIdx.x;
  const int nv = hidden / 8;
  const int tid = static_cast<int>(threadIdx.x);
  u32x4v* hr = reinterpret_cast<u32x4v*>(h + row * hidden);
  const u32x4v* ar = add ? reinterpret_cast<const u32x4v*>(a + row * hidden) : nullptr;
  const u32x4v* wr = reinterpret_cast<const u32x4v*>(w);
  u32x4v* xr = reinterpret_cast<u32x4v*>(x + row * hidden);
  u32x4v hv[R], av[R], wv[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = tid + r * kNormVecThreads;
    if (i < nv) {
      hv[r] = hr[i];
      av[r] = add ? ar[i] : u32x4v{0u, 0u, 0u, 0u};
      wv[r] = wr[i];
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = tid + r * kNormVecThreads;
    if (i < nv) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float lo = __uint_as_float(hv[r][k] << 16), hi = __uint_as_float(hv[r][k] & 0xffff0000u);
        if (add) {
          const uint32_t slo = to_bf(lo + __uint_as_float(av[r][k] << 16));
          const uint32_t shi = to_bf(hi + __uint_as_float(av[r][k] & 0xffff0000u));
          hv[r][k] = slo | (shi << 16);
          lo = bf(static_cast<uint16_t>(slo));
          hi = bf(static_cast<uint16_t>(shi));
        }
        ss = fmaf(lo, lo, ss);
        ss = fmaf(hi, hi, ss);
      }
      if (add) hr[i] = hv[r];
    }
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) ss += __shfl_xor(ss, m, 64);
  if ((tid & 63) == 0) s_part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormVecThreads / 64; ++i) tot += s_part[i];
  const float rs = 1.0f / sqrtf(tot / static_cast<float>(hidden) + eps);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = tid + r * kNormVecThreads;
    if (i < nv) {
      u32x4v o;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float lo = __uint_as_float(hv[r][k] << 16), hi = __uint_as_float(hv[r][k] & 0xffff0000u);
        const float wlo = __uint_as_float(wv[r][k] << 16), whi = __uint_as_float(wv[r][k] & 0xffff0000u);
        const uint32_t olo = to_bf(wlo * bf(to_bf(lo * rs)));
        const uint32_t ohi = to_bf(whi * bf(to_bf(hi * rs)));
        o[k] = olo | (ohi << 16);
      }
      xr[i] = o;
    }
  }
}

// Thread per (b, head, d): heads [0, H) are q (to q_out [B, H, D]), [H,
// H + KVH) are k (to k_cache[b, pos]), [H + KVH, H + 2 KVH) are v (to
// v_cache[b, pos], unrotated).  RoPE in the rotate-half convention with
// torch's bf16 rounding of each product and of the sum:
// out = bf16(bf16(x * cos) + bf16(rot(x) * sin)), rot(x) = (-x[D/2:], x[:D/2]).
__global__ __launch_bounds__(256) void rope_write_kernel(const uint16_t* __restrict__ qkv,
                                                         const uint16_t* __restrict__ cos_,
                                                         const uint16_t* __restrict__ sin_,
                                                         uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
                                                         uint16_t* __restrict__ v_cache, int B, int H, int KVH,
                                                         int D, long long storage, int pos) {
  const long long total = static_cast<long long>(B) * (H + 2 * KVH) * D;
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int d = static_cast<int>(i % D);
  const int hh = static_cast<int>((i / D) % (H + 2 * KVH));
  const int b = static_cast<int>(i / (static_cast<long long>(D) * (H + 2 * KVH)));
  const uint16_t* src = qkv + (static_cast<size_t>(b) * (H + 2 * KVH) + hh) * D;
  const int half = D / 2;
  if (hh >= H + KVH) {  // v: copied
    v_cache[((static_cast<size_t>(b) * storage + pos) * KVH + (hh - H - KVH)) * D + d] = src[d];
    return;
  }
  const float x = bf(src[d]);
  const float rx = (d < half) ? -bf(src[d + half]) : bf(src[d - half]);
  const uint16_t o = to_bf(bf(to_bf(x * bf(cos_[d]))) + bf(to_bf(rx * bf(sin_[d]))));
  if (hh < H) {
    q_out[(static_cast<size_t>(b) * H + hh) * D + d] = o;
  } else {
    k_cache[((static_cast<size_t>(b) * storage + pos) * KVH + (hh - H)) * D + d] = o;
  }
}

// out = bf16(bf16(silu(gate)) * up), gate = gu[:, :inter], up = gu[:, inter:];
// silu in float32, x / (1 + exp(-x)), as torch evaluates it for bf16.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ out,
                                                       int rows, int inter) {
  const long long total = static_cast<long long>(rows) * inter;
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const long long r = i / inter;
  const int c = static_cast<int>(i % inter);
  const float g = bf(gu[r * 2 * inter + c]);
  const float u = bf(gu[r * 2 * inter + inter + c]);
  const float s = bf(to_bf(g / (1.0f + expf(-g))));
  out[i] = to_bf(s * u);
}

// ------------------------------------------------------------------ linear
// y[M, N] = bf16(x[M, K] . W[N, K]^T) for the decode step's few rows
// (M <= 8): the weights are read from HBM once, so the product runs at the
// HBM bound, not on matrix cores.  A workgroup of 16 waves per CU stages x
// (zero-padded to MP rows and Kp columns) in LDS once; then each wave streams
// pairs of weight rows, 16 bytes per lane per 512-column segment, four
// segments (a "chunk" of 2048 columns) per row at a time, with two such
// units in flight while one is multiplied (v_dot2 with float32
// accumulation).  At the end of a row pair the wave's M x 2 partial sums are
// reduced across the 64 lanes by halving exchanges, so each output ends in
// one lane.  Rows beyond N and columns beyond K read as zero through the
// buffer descriptors' range checks.
// kLinSwiglu: W holds 2N rows (gate rows, then up rows); the pair of wave
// rows is (n, n + N) and the output is bf16(bf16(silu(g)) * u) with g and u
// rounded to bf16 first, the roundings of silu_mul_kernel after a bf16
// product.
// kLinRope: W is the fused q/k/v projection, N = (H + 2 KVH) D rows, head by
// head; the pair is (d, d + D/2) of one head, the two elements rotate-half
// RoPE combines, and the output goes where rope_write_kernel puts it (q
// rotated to q_out, k rotated and v as is to the caches at pos), in its
// roundings applied to the bf16 products; y is not written.
constexpr int kLinPlain = 0, kLinSwiglu = 1, kLinRope = 2;
struct RopeOut {
  const uint16_t* cos;
  const uint16_t* sin;
  uint16_t* q;
  uint16_t* k;
  uint16_t* v;
  int H, KVH, D, pos;
  long long storage;
};
constexpr int kLinWaves = 16;
constexpr int kLinThreads = kLinWaves * 64;
constexpr int kLinSeg = 512;                // columns per wave-wide 16-byte load
constexpr int kLinChunkSegs = 4;            // segments per row loaded at once
constexpr int kLinChunk = kLinSeg * kLinChunkSegs;
constexpr int kLinLdsVecs = 8192;           // 16-byte LDS slots: MP * Kp <= 65536
constexpr int kBufWord3 = 0x00020000;       // raw buffer descriptor, gfx9 family
constexpr int kBufNontemporal = 2;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Eight bf16 products summed into acc, two per v_dot2 (the whole vector is
// reinterpreted, then split into pairs: a bit cast of one 32-bit component
// of a vector lvalue has been seen to read the first component instead).
__device__ __forceinline__ float dot8(const u32x4 a, const u32x4 b, float acc) {
  const bf16x8 av = __builtin_bit_cast(bf16x8, a), bv = __builtin_bit_cast(bf16x8, b);
  acc = __builtin_amdgcn_fdot2_f32_bf16(av.s01, bv.s01, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(av.s23, bv.s23, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(av.s45, bv.s45, acc, false);
  return __builtin_amdgcn_fdot2_f32_bf16(av.s67, bv.s67, acc, false);
}

template <int J>
__device__ __forceinline__ float fxor(float v, int lane) {
  return __int_as_float(lane_xor<J>(__float_as_int(v), lane));
}

// Sums of V per-lane values over the wave, each ending in its own lanes.
// Halving exchanges at distance D = 32, 16, ...: both lanes of a pair add
// the pair's copies of both halves and keep the half their bit D selects
// (upper for the lane with the bit set), so after log2(V) steps the lane's
// element 0 is index lane >> (6 - log2 V); the remaining distances then sum
// it over the other lanes.  Every index goes through the same tree of
// lanes, so a value's sum does not depend on its index.
template <int V, int D, typename T>
__device__ __forceinline__ void lane_reduce(T& acc, int lane) {
  if constexpr (V > 1) {
    constexpr int H = V / 2;
    const bool hi = (lane & D) != 0;
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const float lo = acc[i] + fxor<D>(acc[i], lane);
      const float up = acc[i + H] + fxor<D>(acc[i + H], lane);
      acc[i] = hi ? up : lo;
    }
    lane_reduce<H, D / 2>(acc, lane);
  } else if constexpr (D >= 1) {
    acc[0] += fxor<D>(acc[0], lane);
    lane_reduce<1, D / 2>(acc, lane);
  }
}

template <int MP, int MODE>
__global__ __launch_bounds__(kLinThreads, 1) void linear_kernel(const uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ W,
                                                                uint16_t* __restrict__ y, int M, int N, int K, int Kp,
                                                                int nbatch, RopeOut ro) {
  __shared__ u32x4 xs[kLinLdsVecs];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kv = Kp / 8;  // LDS slots per x row
  const int nch = Kp / kLinChunk;
  const int stride = gridDim.x * kLinWaves;
  const int rows_total = MODE == kLinSwiglu ? 2 * N : N;
  const int half = ro.D / 2;
  const uint32_t row_bytes = static_cast<uint32_t>(K) * 2u;

  // the wave's batches (row pairs): wave * grid + block, then every stride
  int b = wave * gridDim.x + blockIdx.x;
  auto rows_of = [&](int bb, int& r0, int& r1) {
    if constexpr (MODE == kLinSwiglu) {
      r0 = bb;
      r1 = bb + N;
    } else if constexpr (MODE == kLinRope) {
      const int head = bb / half;
      r0 = head * ro.D + (bb - head * half);
      r1 = r0 + half;
    } else {
      r0 = 2 * bb;
      r1 = 2 * bb + 1;
    }
  };
  // Loads of chunk c of pair bb; a pair past the last (bb >= nbatch) or a
  // row past the weight reads zeros without touching memory, so every unit
  // issues the same number of loads.
  auto issue = [&](int bb, int c, u32x4 (&w0)[kLinChunkSegs], u32x4 (&w1)[kLinChunkSegs]) {
    int r0, r1;
    rows_of(bb, r0, r1);
    const bool ok0 = bb < nbatch && r0 < rows_total, ok1 = bb < nbatch && r1 < rows_total;
    const __amdgpu_buffer_rsrc_t rs0 = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(W) + (ok0 ? static_cast<size_t>(r0) * K : 0), (short)0, ok0 ? (int)row_bytes : 0,
        kBufWord3);
    const __amdgpu_buffer_rsrc_t rs1 = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(W) + (ok1 ? static_cast<size_t>(r1) * K : 0), (short)0, ok1 ? (int)row_bytes : 0,
        kBufWord3);
    const int off = (c * kLinChunk + lane * 8) * 2;
#pragma unroll
    for (int s = 0; s < kLinChunkSegs; ++s) {
      w0[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs0, off + s * kLinSeg * 2, 0,
                                                                              kBufNontemporal));
      w1[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs1, off + s * kLinSeg * 2, 0,
                                                                              kBufNontemporal));
    }
  };

  // (b, c): the unit multiplied next; (ib, ic): the next unit to load
  int c = 0, ib = b, ic = 0;
  auto advance = [&](int& bb, int& cc) {
    if (cc + 1 < nch) {
      ++cc;
    } else {
      cc = 0;
      bb += stride;
    }
  };
  // the wave's first two units of weights go out before x is staged, so the
  // wait for x overlaps their latency
  u32x4 wa[kLinChunkSegs], wb[kLinChunkSegs], wc[kLinChunkSegs], wd[kLinChunkSegs];
  issue(ib, ic, wa, wb);
  advance(ib, ic);
  issue(ib, ic, wc, wd);
  advance(ib, ic);
  for (int i = threadIdx.x; i < MP * kv; i += kLinThreads) {
    const int m = i / kv, j = i - m * kv;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (m < M && j < K / 8) v = *reinterpret_cast<const u32x4*>(x + static_cast<size_t>(m) * K + 8 * j);
    xs[i] = v;
  }
  __syncthreads();

  constexpr int V = 2 * MP;  // partial sums per lane: (m, row of the pair)
  constexpr int LOGV = V == 2 ? 1 : V == 4 ? 2 : V == 8 ? 3 : 4;
  // a vector value, not an array: the exchanges below select between two
  // of its elements, which on an array the compiler may turn into a select
  // of addresses and place the array in LDS
  typedef float accv_t __attribute__((ext_vector_type(V)));
  accv_t acc = {};
  // Multiplies the unit (b, c) held in cur (and at the end of a pair
  // reduces and stores its sums), then loads the unit two ahead into cur;
  // false when no unit is left.  The loop alternates two register
  // sets, so two units are in flight and a load never waits for the
  // registers it fills.
  auto step = [&](u32x4 (&cura)[kLinChunkSegs], u32x4 (&curb)[kLinChunkSegs]) -> bool {
    if (b >= nbatch) return false;
    const u32x4* xc = xs + c * (kLinChunk / 8) + lane;
#pragma unroll
    for (int s = 0; s < kLinChunkSegs; ++s) {
#pragma unroll
      for (int m = 0; m < MP; ++m) {
        const u32x4 xv = xc[m * kv + s * (kLinSeg / 8)];
        acc[2 * m] = dot8(xv, cura[s], acc[2 * m]);
        acc[2 * m + 1] = dot8(xv, curb[s], acc[2 * m + 1]);
      }
    }
    if (c + 1 == nch) {
      lane_reduce<V, 32>(acc, lane);
      const int idx = lane >> (6 - LOGV);
      const int m = idx >> 1;
      const bool lead = (lane & ((64 >> LOGV) - 1)) == 0;
      int r0, r1;
      rows_of(b, r0, r1);
      if constexpr (MODE == kLinSwiglu) {
        const float u = fxor<(64 >> LOGV)>(acc[0], lane);  // the (m, up) sum
        if (lead && (idx & 1) == 0 && m < M) {
          const float g = bf(to_bf(acc[0]));
          const float sg = bf(to_bf(g / (1.0f + expf(-g))));
          y[static_cast<size_t>(m) * N + r0] = to_bf(sg * bf(to_bf(u)));
        }
      } else if constexpr (MODE == kLinRope) {
        const float u = fxor<(64 >> LOGV)>(acc[0], lane);  // the (m, d + D/2) sum
        if (lead && (idx & 1) == 0 && m < M) {
          const int head = r0 / ro.D, d = r0 - head * ro.D;
          const uint16_t x0 = to_bf(acc[0]), x1 = to_bf(u);
          if (head >= ro.H + ro.KVH) {  // v: as is
            uint16_t* dst = ro.v + ((static_cast<size_t>(m) * ro.storage + ro.pos) * ro.KVH + (head - ro.H - ro.KVH)) *
                                       ro.D;
            dst[d] = x0;
            dst[d + half] = x1;
          } else {
            // out = bf16(bf16(x * cos) + bf16(rot(x) * sin)), rot(x) = (-x[D/2:], x[:D/2])
            const float f0 = bf(x0), f1 = bf(x1);
            const uint16_t o0 = to_bf(bf(to_bf(f0 * bf(ro.cos[d]))) + bf(to_bf(-f1 * bf(ro.sin[d]))));
            const uint16_t o1 = to_bf(bf(to_bf(f1 * bf(ro.cos[d + half]))) + bf(to_bf(f0 * bf(ro.sin[d + half]))));
            uint16_t* dst = head < ro.H ? ro.q + (static_cast<size_t>(m) * ro.H + head) * ro.D
                                        : ro.k + ((static_cast<size_t>(m) * ro.storage + ro.pos) * ro.KVH +
                                                  (head - ro.H)) * ro.D;
            dst[d] = o0;
            dst[d + half] = o1;
          }
        }
      } else {
        const int r = (idx & 1) ? r1 : r0;
        if (lead && m < M && r < N) y[static_cast<size_t>(m) * N + r] = to_bf(acc[0]);
      }
      acc = accv_t{};
    }
    issue(ib, ic, cura, curb);
    advance(ib, ic);
    advance(b, c);
    return true;
  };
  while (step(wa, wb) && step(wc, wd)) {
  }
}

// ------------------------------------------------------------------ argmax
// Index of the maximum of each row of x [rows, n] (float32), torch.argmax's
// choice: NaN counts as larger than any number, and among equal values (or
// NaNs) the first index wins.  One 1024-thread workgroup per row; each thread
// scans a strided slice (batches of eight 16-byte loads when the row allows),
// then the waves and the workgroup keep the better (value, index) pair.
constexpr int kArgmaxThreads = 1024;
__device__ __forceinline__ bool argmax_better(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na != nb) return na;
  if (!na && a != b) return a > b;
  return ia < ib;
}
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* __restrict__ x, int n,
                                                                long long* __restrict__ out, int vec) {
  __shared__ float s_v[kArgmaxThreads / 64];
  __shared__ int s_i[kArgmaxThreads / 64];
  const float* xr = x + static_cast<size_t>(blockIdx.x) * n;
  const int tid = static_cast<int>(threadIdx.x);
  float best = -__builtin_inff();
  int bi = 0x7fffffff;
  if (vec) {
    typedef float f32x4v __attribute__((ext_vector_type(4)));
    const f32x4v* xv = reinterpret_cast<const f32x4v*>(xr);
    // eight independent 16-byte loads per thread in flight before any is
    // compared (the pair rule orders by index, so the visiting order is free)
    const int nv = n / 4;
    for (int base = tid; base < nv; base += 8 * kArgmaxThreads) {
      f32x4v v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = base + u * kArgmaxThreads;
        if (i < nv) v[u] = xv[i];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = base + u * kArgmaxThreads;
        if (i < nv) {
#pragma unroll
          for (int k = 0; k < 4; ++k)
            if (argmax_better(v[u][k], 4 * i + k, best, bi)) {
              best = v[u][k];
              bi = 4 * i + k;
            }
        }
      }
    }
    for (int i = (n / 4) * 4 + tid; i < n; i += kArgmaxThreads)
      if (argmax_better(xr[i], i, best, bi)) {
        best = xr[i];
        bi = i;
      }
  } else {
    for (int i = tid; i < n; i += kArgmaxThreads)
      if (argmax_better(xr[i], i, best, bi)) {
        best = xr[i];
        bi = i;
      }
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const float ov = __shfl_xor(best, m, 64);
    const int oi = __shfl_xor(bi, m, 64);
    if (argmax_better(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  if ((tid & 63) == 0) {
    s_v[tid >> 6] = best;
    s_i[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgmaxThreads / 64; ++w)
      if (argmax_better(s_v[w], s_i[w], best, bi)) {
        best = s_v[w];
        bi = s_i[w];
      }
    out[blockIdx.x] = bi;
  }
}

}  // namespace rt
}  // namespace santa

using namespace santa;

extern "C" int santa_rt_add_rms_norm(void* h, const void* a, const void* w, void* x, int rows, int hidden, float eps,
                                     hipStream_t stream) {
  if (!h || !w || !x || rows < 0 || hidden <= 0) return set_error(SANTA_ERR_INVALID, "bad add_rms_norm arguments");
  if (rows == 0) return clear_error();
  const int nv = hidden / 8;
  const bool vec = hidden % 8 == 0 && nv <= 4 * rt::kNormVecThreads &&
                   ((reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(a) |
                     reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x)) % 16) == 0;
  uint16_t* hp = static_cast<uint16_t*>(h);
  const uint16_t* ap = static_cast<const uint16_t*>(a);
  const uint16_t* wp = static_cast<const uint16_t*>(w);
  uint16_t* xp = static_cast<uint16_t*>(x);
  const int add = a ? 1 : 0;
  if (vec && nv <= rt::kNormVecThreads)
    hipLaunchKernelGGL(rt::add_rms_norm_vec_kernel<1>, dim3(rows), dim3(rt::kNormVecThreads), 0, stream, hp, ap, wp,
                       xp, hidden, eps, add);
  else if (vec && nv <= 2 * rt::kNormVecThreads)
    hipLaunchKernelGGL(rt::add_rms_norm_vec_kernel<2>, dim3(rows), dim3(rt::kNormVecThreads), 0, stream, hp, ap, wp,
                       xp, hidden, eps, add);
  else if (vec)
    hipLaunchKernelGGL(rt::add_rms_norm_vec_kernel<4>, dim3(rows), dim3(rt::kNormVecThreads), 0, stream, hp, ap, wp,
                       xp, hidden, eps, add);
  else
    hipLaunchKernelGGL(rt::add_rms_norm_kernel, dim3(rows), dim3(rt::kNormThreads), 0, stream, hp, ap, wp, xp, hidden,
                       eps, add);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "add_rms_norm launch failed: %s", hipGetErrorString(e));
  return clear_error();
}

extern "C" int santa_rt_rope_write(const void* qkv, const void* cos_, const void* sin_, void* q_out, void* k_cache,
                                   void* v_cache, int B, int H, int KVH, int D, long long storage, int pos,
                                   hipStream_t stream) {
  if (!qkv || !cos_ || !sin_ || !q_out || !k_cache || !v_cache || B <= 0 || H <= 0 || KVH <= 0 || D <= 0 ||
      D % 2 != 0 || pos < 0 || pos >= storage)
    return set_error(SANTA_ERR_INVALID, "bad rope_write arguments");
  const long long total = static_cast<long long>(B) * (H + 2 * KVH) * D;
  const unsigned grid = static_cast<unsigned>((total + 255) / 256);
  hipLaunchKernelGGL(rt::rope_write_kernel, dim3(grid), dim3(256), 0, stream, static_cast<const uint16_t*>(qkv),
                     static_cast<const uint16_t*>(cos_), static_cast<const uint16_t*>(sin_),
                     static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                     B, H, KVH, D, storage, pos);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "rope_write launch failed: %s", hipGetErrorString(e));
  return clear_error();
}

namespace {
// The shape checks and launch shared by the santa_rt_linear entry points
// (rows: the weight's row count, N the output width the kernel indexes).
int launch_linear(int mode, const void* x, const void* w, void* y, int M, int N, int K, int rows,
                  const rt::RopeOut& ro, hipStream_t stream) {
  if (!x || !w || M < 1 || M > 8 || N <= 0 || K <= 0 || K % 8 != 0 ||
      (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16 != 0)
    return set_error(SANTA_ERR_INVALID, "bad linear arguments (M in 1..8, K a multiple of 8, x and w 16-byte aligned)");
  const int MP = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  const long long Kp = (static_cast<long long>(K) + rt::kLinChunk - 1) / rt::kLinChunk * rt::kLinChunk;
  if (MP * Kp / 8 > rt::kLinLdsVecs)
    return set_error(SANTA_ERR_INVALID, "linear: M x K too large for the staged rows (M rounded up to 1, 2, 4 or 8, "
                                        "times K rounded up to 2048, at most 65536)");
  if (static_cast<long long>(rows) * K * 2 > 0x7fffffffffffLL) return set_error(SANTA_ERR_INVALID, "linear: weight too large");
  const int nbatch = mode == rt::kLinPlain ? (N + 1) / 2 : mode == rt::kLinSwiglu ? N : N / 2;
  // the CU count of the current device, queried on each call (cheap next to
  // a weight-streaming kernel, and free of shared state between host threads)
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0) cus = c;
  }
  const unsigned grid = static_cast<unsigned>(nbatch < cus ? nbatch : cus);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wp = static_cast<const uint16_t*>(w);
  uint16_t* yp = static_cast<uint16_t*>(y);
  const int kp = static_cast<int>(Kp);
#define SANTA_LIN(MPV)                                                                                            \
  if (mode == rt::kLinSwiglu)                                                                                     \
    hipLaunchKernelGGL((rt::linear_kernel<MPV, rt::kLinSwiglu>), dim3(grid), dim3(rt::kLinThreads), 0, stream, xp, \
                       wp, yp, M, N, K, kp, nbatch, ro);                                                          \
  else if (mode == rt::kLinRope)                                                                                  \
    hipLaunchKernelGGL((rt::linear_kernel<MPV, rt::kLinRope>), dim3(grid), dim3(rt::kLinThreads), 0, stream, xp,   \
                       wp, yp, M, N, K, kp, nbatch, ro);                                                          \
  else                                                                                                            \
    hipLaunchKernelGGL((rt::linear_kernel<MPV, rt::kLinPlain>), dim3(grid), dim3(rt::kLinThreads), 0, stream, xp,  \
                       wp, yp, M, N, K, kp, nbatch, ro);
  switch (MP) {
    case 1: SANTA_LIN(1) break;
    case 2: SANTA_LIN(2) break;
    case 4: SANTA_LIN(4) break;
    default: SANTA_LIN(8) break;
  }
#undef SANTA_LIN
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "linear launch failed: %s", hipGetErrorString(e));
  return clear_error();
}
}  // namespace

extern "C" int santa_rt_linear(const void* x, const void* w, void* y, int M, int N, int K, int swiglu,
                               hipStream_t stream) {
  if (!y) return set_error(SANTA_ERR_INVALID, "bad linear arguments (null output)");
  const rt::RopeOut none{nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, 2, 0, 0};
  return launch_linear(swiglu ? rt::kLinSwiglu : rt::kLinPlain, x, w, y, M, N, K, swiglu ? 2 * N : N, none, stream);
}

extern "C" int santa_rt_linear_rope(const void* x, const void* w, int M, int K, const void* cos_, const void* sin_,
                                    void* q_out, void* k_cache, void* v_cache, int H, int KVH, int D,
                                    long long storage, int pos, hipStream_t stream) {
  if (!cos_ || !sin_ || !q_out || !k_cache || !v_cache || H <= 0 || KVH <= 0 || D <= 0 || D % 2 != 0 || pos < 0 ||
      pos >= storage)
    return set_error(SANTA_ERR_INVALID, "bad linear_rope arguments");
  const long long n = static_cast<long long>(H + 2 * KVH) * D;
  if (n > 0x7fffffff) return set_error(SANTA_ERR_INVALID, "linear_rope: projection too wide");
  const rt::RopeOut ro{static_cast<const uint16_t*>(cos_), static_cast<const uint16_t*>(sin_),
                       static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                       H, KVH, D, pos, storage};
  return launch_linear(rt::kLinRope, x, w, q_out, M, static_cast<int>(n), K, static_cast<int>(n), ro, stream);
}

extern "C" int santa_rt_argmax(const float* x, int rows, int n, long long* out, hipStream_t stream) {
  if (!x || !out || rows < 0 || n <= 0) return set_error(SANTA_ERR_INVALID, "bad argmax arguments");
  if (rows == 0) return clear_error();
  const int vec = (n % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0) ? 1 : 0;
  hipLaunchKernelGGL(rt::argmax_kernel, dim3(rows), dim3(rt::kArgmaxThreads), 0, stream, x, n, out, vec);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "argmax launch failed: %s", hipGetErrorString(e));
  return clear_error();
}

extern "C" int santa_rt_silu_mul(const void* gu, void* out, int rows, int inter, hipStream_t stream) {
  if (!gu || !out || rows < 0 || inter <= 0) return set_error(SANTA_ERR_INVALID, "bad silu_mul arguments");
  if (rows == 0) return clear_error();
  const long long total = static_cast<long long>(rows) * inter;
  const unsigned grid = static_cast<unsigned>((total + 255) / 256);
  hipLaunchKernelGGL(rt::silu_mul_kernel, dim3(grid), dim3(256), 0, stream, static_cast<const uint16_t*>(gu),
                     static_cast<uint16_t*>(out), rows, inter);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SANTA_ERR_HIP, "silu_mul launch failed: %s", hipGetErrorString(e));
  return clear_error();
}
