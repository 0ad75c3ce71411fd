/*
 * santa_oracle.c -- CPU restatement of the S^2ANTA sampled-attention decode
 * algorithm (santa_flash fixed tile budget, santa_prop proportional budget).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (santa_amd/, the C-ABI
 * library, the torch extension modules) links, imports or calls this file.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * and only as the checker / the timed CPU baseline.
 *
 * Arithmetic rules: IEEE-754 binary32, round-to-nearest-even, no contraction
 * (built with -ffp-contract=off); every fused multiply-add is an explicit
 * fmaf().  EXP is this project's own exponential (so_expf below), because the
 * reference's __expf and fast-math division are NVIDIA math that is neither
 * reproducible nor to be reproduced.  Everything else follows the reference's
 * association order, thread by thread, as cited per function.
 *
 * Citations are path:line in the upstream reference tree, with
 *   flash/ = flash_style_fused_santa_fixed_tile_budgets/
 *   prop/  = santa_fused_proportional_tile_budgets/
 *
 * Parity pins (see tests/test_oracle.py):
 *   so_splitmix64 / so_u01 : SplitMix64 known-answer vector + u01 anchors.
 *   so_expf                : <= 2 ulp against libm expf, exp(0) == 1 exactly.
 *   conversions            : exhaustive against numpy's bf16/f16 casts.
 *   flash / prop tiles     : closed forms (uniform tile -> rows 75 and 203),
 *                            invariants (sum of counts, floor/ceil bounds),
 *                            brute-force float64 scores, torch SDPA limit.
 *   bitonic budgets        : invariants (sum S_t == S, floor/ceil bounds) and
 *                            an independent Python model of the network.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define SO_D 128      /* flash: the reference's only head_dim */
#define SO_MAX_D 1024  /* prop: any multiple of 16 up to this */
#define SO_MAX_GH 16
#define SO_MAX_BN 512
#define SO_LANES 32

/* ------------------------------------------------------------------ */
/* bit helpers and 16-bit conversions                                  */
/* flash/santa_cuda_kernel.cu:33-55 (bf16 -> f32 by <<16; RNE back)    */
/* ------------------------------------------------------------------ */
static inline float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t bits_from_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float so_bf16_to_f32(uint16_t h) { return f32_from_bits((uint32_t)h << 16); }

uint16_t so_f32_to_bf16(float f) {
  uint32_t u = bits_from_f32(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float so_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t m = (uint32_t)h & 0x3ffu;
  if (e == 0) {
    float f = (float)m * 0x1p-24f; /* exact: m < 2^10 */
    return sign ? -f : f;
  }
  if (e == 31) return f32_from_bits(sign | 0x7f800000u | (m << 13));
  return f32_from_bits(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t so_f32_to_f16(float f) {
  uint32_t x = bits_from_f32(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x0200u : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (ax < 0x38800000u) {
    float scaled = f32_from_bits(ax) * 0x1p24f; /* exact power-of-two scaling */
    uint32_t m = (uint32_t)rintf(scaled);       /* RNE to the f16 subnormal grid */
    return (uint16_t)(sign | m);
  }
  uint32_t r = ax + 0x0fffu + ((ax >> 13) & 1u);
  return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
}

static inline float ld16(const uint16_t* p, size_t i, int is_bf16) {
  return is_bf16 ? so_bf16_to_f32(p[i]) : so_f16_to_f32(p[i]);
}
static inline uint16_t st16(float f, int is_bf16) {
  return is_bf16 ? so_f32_to_bf16(f) : so_f32_to_f16(f);
}

/* ------------------------------------------------------------------ */
/* RNG: flash/santa_cuda_kernel.cu:74-87 (dup prop/...kernel.cu:557-570) */
/* ------------------------------------------------------------------ */
uint64_t so_splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ULL;
  uint64_t z = x;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

float so_u01(uint64_t seed, int key, int t) {
  uint64_t x = seed ^ (((uint64_t)(int64_t)key << 32) ^ (uint64_t)(int64_t)t);
  uint64_t r = so_splitmix64(x);
  double u = (double)(r >> 11) * (1.0 / 9007199254740992.0);
  return (float)u;
}

/* ------------------------------------------------------------------ */
/* EXP: this project's own binary32 exponential.                        */
/* Cody-Waite reduction x = n*ln2 + r with ln2 split hi/lo (hi has 15    */
/* significant bits, so n*hi is exact for |n| <= 256), degree-7 Taylor   */
/* polynomial in Horner form with explicit fma, and scaling by 2^n in    */
/* two exact power-of-two multiplies so that subnormal results round     */
/* once.  exp(0) == 1 exactly.  Stands in for the reference's __expf at  */
/* flash/santa_cuda_kernel.cu:249,436 and prop/...kernel.cu:238,411,641. */
/* ------------------------------------------------------------------ */
float so_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -103.97208404541015625f) return 0.0f;
  const float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(n, -0.693145751953125f, x);
  r = fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.984126984126984e-4f;
  p = fmaf(p, r, 1.3888888888888889e-3f);
  p = fmaf(p, r, 8.3333333333333333e-3f);
  p = fmaf(p, r, 4.1666666666666667e-2f);
  p = fmaf(p, r, 1.6666666666666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const int n1 = ni / 2;
  const int n2 = ni - n1;
  const float s1 = f32_from_bits((uint32_t)(n1 + 127) << 23);
  const float s2 = f32_from_bits((uint32_t)(n2 + 127) << 23);
  return (p * s1) * s2;
}

/* ------------------------------------------------------------------ */
/* 32-lane primitives, simulated lane by lane                           */
/* ------------------------------------------------------------------ */

/* __shfl_down_sync tree: v[l] += v[l+off] (own value if l+off >= 32),
 * off = 16,8,4,2,1; returns lane 0.  flash/santa_cuda_kernel.cu:205-211,256-260. */
static float lane_tree_down(const float* in) {
  float v[SO_LANES], t[SO_LANES];
  memcpy(v, in, sizeof(v));
  for (int off = 16; off > 0; off >>= 1) {
    for (int l = 0; l < SO_LANES; ++l) t[l] = v[l] + ((l + off < SO_LANES) ? v[l + off] : v[l]);
    memcpy(v, t, sizeof(v));
  }
  return v[0];
}

/* The shfl_down tree over P lanes (P <= SO_MAX_D / 4): at offsets N/2, N/4,
 * ..., 1 (N the next power of two >= P) lane l < offset adds lane l + offset
 * when that lane holds a value; lanes from P on hold none.  For P = 32 this is
 * lane_tree_down. */
static float lane_tree_down_p(const float* in, int P) {
  float v[SO_MAX_D / 4];
  memcpy(v, in, (size_t)P * sizeof(float));
  int N = 1;
  while (N < P) N <<= 1;
  int n = P; /* lanes 0 .. n-1 hold values */
  for (int off = N / 2; off > 0; off >>= 1) {
    for (int l = 0; l < off; ++l)
      if (l + off < n) v[l] = v[l] + v[l + off];
    if (n > off) n = off;
  }
  return v[0];
}

/* warp_exclusive_scan_sum: Hillis-Steele with simultaneous update, then
 * res - v.  flash/santa_cuda_kernel.cu:60-69. */
static void lane_scan_excl(const float* x, float* pre) {
  float res[SO_LANES], t[SO_LANES];
  memcpy(res, x, sizeof(res));
  for (int off = 1; off < SO_LANES; off <<= 1) {
    for (int l = 0; l < SO_LANES; ++l) t[l] = (l >= off) ? (res[l] + res[l - off]) : res[l];
    memcpy(res, t, sizeof(res));
  }
  for (int l = 0; l < SO_LANES; ++l) pre[l] = res[l] - x[l];
}

/* ------------------------------------------------------------------ */
/* Host planning: flash/santa_cuda.cpp:36-44,197-210                    */
/* ------------------------------------------------------------------ */
int so_auto_block_n(int L) {
  if (L <= 1536) return 32;
  if (L <= 3072) return 64;
  return 256;
}

int so_flash_s_per_tile(int64_t S, int T_c) {
  if (S <= 0) return 0;
  int s = (int)(S / T_c);
  return s < 1 ? 1 : s;
}

float so_q_scale(int D) { return 1.0f / sqrtf((float)D); }

/* ------------------------------------------------------------------ */
/* Tile statistics shared by flash K1 and prop vec pass-1.              */
/* scores: flash/santa_cuda_kernel.cu:161-221 (prop/...:314-379)        */
/* max   : :223-241 ; u, ell, u16 : :243-273 (prop/...:403-440)          */
/* NT = threads of the reference block (256 for BN=256, else 128),      */
/* which fixes the association of ell.                                   */
/* ------------------------------------------------------------------ */
typedef struct {
  int len;
  float m[SO_MAX_GH];
  float ell[SO_MAX_GH];
  uint16_t ub[SO_MAX_BN * SO_MAX_GH]; /* [r*GH + g] */
} tile_stats_t;

static void tile_stats_vec(const float* qf /*[GH][128] scaled*/, const uint16_t* K, size_t row0_off,
                           size_t row_stride, int len, int GH, int NT, int is_bf16, tile_stats_t* ts,
                           float* scores /*[BN*GH] scratch*/) {
  ts->len = len;
  for (int g = 0; g < GH; ++g) ts->m[g] = -INFINITY;
  for (int r = 0; r < len; ++r) {
    const uint16_t* krow = K + row0_off + (size_t)r * row_stride;
    float kf[SO_D];
    for (int d = 0; d < SO_D; ++d) kf[d] = ld16(krow, (size_t)d, is_bf16);
    for (int g = 0; g < GH; ++g) {
      const float* q = qf + (size_t)g * SO_D;
      float lanes[SO_LANES];
      for (int l = 0; l < SO_LANES; ++l) {
        float s = 0.0f;
        s = fmaf(q[4 * l + 0], kf[4 * l + 0], s);
        s = fmaf(q[4 * l + 1], kf[4 * l + 1], s);
        s = fmaf(q[4 * l + 2], kf[4 * l + 2], s);
        s = fmaf(q[4 * l + 3], kf[4 * l + 3], s);
        lanes[l] = s;
      }
      const float s = lane_tree_down(lanes);
      scores[r * GH + g] = s;
      ts->m[g] = fmaxf(ts->m[g], s);
    }
  }
  /* u = EXP(s - m), ell partials per reference thread, then 32-lane trees,
   * then a sequential sum over warps. */
  const int NW = NT / 32;
  float W[SO_MAX_GH][32];
  for (int w = 0; w < NW; ++w) {
    float lanes[SO_MAX_GH][SO_LANES];
    for (int lane = 0; lane < SO_LANES; ++lane) {
      const int tid = w * 32 + lane;
      float acc[SO_MAX_GH];
      for (int g = 0; g < GH; ++g) acc[g] = 0.0f;
      for (int idx = tid; idx < len * GH; idx += NT) {
        const int r = idx / GH;
        const int g = idx - r * GH;
        const float u = so_expf(scores[r * GH + g] - ts->m[g]);
        acc[g] += u;
        ts->ub[r * GH + g] = st16(u, is_bf16);
      }
      for (int g = 0; g < GH; ++g) lanes[g][lane] = acc[g];
    }
    for (int g = 0; g < GH; ++g) W[g][w] = lane_tree_down(lanes[g]);
  }
  for (int g = 0; g < GH; ++g) {
    float ell = 0.0f;
    for (int w = 0; w < NW; ++w) ell += W[g][w];
    ts->ell[g] = ell;
  }
}

/* Systematic counts for one head of one tile:
 * flash/santa_cuda_kernel.cu:275-311 (prop/...kernel.cu:771-807).
 * x_r = f32(u16[r]) * invdel; 32-lane scan with carry; floor differences. */
static void tile_counts(const uint16_t* ub, int ub_stride, int len, float invdel, float a0, int is_bf16,
                        int16_t* c_out) {
  float carry = 0.0f;
  for (int base = 0; base < len; base += 32) {
    float x[SO_LANES], pre[SO_LANES];
    for (int l = 0; l < SO_LANES; ++l) {
      const int r = base + l;
      x[l] = (r < len && invdel > 0.0f) ? ld16(ub, (size_t)r * (size_t)ub_stride, is_bf16) * invdel : 0.0f;
    }
    lane_scan_excl(x, pre);
    for (int l = 0; l < SO_LANES; ++l) {
      const int r = base + l;
      if (r >= len) continue;
      const float pre_g = carry + pre[l];
      const float cum_g = pre_g + x[l];
      const float f_prev = floorf(a0 + pre_g);
      const float f_curr = floorf(a0 + cum_g);
      const float diff = f_curr - f_prev;
      int c = (diff != diff) ? 0 : (diff >= 2147483648.0f ? 2147483647 : (diff < -2147483648.0f ? (-2147483647 - 1) : (int)diff));
      c = c < 0 ? 0 : c;
      c = c > 32767 ? 32767 : c;
      c_out[r] = (int16_t)c;
    }
    const int remain = len - base;
    const int last = (remain > 0) ? (remain - 1 < 31 ? remain - 1 : 31) : 0;
    const float chunk_total = pre[last] + x[last];
    carry = carry + chunk_total;
  }
}

/* Emission list: rows with any count across the group, ascending.
 * flash/santa_cuda_kernel.cu:314-345. */
static int tile_emit(const int16_t* c /*[GH][BN]*/, int BN, int GH, int len, int* emit) {
  int ne = 0;
  for (int r = 0; r < len; ++r) {
    int sum = 0;
    for (int g = 0; g < GH; ++g) sum += (int)c[(size_t)g * BN + r];
    if (sum > 0) emit[ne++] = r;
  }
  return ne;
}

/* Count-weighted V sum for one head, ascending emitted rows, skipping
 * zero counts, one fma per element.  flash/santa_cuda_kernel.cu:347-379
 * (prop/...kernel.cu:843-857 with its a*b+c contracted to fma). */
static void tile_pv(const int16_t* c_g, const int* emit, int ne, const uint16_t* V, size_t v_row0,
                    size_t row_stride, int D, int is_bf16, float* acc /*[D]*/) {
  for (int d = 0; d < D; ++d) acc[d] = 0.0f;
  for (int i = 0; i < ne; ++i) {
    const int r = emit[i];
    const int cc = (int)c_g[r];
    if (cc == 0) continue;
    const float cf = (float)cc;
    const uint16_t* vrow = V + v_row0 + (size_t)r * row_stride;
    for (int d = 0; d < D; ++d) acc[d] = fmaf(cf, ld16(vrow, (size_t)d, is_bf16), acc[d]);
  }
}

/* ------------------------------------------------------------------ */
/* santa_flash: fused tile (K1) for every (b, kv, t), then the split-KV */
/* merge (K2) with the reference's association.                          */
/* flash/santa_cuda.cpp:174-343, flash/santa_cuda_kernel.cu:96-470       */
/*                                                                      */
/* Layouts (contiguous): q [B,H,128]; K,V [B,L_storage,KVH,128].          */
/* Optional outputs (NULL to skip):                                      */
/*   m_tiles, ell_tiles [B,H,T_c]; counts [B,H,T_c*BN] int16;            */
/*   out_tiles [B,H,T_c,128]; rowmask [B,KVH,L_valid] int32.             */
/* ------------------------------------------------------------------ */
/* b_offset: sequence b of these inputs is sequence b + b_offset of the     */
/* batch, so its RNG key is (b + b_offset) * H + h (flash/santa_cuda_       */
/* kernel.cu:281) -- one sequence of a ragged batch decoded on its own.    */
int so_flash_decode_at(const uint16_t* Q, const uint16_t* K, const uint16_t* V, int is_bf16, int B, int H,
                       int KVH, int L_valid, int L_storage, int BN, int S_pt, uint64_t seed, float* out_f32,
                       uint16_t* out16, float* m_star, float* m_tiles_o, float* ell_tiles_o, int16_t* counts_o,
                       float* out_tiles_o, int* rowmask, int nthreads, int b_offset) {
  if (KVH <= 0 || H % KVH != 0) return -1;
  const int GH = H / KVH;
  if (GH > SO_MAX_GH || BN > SO_MAX_BN || (BN != 32 && BN != 64 && BN != 256)) return -2;
  if (L_valid < 0 || L_valid > L_storage) return -3;
  const int T_c = (L_valid + BN - 1) / BN;
  const int NT = (BN == 256) ? 256 : 128;
  const float q_scale = so_q_scale(SO_D);
  const size_t row_stride = (size_t)KVH * SO_D;

  float* m_tiles = (float*)malloc(sizeof(float) * (size_t)B * H * (T_c > 0 ? T_c : 1));
  float* ell_tiles = (float*)malloc(sizeof(float) * (size_t)B * H * (T_c > 0 ? T_c : 1));
  float* out_tiles = (float*)malloc(sizeof(float) * (size_t)B * H * (T_c > 0 ? T_c : 1) * SO_D);
  if (!m_tiles || !ell_tiles || !out_tiles) { free(m_tiles); free(ell_tiles); free(out_tiles); return -4; }

  const long n_items = (long)B * KVH * T_c;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 4)
#endif
  for (long it = 0; it < n_items; ++it) {
    const int t = (int)(it % T_c);
    const int kv = (int)((it / T_c) % KVH);
    const int b = (int)(it / ((long)T_c * KVH));
    const int h0 = kv * GH;
    const int n0 = t * BN;
    const int n1 = (n0 + BN < L_valid) ? n0 + BN : L_valid;
    const int len = n1 - n0;

    float qf[SO_MAX_GH * SO_D];
    for (int g = 0; g < GH; ++g)
      for (int d = 0; d < SO_D; ++d)
        qf[g * SO_D + d] = ld16(Q, ((size_t)b * H + h0 + g) * SO_D + d, is_bf16) * q_scale;

    tile_stats_t ts;
    float scores[SO_MAX_BN * SO_MAX_GH];
    const size_t row0 = ((size_t)b * L_storage + n0) * row_stride + (size_t)kv * SO_D;
    tile_stats_vec(qf, K, row0, row_stride, len, GH, NT, is_bf16, &ts, scores);

    int16_t c[SO_MAX_GH * SO_MAX_BN];
    memset(c, 0, sizeof(c));
    for (int g = 0; g < GH; ++g) {
      const float ell = ts.ell[g];
      const float invdel = (S_pt > 0 && ell > 1e-20f) ? ((float)S_pt / ell) : 0.0f;
      const float a0 = so_u01(seed, (b + b_offset) * H + h0 + g, t);
      tile_counts(ts.ub + g, GH, len, invdel, a0, is_bf16, c + (size_t)g * BN);
    }
    int emit[SO_MAX_BN];
    const int ne = tile_emit(c, BN, GH, len, emit);
    if (rowmask)
      for (int i = 0; i < ne; ++i) rowmask[((size_t)b * KVH + kv) * L_valid + n0 + emit[i]] = 1;

    for (int g = 0; g < GH; ++g) {
      const int h = h0 + g;
      const size_t mt = ((size_t)b * H + h) * T_c + t;
      float* acc = out_tiles + mt * SO_D;
      if (len <= 0) {
        m_tiles[mt] = -INFINITY;
        ell_tiles[mt] = 0.0f;
        for (int d = 0; d < SO_D; ++d) acc[d] = 0.0f;
      } else {
        m_tiles[mt] = ts.m[g];
        ell_tiles[mt] = ts.ell[g];
        tile_pv(c + (size_t)g * BN, emit, ne, V, row0, row_stride, SO_D, is_bf16, acc);
      }
      if (counts_o) {
        int16_t* dst = counts_o + (((size_t)b * H + h) * T_c + t) * BN;
        for (int r = 0; r < BN; ++r) dst[r] = (r < len) ? c[(size_t)g * BN + r] : 0;
      }
    }
  }

  /* K2: flash/santa_cuda_kernel.cu:386-470, TPB = 256 (launcher :637). */
  const int TPB = 256;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (long bh = 0; bh < (long)B * H; ++bh) {
    const float* mt = m_tiles + (size_t)bh * T_c;
    const float* lt = ell_tiles + (size_t)bh * T_c;
    float red[256];
    for (int tid = 0; tid < TPB; ++tid) {
      float lm = -INFINITY;
      for (int t = tid; t < T_c; t += TPB) lm = fmaxf(lm, mt[t]);
      red[tid] = lm;
    }
    for (int s = TPB >> 1; s > 32; s >>= 1)
      for (int tid = 0; tid < s; ++tid) red[tid] = fmaxf(red[tid], red[tid + s]);
    for (int off = 32; off > 0; off >>= 1)
      for (int tid = 0; tid < off; ++tid) red[tid] = fmaxf(red[tid], red[tid + off]);
    const float ms = red[0];
    if (m_star) m_star[bh] = ms;

    float* w = (float*)malloc(sizeof(float) * (T_c > 0 ? T_c : 1));
    for (int tid = 0; tid < TPB; ++tid) {
      float z = 0.0f;
      for (int t = tid; t < T_c; t += TPB) {
        const float wt = so_expf(mt[t] - ms) * lt[t];
        w[t] = wt;
        z += wt;
      }
      red[tid] = z;
    }
    for (int s = TPB >> 1; s > 32; s >>= 1)
      for (int tid = 0; tid < s; ++tid) red[tid] = red[tid] + red[tid + s];
    for (int off = 32; off > 0; off >>= 1) {
      float nv[32];
      for (int tid = 0; tid < 32; ++tid) nv[tid] = red[tid] + red[tid + off];
      for (int tid = 0; tid < 32; ++tid) red[tid] = nv[tid];
    }
    const float Z = red[0];
    const float inv_norm = (S_pt > 0 && Z > 0.0f) ? (1.0f / (Z * (float)S_pt)) : 0.0f;
    for (int d = 0; d < SO_D; ++d) {
      float num = 0.0f;
      for (int t = 0; t < T_c; ++t) num = fmaf(w[t], out_tiles[((size_t)bh * T_c + t) * SO_D + d], num);
      const float y = num * inv_norm;
      if (out_f32) out_f32[(size_t)bh * SO_D + d] = y;
      if (out16) out16[(size_t)bh * SO_D + d] = st16(y, is_bf16);
    }
    free(w);
  }

  if (m_tiles_o) memcpy(m_tiles_o, m_tiles, sizeof(float) * (size_t)B * H * T_c);
  if (ell_tiles_o) memcpy(ell_tiles_o, ell_tiles, sizeof(float) * (size_t)B * H * T_c);
  if (out_tiles_o) memcpy(out_tiles_o, out_tiles, sizeof(float) * (size_t)B * H * T_c * SO_D);
  free(m_tiles);
  free(ell_tiles);
  free(out_tiles);
  return 0;
}

int so_flash_decode(const uint16_t* Q, const uint16_t* K, const uint16_t* V, int is_bf16, int B, int H,
                    int KVH, int L_valid, int L_storage, int BN, int S_pt, uint64_t seed, float* out_f32,
                    uint16_t* out16, float* m_star, float* m_tiles_o, float* ell_tiles_o, int16_t* counts_o,
                    float* out_tiles_o, int* rowmask, int nthreads) {
  return so_flash_decode_at(Q, K, V, is_bf16, B, H, KVH, L_valid, L_storage, BN, S_pt, seed, out_f32, out16,
                            m_star, m_tiles_o, ell_tiles_o, counts_o, out_tiles_o, rowmask, nthreads, 0);
}

/* ------------------------------------------------------------------ */
/* santa_prop                                                           */
/* ------------------------------------------------------------------ */

/* Pass-1 of the general ("WMMA") path, prop/santa_cuda_kernel.cu:87-267:
 * q' = TK(f32(q) * scale) (:121-140).  The reference's scores come from a
 * 16x16x16 MMA whose internal association is unspecified; this build fixes
 * it for every D (a multiple of 16) to the vec path's form extended to D
 * dims: virtual lane v chains dims 4v .. 4v+3 with fma, then the shfl_down
 * tree over the D/4 virtual lanes (lane_tree_down_p); for D = 128 that is
 * exactly the vec path's 32-lane association (A.2).  The GPU kernels and
 * this restatement agree bit for bit.  ell: per 16-row slab a sequential sum
 * (:229-246), then a sequential sum over slabs (:257-259). */
static void tile_stats_general(const uint16_t* Qh /*[GH][D] raw*/, const uint16_t* K, size_t row0_off,
                               size_t row_stride, int len, int BN, int GH, int D, int is_bf16, float q_scale,
                               tile_stats_t* ts, float* scores) {
  ts->len = len;
  float qr[SO_MAX_GH * SO_MAX_D];
  for (int g = 0; g < GH; ++g)
    for (int d = 0; d < D; ++d) {
      const float qv = ld16(Qh, (size_t)g * D + d, is_bf16) * q_scale;
      const uint16_t qb = st16(qv, is_bf16);
      qr[g * D + d] = ld16(&qb, 0, is_bf16);
    }
  for (int g = 0; g < GH; ++g) ts->m[g] = -INFINITY;
  for (int r = 0; r < len; ++r) {
    const uint16_t* krow = K + row0_off + (size_t)r * row_stride;
    float kf[SO_MAX_D];
    for (int d = 0; d < D; ++d) kf[d] = ld16(krow, (size_t)d, is_bf16);
    for (int g = 0; g < GH; ++g) {
      const float* q = qr + (size_t)g * D;
      float lanes[SO_MAX_D / 4];
      for (int l = 0; l < D / 4; ++l) {
        float sl = 0.0f;
        sl = fmaf(q[4 * l + 0], kf[4 * l + 0], sl);
        sl = fmaf(q[4 * l + 1], kf[4 * l + 1], sl);
        sl = fmaf(q[4 * l + 2], kf[4 * l + 2], sl);
        sl = fmaf(q[4 * l + 3], kf[4 * l + 3], sl);
        lanes[l] = sl;
      }
      const float sf = lane_tree_down_p(lanes, D / 4);
      scores[r * GH + g] = sf;
      ts->m[g] = fmaxf(ts->m[g], sf);
    }
  }
  const int NW = BN / 16;
  for (int g = 0; g < GH; ++g) {
    float ell = 0.0f;
    for (int w = 0; w < NW; ++w) {
      float part = 0.0f;
      for (int j = 0; j < 16; ++j) {
        const int r = w * 16 + j;
        if (r < len) {
          const float u = so_expf(scores[r * GH + g] - ts->m[g]);
          part += u;
          ts->ub[r * GH + g] = st16(u, is_bf16);
        }
      }
      ell += part;
    }
    ts->ell[g] = ell;
  }
}

/* Largest-remainder tile budgets, prop/santa_cuda_kernel.cu:577-726.
 * The reference sums Z with shared-memory float atomics (order undefined,
 * :637-645); this restatement fixes the order the HIP kernel uses:
 * 128 per-thread partials (t = tid, tid+128, ... in ascending order),
 * then a pairwise tree red[i] += red[i+s] for s = 64, 32, ..., 1.
 * The bitonic network keeps the reference's padding semantics: reads past
 * T_c see (-inf, -1) and writes past T_c are dropped (:689-703). */
void so_prop_budgets(const float* m_tiles, const float* ell_tiles, int T_c, int S, uint64_t seed, int h,
                     float* m_star, int* S_tiles, float* invdelta, float* a0) {
  float ms = -3.402823466e+38f;
  for (int t = 0; t < T_c; ++t) ms = fmaxf(ms, m_tiles[t]);
  if (m_star) *m_star = ms;
  float* W = (float*)malloc(sizeof(float) * (T_c > 0 ? T_c : 1));
  float red[128];
  for (int tid = 0; tid < 128; ++tid) {
    float z = 0.0f;
    for (int t = tid; t < T_c; t += 128) {
      const float wt = so_expf(m_tiles[t] - ms) * ell_tiles[t];
      W[t] = wt;
      z += wt;
    }
    red[tid] = z;
  }
  for (int s = 64; s > 0; s >>= 1)
    for (int tid = 0; tid < s; ++tid) red[tid] = red[tid] + red[tid + s];
  const float Z = red[0];
  if (S <= 0 || !(Z > 0.0f)) {
    for (int t = 0; t < T_c; ++t) {
      S_tiles[t] = 0;
      invdelta[t] = 0.0f;
      a0[t] = so_u01(seed, h, t);
    }
    free(W);
    return;
  }
  float* frac = (float*)malloc(sizeof(float) * (T_c > 0 ? T_c : 1));
  int* idx = (int*)malloc(sizeof(int) * (T_c > 0 ? T_c : 1));
  long sum_base = 0;
  for (int t = 0; t < T_c; ++t) {
    const float q = (float)S * (W[t] / Z);
    const float fq = floorf(q);
    const int bt = (fq != fq) ? 0 : (fq >= 2147483648.0f ? 2147483647 : (int)fq);
    S_tiles[t] = bt;
    sum_base += bt;
    const float ft = q - (float)bt;
    const float jitter = 1.0e-7f * so_u01(seed, h, t);
    frac[t] = ft + jitter;
    idx[t] = t;
  }
  long rem = (long)S - sum_base;
  if (rem < 0) rem = 0;
  if (rem > T_c) rem = T_c;
  int N = 1;
  while (N < T_c) N <<= 1;
  for (int k = 2; k <= N; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = 0; i < N; ++i) {
        const int ixj = i ^ j;
        if (ixj <= i) continue;
        const int up = ((i & k) != 0);
        float ai = (i < T_c) ? frac[i] : -INFINITY;
        float aj = (ixj < T_c) ? frac[ixj] : -INFINITY;
        int ii = (i < T_c) ? idx[i] : -1;
        int ij = (ixj < T_c) ? idx[ixj] : -1;
        if ((ai > aj) == up) {
          const float tf = ai; ai = aj; aj = tf;
          const int ti = ii; ii = ij; ij = ti;
        }
        if (i < T_c) { frac[i] = ai; idx[i] = ii; }
        if (ixj < T_c) { frac[ixj] = aj; idx[ixj] = ij; }
      }
    }
  }
  for (long r = 0; r < rem; ++r) {
    const int best = (r < T_c) ? idx[r] : -1;
    if (best >= 0) S_tiles[best] += 1;
  }
  for (int t = 0; t < T_c; ++t) {
    const float ell = ell_tiles[t];
    const int St = S_tiles[t];
    invdelta[t] = (St > 0 && ell > 1e-20f) ? ((float)St / ell) : 0.0f;
    a0[t] = so_u01(seed, h, t);
  }
  free(W);
  free(frac);
  free(idx);
}

/* santa_prop decode for one sequence: prop/santa_cuda.cpp:270-352.
 * pass1_mode: 0 = vec path (GH=4, D=128, BN=256),
 *             1 = general path (q rounded to the storage dtype after scaling,
 *                 per-slab ell; see tile_stats_general).
 * D: a multiple of 16 up to 256; BN: a multiple of 16 up to 512; GH <= 16.
 * Layouts: q [H,D]; K,V [L,KVH,D]. Optional outputs may be NULL:
 *   m_tiles, ell_tiles, invdelta, a0 [H,T_c]; S_tiles [H,T_c] int32;
 *   u_stash [L,H] 16-bit; counts [H,T_c*BN] int16; rowmask [KVH,L]. */
int so_prop_decode_d(const uint16_t* Q, const uint16_t* K, const uint16_t* V, int is_bf16, int H, int KVH, int D,
                     int L, int BN, int S, uint64_t seed, int pass1_mode, float* out_f32, uint16_t* out16,
                     float* m_star, float* m_tiles_o, float* ell_tiles_o, int* S_tiles_o, float* invdelta_o,
                     float* a0_o, uint16_t* u_stash_o, int16_t* counts_o, int* rowmask) {
  if (KVH <= 0 || H % KVH != 0) return -1;
  const int GH = H / KVH;
  if (GH > SO_MAX_GH || BN > SO_MAX_BN || BN <= 0 || (BN % 16) != 0) return -2;
  if (D <= 0 || D > SO_MAX_D || (D % 16) != 0) return -6;
  if (pass1_mode == 0 && !(GH == 4 && BN == 256 && D == SO_D)) return -5;
  const int T_c = (L + BN - 1) / BN;
  const size_t TT = (size_t)(T_c > 0 ? T_c : 1);
  const float q_scale = so_q_scale(D);
  const size_t row_stride = (size_t)KVH * D;

  float* m_tiles = (float*)calloc((size_t)H * TT, sizeof(float));
  float* ell_tiles = (float*)calloc((size_t)H * TT, sizeof(float));
  uint16_t* u_stash = (uint16_t*)calloc((size_t)(L > 0 ? L : 1) * H, sizeof(uint16_t));
  int* S_tiles = (int*)calloc((size_t)H * TT, sizeof(int));
  float* invdelta = (float*)calloc((size_t)H * TT, sizeof(float));
  float* a0 = (float*)calloc((size_t)H * TT, sizeof(float));
  float* out_acc = (float*)calloc((size_t)H * D, sizeof(float));

  /* pass 1 */
  for (int kv = 0; kv < KVH; ++kv) {
    const int h0 = kv * GH;
    float qf[SO_MAX_GH * SO_D];
    if (pass1_mode == 0)
      for (int g = 0; g < GH; ++g)
        for (int d = 0; d < SO_D; ++d) qf[g * SO_D + d] = ld16(Q, (size_t)(h0 + g) * SO_D + d, is_bf16) * q_scale;
    for (int t = 0; t < T_c; ++t) {
      const int n0 = t * BN;
      const int len = (n0 + BN < L ? n0 + BN : L) - n0;
      tile_stats_t ts;
      float scores[SO_MAX_BN * SO_MAX_GH];
      const size_t row0 = (size_t)n0 * row_stride + (size_t)kv * D;
      if (pass1_mode == 0)
        tile_stats_vec(qf, K, row0, row_stride, len, GH, 256, is_bf16, &ts, scores);
      else
        tile_stats_general(Q + (size_t)h0 * D, K, row0, row_stride, len, BN, GH, D, is_bf16, q_scale, &ts, scores);
      for (int g = 0; g < GH; ++g) {
        m_tiles[(size_t)(h0 + g) * T_c + t] = ts.m[g];
        ell_tiles[(size_t)(h0 + g) * T_c + t] = ts.ell[g];
        for (int r = 0; r < len; ++r) u_stash[(size_t)(n0 + r) * H + h0 + g] = ts.ub[r * GH + g];
      }
    }
  }
  /* budgets */
  for (int h = 0; h < H; ++h)
    so_prop_budgets(m_tiles + (size_t)h * T_c, ell_tiles + (size_t)h * T_c, T_c, S, seed, h,
                    m_star ? m_star + h : NULL, S_tiles + (size_t)h * T_c, invdelta + (size_t)h * T_c,
                    a0 + (size_t)h * T_c);
  /* pass 2: prop/santa_cuda_kernel.cu:734-864; out accumulated tile by
   * tile in ascending t (the reference's global atomicAdd, :861-863, in
   * the deterministic order the HIP kernel uses). */
  for (int kv = 0; kv < KVH; ++kv) {
    const int h0 = kv * GH;
    for (int t = 0; t < T_c; ++t) {
      const int n0 = t * BN;
      const int len = (n0 + BN < L ? n0 + BN : L) - n0;
      int16_t c[SO_MAX_GH * SO_MAX_BN];
      memset(c, 0, sizeof(c));
      for (int g = 0; g < GH; ++g) {
        const int h = h0 + g;
        tile_counts(u_stash + (size_t)n0 * H + h, H, len, invdelta[(size_t)h * T_c + t], a0[(size_t)h * T_c + t],
                    is_bf16, c + (size_t)g * BN);
      }
      int emit[SO_MAX_BN];
      const int ne = tile_emit(c, BN, GH, len, emit);
      if (rowmask)
        for (int i = 0; i < ne; ++i) rowmask[(size_t)kv * L + n0 + emit[i]] = 1;
      for (int g = 0; g < GH; ++g) {
        const int h = h0 + g;
        if (counts_o) {
          int16_t* dst = counts_o + ((size_t)h * T_c + t) * BN;
          for (int r = 0; r < BN; ++r) dst[r] = (r < len) ? c[(size_t)g * BN + r] : 0;
        }
        if (ne == 0) continue;
        float acc[SO_MAX_D];
        tile_pv(c + (size_t)g * BN, emit, ne, V, (size_t)n0 * row_stride + (size_t)kv * D, row_stride, D, is_bf16,
                acc);
        for (int d = 0; d < D; ++d) out_acc[(size_t)h * D + d] += acc[d];
      }
    }
  }
  /* cast + scale: prop/santa_cuda.cpp:333, prop/santa_cuda_kernel.cu:976-985 */
  const float scale_out = (S > 0) ? (1.0f / (float)S) : 0.0f;
  for (int i = 0; i < H * D; ++i) {
    const float y = out_acc[i] * scale_out;
    if (out_f32) out_f32[i] = y;
    if (out16) out16[i] = st16(y, is_bf16);
  }
  if (m_tiles_o) memcpy(m_tiles_o, m_tiles, sizeof(float) * (size_t)H * T_c);
  if (ell_tiles_o) memcpy(ell_tiles_o, ell_tiles, sizeof(float) * (size_t)H * T_c);
  if (S_tiles_o) memcpy(S_tiles_o, S_tiles, sizeof(int) * (size_t)H * T_c);
  if (invdelta_o) memcpy(invdelta_o, invdelta, sizeof(float) * (size_t)H * T_c);
  if (a0_o) memcpy(a0_o, a0, sizeof(float) * (size_t)H * T_c);
  if (u_stash_o) memcpy(u_stash_o, u_stash, sizeof(uint16_t) * (size_t)L * H);
  free(m_tiles);
  free(ell_tiles);
  free(u_stash);
  free(S_tiles);
  free(invdelta);
  free(a0);
  free(out_acc);
  return 0;
}

int so_prop_decode(const uint16_t* Q, const uint16_t* K, const uint16_t* V, int is_bf16, int H, int KVH, int L,
                   int BN, int S, uint64_t seed, int pass1_mode, float* out_f32, uint16_t* out16,
                   float* m_star, float* m_tiles_o, float* ell_tiles_o, int* S_tiles_o, float* invdelta_o,
                   float* a0_o, uint16_t* u_stash_o, int16_t* counts_o, int* rowmask) {
  return so_prop_decode_d(Q, K, V, is_bf16, H, KVH, SO_D, L, BN, S, seed, pass1_mode, out_f32, out16, m_star,
                          m_tiles_o, ell_tiles_o, S_tiles_o, invdelta_o, a0_o, u_stash_o, counts_o, rowmask);
}

/* Element-wise helpers exported for the known-answer tests. */
void so_expf_array(const float* x, float* y, long n) {
  for (long i = 0; i < n; ++i) y[i] = so_expf(x[i]);
}
void so_u01_array(uint64_t seed, const int* key, const int* t, float* out, long n) {
  for (long i = 0; i < n; ++i) out[i] = so_u01(seed, key[i], t[i]);
}
void so_counts_1d(const uint16_t* ub, int len, float invdel, float a0, int is_bf16, int16_t* c_out) {
  tile_counts(ub, 1, len, invdel, a0, is_bf16, c_out);
}
void so_f32_to_h16_array(const float* x, uint16_t* y, long n, int is_bf16) {
  for (long i = 0; i < n; ++i) y[i] = st16(x[i], is_bf16);
}
void so_h16_to_f32_array(const uint16_t* x, float* y, long n, int is_bf16) {
  for (long i = 0; i < n; ++i) y[i] = ld16(x, (size_t)i, is_bf16);
}
