// santa_flash.hip -- santa_flash (fixed tile budget) decode kernels for gfx950.
//
// Work item = one KV tile (block_n consecutive tokens) of one (b, kv) group.
// A 256-thread workgroup (4 wave64) handles one item:
//
//  A  scores   Each K row (128 x 16-bit = 256 B) is read by 8 lanes, lane p
//              holding the reference's virtual lanes {sigma(p) + 8 i}, i < 4
//              (4 dims each).  The first two levels of the reference's
//              32-lane score tree are in-lane adds; the last three are DPP
//              (row_half_mirror, quad xor2, quad xor1).  sigma = [0,1,2,3,7,6,
//              5,4] makes row_half_mirror pair virtual lanes l and l+4, so the
//              pairing -- and therefore every score bit -- equals the
//              reference's (flash/santa_cuda_kernel.cu:183-211).  All GH query
//              heads of the group reuse the row from registers; q lives in
//              VGPRs for the whole tile.
//  B  tile max per head (exact in any order).
//  C  u = exp(s - m), the 16-bit u, and ell with the reference's
//     per-thread / 32-lane-tree / per-warp association (:243-273).
//  D  systematic counts: 32-row Hillis-Steele scans per head run in
//     parallel; the cross-chunk carries are the reference's sequential
//     float sums (:275-311).
//  E  emission compaction by wave ballots, ascending rows (:314-345).
//  F  count-weighted V sum over the emitted rows, one head per wave,
//     fma per element in ascending row order (:347-379).
//
// A second kernel merges the tiles of each (b, h) (split-KV reduction,
// :386-470) with the same association as the reference's finalize.
#include "santa_device.h"
#include "santa_amd.h"
#include "santa_internal.h"

namespace santa {
namespace flash {

constexpr int kD = 128;
constexpr int kThreads = 256;

template <bool BF16, int GH, int BN>
__global__ __launch_bounds__(kThreads, 2) void fused_tile_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V, int H, int KVH,
    int L_valid, int L_storage, int T_c, float q_scale, int S_pt, uint64_t seed, float* __restrict__ m_tiles,
    float* __restrict__ ell_tiles, float* __restrict__ out_tiles, int* __restrict__ emit_cnt,
    int16_t* __restrict__ dbg_counts) {
  static_assert(BN == 32 || BN == 64 || BN == 256, "block_n");
  static_assert(GH == 4 || GH == 8, "group size");
  constexpr int NT_REF = (BN == 256) ? 256 : 128;  // reference block size (launchers :521,:559)
  constexpr int NW_REF = NT_REF / 32;
  constexpr int ITERS = BN / 32;                   // 32 rows per workgroup iteration
  constexpr int CHUNKS = BN / 32;

  // Linear item id with kv fastest: the 8 KV heads of one token range are
  // read by consecutive workgroups, so each 2 KB NHD token row is streamed
  // by neighbours at about the same time.
  const int id = static_cast<int>(blockIdx.x);
  const int kv = id % KVH;
  const int t = (id / KVH) % T_c;
  const int b = id / (KVH * T_c);
  const int h0 = kv * GH;
  const int n0 = t * BN;
  const int len = min(BN, L_valid - n0);

  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int p = lane & 7;
  const int grp = lane >> 3;
  const int sig = (p < 4) ? p : (11 - p);

  __shared__ float s_sc[BN * GH];
  __shared__ uint16_t s_ub[BN * GH];
  __shared__ int16_t s_cnt[GH * BN];
  __shared__ int16_t s_emit[BN];
  __shared__ float s_acc[NT_REF];
  __shared__ float s_W[NW_REF * GH];
  __shared__ float s_m[GH], s_invdel[GH], s_a0[GH];
  __shared__ float s_T[GH * CHUNKS];
  __shared__ int s_wcnt[4];

  const size_t row_stride = static_cast<size_t>(KVH) * kD;

  // ---- q for this lane's 16 dims of every head, scaled once (A.1) --------
  float qf[GH][4][4];
#pragma unroll
  for (int g = 0; g < GH; ++g) {
    const uint16_t* qp = Q + (static_cast<size_t>(b) * H + h0 + g) * kD + 4 * sig;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint2 w = *reinterpret_cast<const uint2*>(qp + 32 * i);
      qf[g][i][0] = lo16_to_f32<BF16>(w.x) * q_scale;
      qf[g][i][1] = hi16_to_f32<BF16>(w.x) * q_scale;
      qf[g][i][2] = lo16_to_f32<BF16>(w.y) * q_scale;
      qf[g][i][3] = hi16_to_f32<BF16>(w.y) * q_scale;
    }
  }

  // ---- A: scores ----------------------------------------------------------
  const uint16_t* Kt = K + (static_cast<size_t>(b) * L_storage + n0) * row_stride +
                       static_cast<size_t>(kv) * kD + 4 * sig;
  uint2 kw[ITERS][4];
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int r = it * 32 + wave * 8 + grp;
    const int rr = min(r, len - 1);
    const uint16_t* kp = Kt + static_cast<size_t>(rr) * row_stride;
#pragma unroll
    for (int i = 0; i < 4; ++i) kw[it][i] = *reinterpret_cast<const uint2*>(kp + 32 * i);
  }
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int r = it * 32 + wave * 8 + grp;
    float k[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      k[i][0] = lo16_to_f32<BF16>(kw[it][i].x);
      k[i][1] = hi16_to_f32<BF16>(kw[it][i].x);
      k[i][2] = lo16_to_f32<BF16>(kw[it][i].y);
      k[i][3] = hi16_to_f32<BF16>(kw[it][i].y);
    }
    float s[GH];
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      float pp[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = fmaf(qf[g][i][0], k[i][0], 0.0f);
        a = fmaf(qf[g][i][1], k[i][1], a);
        a = fmaf(qf[g][i][2], k[i][2], a);
        a = fmaf(qf[g][i][3], k[i][3], a);
        pp[i] = a;
      }
      const float a0 = pp[0] + pp[2];  // virtual lanes l, l+16
      const float a1 = pp[1] + pp[3];  // l+8, l+24
      const float bb = a0 + a1;        // l, l+8
      const float c = bb + dpp<kDppRowHalfMirror>(bb);  // l, l+4
      const float d = c + dpp<kDppQuadXor2>(c);         // l, l+2
      s[g] = d + dpp<kDppQuadXor1>(d);                  // l, l+1
    }
    if (p == 0 && r < len) {
#pragma unroll
      for (int g = 0; g < GH; ++g) s_sc[r * GH + g] = s[g];
    }
  }
  __syncthreads();

  // ---- B: tile max per head (A.3) ------------------------------------------
#pragma unroll
  for (int g = wave; g < GH; g += 4) {
    float mx = -__builtin_inff();
    for (int r = lane; r < len; r += 64) mx = fmaxf(mx, s_sc[r * GH + g]);
    mx = wave_max(mx);
    if (lane == 0) s_m[g] = mx;
  }
  __syncthreads();

  // ---- C: u, 16-bit u and ell (A.4) ---------------------------------------
  if (tid < NT_REF) {
    const int g = tid % GH;
    const float mg = s_m[g];
    float acc = 0.0f;
    for (int idx = tid; idx < len * GH; idx += NT_REF) {
      const float u = santa_expf(s_sc[idx] - mg);
      acc += u;
      s_ub[idx] = f32_to_h16<BF16>(u);
    }
    s_acc[tid] = acc;
  }
  __syncthreads();
  if (tid < NW_REF * GH) {
    const int w = tid / GH;
    const int g = tid % GH;
    float v[32];
#pragma unroll
    for (int l = 0; l < 32; ++l) v[l] = ((l % GH) == g) ? s_acc[w * 32 + l] : 0.0f;
    s_W[w * GH + g] = tree32(v);
  }
  __syncthreads();
  if (tid < GH) {
    float ell = 0.0f;
#pragma unroll
    for (int w = 0; w < NW_REF; ++w) ell += s_W[w * GH + tid];
    const float invdel = (S_pt > 0 && ell > 1e-20f) ? (static_cast<float>(S_pt) / ell) : 0.0f;
    s_invdel[tid] = invdel;
    s_a0[tid] = u01(seed, b * H + h0 + tid, t);
    const size_t mt = (static_cast<size_t>(b) * H + h0 + tid) * T_c + t;
    m_tiles[mt] = s_m[tid];
    ell_tiles[mt] = ell;
  }
  __syncthreads();

  // ---- D: systematic counts (A.5-A.7) --------------------------------------
  const int r = tid;
  const int chunk = r >> 5;
  const int lam = r & 31;
  float xg[GH], preg[GH];
  if (tid < BN) {
    const int remain = len - chunk * 32;
    const int last = (remain > 0) ? min(31, remain - 1) : 0;
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      const float invdel = s_invdel[g];
      const float x = (r < len && invdel > 0.0f) ? h16_to_f32<BF16>(s_ub[r * GH + g]) * invdel : 0.0f;
      float res = x;
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) {
        const float n = __shfl_up(res, o, 32);
        if (lam >= o) res = res + n;
      }
      const float pre = res - x;
      xg[g] = x;
      preg[g] = pre;
      if (lam == last && remain > 0) s_T[g * CHUNKS + chunk] = pre + x;
    }
  }
  __syncthreads();
  int flag_sum = 0;
  if (tid < BN) {
#pragma unroll
    for (int g = 0; g < GH; ++g) {
      int c = 0;
      if (r < len) {
        float carry = 0.0f;
        for (int k = 0; k < chunk; ++k) carry = carry + s_T[g * CHUNKS + k];
        const float pg = carry + preg[g];
        const float cum = pg + xg[g];
        c = count_from_floors(s_a0[g], pg, cum);
      }
      s_cnt[g * BN + r] = static_cast<int16_t>(c);
      flag_sum += c;
      if (dbg_counts) dbg_counts[((static_cast<size_t>(b) * H + h0 + g) * T_c + t) * BN + r] = static_cast<int16_t>(c);
    }
  }

  // ---- E: emission list (A.8) ----------------------------------------------
  const bool flag = (tid < BN) && (flag_sum > 0);
  const uint64_t bal = __ballot(flag);
  const int pos = __popcll(bal & ((1ull << lane) - 1ull));
  if (lane == 0) s_wcnt[wave] = __popcll(bal);
  __syncthreads();
  int off = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) off += (w < wave) ? s_wcnt[w] : 0;
  if (flag) s_emit[off + pos] = static_cast<int16_t>(r);
  const int E = s_wcnt[0] + s_wcnt[1] + s_wcnt[2] + s_wcnt[3];
  if (tid == 0) emit_cnt[(static_cast<size_t>(b) * KVH + kv) * T_c + t] = E;
  __syncthreads();

  // ---- F: count-weighted V sum (A.9) ---------------------------------------
  const uint16_t* Vt = V + (static_cast<size_t>(b) * L_storage + n0) * row_stride + static_cast<size_t>(kv) * kD +
                       2 * lane;
#pragma unroll
  for (int g = wave; g < GH; g += 4) {
    float acc0 = 0.0f, acc1 = 0.0f;
    for (int base = 0; base < E; base += 8) {
      uint32_t vw[8];
      float cf[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int ii = base + j;
        const int rr = (ii < E) ? static_cast<int>(s_emit[ii]) : 0;
        const int c = (ii < E) ? static_cast<int>(s_cnt[g * BN + rr]) : 0;
        cf[j] = static_cast<float>(c);
        vw[j] = (c != 0) ? *reinterpret_cast<const uint32_t*>(Vt + static_cast<size_t>(rr) * row_stride) : 0u;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (cf[j] != 0.0f) {
          acc0 = fmaf(cf[j], lo16_to_f32<BF16>(vw[j]), acc0);
          acc1 = fmaf(cf[j], hi16_to_f32<BF16>(vw[j]), acc1);
        }
      }
    }
    float2* op = reinterpret_cast<float2*>(out_tiles + ((static_cast<size_t>(b) * H + h0 + g) * T_c + t) * kD) + lane;
    *op = make_float2(acc0, acc1);
  }
}

// Split-KV merge (flash/santa_cuda_kernel.cu:386-470): one workgroup per
// (b, h); max and Z trees with the reference's pairing (strides 128 .. 1),
// numerator accumulated over tiles in ascending order with fma.
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

template <bool BF16, int GH, int BN>
static hipError_t launch_tiles_t(const void* q, const void* K, const void* V, int B, int H, int KVH, int L_valid,
                                 int L_storage, int T_c, int S_pt, uint64_t seed, float* m_tiles, float* ell_tiles,
                                 float* out_tiles, int* emit_cnt, int16_t* counts, hipStream_t stream) {
  const float q_scale = 1.0f / sqrtf(static_cast<float>(kD));
  const unsigned grid = static_cast<unsigned>(B) * static_cast<unsigned>(KVH) * static_cast<unsigned>(T_c);
  hipLaunchKernelGGL((fused_tile_kernel<BF16, GH, BN>), dim3(grid), dim3(kThreads), 0, stream,
                     static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(K),
                     static_cast<const uint16_t*>(V), H, KVH, L_valid, L_storage, T_c, q_scale, S_pt, seed, m_tiles,
                     ell_tiles, out_tiles, emit_cnt, counts);
  return hipGetLastError();
}

template <bool BF16, int GH>
static hipError_t launch_tiles_bn(int bn, const void* q, const void* K, const void* V, int B, int H, int KVH,
                                  int L_valid, int L_storage, int T_c, int S_pt, uint64_t seed, float* m_tiles,
                                  float* ell_tiles, float* out_tiles, int* emit_cnt, int16_t* counts,
                                  hipStream_t stream) {
  switch (bn) {
    case 32:
      return launch_tiles_t<BF16, GH, 32>(q, K, V, B, H, KVH, L_valid, L_storage, T_c, S_pt, seed, m_tiles,
                                          ell_tiles, out_tiles, emit_cnt, counts, stream);
    case 64:
      return launch_tiles_t<BF16, GH, 64>(q, K, V, B, H, KVH, L_valid, L_storage, T_c, S_pt, seed, m_tiles,
                                          ell_tiles, out_tiles, emit_cnt, counts, stream);
    default:
      return launch_tiles_t<BF16, GH, 256>(q, K, V, B, H, KVH, L_valid, L_storage, T_c, S_pt, seed, m_tiles,
                                           ell_tiles, out_tiles, emit_cnt, counts, stream);
  }
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
  const int T_c = (L_valid + block_n - 1) / block_n;
  const int GH = H / KVH;
  hipError_t e;
  if (dtype == SANTA_BF16) {
    e = (GH == 4) ? flash::launch_tiles_bn<true, 4>(block_n, q, K, V, B, H, KVH, L_valid, L_storage, T_c, S_per_tile,
                                                    seed, m_tiles, ell_tiles, out_tiles, emit_cnt, counts, stream)
                  : flash::launch_tiles_bn<true, 8>(block_n, q, K, V, B, H, KVH, L_valid, L_storage, T_c, S_per_tile,
                                                    seed, m_tiles, ell_tiles, out_tiles, emit_cnt, counts, stream);
  } else {
    e = (GH == 4) ? flash::launch_tiles_bn<false, 4>(block_n, q, K, V, B, H, KVH, L_valid, L_storage, T_c, S_per_tile,
                                                     seed, m_tiles, ell_tiles, out_tiles, emit_cnt, counts, stream)
                  : flash::launch_tiles_bn<false, 8>(block_n, q, K, V, B, H, KVH, L_valid, L_storage, T_c, S_per_tile,
                                                     seed, m_tiles, ell_tiles, out_tiles, emit_cnt, counts, stream);
  }
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
  if (shmem > 160 * 1024) return set_error(SANTA_ERR_UNSUPPORTED, "T_c too large for the finalize kernel");
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
  size_t m, ell, out, emit, total;
};
FlashWs flash_ws_layout(int B, int H, int KVH, int D, int T_c) {
  FlashWs w{};
  const size_t bht = static_cast<size_t>(B) * H * T_c;
  size_t off = 0;
  w.m = off;
  off = santa::align_up(off + bht * sizeof(float));
  w.ell = off;
  off = santa::align_up(off + bht * sizeof(float));
  w.out = off;
  off = santa::align_up(off + bht * static_cast<size_t>(D) * sizeof(float));
  w.emit = off;
  off = santa::align_up(off + static_cast<size_t>(B) * KVH * T_c * sizeof(int));
  w.total = off;
  return w;
}
}  // namespace

extern "C" size_t santa_flash_workspace_size(int B, int H, int KVH, int D, int T_c) {
  return flash_ws_layout(B, H, KVH, D, T_c).total;
}

extern "C" int santa_flash_decode(const void* q, const void* K, const void* V, int dtype, int B, int H, int KVH,
                                  int D, int L_valid, int L_storage, int block_n, int S_per_tile, uint64_t seed,
                                  void* out, float* m_star, int* vrows, void* workspace, size_t workspace_bytes,
                                  hipStream_t stream) {
  int st = check_flash_shape(dtype, B, H, KVH, D, L_valid, L_storage, block_n);
  if (st != SANTA_OK) return st;
  const int T_c = (L_valid + block_n - 1) / block_n;
  const FlashWs w = flash_ws_layout(B, H, KVH, D, T_c);
  if (!workspace || workspace_bytes < w.total)
    return set_error(SANTA_ERR_WORKSPACE, "workspace too small: need %zu bytes, got %zu", w.total, workspace_bytes);
  char* base = static_cast<char*>(workspace);
  float* m_tiles = reinterpret_cast<float*>(base + w.m);
  float* ell_tiles = reinterpret_cast<float*>(base + w.ell);
  float* out_tiles = reinterpret_cast<float*>(base + w.out);
  int* emit = reinterpret_cast<int*>(base + w.emit);
  st = santa_flash_fused_tiles(q, K, V, dtype, B, H, KVH, D, L_valid, L_storage, block_n, S_per_tile, seed, m_tiles,
                               ell_tiles, out_tiles, emit, nullptr, stream);
  if (st != SANTA_OK) return st;
  return santa_flash_finalize(m_tiles, ell_tiles, out_tiles, emit, dtype, B, H, KVH, D, T_c, S_per_tile, out, m_star,
                              vrows, stream);
}
