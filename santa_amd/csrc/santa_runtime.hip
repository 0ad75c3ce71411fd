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

}  // namespace rt
}  // namespace santa

using namespace santa;

extern "C" int santa_rt_add_rms_norm(void* h, const void* a, const void* w, void* x, int rows, int hidden, float eps,
                                     hipStream_t stream) {
  if (!h || !w || !x || rows < 0 || hidden <= 0) return set_error(SANTA_ERR_INVALID, "bad add_rms_norm arguments");
  if (rows == 0) return clear_error();
  hipLaunchKernelGGL(rt::add_rms_norm_kernel, dim3(rows), dim3(rt::kNormThreads), 0, stream,
                     static_cast<uint16_t*>(h), static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(w),
                     static_cast<uint16_t*>(x), hidden, eps, a ? 1 : 0);
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
