// ext_prop.cpp -- the `santa_prop_batch_cuda` Python extension module for
// PyTorch-ROCm: the drop-in for the reference's module of the same name
// (prop/santa_cuda.cpp:270-358).  Input checks and their messages, the
// SANTA_PASS1 environment switch (read on every call), the block_n
// normalization and the return tuple follow the reference; the launches go
// through the C ABI of libsanta_amd.so on the current HIP stream.
#include <torch/extension.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <tuple>
#include <vector>

#include "santa_amd.h"

namespace {

// prop/santa_cuda.cpp:144-166
void check_inputs_q_kv(const at::Tensor& q_h, const at::Tensor& K_g, const at::Tensor& V_g) {
  TORCH_CHECK(q_h.is_cuda(), "q_h must be CUDA");
  TORCH_CHECK(K_g.is_cuda() && V_g.is_cuda(), "K_g and V_g must be CUDA");
  TORCH_CHECK((q_h.scalar_type() == at::kBFloat16 || q_h.scalar_type() == at::kHalf), "q_h must be bf16 or f16");
  TORCH_CHECK((K_g.scalar_type() == at::kBFloat16 || K_g.scalar_type() == at::kHalf) &&
                  K_g.scalar_type() == V_g.scalar_type(),
              "K_g/V_g must be bf16 or f16 and match");
  TORCH_CHECK(q_h.scalar_type() == K_g.scalar_type(), "q_h dtype must match K_g/V_g");
  TORCH_CHECK(q_h.dim() == 2 && K_g.dim() == 3 && V_g.dim() == 3, "bad ranks");
  TORCH_CHECK(q_h.device() == K_g.device() && q_h.device() == V_g.device(), "device mismatch");
  TORCH_CHECK(K_g.size(0) == V_g.size(0) && K_g.size(1) == V_g.size(1) && K_g.size(2) == V_g.size(2),
              "K_g and V_g must have the same shape");
  TORCH_CHECK(q_h.size(1) == K_g.size(2), "D mismatch (q_h.size(1) vs K_g.size(2))");
  TORCH_CHECK(K_g.size(1) > 0 && q_h.size(0) % K_g.size(1) == 0,
              "H must be divisible by KVH (expected KVH == K_g.size(1) for NHD)");
  TORCH_CHECK(K_g.is_contiguous() && V_g.is_contiguous(), "K_g/V_g must be contiguous with layout [L, KVH, D] (NHD)");
}

struct Plan {
  int H, D, L, KVH, bn, T_c, path, dtype;
};

Plan plan_call(const at::Tensor& q_h, const at::Tensor& K_g, const at::Tensor& V_g, int64_t block_n) {
  check_inputs_q_kv(q_h, K_g, V_g);
  Plan p{};
  p.H = static_cast<int>(q_h.size(0));
  p.D = static_cast<int>(q_h.size(1));
  p.L = static_cast<int>(K_g.size(0));
  p.KVH = static_cast<int>(K_g.size(1));
  const int rc = santa_prop_plan(p.L, p.H, p.KVH, p.D, block_n, std::getenv("SANTA_PASS1"), &p.bn, &p.T_c, &p.path);
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  p.dtype = (q_h.scalar_type() == at::kBFloat16) ? SANTA_BF16 : SANTA_F16;
  TORCH_CHECK(reinterpret_cast<uintptr_t>(V_g.data_ptr()) % 4 == 0 && reinterpret_cast<uintptr_t>(K_g.data_ptr()) % 16 == 0,
              "K_g/V_g storage must be 16-byte aligned");
  return p;
}

at::Tensor aligned_q(const at::Tensor& q_h) {
  at::Tensor q = q_h.contiguous();
  if (reinterpret_cast<uintptr_t>(q.data_ptr()) % 8 != 0) q = q.clone();
  return q;
}

// Small per-call metadata (lengths, budgets) to the device without a host
// synchronisation: staged in pinned memory from torch's caching host
// allocator, which keeps the buffer until the copy on the current stream has
// run, then copied asynchronously.  The last few uploads are kept per
// (device, stream) and reused when the contents are equal: a decode step
// calls the attention of every layer with the same lengths.  A reuse on the
// stream the copy was made on is ordered after that copy, and an entry is
// never written again, so kernels still reading it are unaffected.  (The
// cache is never destroyed: tensors freed at process exit could outlive the
// HIP runtime.)
at::Tensor to_device_async(const std::vector<int32_t>& host, const at::Device& dev) {
  struct Entry {
    int device;
    hipStream_t stream;
    std::vector<int32_t> host;
    at::Tensor t;
  };
  static auto* cache = new std::vector<Entry>();  // callers hold the GIL
  const hipStream_t stream = c10::hip::getCurrentHIPStream(dev.index()).stream();
  for (const Entry& e : *cache)
    if (e.device == dev.index() && e.stream == stream && e.host == host) return e.t;
  at::Tensor pinned = at::empty({static_cast<int64_t>(host.size())},
                                at::TensorOptions().dtype(at::kInt).pinned_memory(true));
  std::copy(host.begin(), host.end(), pinned.data_ptr<int32_t>());
  at::Tensor t = pinned.to(dev, /*non_blocking=*/true);
  if (cache->size() >= 8) cache->erase(cache->begin());
  cache->push_back(Entry{dev.index(), stream, host, t});
  return t;
}

hipStream_t current_stream(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// Returns (out [H,D] in q's dtype, m_star [H] f32, vrows [KVH] i32 or [0]).
std::tuple<at::Tensor, at::Tensor, at::Tensor> decode_systematic_scalar(at::Tensor q_h, at::Tensor K_g,
                                                                        at::Tensor V_g, int64_t S, uint64_t seed,
                                                                        int64_t block_n, bool want_vrows) {
  const Plan p = plan_call(q_h, K_g, V_g, block_n);
  c10::DeviceGuard guard(q_h.device());
  const at::Tensor q = aligned_q(q_h);
  auto optsF = q.options().dtype(at::kFloat);
  auto optsI = q.options().dtype(at::kInt);
  at::Tensor out = at::empty({p.H, p.D}, q.options());
  at::Tensor m_star = at::empty({p.H}, optsF);
  at::Tensor vrows = want_vrows ? at::empty({p.KVH}, optsI) : at::empty({0}, optsI);
  const size_t ws_bytes = santa_prop_workspace_size(p.H, p.KVH, p.D, p.L, p.T_c);
  at::Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  const int rc = santa_prop_decode(q.data_ptr(), K_g.data_ptr(), V_g.data_ptr(), p.dtype, p.H, p.KVH, p.D, p.L, p.bn,
                                   p.path, static_cast<int>(S), seed, out.data_ptr(), m_star.data_ptr<float>(),
                                   want_vrows ? vrows.data_ptr<int>() : nullptr, ws.data_ptr(), ws_bytes,
                                   current_stream(q));
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  return std::make_tuple(out, m_star, vrows);
}

// Test-only: every intermediate of one call through the three stage entry
// points.  Returns (m_tiles [H,T_c], ell_tiles, m_star [H], S_tiles [H,T_c]
// i32, invdelta, a0, u_stash [L,H] (q dtype), counts [H,T_c,block_n] i16,
// out [H,D], vrows [KVH]).
std::vector<at::Tensor> debug_pass(at::Tensor q_h, at::Tensor K_g, at::Tensor V_g, int64_t S, uint64_t seed,
                                   int64_t block_n) {
  const Plan p = plan_call(q_h, K_g, V_g, block_n);
  c10::DeviceGuard guard(q_h.device());
  const at::Tensor q = aligned_q(q_h);
  auto optsF = q.options().dtype(at::kFloat);
  auto optsI = q.options().dtype(at::kInt);
  at::Tensor m_tiles = at::empty({p.H, p.T_c}, optsF);
  at::Tensor ell_tiles = at::empty({p.H, p.T_c}, optsF);
  at::Tensor m_star = at::empty({p.H}, optsF);
  at::Tensor S_tiles = at::empty({p.H, p.T_c}, optsI);
  at::Tensor invdelta = at::empty({p.H, p.T_c}, optsF);
  at::Tensor a0 = at::empty({p.H, p.T_c}, optsF);
  at::Tensor stash = at::empty({p.L, p.H}, q.options());
  at::Tensor counts = at::empty({p.H, p.T_c, p.bn}, q.options().dtype(at::kShort));
  at::Tensor out = at::empty({p.H, p.D}, q.options());
  at::Tensor vrows = at::empty({p.KVH}, optsI);
  const size_t ws_bytes = santa_prop_workspace_size(p.H, p.KVH, p.D, p.L, p.T_c);
  at::Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  hipStream_t st = current_stream(q);
  int rc = santa_prop_pass1(q.data_ptr(), K_g.data_ptr(), p.dtype, p.H, p.KVH, p.D, p.L, p.bn, p.path,
                            m_tiles.data_ptr<float>(), ell_tiles.data_ptr<float>(), stash.data_ptr(), st);
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  rc = santa_prop_tile_budgets(m_tiles.data_ptr<float>(), ell_tiles.data_ptr<float>(), p.H, p.T_c,
                               static_cast<int>(S), seed, m_star.data_ptr<float>(), S_tiles.data_ptr<int>(),
                               invdelta.data_ptr<float>(), a0.data_ptr<float>(), st);
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  rc = santa_prop_pass2(V_g.data_ptr(), stash.data_ptr(), p.dtype, p.H, p.KVH, p.D, p.L, p.bn, static_cast<int>(S),
                        invdelta.data_ptr<float>(), a0.data_ptr<float>(), counts.data_ptr<int16_t>(), out.data_ptr(),
                        vrows.data_ptr<int>(), ws.data_ptr(), ws_bytes, st);
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  return {m_tiles, ell_tiles, m_star, S_tiles, invdelta, a0, stash, counts, out, vrows};
}

// A Python int (same value for every sequence) or a length-B sequence / 1-D
// tensor of ints.
std::vector<int64_t> per_sequence(const py::object& v, int64_t B, const char* name) {
  std::vector<int64_t> out;
  if (py::isinstance<py::int_>(v)) {
    out.assign(static_cast<size_t>(B), v.cast<int64_t>());
    return out;
  }
  if (THPVariable_Check(v.ptr())) {
    const at::Tensor t = v.cast<at::Tensor>().to(at::kCPU).to(at::kLong).contiguous();
    TORCH_CHECK(t.dim() == 1 && t.numel() == B, name, " must be an int or have one entry per sequence (", B, ")");
    const int64_t* p = t.data_ptr<int64_t>();
    out.assign(p, p + B);
    return out;
  }
  out = v.cast<std::vector<int64_t>>();
  TORCH_CHECK(static_cast<int64_t>(out.size()) == B, name, " must be an int or have one entry per sequence (", B, ")");
  return out;
}

// Batched (and ragged) santa_prop: q_h [B,H,D], K_g/V_g [B,L_storage,KVH,D];
// S and valid_len are ints or per-sequence lists / tensors.  Sequence b is
// decoded exactly as decode_systematic_scalar on K_g[b, :valid_len[b]] with
// budget S[b].  Returns (out [B,H,D], m_star [B,H], vrows [B,KVH] or [0]).
std::tuple<at::Tensor, at::Tensor, at::Tensor> decode_batched(at::Tensor q_h, at::Tensor K_g, at::Tensor V_g,
                                                              py::object S, uint64_t seed, int64_t block_n,
                                                              bool want_vrows, py::object valid_len) {
  TORCH_CHECK(q_h.is_cuda(), "q_h must be CUDA");
  TORCH_CHECK(K_g.is_cuda() && V_g.is_cuda(), "K_g and V_g must be CUDA");
  TORCH_CHECK((q_h.scalar_type() == at::kBFloat16 || q_h.scalar_type() == at::kHalf), "q_h must be bf16 or f16");
  TORCH_CHECK((K_g.scalar_type() == at::kBFloat16 || K_g.scalar_type() == at::kHalf) &&
                  K_g.scalar_type() == V_g.scalar_type(),
              "K_g/V_g must be bf16 or f16 and match");
  TORCH_CHECK(q_h.scalar_type() == K_g.scalar_type(), "q_h dtype must match K_g/V_g");
  TORCH_CHECK(q_h.dim() == 3 && K_g.dim() == 4 && V_g.dim() == 4,
              "Batched path expects q_h [B,H,D], K_g/V_g [B,L,KVH,D]");
  TORCH_CHECK(q_h.device() == K_g.device() && q_h.device() == V_g.device(), "device mismatch");
  TORCH_CHECK(K_g.sizes() == V_g.sizes(), "K_g and V_g must have the same shape");
  TORCH_CHECK(q_h.size(0) == K_g.size(0), "Batch mismatch between q_h and K_g/V_g");
  TORCH_CHECK(q_h.size(2) == K_g.size(3), "D mismatch (q_h.size(2) vs K_g.size(3))");
  TORCH_CHECK(K_g.size(2) > 0 && q_h.size(1) % K_g.size(2) == 0,
              "H must be divisible by KVH (expected KVH == K_g.size(2) for NHD)");
  TORCH_CHECK(K_g.is_contiguous() && V_g.is_contiguous(), "K_g/V_g must be contiguous with layout [B, L, KVH, D] (NHD)");
  const int B = static_cast<int>(q_h.size(0)), H = static_cast<int>(q_h.size(1)), D = static_cast<int>(q_h.size(2));
  const int L_st = static_cast<int>(K_g.size(1)), KVH = static_cast<int>(K_g.size(2));
  const std::vector<int64_t> Ss = per_sequence(S, B, "S");
  std::vector<int64_t> lens = per_sequence(valid_len, B, "valid_len");
  const char* env = std::getenv("SANTA_PASS1");
  std::vector<int> bn(B), tc(B), path(B);
  for (int b = 0; b < B; ++b) {
    if (lens[b] <= 0) lens[b] = L_st;
    TORCH_CHECK(lens[b] <= L_st, "valid_len exceeds storage length: valid_len=", lens[b], " storage=", L_st);
    const int rc = santa_prop_plan(static_cast<int>(lens[b]), H, KVH, D, block_n, env, &bn[b], &tc[b], &path[b]);
    TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  }
  c10::DeviceGuard guard(q_h.device());
  const at::Tensor q = aligned_q(q_h);
  const int dtype = (q.scalar_type() == at::kBFloat16) ? SANTA_BF16 : SANTA_F16;
  TORCH_CHECK(reinterpret_cast<uintptr_t>(K_g.data_ptr()) % 16 == 0 && reinterpret_cast<uintptr_t>(V_g.data_ptr()) % 4 == 0,
              "K_g/V_g storage must be 16-byte aligned");
  auto optsF = q.options().dtype(at::kFloat);
  auto optsI = q.options().dtype(at::kInt);
  at::Tensor out = at::empty({B, H, D}, q.options());
  at::Tensor m_star = at::empty({B, H}, optsF);
  at::Tensor vrows = want_vrows ? at::empty({B, KVH}, optsI) : at::empty({0}, optsI);
  hipStream_t st = current_stream(q);
  bool uniform = true;
  for (int b = 1; b < B; ++b) uniform = uniform && bn[b] == bn[0] && path[b] == path[0];
  if (uniform) {
    long long total = 0;
    int max_len = 0, max_tiles = 0;
    std::vector<int32_t> host(2 * static_cast<size_t>(B));
    for (int b = 0; b < B; ++b) {
      total += tc[b];
      max_len = std::max(max_len, static_cast<int>(lens[b]));
      max_tiles = std::max(max_tiles, tc[b]);
      host[b] = static_cast<int32_t>(lens[b]);
      host[B + b] = static_cast<int32_t>(Ss[b]);
    }
    at::Tensor meta = to_device_async(host, q.device());
    const size_t ws_bytes = santa_prop_batched_workspace_size(B, H, KVH, D, L_st, max_tiles, total);
    at::Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
    const int rc = santa_prop_decode_batched(q.data_ptr(), K_g.data_ptr(), V_g.data_ptr(), dtype, B, H, KVH, D, L_st,
                                             meta.data_ptr<int>(), meta.data_ptr<int>() + B, max_len, total, bn[0],
                                             path[0], seed, out.data_ptr(), m_star.data_ptr<float>(),
                                             want_vrows ? vrows.data_ptr<int>() : nullptr, ws.data_ptr(), ws_bytes, st);
    TORCH_CHECK(rc == SANTA_OK, santa_last_error());
    return std::make_tuple(out, m_star, vrows);
  }
  // sequences on different block sizes / pass-1 paths: one launch sequence each
  const size_t row = static_cast<size_t>(KVH) * D * K_g.element_size();
  for (int b = 0; b < B; ++b) {
    const size_t ws_bytes = santa_prop_workspace_size(H, KVH, D, static_cast<int>(lens[b]), tc[b]);
    at::Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
    const char* Kb = static_cast<const char*>(K_g.data_ptr()) + static_cast<size_t>(b) * L_st * row;
    const char* Vb = static_cast<const char*>(V_g.data_ptr()) + static_cast<size_t>(b) * L_st * row;
    const int rc = santa_prop_decode(static_cast<const char*>(q.data_ptr()) + static_cast<size_t>(b) * H * D * q.element_size(),
                                     Kb, Vb, dtype, H, KVH, D, static_cast<int>(lens[b]), bn[b], path[b],
                                     static_cast<int>(Ss[b]), seed,
                                     static_cast<char*>(out.data_ptr()) + static_cast<size_t>(b) * H * D * out.element_size(),
                                     m_star.data_ptr<float>() + static_cast<size_t>(b) * H,
                                     want_vrows ? vrows.data_ptr<int>() + static_cast<size_t>(b) * KVH : nullptr,
                                     ws.data_ptr(), ws_bytes, st);
    TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  }
  return std::make_tuple(out, m_star, vrows);
}

// Paged santa_prop (an addition over the reference, whose caches are
// contiguous NHD, README.md:257): K_pages / V_pages [num_pages, page_size,
// KVH, D], block_table int32 [B, table_stride] on the device; seq_lens and S
// are ints or per-sequence lists / tensors.  Sequence b is decoded exactly as
// decode_systematic_scalar on its seq_lens[b] tokens stored contiguously.
std::tuple<at::Tensor, at::Tensor, at::Tensor> decode_paged(at::Tensor q_h, at::Tensor K_pages, at::Tensor V_pages,
                                                            at::Tensor block_table, py::object seq_lens, py::object S,
                                                            uint64_t seed, int64_t block_n, bool want_vrows) {
  TORCH_CHECK(q_h.is_cuda(), "q_h must be CUDA");
  TORCH_CHECK(K_pages.is_cuda() && V_pages.is_cuda(), "K_pages and V_pages must be CUDA");
  TORCH_CHECK(block_table.is_cuda(), "block_table must be CUDA");
  TORCH_CHECK((q_h.scalar_type() == at::kBFloat16 || q_h.scalar_type() == at::kHalf), "q_h must be bf16 or f16");
  TORCH_CHECK(K_pages.scalar_type() == q_h.scalar_type() && V_pages.scalar_type() == q_h.scalar_type(),
              "q_h dtype must match K_pages/V_pages");
  TORCH_CHECK(q_h.device() == K_pages.device() && q_h.device() == V_pages.device() &&
                  q_h.device() == block_table.device(),
              "device mismatch");
  TORCH_CHECK(q_h.dim() == 3 && K_pages.dim() == 4 && V_pages.dim() == 4,
              "Paged path expects q_h [B,H,D], K_pages/V_pages [num_pages,page_size,KVH,D]");
  TORCH_CHECK(K_pages.sizes() == V_pages.sizes(), "K_pages and V_pages must have the same shape");
  TORCH_CHECK(K_pages.is_contiguous() && V_pages.is_contiguous(), "K_pages/V_pages must be contiguous");
  TORCH_CHECK(block_table.scalar_type() == at::kInt && block_table.dim() == 2 && block_table.is_contiguous(),
              "block_table must be a contiguous int32 [B, pages_per_sequence] tensor");
  TORCH_CHECK(q_h.size(2) == K_pages.size(3), "D mismatch (q_h.size(2) vs K_pages.size(3))");
  TORCH_CHECK(K_pages.size(2) > 0 && q_h.size(1) % K_pages.size(2) == 0,
              "H must be divisible by KVH (expected KVH == K_pages.size(2) for NHD)");
  const int B = static_cast<int>(q_h.size(0)), H = static_cast<int>(q_h.size(1)), D = static_cast<int>(q_h.size(2));
  const int num_pages = static_cast<int>(K_pages.size(0)), page_size = static_cast<int>(K_pages.size(1));
  const int KVH = static_cast<int>(K_pages.size(2));
  TORCH_CHECK(block_table.size(0) == B, "block_table must have one row per sequence (", B, ")");
  const int stride = static_cast<int>(block_table.size(1));
  const long long capacity = static_cast<long long>(stride) * page_size;
  const std::vector<int64_t> Ss = per_sequence(S, B, "S");
  const std::vector<int64_t> lens = per_sequence(seq_lens, B, "seq_lens");
  const char* env = std::getenv("SANTA_PASS1");
  std::vector<int> bn(B), tc(B), path(B);
  for (int b = 0; b < B; ++b) {
    TORCH_CHECK(lens[b] > 0, "seq_lens must be > 0; got ", lens[b]);
    TORCH_CHECK(lens[b] <= capacity, "seq_lens exceeds the block table's capacity: ", lens[b], " > ", capacity);
    const int rc = santa_prop_plan(static_cast<int>(lens[b]), H, KVH, D, block_n, env, &bn[b], &tc[b], &path[b]);
    TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  }
  c10::DeviceGuard guard(q_h.device());
  const at::Tensor q = aligned_q(q_h);
  const int dtype = (q.scalar_type() == at::kBFloat16) ? SANTA_BF16 : SANTA_F16;
  TORCH_CHECK(reinterpret_cast<uintptr_t>(K_pages.data_ptr()) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(V_pages.data_ptr()) % 4 == 0,
              "K_pages/V_pages storage must be 16-byte aligned");
  auto optsF = q.options().dtype(at::kFloat);
  auto optsI = q.options().dtype(at::kInt);
  at::Tensor out = at::empty({B, H, D}, q.options());
  at::Tensor m_star = at::empty({B, H}, optsF);
  at::Tensor vrows = want_vrows ? at::empty({B, KVH}, optsI) : at::empty({0}, optsI);
  hipStream_t st = current_stream(q);
  std::vector<int32_t> host(2 * static_cast<size_t>(B));
  for (int b = 0; b < B; ++b) {
    host[b] = static_cast<int32_t>(lens[b]);
    host[B + b] = static_cast<int32_t>(Ss[b]);
  }
  at::Tensor meta = to_device_async(host, q.device());
  // one launch sequence over [b0, b1) with a common block size and pass-1 path
  auto launch = [&](int b0, int b1) {
    const int nb = b1 - b0;
    long long total = 0;
    int max_len = 0, max_tiles = 0;
    for (int b = b0; b < b1; ++b) {
      total += tc[b];
      max_len = std::max(max_len, static_cast<int>(lens[b]));
      max_tiles = std::max(max_tiles, tc[b]);
    }
    const size_t ws_bytes = santa_prop_batched_workspace_size(nb, H, KVH, D, max_len, max_tiles, total);
    at::Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
    const int rc = santa_prop_decode_paged(
        static_cast<const char*>(q.data_ptr()) + static_cast<size_t>(b0) * H * D * q.element_size(), K_pages.data_ptr(),
        V_pages.data_ptr(), dtype, nb, H, KVH, D, num_pages, page_size,
        block_table.data_ptr<int>() + static_cast<size_t>(b0) * stride, stride, meta.data_ptr<int>() + b0,
        meta.data_ptr<int>() + B + b0, max_len, total, bn[b0], path[b0], seed,
        static_cast<char*>(out.data_ptr()) + static_cast<size_t>(b0) * H * D * out.element_size(),
        m_star.data_ptr<float>() + static_cast<size_t>(b0) * H,
        want_vrows ? vrows.data_ptr<int>() + static_cast<size_t>(b0) * KVH : nullptr, ws.data_ptr(), ws_bytes, st);
    TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  };
  bool uniform = true;
  for (int b = 1; b < B; ++b) uniform = uniform && bn[b] == bn[0] && path[b] == path[0];
  if (uniform) {
    launch(0, B);
  } else {
    // sequences on different block sizes / pass-1 paths: one launch sequence each
    for (int b = 0; b < B; ++b) launch(b, b + 1);
  }
  return std::make_tuple(out, m_star, vrows);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "S^2ANTA-Prop sampled-attention decode for MI355X (gfx950)";
  m.def("decode_systematic_scalar", &decode_systematic_scalar, py::arg("q_h"), py::arg("K_g"), py::arg("V_g"),
        py::arg("S"), py::arg("seed") = 42ULL, py::arg("block_n") = 0, py::arg("want_vrows") = false);
  m.def("decode_systematic_batched", &decode_batched, py::arg("q_h"), py::arg("K_g"), py::arg("V_g"), py::arg("S"),
        py::arg("seed") = 42ULL, py::arg("block_n") = 0, py::arg("want_vrows") = false,
        py::arg("valid_len") = py::int_(-1));
  m.def("decode_systematic_paged", &decode_paged, py::arg("q_h"), py::arg("K_pages"), py::arg("V_pages"),
        py::arg("block_table"), py::arg("seq_lens"), py::arg("S"), py::arg("seed") = 42ULL, py::arg("block_n") = 0,
        py::arg("want_vrows") = false);
  m.def("_debug_pass", &debug_pass, py::arg("q_h"), py::arg("K_g"), py::arg("V_g"), py::arg("S"),
        py::arg("seed") = 42ULL, py::arg("block_n") = 0);
  m.def("_library_version", []() { return std::string(santa_version()); });
}
