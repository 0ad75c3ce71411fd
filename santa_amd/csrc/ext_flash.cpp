// ext_flash.cpp -- the `santa_flash_batch_cuda` Python extension module for
// PyTorch-ROCm: the drop-in for the reference's module of the same name
// (flash/santa_cuda.cpp:174-359).  Input checks and their messages, the
// planning and the return tuple follow the reference; the launches go
// through the C ABI of libsanta_amd.so on the current HIP stream.
#include <torch/extension.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <algorithm>
#include <string>
#include <tuple>
#include <vector>

#include "santa_amd.h"
#include "santa_internal.h"

namespace {

struct ShapeInfo {
  bool batched;
  int B, H, D, L_storage, KVH;
};

// flash/santa_cuda.cpp:123-171
ShapeInfo check_inputs_q_kv(const at::Tensor& q_h, const at::Tensor& K_g, const at::Tensor& V_g) {
  TORCH_CHECK(q_h.is_cuda(), "q_h must be CUDA");
  TORCH_CHECK(K_g.is_cuda() && V_g.is_cuda(), "K_g and V_g must be CUDA");
  TORCH_CHECK((q_h.scalar_type() == at::kBFloat16 || q_h.scalar_type() == at::kHalf), "q_h must be bf16 or f16");
  TORCH_CHECK((K_g.scalar_type() == at::kBFloat16 || K_g.scalar_type() == at::kHalf), "K_g must be bf16 or f16");
  TORCH_CHECK(K_g.scalar_type() == V_g.scalar_type(), "K_g and V_g must have the same dtype");
  TORCH_CHECK(q_h.scalar_type() == K_g.scalar_type(), "q_h dtype must match K_g/V_g dtype");
  TORCH_CHECK(q_h.device() == K_g.device() && q_h.device() == V_g.device(), "device mismatch");
  TORCH_CHECK(K_g.is_contiguous() && V_g.is_contiguous(),
              "K_g/V_g must be contiguous. Expected [L,KVH,D] for single or [B,L,KVH,D] for batch.");
  ShapeInfo info{};
  if (q_h.dim() == 2) {
    TORCH_CHECK(K_g.dim() == 3 && V_g.dim() == 3, "Single-request path expects q_h [H,D], K_g/V_g [L,KVH,D]");
    TORCH_CHECK(K_g.size(0) == V_g.size(0) && K_g.size(1) == V_g.size(1) && K_g.size(2) == V_g.size(2),
                "K_g and V_g must have the same shape");
    TORCH_CHECK(q_h.size(1) == K_g.size(2), "D mismatch (q_h.size(1) vs K_g.size(2))");
    info.batched = false;
    info.B = 1;
    info.H = static_cast<int>(q_h.size(0));
    info.D = static_cast<int>(q_h.size(1));
    info.L_storage = static_cast<int>(K_g.size(0));
    info.KVH = static_cast<int>(K_g.size(1));
    return info;
  }
  TORCH_CHECK(q_h.dim() == 3 && K_g.dim() == 4 && V_g.dim() == 4,
              "Batched path expects q_h [B,H,D], K_g/V_g [B,L,KVH,D]");
  TORCH_CHECK(K_g.size(0) == V_g.size(0) && K_g.size(1) == V_g.size(1) && K_g.size(2) == V_g.size(2) &&
                  K_g.size(3) == V_g.size(3),
              "K_g and V_g must have the same shape");
  TORCH_CHECK(q_h.size(0) == K_g.size(0), "Batch mismatch between q_h and K_g/V_g");
  TORCH_CHECK(q_h.size(2) == K_g.size(3), "D mismatch (q_h.size(2) vs K_g.size(3))");
  info.batched = true;
  info.B = static_cast<int>(q_h.size(0));
  info.H = static_cast<int>(q_h.size(1));
  info.D = static_cast<int>(q_h.size(2));
  info.L_storage = static_cast<int>(K_g.size(1));
  info.KVH = static_cast<int>(K_g.size(2));
  return info;
}

struct Plan {
  ShapeInfo info;
  int L, bn, T_c, S_pt, dtype;
};

// flash/santa_cuda.cpp:182-210 (same order of checks and messages).
Plan plan_call(const at::Tensor& q, const at::Tensor& K_g, const at::Tensor& V_g, int64_t S, int64_t block_n,
               int64_t valid_len) {
  Plan p{};
  p.info = check_inputs_q_kv(q, K_g, V_g);
  const int H = p.info.H, KVH = p.info.KVH, D = p.info.D;
  const int L = (valid_len > 0) ? static_cast<int>(valid_len) : p.info.L_storage;
  TORCH_CHECK(L > 0, "valid_len must be > 0; got ", L);
  TORCH_CHECK(L <= p.info.L_storage, "valid_len exceeds storage length: valid_len=", L, " storage=",
              p.info.L_storage);
  TORCH_CHECK(D == 128, "This build supports only D=128. Got D=", D);
  TORCH_CHECK(KVH > 0 && H % KVH == 0, "H must be divisible by KVH. Got H=", H, " KVH=", KVH);
  const int GH = H / KVH;
  TORCH_CHECK(GH == 4 || GH == 8, "This build supports only GH=4 or GH=8 (H/KVH). Got GH=", GH, " (H=", H,
              " KVH=", KVH, ")");
  const int rc = santa_flash_plan(p.info.L_storage, valid_len, block_n, S, &p.L, &p.bn, &p.T_c, &p.S_pt);
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  p.dtype = (q.scalar_type() == at::kBFloat16) ? SANTA_BF16 : SANTA_F16;
  TORCH_CHECK(reinterpret_cast<uintptr_t>(K_g.data_ptr()) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(V_g.data_ptr()) % 16 == 0,
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

std::tuple<at::Tensor, at::Tensor, at::Tensor> decode_ragged(at::Tensor q_h, at::Tensor K_g, at::Tensor V_g,
                                                             int64_t S, uint64_t seed, int64_t block_n,
                                                             bool want_vrows, std::vector<int64_t> lens);

// valid_len: an int (the reference's form), or -- an addition over the
// reference -- one length per sequence (list or 1-D tensor) for the batched
// form.
std::tuple<at::Tensor, at::Tensor, at::Tensor> decode_systematic_scalar(at::Tensor q_h, at::Tensor K_g,
                                                                        at::Tensor V_g, int64_t S, uint64_t seed,
                                                                        int64_t block_n, bool want_vrows,
                                                                        py::object valid_len_obj) {
  int64_t valid_len = -1;
  if (py::isinstance<py::int_>(valid_len_obj)) {
    valid_len = valid_len_obj.cast<int64_t>();
  } else {
    std::vector<int64_t> lens;
    if (THPVariable_Check(valid_len_obj.ptr())) {
      const at::Tensor t = valid_len_obj.cast<at::Tensor>().to(at::kCPU).to(at::kLong).contiguous();
      TORCH_CHECK(t.dim() == 1, "valid_len must be an int or a 1-D list of per-sequence lengths");
      lens.assign(t.data_ptr<int64_t>(), t.data_ptr<int64_t>() + t.numel());
    } else {
      lens = valid_len_obj.cast<std::vector<int64_t>>();
    }
    TORCH_CHECK(q_h.dim() == 3, "per-sequence valid_len needs the batched form q_h [B,H,D]");
    TORCH_CHECK(static_cast<int64_t>(lens.size()) == q_h.size(0),
                "valid_len must be an int or have one entry per sequence (", q_h.size(0), ")");
    bool uniform = true;
    for (size_t i = 1; i < lens.size(); ++i) uniform = uniform && lens[i] == lens[0];
    if (!uniform) return decode_ragged(q_h, K_g, V_g, S, seed, block_n, want_vrows, lens);
    valid_len = lens.empty() ? -1 : lens[0];
  }
  const Plan p = plan_call(q_h, K_g, V_g, S, block_n, valid_len);
  c10::DeviceGuard guard(q_h.device());
  const at::Tensor q = aligned_q(q_h);
  const ShapeInfo& in = p.info;
  auto optsF = q.options().dtype(at::kFloat);
  auto optsI = q.options().dtype(at::kInt);
  at::Tensor out = in.batched ? at::empty({in.B, in.H, in.D}, q.options()) : at::empty({in.H, in.D}, q.options());
  at::Tensor m_star = in.batched ? at::empty({in.B, in.H}, optsF) : at::empty({in.H}, optsF);
  at::Tensor vrows = at::empty({0}, optsI);
  if (want_vrows) vrows = in.batched ? at::empty({in.B, in.KVH}, optsI) : at::empty({in.KVH}, optsI);
  const size_t ws_bytes = santa_flash_workspace_size(in.B, in.H, in.KVH, in.D, p.T_c);
  at::Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  const int rc = santa_flash_decode(q.data_ptr(), K_g.data_ptr(), V_g.data_ptr(), p.dtype, in.B, in.H, in.KVH, in.D,
                                    p.L, in.L_storage, p.bn, p.S_pt, seed, out.data_ptr(),
                                    m_star.data_ptr<float>(), want_vrows ? vrows.data_ptr<int>() : nullptr,
                                    ws.data_ptr(), ws_bytes, current_stream(q));
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  return std::make_tuple(out, m_star, vrows);
}

// Ragged batch: block_n planned from the longest sequence (or given), one
// launch pair over all sequences (santa_flash_decode_ragged).
std::tuple<at::Tensor, at::Tensor, at::Tensor> decode_ragged(at::Tensor q_h, at::Tensor K_g, at::Tensor V_g,
                                                             int64_t S, uint64_t seed, int64_t block_n,
                                                             bool want_vrows, std::vector<int64_t> lens) {
  const ShapeInfo in = check_inputs_q_kv(q_h, K_g, V_g);
  int64_t max_len = 0;
  for (int64_t& l : lens) {
    if (l <= 0) l = in.L_storage;
    TORCH_CHECK(l <= in.L_storage, "valid_len exceeds storage length: valid_len=", l, " storage=", in.L_storage);
    max_len = std::max(max_len, l);
  }
  // checks and block_n as for a uniform call at the longest length
  const Plan p = plan_call(q_h, K_g, V_g, S, block_n, max_len);
  c10::DeviceGuard guard(q_h.device());
  const at::Tensor q = aligned_q(q_h);
  long long total = 0;
  std::vector<int32_t> host(lens.size());
  for (size_t b = 0; b < lens.size(); ++b) {
    host[b] = static_cast<int32_t>(lens[b]);
    total += (lens[b] + p.bn - 1) / p.bn;
  }
  at::Tensor dlens = to_device_async(host, q.device());
  auto optsF = q.options().dtype(at::kFloat);
  auto optsI = q.options().dtype(at::kInt);
  at::Tensor out = at::empty({in.B, in.H, in.D}, q.options());
  at::Tensor m_star = at::empty({in.B, in.H}, optsF);
  at::Tensor vrows = want_vrows ? at::empty({in.B, in.KVH}, optsI) : at::empty({0}, optsI);
  const size_t ws_bytes = santa_flash_ragged_workspace_size(in.B, in.H, in.KVH, in.D, p.T_c, total);
  at::Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  const int rc = santa_flash_decode_ragged(q.data_ptr(), K_g.data_ptr(), V_g.data_ptr(), p.dtype, in.B, in.H, in.KVH,
                                           in.D, in.L_storage, dlens.data_ptr<int>(), static_cast<int>(max_len), total,
                                           p.bn, S, seed, out.data_ptr(), m_star.data_ptr<float>(),
                                           want_vrows ? vrows.data_ptr<int>() : nullptr, ws.data_ptr(), ws_bytes,
                                           current_stream(q));
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  return std::make_tuple(out, m_star, vrows);
}

// Paged KV (an addition over the reference, whose caches are contiguous NHD,
// README.md:257): K_pages / V_pages [num_pages, page_size, KVH, D], block_table
// int32 [B, table_stride] on the device, seq_lens an int or one length per
// sequence.  Token n of sequence b is row n % page_size of page
// block_table[b, n / page_size].  block_n is planned from the longest
// sequence (or given) as in the ragged call, whose results this call
// reproduces bit for bit on the same tokens stored contiguously.
std::tuple<at::Tensor, at::Tensor, at::Tensor> decode_paged(at::Tensor q_h, at::Tensor K_pages, at::Tensor V_pages,
                                                            at::Tensor block_table, py::object seq_lens, int64_t S,
                                                            uint64_t seed, int64_t block_n, bool want_vrows) {
  TORCH_CHECK(q_h.is_cuda(), "q_h must be CUDA");
  TORCH_CHECK(K_pages.is_cuda() && V_pages.is_cuda(), "K_pages and V_pages must be CUDA");
  TORCH_CHECK(block_table.is_cuda(), "block_table must be CUDA");
  TORCH_CHECK((q_h.scalar_type() == at::kBFloat16 || q_h.scalar_type() == at::kHalf), "q_h must be bf16 or f16");
  TORCH_CHECK(K_pages.scalar_type() == q_h.scalar_type() && V_pages.scalar_type() == q_h.scalar_type(),
              "q_h dtype must match K_pages/V_pages dtype");
  TORCH_CHECK(q_h.device() == K_pages.device() && q_h.device() == V_pages.device() &&
                  q_h.device() == block_table.device(),
              "device mismatch");
  TORCH_CHECK(q_h.dim() == 3 && K_pages.dim() == 4 && V_pages.dim() == 4,
              "Paged path expects q_h [B,H,D], K_pages/V_pages [num_pages,page_size,KVH,D]");
  TORCH_CHECK(K_pages.sizes() == V_pages.sizes(), "K_pages and V_pages must have the same shape");
  TORCH_CHECK(K_pages.is_contiguous() && V_pages.is_contiguous(), "K_pages/V_pages must be contiguous");
  TORCH_CHECK(block_table.scalar_type() == at::kInt && block_table.dim() == 2 && block_table.is_contiguous(),
              "block_table must be a contiguous int32 [B, pages_per_sequence] tensor");
  const int B = static_cast<int>(q_h.size(0)), H = static_cast<int>(q_h.size(1)), D = static_cast<int>(q_h.size(2));
  const int num_pages = static_cast<int>(K_pages.size(0)), page_size = static_cast<int>(K_pages.size(1));
  const int KVH = static_cast<int>(K_pages.size(2));
  TORCH_CHECK(q_h.size(2) == K_pages.size(3), "D mismatch (q_h.size(2) vs K_pages.size(3))");
  TORCH_CHECK(block_table.size(0) == B, "block_table must have one row per sequence (", B, ")");
  const int stride = static_cast<int>(block_table.size(1));
  const long long capacity = static_cast<long long>(stride) * page_size;
  std::vector<int64_t> lens;
  if (py::isinstance<py::int_>(seq_lens)) {
    lens.assign(static_cast<size_t>(B), seq_lens.cast<int64_t>());
  } else if (THPVariable_Check(seq_lens.ptr())) {
    const at::Tensor t = seq_lens.cast<at::Tensor>().to(at::kCPU).to(at::kLong).contiguous();
    TORCH_CHECK(t.dim() == 1, "seq_lens must be an int or a 1-D list of per-sequence lengths");
    lens.assign(t.data_ptr<int64_t>(), t.data_ptr<int64_t>() + t.numel());
  } else {
    lens = seq_lens.cast<std::vector<int64_t>>();
  }
  TORCH_CHECK(static_cast<int64_t>(lens.size()) == B, "seq_lens must be an int or have one entry per sequence (", B,
              ")");
  int64_t max_len = 0;
  for (const int64_t l : lens) {
    TORCH_CHECK(l > 0, "valid_len must be > 0; got ", l);
    TORCH_CHECK(l <= capacity, "seq_lens exceeds the block table's capacity: ", l, " > ", capacity);
    max_len = std::max(max_len, l);
  }
  TORCH_CHECK(D == 128, "This build supports only D=128. Got D=", D);
  TORCH_CHECK(KVH > 0 && H % KVH == 0, "H must be divisible by KVH. Got H=", H, " KVH=", KVH);
  const int GH = H / KVH;
  TORCH_CHECK(GH == 4 || GH == 8, "This build supports only GH=4 or GH=8 (H/KVH). Got GH=", GH, " (H=", H,
              " KVH=", KVH, ")");
  int L = 0, bn = 0, T_c = 0, S_pt = 0;
  int rc = santa_flash_plan(max_len, max_len, block_n, S, &L, &bn, &T_c, &S_pt);
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  TORCH_CHECK(reinterpret_cast<uintptr_t>(K_pages.data_ptr()) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(V_pages.data_ptr()) % 16 == 0,
              "K_pages/V_pages storage must be 16-byte aligned");
  c10::DeviceGuard guard(q_h.device());
  const at::Tensor q = aligned_q(q_h);
  long long total = 0;
  std::vector<int32_t> host(lens.size());
  for (size_t b = 0; b < lens.size(); ++b) {
    host[b] = static_cast<int32_t>(lens[b]);
    total += (lens[b] + bn - 1) / bn;
  }
  at::Tensor dlens = to_device_async(host, q.device());
  auto optsF = q.options().dtype(at::kFloat);
  auto optsI = q.options().dtype(at::kInt);
  at::Tensor out = at::empty({B, H, D}, q.options());
  at::Tensor m_star = at::empty({B, H}, optsF);
  at::Tensor vrows = want_vrows ? at::empty({B, KVH}, optsI) : at::empty({0}, optsI);
  const size_t ws_bytes = santa_flash_ragged_workspace_size(B, H, KVH, D, T_c, total);
  at::Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  const int dtype = (q.scalar_type() == at::kBFloat16) ? SANTA_BF16 : SANTA_F16;
  rc = santa_flash_decode_paged(q.data_ptr(), K_pages.data_ptr(), V_pages.data_ptr(), dtype, B, H, KVH, D, num_pages,
                                page_size, block_table.data_ptr<int>(), stride, dlens.data_ptr<int>(),
                                static_cast<int>(max_len), total, bn, S, seed, out.data_ptr(),
                                m_star.data_ptr<float>(), want_vrows ? vrows.data_ptr<int>() : nullptr, ws.data_ptr(),
                                ws_bytes, current_stream(q));
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  return std::make_tuple(out, m_star, vrows);
}

// Test-only: the per-tile statistics behind one decode call.
// Returns (m_tiles [B,H,T_c], ell_tiles [B,H,T_c], counts [B,H,T_c,block_n] i16,
//          out_tiles [B,H,T_c,D] f32, emit_cnt [B,KVH,T_c] i32).
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> debug_tiles(
    at::Tensor q_h, at::Tensor K_g, at::Tensor V_g, int64_t S, uint64_t seed, int64_t block_n, int64_t valid_len) {
  const Plan p = plan_call(q_h, K_g, V_g, S, block_n, valid_len);
  c10::DeviceGuard guard(q_h.device());
  const at::Tensor q = aligned_q(q_h);
  const ShapeInfo& in = p.info;
  auto optsF = q.options().dtype(at::kFloat);
  at::Tensor m_tiles = at::empty({in.B, in.H, p.T_c}, optsF);
  at::Tensor ell_tiles = at::empty({in.B, in.H, p.T_c}, optsF);
  at::Tensor counts = at::empty({in.B, in.H, p.T_c, p.bn}, q.options().dtype(at::kShort));
  at::Tensor out_tiles = at::empty({in.B, in.H, p.T_c, in.D}, optsF);
  at::Tensor emit = at::empty({in.B, in.KVH, p.T_c}, q.options().dtype(at::kInt));
  const int rc = santa_flash_fused_tiles(q.data_ptr(), K_g.data_ptr(), V_g.data_ptr(), p.dtype, in.B, in.H, in.KVH,
                                         in.D, p.L, in.L_storage, p.bn, p.S_pt, seed, m_tiles.data_ptr<float>(),
                                         ell_tiles.data_ptr<float>(), out_tiles.data_ptr<float>(),
                                         emit.data_ptr<int>(), counts.data_ptr<int16_t>(), current_stream(q));
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  return std::make_tuple(m_tiles, ell_tiles, counts, out_tiles, emit);
}

// Test-only: the block_n = 256 production tile pass (the wave kernel) with
// its per-tile statistics written out.  Returns (m_tiles [B,H,T_c],
// ell_tiles, counts [B,H,T_c,256] i16).
std::tuple<at::Tensor, at::Tensor, at::Tensor> debug_wave(at::Tensor q_h, at::Tensor K_g, at::Tensor V_g, int64_t S,
                                                          uint64_t seed, int64_t valid_len) {
  const Plan p = plan_call(q_h, K_g, V_g, S, 256, valid_len);
  c10::DeviceGuard guard(q_h.device());
  const at::Tensor q = aligned_q(q_h);
  const ShapeInfo& in = p.info;
  auto optsF = q.options().dtype(at::kFloat);
  at::Tensor m_tiles = at::empty({in.B, in.H, p.T_c}, optsF);
  at::Tensor ell_tiles = at::empty({in.B, in.H, p.T_c}, optsF);
  at::Tensor counts = at::empty({in.B, in.H, p.T_c, 256}, q.options().dtype(at::kShort));
  const size_t ws_bytes = santa_flash_workspace_size(in.B, in.H, in.KVH, in.D, p.T_c);
  at::Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  const hipError_t e = santa::flash::launch_wave_debug(q.data_ptr(), K_g.data_ptr(), V_g.data_ptr(), p.dtype, in.B,
                                                       in.H, in.KVH, p.L, in.L_storage, p.S_pt, seed, ws.data_ptr(),
                                                       m_tiles.data_ptr<float>(), ell_tiles.data_ptr<float>(),
                                                       counts.data_ptr<int16_t>(), current_stream(q));
  TORCH_CHECK(e == hipSuccess, "wave kernel launch failed: ", hipGetErrorString(e));
  return std::make_tuple(m_tiles, ell_tiles, counts);
}

// Test-only: the reference-structured launch pair (per-tile partials, then
// the finalize with the reference's merge association).  Returns the same
// tuple as decode_systematic_scalar.
std::tuple<at::Tensor, at::Tensor, at::Tensor> decode_reference_order(at::Tensor q_h, at::Tensor K_g, at::Tensor V_g,
                                                                      int64_t S, uint64_t seed, int64_t block_n,
                                                                      bool want_vrows, int64_t valid_len) {
  const Plan p = plan_call(q_h, K_g, V_g, S, block_n, valid_len);
  c10::DeviceGuard guard(q_h.device());
  const at::Tensor q = aligned_q(q_h);
  const ShapeInfo& in = p.info;
  auto optsF = q.options().dtype(at::kFloat);
  auto optsI = q.options().dtype(at::kInt);
  at::Tensor m_tiles = at::empty({in.B, in.H, p.T_c}, optsF);
  at::Tensor ell_tiles = at::empty({in.B, in.H, p.T_c}, optsF);
  at::Tensor out_tiles = at::empty({in.B, in.H, p.T_c, in.D}, optsF);
  at::Tensor emit = at::empty({in.B, in.KVH, p.T_c}, optsI);
  hipStream_t st = current_stream(q);
  int rc = santa_flash_fused_tiles(q.data_ptr(), K_g.data_ptr(), V_g.data_ptr(), p.dtype, in.B, in.H, in.KVH, in.D, p.L,
                                   in.L_storage, p.bn, p.S_pt, seed, m_tiles.data_ptr<float>(),
                                   ell_tiles.data_ptr<float>(), out_tiles.data_ptr<float>(), emit.data_ptr<int>(),
                                   nullptr, st);
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  at::Tensor out = in.batched ? at::empty({in.B, in.H, in.D}, q.options()) : at::empty({in.H, in.D}, q.options());
  at::Tensor m_star = in.batched ? at::empty({in.B, in.H}, optsF) : at::empty({in.H}, optsF);
  at::Tensor vrows = at::empty({0}, optsI);
  if (want_vrows) vrows = in.batched ? at::empty({in.B, in.KVH}, optsI) : at::empty({in.KVH}, optsI);
  rc = santa_flash_finalize(m_tiles.data_ptr<float>(), ell_tiles.data_ptr<float>(), out_tiles.data_ptr<float>(),
                            emit.data_ptr<int>(), p.dtype, in.B, in.H, in.KVH, in.D, p.T_c, p.S_pt, out.data_ptr(),
                            m_star.data_ptr<float>(), want_vrows ? vrows.data_ptr<int>() : nullptr, st);
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
  return std::make_tuple(out, m_star, vrows);
}

// Bench-only: the production tile pass alone (chunk partials into `ws`,
// a uint8 tensor of at least santa_flash_workspace_size bytes).
void decode_tiles_only(at::Tensor q_h, at::Tensor K_g, at::Tensor V_g, int64_t S, uint64_t seed, int64_t block_n,
                       int64_t valid_len, at::Tensor ws) {
  const Plan p = plan_call(q_h, K_g, V_g, S, block_n, valid_len);
  c10::DeviceGuard guard(q_h.device());
  const at::Tensor q = aligned_q(q_h);
  const ShapeInfo& in = p.info;
  TORCH_CHECK(ws.is_cuda() && ws.scalar_type() == at::kByte && ws.is_contiguous(), "ws must be a CUDA uint8 tensor");
  const int rc = santa_flash_decode_tiles(q.data_ptr(), K_g.data_ptr(), V_g.data_ptr(), p.dtype, in.B, in.H, in.KVH,
                                          in.D, p.L, in.L_storage, p.bn, p.S_pt, seed, ws.data_ptr(),
                                          static_cast<size_t>(ws.numel()), current_stream(q));
  TORCH_CHECK(rc == SANTA_OK, santa_last_error());
}

// Test-only: the kernels' exponential applied to a float32 CUDA tensor.
at::Tensor device_expf(at::Tensor x) {
  TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kFloat, "x must be a CUDA float32 tensor");
  c10::DeviceGuard guard(x.device());
  at::Tensor xc = x.contiguous();
  at::Tensor y = at::empty_like(xc);
  const hipError_t e = santa::flash::launch_expf(xc.data_ptr<float>(), y.data_ptr<float>(),
                                                 static_cast<size_t>(xc.numel()), current_stream(xc));
  TORCH_CHECK(e == hipSuccess, "expf launch failed: ", hipGetErrorString(e));
  return y;
}

// Test-only: the score path's broadcast MFMA and fmaf on the same operands;
// a, b [n, 64], c [n, 64, 4] float32 CUDA tensors -> (mfma, fma) [n, 16, 64, 4].
std::tuple<at::Tensor, at::Tensor> mfma_fma_check(at::Tensor a, at::Tensor b, at::Tensor c) {
  TORCH_CHECK(a.is_cuda() && a.scalar_type() == at::kFloat && a.dim() == 2 && a.size(1) == 64,
              "a must be a CUDA float32 tensor [n, 64]");
  TORCH_CHECK(b.is_cuda() && b.scalar_type() == at::kFloat && b.sizes() == a.sizes(), "b must match a");
  TORCH_CHECK(c.is_cuda() && c.scalar_type() == at::kFloat && c.dim() == 3 && c.size(0) == a.size(0) &&
                  c.size(1) == 64 && c.size(2) == 4,
              "c must be a CUDA float32 tensor [n, 64, 4]");
  c10::DeviceGuard guard(a.device());
  const at::Tensor ac = a.contiguous(), bc = b.contiguous(), cc = c.contiguous();
  at::Tensor mo = at::empty({a.size(0), 16, 64, 4}, a.options());
  at::Tensor fo = at::empty_like(mo);
  const hipError_t e = santa::flash::launch_mfma_check(ac.data_ptr<float>(), bc.data_ptr<float>(),
                                                       cc.data_ptr<float>(), mo.data_ptr<float>(),
                                                       fo.data_ptr<float>(), static_cast<int>(a.size(0)),
                                                       current_stream(ac));
  TORCH_CHECK(e == hipSuccess, "mfma check launch failed: ", hipGetErrorString(e));
  return {mo, fo};
}

// The kernel santa_flash_decode_tiles runs for this shape (bench label).
std::string tile_pass_kernel(int64_t B, int64_t H, int64_t KVH, int64_t T_c, int64_t block_n) {
  TORCH_CHECK(B > 0 && H > 0 && KVH > 0 && H % KVH == 0 && T_c > 0, "bad shape");
  const std::string gh = "GH " + std::to_string(H / KVH);
  if (block_n == 256 && !santa::flash::uniform_small_pass(static_cast<int>(B), static_cast<int>(KVH),
                                                         static_cast<int>(T_c), static_cast<int>(H / KVH)))
    return "santa::flash::wave_kernel (block_n 256, " + gh +
           (santa::flash::rows_layout(static_cast<int>(KVH)) ? ", rows layout)" : ", four-wave layout)");
  return "santa::flash::tile_kernel (block_n " + std::to_string(block_n) + ", " + gh + ", online)";
}

int64_t workspace_bytes(int64_t B, int64_t H, int64_t KVH, int64_t D, int64_t T_c) {
  return static_cast<int64_t>(santa_flash_workspace_size(static_cast<int>(B), static_cast<int>(H),
                                                         static_cast<int>(KVH), static_cast<int>(D),
                                                         static_cast<int>(T_c)));
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "S^2ANTA-Flash sampled-attention decode for MI355X (gfx950)";
  m.def("decode_systematic_scalar", &decode_systematic_scalar, py::arg("q_h"), py::arg("K_g"), py::arg("V_g"),
        py::arg("S"), py::arg("seed") = 42ULL, py::arg("block_n") = 0, py::arg("want_vrows") = false,
        py::arg("valid_len") = py::int_(-1));
  m.def("decode_systematic_batched", &decode_systematic_scalar, py::arg("q_h"), py::arg("K_g"), py::arg("V_g"),
        py::arg("S"), py::arg("seed") = 42ULL, py::arg("block_n") = 0, py::arg("want_vrows") = false,
        py::arg("valid_len") = py::int_(-1));
  m.def("decode_systematic_paged", &decode_paged, py::arg("q_h"), py::arg("K_pages"), py::arg("V_pages"),
        py::arg("block_table"), py::arg("seq_lens"), py::arg("S"), py::arg("seed") = 42ULL, py::arg("block_n") = 0,
        py::arg("want_vrows") = false);
  m.def("_debug_tiles", &debug_tiles, py::arg("q_h"), py::arg("K_g"), py::arg("V_g"), py::arg("S"),
        py::arg("seed") = 42ULL, py::arg("block_n") = 0, py::arg("valid_len") = -1);
  m.def("_debug_wave", &debug_wave, py::arg("q_h"), py::arg("K_g"), py::arg("V_g"), py::arg("S"),
        py::arg("seed") = 42ULL, py::arg("valid_len") = -1);
  m.def("_decode_reference_order", &decode_reference_order, py::arg("q_h"), py::arg("K_g"), py::arg("V_g"),
        py::arg("S"), py::arg("seed") = 42ULL, py::arg("block_n") = 0, py::arg("want_vrows") = false,
        py::arg("valid_len") = -1);
  m.def("_decode_tiles_only", &decode_tiles_only, py::arg("q_h"), py::arg("K_g"), py::arg("V_g"), py::arg("S"),
        py::arg("seed"), py::arg("block_n"), py::arg("valid_len"), py::arg("ws"));
  m.def("_workspace_bytes", &workspace_bytes);
  m.def("_tile_pass_kernel", &tile_pass_kernel, py::arg("B"), py::arg("H"), py::arg("KVH"), py::arg("T_c"),
        py::arg("block_n"));
  m.def("_device_expf", &device_expf, py::arg("x"));
  m.def("_mfma_fma_check", &mfma_fma_check, py::arg("a"), py::arg("b"), py::arg("c"));
  m.def("_library_version", []() { return std::string(santa_version()); });
}
