// pa_torch.cpp - thin PyTorch-ROCm binding over the C ABI in pa_decode.h.
//
// Mirrors the reference's pybind11 module (cuda/binding.cpp:3-15), whose
// `forward_v4` entry called paged_attn_decode_cuda_v4_launch
// (cuda/kernel_v4_split_k.cu:205-268).  This file holds no kernels: it reads
// shapes, strides and data pointers from the tensors, allocates the output
// from PyTorch's caching allocator, and calls
// pad_decode_launch_ex() (dense table), pad_decode_launch_kv8() (dense
// table, fp8 caches) or pad_decode_launch_call() (CSR index, work lists) on
// PyTorch's current HIP stream of q's device, with persistent split scratch
// (workspace + arrival counters) per (device, stream).
// plan_worklist / plan_worklist_csr and forward_worklist / forward_worklist_csr
// split a decode into a plan (once per decode step) and runs (once per
// layer) over pad_decode_plan_worklist_call / pad_decode_launch_call.  The
// CSR and work-list entries take fp16 or fp8 (e4m3fn / e5m2) caches.
// Argument errors surface as RuntimeError (the reference used TORCH_CHECK,
// cuda/kernel_v4_split_k.cu:216-223).  No host synchronisation.

#include <torch/extension.h>

#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <climits>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "pa_decode.h"

namespace {

int cached_cus(int device) {
  static int cus[64] = {0};
  if (device < 0 || device >= 64) return 256;
  if (cus[device] <= 0) {
    int n = 0;
    if (pad_device_num_cus(&n) != PAD_OK || n <= 0) n = 256;
    cus[device] = n;
  }
  return cus[device];
}

// Per (device, stream) scratch kept across calls: the fp32 partial
// workspace (no state between launches) and the int32 arrival counters,
// which start at zero and are left at zero by every launch.  Launches on one
// stream are ordered, so reusing both on their stream is safe.  When a call
// needs more, a buffer of at least twice the size replaces it (counters
// zero-filled, on the same stream), and the replaced buffer is kept alive
// for the rest of the process: a HIP graph captured earlier on this stream
// holds its raw address and writes partials and counters there on every
// replay, so returning it to the caching allocator would let those replays
// corrupt whatever tensor got the memory next.  Growth can therefore never
// happen during stream capture (the new buffer would also come from the
// capture's private pool); such a call raises, and one eager call of the
// largest shape on the capturing stream beforehand sizes the scratch.
struct StreamScratch {
  torch::Tensor workspace;
  torch::Tensor counters;
  std::vector<torch::Tensor> retired;  // replaced buffers, still referenced by captured graphs
};

bool stream_capturing(hipStream_t stream) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(stream, &status);
  TORCH_CHECK(e == hipSuccess, "pa_decode: hipStreamIsCapturing failed: ", hipGetErrorString(e));
  return status != hipStreamCaptureStatusNone;
}

StreamScratch& stream_scratch(const torch::Tensor& like, hipStream_t stream, size_t ws_bytes,
                              int64_t num_counters) {
  static std::mutex mu;
  static std::map<std::pair<int, uintptr_t>, StreamScratch> cache;
  std::lock_guard<std::mutex> lock(mu);
  StreamScratch& sc = cache[{like.get_device(), reinterpret_cast<uintptr_t>(stream)}];
  const bool grow_ws = !sc.workspace.defined() || static_cast<size_t>(sc.workspace.numel()) < ws_bytes;
  const bool grow_cnt = !sc.counters.defined() || sc.counters.numel() < num_counters;
  if ((grow_ws || grow_cnt) && stream_capturing(stream)) {
    TORCH_CHECK(false,
                "pa_decode: this call needs more split scratch than the capturing stream holds, and scratch "
                "cannot grow during HIP graph capture (a captured graph keeps the addresses it was captured "
                "with). Run one eager call with the largest shape on the capture stream before capturing.");
  }
  if (grow_ws) {
    const size_t old = sc.workspace.defined() ? static_cast<size_t>(sc.workspace.numel()) : 0;
    const size_t want = ws_bytes > 2 * old ? ws_bytes : 2 * old;
    const int64_t grown = static_cast<int64_t>(((want + (1u << 20) - 1) >> 20) << 20);
    if (sc.workspace.defined()) sc.retired.push_back(sc.workspace);
    sc.workspace = torch::empty({grown}, like.options().dtype(at::kByte));
  }
  if (grow_cnt) {
    const int64_t old = sc.counters.defined() ? sc.counters.numel() : 0;
    const int64_t want = num_counters > 2 * old ? num_counters : 2 * old;
    const int64_t grown = ((want + 4095) / 4096) * 4096;
    if (sc.counters.defined()) sc.retired.push_back(sc.counters);
    sc.counters = torch::zeros({grown}, like.options().dtype(at::kInt));
  }
  return sc;
}

void fill_dims(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
               const torch::Tensor& bt, const torch::Tensor& sl, const torch::Tensor& out,
               pad_decode_dims* d) {
  d->batch = static_cast<int32_t>(q.size(0));
  d->num_q_heads = static_cast<int32_t>(q.size(1));
  d->head_dim = static_cast<int32_t>(q.size(2));
  d->num_pages = k.size(0);
  d->page_size = static_cast<int32_t>(k.size(1));
  d->num_kv_heads = static_cast<int32_t>(k.size(2));
  d->max_pages = static_cast<int32_t>(bt.size(1));
  for (int i = 0; i < 3; ++i) d->q_stride[i] = q.stride(i);
  for (int i = 0; i < 4; ++i) {
    d->k_stride[i] = k.stride(i);
    d->v_stride[i] = v.stride(i);
  }
  d->bt_stride[0] = bt.stride(0);
  d->bt_stride[1] = bt.stride(1);
  d->sl_stride = sl.stride(0);
  for (int i = 0; i < 3; ++i) d->out_stride[i] = out.stride(i);
}

// Checks shared by the dense-table entries (dtypes are cache_format()'s).
void check_dense(const torch::Tensor& q, const torch::Tensor& k_cache, const torch::Tensor& v_cache,
                 const torch::Tensor& block_table, const torch::Tensor& seq_lens) {
  TORCH_CHECK(q.is_cuda() && k_cache.is_cuda() && v_cache.is_cuda() && block_table.is_cuda() &&
                  seq_lens.is_cuda(),
              "pa_decode: all tensors must be on the GPU");
  TORCH_CHECK(q.device() == k_cache.device() && q.device() == v_cache.device() &&
                  q.device() == block_table.device() && q.device() == seq_lens.device(),
              "pa_decode: all tensors must be on the same device");
  TORCH_CHECK(block_table.scalar_type() == at::kInt && seq_lens.scalar_type() == at::kInt,
              "pa_decode: block_table and seq_lens must be int32");
  TORCH_CHECK(q.dim() == 3, "pa_decode: q must be [batch, num_q_heads, head_dim]");
  TORCH_CHECK(k_cache.dim() == 4, "pa_decode: k_cache must be [num_pages, page_size, num_kv_heads, head_dim]");
  TORCH_CHECK(v_cache.sizes() == k_cache.sizes(), "pa_decode: v_cache shape must match k_cache");
  TORCH_CHECK(block_table.dim() == 2 && block_table.size(0) == q.size(0),
              "pa_decode: block_table must be [batch, max_pages]");
  TORCH_CHECK(seq_lens.dim() == 1 && seq_lens.size(0) == q.size(0), "pa_decode: seq_lens must be [batch]");
  TORCH_CHECK(k_cache.size(3) == q.size(2), "pa_decode: q head_dim must match the KV cache head_dim");
}

// PAD_KV_* format of a call: float16 q with float16 or fp8 (float8_e4m3fn /
// float8_e5m2) caches, or bfloat16 q with bfloat16 or fp8 caches; k_cache
// and v_cache alike.  The output has q's dtype.
int cache_format(const torch::Tensor& q, const torch::Tensor& k_cache, const torch::Tensor& v_cache) {
  const at::ScalarType kt = k_cache.scalar_type();
  TORCH_CHECK(v_cache.scalar_type() == kt, "pa_decode: k_cache and v_cache must have the same dtype");
  if (q.scalar_type() == at::kBFloat16) {
    if (kt == at::kBFloat16) return PAD_KV_BF16;
    if (kt == at::kFloat8_e4m3fn) return PAD_KV_FP8_E4M3FN_BF16;
    if (kt == at::kFloat8_e5m2) return PAD_KV_FP8_E5M2_BF16;
    TORCH_CHECK(false, "pa_decode: with bfloat16 q, k_cache and v_cache must be bfloat16, float8_e4m3fn or "
                       "float8_e5m2");
  }
  TORCH_CHECK(q.scalar_type() == at::kHalf, "pa_decode: q must be float16 or bfloat16");
  if (kt == at::kHalf) return PAD_KV_FP16;
  if (kt == at::kFloat8_e4m3fn) return PAD_KV_FP8_E4M3FN;
  if (kt == at::kFloat8_e5m2) return PAD_KV_FP8_E5M2;
  TORCH_CHECK(false, "pa_decode: with float16 q, k_cache and v_cache must be float16, float8_e4m3fn or float8_e5m2");
  return PAD_KV_FP16;
}

// The page index of one launch: dense (block_table, seq_lens) or CSR
// (indices, indptr, last_page_len), as raw pointers.
struct PageIndex {
  const int32_t* ids = nullptr;  // block_table, or CSR indices
  const int32_t* seq_lens = nullptr;
  const int32_t* indptr = nullptr;
  const int32_t* last_page_len = nullptr;
};

PageIndex dense_index(const torch::Tensor& block_table, const torch::Tensor& seq_lens) {
  PageIndex ix;
  ix.ids = block_table.data_ptr<int32_t>();
  ix.seq_lens = seq_lens.data_ptr<int32_t>();
  return ix;
}

PageIndex csr_index(const torch::Tensor& indptr, const torch::Tensor& indices, const torch::Tensor& last_page_len) {
  PageIndex ix;
  ix.ids = indices.data_ptr<int32_t>();
  ix.indptr = indptr.data_ptr<int32_t>();
  ix.last_page_len = last_page_len.data_ptr<int32_t>();
  return ix;
}

// The dims of a CSR launch: fill_dims() with `indices` as a one-row table
// whose width is the number of entries.
void csr_dims(const torch::Tensor& q, const torch::Tensor& k_cache, const torch::Tensor& v_cache,
              const torch::Tensor& indices, const torch::Tensor& last_page_len, const torch::Tensor& out,
              pad_decode_dims* d) {
  fill_dims(q, k_cache, v_cache, indices.view({1, -1}), last_page_len, out, d);
  d->max_pages = static_cast<int32_t>(indices.size(0));
  d->bt_stride[0] = 0;
  d->bt_stride[1] = 1;
}

// One launch through pad_decode_launch_call() on PyTorch's current stream of
// q's device, with that stream's split scratch sized by the dense (or CSR)
// plan of d.  worklist may be undefined (plan in the kernel).
torch::Tensor launch_call(const torch::Tensor& q, const torch::Tensor& k_cache, const torch::Tensor& v_cache,
                          const torch::Tensor& out, const pad_decode_dims& d, const PageIndex& ix,
                          const torch::Tensor& worklist, double scale, int64_t num_splits, int64_t engine,
                          int kv_format, double k_scale, double v_scale) {
  const bool csr = ix.indptr != nullptr;
  pad_decode_plan_t plan;
  const int cus = cached_cus(q.get_device());
  int st = csr ? pad_decode_plan_csr(&d, static_cast<int>(num_splits), cus, &plan)
               : pad_decode_plan(&d, static_cast<int>(num_splits), cus, &plan);
  TORCH_CHECK(st == PAD_OK, "pa_decode: ", pad_status_string(st));
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.get_device()).stream();
  pad_decode_call c;
  std::memset(&c, 0, sizeof(c));
  c.q = q.data_ptr();
  c.k_cache = k_cache.data_ptr();
  c.v_cache = v_cache.data_ptr();
  c.block_table = ix.ids;
  c.seq_lens = ix.seq_lens;
  c.indptr = ix.indptr;
  c.last_page_len = ix.last_page_len;
  c.out = out.data_ptr();
  if (!plan.single_pass) {
    StreamScratch& sc = stream_scratch(q, stream, plan.workspace_bytes, plan.counters);
    c.workspace = sc.workspace.data_ptr();
    c.workspace_bytes = plan.workspace_bytes;
    c.counters = sc.counters.data_ptr<int32_t>();
    c.num_counters = plan.counters;
  }
  if (worklist.defined()) {
    c.worklist = worklist.data_ptr();
    c.worklist_bytes = static_cast<size_t>(worklist.numel());
  }
  c.scale = static_cast<float>(scale);
  c.num_splits = static_cast<int32_t>(num_splits);
  c.engine = static_cast<int32_t>(engine);
  c.kv_format = kv_format;
  c.k_scale = static_cast<float>(k_scale);
  c.v_scale = static_cast<float>(v_scale);
  st = pad_decode_launch_call(&c, &d, stream);
  TORCH_CHECK(st == PAD_OK, "pa_decode: ", pad_status_string(st));
  return out;
}

// Decode over a dense block table: float16 (either engine), bfloat16 q and
// caches (MFMA engine), or float16 q with fp8 caches at unit scales (see
// forward_kv8 for scales).
torch::Tensor forward(torch::Tensor q, torch::Tensor k_cache, torch::Tensor v_cache,
                      torch::Tensor block_table, torch::Tensor seq_lens, double scale,
                      int64_t num_splits, int64_t engine) {
  const int fmt = cache_format(q, k_cache, v_cache);
  check_dense(q, k_cache, v_cache, block_table, seq_lens);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = torch::empty({q.size(0), q.size(1), q.size(2)}, q.options());
  pad_decode_dims d;
  fill_dims(q, k_cache, v_cache, block_table, seq_lens, out, &d);
  if (fmt != PAD_KV_FP16)
    return launch_call(q, k_cache, v_cache, out, d, dense_index(block_table, seq_lens), torch::Tensor(), scale,
                       num_splits, engine, fmt, 1.0, 1.0);

  const int cus = cached_cus(q.get_device());
  pad_decode_plan_t plan;
  int st = pad_decode_plan(&d, static_cast<int>(num_splits), cus, &plan);
  TORCH_CHECK(st == PAD_OK, "pa_decode: ", pad_status_string(st));
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.get_device()).stream();
  void* ws_ptr = nullptr;
  int32_t* counters = nullptr;
  if (!plan.single_pass) {
    StreamScratch& sc = stream_scratch(q, stream, plan.workspace_bytes, plan.counters);
    ws_ptr = sc.workspace.data_ptr();
    counters = sc.counters.data_ptr<int32_t>();
  }
  st = pad_decode_launch_ex(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                            block_table.data_ptr<int32_t>(), seq_lens.data_ptr<int32_t>(), out.data_ptr(),
                            ws_ptr, plan.workspace_bytes, counters, plan.counters, &d, static_cast<float>(scale),
                            static_cast<int>(num_splits), static_cast<int>(engine), nullptr, stream);
  TORCH_CHECK(st == PAD_OK, "pa_decode: ", pad_status_string(st));
  return out;
}

// Decode over fp8 caches (torch.float8_e4m3fn or torch.float8_e5m2, both
// caches the same) holding K / k_scale and V / v_scale; q and the output
// are float16 or bfloat16.  Same plan, scratch and stream as forward().
torch::Tensor forward_kv8(torch::Tensor q, torch::Tensor k_cache, torch::Tensor v_cache,
                          torch::Tensor block_table, torch::Tensor seq_lens, double scale, double k_scale,
                          double v_scale, int64_t num_splits) {
  const at::ScalarType kt = k_cache.scalar_type();
  TORCH_CHECK(kt == at::kFloat8_e4m3fn || kt == at::kFloat8_e5m2,
              "pa_decode: forward_kv8 needs float8_e4m3fn or float8_e5m2 caches");
  const int fmt = cache_format(q, k_cache, v_cache);
  check_dense(q, k_cache, v_cache, block_table, seq_lens);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = torch::empty({q.size(0), q.size(1), q.size(2)}, q.options());
  pad_decode_dims d;
  fill_dims(q, k_cache, v_cache, block_table, seq_lens, out, &d);

  const int cus = cached_cus(q.get_device());
  pad_decode_plan_t plan;
  int st = pad_decode_plan(&d, static_cast<int>(num_splits), cus, &plan);
  TORCH_CHECK(st == PAD_OK, "pa_decode: ", pad_status_string(st));
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.get_device()).stream();
  void* ws_ptr = nullptr;
  int32_t* counters = nullptr;
  if (!plan.single_pass) {
    StreamScratch& sc = stream_scratch(q, stream, plan.workspace_bytes, plan.counters);
    ws_ptr = sc.workspace.data_ptr();
    counters = sc.counters.data_ptr<int32_t>();
  }
  st = pad_decode_launch_kv8(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                             block_table.data_ptr<int32_t>(), seq_lens.data_ptr<int32_t>(), out.data_ptr(),
                             ws_ptr, plan.workspace_bytes, counters, plan.counters, &d, static_cast<float>(scale),
                             fmt, static_cast<float>(k_scale), static_cast<float>(v_scale),
                             static_cast<int>(num_splits), stream);
  TORCH_CHECK(st == PAD_OK, "pa_decode: ", pad_status_string(st));
  return out;
}

// Checks of the CSR entries: q, caches and the (indptr, indices,
// last_page_len) triple on one GPU, int32, contiguous, sized by q's batch.
void check_csr(const torch::Tensor& q, const torch::Tensor& k_cache, const torch::Tensor& v_cache,
               const torch::Tensor& indptr, const torch::Tensor& indices, const torch::Tensor& last_page_len) {
  TORCH_CHECK(q.is_cuda() && k_cache.is_cuda() && v_cache.is_cuda() && indptr.is_cuda() && indices.is_cuda() &&
                  last_page_len.is_cuda(),
              "pa_decode: all tensors must be on the GPU");
  TORCH_CHECK(q.device() == k_cache.device() && q.device() == v_cache.device() && q.device() == indptr.device() &&
                  q.device() == indices.device() && q.device() == last_page_len.device(),
              "pa_decode: all tensors must be on the same device");
  TORCH_CHECK(indptr.scalar_type() == at::kInt && indices.scalar_type() == at::kInt &&
                  last_page_len.scalar_type() == at::kInt,
              "pa_decode: indptr, indices and last_page_len must be int32");
  TORCH_CHECK(q.dim() == 3, "pa_decode: q must be [batch, num_q_heads, head_dim]");
  TORCH_CHECK(k_cache.dim() == 4, "pa_decode: k_cache must be [num_pages, page_size, num_kv_heads, head_dim]");
  TORCH_CHECK(v_cache.sizes() == k_cache.sizes(), "pa_decode: v_cache shape must match k_cache");
  TORCH_CHECK(indptr.dim() == 1 && indptr.size(0) == q.size(0) + 1, "pa_decode: indptr must be [batch + 1]");
  TORCH_CHECK(last_page_len.dim() == 1 && last_page_len.size(0) == q.size(0),
              "pa_decode: last_page_len must be [batch]");
  TORCH_CHECK(indices.dim() == 1 && indices.is_contiguous() && indptr.is_contiguous() &&
                  last_page_len.is_contiguous(),
              "pa_decode: indptr, indices and last_page_len must be contiguous 1-D tensors");
  TORCH_CHECK(indices.size(0) <= INT32_MAX, "pa_decode: too many page ids");
  TORCH_CHECK(k_cache.size(3) == q.size(2), "pa_decode: q head_dim must match the KV cache head_dim");
}

void check_worklist(const torch::Tensor& q, const torch::Tensor& worklist) {
  TORCH_CHECK(worklist.is_cuda() && worklist.device() == q.device() && worklist.scalar_type() == at::kByte &&
                  worklist.is_contiguous(),
              "pa_decode: worklist must be a contiguous uint8 tensor on q's device");
}

// Decode with a CSR page index: the page ids of sequence b are
// indices[indptr[b] : indptr[b+1]] and its last page holds last_page_len[b]
// tokens (the (indptr, indices, last_page_len) triple the reference's
// FlashInfer adapter builds, src/flashinfer_adapter.py:40-65).  fp16 or fp8
// caches (k_scale / v_scale are read for fp8 only).
torch::Tensor forward_csr(torch::Tensor q, torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor indptr,
                          torch::Tensor indices, torch::Tensor last_page_len, double scale, int64_t num_splits,
                          int64_t engine, double k_scale, double v_scale) {
  const int fmt = cache_format(q, k_cache, v_cache);
  check_csr(q, k_cache, v_cache, indptr, indices, last_page_len);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = torch::empty({q.size(0), q.size(1), q.size(2)}, q.options());
  pad_decode_dims d;
  csr_dims(q, k_cache, v_cache, indices, last_page_len, out, &d);
  return launch_call(q, k_cache, v_cache, out, d, csr_index(indptr, indices, last_page_len), torch::Tensor(), scale,
                     num_splits, engine, fmt, k_scale, v_scale);
}

// Plan once, run many (pad_decode_plan_worklist_call / pad_decode_launch_call):
// the dims of a decode with these index tensors and head/page geometry.
// q/k/v/out strides do not enter the plan; num_pages only bounds page ids at
// run time, so the plan uses any positive value.
pad_decode_dims worklist_dims(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                              int64_t page_size, int64_t max_pages) {
  pad_decode_dims d;
  std::memset(&d, 0, sizeof(d));
  d.batch = static_cast<int32_t>(batch);
  d.num_q_heads = static_cast<int32_t>(num_q_heads);
  d.num_kv_heads = static_cast<int32_t>(num_kv_heads);
  d.head_dim = static_cast<int32_t>(head_dim);
  d.page_size = static_cast<int32_t>(page_size);
  d.max_pages = static_cast<int32_t>(max_pages);
  d.num_pages = INT64_MAX;
  d.q_stride[2] = d.k_stride[3] = d.v_stride[3] = d.out_stride[2] = 1;
  return d;
}

// Writes the work list of the launch described by d, ix, num_splits and
// kv_format into a new uint8 tensor on `like`'s device (current stream).
torch::Tensor plan_call(const torch::Tensor& like, const pad_decode_dims& d, const PageIndex& ix,
                        int64_t num_splits, int64_t kv_format) {
  c10::hip::HIPGuardMasqueradingAsCUDA guard(like.device());
  const bool csr = ix.indptr != nullptr;
  size_t bytes = 0;
  int st = pad_decode_worklist_bytes(&d, static_cast<int>(num_splits), cached_cus(like.get_device()),
                                     csr ? 1 : 0, &bytes);
  TORCH_CHECK(st == PAD_OK, "pa_decode: ", pad_status_string(st));
  torch::Tensor wl = torch::empty({static_cast<int64_t>(bytes)}, like.options().dtype(at::kByte));
  pad_decode_call c;
  std::memset(&c, 0, sizeof(c));
  c.block_table = ix.ids;
  c.seq_lens = ix.seq_lens;
  c.indptr = ix.indptr;
  c.last_page_len = ix.last_page_len;
  c.num_splits = static_cast<int32_t>(num_splits);
  c.kv_format = static_cast<int32_t>(kv_format);
  c.k_scale = c.v_scale = 1.0f;
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(like.get_device()).stream();
  st = pad_decode_plan_worklist_call(&c, &d, wl.data_ptr(), bytes, stream);
  TORCH_CHECK(st == PAD_OK, "pa_decode: ", pad_status_string(st));
  return wl;
}

// Work list of a dense-table decode (block_table [B, max_pages], seq_lens
// [B], int32 on the GPU) over caches of kv_format (PAD_KV_*).
torch::Tensor plan_worklist(torch::Tensor block_table, torch::Tensor seq_lens, int64_t num_q_heads,
                            int64_t num_kv_heads, int64_t head_dim, int64_t page_size, int64_t num_splits,
                            int64_t kv_format) {
  TORCH_CHECK(block_table.is_cuda() && seq_lens.is_cuda() && block_table.device() == seq_lens.device(),
              "pa_decode: block_table and seq_lens must be on the same GPU");
  TORCH_CHECK(block_table.scalar_type() == at::kInt && seq_lens.scalar_type() == at::kInt,
              "pa_decode: block_table and seq_lens must be int32");
  TORCH_CHECK(block_table.dim() == 2 && seq_lens.dim() == 1 && seq_lens.size(0) == block_table.size(0),
              "pa_decode: block_table must be [batch, max_pages] and seq_lens [batch]");
  pad_decode_dims d = worklist_dims(block_table.size(0), num_q_heads, num_kv_heads, head_dim, page_size,
                                    block_table.size(1));
  d.bt_stride[0] = block_table.stride(0);
  d.bt_stride[1] = block_table.stride(1);
  d.sl_stride = seq_lens.stride(0);
  return plan_call(block_table, d, dense_index(block_table, seq_lens), num_splits, kv_format);
}

// Work list of a CSR decode (indptr [B + 1], indices [nnz], last_page_len
// [B], int32 on the GPU) over caches of kv_format.
torch::Tensor plan_worklist_csr(torch::Tensor indptr, torch::Tensor indices, torch::Tensor last_page_len,
                                int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                                int64_t num_splits, int64_t kv_format) {
  TORCH_CHECK(indptr.is_cuda() && indices.is_cuda() && last_page_len.is_cuda() &&
                  indptr.device() == indices.device() && indptr.device() == last_page_len.device(),
              "pa_decode: indptr, indices and last_page_len must be on the same GPU");
  TORCH_CHECK(indptr.scalar_type() == at::kInt && indices.scalar_type() == at::kInt &&
                  last_page_len.scalar_type() == at::kInt,
              "pa_decode: indptr, indices and last_page_len must be int32");
  TORCH_CHECK(indptr.dim() == 1 && indices.dim() == 1 && last_page_len.dim() == 1 &&
                  indptr.size(0) == last_page_len.size(0) + 1 && indptr.is_contiguous() &&
                  indices.is_contiguous() && last_page_len.is_contiguous(),
              "pa_decode: indptr [batch + 1], indices [nnz] and last_page_len [batch] must be contiguous");
  TORCH_CHECK(indices.size(0) <= INT32_MAX, "pa_decode: too many page ids");
  pad_decode_dims d = worklist_dims(last_page_len.size(0), num_q_heads, num_kv_heads, head_dim, page_size,
                                    indices.size(0));
  d.bt_stride[1] = 1;
  return plan_call(indices, d, csr_index(indptr, indices, last_page_len), num_splits, kv_format);
}

// Decode from a work list (dense table): forward() with engine 0 (or
// forward_kv8() for fp8 caches), plus the list plan_worklist() wrote for the
// same index tensors and cache format.
torch::Tensor forward_worklist(torch::Tensor q, torch::Tensor k_cache, torch::Tensor v_cache,
                               torch::Tensor block_table, torch::Tensor seq_lens, torch::Tensor worklist,
                               double scale, int64_t num_splits, double k_scale, double v_scale) {
  check_worklist(q, worklist);
  const int fmt = cache_format(q, k_cache, v_cache);
  check_dense(q, k_cache, v_cache, block_table, seq_lens);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = torch::empty({q.size(0), q.size(1), q.size(2)}, q.options());
  pad_decode_dims d;
  fill_dims(q, k_cache, v_cache, block_table, seq_lens, out, &d);
  return launch_call(q, k_cache, v_cache, out, d, dense_index(block_table, seq_lens), worklist, scale, num_splits,
                     0, fmt, k_scale, v_scale);
}

// Decode from a work list (CSR index): forward_csr() with engine 0 plus the
// list plan_worklist_csr() wrote for the same index tensors and cache format.
torch::Tensor forward_worklist_csr(torch::Tensor q, torch::Tensor k_cache, torch::Tensor v_cache,
                                   torch::Tensor indptr, torch::Tensor indices, torch::Tensor last_page_len,
                                   torch::Tensor worklist, double scale, int64_t num_splits, double k_scale,
                                   double v_scale) {
  check_worklist(q, worklist);
  const int fmt = cache_format(q, k_cache, v_cache);
  check_csr(q, k_cache, v_cache, indptr, indices, last_page_len);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = torch::empty({q.size(0), q.size(1), q.size(2)}, q.options());
  pad_decode_dims d;
  csr_dims(q, k_cache, v_cache, indices, last_page_len, out, &d);
  return launch_call(q, k_cache, v_cache, out, d, csr_index(indptr, indices, last_page_len), worklist, scale,
                     num_splits, 0, fmt, k_scale, v_scale);
}

// Same argument list as the reference's forward_v4 binding
// (cuda/kernels.h:60-70): gqa_ratio, head_dim and page_size must agree with
// the tensor shapes.
torch::Tensor forward_v4(torch::Tensor q, torch::Tensor k_cache, torch::Tensor v_cache,
                         torch::Tensor block_table, torch::Tensor seq_lens, double scale,
                         int64_t gqa_ratio, int64_t head_dim, int64_t page_size, int64_t num_splits) {
  TORCH_CHECK(q.dim() == 3 && k_cache.dim() == 4, "pa_decode: bad tensor ranks");
  TORCH_CHECK(gqa_ratio >= 1 && gqa_ratio <= PAD_MAX_GQA,
              "pa_decode: gqa_ratio (", gqa_ratio, ") must be in [1, ", PAD_MAX_GQA, "]");
  TORCH_CHECK(q.size(1) == gqa_ratio * k_cache.size(2), "pa_decode: gqa_ratio does not match the head counts");
  TORCH_CHECK(head_dim == q.size(2), "pa_decode: head_dim does not match q");
  TORCH_CHECK(page_size == k_cache.size(1), "pa_decode: page_size does not match k_cache");
  TORCH_CHECK(num_splits >= 1, "pa_decode: num_splits must be >= 1");
  return forward(q, k_cache, v_cache, block_table, seq_lens, scale, num_splits, 0);
}

// The plan the launch would use, as a dict (host only); with `csr`, the plan
// of a CSR launch whose `indices` hold max_pages entries.
py::dict plan(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
              int64_t page_size, int64_t max_pages, int64_t num_splits, int64_t num_cus, bool csr) {
  pad_decode_dims d;
  std::memset(&d, 0, sizeof(d));
  d.batch = static_cast<int32_t>(batch);
  d.num_q_heads = static_cast<int32_t>(num_q_heads);
  d.num_kv_heads = static_cast<int32_t>(num_kv_heads);
  d.head_dim = static_cast<int32_t>(head_dim);
  d.page_size = static_cast<int32_t>(page_size);
  d.max_pages = static_cast<int32_t>(max_pages);
  d.q_stride[2] = d.k_stride[3] = d.v_stride[3] = d.out_stride[2] = 1;
  pad_decode_plan_t p;
  const int st = csr ? pad_decode_plan_csr(&d, static_cast<int>(num_splits), static_cast<int>(num_cus), &p)
                     : pad_decode_plan(&d, static_cast<int>(num_splits), static_cast<int>(num_cus), &p);
  TORCH_CHECK(st == PAD_OK, "pa_decode: ", pad_status_string(st));
  py::dict r;
  r["num_splits"] = p.num_splits;
  r["pages_per_split"] = p.pages_per_split;
  r["waves_per_group"] = p.waves_per_group;
  r["single_pass"] = p.single_pass;
  r["workspace_bytes"] = p.workspace_bytes;
  r["counters"] = p.counters;
  return r;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("forward", &forward, "Paged-attention decode (q, k_cache, v_cache, block_table, seq_lens, scale, "
                             "num_splits, engine) -> out");
  m.def("forward_v4", &forward_v4, "Paged-attention decode with the reference forward_v4 argument list");
  m.def("forward_kv8", &forward_kv8,
        "Paged-attention decode over fp8 caches (q, k_cache, v_cache, block_table, seq_lens, scale, k_scale, "
        "v_scale, num_splits) -> out");
  m.def("forward_csr", &forward_csr,
        "Paged-attention decode over a CSR page index (q, k_cache, v_cache, indptr, indices, last_page_len, "
        "scale, num_splits, engine, k_scale=1, v_scale=1) -> out; fp16 or fp8 caches",
        py::arg("q"), py::arg("k_cache"), py::arg("v_cache"), py::arg("indptr"), py::arg("indices"),
        py::arg("last_page_len"), py::arg("scale"), py::arg("num_splits"), py::arg("engine"),
        py::arg("k_scale") = 1.0, py::arg("v_scale") = 1.0);
  m.def("plan", &plan, "Split plan for the given shapes (host only)");
  m.def("plan_worklist", &plan_worklist,
        "Work list of a dense-table decode (block_table, seq_lens, num_q_heads, num_kv_heads, head_dim, "
        "page_size, num_splits, kv_format=0) -> uint8 tensor",
        py::arg("block_table"), py::arg("seq_lens"), py::arg("num_q_heads"), py::arg("num_kv_heads"),
        py::arg("head_dim"), py::arg("page_size"), py::arg("num_splits"), py::arg("kv_format") = 0);
  m.def("plan_worklist_csr", &plan_worklist_csr,
        "Work list of a CSR decode (indptr, indices, last_page_len, num_q_heads, num_kv_heads, head_dim, "
        "page_size, num_splits, kv_format=0) -> uint8 tensor",
        py::arg("indptr"), py::arg("indices"), py::arg("last_page_len"), py::arg("num_q_heads"),
        py::arg("num_kv_heads"), py::arg("head_dim"), py::arg("page_size"), py::arg("num_splits"),
        py::arg("kv_format") = 0);
  m.def("forward_worklist", &forward_worklist,
        "Decode from a work list (q, k_cache, v_cache, block_table, seq_lens, worklist, scale, num_splits, "
        "k_scale=1, v_scale=1) -> out; fp16 or fp8 caches",
        py::arg("q"), py::arg("k_cache"), py::arg("v_cache"), py::arg("block_table"), py::arg("seq_lens"),
        py::arg("worklist"), py::arg("scale"), py::arg("num_splits"), py::arg("k_scale") = 1.0,
        py::arg("v_scale") = 1.0);
  m.def("forward_worklist_csr", &forward_worklist_csr,
        "Decode from a work list (q, k_cache, v_cache, indptr, indices, last_page_len, worklist, scale, "
        "num_splits, k_scale=1, v_scale=1) -> out; fp16 or fp8 caches",
        py::arg("q"), py::arg("k_cache"), py::arg("v_cache"), py::arg("indptr"), py::arg("indices"),
        py::arg("last_page_len"), py::arg("worklist"), py::arg("scale"), py::arg("num_splits"),
        py::arg("k_scale") = 1.0, py::arg("v_scale") = 1.0);
  m.def("abi_version", &pad_decode_abi_version, "C ABI version of the linked libpa_decode.so");
}
