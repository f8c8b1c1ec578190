// A compiled caller of the C ABI (include/pa_decode.h), as a host program of
// an inference runtime would be: HIP runtime calls for memory and a stream,
// pa_decode.h for the decode, nothing else.  Used by tests/test_capi_consumer.py.
//
//   capi_consumer <input.bin> <output.bin>
//
// input.bin: int64 header {batch, num_q_heads, num_kv_heads, head_dim,
// page_size, max_pages, num_pages, num_splits} then, raw, q (fp16 [batch,
// hq, d]), k_cache and v_cache (fp16 [num_pages, page_size, hkv, d]),
// block_table (int32 [batch, max_pages]) and seq_lens (int32 [batch]).
// output.bin: out (fp16 [batch, hq, d]).  Exit status 0 on success; any
// failing call prints its status string and exits non-zero.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "pa_decode.h"

#define HIP_OK(x)                                                              \
  do {                                                                         \
    hipError_t e_ = (x);                                                       \
    if (e_ != hipSuccess) {                                                    \
      std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));      \
      return 2;                                                                \
    }                                                                          \
  } while (0)

#define PAD_OK_(x)                                                             \
  do {                                                                         \
    int s_ = (x);                                                              \
    if (s_ != PAD_OK) {                                                        \
      std::fprintf(stderr, "%s failed: %s\n", #x, pad_status_string(s_));      \
      return 3;                                                                \
    }                                                                          \
  } while (0)

static bool read_all(std::FILE* f, void* p, size_t n) { return std::fread(p, 1, n, f) == n; }

int main(int argc, char** argv) {
  if (argc != 3) {
    std::fprintf(stderr, "usage: %s input.bin output.bin\n", argv[0]);
    return 1;
  }
  if (pad_decode_abi_version() != PAD_ABI_VERSION) {
    std::fprintf(stderr, "ABI version %d, header %d\n", pad_decode_abi_version(), PAD_ABI_VERSION);
    return 1;
  }
  std::FILE* in = std::fopen(argv[1], "rb");
  if (!in) return 1;
  int64_t h[8];
  if (!read_all(in, h, sizeof(h))) return 1;
  const int64_t B = h[0], HQ = h[1], HKV = h[2], D = h[3], PS = h[4], MP = h[5], NP = h[6];
  const int splits = static_cast<int>(h[7]);
  const size_t q_n = B * HQ * D, kv_n = NP * PS * HKV * D;
  std::vector<uint16_t> q(q_n), k(kv_n), v(kv_n), out(q_n);
  std::vector<int32_t> bt(B * MP), sl(B);
  if (!read_all(in, q.data(), q_n * 2) || !read_all(in, k.data(), kv_n * 2) || !read_all(in, v.data(), kv_n * 2) ||
      !read_all(in, bt.data(), bt.size() * 4) || !read_all(in, sl.data(), sl.size() * 4))
    return 1;
  std::fclose(in);

  void *dq, *dk, *dv, *dbt, *dsl, *dout;
  HIP_OK(hipMalloc(&dq, q_n * 2));
  HIP_OK(hipMalloc(&dk, kv_n * 2));
  HIP_OK(hipMalloc(&dv, kv_n * 2));
  HIP_OK(hipMalloc(&dbt, bt.size() * 4));
  HIP_OK(hipMalloc(&dsl, sl.size() * 4));
  HIP_OK(hipMalloc(&dout, q_n * 2));
  HIP_OK(hipMemcpy(dq, q.data(), q_n * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dk, k.data(), kv_n * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dv, v.data(), kv_n * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dbt, bt.data(), bt.size() * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dsl, sl.data(), sl.size() * 4, hipMemcpyHostToDevice));

  // Contiguous tensors: element strides of the row-major shapes.
  pad_decode_dims d = {};
  d.batch = static_cast<int32_t>(B);
  d.num_q_heads = static_cast<int32_t>(HQ);
  d.num_kv_heads = static_cast<int32_t>(HKV);
  d.head_dim = static_cast<int32_t>(D);
  d.page_size = static_cast<int32_t>(PS);
  d.max_pages = static_cast<int32_t>(MP);
  d.num_pages = NP;
  d.q_stride[0] = d.out_stride[0] = HQ * D;
  d.q_stride[1] = d.out_stride[1] = D;
  d.q_stride[2] = d.out_stride[2] = 1;
  d.k_stride[0] = d.v_stride[0] = PS * HKV * D;
  d.k_stride[1] = d.v_stride[1] = HKV * D;
  d.k_stride[2] = d.v_stride[2] = D;
  d.k_stride[3] = d.v_stride[3] = 1;
  d.bt_stride[0] = MP;
  d.bt_stride[1] = 1;
  d.sl_stride = 1;

  // Scratch sized by the pure-host queries, counters zeroed once.
  size_t ws_bytes = 0;
  int64_t n_counters = 0;
  PAD_OK_(pad_decode_workspace_bytes(&d, splits, 0, &ws_bytes));
  PAD_OK_(pad_decode_counters_needed(&d, splits, 0, &n_counters));
  void* ws = nullptr;
  int32_t* counters = nullptr;
  HIP_OK(hipMalloc(&ws, ws_bytes > 0 ? ws_bytes : 1));
  HIP_OK(hipMalloc(reinterpret_cast<void**>(&counters), (n_counters > 0 ? n_counters : 1) * sizeof(int32_t)));
  hipStream_t stream;
  HIP_OK(hipStreamCreate(&stream));
  if (n_counters > 0) PAD_OK_(pad_decode_counters_init(counters, n_counters, stream));

  const float scale = 1.0f / std::sqrt(static_cast<float>(D));
  // Two launches in a row: the counters come back to zero, the workspace keeps no state.
  for (int rep = 0; rep < 2; ++rep)
    PAD_OK_(pad_decode_launch(dq, dk, dv, static_cast<const int32_t*>(dbt), static_cast<const int32_t*>(dsl), dout,
                              ws, ws_bytes, counters, n_counters, &d, scale, splits, stream));
  HIP_OK(hipStreamSynchronize(stream));
  HIP_OK(hipMemcpy(out.data(), dout, q_n * 2, hipMemcpyDeviceToHost));

  std::FILE* o = std::fopen(argv[2], "wb");
  if (!o || std::fwrite(out.data(), 2, q_n, o) != q_n) return 1;
  std::fclose(o);
  HIP_OK(hipStreamDestroy(stream));
  for (void* p : {dq, dk, dv, dbt, dsl, dout, ws, static_cast<void*>(counters)}) HIP_OK(hipFree(p));
  return 0;
}
