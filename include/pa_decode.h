/*
 * pa_decode.h - C ABI of the MI355X (gfx950) paged-attention decode library
 * (libpa_decode.so).
 *
 * One operator: single-query decode attention over a paged KV cache with
 * grouped-query attention (GQA),
 *
 *   out[b, h, :] = softmax(scale * q[b, h, :] . K_b^T) . V_b
 *
 * where K_b / V_b are the first seq_lens[b] tokens of the pages listed in
 * block_table[b, :], and kv head = h / (num_q_heads / num_kv_heads).
 * A row with seq_lens[b] == 0 produces zeros.
 *
 * Tensor layouts (element strides, all int64):
 *   q           fp16 [batch, num_q_heads, head_dim]
 *   k_cache     fp16 [num_pages, page_size, num_kv_heads, head_dim]
 *   v_cache     fp16 [num_pages, page_size, num_kv_heads, head_dim]
 *   block_table int32 [batch, max_pages] (may be NULL when max_pages is 0)
 *   seq_lens    int32 [batch]
 *   out         fp16 [batch, num_q_heads, head_dim]
 * head_dim must be contiguous (stride 1) for q, k_cache, v_cache and out.
 * pad_decode_launch_kv8() and pad_decode_launch_call() also take fp8
 * (e4m3fn / e5m2) caches of the same layout, one byte per element, and
 * pad_decode_launch_call() bfloat16 q, caches and out (PAD_KV_BF16).
 *
 * The library replaces the reference's native launcher
 *   torch::Tensor paged_attn_decode_cuda_v4_launch(q, k_cache, v_cache,
 *       block_table, seq_lens, scale, gqa_ratio, head_dim, page_size,
 *       num_splits)
 * declared at cuda/kernels.h:60-70 and defined at
 * cuda/kernel_v4_split_k.cu:205-268, bound to Python as `forward_v4`
 * (cuda/binding.cpp:13-14).  Unlike that launcher, nothing here allocates:
 * the caller passes the output and a workspace sized by
 * pad_decode_workspace_bytes(), and the launch is asynchronous on the
 * caller's stream with no host synchronisation.  Split-K's two phases (the
 * reference's two kernels) run as one kernel launch.
 *
 * Scratch contract.  A launch that splits sequences needs two buffers:
 *  - `workspace` (pad_decode_workspace_bytes()): the fp32 split partials;
 *    no state is kept in it between launches;
 *  - `counters` (pad_decode_counters_needed() int32 entries): one arrival
 *    counter per (sequence, kv head), plus one per split slot when a
 *    sequence may get more than 48 splits (those merge in two levels,
 *    groups of 16 splits first).  They must be zero before the first
 *    launch that uses them (pad_decode_counters_init() or any zero-filled
 *    allocation), and every launch leaves them zero again.
 * Launches that may run at the same time must not share either buffer (give
 * each stream its own).
 *
 * Every entry point returns a pad_status.  Host-only functions
 * (pad_decode_plan, pad_decode_workspace_bytes, pad_status_string,
 * pad_decode_abi_version) touch no device and can be called without a GPU.
 */
#ifndef PA_DECODE_H_
#define PA_DECODE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PAD_ABI_VERSION 6

/* Largest supported GQA group (query heads per KV head); the reference's
 * bound is the same (cuda/kernel_v4_split_k.cu:44). */
#define PAD_MAX_GQA 16
/* Largest split count one call may use. */
#define PAD_MAX_SPLITS 1024

typedef enum pad_status {
  PAD_OK = 0,
  PAD_ERR_NULL_POINTER = 1,      /* a required pointer is NULL            */
  PAD_ERR_INVALID_SHAPE = 2,     /* non-positive or inconsistent sizes    */
  PAD_ERR_UNSUPPORTED_HEAD_DIM = 3, /* head_dim not in {32,64,96,128,256}  */
  PAD_ERR_UNSUPPORTED_GQA = 4,   /* num_q_heads % num_kv_heads != 0 or
                                    group larger than PAD_MAX_GQA          */
  PAD_ERR_STRIDE = 5,            /* head_dim stride != 1                   */
  PAD_ERR_ALIGNMENT = 6,         /* K/V/q/out rows not 16-byte aligned     */
  PAD_ERR_WORKSPACE = 7,         /* workspace or counters NULL / too small */
  PAD_ERR_NUM_SPLITS = 8,        /* num_splits < 0 or > PAD_MAX_SPLITS     */
  PAD_ERR_LAUNCH = 9,            /* the HIP runtime rejected a launch      */
  PAD_ERR_DEVICE = 10,           /* no usable device / device query failed */
  PAD_ERR_SCRATCH_LIMIT = 11,    /* pad_decode_launch_noalloc: the call needs
                                    more than its static scratch holds      */
  PAD_ERR_KV_FORMAT = 12         /* unknown cache format, a format the
                                    entry point or engine does not take, or
                                    an fp8 scale that is not finite and
                                    positive                                */
} pad_status;

/* Data formats of a call (pad_decode_launch_kv8, pad_decode_launch_call):
 * the caches' element type and, for fp8 caches, whether q and out are fp16
 * (PAD_KV_FP8_E4M3FN / _E5M2) or bfloat16 (..._BF16). */
#define PAD_KV_FP16 0         /* IEEE half (every other entry point)          */
#define PAD_KV_FP8_E4M3FN 1   /* OCP fp8 E4M3 "fn": bias 7, no infinities     */
#define PAD_KV_FP8_E5M2 2     /* OCP fp8 E5M2: bias 15, IEEE-like             */
#define PAD_KV_BF16 3         /* bfloat16 q, caches and out (pad_decode_launch_call;
                                 MFMA engine, every head_dim; P is rounded to
                                 bf16 for the PV product)                     */
#define PAD_KV_FP8_E4M3FN_BF16 4  /* e4m3fn caches with bfloat16 q and out    */
#define PAD_KV_FP8_E5M2_BF16 5    /* e5m2 caches with bfloat16 q and out       */

/* Static scratch of pad_decode_launch_noalloc(), per device: fp32 partials
 * and int32 arrival counters.  48 MiB in all, held until the process ends. */
#define PAD_NOALLOC_WORKSPACE_BYTES ((size_t)48 * 1024 * 1024 - (size_t)256 * 1024)
#define PAD_NOALLOC_COUNTERS 65536

/* Shapes and element strides of one call (a plain tensor descriptor). */
typedef struct pad_decode_dims {
  int32_t batch;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t page_size;
  int32_t max_pages;        /* block_table.shape[1]                        */
  int64_t num_pages;        /* k_cache.shape[0]; page ids outside
                               [0, num_pages) read page 0 instead of
                               faulting, so a launch that reads pages
                               needs it > 0 (else PAD_ERR_INVALID_SHAPE)   */
  int64_t q_stride[3];      /* [batch, head, dim]                          */
  int64_t k_stride[4];      /* [page, slot, kv_head, dim]                  */
  int64_t v_stride[4];
  int64_t bt_stride[2];     /* [batch, page column]                        */
  int64_t sl_stride;        /* seq_lens[b] is at seq_lens + b * sl_stride  */
  int64_t out_stride[3];
} pad_decode_dims;

/* Work decomposition chosen for a call: the kernels walk
 * pages_per_split pages of one sequence per workgroup. */
typedef struct pad_decode_plan_t {
  int32_t num_splits;       /* splits per (sequence, kv head)              */
  int32_t pages_per_split;
  int32_t waves_per_group;  /* 64-lane waves per phase-1 workgroup         */
  int32_t single_pass;      /* 1: one split per sequence, no partials      */
  int32_t engine;           /* 0 = MFMA tiles, 1 = VALU/DPP dot products   */
  int32_t reserved;
  size_t workspace_bytes;   /* fp32 partials; 0 if single_pass             */
  int64_t counters;         /* int32 arrival counters; 0 if single_pass    */
} pad_decode_plan_t;

/* Choose the split count and workgroup shape.  num_splits > 0 forces that
 * many splits (the reference's `num_splits` argument,
 * src/kernel_cuda_v4.py:19-27); 0 selects the built-in heuristic, which
 * depends only on shapes and the CU count (num_cus <= 0 means 256).  Pure
 * host function: it reads neither seq_lens nor block_table.  Replaces the
 * reference's fixed default _DEFAULT_NUM_SPLITS = 64
 * (src/kernel_cuda_v4.py:16).
 * The launch grid has G = batch * num_kv_heads * num_splits workgroups.
 * With the heuristic (num_splits == 0), a split plan and batch <= 256, the
 * kernel itself reads every sequence length and re-plans the G workgroups
 * over the pages actually in use (equal page chunks, so ragged batches and
 * sequences shorter than max_pages * page_size stay balanced); with every
 * sequence at full capacity that plan is the static one.  A bandwidth-bound
 * shape with at least one (sequence, kv head) unit per CU gets a grid of 4
 * items per unit: one item per unit (no partials) when every sequence is at
 * full capacity, equal page chunks when the lengths are ragged. */
int pad_decode_plan(const pad_decode_dims* dims, int num_splits, int num_cus,
                    pad_decode_plan_t* plan);

/* pad_decode_plan() for pad_decode_launch_csr(): dims->max_pages is the
 * number of entries of the CSR `indices` array (every sequence's pages), so
 * the plan assumes max_pages / batch pages per sequence (exact when the
 * lengths are equal; ragged batches are re-planned in-kernel from indptr
 * under the heuristic).  An explicit num_splits cuts each sequence's own
 * pages into that many ranges.  The workspace and counters this plan
 * reports never exceed those of pad_decode_plan() on the same dims, so
 * either sizes the scratch of a CSR launch.  Pure host function.  No
 * counterpart in the reference (its FlashInfer adapter planned inside the
 * library, src/flashinfer_adapter.py:100-112). */
int pad_decode_plan_csr(const pad_decode_dims* dims, int num_splits,
                        int num_cus, pad_decode_plan_t* plan);

/* Bytes of workspace pad_decode_launch() needs for these arguments
 * (0 when the plan is single-pass).  Pure host function.  The reference
 * allocated the same partials per call inside its launcher
 * (cuda/kernel_v4_split_k.cu:228-232). */
int pad_decode_workspace_bytes(const pad_decode_dims* dims, int num_splits,
                               int num_cus, size_t* bytes);

/* int32 arrival counters a launch with these arguments needs (0 when the
 * plan is single-pass; otherwise U = batch * num_kv_heads, or U * (1 +
 * num_splits) when U * num_splits > 48, so that a sequence may get more
 * than 48 split items and merge them in two levels).  Pure host
 * function.  No counterpart in the reference, whose two kernel launches
 * needed no arrival counting. */
int pad_decode_counters_needed(const pad_decode_dims* dims, int num_splits,
                               int num_cus, int64_t* count);

/* pad_decode_launch() without workspace or counters arguments: it allocates
 * nothing (no hipMalloc/hipFree, no allocating library call), for callers
 * that cannot allocate - code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation.  No counterpart in the reference.  The
 * split scratch is a static device
 * array of the library, one per GPU, of PAD_NOALLOC_WORKSPACE_BYTES bytes of
 * partials and PAD_NOALLOC_COUNTERS counters; a call whose plan
 * (pad_decode_workspace_bytes() / pad_decode_counters_needed()) needs more
 * returns PAD_ERR_SCRATCH_LIMIT without launching.  The first call on a
 * device looks up its copy's address and queues a small kernel that zeroes
 * the counters on `stream`.  Every call on one GPU shares that GPU's array:
 * calls that may overlap on one GPU (different streams, or graphs replayed
 * concurrently) race and must be serialised by the caller.  Same kernels,
 * plan and results as pad_decode_launch(). */
int pad_decode_launch_noalloc(const void* q, const void* k_cache,
                              const void* v_cache, const int32_t* block_table,
                              const int32_t* seq_lens, void* out,
                              const pad_decode_dims* dims, float scale,
                              int num_splits, void* stream);

/* Zero `num_counters` counters (asynchronously, on `stream`, with a fill
 * kernel, so a call under stream capture records a kernel node); needed once
 * per counter buffer. */
int pad_decode_counters_init(int32_t* counters, int64_t num_counters,
                             void* stream);

/* Launch the decode on `stream` (a hipStream_t; NULL = the null stream).
 * Asynchronous: returns once the kernels are queued.  `scale` is the
 * softmax scale (the reference defaults it to 1/sqrt(head_dim),
 * src/kernel_cuda_v4.py:60).  `num_splits` as in pad_decode_plan().
 * Replaces paged_attn_decode_cuda_v4_launch
 * (cuda/kernel_v4_split_k.cu:205-268). */
int pad_decode_launch(const void* q, const void* k_cache, const void* v_cache,
                      const int32_t* block_table, const int32_t* seq_lens,
                      void* out, void* workspace, size_t workspace_bytes,
                      int32_t* counters, int64_t num_counters,
                      const pad_decode_dims* dims, float scale,
                      int num_splits, void* stream);

/* pad_decode_launch() over fp8 K/V caches: k_cache / v_cache hold one byte
 * per element in `kv_format` (PAD_KV_FP8_E4M3FN or PAD_KV_FP8_E5M2 with fp16
 * q and out, PAD_KV_FP8_E4M3FN_BF16 or PAD_KV_FP8_E5M2_BF16 with bfloat16; the
 * layouts, strides in elements = bytes, of the fp16 caches), and represent
 * K = k_scale * k_cache and V = v_scale * v_cache (per-tensor scales, the
 * convention of serving engines' fp8 KV caches); head_dim 64, 128 or 256.
 * Each element is widened exactly in registers to q's format, so the result
 * equals the fp16 (bfloat16) path's on the dequantized caches up to fp32
 * rounding: k_scale goes into the softmax scale and
 * v_scale into the output normalisation.  Same splits, workspace and
 * counters as pad_decode_launch() (pad_decode_plan(),
 * pad_decode_workspace_bytes(), pad_decode_counters_needed()); workgroups
 * may have more waves, as the rows are half the bytes.  No counterpart in
 * the reference, whose caches are fp16 only (src/kernel_cuda_v4.py:37-48);
 * it is the next data format of the same operator. */
int pad_decode_launch_kv8(const void* q, const void* k_cache,
                          const void* v_cache, const int32_t* block_table,
                          const int32_t* seq_lens, void* out,
                          void* workspace, size_t workspace_bytes,
                          int32_t* counters, int64_t num_counters,
                          const pad_decode_dims* dims, float scale,
                          int kv_format, float k_scale, float v_scale,
                          int num_splits, void* stream);

/* Same as pad_decode_launch(), with the engine forced (0 = MFMA tiles,
 * 1 = VALU/DPP dot products) and, when `events` is not NULL, three
 * hipEvent_t handles recorded on `stream`: before the decode kernel, after
 * it, and at the end of the call (the same point, as the call is one
 * kernel).  For measurement; the outputs are the same as
 * pad_decode_launch()'s.  No counterpart in the reference. */
int pad_decode_launch_ex(const void* q, const void* k_cache,
                         const void* v_cache, const int32_t* block_table,
                         const int32_t* seq_lens, void* out, void* workspace,
                         size_t workspace_bytes, int32_t* counters,
                         int64_t num_counters, const pad_decode_dims* dims,
                         float scale, int num_splits, int engine,
                         void* const* events, void* stream);

/* Decode over a CSR page index instead of the dense block table: the page
 * ids of sequence b are indices[indptr[b] .. indptr[b+1]) (int32, in
 * logical order) and its last page holds last_page_len[b] tokens, so
 * seq_len[b] = (indptr[b+1] - indptr[b] - 1) * page_size + last_page_len[b]
 * (0 for a sequence with no pages).  This is the (indptr, indices,
 * last_page_len) triple the reference's FlashInfer adapter derives from the
 * dense table (src/flashinfer_adapter.py:40-65) and hands to FlashInfer's
 * plan/run (:100-112); here the kernel reads it directly.  In `dims`,
 * max_pages is the number of entries in `indices`; bt_stride and sl_stride
 * are ignored.  Workspace, counters, scale, num_splits, engine and stream
 * are as in pad_decode_launch_ex(), and pad_decode_workspace_bytes() /
 * pad_decode_counters_needed() size the scratch from the same dims. */
int pad_decode_launch_csr(const void* q, const void* k_cache,
                          const void* v_cache, const int32_t* indices,
                          const int32_t* indptr, const int32_t* last_page_len,
                          void* out, void* workspace, size_t workspace_bytes,
                          int32_t* counters, int64_t num_counters,
                          const pad_decode_dims* dims, float scale,
                          int num_splits, int engine, void* stream);

/* Plan once, run many: the split between FlashInfer's
 * BatchDecodeWithPagedKVCacheWrapper.plan() and .run() that the reference's
 * adapter calls (src/flashinfer_adapter.py:100-112) and its benchmark
 * amortises over many runs (bench/bench_flashinfer.py:131-151).
 *
 * pad_decode_plan_worklist() (dense table) / pad_decode_plan_worklist_csr()
 * (CSR index) queue one small kernel on `stream` that writes the work list
 * of a decode with these dims, indices and num_splits into `worklist`
 * (device memory of pad_decode_worklist_bytes() bytes; pass csr = 1 for a
 * CSR plan): for every workgroup of the decode grid, the page range and
 * unit it processes and the page ids its waves read first - what the decode
 * kernel otherwise works out from the sequence lengths at the start of
 * every launch.  pad_decode_launch_worklist() / _csr() then run the decode
 * (MFMA engine) from the list, once per layer of a decode step.  The
 * results are the same as pad_decode_launch() / pad_decode_launch_csr()
 * with the same arguments.
 *
 * The list encodes the sequence lengths and page ids it was planned from:
 * plan again after they change (in a decoding loop, once per step, before
 * the step's first layer).  A list planned for other dims or num_splits is
 * detected (a key in its header) and ignored: the launch then plans in the
 * kernel as pad_decode_launch() does.  No counterparts in the reference. */
int pad_decode_worklist_bytes(const pad_decode_dims* dims, int num_splits,
                              int num_cus, int csr, size_t* bytes);
int pad_decode_plan_worklist(const int32_t* block_table,
                             const int32_t* seq_lens,
                             const pad_decode_dims* dims, int num_splits,
                             void* worklist, size_t worklist_bytes,
                             void* stream);
int pad_decode_plan_worklist_csr(const int32_t* indices, const int32_t* indptr,
                                 const int32_t* last_page_len,
                                 const pad_decode_dims* dims, int num_splits,
                                 void* worklist, size_t worklist_bytes,
                                 void* stream);
int pad_decode_launch_worklist(const void* q, const void* k_cache,
                               const void* v_cache, const int32_t* block_table,
                               const int32_t* seq_lens, void* out,
                               void* workspace, size_t workspace_bytes,
                               int32_t* counters, int64_t num_counters,
                               const pad_decode_dims* dims, float scale,
                               int num_splits, const void* worklist,
                               size_t worklist_bytes, void* stream);
int pad_decode_launch_worklist_csr(const void* q, const void* k_cache,
                                   const void* v_cache, const int32_t* indices,
                                   const int32_t* indptr,
                                   const int32_t* last_page_len, void* out,
                                   void* workspace, size_t workspace_bytes,
                                   int32_t* counters, int64_t num_counters,
                                   const pad_decode_dims* dims, float scale,
                                   int num_splits, const void* worklist,
                                   size_t worklist_bytes, void* stream);

/* Every option of one decode launch in one descriptor, for callers that
 * need a combination the entry points above do not offer (fp8 caches with a
 * CSR page index or a work list).  Fields:
 *   block_table / seq_lens: the dense page index; with a CSR index
 *     (indptr != NULL) block_table is `indices`, seq_lens is unused and
 *     dims->max_pages is the number of entries of `indices`, as for
 *     pad_decode_launch_csr();
 *   worklist / worklist_bytes: optional, a list planned for the same call
 *     (pad_decode_plan_worklist_call()); NULL plans in the kernel;
 *   engine: 0 (MFMA) or 1 (VALU: fp16 only, no work list;
 *     PAD_ERR_INVALID_SHAPE with a work list, PAD_ERR_KV_FORMAT with fp8
 *     or bf16);
 *   kv_format, k_scale, v_scale: PAD_KV_FP16, PAD_KV_BF16 (q, caches and
 *     out all bfloat16), or an fp8 cache format as pad_decode_launch_kv8();
 *     the scales are read for fp8 only.
 * pad_decode_launch_call() runs exactly what the matching entry point runs:
 * pad_decode_launch_ex (no events), _csr, _worklist, _worklist_csr or _kv8,
 * with the same workspace and counters.  No counterpart in the reference. */
typedef struct pad_decode_call {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const int32_t* block_table;
  const int32_t* seq_lens;
  const int32_t* indptr;          /* CSR [batch + 1], or NULL             */
  const int32_t* last_page_len;   /* CSR [batch], or NULL                 */
  void* out;
  void* workspace;
  size_t workspace_bytes;
  int32_t* counters;
  int64_t num_counters;
  const void* worklist;
  size_t worklist_bytes;
  float scale;
  int32_t num_splits;
  int32_t engine;
  int32_t kv_format;
  float k_scale;
  float v_scale;
} pad_decode_call;

int pad_decode_launch_call(const pad_decode_call* call,
                           const pad_decode_dims* dims, void* stream);

/* The work list of the launch `call` describes (its index fields, engine
 * and kv_format; the data pointers are not read), written to `worklist`
 * (pad_decode_worklist_bytes() bytes, csr = indptr != NULL).  A list
 * planned for another kv_format is ignored by the launch, which then plans
 * in the kernel: fp8 launches may run workgroups of more waves. */
int pad_decode_plan_worklist_call(const pad_decode_call* call,
                                  const pad_decode_dims* dims, void* worklist,
                                  size_t worklist_bytes, void* stream);

/* Compute units of the current device (cached per device). */
int pad_device_num_cus(int* num_cus);

/* Static text for a status code. */
const char* pad_status_string(int status);

/* PAD_ABI_VERSION of the built library. */
int pad_decode_abi_version(void);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* PA_DECODE_H_ */
