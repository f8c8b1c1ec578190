// pa_decode.hip - gfx950 (MI355X) paged-attention decode: kernels + C ABI.
//
// Operator contract: the reference oracle paged_attention_decode_reference
// (src/reference.py:8-54) evaluated on fp16 inputs, output in fp16.
// Work decomposition: split-K over the sequence ("FlashDecoding"), the same
// merge algebra as analysis/split_k_derivation.md:16-86, restated here:
//
//   phase 1, per (sequence b, kv head, split s) over its tokens:
//     m_s = max score,  l_s = sum exp(score - m_s),
//     O_s = sum exp(score - m_s) * V                  (not divided by l_s)
//   phase 2, per (b, q head):
//     m = max_s m_s,  w_s = exp(m_s - m) (0 for an empty split),
//     out = (sum_s w_s O_s) / (sum_s w_s l_s)
//
// Scores are kept in base-2 units (score * scale * log2 e) so every
// exponential is a single v_exp_f32 (exp(x) = 2^(x log2 e)).
//
// Design (MI355X-first, not a translation of the reference's kernels):
//  * Splits are page-aligned: split s of a sequence covers logical pages
//    [s*pages_per_split, (s+1)*pages_per_split), so each page and each
//    block_table entry is read by exactly one workgroup.  The reference
//    split by tokens (cuda/kernel_v4_split_k.cu:73-75).
//  * A phase-1 workgroup is 1-8 wave64s; each wave walks 16-token blocks of
//    its split and keeps its own online-softmax state; the waves' states are
//    merged through LDS at the end (one fp32 partial per workgroup).
//  * Engine 0 (MFMA): scores are computed transposed, S^T = K . Q^T, with
//    v_mfma_f32_16x16x16_f16 (16 tokens x 16 padded GQA rows, K = head_dim),
//    and the output as O^T = V^T . P^T.  With S^T every lane already holds
//    P^T in the B-operand layout of the PV product, so P never moves between
//    lanes.  K and V are read as whole token rows (16 lanes cover a row
//    with 16-byte loads); the head_dim index inside each PV tile is
//    permuted so that these V registers are the MFMA A operand as loaded,
//    and K goes through a padded LDS tile into the A layout of S^T.  One
//    K/V tile is shared by the whole GQA group through the B operand.
//  * Engine 1 (VALU): 16 lanes per token, fp16x2 dot products
//    (v_dot2_f32_f16) reduced across the 16 lanes with 4 DPP steps, fp32
//    online softmax and FMA accumulation of P.V.  Kept for the measured
//    comparison against engine 0.
//  * Phase 2 is fused into the same launch: every workgroup of a split
//    sequence publishes its fp32 partial with device-scope stores and counts
//    itself in with an atomic; the last one to arrive folds all partials of
//    its (sequence, kv head) into the fp16 output and resets the counter
//    (past 48 splits in two levels, groups of 16 splits first).  A sequence
//    held by one split is normalised directly.  One kernel launch per call.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <mutex>

#include "pa_decode.h"
#include "pa_decode_timeline.h"  // slot constants; its functions exist only with -DPAD_TIMELINE

namespace pad {

#ifdef PAD_TIMELINE
// Phase timeline, compiled only into the measurement library
// (libpa_decode_tl.so, -DPAD_TIMELINE): thread 0 of every workgroup stores
// s_memrealtime stamps (100 MHz) at fixed points of its path, for the last
// PAD_TL_LAUNCHES launches (a ring indexed by a host-side launch count).
// Slot meanings are the PAD_TL_* constants of pa_decode_timeline.h.
__device__ unsigned long long tl_buf[PAD_TL_LAUNCHES * PAD_TL_MAX_GROUPS * PAD_TL_SLOTS];
static int tl_launches = 0;
#define PAD_TL_AT(lin, slot, value)                                                                      \
  do {                                                                                                   \
    if (threadIdx.x == 0 && (lin) < PAD_TL_MAX_GROUPS)                                                   \
      ::pad::tl_buf[((size_t)a.tl_launch * PAD_TL_MAX_GROUPS + (lin)) * PAD_TL_SLOTS + (slot)] = (value); \
  } while (0)
#define PAD_TL(lin, slot) PAD_TL_AT(lin, slot, __builtin_amdgcn_s_memrealtime())
#else
#define PAD_TL_AT(lin, slot, value) \
  do {                              \
  } while (0)
#define PAD_TL(lin, slot) \
  do {                    \
  } while (0)
#endif

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr float kNegInf = -__builtin_inff();
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kBlockTokens = 16;  // tokens per wave iteration (one MFMA tile)
constexpr int kMaxWaves = 8;
// Fewest 16-token blocks per split (or planned item): each workgroup's fixed
// costs (q load, wave merge, partial publish) stay small against its streaming.
constexpr int kMinBlocks = 16;
// Fewest blocks per split for short latency-bound sequences (split counts up
// to 16, which one merge round trip covers).
constexpr int kMinBlocksShort = 4;
// Units with more splits than this merge in two levels (groups of 16).
constexpr int kTwoLevelSplits = 48;
// LDS of one workgroup (wave merge + MFMA staging) is capped so that the
// widest rows (head_dim 256, 16-row groups) still get 4 waves in a
// workgroup that fits a CU's 160 KB: one 2-wave workgroup per split left
// those shapes latency-bound (16/1 d256 batch 8 x 8192: 35.2 against
// 24.7 us).
constexpr int kLdsBudget = 136 * 1024;
// Headroom (base-2 units) a score may exceed the running reference max before
// the accumulators are rescaled; fp16 weights stay <= 2^8.
constexpr float kRescaleSlack = 8.0f;

// Largest batch the in-kernel work planner handles (4 sequences per lane).
constexpr int kPlanMaxBatch = 256;

struct Phase1Args {
  // Control fields first: they are read at the start of every workgroup.
  int gqa, ps, pps, num_splits, hkv, max_pages, batch;
  int nw;          // waves per workgroup (blockDim.x / 64)
  int ps_shift;    // log2(ps) when ps is a power of two, else -1
  int csr;         // 1: page ids from (indptr, indices, last_page_len)
  int balance;     // 1: items planned from the sequence lengths in-kernel;
                   // 2-4: the same on an oversubscribed grid (balance - 1
                   //    static splits per unit, pps pages each, on the
                   //    first workgroups when every sequence is full)
  int min_chunk;   // planner: fewest pages per item
  int pair_heads;  // 1: workgroups 8 apart take kv heads 2m and 2m+1 (see grid_pos)
  int wl_key;      // key of the launch's plan, matched against the work list's header
  float scale_log2;
  float v_fix;     // fp8 caches: V's scale, applied to the output rows
  const int32_t* bt;      // dense: block_table [B, max_pages]; CSR: indices
  const int32_t* sl;      // dense: seq_lens [B]
  const int32_t* indptr;  // CSR: [B + 1] offsets of each sequence's page ids in bt
  const int32_t* lpl;     // CSR: [B] tokens in each sequence's last page
  const int32_t* worklist;  // precomputed work items (header + one record per workgroup) or nullptr
  int64_t sbb, sbp;
  int64_t ssl;
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  _Float16* out;
  float* o_part;   // [G, gqa, D], one slot per workgroup of the grid
  float2* ml_part; // [G, gqa]  (m in base-2 units, l)
  int* counters;   // [B, Hkv] arrival counts, then per-slot group counts; zero between launches
  int64_t sqb, sqh;
  int64_t skp, sks, skh;
  int64_t svp, svs, svh;
  int64_t sob, soh;
  int64_t num_pages;
#ifdef PAD_TIMELINE
  int tl_launch;   // ring slot of this launch's stamps
#endif
};

// Token -> page index, and pages covering n tokens (shift for power-of-two
// page sizes).
__device__ __forceinline__ int page_of(const Phase1Args& a, int t) {
  return a.ps_shift >= 0 ? (t >> a.ps_shift) : t / a.ps;
}
__device__ __forceinline__ int pages_for(const Phase1Args& a, int n) { return page_of(a, n + a.ps - 1); }
// 16-token block -> page index (page_size a multiple of 16).
__device__ __forceinline__ int block_page(const Phase1Args& a, int jb) {
  return a.ps_shift >= 4 ? (jb >> (a.ps_shift - 4)) : jb / (a.ps / 16);
}

__device__ __forceinline__ float exp2_fast(float x) {
  return __builtin_amdgcn_exp2f(x);  // v_exp_f32; exp2(-inf) = 0
}

__device__ __forceinline__ float shfl_xor_f(float x, int m) {
  return __shfl_xor(x, m, 64);
}

// Sum over the 16 lanes of a DPP row (lanes 16r .. 16r+15), result in all.
__device__ __forceinline__ float row16_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));  // row_half_mirror
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));  // row_mirror
  return x;
}

// NDW dwords (2*NDW halves) loaded from a 4*NDW-byte aligned address.
template <int NDW>
struct HVec {
  uint32_t w[NDW];
  __device__ __forceinline__ _Float16 h(int i) const {
    const uint32_t x = w[i >> 1];
    const uint16_t bits = (i & 1) ? (uint16_t)(x >> 16) : (uint16_t)(x & 0xffffu);
    return __builtin_bit_cast(_Float16, bits);
  }
  __device__ __forceinline__ h2_t h2(int i) const { return __builtin_bit_cast(h2_t, w[i]); }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < NDW; ++i) w[i] = 0u;
  }
};

template <int NDW>
__device__ __forceinline__ HVec<NDW> load_hvec(const _Float16* p) {
  HVec<NDW> r;
  if constexpr (NDW % 4 == 0) {
    const uint4* src = reinterpret_cast<const uint4*>(p);
#pragma unroll
    for (int i = 0; i < NDW / 4; ++i) {
      const uint4 x = src[i];
      r.w[4 * i + 0] = x.x; r.w[4 * i + 1] = x.y; r.w[4 * i + 2] = x.z; r.w[4 * i + 3] = x.w;
    }
  } else if constexpr (NDW % 2 == 0) {
    const uint2* src = reinterpret_cast<const uint2*>(p);
#pragma unroll
    for (int i = 0; i < NDW / 2; ++i) {
      const uint2 x = src[i];
      r.w[2 * i + 0] = x.x; r.w[2 * i + 1] = x.y;
    }
  } else {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
    for (int i = 0; i < NDW; ++i) r.w[i] = src[i];
  }
  return r;
}

// Same as load_hvec, with the non-temporal hint: K/V are streamed once per
// call, so they should not displace the reused lines (q, block_table,
// partials) in the caches.
template <int NDW>
__device__ __forceinline__ HVec<NDW> load_hvec_stream(const _Float16* p) {
  typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
  typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
  HVec<NDW> r;
  if constexpr (NDW % 4 == 0) {
#pragma unroll
    for (int i = 0; i < NDW / 4; ++i) {
      const u4_t x = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p) + i);
      r.w[4 * i + 0] = x[0]; r.w[4 * i + 1] = x[1]; r.w[4 * i + 2] = x[2]; r.w[4 * i + 3] = x[3];
    }
  } else if constexpr (NDW % 2 == 0) {
#pragma unroll
    for (int i = 0; i < NDW / 2; ++i) {
      const u2_t x = __builtin_nontemporal_load(reinterpret_cast<const u2_t*>(p) + i);
      r.w[2 * i + 0] = x[0]; r.w[2 * i + 1] = x[1];
    }
  } else if constexpr (NDW % 3 == 0) {
    // head_dim 96: 12-byte row segments, one 3-dword load each.
    typedef uint32_t u3_t __attribute__((ext_vector_type(3)));
#pragma unroll
    for (int i = 0; i < NDW / 3; ++i) {
      const u3_t x = __builtin_nontemporal_load(reinterpret_cast<const u3_t*>(p) + i);
      r.w[3 * i + 0] = x[0]; r.w[3 * i + 1] = x[1]; r.w[3 * i + 2] = x[2];
    }
  } else {
#pragma unroll
    for (int i = 0; i < NDW; ++i) r.w[i] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p) + i);
  }
  return r;
}

// Raw buffer resource over [base, base + bytes) (gfx9 raw-buffer word 3:
// 32-bit data format, no swizzle); out-of-range accesses are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Device-scope (SC1) accesses: coherent across all CUs and XCDs without
// cache maintenance instructions.
constexpr int kCachePolicyDevice = 16;  // SC1
typedef int32_t i2_t __attribute__((ext_vector_type(2)));
typedef int32_t i4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void store_device(__amdgpu_buffer_rsrc_t r, uint32_t off, f4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i4_t, v), r, off, 0, kCachePolicyDevice);
}
__device__ __forceinline__ void store_device(__amdgpu_buffer_rsrc_t r, uint32_t off, float2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i2_t, v), r, off, 0, kCachePolicyDevice);
}
__device__ __forceinline__ f4_t load_device_f4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCachePolicyDevice));
}
__device__ __forceinline__ float2 load_device_f2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kCachePolicyDevice));
}

// N consecutive splits' partials of one (row, 4 columns) element, loaded
// with device-scope loads (the (m, l) pairs first, in split order, then the
// O vectors) and folded in split order:
//   m' = max(m, m_s),  l' = l 2^(m - m') + l_s 2^(m_s - m'),
//   acc' = acc 2^(m - m') + O_s 2^(m_s - m').
// Every load is unconditional: offsets past the unit's region read as zeros
// (buffer range check) and are not folded, so the loads of a batch need no
// branch and each fold step waits only for its own split's data.
template <int N>
struct MergeBatch {
  float2 ml[N];
  f4_t o[N];
  // Entry sp0 + j sits in split slot (sp0 + j) * stride.
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t o_rsrc, __amdgpu_buffer_rsrc_t ml_rsrc, int sp0,
                                       int stride, int gqa, int row, int col, int d) {
#pragma unroll
    for (int j = 0; j < N; ++j) ml[j] = load_device_f2(ml_rsrc, (uint32_t)((sp0 + j) * stride * gqa + row) * 8u);
#pragma unroll
    for (int j = 0; j < N; ++j)
      o[j] = load_device_f4(o_rsrc, ((uint32_t)((sp0 + j) * stride * gqa + row) * (uint32_t)d + col) * 4u);
  }
  // Entries at or past `end` fold with m_s = -inf, i.e. weight 0 (their
  // loads read zeros: they lie past the unit's region): the fold has no
  // branch, so the compiler cannot sink a load into a conditional step and
  // serialise the round trips.  The first entry always exists, so m is
  // finite before any such step and alpha stays 1.
  __device__ __forceinline__ void fold(int sp0, int end, float& m, float& l, f4_t& acc) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      // Every published split is non-empty, so its m is finite.
      const float ms = sp0 + j < end ? ml[j].x : kNegInf;
      const float m_new = fmaxf(m, ms);
      const float alpha = exp2_fast(m - m_new);  // 0 while m is -inf
      const float beta = exp2_fast(ms - m_new);
      l = l * alpha + ml[j].y * beta;
      acc = acc * alpha + o[j] * beta;
      m = m_new;
    }
  }
};

// Folds entries [first, first + count) of one element (entry i in split
// slot i * stride), one memory round trip per batch: 4, 8 or 16 entries for
// counts up to 4, 8 and 16, batches of 16 beyond.  Entries a batch reads
// past the count must lie past the unit's region (they read zeros).
__device__ __forceinline__ void merge_partials(__amdgpu_buffer_rsrc_t o_rsrc, __amdgpu_buffer_rsrc_t ml_rsrc,
                                               int first, int count, int stride, int gqa, int row, int col, int d,
                                               float& m, float& l, f4_t& acc) {
  const int end = first + count;
  if (count <= 4) {
    MergeBatch<4> p;
    p.load(o_rsrc, ml_rsrc, first, stride, gqa, row, col, d);
    p.fold(first, end, m, l, acc);
    return;
  }
  if (count <= 8) {
    MergeBatch<8> p;
    p.load(o_rsrc, ml_rsrc, first, stride, gqa, row, col, d);
    p.fold(first, end, m, l, acc);
    return;
  }
  for (int sp0 = first; sp0 < end; sp0 += 16) {
    MergeBatch<16> p;
    p.load(o_rsrc, ml_rsrc, sp0, stride, gqa, row, col, d);
    p.fold(sp0, end, m, l, acc);
  }
}

// Reads an int32 at a wave-uniform address with a scalar load (constant
// address space): the value lands in an SGPR and its wait counts on the
// LDS/scalar counter, so it never has to drain the K/V vector loads in
// flight, as a vector load of the same word would (vector loads complete in
// order).  The memory must stay unchanged while the kernel runs.
__device__ __forceinline__ int32_t load_uniform_i32(const int32_t* p) {
  return *(const __attribute__((address_space(4))) int32_t*)p;
}

__device__ __forceinline__ int clamp_page(int phys, int64_t num_pages) {
  // Keeps every access inside the cache for an invalid block_table entry
  // (the reference documents valid ids as a precondition and does not
  // check them on the device; here a bad id reads page 0 instead of
  // faulting).
  return (phys < 0 || (int64_t)phys >= num_pages) ? 0 : phys;
}

// ---------------------------------------------------------------------------
// Per-wave state handed to the workgroup merge, written to LDS in one format
// for both engines:  sm_ml[w*16 + row] = (m, l),
// sm_o[(w*gqa + row)*wave_row_floats<D>() + d].  The 16-byte row pad puts
// the 16 rows a wave writes with one instruction in different LDS banks.
// ---------------------------------------------------------------------------
template <int D>
constexpr int wave_row_floats() { return D + 4; }

// One 16-token block of K and V in registers as loaded: lane (g, r16) holds
// its D/16 elements of token 4g+i (fp16: D/32 dwords; fp8 caches: D/64
// dwords of codes, widened to fp16 only where compute() uses them, so that
// the loads of the next block stay in flight across the current one).
template <int D, int ES = 2>
struct KVTile {
  HVec<D * ES / 64> k[4];
  HVec<D * ES / 64> v[4];
};

// Bytes per token row of a wave's K staging tile in LDS (16 rows): the row
// plus 16 bytes of padding, so the 16-row column reads of the MFMA operand
// fall in different banks.
template <int D>
constexpr int k_stage_row_bytes() { return D * 2 + 16; }
template <int D>
constexpr int k_stage_bytes() { return 16 * k_stage_row_bytes<D>(); }

// Engine 0: MFMA 16x16x16 f16 tiles, two blocks in flight per wave (the
// loads of block j+nw are issued before block j is computed).
// With whole-page blocks, the page id of the wave's first block is read
// before the sequence length is known, so its latency overlaps the
// seq_lens read (the column is clamped into the table; its value is only
// used when the block exists).
__device__ __forceinline__ int first_page_id(const Phase1Args& a, const int32_t* ids_row, int64_t ids_stride,
                                             int col_max, int p_first, int wave) {
  if (col_max < 0) return 0;
  const int col = min(p_first + block_page(a, wave), col_max);
  return load_uniform_i32(ids_row + (int64_t)col * ids_stride);
}

// Block-addressing modes of the MFMA wave loop (template parameter MODE):
//   kModeGeneric  any other page size (>= 3): a block spans up to 6 pages;
//   kModeUniform  page_size % 16 == 0: a 16-token block lies in one page;
//   kModeSubpage + s  page_size = 2^s < 16: a block covers 16 >> s whole
//                 pages (items start on page boundaries).
constexpr int kModeGeneric = 0;
constexpr int kModeUniform = 1;
constexpr int kModeSubpage = 2;

// Element formats (template parameter KVF of the MFMA engine): fp16; an
// OCP fp8 cache format, widened to fp16 in registers where compute() uses a
// block, so that everything downstream (K staging, both MFMAs, the softmax)
// is the fp16 path; or bfloat16 q, caches and output, which run the same
// path on bf16 MFMAs (P rounded to bf16, as fp16 P is to fp16).
constexpr int kKvF16 = 0;
constexpr int kKvE4M3 = 1;   // float8_e4m3fn caches, fp16 q and output
constexpr int kKvE5M2 = 2;   // float8_e5m2 caches, fp16 q and output
constexpr int kKvBF16 = 3;   // bfloat16 q, caches and output
constexpr int kKvE4M3B = 4;  // float8_e4m3fn caches, bfloat16 q and output
constexpr int kKvE5M2B = 5;  // float8_e5m2 caches, bfloat16 q and output

template <int KVF>
constexpr bool kv_is_fp8() { return KVF == kKvE4M3 || KVF == kKvE5M2 || KVF == kKvE4M3B || KVF == kKvE5M2B; }
template <int KVF>
constexpr bool kv_is_e4m3() { return KVF == kKvE4M3 || KVF == kKvE4M3B; }
// bfloat16 q, P and output (and MFMAs); fp16 otherwise.
template <int KVF>
constexpr bool q_is_bf16() { return KVF == kKvBF16 || KVF == kKvE4M3B || KVF == kKvE5M2B; }
template <int KVF>
constexpr int kv_elem_bytes() { return kv_is_fp8<KVF>() ? 1 : 2; }

// One 16x16x16 MFMA step on 16-bit operands held as fp16 vectors: fp16, or
// the bit patterns of bfloat16 values (q_is_bf16).
template <int KVF>
__device__ __forceinline__ f4_t mfma16(h4_t a, h4_t b, f4_t c) {
  if constexpr (q_is_bf16<KVF>()) {
    typedef short s4_t __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4_t, a), __builtin_bit_cast(s4_t, b), c,
                                                     0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
}

// x rounded (to nearest even) to the output format, as 16 bits in an fp16
// slot: fp16, or bfloat16 (q_is_bf16).
template <int KVF>
__device__ __forceinline__ _Float16 round16(float x) {
  if constexpr (q_is_bf16<KVF>())
    return __builtin_bit_cast(_Float16, (__bf16)x);
  else
    return (_Float16)x;
}

// Four fp8 codes (one dword, element i in byte i) as four 16-bit values
// (two dwords: elements 0-1 in lo, 2-3 in hi) in the compute format, fp16
// or bfloat16, with gfx950's scaled conversions (v_cvt_scalef32_pk_f16_fp8 /
// _bf8, or _pk_bf16_fp8 / _bf8, one per pair).  Their scale operand acts
// through its exponent only, so it is 1 here and the launch folds the
// caller's k_scale / v_scale into the softmax scale and the output
// normalisation.  At scale 1 every code converts exactly, NaN codes to NaNs
// (every e4m3fn value and every e5m2 value is an fp16 and a bf16 value).
template <int KVF>
__device__ __forceinline__ void fp8x4_to_16x4(uint32_t w, uint32_t& lo, uint32_t& hi) {
  if constexpr (q_is_bf16<KVF>()) {
    typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
    b2_t a, b;
    if constexpr (kv_is_e4m3<KVF>()) {
      a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
      b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
    } else {
      a = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, false);
      b = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, true);
    }
    lo = __builtin_bit_cast(uint32_t, a);
    hi = __builtin_bit_cast(uint32_t, b);
  } else {
    h2_t a, b;
    if constexpr (kv_is_e4m3<KVF>()) {
      a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false);
      b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true);
    } else {
      a = __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, 1.0f, false);
      b = __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, 1.0f, true);
    }
    lo = __builtin_bit_cast(uint32_t, a);
    hi = __builtin_bit_cast(uint32_t, b);
  }
}

// head_dim 256 keeps the Q^T operand in LDS instead of 32 VGPRs per lane
// (with it in registers the kernel spilled 25-38 VGPRs to scratch inside
// the streaming loop).  One padded 16-row copy per workgroup: every lane
// writes its own fragments and reads back only those addresses, so no
// barrier is needed (the waves write identical values).
template <int D>
constexpr bool q_in_lds() { return D >= 256; }

template <int D, int MODE, int KVF = kKvF16>
__device__ __forceinline__ void wave_loop_mfma(const Phase1Args& a, int phys_first, const int32_t* bt_row,
                                               int64_t ids_stride, int b, int kvh, int t_begin, int t_end,
                                               int nblk, int wave, int nw, int lane, float2* sm_ml, float* sm_o,
                                               char* k_stage, char* q_stage) {
  constexpr int DK = D / 32;  // 16-byte K chunks per lane per token
  constexpr int DT = D / 16;  // PV output tiles; V halves per lane per token
  constexpr int NDW = DT / 2;
  constexpr int ES = kv_elem_bytes<KVF>();  // bytes per cache element
  static_assert(!kv_is_fp8<KVF>() || NDW % 2 == 0, "fp8 caches: head_dim a multiple of 64");
  // A lane's DT halves of a token row are NSEG segments of SEG dwords, so
  // that the 16 lanes of a group read 16*SEG*4 contiguous bytes per load
  // instruction: half dt is head_dim slot dim(r16, dt) =
  // (dt / (2*SEG)) * (D / NSEG) + r16 * 2*SEG + dt % (2*SEG).  One segment
  // (the slice r16*DT .. +DT) up to head_dim 128; head_dim 256 reads two
  // 256-byte row halves rather than 16 strided 32-byte slices.
  constexpr int SEG = NDW > 4 ? 4 : NDW;
  constexpr int NSEG = NDW / SEG;
  constexpr int SEG_HALVES = D / NSEG;  // head_dim distance between segments
  // Dwords per lane per token row as loaded (fp8: half of NDW).
  constexpr int NDWR = NDW * ES / 2;
  using Tile = KVTile<D, ES>;
  auto load_slice = [](const char* p) -> HVec<NDWR> {
    if constexpr (kv_is_fp8<KVF>()) {
      // fp8: the same segments at one byte per element, kept as codes.
      HVec<NDWR> r;
#pragma unroll
      for (int sg = 0; sg < NSEG; ++sg) {
        const HVec<SEG / 2> x = load_hvec_stream<SEG / 2>(reinterpret_cast<const _Float16*>(p + sg * SEG_HALVES));
#pragma unroll
        for (int w = 0; w < SEG / 2; ++w) r.w[sg * (SEG / 2) + w] = x.w[w];
      }
      return r;
    } else if constexpr (NSEG == 1) {
      return load_hvec_stream<NDW>(reinterpret_cast<const _Float16*>(p));
    } else {
      HVec<NDW> r;
#pragma unroll
      for (int sg = 0; sg < NSEG; ++sg) {
        const HVec<SEG> x = load_hvec_stream<SEG>(reinterpret_cast<const _Float16*>(p) + sg * SEG_HALVES);
#pragma unroll
        for (int w = 0; w < SEG; ++w) r.w[sg * SEG + w] = x.w[w];
      }
      return r;
    }
  };
  // A loaded row in the fp16 layout (fp8 codes: four per dword, widened).
  auto widen = [](const HVec<NDWR>& x) -> HVec<NDW> {
    if constexpr (!kv_is_fp8<KVF>()) {
      return x;
    } else {
      HVec<NDW> r;
#pragma unroll
      for (int w = 0; w < NDWR; ++w) fp8x4_to_16x4<KVF>(x.w[w], r.w[2 * w], r.w[2 * w + 1]);
      return r;
    }
  };
  const int g = lane >> 4;
  const int r16 = lane & 15;
  const bool row_ok = r16 < a.gqa;
  // The wave's Q^T operand (B of S^T = K.Q^T: row r16, head_dim slots
  // kp*32 + g*8 + [0,8)), loaded after the first K/V block is in flight.
  h8_t qv[q_in_lds<D>() ? 1 : DK];
  auto q_slot = [&](int kp) -> h8_t* {
    return reinterpret_cast<h8_t*>(q_stage + r16 * k_stage_row_bytes<D>() + (kp * 32 + g * 8) * 2);
  };
  auto load_q = [&]() {
    const _Float16* qrow = a.q + (int64_t)b * a.sqb + (int64_t)(kvh * a.gqa + (row_ok ? r16 : 0)) * a.sqh;
#pragma unroll
    for (int kp = 0; kp < DK; ++kp) {
      const h8_t x = *reinterpret_cast<const h8_t*>(qrow + kp * 32 + g * 8);
      if constexpr (q_in_lds<D>())
        *q_slot(kp) = row_ok ? x : (h8_t)0;
      else
        qv[kp] = row_ok ? x : (h8_t)0;
    }
  };

  float m_run = kNegInf;
  float l_run = 0.f;
  f4_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = (f4_t)0.f;

  const char* k_head = reinterpret_cast<const char*>(a.k) + (int64_t)kvh * a.skh * ES;
  const char* v_head = reinterpret_cast<const char*>(a.v) + (int64_t)kvh * a.svh * ES;
  // Lane byte offsets inside a 16-token slab of one page (loop invariant).
  // K and V are both read as whole token rows: lane (g, r16) reads row
  // 4g+i, segments at head_dim r16*2*SEG (+ D/NSEG), so one load
  // instruction covers four rows (contiguous 256 B each at head_dim 128).  K then goes through LDS
  // into the MFMA operand layout (token per lane%16).
  // Sub-page blocks: token 4g+i sits in slot (4g+i) mod page_size of its
  // page (blocks start on page boundaries), again loop invariant.
  constexpr int SUB_SHIFT = MODE >= kModeSubpage ? MODE - kModeSubpage : 0;
  constexpr int SUB_PAGES = 16 >> SUB_SHIFT;  // pages per 16-token block
  uint32_t koff[4], voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = MODE >= kModeSubpage ? (4 * g + i) & ((1 << SUB_SHIFT) - 1) : 4 * g + i;
    koff[i] = (uint32_t)(((int64_t)row * a.sks + r16 * 2 * SEG) * ES);
    voff[i] = (uint32_t)(((int64_t)row * a.svs + r16 * 2 * SEG) * ES);
  }
  constexpr int KROW = k_stage_row_bytes<D>();
  const int p_first = page_of(a, t_begin);
  // Sub-page and generic blocks: the raw page ids of the block the next
  // load() reads, read with scalar loads one block ahead like pid_next;
  // columns past the item's last page are clamped to it (its tokens are
  // masked).  Generic mode (page sizes >= 3 that neither divide nor are a
  // multiple of 16; the MFMA engine sends 1 and 2 to the sub-page mode):
  // 16 tokens starting anywhere in a page span at most
  // floor((ps + 14) / ps) + 1 <= 6 pages, the block's first page and its
  // first token's slot (gen_r0) are found by an exact float-reciprocal
  // division, and each token's page index and slot follow from
  // pos = gen_r0 + token: (pos + 0.5) / ps is never within 0.5 / ps of an
  // integer, so truncating its float value is exact for the small pos here.
  constexpr int GEN_PAGES = 6;
  int ids_next[MODE >= kModeSubpage ? SUB_PAGES : (MODE == kModeGeneric ? GEN_PAGES : 1)];
  const int p_last = t_end > t_begin ? page_of(a, t_end - 1) : p_first;
  const float inv_ps = 1.0f / (float)a.ps;
  int gen_r0 = 0;
  auto fetch_ids = [&](int jb) {
    if constexpr (MODE >= kModeSubpage) {
      const int p0 = p_first + jb * SUB_PAGES;
#pragma unroll
      for (int k = 0; k < SUB_PAGES; ++k)
        ids_next[k] = load_uniform_i32(bt_row + (int64_t)min(p0 + k, p_last) * ids_stride);
    } else if constexpr (MODE == kModeGeneric) {
      const int t0 = t_begin + jb * kBlockTokens;
      int p0 = __builtin_amdgcn_readfirstlane((int)(((float)t0 + 0.5f) * inv_ps));
      p0 -= p0 * a.ps > t0 ? 1 : 0;  // exact for t0 < 2^23
      p0 += (p0 + 1) * a.ps <= t0 ? 1 : 0;
      gen_r0 = t0 - p0 * a.ps;
#pragma unroll
      for (int k = 0; k < GEN_PAGES; ++k)
        ids_next[k] = load_uniform_i32(bt_row + (int64_t)min(p0 + k, p_last) * ids_stride);
    }
  };

  // Uniform mode: raw page id of the block the next load() reads.  Each load()
  // consumes it and issues the scalar read of the following block's id, so
  // that read is in flight during a whole compute() (calls come in block
  // order wave, wave+nw, ...; past the split the last block's id is reread).
  int pid_next = phys_first;

  auto load = [&](Tile& t, int jb) {
    if constexpr (MODE == kModeUniform) {
      // page_size % 16 == 0 and splits start on page boundaries: the block
      // lives in one page, so its page id and base address are wave-uniform.
      const int jp = block_page(a, jb);
      const int slot0 = jb * kBlockTokens - jp * a.ps;
      const int phys = clamp_page(pid_next, a.num_pages);
      const int page_after = p_first + block_page(a, min(jb + nw, nblk - 1));
      pid_next = load_uniform_i32(bt_row + (int64_t)page_after * ids_stride);
      const char* kb = k_head + ((int64_t)phys * a.skp + (int64_t)slot0 * a.sks) * ES;
      const char* vb = v_head + ((int64_t)phys * a.svp + (int64_t)slot0 * a.svs) * ES;
#pragma unroll
      for (int i = 0; i < 4; ++i) t.k[i] = load_slice(kb + koff[i]);
#pragma unroll
      for (int i = 0; i < 4; ++i) t.v[i] = load_slice(vb + voff[i]);
    } else if constexpr (MODE >= kModeSubpage) {
      // page_size divides 16: the block covers SUB_PAGES whole pages whose
      // ids arrived during the previous compute(); lane group g picks the
      // page of its token 4g+i.  Past the item's end the clamped ids still
      // name valid pages (the tokens are masked in compute).
      // The ids are used up before the next block's are fetched into the
      // same registers.
#pragma unroll
      for (int k = 0; k < SUB_PAGES; ++k) ids_next[k] = clamp_page(ids_next[k], a.num_pages);
      const int64_t kpage = a.skp * ES, vpage = a.svp * ES;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c0 = ids_next[i >> SUB_SHIFT], c1 = ids_next[(4 + i) >> SUB_SHIFT];
        const int c2 = ids_next[(8 + i) >> SUB_SHIFT], c3 = ids_next[(12 + i) >> SUB_SHIFT];
        const int phys = g == 0 ? c0 : (g == 1 ? c1 : (g == 2 ? c2 : c3));
        t.k[i] = load_slice(k_head + (int64_t)phys * kpage + koff[i]);
        t.v[i] = load_slice(v_head + (int64_t)phys * vpage + voff[i]);
      }
      fetch_ids(min(jb + nw, nblk - 1));
    } else {
      // Generic page size (>= 3): token 4g+i is at pos = gen_r0 + 4g+i from
      // the start of the block's first page, i.e. in page pos / ps of the
      // block's (up to 6) prefetched ids, slot pos mod ps.  The ids are used
      // up before the next block's are fetched into the same registers.
#pragma unroll
      for (int k = 0; k < GEN_PAGES; ++k) ids_next[k] = clamp_page(ids_next[k], a.num_pages);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pos = gen_r0 + 4 * g + i;
        const int idx = (int)(((float)pos + 0.5f) * inv_ps);
        const int slot = pos - idx * a.ps;
        // idx in [0, 6): a binary mux over idx's bits.  (An equality select
        // chain was folded into an indexed read of the id array, which the
        // compiler placed in scratch memory: a vector memory round trip per
        // token that also drained the K/V loads in flight.)
        static_assert(GEN_PAGES == 6, "mux below covers 6 page ids");
        const bool b0 = (idx & 1) != 0;
        const int p01 = b0 ? ids_next[1] : ids_next[0];
        const int p23 = b0 ? ids_next[3] : ids_next[2];
        const int p45 = b0 ? ids_next[5] : ids_next[4];
        const int p03 = (idx & 2) ? p23 : p01;
        const int phys = (idx & 4) ? p45 : p03;
        const char* kr = k_head + ((int64_t)phys * a.skp + (int64_t)slot * a.sks + r16 * 2 * SEG) * ES;
        const char* vr = v_head + ((int64_t)phys * a.svp + (int64_t)slot * a.svs + r16 * 2 * SEG) * ES;
        t.k[i] = load_slice(kr);
        t.v[i] = load_slice(vr);
      }
      fetch_ids(min(jb + nw, nblk - 1));
    }
  };

  auto compute = [&](Tile& t, int jb) {
    const int t0 = t_begin + jb * kBlockTokens;
    const bool full = t0 + kBlockTokens <= t_end;
    // K rows -> LDS (row 4g+i, the lane's segments), then the MFMA A operand back
    // out: lane (g, r16) takes token r16, head_dim kp*32 + g*8 + [0, 8).
    // LDS accesses of one wave complete in order, so the reads see the
    // writes, and the next block's writes follow these reads.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t* dst = reinterpret_cast<uint32_t*>(k_stage + (4 * g + i) * KROW + r16 * SEG * 4);
      const HVec<NDW> kr = widen(t.k[i]);
#pragma unroll
      for (int w = 0; w < NDW; ++w) dst[(w / SEG) * (SEG_HALVES / 2) + w % SEG] = kr.w[w];
    }
    h8_t kk[DK];
#pragma unroll
    for (int kp = 0; kp < DK; ++kp)
      kk[kp] = *reinterpret_cast<const h8_t*>(k_stage + r16 * KROW + (kp * 32 + g * 8) * 2);
    // S^T[token 4g+i][row r16] over head_dim.
    f4_t sacc = (f4_t)0.f;
#pragma unroll
    for (int kp = 0; kp < DK; ++kp) {
      const h4_t k_lo = __builtin_shufflevector(kk[kp], kk[kp], 0, 1, 2, 3);
      const h4_t k_hi = __builtin_shufflevector(kk[kp], kk[kp], 4, 5, 6, 7);
      h8_t qk;
      if constexpr (q_in_lds<D>())
        qk = *q_slot(kp);
      else
        qk = qv[kp];
      const h4_t q_lo = __builtin_shufflevector(qk, qk, 0, 1, 2, 3);
      const h4_t q_hi = __builtin_shufflevector(qk, qk, 4, 5, 6, 7);
      sacc = mfma16<KVF>(k_lo, q_lo, sacc);
      sacc = mfma16<KVF>(k_hi, q_hi, sacc);
    }
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = sacc[i] * a.scale_log2;
    if (!full) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool valid = t0 + 4 * g + i < t_end;
        x[i] = valid ? x[i] : kNegInf;
        if (!valid) t.v[i].zero();  // stale cache slots may hold NaN/Inf
      }
    }
    float bm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    bm = fmaxf(bm, shfl_xor_f(bm, 16));
    bm = fmaxf(bm, shfl_xor_f(bm, 32));
    // Lazy rescaling: the reference m_run only moves when a score exceeds it
    // by more than kRescaleSlack (base-2 units), so weights stay <= 2^slack
    // and the O/l rescale is skipped (wave-uniformly) on most blocks.  Any
    // reference value gives the same O/l; partials carry it as their m.
    // Every block holds at least one valid token, so bm is finite.
    if (__builtin_amdgcn_ballot_w64(bm > m_run + kRescaleSlack) != 0) {
      const float m_new = fmaxf(m_run, bm);
      const float alpha = exp2_fast(m_run - m_new);  // 0 on the first block
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
      m_run = m_new;
    }
    h4_t ph;
    float psum = 0.f;  // l accumulates the same rounded weights P.V uses
    if constexpr (q_is_bf16<KVF>()) {
      // Pairs through the packed conversion; a rounded bf16 pair's floats
      // are its high and low halves shifted into place.
      typedef float f2_t __attribute__((ext_vector_type(2)));
      typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
      uint32_t u[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f2_t pf = {exp2_fast(x[2 * j] - m_run), exp2_fast(x[2 * j + 1] - m_run)};
        u[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(pf, b2_t));
        psum += __uint_as_float(u[j] << 16) + __uint_as_float(u[j] & 0xffff0000u);
      }
      typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
      ph = __builtin_bit_cast(h4_t, u2_t{u[0], u[1]});
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const _Float16 p = (_Float16)exp2_fast(x[i] - m_run);
        ph[i] = p;
        psum += (float)p;
      }
    }
    l_run += psum;
    HVec<NDW> vr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) vr[i] = widen(t.v[i]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      h4_t av;
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = vr[i].h(dt);
      o[dt] = mfma16<KVF>(av, ph, o[dt]);
    }
  };

  // This wave's blocks are wave, wave+nw, ...  The steady-state loop issues
  // the next block's loads unconditionally before computing the current one
  // (no control-flow join on the in-flight registers); the last one or two
  // blocks are peeled.
  const int n_mine = wave < nblk ? (nblk - wave + nw - 1) / nw : 0;
  Tile ta, tb;
  if (n_mine > 0) {
    int it = 0;
    fetch_ids(wave);
    load(ta, wave);
    load_q();
    for (; it + 2 < n_mine; it += 2) {
      load(tb, wave + (it + 1) * nw);
      compute(ta, wave + it * nw);
      load(ta, wave + (it + 2) * nw);
      compute(tb, wave + (it + 1) * nw);
    }
    if (it + 1 < n_mine) {
      load(tb, wave + (it + 1) * nw);
      compute(ta, wave + it * nw);
      compute(tb, wave + (it + 1) * nw);
    } else {
      compute(ta, wave + it * nw);
    }
  }

  // Row totals: the four 16-lane groups hold disjoint token subsets.
  float l_tot = l_run + shfl_xor_f(l_run, 16);
  l_tot += shfl_xor_f(l_tot, 32);
  auto o_slot = [&](int i, int dt) {
    return (dt / (2 * SEG)) * SEG_HALVES + (4 * g + i) * 2 * SEG + dt % (2 * SEG);
  };
  if (row_ok) {
    if (g == 0) sm_ml[wave * 16 + r16] = make_float2(m_run, l_tot);
    // Lane owns O[row r16][dim(4g+i, dt)]: for each i, NSEG runs of 2*SEG
    // consecutive floats, written as 16- or 8-byte vectors.
    float* dst = sm_o + (wave * a.gqa + r16) * wave_row_floats<D>();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT % 4 == 0) {
#pragma unroll
        for (int dt = 0; dt < DT; dt += 4)
          *reinterpret_cast<f4_t*>(dst + o_slot(i, dt)) = f4_t{o[dt][i], o[dt + 1][i], o[dt + 2][i], o[dt + 3][i]};
      } else {
#pragma unroll
        for (int dt = 0; dt < DT; dt += 2)
          *reinterpret_cast<float2*>(dst + o_slot(i, dt)) = make_float2(o[dt][i], o[dt + 1][i]);
      }
    }
  }
}

// Engine 1: VALU dot products with DPP row reductions.
template <int D, bool UNIFORM, int GQA_T>
__device__ __forceinline__ void wave_loop_valu(const Phase1Args& a, const int32_t* bt_row, int64_t ids_stride,
                                               int b, int kvh, int t_begin, int t_end, int nblk, int wave,
                                               int nw, int lane, float2* sm_ml, float* sm_o) {
  constexpr int DT = D / 16;  // halves per lane per token
  constexpr int NDW = DT / 2;
  const int g = lane >> 4;    // token group: tokens 4g+i of each block
  const int r16 = lane & 15;  // head_dim slice r16*DT .. +DT
  const int gqa = a.gqa;

  HVec<NDW> qh[GQA_T];
#pragma unroll
  for (int r = 0; r < GQA_T; ++r) {
    if (r < gqa) {
      const _Float16* qrow = a.q + (int64_t)b * a.sqb + (int64_t)(kvh * gqa + r) * a.sqh;
      qh[r] = load_hvec<NDW>(qrow + r16 * DT);
    } else {
      qh[r].zero();
    }
  }
  float m_run[GQA_T], l_run[GQA_T], acc[GQA_T][DT];
#pragma unroll
  for (int r = 0; r < GQA_T; ++r) {
    m_run[r] = kNegInf;
    l_run[r] = 0.f;
#pragma unroll
    for (int e = 0; e < DT; ++e) acc[r][e] = 0.f;
  }

  const int64_t koff_h = (int64_t)kvh * a.skh;
  const int64_t voff_h = (int64_t)kvh * a.svh;

  for (int j = wave; j < nblk; j += nw) {
    const int t0 = t_begin + j * kBlockTokens;
    const _Float16* krow[4];
    const _Float16* vrow[4];
    if constexpr (UNIFORM) {
      const int page = page_of(a, t0);
      const int phys = clamp_page(load_uniform_i32(bt_row + (int64_t)page * ids_stride), a.num_pages);
      const int slot0 = t0 - page * a.ps;
      const _Float16* kbase = a.k + (int64_t)phys * a.skp + koff_h + (int64_t)slot0 * a.sks;
      const _Float16* vbase = a.v + (int64_t)phys * a.svp + voff_h + (int64_t)slot0 * a.svs;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        krow[i] = kbase + (int64_t)(4 * g + i) * a.sks;
        vrow[i] = vbase + (int64_t)(4 * g + i) * a.svs;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tv = min(t0 + 4 * g + i, t_end - 1);
        const int page = page_of(a, tv);
        const int phys = clamp_page(bt_row[(int64_t)page * ids_stride], a.num_pages);
        const int slot = tv - page * a.ps;
        krow[i] = a.k + (int64_t)phys * a.skp + koff_h + (int64_t)slot * a.sks;
        vrow[i] = a.v + (int64_t)phys * a.svp + voff_h + (int64_t)slot * a.svs;
      }
    }
    HVec<NDW> kk[4], vv[4];
    bool valid[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kk[i] = load_hvec<NDW>(krow[i] + r16 * DT);
      vv[i] = load_hvec<NDW>(vrow[i] + r16 * DT);
      valid[i] = t0 + 4 * g + i < t_end;
      if (!valid[i]) vv[i].zero();
    }
    float vf[4][DT];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int e = 0; e < DT; ++e) vf[i][e] = (float)vv[i].h(e);
    }

#pragma unroll
    for (int r = 0; r < GQA_T; ++r) {
      if (r >= gqa) break;
      float sc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float part = 0.f;
#pragma unroll
        for (int w = 0; w < NDW; ++w) part = __builtin_amdgcn_fdot2(qh[r].h2(w), kk[i].h2(w), part, false);
        part = row16_sum(part);
        sc[i] = valid[i] ? part * a.scale_log2 : kNegInf;
      }
      const float bm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      const float m_new = fmaxf(m_run[r], bm);
      if (m_new == kNegInf) continue;  // this group has seen no valid token yet
      const float alpha = exp2_fast(m_run[r] - m_new);
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = exp2_fast(sc[i] - m_new);
      l_run[r] = l_run[r] * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
      for (int e = 0; e < DT; ++e) {
        float t = acc[r][e] * alpha;
#pragma unroll
        for (int i = 0; i < 4; ++i) t = fmaf(p[i], vf[i][e], t);
        acc[r][e] = t;
      }
      m_run[r] = m_new;
    }
  }

  // Merge the four token groups of this wave (lanes r16, r16+16, ...).
#pragma unroll
  for (int r = 0; r < GQA_T; ++r) {
    if (r >= gqa) break;
    float M = fmaxf(m_run[r], shfl_xor_f(m_run[r], 16));
    M = fmaxf(M, shfl_xor_f(M, 32));
    const float c = (m_run[r] == kNegInf) ? 0.f : exp2_fast(m_run[r] - M);
    float l = l_run[r] * c;
    l += shfl_xor_f(l, 16);
    l += shfl_xor_f(l, 32);
#pragma unroll
    for (int e = 0; e < DT; ++e) {
      float v = acc[r][e] * c;
      v += shfl_xor_f(v, 16);
      v += shfl_xor_f(v, 32);
      acc[r][e] = v;
    }
    if (g == 0) {
      if (r16 == 0) sm_ml[wave * 16 + r] = make_float2(M, l);
      float* dst = sm_o + (wave * gqa + r) * wave_row_floats<D>() + r16 * DT;
#pragma unroll
      for (int e = 0; e < DT; ++e) dst[e] = acc[r][e];
    }
  }
}

// ---------------------------------------------------------------------------
// Work items.  Workgroup (s, h, b) of the grid (grid_pos: the grid
// coordinates, or a bijection of them that pairs kv heads on an XCD) has
// index g = s + S*(h + Hkv*b) and processes one item: a page range of one
// (sequence, kv head) unit, writing its partial to slot g of the workspace.
// The items of a unit occupy the consecutive slots [slot0, slot0 + nsplit).
//  * Static items (an explicit split count, or every sequence at full
//    capacity): item g is split s of unit (b, h), pages [s*pps, (s+1)*pps).
//  * Planned items (heuristic split count, batch <= kPlanMaxBatch): every
//    workgroup reads all sequence lengths and computes the same plan - the
//    smallest chunk of c pages (c >= min_chunk) such that the units need at
//    most G items, each unit cut into ceil(pages/c) chunks (an empty unit
//    keeps one item, which writes its zero rows) - then takes item g in
//    (sequence, kv head, chunk) order.  Ragged batches thus spread their
//    pages evenly over the grid instead of leaving the splits of short
//    sequences empty.
// ---------------------------------------------------------------------------
struct WorkItem {
  int b, kvh;
  int p_begin, p_end;  // logical pages [p_begin, p_end) of sequence b
  int L;               // tokens of sequence b
  int nsplit;          // items of the unit; 0: the unit is empty (write zeros)
  int slot0;           // workspace slot of the unit's first item
  int col_max;         // last page-id column that may be read speculatively
  int valid;           // 0: no item for this workgroup
  const int32_t* ids_row;
  int64_t ids_stride;
};

// Wave-wide integer reductions: DPP within each 16-lane row, then the four
// row results combined through readlane (wave-uniform result).
__device__ __forceinline__ int row16_sum_i32(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  x += __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  x += __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false);  // row_half_mirror
  x += __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false);  // row_mirror
  return x;
}

__device__ __forceinline__ int wave_sum_i32(int x) {
  x = row16_sum_i32(x);
  return __builtin_amdgcn_readlane(x, 0) + __builtin_amdgcn_readlane(x, 16) + __builtin_amdgcn_readlane(x, 32) +
         __builtin_amdgcn_readlane(x, 48);
}

__device__ __forceinline__ int wave_max_i32(int x) {
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false));
  return max(max(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
             max(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}

// Inclusive prefix sum over the 64 lanes: row_shr steps (bound_ctrl shifts
// in zeros) scan each 16-lane row, then each row adds the totals of the rows
// before it.
__device__ __forceinline__ int wave_incl_scan_i32(int x, int lane) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(x, 15);
  const int r1 = __builtin_amdgcn_readlane(x, 31);
  const int r2 = __builtin_amdgcn_readlane(x, 47);
  const int row = lane >> 4;
  return x + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

// CSR row of sequence b: first page-id offset, page count and tokens.  The
// offsets are clamped into indices[0, max_pages) (max_pages holds the
// length of `indices` in CSR mode), so a malformed indptr cannot make the
// kernel read outside the array; last_page_len is clamped to the page.
__device__ __forceinline__ void csr_row(const Phase1Args& a, int b, int* row, int* pages, int* len) {
  const int r0 = min(max(a.indptr[b], 0), a.max_pages);
  const int r1 = min(max(a.indptr[b + 1], r0), a.max_pages);
  *row = r0;
  *pages = r1 - r0;
  *len = *pages > 0 ? (*pages - 1) * a.ps + min(max(a.lpl[b], 1), a.ps) : 0;
}

// Sequence table spread over the wave: lane l holds sequences l + 64k,
// k < NK (NK = 1 for batches up to 64, else 4).
template <int NK>
struct SeqTable {
  int len[NK];    // tokens (0 past the batch)
  int pages[NK];  // pages in use
  int row[NK];    // CSR: offset of the sequence's page ids in `indices`
};

// Raw words of the sequence table for up to 256 sequences (lane l holds
// sequences l + 64k): CSR indptr[b], indptr[b + 1] and last_page_len[b];
// the dense table reads seq_lens[b] into all three.  A workgroup issues
// these loads before its first page-id read and uses them after it, so the
// two share one memory round trip; every load is unconditional (a lane past
// the batch re-reads the last sequence's words), so no branch has to wait
// for any of them.
struct SeqRaw {
  int r0[4], r1[4], r2[4];
};

__device__ __forceinline__ SeqRaw issue_seq_table(const Phase1Args& a, int lane) {
  SeqRaw r;
  const int32_t* p0 = a.csr ? a.indptr : a.sl;
  const int32_t* p1 = a.csr ? a.indptr + 1 : a.sl;
  const int32_t* p2 = a.csr ? a.lpl : a.sl;
  const int64_t stride = a.csr ? 1 : a.ssl;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t off = (int64_t)min(lane + 64 * k, a.batch - 1) * stride;
    r.r0[k] = p0[off];
    r.r1[k] = p1[off];
    r.r2[k] = p2[off];
  }
  return r;
}

template <int NK>
__device__ __forceinline__ SeqTable<NK> seq_table(const Phase1Args& a, const SeqRaw& r, int lane) {
  SeqTable<NK> t;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const bool in = lane + 64 * k < a.batch;
    int len, pages, row = 0;
    if (a.csr) {
      row = min(max(r.r0[k], 0), a.max_pages);
      pages = min(max(r.r1[k], row), a.max_pages) - row;
      len = pages > 0 ? (pages - 1) * a.ps + min(max(r.r2[k], 1), a.ps) : 0;
    } else {
      len = max(r.r0[k], 0);
      pages = min(pages_for(a, len), a.max_pages);
    }
    t.len[k] = in ? len : 0;
    t.pages[k] = in ? pages : 0;
    t.row[k] = in ? row : 0;
  }
  return t;
}

// Value of lane (b % 64) of register k = b / 64 (b wave-uniform).
template <int NK>
__device__ __forceinline__ int seq_lane_value(const int (&v)[NK], int b) {
  const int l = b & 63;
  int x = __builtin_amdgcn_readlane(v[0], l);
#pragma unroll
  for (int k = 1; k < NK; ++k)
    if ((b >> 6) == k) x = __builtin_amdgcn_readlane(v[k], l);
  return x;
}

// ceil(p / c) for 0 <= p, c < 2^23: a float estimate corrected with exact
// 24-bit products (the estimate is within one of the quotient).
__device__ __forceinline__ int ceil_div_u23(int p, int c, float rc) {
  int n = (int)__builtin_ceilf((float)p * rc);
  n += (int)__umul24(n, c) < p ? 1 : 0;
  n -= (n > 0 && (int)__umul24(n - 1, c) >= p) ? 1 : 0;
  return n;
}

// Items per sequence with chunks of c pages (an empty sequence keeps one).
__device__ __forceinline__ int items_for(int pages, int c, float rc) { return max(ceil_div_u23(pages, c, rc), 1); }

// Items the units need for each of J chunk sizes (wave-uniform totals).  The
// J evaluations are independent, so their latencies overlap.
template <int NK, int J>
__device__ __forceinline__ void plan_counts(const Phase1Args& a, const SeqTable<NK>& t, const int (&c)[J],
                                            int (&n)[J], int lane) {
  float rc[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    rc[j] = 1.0f / (float)c[j];
    n[j] = 0;
  }
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const bool in = lane + 64 * k < a.batch;
#pragma unroll
    for (int j = 0; j < J; ++j) n[j] += in ? items_for(t.pages[k], c[j], rc[j]) : 0;
  }
#pragma unroll
  for (int j = 0; j < J; ++j) n[j] = row16_sum_i32(n[j]);
#pragma unroll
  for (int j = 0; j < J; ++j)
    n[j] = (__builtin_amdgcn_readlane(n[j], 0) + __builtin_amdgcn_readlane(n[j], 16) +
            __builtin_amdgcn_readlane(n[j], 32) + __builtin_amdgcn_readlane(n[j], 48)) *
           a.hkv;
}

template <int NK>
__device__ WorkItem plan_item(const Phase1Args& a, const SeqTable<NK>& t, int g, int G, int lane) {
  WorkItem w{};  // a slot without an item keeps defined (zero) fields
  w.ids_row = a.bt;
  int tot = 0, pmax = 0;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    tot += t.pages[k];
    pmax = max(pmax, t.pages[k]);
  }
  tot = wave_sum_i32(tot);
  pmax = max(wave_max_i32(pmax), 1);
  // Chunk size: the smallest c >= c_lo whose item count fits the grid would
  // be ideal, but every probe costs a pass over the table, so at most two
  // are made.  c_lo = ceil(unit pages / G) (fits when the lengths divide
  // evenly); then c_est, which assumes each non-empty unit rounds up by half
  // a chunk; failing that c_hi = ceil(unit pages / (G - units)), which
  // always fits since sum(ceil(p / c)) <= unit pages / c + units (and so
  // does pmax: one item per unit, G >= units).
  const int units = a.batch * a.hkv;
  const int64_t unit_pages = (int64_t)tot * a.hkv;
  int c = min(max(max(a.min_chunk, (int)((unit_pages + G - 1) / G)), 1), pmax);
  int n1[1], c1[1] = {c};
  plan_counts<NK, 1>(a, t, c1, n1, lane);
  if (n1[0] > G) {
    int c_hi = pmax;
    if (G > units) c_hi = min(c_hi, (int)((unit_pages + (G - units) - 1) / (G - units)));
    const int half = G - units / 2;
    int c_est = half > 0 ? (int)((unit_pages + half - 1) / half) : c_hi;
    c_est = max(c + 1, min(c_est, c_hi));
    c1[0] = c_est;
    plan_counts<NK, 1>(a, t, c1, n1, lane);
    c = n1[0] <= G ? c_est : max(c_hi, c_est);
  }
  // Locate item g: units in (sequence, kv head) order, n_b items each.
  w.valid = 0;
  int carry = 0;
  const float rc = 1.0f / (float)c;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    if (64 * k >= a.batch) break;
    const int b = lane + 64 * k;
    const int nb = b < a.batch ? items_for(t.pages[k], c, rc) : 0;
    const int x = nb * a.hkv;
    const int incl = wave_incl_scan_i32(x, lane) + carry;
    const int excl = incl - x;
    const uint64_t hit = __builtin_amdgcn_ballot_w64(b < a.batch && excl <= g && g < incl);
    if (hit != 0) {
      const int l = (int)__builtin_ctzll(hit);
      const int first = __builtin_amdgcn_readlane(excl, l);
      const int n = __builtin_amdgcn_readlane(nb, l);
      const int pages = __builtin_amdgcn_readlane(t.pages[k], l);
      const int r = g - first;
      w.b = 64 * k + l;
      w.kvh = r / n;
      const int chunk = r - w.kvh * n;
      w.p_begin = chunk * c;
      w.p_end = min(w.p_begin + c, pages);
      w.L = __builtin_amdgcn_readlane(t.len[k], l);
      w.nsplit = pages > 0 ? n : 0;
      w.slot0 = first + w.kvh * n;
      w.col_max = pages - 1;
      w.ids_row = a.csr ? a.bt + __builtin_amdgcn_readlane(t.row[k], l) : a.bt + (int64_t)w.b * a.sbb;
      w.valid = 1;
      break;
    }
    carry = __builtin_amdgcn_readlane(incl, 63);
  }
  w.ids_stride = a.csr ? 1 : a.sbp;
  return w;
}

// The static item of workgroup (s, kvh, b) given the sequence's length and
// page count.  The dense table splits every row's max_pages columns into
// num_splits ranges of pps pages; a CSR index has no common row width, so
// each sequence's own pages are cut into num_splits ranges.
__device__ __forceinline__ WorkItem static_item(const Phase1Args& a, int s, int kvh, int b, int L, int pages,
                                                const int32_t* ids_row, int64_t ids_stride) {
  WorkItem w;
  const int pps = a.csr ? max((pages + a.num_splits - 1) / a.num_splits, 1) : a.pps;
  w.b = b;
  w.kvh = kvh;
  w.L = L;
  w.p_begin = s * pps;
  w.p_end = min(w.p_begin + pps, pages);
  w.nsplit = (pages + pps - 1) / pps;
  w.slot0 = (b * a.hkv + kvh) * a.num_splits;
  w.col_max = a.csr ? pages - 1 : a.max_pages - 1;
  // Splits past the sequence's last page do nothing, except split 0 of an
  // empty sequence, which writes its zero rows.
  w.valid = s < w.nsplit || s == 0;
  w.ids_row = ids_row;
  w.ids_stride = ids_stride;
  return w;
}

// Planned mode: read every sequence length; with every sequence at full
// capacity the static split is already even (balance == 1) or, on an
// oversubscribed grid (balance >= 2), the static splits run on the first
// workgroups (one item per unit, workgroup g = unit, when the static rule
// gives one split) and the other workgroups exit; otherwise plan the items.
template <int NK>
__device__ __forceinline__ WorkItem resolve_item(const Phase1Args& a, const SeqRaw& raw, int s, int h, int bz, int g,
                                                 int G, int lin, const int32_t* static_row, int lane) {
  const SeqTable<NK> t = seq_table<NK>(a, raw, lane);
  bool full = !a.csr;
#pragma unroll
  for (int k = 0; k < NK; ++k)
    if (lane + 64 * k < a.batch && t.pages[k] != a.max_pages) full = false;
  if (__builtin_amdgcn_ballot_w64(!full) == 0) {
    if (a.balance >= 2) {
      // The static splits, s0 per unit of pps pages, on the first units * s0
      // workgroups in order: unit g / s0, split g mod s0, whose partials
      // take the unit's s0 consecutive slots (the launch keeps head pairing
      // off when s0 > 1, so g is the linear index and the active workgroups
      // spread over the XCDs).  With s0 = 1 (pps = max_pages) each unit is
      // one item that writes the output rows and never a partial, so its
      // slot is the workgroup's own (g, which the work list's record check
      // expects); with pair_heads, units 2r and 2r+1 (kv heads 2m, 2m+1 of
      // one sequence) then go to workgroups 8 apart, as grid_pos does for
      // splits.
      WorkItem w;
      const int units = a.batch * a.hkv;
      const int s0 = a.balance - 1;  // 1, 2 or 3 (setup_launch)
      const bool paired = s0 == 1 && a.pair_heads && units % 16 == 0;
      const int gu = paired ? 2 * (((lin >> 4) << 3) | (lin & 7)) + ((lin >> 3) & 1) : g;
      // g / s0 by a shift or a multiply (exact for g < 2^16; G is far below)
      const int q = s0 == 2 ? g >> 1 : s0 == 3 ? (int)(((uint32_t)g * 43691u) >> 17) : (paired ? (lin < units ? gu : units) : g);
      const int u = min(q, units - 1);
      w.b = u / a.hkv;
      w.kvh = u - w.b * a.hkv;
      w.p_begin = s0 > 1 ? (g - q * s0) * a.pps : 0;
      w.p_end = min(w.p_begin + a.pps, a.max_pages);
      w.L = seq_lane_value<NK>(t.len, w.b);
      w.nsplit = a.max_pages > 0 ? s0 : 0;
      w.slot0 = s0 > 1 ? q * s0 : g;
      w.col_max = a.max_pages - 1;
      w.valid = q < units;
      w.ids_row = a.bt + (int64_t)w.b * a.sbb;
      w.ids_stride = a.sbp;
      return w;
    }
    return static_item(a, s, h, bz, seq_lane_value<NK>(t.len, bz), a.max_pages, static_row, a.sbp);
  }
  return plan_item<NK>(a, t, g, G, lane);
}

// The work item of workgroup (s, h, bz) = slot g: the in-kernel plan when
// a.balance is set, else the static split.  raw is issue_seq_table()'s
// loads; static_len is seq_lens[bz] (dense) or any word (CSR).  The decode
// kernel and the work-list planner both call this, so a planned launch runs
// exactly the items of an unplanned one.
__device__ __forceinline__ WorkItem resolve_workgroup(const Phase1Args& a, const SeqRaw& raw, int s, int h, int bz,
                                                      int g, int G, int lin, const int32_t* static_row,
                                                      int static_len, int lane) {
  if (a.balance) {
    if (a.batch <= 64) return resolve_item<1>(a, raw, s, h, bz, g, G, lin, static_row, lane);
    return resolve_item<4>(a, raw, s, h, bz, g, G, lin, static_row, lane);
  }
  if (a.csr) {
    int row, pages, L;
    csr_row(a, bz, &row, &pages, &L);
    return static_item(a, s, h, bz, L, pages, a.bt + row, 1);
  }
  const int L = max(static_len, 0);
  return static_item(a, s, h, bz, L, min(pages_for(a, L), a.max_pages), static_row, a.sbp);
}

// Work list (pad_decode_plan_worklist): a header of kWlHeaderInts int32
// {magic, plan key, G} and one record of kWlRecordInts int32 per workgroup
// slot g: {b, kvh, p_begin, p_end, L, nsplit, slot0, col_max, valid, row
// (CSR offset of the sequence's ids, else 0), 6 unused, then the raw page id
// of the first block of waves 0-7 (whole-page blocks; 0 otherwise), 8
// unused}.
constexpr int kWlHeaderInts = 32;
constexpr int kWlRecordInts = 32;
constexpr int kWlMagic = 0x574c4150;  // "PALW"

// Record g of a.worklist as a work item and the raw first page id of this
// wave's first block.  False (use the in-kernel plan) when the header does
// not carry this launch's plan key.  A record that does not describe an
// item of this launch's shapes is treated as no item, so a stale list can
// give wrong rows but never reads or writes out of bounds.
__device__ __forceinline__ bool worklist_item(const Phase1Args& a, int g, int G, int wave, WorkItem& w, int& pid) {
  const int32_t* r = a.worklist + kWlHeaderInts + (int64_t)kWlRecordInts * g;
  const int magic = load_uniform_i32(a.worklist);
  const int key = load_uniform_i32(a.worklist + 1);
  int f[10];
#pragma unroll
  for (int i = 0; i < 10; ++i) f[i] = load_uniform_i32(r + i);
  pid = load_uniform_i32(r + 16 + wave);
  // The record's values are only used past the header check, so the
  // compiler would sink their loads below it: a second round trip.  Pinning
  // them here keeps the header and the record in one.
#pragma unroll
  for (int i = 0; i < 10; ++i) asm volatile("" : "+s"(f[i]));
  asm volatile("" : "+s"(pid));
  if (magic != kWlMagic || key != a.wl_key) return false;
  w.b = f[0];
  w.kvh = f[1];
  w.p_begin = f[2];
  w.p_end = f[3];
  w.L = f[4];
  w.nsplit = f[5];
  w.slot0 = f[6];
  w.col_max = f[7];
  const int row = f[9];
  const bool ok = f[8] != 0 && w.b >= 0 && w.b < a.batch && w.kvh >= 0 && w.kvh < a.hkv && w.p_begin >= 0 &&
                  w.p_begin <= w.p_end && w.p_end <= w.col_max + 1 && w.L >= 0 && w.nsplit >= 0 &&
                  w.nsplit <= G && w.slot0 >= 0 && w.slot0 <= G - w.nsplit &&
                  (w.nsplit == 0 || (g >= w.slot0 && g < w.slot0 + w.nsplit)) && row >= 0 &&
                  (int64_t)row + w.col_max < a.max_pages;
  w.valid = ok ? 1 : 0;
  w.ids_row = a.csr ? a.bt + row : a.bt + (int64_t)(ok ? w.b : 0) * a.sbb;
  w.ids_stride = a.csr ? 1 : a.sbp;
  return true;
}

// Minimum waves per SIMD each phase-1 instantiation is compiled for (it
// caps the registers per lane at 512 / waves).  The generic page-size mode
// of head_dim 128 gets 2 (256 registers): its six prefetched page ids did
// not fit 168 registers without one VGPR spilled to scratch; so do the
// bfloat16 sub-page modes of head_dim 128 (2 VGPRs spilled at page size 4).
constexpr int phase1_waves_per_simd(int d, int engine, int mode, int kvf) {
  const bool wide = d == 128 && (mode == 0 || ((kvf == kKvBF16 || kvf == kKvE4M3B || kvf == kKvE5M2B) &&
                                                 mode >= kModeSubpage));
  return engine == 0 ? (d <= 128 ? (wide ? 2 : 3) : 1) : 1;
}

// Most waves in one workgroup.  head_dim 256 takes at most 4, so that each
// SIMD runs one wave of the workgroup and that wave has the whole register
// file (256 VGPRs plus AGPRs for spills): with 5 or more waves two share a
// SIMD's 256 VGPRs, and the loop spilled 7-10 VGPRs to scratch memory.
constexpr int max_group_waves(int d) { return d >= 256 ? 4 : kMaxWaves; }

// The (split, kv head, sequence) of this workgroup.  Normally the grid
// coordinates.  With pair_heads (head_dim rows that are not a multiple of
// 128 bytes, so kv heads 2m and 2m+1 share a cache line in every token
// slot; an even head count; G a multiple of 16) linear workgroup L takes
// head parity (L / 8) mod 2 and the rest of its position from the other
// bits: the two workgroups of a head pair are 8 apart, which the dispatcher
// places on the same XCD one after the other, so the line they share is
// fetched into that XCD's L2 once.  Any bijection of the grid is correct;
// this one only changes what shares a cache.
__device__ __forceinline__ void grid_pos(const Phase1Args& a, int& s, int& h, int& bz, int& lin) {
  s = blockIdx.x;
  h = blockIdx.y;
  bz = blockIdx.z;
  lin = blockIdx.x + a.num_splits * (blockIdx.y + a.hkv * blockIdx.z);
  if (a.pair_heads) {
    const int rest = ((lin >> 4) << 3) | (lin & 7);
    const int q = rest / a.num_splits;
    const int half = a.hkv >> 1;
    s = rest - q * a.num_splits;
    bz = q / half;
    h = 2 * (q - bz * half) + ((lin >> 3) & 1);
  }
}

// Work-list planner: one wave per workgroup slot of the decode grid, run
// once per decode step (the sequence lengths and page ids it reads must not
// change before the launches that use the list).  Lane i < 32 writes word i
// of the record; slot 0 also writes the header.
__global__ __launch_bounds__(64) void pad_plan_kernel(const Phase1Args a, int32_t* wl) {
  int s, h, bz, lin;
  grid_pos(a, s, h, bz, lin);
  const int lane = threadIdx.x;
  const int g = s + a.num_splits * (h + a.hkv * bz);
  const int G = a.num_splits * a.hkv * a.batch;
  const int32_t* static_row = a.bt + (int64_t)bz * a.sbb;
  const SeqRaw raw = issue_seq_table(a, lane);
  const int static_len = load_uniform_i32(a.csr ? a.indptr : a.sl + (int64_t)bz * a.ssl);
  const WorkItem it = resolve_workgroup(a, raw, s, h, bz, g, G, lin, static_row, static_len, lane);
  int v = 0;
  switch (lane) {
    case 0: v = it.b; break;
    case 1: v = it.kvh; break;
    case 2: v = it.p_begin; break;
    case 3: v = it.p_end; break;
    case 4: v = it.L; break;
    case 5: v = it.nsplit; break;
    case 6: v = it.slot0; break;
    case 7: v = it.col_max; break;
    case 8: v = it.valid; break;
    case 9: v = a.csr ? (int)(it.ids_row - a.bt) : 0; break;
    default: break;
  }
  // A slot without an item gets an all-zero record (valid = 0), so lists
  // planned from the same inputs are identical word for word.
  if (!it.valid) v = 0;
  // The first page id of wave w's first block, as the decode kernel's
  // first_page_id() reads it (whole-page blocks only).
  const int w = lane - 16;
  if (w >= 0 && w < a.nw && it.valid && it.col_max >= 0 && a.ps % kBlockTokens == 0) {
    const int col = min(it.p_begin + block_page(a, w), it.col_max);
    v = it.ids_row[(int64_t)col * it.ids_stride];
  }
  int32_t* r = wl + kWlHeaderInts + (int64_t)kWlRecordInts * g;
  if (lane < kWlRecordInts) r[lane] = v;
  if (g == 0 && lane < kWlHeaderInts) wl[lane] = lane == 0 ? kWlMagic : (lane == 1 ? a.wl_key : (lane == 2 ? G : 0));
}

// Phase 1: one workgroup per (split, kv head, sequence).  KVF: the caches'
// element format (fp16, or fp8 on the MFMA engine).
template <int D, int MODE, int ENGINE, int GQA_T, int KVF = kKvF16>
__global__ __launch_bounds__(max_group_waves(D) * 64)
    __attribute__((amdgpu_waves_per_eu(phase1_waves_per_simd(D, ENGINE, MODE, KVF))))
void pad_phase1_kernel(const Phase1Args a) {
#ifdef PAD_TIMELINE
  const unsigned long long tl_entry = __builtin_amdgcn_s_memrealtime();
  const unsigned long long tl_xcc = (unsigned long long)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15) << 32;
#define PAD_TL_NOTE(item_slot, flags) \
  PAD_TL_AT(lin, PAD_TL_INFO, (unsigned long long)(uint32_t)(item_slot) | tl_xcc | ((unsigned long long)(flags) << 40))
#else
#define PAD_TL_NOTE(item_slot, flags) \
  do {                                \
  } while (0)
#endif
  extern __shared__ float4 smem_f4[];
  float2* sm_ml = reinterpret_cast<float2*>(smem_f4);  // [nw][16]
  const int nw = a.nw;
  float* sm_o = reinterpret_cast<float*>(smem_f4) + nw * 32;  // [nw][gqa][D + 4]
  // [nw] K staging tiles (MFMA engine), after the wave states.
  char* k_stage_all = reinterpret_cast<char*>(sm_o + nw * a.gqa * wave_row_floats<D>());

  int s, h, bz, lin;
  grid_pos(a, s, h, bz, lin);
  PAD_TL_AT(blockIdx.x + a.num_splits * (blockIdx.y + a.hkv * blockIdx.z), PAD_TL_ENTRY, tl_entry);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = s + a.num_splits * (h + a.hkv * bz);
  const int G = a.num_splits * a.hkv * a.batch;

  // With a work list, the item and its first page ids arrive in one round
  // trip.  Otherwise, with the dense table, read the first page id of this
  // workgroup's static split before the sequence lengths arrive; it stays
  // valid whenever the item turns out to be the static one.
  WorkItem it;
  int phys_first = 0;
  bool first_known;
  if (a.worklist != nullptr && worklist_item(a, g, G, wave, it, phys_first)) {
    first_known = true;
  } else {
    // The sequence table's loads go first, then the page id and this
    // workgroup's sequence length: one round trip for all of them.  The
    // page-id read has no branch (a CSR index or an empty table reads a
    // valid word that is never used), as a value loaded under a branch
    // would be waited for where the branch joins, before the later loads.
    const SeqRaw raw = issue_seq_table(a, lane);
    const int32_t* static_row = a.bt + (int64_t)bz * a.sbb;
    if constexpr (ENGINE == 0 && MODE == kModeUniform) {
      const int col = min(s * a.pps + block_page(a, wave), a.max_pages - 1);
      const bool use = !a.csr && a.max_pages > 0;
      phys_first = load_uniform_i32(use ? static_row + (int64_t)col * a.sbp : (a.csr ? a.indptr : a.sl));
    }
    const int static_len = load_uniform_i32(a.csr ? a.indptr : a.sl + (int64_t)bz * a.ssl);
    it = resolve_workgroup(a, raw, s, h, bz, g, G, lin, static_row, static_len, lane);
    first_known = !a.csr && it.b == bz && it.p_begin == s * a.pps;
  }
  PAD_TL(lin, PAD_TL_ITEM);
  if (!it.valid) {
    PAD_TL_NOTE(-1, PAD_TL_F_NO_ITEM);
    PAD_TL(lin, PAD_TL_EXIT);
    return;
  }
  const int b = it.b;
  const int kvh = it.kvh;
  const int nsplit = it.nsplit;
  const int gqa = a.gqa;
  const int total4 = gqa * (D / 4);
  _Float16* out_bh = a.out + (int64_t)b * a.sob + (int64_t)(kvh * gqa) * a.soh;
  if (nsplit == 0) {  // seq_len == 0: the output rows are zeros
    for (int e = threadIdx.x; e < total4; e += nw * 64) {
      const int row = e / (D / 4);
      *reinterpret_cast<h4_t*>(out_bh + (int64_t)row * a.soh + (e - row * (D / 4)) * 4) = (h4_t)0;
    }
    PAD_TL_NOTE(g, PAD_TL_F_SINGLE);
    PAD_TL(lin, PAD_TL_EXIT);
    return;
  }
  if constexpr (ENGINE == 0 && MODE == kModeUniform) {
    if (!first_known) phys_first = first_page_id(a, it.ids_row, it.ids_stride, it.col_max, it.p_begin, wave);
  }
  const int t_begin = it.p_begin * a.ps;
  const int t_end = min(it.p_end * a.ps, it.L);
  const int nblk = (t_end - t_begin + kBlockTokens - 1) / kBlockTokens;

  if constexpr (ENGINE == 0) {
    wave_loop_mfma<D, MODE, KVF>(a, phys_first, it.ids_row, it.ids_stride, b, kvh, t_begin, t_end, nblk, wave,
                                 nw, lane, sm_ml, sm_o, k_stage_all + wave * k_stage_bytes<D>(),
                                 k_stage_all + nw * k_stage_bytes<D>());
  } else {
    wave_loop_valu<D, MODE == kModeUniform, GQA_T>(a, it.ids_row, it.ids_stride, b, kvh, t_begin, t_end, nblk, wave, nw, lane,
                                      sm_ml, sm_o);
  }
  __syncthreads();
  PAD_TL(lin, PAD_TL_LOOP_END);

  // Merge the waves' states: threads over (row, 4 consecutive d).  With a
  // single split the result is final; otherwise it is this split's partial.
  // Partials are stored and later loaded with device-scope (SC1) buffer
  // accesses, which are coherent across the XCDs' L2 caches on their own, so
  // publishing a partial needs no cache writeback.  The items of a (sequence,
  // kv head) own consecutive slots, addressed with 32-bit byte offsets.
  const int64_t seq_row0 = (int64_t)it.slot0 * gqa;
  const uint32_t region_rows = (uint32_t)(nsplit * gqa);
  const __amdgpu_buffer_rsrc_t o_rsrc = make_rsrc(a.o_part + seq_row0 * D, region_rows * D * 4u);
  const __amdgpu_buffer_rsrc_t ml_rsrc = make_rsrc(a.ml_part + seq_row0, region_rows * 8u);
  const int my_split = g - it.slot0;
  for (int e = threadIdx.x; e < total4; e += nw * 64) {
    const int row = e / (D / 4);
    const int col = (e - row * (D / 4)) * 4;
    // Unrolled over the largest wave count, so all LDS reads issue together.
    float2 ml[kMaxWaves];
    f4_t ow[kMaxWaves];
#pragma unroll
    for (int w = 0; w < kMaxWaves; ++w) {
      if (w < nw) {
        ml[w] = sm_ml[w * 16 + row];
        ow[w] = *reinterpret_cast<const f4_t*>(sm_o + (w * gqa + row) * wave_row_floats<D>() + col);
      }
    }
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kMaxWaves; ++w)
      if (w < nw) M = fmaxf(M, ml[w].x);
    f4_t acc = (f4_t)0.f;
    float Ls = 0.f;
#pragma unroll
    for (int w = 0; w < kMaxWaves; ++w) {
      if (w < nw) {
        const float c = (ml[w].x == kNegInf) ? 0.f : exp2_fast(ml[w].x - M);
        Ls += c * ml[w].y;
        acc += c * ow[w];
      }
    }
    if (nsplit == 1) {
      // Ls >= 1: the max token contributes 2^0.  fp8 caches: V's scale too.
      const float inv = (kv_is_fp8<KVF>() ? a.v_fix : 1.f) / Ls;
      h4_t hv;
#pragma unroll
      for (int i = 0; i < 4; ++i) hv[i] = round16<KVF>(acc[i] * inv);
      *reinterpret_cast<h4_t*>(out_bh + (int64_t)row * a.soh + col) = hv;
    } else {
      const uint32_t r = (uint32_t)(my_split * gqa + row);
      store_device(o_rsrc, (r * D + col) * 4u, acc);
      if (col == 0) store_device(ml_rsrc, r * 8u, make_float2(M, Ls));
    }
  }
  if (nsplit == 1) {
    PAD_TL(lin, PAD_TL_PUBLISHED);
    PAD_TL_NOTE(g, PAD_TL_F_SINGLE);
    PAD_TL(lin, PAD_TL_EXIT);
    return;
  }

  // Split-K merge, fused: the last workgroup of this (sequence, kv head) to
  // arrive folds every split's partial into the output.  A workgroup counts
  // itself in only after its partial stores have completed at device scope
  // (vmcnt(0) covers stores on this architecture); the last one to arrive
  // reads the partials with device-scope loads and resets the counter to
  // zero for the next launch.
  //
  // Past kTwoLevelSplits splits one workgroup reading every partial is the
  // tail (256 splits of 8 rows: 1 MB, ~17 us), so the merge takes two
  // levels: the last arrival of each group of 16 consecutive splits folds
  // the group into the slot of its first split (nothing else reads those
  // slots any more), publishes it like a partial and counts the group in;
  // the last group folds the group results.
  __shared__ int s_last;
  int* unit_counter = a.counters + (int64_t)b * a.hkv + kvh;
  int stride = 1, count = nsplit;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  PAD_TL(lin, PAD_TL_PUBLISHED);
  int tl_flags = 0;
  (void)tl_flags;
  if (nsplit > kTwoLevelSplits) {
    const int grp0 = my_split & ~15;  // first split of this group
    const int gsize = min(16, nsplit - grp0);
    int* group_counter = a.counters + (int64_t)a.batch * a.hkv + it.slot0 + grp0;
    if (threadIdx.x == 0) s_last = (atomicAdd(group_counter, 1) == gsize - 1);
    __syncthreads();
    if (!s_last) {
      PAD_TL(lin, PAD_TL_ARRIVED);
      PAD_TL_NOTE(g, 0);
      PAD_TL(lin, PAD_TL_EXIT);
      return;
    }
    tl_flags = PAD_TL_F_GROUP;
    // Each element's O is read and then overwritten by its own thread, but
    // a row's (m, l) is read by every thread of the row, and a row can span
    // waves and loop passes (head_dim 96: 24 elements per row): the group's
    // (m, l) goes to LDS first and to the slot only after a barrier.
    for (int e = threadIdx.x; e < total4; e += nw * 64) {
      const int row = e / (D / 4);
      const int col = (e - row * (D / 4)) * 4;
      float m = kNegInf, l = 0.f;
      f4_t acc = (f4_t)0.f;
      merge_partials(o_rsrc, ml_rsrc, grp0, gsize, 1, gqa, row, col, D, m, l, acc);
      const uint32_t r = (uint32_t)(grp0 * gqa + row);
      store_device(o_rsrc, (r * D + col) * 4u, acc);
      if (col == 0) sm_ml[row] = make_float2(m, l);
    }
    __syncthreads();
    if (threadIdx.x < gqa) store_device(ml_rsrc, (uint32_t)(grp0 * gqa + threadIdx.x) * 8u, sm_ml[threadIdx.x]);
    if (threadIdx.x == 0) atomicExch(group_counter, 0);
    stride = 16;
    count = (nsplit + 15) >> 4;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  if (threadIdx.x == 0) s_last = (atomicAdd(unit_counter, 1) == count - 1);
  __syncthreads();
  PAD_TL(lin, PAD_TL_ARRIVED);
  if (!s_last) {
    PAD_TL_NOTE(g, tl_flags);
    PAD_TL(lin, PAD_TL_EXIT);
    return;
  }
  for (int e = threadIdx.x; e < total4; e += nw * 64) {
    const int row = e / (D / 4);
    const int col = (e - row * (D / 4)) * 4;
    float m = kNegInf, l = 0.f;
    f4_t acc = (f4_t)0.f;
    merge_partials(o_rsrc, ml_rsrc, 0, count, stride, gqa, row, col, D, m, l, acc);
    const float inv = (kv_is_fp8<KVF>() ? a.v_fix : 1.f) / l;
    h4_t hv;
#pragma unroll
    for (int i = 0; i < 4; ++i) hv[i] = round16<KVF>(acc[i] * inv);
    *reinterpret_cast<h4_t*>(out_bh + (int64_t)row * a.soh + col) = hv;
  }
  if (threadIdx.x == 0) atomicExch(unit_counter, 0);
  PAD_TL(lin, PAD_TL_MERGED);
  PAD_TL_NOTE(g, tl_flags | PAD_TL_F_MERGER);
  PAD_TL(lin, PAD_TL_EXIT);
#undef PAD_TL_NOTE
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------

static bool head_dim_supported(int d) { return d == 32 || d == 64 || d == 96 || d == 128 || d == 256; }

static int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// VALU engine instantiations exist for these (head_dim, group) pairs.
static bool valu_supported(int d, int gqa) { return (d == 64 || d == 128) && gqa <= 8; }

// Dynamic LDS of a workgroup: wave (m, l) [nw][16], wave O [nw][gqa][D + 4],
// and for the MFMA engine one padded 16-row K staging tile per wave plus,
// for head_dim 256, one padded 16-row copy of Q^T.
static size_t group_lds_bytes(int nw, int gqa, int d, int engine) {
  const size_t stage = engine == 0 ? (size_t)16 * (d * 2 + 16) : 0;
  const size_t q_stage = (engine == 0 && d >= 256) ? stage : 0;
  return (size_t)nw * (16 * sizeof(float2) + (size_t)gqa * (d + 4) * sizeof(float) + stage) + q_stage;
}

static int lds_wave_cap(int gqa, int d, int engine) {
  const size_t per_wave = group_lds_bytes(1, gqa, d, engine) - group_lds_bytes(0, gqa, d, engine);
  int cap = (int)((kLdsBudget - group_lds_bytes(0, gqa, d, engine)) / per_wave);
  if (cap > max_group_waves(d)) cap = max_group_waves(d);
  if (cap < 1) cap = 1;
  return cap;
}

static int validate_dims(const pad_decode_dims* d) {
  if (!d) return PAD_ERR_NULL_POINTER;
  if (d->batch < 0 || d->num_q_heads <= 0 || d->num_kv_heads <= 0 || d->head_dim <= 0 ||
      d->page_size <= 0 || d->max_pages < 0 || d->num_pages < 0)
    return PAD_ERR_INVALID_SHAPE;
  if (!head_dim_supported(d->head_dim)) return PAD_ERR_UNSUPPORTED_HEAD_DIM;
  if (d->num_q_heads % d->num_kv_heads != 0) return PAD_ERR_UNSUPPORTED_GQA;
  if (d->num_q_heads / d->num_kv_heads > PAD_MAX_GQA) return PAD_ERR_UNSUPPORTED_GQA;
  if (d->q_stride[2] != 1 || d->k_stride[3] != 1 || d->v_stride[3] != 1 || d->out_stride[2] != 1)
    return PAD_ERR_STRIDE;
  return PAD_OK;
}

// Workspace layout (from the first 256-byte boundary of the buffer); the
// workspace holds no state between launches.  One slot per workgroup of the
// (S, Hkv, B) grid, G = B * Hkv * S slots:
//   o_part   fp32  [G, gqa, D] unnormalised split outputs
//   ml_part  fp32x2 [G, gqa]   (m in base-2 units, l)
// Returns the bytes needed (including 256 bytes of alignment slack) and,
// when `ws` is given, the region pointers.
static size_t workspace_layout(const pad_decode_dims* d, int S, void* ws, float** o_part, float2** ml_part) {
  const int gqa = d->num_q_heads / d->num_kv_heads;
  const size_t rows = (size_t)d->batch * d->num_kv_heads * (size_t)S * gqa;
  const size_t o_bytes = rows * (size_t)d->head_dim * sizeof(float);
  if (ws) {
    const uintptr_t base = ((uintptr_t)ws + 255u) & ~(uintptr_t)255u;
    *o_part = reinterpret_cast<float*>(base);
    *ml_part = reinterpret_cast<float2*>(base + o_bytes);
  }
  return 256 + o_bytes + rows * sizeof(float2);
}

// Splits per unit on an oversubscribed grid (see oversubscribed_shape), at
// least; and at least this many workgroups per CU.
constexpr int kOversubscribeSplits = 4;
constexpr int kOversubscribeGroupsPerCu = 8;

// A bandwidth-bound shape with a batch the in-kernel planner handles and
// either more than one (sequence, kv head) unit per two CUs, where the
// power-of-two rule gives one split per unit, or more than one per four CUs
// where its two splits per unit leave CUs idle.  The static splits are
// enough for uniform lengths (measured: C2 batch 128 81.4 us with one split
// against 93.9 us with 4 static splits), but ragged ones leave their longest
// units running alone at the end (C5: 2930 us with one workgroup per unit,
// 2656 us with kOversubscribeSplits planned items per unit, 2767 us with 8;
// C3's lengths at batch 66-127, 132-254 units: 101-113 us with one
// workgroup per unit, 58-100 us planned over oversubscribe_splits items per
// unit; at batch 33-48, 66-96 units: 51-53 us with two splits per unit,
// 34-46 us planned).  The launch therefore sizes the grid for several items
// per unit and the kernel decides from the lengths: all at full capacity,
// the static splits on the first workgroups; otherwise equal page chunks.
// fp8 caches (kv_bytes 1) keep the regime from one unit per CU up: their
// items carry half the bytes, and the grids below that (and the 8-per-CU
// floor of oversubscribe_splits) measured slower for them than the static
// splits (12/2 heads, lengths up to 4096, batch 40 / 96: 25.7 / 41.1 us
// against 18.8 / 31.4 us).
static bool oversubscribed_shape(const pad_decode_dims* d, int num_splits, int num_cus, bool latency_bound,
                                 int kv_bytes = 2) {
  const int64_t units = (int64_t)(d->batch > 0 ? d->batch : 1) * d->num_kv_heads;
  const bool many = kv_bytes == 1 ? units >= num_cus
                                  : units * 2 > num_cus || (units * 4 > num_cus && units * 2 < num_cus);
  return num_splits == 0 && !latency_bound && many && d->batch <= kPlanMaxBatch && d->max_pages < (1 << 23);
}

// Items per unit of an oversubscribed grid: kOversubscribeSplits, or more
// below two units per CU, so that the grid holds kOversubscribeGroupsPerCu
// workgroups per CU and a ragged batch's long units end in several smaller
// items (up to 16 items just above one unit per two CUs).  Measured on C5's
// lengths (batch 256, page 16, 512-32768 tokens) with 4 / 8 / 16 items per
// unit: 256 units (one GPU's share of C5 over 8 GPUs by kv heads, 8/1
// heads) 426 / 391 / 403 us; 512 units 759 / 750 / 803 us; 1024 units
// 1463 / 1509 / 1606 us; the whole C5, 2048 units, 2833 / 2916 / 3164 us.
// On C3's lengths (1-8192 tokens, page 32) this rule and a flat 4 items
// tie: 132 / 160 / 192 / 254 units 59.6 / 70.4 / 79.3 / 99.7 us against
// 58.1 / 72.0 / 76.3 / 104.9 us.
static int64_t oversubscribe_splits(int64_t units, int num_cus) {
  const int64_t want = ((int64_t)kOversubscribeGroupsPerCu * num_cus + units - 1) / units;
  return want > kOversubscribeSplits ? want : kOversubscribeSplits;
}

// Pages of one sequence the plan assumes: the dense table's row width, or
// for a CSR index (max_pages = entries of `indices`, the whole batch's
// pages) the mean per sequence, which is exact for equal lengths; ragged
// CSR batches are re-planned in-kernel from indptr anyway.
static int plan_pages_per_seq(const pad_decode_dims* d, bool csr) {
  if (d->max_pages <= 0) return 1;
  if (!csr || d->batch <= 1) return d->max_pages;
  return ceil_div(d->max_pages, d->batch);
}

static bool latency_bound_shape(const pad_decode_dims* d, int num_cus, bool csr) {
  const int max_pages = plan_pages_per_seq(d, csr);
  const int64_t units = (int64_t)(d->batch > 0 ? d->batch : 1) * d->num_kv_heads;
  const int64_t blocks_per_seq = ((int64_t)max_pages * d->page_size + kBlockTokens - 1) / kBlockTokens;
  return units * blocks_per_seq <= 16 * (int64_t)num_cus;
}

// kv_bytes: bytes per K/V element (2 for fp16, 1 for fp8 caches).
// pps_full, if given, receives the pages per split of the static splits
// (the power-of-two rule), which an oversubscribed grid runs when every
// sequence is at full capacity.
static int plan_impl(const pad_decode_dims* d, int num_splits, int num_cus, int engine, bool csr,
                     pad_decode_plan_t* p, int kv_bytes = 2, int* pps_full = nullptr) {
  const int st = validate_dims(d);
  if (st != PAD_OK) return st;
  if (num_splits < 0 || num_splits > PAD_MAX_SPLITS) return PAD_ERR_NUM_SPLITS;
  if (num_cus <= 0) num_cus = 256;
  const int gqa = d->num_q_heads / d->num_kv_heads;
  const int max_pages = plan_pages_per_seq(d, csr);
  const int64_t units = (int64_t)(d->batch > 0 ? d->batch : 1) * d->num_kv_heads;

  // Regimes (fitted to measured split sweeps of C2 batch 1-64, C3 and C4 on
  // MI355X).  Bandwidth-bound shapes run one 4-wave workgroup per CU: that
  // streamed faster than two (batch 64: 44.0 vs 46.8 us; C4: 86 vs 94 us),
  // and fewer, longer splits shorten the merge.  Latency-bound shapes (at
  // most 16 blocks of work per CU) run 8-wave workgroups on at most half the
  // CUs: fewer splits to merge, each streamed by more waves (batch 8: 11.9
  // vs 13.2 us).
  const int64_t blocks_per_seq = ((int64_t)max_pages * d->page_size + kBlockTokens - 1) / kBlockTokens;
  const bool latency_bound = latency_bound_shape(d, num_cus, csr);
  int S;
  int pps;
  if (num_splits > 0) {
    // Caller's split count, page-aligned: pages_per_split = ceil(max_pages/S).
    // Splits past a sequence's last page are empty (never read).
    S = num_splits;
    pps = ceil_div(max_pages, S);
    if (pps_full) *pps_full = pps;
  } else {
    // A power-of-two split count (the splits of a power-of-two page count
    // are then equal) with at least kMinBlocks 16-token blocks per split, so
    // each workgroup's fixed costs (q load, wave merge, partial publish)
    // stay small against its streaming.  Where the largest count that fits
    // the workgroup budget is at least 1.5 times that, it is taken instead:
    // the power of two would leave a third of the budget idle (C2, uniform:
    // batch 40, 80 units, 35.1 us with 2 splits against 31.2 us with 3;
    // batch 20 20.8 against 19.2 us with 6; batch 5 12.3 against 11.7 us with
    // 12), while smaller steps lose to the longer merge (batch 7, 8 -> 9
    // splits, and batch 12, 8 -> 10: +2%).
    const int64_t max_groups = latency_bound ? num_cus / 2 : num_cus;
    int64_t s_want = 1;
    while (s_want * 2 * units <= max_groups) s_want *= 2;
    const int64_t s_fit = max_groups / units;
    if (2 * s_fit >= 3 * s_want) s_want = s_fit;
    int64_t s_static = s_want;
    if (oversubscribed_shape(d, num_splits, num_cus, latency_bound, kv_bytes)) {
      s_want = kv_bytes == 1 ? kOversubscribeSplits : oversubscribe_splits(units, num_cus);
      // Rows of at most 128 bytes run 8-wave workgroups (below): half as
      // many items, so that each wave streams as many blocks as in a 4-wave
      // workgroup (fp16 head_dim 64, 32/8 heads, lengths up to 4096, batch
      // 20: 30.1 us with the full item count, 25.9 us with half).
      if (d->head_dim * kv_bytes <= 128 && units <= num_cus && kv_bytes == 2) s_want /= 2;
    }
    int64_t s_cap = blocks_per_seq / kMinBlocks;
    // Latency-bound short sequences: a wave's serial chain of blocks costs
    // more than a merge of up to 16 splits (one round trip), so splits may
    // go down to 4 blocks (C1, 1024 tokens: 9.2 us at 16 splits against
    // 10.3 us at the 4 that 16-block splits allow).
    if (latency_bound) {
      const int64_t short_cap = blocks_per_seq / kMinBlocksShort < 16 ? blocks_per_seq / kMinBlocksShort : 16;
      if (s_cap < short_cap) s_cap = short_cap;
    }
    if (s_cap < 1) s_cap = 1;
    if (s_want > s_cap) s_want = s_cap;
    if (s_want > PAD_MAX_SPLITS) s_want = PAD_MAX_SPLITS;
    if (s_static > s_want) s_static = s_want;
    if (pps_full) *pps_full = ceil_div(max_pages, s_static);
    if (csr) {
      // Never more splits (hence scratch) than the dense plan of the same
      // dims, so pad_decode_workspace_bytes() also sizes a CSR launch.
      pad_decode_plan_t dense;
      plan_impl(d, 0, num_cus, engine, false, &dense);
      if (s_want > dense.num_splits) s_want = dense.num_splits;
    }
    pps = ceil_div(max_pages, s_want);
    S = ceil_div(max_pages, pps);
  }
  // Waves per workgroup: never more than the split has blocks or the wave
  // workgroup LDS budget allows.
  const int64_t split_tokens = (int64_t)pps * d->page_size;
  int nw = (int)((split_tokens + kBlockTokens - 1) / kBlockTokens);
  // Bandwidth-bound shapes run 4 waves per workgroup, except rows of at
  // most 128 bytes (fp16 head_dim <= 64, fp8 head_dim <= 128) with at most
  // one (sequence, kv head) unit per CU: their 16-token tiles are half the
  // bytes or less, and 8 waves keep as many bytes in flight per CU (32/8 d64
  // batch 32: 25.8 against 29.9 us; 16/4 d32: 17.8 against 21.9 us).  With
  // more units than CUs, 4-wave workgroups let several units share a CU
  // (16/16 d64 batch 32: 46.9 against 47.9 us).  The split count depends on
  // kv_bytes only through the oversubscribed regime, which gives fp8 caches
  // fewer items than fp16 ones, never more, so the fp16 plan's scratch
  // sizes always cover the fp8 plan's.
  const bool narrow_rows = d->head_dim * kv_bytes <= 128 && units <= num_cus;
  const int nw_max = (latency_bound || narrow_rows) ? kMaxWaves : kMaxWaves / 2;
  if (nw > nw_max) nw = nw_max;
  const int cap = lds_wave_cap(gqa, d->head_dim, engine);
  if (nw > cap) nw = cap;
  if (nw < 1) nw = 1;

  p->num_splits = S;
  p->pages_per_split = pps;
  p->waves_per_group = nw;
  p->single_pass = (S == 1) ? 1 : 0;
  p->engine = engine;
  p->reserved = 0;
  p->counters = 0;
  p->workspace_bytes = p->single_pass ? 0 : workspace_layout(d, S, nullptr, nullptr, nullptr);
  // One arrival counter per unit and, where a unit may get more than
  // kTwoLevelSplits items, one per item slot for the merge's groups.
  const int64_t units64 = (int64_t)d->batch * d->num_kv_heads;
  p->counters = p->single_pass ? 0 : units64 + (units64 * S > kTwoLevelSplits ? units64 * S : 0);
  return PAD_OK;
}

static int g_num_cus[64];

static int device_cus(int* out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return PAD_ERR_DEVICE;
  if (dev < 0 || dev >= 64) return PAD_ERR_DEVICE;
  if (g_num_cus[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return PAD_ERR_DEVICE;
    g_num_cus[dev] = n;
  }
  *out = g_num_cus[dev];
  return PAD_OK;
}

template <int D, int MODE, int ENGINE, int GQA_T, int KVF = kKvF16>
static hipError_t launch_p1(const Phase1Args& a, dim3 grid, int nw, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((pad_phase1_kernel<D, MODE, ENGINE, GQA_T, KVF>), grid, dim3(nw * 64), lds, st, a);
  return hipGetLastError();
}

// fp8 caches (head_dim 64, 128 or 256) and bfloat16 (every head_dim), MFMA
// engine: block mode from the page size, as for fp16.
template <int D, int KVF>
static hipError_t dispatch_kvf(const Phase1Args& a, dim3 grid, int nw, size_t lds, hipStream_t st) {
  if (a.ps % kBlockTokens == 0) return launch_p1<D, kModeUniform, 0, 0, KVF>(a, grid, nw, lds, st);
  switch (a.ps) {
    case 1: return launch_p1<D, kModeSubpage + 0, 0, 0, KVF>(a, grid, nw, lds, st);
    case 2: return launch_p1<D, kModeSubpage + 1, 0, 0, KVF>(a, grid, nw, lds, st);
    case 4: return launch_p1<D, kModeSubpage + 2, 0, 0, KVF>(a, grid, nw, lds, st);
    case 8: return launch_p1<D, kModeSubpage + 3, 0, 0, KVF>(a, grid, nw, lds, st);
    default: break;
  }
  return launch_p1<D, kModeGeneric, 0, 0, KVF>(a, grid, nw, lds, st);
}

template <int KVF>
static hipError_t dispatch_kvf_dim(const Phase1Args& a, int head_dim, dim3 grid, int nw, size_t lds, hipStream_t st) {
  if constexpr (KVF == kKvBF16) {
    if (head_dim == 32) return dispatch_kvf<32, KVF>(a, grid, nw, lds, st);
    if (head_dim == 96) return dispatch_kvf<96, KVF>(a, grid, nw, lds, st);
  }
  switch (head_dim) {
    case 64: return dispatch_kvf<64, KVF>(a, grid, nw, lds, st);
    case 128: return dispatch_kvf<128, KVF>(a, grid, nw, lds, st);
    case 256: return dispatch_kvf<256, KVF>(a, grid, nw, lds, st);
    default: return hipErrorInvalidValue;
  }
}

template <int D, int MODE>
static hipError_t dispatch_engine(const Phase1Args& a, dim3 grid, int nw, size_t lds, int engine,
                                  hipStream_t st) {
  if (engine == 1) {
    if constexpr ((D == 64 || D == 128) && MODE <= kModeUniform) {
      if (a.gqa == 1) return launch_p1<D, MODE, 1, 1>(a, grid, nw, lds, st);
      if (a.gqa == 2) return launch_p1<D, MODE, 1, 2>(a, grid, nw, lds, st);
      if (a.gqa <= 4) return launch_p1<D, MODE, 1, 4>(a, grid, nw, lds, st);
      if (a.gqa <= 6) return launch_p1<D, MODE, 1, 6>(a, grid, nw, lds, st);
      return launch_p1<D, MODE, 1, 8>(a, grid, nw, lds, st);
    }
    return hipErrorInvalidValue;
  }
  return launch_p1<D, MODE, 0, 0>(a, grid, nw, lds, st);
}

// Block-addressing mode from the page size (the VALU engine has the uniform
// and generic modes only).
template <int D>
static hipError_t dispatch_phase1(const Phase1Args& a, dim3 grid, int nw, size_t lds, int engine,
                                  hipStream_t st) {
  if (a.ps % kBlockTokens == 0) return dispatch_engine<D, kModeUniform>(a, grid, nw, lds, engine, st);
  if (engine == 0) {
    switch (a.ps) {
      case 1: return dispatch_engine<D, kModeSubpage + 0>(a, grid, nw, lds, engine, st);
      case 2: return dispatch_engine<D, kModeSubpage + 1>(a, grid, nw, lds, engine, st);
      case 4: return dispatch_engine<D, kModeSubpage + 2>(a, grid, nw, lds, engine, st);
      case 8: return dispatch_engine<D, kModeSubpage + 3>(a, grid, nw, lds, engine, st);
      default: break;
    }
  }
  return dispatch_engine<D, kModeGeneric>(a, grid, nw, lds, engine, st);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Everything one decode launch needs: kernel arguments, plan, grid, LDS.
struct Launch {
  Phase1Args a;
  pad_decode_plan_t plan;
  dim3 grid;
  int nw;
  size_t lds;
  bool empty;  // batch 0: nothing to launch
};

// Key of a launch's plan, stored in a work list's header: the fields that
// decide the grid and which item each workgroup gets (FNV-1a).
static int plan_key(const Phase1Args& a) {
  const int f[] = {a.batch, a.hkv, a.max_pages, a.num_splits, a.nw, a.csr, a.balance,
                   a.ps, a.pps, a.gqa, a.pair_heads, a.min_chunk};
  uint32_t h = 2166136261u;
  for (int x : f) {
    h ^= (uint32_t)x;
    h *= 16777619u;
  }
  return (int)(h & 0x7fffffff);
}

// Dense page table: bt = block_table, sl = seq_lens, indptr = lpl = NULL.
// CSR: bt = indices, indptr / lpl given, sl unused (dims->max_pages is the
// number of entries in indices).  io: also check q/k/v/out and the scratch
// (a work-list plan reads only the index arrays).
static int setup_launch(const void* q, const void* k, const void* v, const int32_t* bt, const int32_t* sl,
                        const int32_t* indptr, const int32_t* lpl, void* out, void* ws, size_t ws_bytes,
                        int32_t* counters, int64_t num_counters, const pad_decode_dims* d, float scale,
                        int num_splits, int engine, bool io, Launch* L, int kv_bytes = 2) {
  if (engine != 0 && engine != 1) return PAD_ERR_INVALID_SHAPE;
  // Page ids are bounds-checked against num_pages on the device (an id
  // outside [0, num_pages) reads page 0), so a launch that reads pages needs
  // the real cache size.
  if (d && d->batch > 0 && d->max_pages > 0 && d->num_pages <= 0) return PAD_ERR_INVALID_SHAPE;
  int cus = 0;
  int st = device_cus(&cus);
  if (st != PAD_OK) return st;
  const bool csr = indptr != nullptr || lpl != nullptr;
  pad_decode_plan_t& plan = L->plan;
  int pps_full = 0;
  st = plan_impl(d, num_splits, cus, engine, csr, &plan, kv_bytes, &pps_full);
  if (st != PAD_OK) return st;
  const int gqa = d->num_q_heads / d->num_kv_heads;
  if (engine == 1 && !valu_supported(d->head_dim, gqa)) return PAD_ERR_UNSUPPORTED_GQA;
  L->empty = d->batch == 0;
  if (L->empty) return PAD_OK;
  // The page-id array may be NULL only when it has no entries (a [batch, 0]
  // table, or an empty CSR index): then no sequence has a page to read.
  if ((!bt && d->max_pages > 0) || (csr ? (!indptr || !lpl) : !sl)) return PAD_ERR_NULL_POINTER;
  if (io) {
    if (!q || !k || !v || !out) return PAD_ERR_NULL_POINTER;
    // 16-byte rows: every K/V/q/out row start must be 16-byte aligned.
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out)) return PAD_ERR_ALIGNMENT;
    if ((d->q_stride[0] | d->q_stride[1]) % 8 || (d->out_stride[0] | d->out_stride[1]) % 8 ||
        (d->k_stride[0] | d->k_stride[1] | d->k_stride[2]) % 8 ||
        (d->v_stride[0] | d->v_stride[1] | d->v_stride[2]) % 8)
      return PAD_ERR_ALIGNMENT;
    if (!plan.single_pass && (!ws || ws_bytes < plan.workspace_bytes)) return PAD_ERR_WORKSPACE;
    if (!plan.single_pass && (!counters || num_counters < plan.counters)) return PAD_ERR_WORKSPACE;
  }

  const int S = plan.num_splits;
  float* o_part = nullptr;
  float2* ml_part = nullptr;
  if (io && !plan.single_pass) workspace_layout(d, S, ws, &o_part, &ml_part);

  Phase1Args& a = L->a;
  a.q = static_cast<const _Float16*>(q);
  a.k = static_cast<const _Float16*>(k);
  a.v = static_cast<const _Float16*>(v);
  a.bt = bt;
  a.sl = sl;
  a.indptr = indptr;
  a.lpl = lpl;
  a.worklist = nullptr;
  a.out = static_cast<_Float16*>(out);
  a.o_part = o_part;
  a.ml_part = ml_part;
  a.counters = counters;
  a.sqb = d->q_stride[0];
  a.sqh = d->q_stride[1];
  a.skp = d->k_stride[0];
  a.sks = d->k_stride[1];
  a.skh = d->k_stride[2];
  a.svp = d->v_stride[0];
  a.svs = d->v_stride[1];
  a.svh = d->v_stride[2];
  a.sbb = csr ? 0 : d->bt_stride[0];
  a.sbp = csr ? 1 : d->bt_stride[1];
  a.ssl = d->sl_stride;
  a.sob = d->out_stride[0];
  a.soh = d->out_stride[1];
  a.num_pages = d->num_pages;
  a.gqa = gqa;
  a.ps = d->page_size;
  a.pps = plan.pages_per_split;
  a.num_splits = S;
  a.hkv = d->num_kv_heads;
  a.max_pages = d->max_pages;
  a.batch = d->batch;
  a.csr = csr ? 1 : 0;
  // The in-kernel planner evens out ragged batches; an explicit split count
  // keeps its meaning (that many page-aligned splits per sequence).
  a.balance = 0;
  if (num_splits == 0 && !plan.single_pass && d->batch <= kPlanMaxBatch && d->max_pages < (1 << 23))
    a.balance = oversubscribed_shape(d, num_splits, cus, latency_bound_shape(d, cus, csr), kv_bytes) ? 2 : 1;
  a.min_chunk = ceil_div(kMinBlocks * kBlockTokens, d->page_size);
  a.pair_heads = ((d->head_dim * 2) % 128 != 0 && d->num_kv_heads % 2 == 0 &&
                  ((int64_t)S * d->num_kv_heads * d->batch) % 16 == 0) ? 1 : 0;
  if (a.balance == 2) {
    // An oversubscribed grid runs the static splits when every sequence is
    // at full capacity: pps is theirs (the grid's own split is the planner's
    // business), and balance = 1 + their count s0 per unit.  More than one
    // unit per four CUs leaves at most 3 (the budget over the units); with
    // more than one they take the first workgroups in order, unit-major,
    // so head pairing stays off.
    const int s0 = pps_full > 0 && d->max_pages > pps_full ? ceil_div(d->max_pages, pps_full) : 1;
    if (s0 <= 3) {
      a.pps = pps_full;
      a.balance = 1 + s0;
      if (s0 > 1) a.pair_heads = 0;
    } else {
      a.balance = 1;  // not reached; the planner of the grid as it is
    }
  }
  a.ps_shift = -1;
  for (int sh = 0; sh < 31; ++sh)
    if ((1 << sh) == d->page_size) a.ps_shift = sh;
  a.scale_log2 = scale * kLog2e;
  a.v_fix = 1.0f;
  a.nw = plan.waves_per_group;
  a.wl_key = plan_key(a);
#ifdef PAD_TIMELINE
  a.tl_launch = 0;
#endif
  L->nw = plan.waves_per_group;
  L->lds = group_lds_bytes(L->nw, gqa, d->head_dim, engine);
  L->grid = dim3(S, d->num_kv_heads, d->batch);
  return PAD_OK;
}

// Bytes of the work list of this plan: header plus one record per workgroup.
static size_t worklist_bytes_for(const pad_decode_plan_t& plan, const pad_decode_dims* d) {
  const int64_t G = (int64_t)plan.num_splits * d->num_kv_heads * d->batch;
  return sizeof(int32_t) * (size_t)(kWlHeaderInts + kWlRecordInts * G);
}

// A known format; bfloat16 and fp8 on the MFMA engine; fp8 with head_dim
// 64/128/256 and finite positive scales (the scales are read for fp8 only).
static bool kv_format_fp8(int f) {
  return f == PAD_KV_FP8_E4M3FN || f == PAD_KV_FP8_E5M2 || f == PAD_KV_FP8_E4M3FN_BF16 || f == PAD_KV_FP8_E5M2_BF16;
}

static int check_kv_format(int kv_format, int engine, const pad_decode_dims* d, float k_scale, float v_scale) {
  if (kv_format == PAD_KV_FP16) return PAD_OK;
  if (kv_format == PAD_KV_BF16) return engine == 0 ? PAD_OK : PAD_ERR_KV_FORMAT;
  if (!kv_format_fp8(kv_format)) return PAD_ERR_KV_FORMAT;
  if (engine != 0) return PAD_ERR_KV_FORMAT;
  if (d && d->head_dim != 64 && d->head_dim != 128 && d->head_dim != 256) return PAD_ERR_UNSUPPORTED_HEAD_DIM;
  if (!(k_scale > 0.0f) || !(v_scale > 0.0f) || k_scale > 1.0e30f || v_scale > 1.0e30f) return PAD_ERR_KV_FORMAT;
  return PAD_OK;
}

// kv_format: PAD_KV_FP16, or an fp8 format with per-tensor scales k_scale,
// v_scale (the caches hold K / k_scale and V / v_scale).
static int launch_impl(const void* q, const void* k, const void* v, const int32_t* bt, const int32_t* sl,
                       const int32_t* indptr, const int32_t* lpl, void* out, void* ws, size_t ws_bytes,
                       int32_t* counters, int64_t num_counters, const pad_decode_dims* d, float scale,
                       int num_splits, int engine, void* const* events, void* stream,
                       const void* worklist = nullptr, size_t worklist_bytes = 0, int kv_format = PAD_KV_FP16,
                       float k_scale = 1.0f, float v_scale = 1.0f) {
  int st = check_kv_format(kv_format, engine, d, k_scale, v_scale);
  if (st != PAD_OK) return st;
  Launch L;
  const bool fp8 = kv_format_fp8(kv_format);
  st = setup_launch(q, k, v, bt, sl, indptr, lpl, out, ws, ws_bytes, counters, num_counters, d, scale,
                    num_splits, engine, true, &L, fp8 ? 1 : 2);
  if (st != PAD_OK || L.empty) return st;
  if (fp8) {
    // The caches hold K / k_scale and V / v_scale: k_scale multiplies every
    // score, v_scale every output row.
    L.a.scale_log2 *= k_scale;
    L.a.v_fix = v_scale;
  }
  if (worklist != nullptr) {
    if (worklist_bytes < worklist_bytes_for(L.plan, d)) return PAD_ERR_WORKSPACE;
    L.a.worklist = static_cast<const int32_t*>(worklist);
  }
#ifdef PAD_TIMELINE
  L.a.tl_launch = tl_launches++ % PAD_TL_LAUNCHES;
#endif
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  if (events && events[0] && hipEventRecord(reinterpret_cast<hipEvent_t>(events[0]), hs) != hipSuccess)
    return PAD_ERR_LAUNCH;
  hipError_t e;
  if (kv_format == PAD_KV_FP8_E4M3FN) {
    e = dispatch_kvf_dim<kKvE4M3>(L.a, d->head_dim, L.grid, L.nw, L.lds, hs);
  } else if (kv_format == PAD_KV_FP8_E5M2) {
    e = dispatch_kvf_dim<kKvE5M2>(L.a, d->head_dim, L.grid, L.nw, L.lds, hs);
  } else if (kv_format == PAD_KV_BF16) {
    e = dispatch_kvf_dim<kKvBF16>(L.a, d->head_dim, L.grid, L.nw, L.lds, hs);
  } else if (kv_format == PAD_KV_FP8_E4M3FN_BF16) {
    e = dispatch_kvf_dim<kKvE4M3B>(L.a, d->head_dim, L.grid, L.nw, L.lds, hs);
  } else if (kv_format == PAD_KV_FP8_E5M2_BF16) {
    e = dispatch_kvf_dim<kKvE5M2B>(L.a, d->head_dim, L.grid, L.nw, L.lds, hs);
  } else switch (d->head_dim) {
    case 32: e = dispatch_phase1<32>(L.a, L.grid, L.nw, L.lds, engine, hs); break;
    case 64: e = dispatch_phase1<64>(L.a, L.grid, L.nw, L.lds, engine, hs); break;
    case 96: e = dispatch_phase1<96>(L.a, L.grid, L.nw, L.lds, engine, hs); break;
    case 128: e = dispatch_phase1<128>(L.a, L.grid, L.nw, L.lds, engine, hs); break;
    default: e = dispatch_phase1<256>(L.a, L.grid, L.nw, L.lds, engine, hs); break;
  }
  if (e != hipSuccess) return PAD_ERR_LAUNCH;
  if (events && events[1] && hipEventRecord(reinterpret_cast<hipEvent_t>(events[1]), hs) != hipSuccess)
    return PAD_ERR_LAUNCH;
  if (events && events[2] && hipEventRecord(reinterpret_cast<hipEvent_t>(events[2]), hs) != hipSuccess)
    return PAD_ERR_LAUNCH;
  return PAD_OK;
}

// Writes the work list of a launch with these dims and indices (one wave per
// workgroup slot of the decode grid).
// kv_bytes: bytes per K/V element of the launch the list is for (the wave
// count, and so the list's plan key, depends on it).
static int plan_worklist_impl(const int32_t* bt, const int32_t* sl, const int32_t* indptr, const int32_t* lpl,
                              const pad_decode_dims* d, int num_splits, void* worklist, size_t worklist_bytes,
                              void* stream, int kv_bytes = 2) {
  Launch L;
  int st = setup_launch(nullptr, nullptr, nullptr, bt, sl, indptr, lpl, nullptr, nullptr, 0, nullptr, 0, d, 1.0f,
                        num_splits, 0, false, &L, kv_bytes);
  if (st != PAD_OK) return st;
  if (!worklist) return PAD_ERR_NULL_POINTER;
  if (worklist_bytes < worklist_bytes_for(L.plan, d)) return PAD_ERR_WORKSPACE;
  if (L.empty) return PAD_OK;
  hipLaunchKernelGGL(pad_plan_kernel, L.grid, dim3(64), 0, reinterpret_cast<hipStream_t>(stream), L.a,
                     static_cast<int32_t*>(worklist));
  return hipGetLastError() == hipSuccess ? PAD_OK : PAD_ERR_LAUNCH;
}

// ---------------------------------------------------------------------------
// Allocation-free launches (pad_decode_launch_noalloc): the split scratch is
// a file-scope device array instead of caller memory.  Layout: the int32
// arrival counters first (PAD_NOALLOC_COUNTERS of them), then the partials
// workspace (PAD_NOALLOC_WORKSPACE_BYTES).  Every GPU the library runs on
// holds its own copy until the process ends.  In host code `scratch` names a
// host-side stand-in, not device memory: the per-device address comes from
// hipGetSymbolAddress once per device and only that address is used.
// ---------------------------------------------------------------------------
constexpr size_t kNoallocCounterBytes = (size_t)PAD_NOALLOC_COUNTERS * sizeof(int32_t);
static __device__ __align__(256) unsigned char scratch[kNoallocCounterBytes + PAD_NOALLOC_WORKSPACE_BYTES];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// Zeroes n int32 values with vector stores (used for the counters once per
// device; a kernel rather than hipMemsetAsync so that a call made under
// stream capture records a kernel node).
__global__ void pad_zero_i32_kernel(int32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

// The current device's scratch address; the first call on a device looks it
// up (with that device current) and queues a clear of its counters on
// `stream`, ahead of the caller's launch.  The array is zero when the code
// object loads, and every launch leaves the counters zero again, so the
// clear only makes that state explicit.
static int noalloc_scratch(hipStream_t stream, unsigned char** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return PAD_ERR_DEVICE;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return PAD_ERR_DEVICE;
    hipLaunchKernelGGL(pad_zero_i32_kernel, dim3(64), dim3(256), 0, stream, static_cast<int32_t*>(ptr),
                       (int64_t)PAD_NOALLOC_COUNTERS);
    if (hipGetLastError() != hipSuccess) return PAD_ERR_LAUNCH;
    g_scratch_ptr[dev] = ptr;
  }
  *out = static_cast<unsigned char*>(g_scratch_ptr[dev]);
  return PAD_OK;
}

static int launch_noalloc(const void* q, const void* k, const void* v, const int32_t* bt, const int32_t* sl,
                          void* out, const pad_decode_dims* d, float scale, int num_splits, void* stream) {
  if (d && d->batch > 0 && d->max_pages > 0 && d->num_pages <= 0) return PAD_ERR_INVALID_SHAPE;
  int cus = 0;
  int st = device_cus(&cus);
  if (st != PAD_OK) return st;
  pad_decode_plan_t plan;
  st = plan_impl(d, num_splits, cus, 0, false, &plan);
  if (st != PAD_OK) return st;
  if (plan.workspace_bytes > PAD_NOALLOC_WORKSPACE_BYTES || plan.counters > PAD_NOALLOC_COUNTERS)
    return PAD_ERR_SCRATCH_LIMIT;
  unsigned char* base = nullptr;
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  st = noalloc_scratch(hs, &base);
  if (st != PAD_OK) return st;
  return launch_impl(q, k, v, bt, sl, nullptr, nullptr, out, base + kNoallocCounterBytes,
                     PAD_NOALLOC_WORKSPACE_BYTES, reinterpret_cast<int32_t*>(base), PAD_NOALLOC_COUNTERS, d, scale,
                     num_splits, 0, nullptr, stream);
}

}  // namespace pad

extern "C" {

int pad_decode_plan(const pad_decode_dims* dims, int num_splits, int num_cus, pad_decode_plan_t* plan) {
  if (!plan) return PAD_ERR_NULL_POINTER;
  return pad::plan_impl(dims, num_splits, num_cus, 0, false, plan);
}

int pad_decode_plan_csr(const pad_decode_dims* dims, int num_splits, int num_cus, pad_decode_plan_t* plan) {
  if (!plan) return PAD_ERR_NULL_POINTER;
  return pad::plan_impl(dims, num_splits, num_cus, 0, true, plan);
}

int pad_decode_workspace_bytes(const pad_decode_dims* dims, int num_splits, int num_cus, size_t* bytes) {
  if (!bytes) return PAD_ERR_NULL_POINTER;
  pad_decode_plan_t p;
  const int st = pad::plan_impl(dims, num_splits, num_cus, 0, false, &p);
  if (st != PAD_OK) return st;
  *bytes = p.workspace_bytes;
  return PAD_OK;
}

int pad_decode_counters_needed(const pad_decode_dims* dims, int num_splits, int num_cus, int64_t* count) {
  if (!count) return PAD_ERR_NULL_POINTER;
  pad_decode_plan_t p;
  const int st = pad::plan_impl(dims, num_splits, num_cus, 0, false, &p);
  if (st != PAD_OK) return st;
  *count = p.counters;
  return PAD_OK;
}

int pad_decode_launch(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                      const int32_t* seq_lens, void* out, void* workspace, size_t workspace_bytes,
                      int32_t* counters, int64_t num_counters, const pad_decode_dims* dims, float scale,
                      int num_splits, void* stream) {
  return pad::launch_impl(q, k_cache, v_cache, block_table, seq_lens, nullptr, nullptr, out, workspace,
                          workspace_bytes, counters, num_counters, dims, scale, num_splits, 0, nullptr, stream);
}

int pad_decode_launch_csr(const void* q, const void* k_cache, const void* v_cache, const int32_t* indices,
                          const int32_t* indptr, const int32_t* last_page_len, void* out, void* workspace,
                          size_t workspace_bytes, int32_t* counters, int64_t num_counters,
                          const pad_decode_dims* dims, float scale, int num_splits, int engine, void* stream) {
  if (!indptr || !last_page_len) return PAD_ERR_NULL_POINTER;
  return pad::launch_impl(q, k_cache, v_cache, indices, nullptr, indptr, last_page_len, out, workspace,
                          workspace_bytes, counters, num_counters, dims, scale, num_splits, engine, nullptr, stream);
}

int pad_decode_launch_ex(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                         const int32_t* seq_lens, void* out, void* workspace, size_t workspace_bytes,
                         int32_t* counters, int64_t num_counters, const pad_decode_dims* dims, float scale,
                         int num_splits, int engine, void* const* events, void* stream) {
  return pad::launch_impl(q, k_cache, v_cache, block_table, seq_lens, nullptr, nullptr, out, workspace,
                          workspace_bytes, counters, num_counters, dims, scale, num_splits, engine, events, stream);
}

int pad_decode_launch_kv8(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                          const int32_t* seq_lens, void* out, void* workspace, size_t workspace_bytes,
                          int32_t* counters, int64_t num_counters, const pad_decode_dims* dims, float scale,
                          int kv_format, float k_scale, float v_scale, int num_splits, void* stream) {
  // fp16 caches: pad_decode_launch; bfloat16: pad_decode_launch_call
  if (!pad::kv_format_fp8(kv_format)) return PAD_ERR_KV_FORMAT;
  return pad::launch_impl(q, k_cache, v_cache, block_table, seq_lens, nullptr, nullptr, out, workspace,
                          workspace_bytes, counters, num_counters, dims, scale, num_splits, 0, nullptr, stream,
                          nullptr, 0, kv_format, k_scale, v_scale);
}

int pad_decode_launch_noalloc(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                              const int32_t* seq_lens, void* out, const pad_decode_dims* dims, float scale,
                              int num_splits, void* stream) {
  return pad::launch_noalloc(q, k_cache, v_cache, block_table, seq_lens, out, dims, scale, num_splits, stream);
}

int pad_decode_worklist_bytes(const pad_decode_dims* dims, int num_splits, int num_cus, int csr, size_t* bytes) {
  if (!bytes) return PAD_ERR_NULL_POINTER;
  pad_decode_plan_t p;
  const int st = pad::plan_impl(dims, num_splits, num_cus, 0, csr != 0, &p);
  if (st != PAD_OK) return st;
  *bytes = pad::worklist_bytes_for(p, dims);
  return PAD_OK;
}

int pad_decode_plan_worklist(const int32_t* block_table, const int32_t* seq_lens, const pad_decode_dims* dims,
                             int num_splits, void* worklist, size_t worklist_bytes, void* stream) {
  return pad::plan_worklist_impl(block_table, seq_lens, nullptr, nullptr, dims, num_splits, worklist, worklist_bytes,
                                 stream);
}

int pad_decode_plan_worklist_csr(const int32_t* indices, const int32_t* indptr, const int32_t* last_page_len,
                                 const pad_decode_dims* dims, int num_splits, void* worklist, size_t worklist_bytes,
                                 void* stream) {
  if (!indptr || !last_page_len) return PAD_ERR_NULL_POINTER;
  return pad::plan_worklist_impl(indices, nullptr, indptr, last_page_len, dims, num_splits, worklist,
                                 worklist_bytes, stream);
}

int pad_decode_launch_worklist(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                               const int32_t* seq_lens, void* out, void* workspace, size_t workspace_bytes,
                               int32_t* counters, int64_t num_counters, const pad_decode_dims* dims, float scale,
                               int num_splits, const void* worklist, size_t worklist_bytes, void* stream) {
  if (!worklist) return PAD_ERR_NULL_POINTER;
  return pad::launch_impl(q, k_cache, v_cache, block_table, seq_lens, nullptr, nullptr, out, workspace,
                          workspace_bytes, counters, num_counters, dims, scale, num_splits, 0, nullptr, stream,
                          worklist, worklist_bytes);
}

int pad_decode_launch_worklist_csr(const void* q, const void* k_cache, const void* v_cache, const int32_t* indices,
                                   const int32_t* indptr, const int32_t* last_page_len, void* out, void* workspace,
                                   size_t workspace_bytes, int32_t* counters, int64_t num_counters,
                                   const pad_decode_dims* dims, float scale, int num_splits, const void* worklist,
                                   size_t worklist_bytes, void* stream) {
  if (!indptr || !last_page_len || !worklist) return PAD_ERR_NULL_POINTER;
  return pad::launch_impl(q, k_cache, v_cache, indices, nullptr, indptr, last_page_len, out, workspace,
                          workspace_bytes, counters, num_counters, dims, scale, num_splits, 0, nullptr, stream,
                          worklist, worklist_bytes);
}

int pad_decode_launch_call(const pad_decode_call* c, const pad_decode_dims* dims, void* stream) {
  if (!c) return PAD_ERR_NULL_POINTER;
  const bool csr = c->indptr != nullptr || c->last_page_len != nullptr;
  if (csr && (!c->indptr || !c->last_page_len)) return PAD_ERR_NULL_POINTER;
  if (c->worklist && c->engine != 0) return PAD_ERR_INVALID_SHAPE;  // work lists serve the MFMA engine
  return pad::launch_impl(c->q, c->k_cache, c->v_cache, c->block_table, csr ? nullptr : c->seq_lens, c->indptr,
                          c->last_page_len, c->out, c->workspace, c->workspace_bytes, c->counters, c->num_counters,
                          dims, c->scale, c->num_splits, c->engine, nullptr, stream, c->worklist, c->worklist_bytes,
                          c->kv_format, c->k_scale, c->v_scale);
}

int pad_decode_plan_worklist_call(const pad_decode_call* c, const pad_decode_dims* dims, void* worklist,
                                  size_t worklist_bytes, void* stream) {
  if (!c) return PAD_ERR_NULL_POINTER;
  const bool csr = c->indptr != nullptr || c->last_page_len != nullptr;
  if (csr && (!c->indptr || !c->last_page_len)) return PAD_ERR_NULL_POINTER;
  if (c->engine != 0) return PAD_ERR_INVALID_SHAPE;  // work lists serve the MFMA engine
  const int st = pad::check_kv_format(c->kv_format, 0, dims, c->k_scale, c->v_scale);
  if (st != PAD_OK) return st;
  const bool fp8 = pad::kv_format_fp8(c->kv_format);
  return pad::plan_worklist_impl(c->block_table, csr ? nullptr : c->seq_lens, c->indptr, c->last_page_len, dims,
                                 c->num_splits, worklist, worklist_bytes, stream, fp8 ? 1 : 2);
}

int pad_decode_counters_init(int32_t* counters, int64_t num_counters, void* stream) {
  if (!counters) return PAD_ERR_NULL_POINTER;
  if (num_counters <= 0) return PAD_OK;
  // A fill kernel, not hipMemsetAsync: under stream capture this records a
  // kernel node, which replays correctly.
  const int64_t blocks = (num_counters + 255) / 256;
  hipLaunchKernelGGL(pad::pad_zero_i32_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), counters, num_counters);
  return hipGetLastError() == hipSuccess ? PAD_OK : PAD_ERR_LAUNCH;
}

int pad_device_num_cus(int* num_cus) {
  if (!num_cus) return PAD_ERR_NULL_POINTER;
  return pad::device_cus(num_cus);
}

const char* pad_status_string(int status) {
  switch (status) {
    case PAD_OK: return "ok";
    case PAD_ERR_NULL_POINTER: return "a required pointer is NULL";
    case PAD_ERR_INVALID_SHAPE: return "invalid shape (non-positive or inconsistent sizes)";
    case PAD_ERR_UNSUPPORTED_HEAD_DIM: return "unsupported head_dim (supported: 32, 64, 96, 128, 256)";
    case PAD_ERR_UNSUPPORTED_GQA:
      return "unsupported GQA group (num_q_heads must be a multiple of num_kv_heads, ratio <= 16)";
    case PAD_ERR_STRIDE: return "head_dim must be contiguous (stride 1) for q, k_cache, v_cache and out";
    case PAD_ERR_ALIGNMENT: return "q/k_cache/v_cache/out rows must be 16-byte aligned";
    case PAD_ERR_WORKSPACE:
      return "workspace/counters NULL or smaller than pad_decode_workspace_bytes()/pad_decode_counters_needed()";
    case PAD_ERR_NUM_SPLITS: return "num_splits must be in [0, 1024]";
    case PAD_ERR_LAUNCH: return "kernel launch failed";
    case PAD_ERR_DEVICE: return "no usable HIP device";
    case PAD_ERR_SCRATCH_LIMIT:
      return "the call needs more split scratch than pad_decode_launch_noalloc's static buffer holds "
             "(PAD_NOALLOC_WORKSPACE_BYTES of partials, PAD_NOALLOC_COUNTERS counters); use pad_decode_launch";
    case PAD_ERR_KV_FORMAT:
      return "unsupported K/V cache format or scale (fp8: PAD_KV_FP8_E4M3FN / _E5M2 (fp16 q) or _BF16 (bfloat16 "
             "q), MFMA engine, head_dim 64/128/256, finite positive k_scale and v_scale; PAD_KV_BF16: MFMA engine)";
    default: return "unknown status";
  }
}

int pad_decode_abi_version(void) { return PAD_ABI_VERSION; }

#ifdef PAD_TIMELINE
int pad_timeline_read(void* host, size_t bytes) {
  if (!host) return PAD_ERR_NULL_POINTER;
  const size_t n = bytes < sizeof(pad::tl_buf) ? bytes : sizeof(pad::tl_buf);
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(pad::tl_buf), n, 0, hipMemcpyDeviceToHost) == hipSuccess
             ? PAD_OK
             : PAD_ERR_DEVICE;
}

int pad_timeline_reset(void) {
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(pad::tl_buf)) != hipSuccess) return PAD_ERR_DEVICE;
  if (hipMemset(p, 0, sizeof(pad::tl_buf)) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
    return PAD_ERR_DEVICE;
  pad::tl_launches = 0;
  return PAD_OK;
}
#endif

}  // extern "C"
