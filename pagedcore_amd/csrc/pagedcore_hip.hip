// Paged KV-cache hot path for MI355X (gfx950): KV append, paged decode attention with
// split-K partitions, and the partition reduce. Exposed through the C ABI declared in
// include/pagedcore_hip.h. No allocation happens here; every buffer comes from the caller.
//
// Pool layout (fixed by the reference allocator, src/pagedcore/kv_cache.py:39-43):
//   fp16 [22 layers][2 kinds][num_blocks][16 slots][4 kv heads][64 dims]
// One (layer, kind, block) is 8 KiB contiguous; one (block, kv head) is 16 rows of 128 B
// at a 512 B stride.

#include <hip/hip_runtime.h>

#include <algorithm>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "pagedcore_hip.h"

namespace {

constexpr int kAbiVersion = 6;
constexpr int kLayers = 22;
constexpr int kSlots = 16;
constexpr int kKVHeads = 4;
constexpr int kQHeads = 32;
constexpr int kGroup = kQHeads / kKVHeads;  // 8 query heads per kv head
constexpr int kHeadDim = 64;
constexpr int64_t kRowElems = kKVHeads * kHeadDim;  // 256 fp16 per token row
constexpr int64_t kBlockElems = kSlots * kRowElems;  // 4096 fp16 per (layer, kind, block)
constexpr int kRowChunks = kRowElems * 2 / 16;       // 32 chunks of 16 B per token row

thread_local char g_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return code;
}

int ok() {
  g_error[0] = '\0';
  return PC_OK;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(PC_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(err));
  }
  return ok();
}

// ---------------------------------------------------------------------------------------
// KV append: token rows -> pool slots. Raw 16-bit moves only, so the copy is bit-exact.
// ---------------------------------------------------------------------------------------

constexpr int kAppendThreads = 256;
constexpr int kAppendChunksPerThread = 4;  // loads issued before stores for memory-level parallelism

struct AppendChunk {
  uint4 data;
  int64_t dst;  // destination in 16 B units, -1 = nothing to store
};

struct AppendArgs {
  const char* key;
  const char* value;
  const int64_t* slot_mapping;
  int64_t key_layer_bytes, key_token_bytes, value_layer_bytes, value_token_bytes;
  int64_t slot_limit;
  int layer_begin;
  uint32_t num_tokens, total_rows;
};

// Chunk q (16 B) of the flattened work: q = ((l * T + t) * 2 + kind) * 32 + c.
__device__ __forceinline__ AppendChunk append_load(const AppendArgs& a, uint32_t q) {
  AppendChunk out;
  out.dst = -1;
  const uint32_t row = q / kRowChunks;
  if (row < a.total_rows) {
    const uint32_t c = q % kRowChunks;
    const uint32_t kind = row & 1u;
    const uint32_t rest = row >> 1;
    const uint32_t t = rest % a.num_tokens;
    const uint32_t l = rest / a.num_tokens;
    const int64_t slot = a.slot_mapping[t];
    if (slot >= 0 && slot < a.slot_limit) {
      const char* src = kind ? a.value + l * a.value_layer_bytes + t * a.value_token_bytes
                             : a.key + l * a.key_layer_bytes + t * a.key_token_bytes;
      out.data = *reinterpret_cast<const uint4*>(src + c * 16);
      // pool row (layer, kind, slot) in units of one 512 B row, then the chunk.
      out.dst = ((static_cast<int64_t>(a.layer_begin + l) * 2 + kind) * a.slot_limit + slot) *
                    kRowChunks + c;
    }
  }
  return out;
}

// Each thread moves four 16 B chunks, issuing all loads before any store.
__global__ __launch_bounds__(kAppendThreads) void kv_append_vec_kernel(uint4* __restrict__ pool,
                                                                       AppendArgs a) {
  const uint32_t first = blockIdx.x * (kAppendThreads * kAppendChunksPerThread) + threadIdx.x;
  const AppendChunk c0 = append_load(a, first);
  const AppendChunk c1 = append_load(a, first + kAppendThreads);
  const AppendChunk c2 = append_load(a, first + 2 * kAppendThreads);
  const AppendChunk c3 = append_load(a, first + 3 * kAppendThreads);
  if (c0.dst >= 0) pool[c0.dst] = c0.data;
  if (c1.dst >= 0) pool[c1.dst] = c1.data;
  if (c2.dst >= 0) pool[c2.dst] = c2.data;
  if (c3.dst >= 0) pool[c3.dst] = c3.data;
}
static_assert(kAppendChunksPerThread == 4, "kv_append_vec_kernel moves four chunks per thread");

// Fallback for sources whose rows are not 16 B aligned: one fp16 word per thread.
__global__ __launch_bounds__(kAppendThreads) void kv_append_word_kernel(
    uint16_t* __restrict__ pool, int64_t num_blocks, int layer_begin, uint32_t num_tokens,
    uint64_t total_words, const char* __restrict__ key, int64_t key_layer_bytes,
    int64_t key_token_bytes, const char* __restrict__ value, int64_t value_layer_bytes,
    int64_t value_token_bytes, const int64_t* __restrict__ slot_mapping) {
  const int64_t slot_limit = num_blocks * kSlots;
  const uint64_t w = static_cast<uint64_t>(blockIdx.x) * kAppendThreads + threadIdx.x;
  if (w >= total_words) return;
  const uint32_t e = w % kRowElems;
  const uint64_t row = w / kRowElems;
  const uint32_t kind = row & 1u;
  const uint64_t rest = row >> 1;
  const uint32_t t = rest % num_tokens;
  const uint32_t l = rest / num_tokens;
  const int64_t slot = slot_mapping[t];
  if (slot < 0 || slot >= slot_limit) return;
  const char* src = kind ? value + l * value_layer_bytes + t * value_token_bytes
                         : key + l * key_layer_bytes + t * key_token_bytes;
  pool[((static_cast<int64_t>(layer_begin + l) * 2 + kind) * slot_limit + slot) * kRowElems + e] =
      *reinterpret_cast<const uint16_t*>(src + e * 2);
}

// ---------------------------------------------------------------------------------------
// Paged decode attention.
//
// Split-K over work items: item i of sequence b covers blocks [W i, W i + W) of its table
// (W = partition_blocks, 1/2/4/8) for all 4 kv heads. One workgroup of W waves per item;
// wave w owns block W i + w and issues every load of that block at once:
//   * K, 8 KiB: per kv head h two 16 B loads per lane, lane (c = lane % 16, g = lane / 16)
//     taking K[slot c][h][8g .. 8g + 7] and [32 + 8g ..] -- already the A operand of
//     v_mfma_f32_16x16x32_f16;
//   * V, 8 KiB: eight 16 B loads per lane, each instruction one contiguous KiB (whole 128 B
//     lines), staged through LDS rows of 512 B + 32 B pad.
// No wave ever waits for a second round of loads, so the whole grid's requests are in the
// memory queues at once and the kernel drains HBM at its streaming rate.
//
// Per kv head (all in registers, one block so no online rescaling):
//   * S^T[16 tokens][16] = K . Q^T on the matrix core (columns 8..15 repeat q heads 0..7);
//     lane (c, g) receives the raw dots of q head 8h + c % 8 for tokens 4g .. 4g + 3;
//   * masked tokens (past the context) become -inf and their V rows are zeroed in LDS,
//     so poisoned tail slots never reach a product (0 x NaN would);
//   * p = 2^((dot - max) log2(e) / 8): the 1/8 scale is applied to the exact difference;
//   * O[16][16 dims] += P . V with v_mfma_f32_16x16x16f16: rows 0..7 carry the fp16
//     rounding of p, rows 8..15 the remainder scaled by 2^18, so the product keeps fp32
//     accuracy; V reaches the B layout through transposing LDS reads (ds_read_b64_tr_b16).
// The W waves then meet in LDS: each thread folds D = 32 / W outputs of one q head over
// the waves (max / rescale / sum). A sequence that fits one item writes fp16 output;
// otherwise the item's (max, sum, unnormalized output) goes to the workspace and the
// sequence's items are merged by paged_decode_merge_kernel, or -- flags 0 -- by the last
// workgroup of the sequence to finish (atomic ticket).
// ---------------------------------------------------------------------------------------

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef short short4_t __attribute__((ext_vector_type(4)));

constexpr int kDefaultPartitionBlocks = 8;
constexpr int kVPitch = 544;                   // bytes per staged V row: 512 B of data + 32 B pad
constexpr int kWaveLds = kSlots * kVPitch;     // 8704 B of LDS per wave
constexpr int kItemOutputs = kQHeads * kHeadDim;  // 2048 fp32 outputs per item
constexpr int kMergeThreads = 256;             // separate merge: one workgroup per (sequence, 8 q heads)
// Plan record: {sequence, item, context length, closer flag, block ids of the item's W
// blocks (0 past the sequence's last block)}, padded to a multiple of 4 int32.
constexpr int kPlanHeader = 4;
// Ticket polls a closer makes before giving up on its siblings (each a round trip of about
// a microsecond plus a short sleep): ends the wait well under a second in any case.
constexpr int kCloserPolls = 1 << 16;
constexpr int plan_fields(int w) { return kPlanHeader + (w + 3) / 4 * 4; }
// log2(e) / sqrt(64): turns a raw q.k difference into a base-2 exponent.
constexpr float kScoreToLog2 = 0.18033688011112042f;
// Scale of the low (remainder) part of p in the PV product (2^18).
constexpr float kLowScale = 262144.0f;
static_assert(kWaveLds >= (kItemOutputs + 2 * kQHeads) * 4, "a wave's LDS also holds its partial");

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Max / sum over the 4 lanes l, l^16, l^32, l^48 (one q head's 4 token groups); every
// lane gets the result.
__device__ __forceinline__ float max_over_groups(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

__device__ __forceinline__ float sum_over_groups(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// Reduce-scatter of a PV tile pair over the wave halves: lanes < 32 get
// x[l] + x[l + 32] / 2^18, lanes >= 32 get y[l - 32] + y[l] / 2^18 (the high rows of a
// 16x16 tile sit in lanes 0..31, its scaled low rows in lanes 32..63).
__device__ __forceinline__ float fold_low_rows(float x, float y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return fmaf(__uint_as_float(r[1]), 1.0f / kLowScale, __uint_as_float(r[0]));
}

// LDS ordering inside one wave: the compiler keeps LDS accesses on their side of this
// point and the wave's LDS operations complete in issue order.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct AttnArgs {
  _Float16* out;
  const _Float16* query;
  const _Float16* pool;
  int64_t num_blocks;
  const int32_t* block_tables;
  const int32_t* context_lens;
  float* ws_out;     // [batch][max_items][32 q heads][64] unnormalized item outputs
  float* ws_ml;      // [batch][max_items][32 q heads][2] (max of raw dots, sum of p)
  int32_t* tickets;  // [batch] merge tickets, zero between calls
  const int32_t* work_items;  // (sequence, item) pairs, or null: every (sequence, item slot)
  int layer, max_blocks, batch, max_items, fused_merge;
};

// Items of a sequence (0 for an empty one); nblk = its block count, clamped to the table.
__device__ __forceinline__ int items_of(int len, int max_blocks, int w, int& nblk) {
  nblk = len > 0 ? min((len - 1) / kSlots + 1, max_blocks) : 0;
  return (nblk + w - 1) / w;
}

// Agent-coherent accesses (global_store / global_load ... sc1): partials published by a
// workgroup on one XCD are visible to a workgroup on any XCD without a cache writeback or
// invalidate. The plain variants serve the separate merge kernel, which runs after the
// item kernel has completed.
template <bool kCoherent>
__device__ __forceinline__ void store_f2(float* p, float x, float y) {
  if constexpr (kCoherent) {
    const uint64_t bits = (static_cast<uint64_t>(__float_as_uint(y)) << 32) | __float_as_uint(x);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *reinterpret_cast<float2_t*>(p) = float2_t{x, y};
  }
}

template <bool kCoherent>
__device__ __forceinline__ float2_t load_f2(const float* p) {
  if constexpr (kCoherent) {
    const uint64_t x = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    return float2_t{__uint_as_float(static_cast<uint32_t>(x)), __uint_as_float(static_cast<uint32_t>(x >> 32))};
  } else {
    return *reinterpret_cast<const float2_t*>(p);
  }
}

// Items whose partials one merge round trip loads, for D outputs per thread.
constexpr int merge_batch(int d) { return d <= 2 ? 32 : (d <= 4 ? 16 : (d <= 8 ? 8 : 4)); }

// Folds items [i_begin, nitems) of sequence b into the running state (m, l, o) for dims
// [o0, o0 + D) of q head `qhead` (D even) with the online-softmax rule; the loads of
// merge_batch(D) items are issued before any of them is used. Returns the normalized
// outputs in `res`.
template <bool kCoherent, int D>
__device__ __forceinline__ void merge_items_from(const AttnArgs& a, int b, int i_begin, int nitems, int qhead, int o0,
                                                 float m, float l, float (&o)[D], float (&res)[D]) {
  constexpr int kBatch = merge_batch(D);
  const int64_t first = static_cast<int64_t>(b) * a.max_items;
#pragma unroll 1
  for (int i0 = i_begin; i0 < nitems; i0 += kBatch) {
    float2_t ml[kBatch];
    float2_t x[kBatch][D / 2];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int64_t p = first + min(i0 + j, nitems - 1);  // clamped: always in bounds
      ml[j] = load_f2<kCoherent>(a.ws_ml + (p * kQHeads + qhead) * 2);
      const float* xp = a.ws_out + p * kItemOutputs + qhead * kHeadDim + o0;
#pragma unroll
      for (int i = 0; i < D / 2; ++i) x[j][i] = load_f2<kCoherent>(xp + 2 * i);
    }
    // Branch-free fold (a branch would let the compiler sink each load to its use): a
    // clamped duplicate gets weight 0; m is finite from the first item on, so m_new is too.
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const float mp = (i0 + j < nitems) ? ml[j][0] : -INFINITY;
      const float m_new = fmaxf(m, mp);
      const float s_old = exp2_fast((m - m_new) * kScoreToLog2);  // 0 while m = -inf
      const float s_new = exp2_fast((mp - m_new) * kScoreToLog2);  // 0 for a duplicate
      // Explicit fmaf: every instantiation (and so both merge modes) rounds identically.
      l = fmaf(ml[j][1], s_new, l * s_old);
#pragma unroll
      for (int i = 0; i < D / 2; ++i) {
        o[2 * i] = fmaf(x[j][i][0], s_new, o[2 * i] * s_old);
        o[2 * i + 1] = fmaf(x[j][i][1], s_new, o[2 * i + 1] * s_old);
      }
      m = m_new;
    }
  }
  const float inv = 1.0f / l;
#pragma unroll
  for (int i = 0; i < D; ++i) res[i] = o[i] * inv;
}

template <bool kCoherent, int D>
__device__ __forceinline__ void merge_items(const AttnArgs& a, int b, int nitems, int qhead, int o0, float (&res)[D]) {
  float o[D];
#pragma unroll
  for (int i = 0; i < D; ++i) o[i] = 0.f;
  merge_items_from<kCoherent, D>(a, b, 0, nitems, qhead, o0, -INFINITY, 0.f, o, res);
}

// The closer's fold: items [0, nitems) of sequence b in item order with the same
// arithmetic as merge_items, item `own` taken from registers (m_own, l_own, x_own) and the
// others through agent-coherent loads. Unused batch slots and the own item's (never
// written) workspace entries are selected out, never multiplied, so the result is
// bit-identical to the separate merge.
template <int D>
__device__ __forceinline__ void merge_with_own(const AttnArgs& a, int b, int nitems, int own, int qhead, int o0,
                                               float m_own, float l_own, const float (&x_own)[D], float (&res)[D]) {
  constexpr int kBatch = merge_batch(D);
  float m = -INFINITY, l = 0.f, o[D];
#pragma unroll
  for (int i = 0; i < D; ++i) o[i] = 0.f;
  const int64_t first = static_cast<int64_t>(b) * a.max_items;
#pragma unroll 1
  for (int i0 = 0; i0 < nitems; i0 += kBatch) {
    float2_t ml[kBatch];
    float2_t x[kBatch][D / 2];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int64_t p = first + min(i0 + j, nitems - 1);  // clamped: always in bounds
      ml[j] = load_f2<true>(a.ws_ml + (p * kQHeads + qhead) * 2);
      const float* xp = a.ws_out + p * kItemOutputs + qhead * kHeadDim + o0;
#pragma unroll
      for (int i = 0; i < D / 2; ++i) x[j][i] = load_f2<true>(xp + 2 * i);
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int idx = i0 + j;
      const bool used = idx < nitems;
      const bool mine = idx == own;
      const float mp = !used ? -INFINITY : (mine ? m_own : ml[j][0]);
      const float lp = !used ? 0.f : (mine ? l_own : ml[j][1]);
      const float m_new = fmaxf(m, mp);
      const float s_old = exp2_fast((m - m_new) * kScoreToLog2);
      const float s_new = exp2_fast((mp - m_new) * kScoreToLog2);
      l = fmaf(lp, s_new, l * s_old);
#pragma unroll
      for (int i = 0; i < D / 2; ++i) {
        const float x0 = !used ? 0.f : (mine ? x_own[2 * i] : x[j][i][0]);
        const float x1 = !used ? 0.f : (mine ? x_own[2 * i + 1] : x[j][i][1]);
        o[2 * i] = fmaf(x0, s_new, o[2 * i] * s_old);
        o[2 * i + 1] = fmaf(x1, s_new, o[2 * i + 1] * s_old);
      }
      m = m_new;
    }
  }
  const float inv = 1.0f / l;
#pragma unroll
  for (int i = 0; i < D; ++i) res[i] = o[i] * inv;
}

template <int D>
__device__ __forceinline__ void store_out(_Float16* dst, const float (&v)[D]) {
#pragma unroll
  for (int i = 0; i < D; i += 2) {
    *reinterpret_cast<half2_t*>(dst + i) = half2_t{static_cast<_Float16>(v[i]), static_cast<_Float16>(v[i + 1])};
  }
}

template <int W, bool kPlanned>
__global__ __launch_bounds__(64 * W) void paged_decode_item_kernel(AttnArgs a) {
  constexpr int D = kItemOutputs / (64 * W);  // outputs per thread in the workgroup merge
  __shared__ __attribute__((aligned(16))) char lds[W * kWaveLds];
  __shared__ int32_t ticket_slot;

  // Wave index as a scalar, so every per-wave address below is scalar arithmetic and the
  // block-id loads are scalar loads.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = lane & 15;
  const int g = lane >> 4;

  int b, item, len;
  int32_t id;
  bool closer;  // merges the sequence's items (fused merge)
  const int blk_in_item = wave;
  if constexpr (kPlanned) {
    // Planned grid: one workgroup per item that exists. The record header and this
    // wave's block id are requested together, before any branch, so the KV loads leave
    // after a single round trip.
    const int32_t* rec = a.work_items + static_cast<int64_t>(blockIdx.x) * plan_fields(W);
    const int4 hdr = *reinterpret_cast<const int4*>(rec);
    id = rec[kPlanHeader + blk_in_item];
    // A record outside the batch or the workspace is skipped at the item check below; it
    // is clamped, not branched on, here so that no load waits behind the check.
    const bool in_range = static_cast<uint32_t>(hdr.x) < static_cast<uint32_t>(a.batch) &&
                          static_cast<uint32_t>(hdr.y) < static_cast<uint32_t>(a.max_items);
    b = in_range ? hdr.x : 0;
    item = in_range ? hdr.y : a.max_items;
    len = hdr.z;
    closer = hdr.w != 0;
    // The block id is consumed here so that its load leaves with the header's instead
    // of after the item check below.
    asm volatile("" ::"s"(id));
  } else {
    // Full grid: item slots past a sequence's length exit below; the length and this
    // wave's block id come from the device tables in one round trip.
    b = blockIdx.x % a.batch;
    item = blockIdx.x / a.batch;
    id = a.block_tables[static_cast<int64_t>(b) * a.max_blocks + min(item * W + blk_in_item, a.max_blocks - 1)];
    len = a.context_lens[b];
  }
  const int blk = item * W + blk_in_item;
  // B operand = Q^T per kv head h: column c is q head 8h + c % 8.
  const _Float16* qrow = a.query + (static_cast<int64_t>(b) * kQHeads + (c & 7)) * kHeadDim + 8 * g;
  half8_t qa[kKVHeads], qb[kKVHeads];
#pragma unroll
  for (int h = 0; h < kKVHeads; ++h) {
    qa[h] = *reinterpret_cast<const half8_t*>(qrow + h * kGroup * kHeadDim);
    qb[h] = *reinterpret_cast<const half8_t*>(qrow + h * kGroup * kHeadDim + 32);
  }
  int nblk;
  const int nitems = items_of(len, a.max_blocks, W, nblk);
  if (item >= nitems) return;  // uniform over the workgroup
  if constexpr (!kPlanned) closer = item == nitems - 1;  // the sequence's highest workgroup index
  const bool active = blk < nblk;  // uniform over the wave; wave 0 is always active

  char* vl = lds + wave * kWaveLds;
  float* part = reinterpret_cast<float*>(vl);  // after PV: [32 q heads][64] outputs, then (m, l) pairs
  if (active) {
    uint32_t phys = static_cast<uint32_t>(id);
    const bool bad = phys >= static_cast<uint64_t>(a.num_blocks);  // negative ids wrap to huge values
    if (bad) phys = 0;  // never dereferenced out of the pool
    const int64_t kind_elems = a.num_blocks * kBlockElems;
    const _Float16* kblk = a.pool + static_cast<int64_t>(a.layer) * 2 * kind_elems + static_cast<int64_t>(phys) * kBlockElems;
    const char* vblk = reinterpret_cast<const char*>(kblk + kind_elems);
    half8_t k0[kKVHeads], k1[kKVHeads];
#pragma unroll
    for (int h = 0; h < kKVHeads; ++h) {
      k0[h] = *reinterpret_cast<const half8_t*>(kblk + c * kRowElems + h * kHeadDim + 8 * g);
      k1[h] = *reinterpret_cast<const half8_t*>(kblk + c * kRowElems + h * kHeadDim + 32 + 8 * g);
    }
    uint4 vraw[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) vraw[q] = *reinterpret_cast<const uint4*>(vblk + q * 1024 + lane * 16);

    const int valid = len - blk * kSlots;  // >= 1; below 16 only in the sequence's last block
    // V rows to LDS; in the sequence's last block the rows of masked slots are zeroed.
    char* vdst = vl + (lane >> 5) * kVPitch + (lane & 31) * 16;
    if (valid >= kSlots) {
#pragma unroll
      for (int q = 0; q < 8; ++q) *reinterpret_cast<uint4*>(vdst + 2 * q * kVPitch) = vraw[q];
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int slot = 2 * q + (lane >> 5);
        *reinterpret_cast<uint4*>(vdst + 2 * q * kVPitch) = slot < valid ? vraw[q] : uint4{0, 0, 0, 0};
      }
    }
    wave_lds_fence();

    float o[kKVHeads][2][4];
    float mh[kKVHeads], lh[kKVHeads];
#pragma unroll
    for (int h = 0; h < kKVHeads; ++h) {
      float4_t s = {0.f, 0.f, 0.f, 0.f};
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0[h], qa[h], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1[h], qb[h], s, 0, 0, 0);
      float sc[4] = {s[0], s[1], s[2], s[3]};
      if (valid < kSlots) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] = 4 * g + r < valid ? sc[r] : -INFINITY;
      }
      // Block max of q head c % 8 over all 16 tokens (finite: token 0 is always valid).
      const float mblk = max_over_groups(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
      float p[4];
      // exp2(-inf) = 0: masked tokens get no weight.
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = exp2_fast((sc[r] - mblk) * kScoreToLog2);
      lh[h] = sum_over_groups((p[0] + p[1]) + (p[2] + p[3]));
      mh[h] = mblk;
      // A operand: row c holds p of q head c % 8 for tokens 4g .. 4g + 3: for c < 8 the
      // fp16 rounding of p, for c >= 8 the remainder scaled by 2^18 (p <= 1 bounds it by
      // 2^7, and the scale keeps p down to 2^-32 in fp16's normal range).
      half4_t pa;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float hi = static_cast<float>(static_cast<_Float16>(p[r]));
        pa[r] = static_cast<_Float16>(c >= kGroup ? (p[r] - hi) * kLowScale : p[r]);
      }
      // Lane (c, g) reads row 4g + c/4, dims 16nt + 4(c%4) .. + 3 of head h; the
      // transposing read hands it V[tokens 4g .. 4g + 3][dim 16nt + c], the B operand.
      const char* vrow = vl + (4 * g + (c >> 2)) * kVPitch + h * kHeadDim * 2 + 8 * (c & 3);
      float4_t acc[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const short4_t raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            reinterpret_cast<__attribute__((address_space(3))) short4_t*>(reinterpret_cast<uintptr_t>(vrow + 32 * nt)));
        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4_t, raw),
                                                        float4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      }
      // High rows plus unscaled low rows: lane (c, g) then holds q head 8h + 4(g & 1) + r,
      // dim 16(2k + g / 2) + c (lanes g < 2 from tile 2k, g >= 2 from tile 2k + 1).
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[h][k][r] = fold_low_rows(acc[2 * k][r], acc[2 * k + 1][r]);
    }
    // The partial overwrites this wave's V rows: every PV read above has been issued.
    wave_lds_fence();
#pragma unroll
    for (int h = 0; h < kKVHeads; ++h)
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int qh = kGroup * h + 4 * (g & 1) + r;
          part[qh * kHeadDim + 16 * (2 * k + (g >> 1)) + c] = bad ? NAN : o[h][k][r];
        }
    if (lane < kGroup) {
#pragma unroll
      for (int h = 0; h < kKVHeads; ++h) {
        *reinterpret_cast<float2_t*>(part + kItemOutputs + (kGroup * h + lane) * 2) = float2_t{mh[h], lh[h]};
      }
    }
  }
  __syncthreads();

  // Workgroup merge: thread t folds outputs [t D, t D + D) -- q head t D / 64 -- over the
  // item's active waves.
  const int t = threadIdx.x;
  const int qhead = (t * D) / kHeadDim;
  const int o0 = (t * D) % kHeadDim;
  const int nact = min(W, nblk - item * W);
  float m = -INFINITY;
  for (int w = 0; w < nact; ++w) {
    m = fmaxf(m, reinterpret_cast<const float*>(lds + w * kWaveLds)[kItemOutputs + qhead * 2]);
  }
  float l = 0.f, acc[D];
#pragma unroll
  for (int i = 0; i < D; ++i) acc[i] = 0.f;
  for (int w = 0; w < nact; ++w) {
    const float* pw = reinterpret_cast<const float*>(lds + w * kWaveLds);
    const float2_t ml = *reinterpret_cast<const float2_t*>(pw + kItemOutputs + qhead * 2);
    const float e = exp2_fast((ml[0] - m) * kScoreToLog2);
    l += ml[1] * e;
#pragma unroll
    for (int i = 0; i < D; i += 4) {
      const float4_t x = *reinterpret_cast<const float4_t*>(pw + qhead * kHeadDim + o0 + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i + j] += x[j] * e;
    }
  }
  _Float16* out = a.out + (static_cast<int64_t>(b) * kQHeads + qhead) * kHeadDim + o0;
  if (nitems == 1) {
    float res[D];
    const float inv = 1.0f / l;
#pragma unroll
    for (int i = 0; i < D; ++i) res[i] = acc[i] * inv;
    store_out<D>(out, res);
    return;
  }
  const int64_t pidx = static_cast<int64_t>(b) * a.max_items + item;
  float* ws_out = a.ws_out + pidx * kItemOutputs + qhead * kHeadDim + o0;
  float* ws_ml = a.ws_ml + (pidx * kQHeads + qhead) * 2;
  if (!a.fused_merge) {
#pragma unroll
    for (int i = 0; i < D; i += 4) *reinterpret_cast<float4_t*>(ws_out + i) = float4_t{acc[i], acc[i + 1], acc[i + 2], acc[i + 3]};
    if (o0 == 0) store_f2<false>(ws_ml, m, l);
    return;
  }

  // Fused merge. Every item but the closer publishes its partial with agent-coherent
  // stores, waits until they have completed, then bumps the sequence's ticket. The closer
  // (dispatched after all of them) waits -- a bounded number of polls -- until the ticket
  // shows every sibling, folds the siblings' partials (agent-coherent loads) and its own
  // (registers) in item order, writes the output and re-arms the ticket.
  if (!closer) {
#pragma unroll
    for (int i = 0; i < D; i += 2) store_f2<true>(ws_out + i, acc[i], acc[i + 1]);
    if (o0 == 0) store_f2<true>(ws_ml, m, l);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): every store of this thread has completed
    __syncthreads();
    if (t == 0) __hip_atomic_fetch_add(&a.tickets[b], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if (t == 0) {
    int seen = 0;
    for (int poll = 0; poll < kCloserPolls; ++poll) {
      seen = __hip_atomic_load(&a.tickets[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (seen >= nitems - 1) break;
      __builtin_amdgcn_s_sleep(8);
    }
    ticket_slot = seen;
  }
  __syncthreads();
  float res[D];
  if (ticket_slot != nitems - 1) {
    // The siblings never all arrived within the poll budget: the row becomes NaN rather
    // than a wait without end.
#pragma unroll
    for (int i = 0; i < D; ++i) res[i] = NAN;
  } else {
    merge_with_own<D>(a, b, nitems, item, qhead, o0, m, l, acc, res);
  }
  store_out<D>(out, res);
  if (t == 0) __hip_atomic_store(&a.tickets[b], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Separate merge of every multi-item sequence: one workgroup per (sequence, group of 8 q
// heads); thread t folds dims 2(t % 32), +1 of q head 8 (blockIdx % 4) + t / 32, loading
// up to merge_batch(2) = 32 items' partials per round trip.
__global__ __launch_bounds__(kMergeThreads) void paged_decode_merge_kernel(AttnArgs a, int w) {
  const int b = blockIdx.x / kKVHeads;
  const int qhead = kGroup * (blockIdx.x % kKVHeads) + threadIdx.x / 32;
  const int o0 = 2 * (threadIdx.x % 32);
  int nblk;
  const int nitems = items_of(a.context_lens[b], a.max_blocks, w, nblk);
  if (nitems <= 1) return;
  float res[2];
  merge_items<false, 2>(a, b, nitems, qhead, o0, res);
  store_out<2>(a.out + (static_cast<int64_t>(b) * kQHeads + qhead) * kHeadDim + o0, res);
}

// ---------------------------------------------------------------------------------------
// Host-side validation and workspace layout.
// ---------------------------------------------------------------------------------------

int max_items(int32_t max_blocks, int32_t partition_blocks) {
  return (max_blocks + partition_blocks - 1) / partition_blocks;
}

bool valid_partition(int32_t p) { return p == 1 || p == 2 || p == 4 || p == 8; }

int check_attn_shape(int32_t batch, int32_t max_blocks, int32_t partition_blocks) {
  if (batch < 0 || batch > (1 << 20)) return set_error(PC_ERR_ARGUMENT, "batch %d out of range", batch);
  if (max_blocks < 1 || max_blocks > (1 << 16)) {
    return set_error(PC_ERR_ARGUMENT, "max_blocks %d out of range [1, 65536]", max_blocks);
  }
  if (!valid_partition(partition_blocks)) {
    return set_error(PC_ERR_ARGUMENT, "partition_blocks %d is not 1, 2, 4 or 8", partition_blocks);
  }
  const int64_t grid = static_cast<int64_t>(batch) * max_items(max_blocks, partition_blocks);
  if (grid > INT32_MAX) return set_error(PC_ERR_ARGUMENT, "attention grid too large");
  return PC_OK;
}

// Workspace = ws_out floats | ws_ml floats, each region 256 B aligned.
struct WorkspaceLayout {
  int64_t out_offset, ml_offset, bytes;
};

WorkspaceLayout workspace_layout(int32_t batch, int32_t max_blocks, int32_t partition_blocks) {
  auto round_up = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int64_t items = static_cast<int64_t>(batch) * max_items(max_blocks, partition_blocks);
  WorkspaceLayout w;
  w.out_offset = 0;
  w.ml_offset = round_up(items * kItemOutputs * 4);
  w.bytes = w.ml_offset + round_up(items * kQHeads * 2 * 4);
  return w;
}

bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

template <int W>
void launch_items(const AttnArgs& a, unsigned grid, hipStream_t s) {
  if (a.work_items) {
    hipLaunchKernelGGL((paged_decode_item_kernel<W, true>), dim3(grid), dim3(64 * W), 0, s, a);
  } else {
    hipLaunchKernelGGL((paged_decode_item_kernel<W, false>), dim3(grid), dim3(64 * W), 0, s, a);
  }
}

}  // namespace

extern "C" {

int pc_abi_version(void) { return kAbiVersion; }

const char* pc_last_error(void) { return g_error; }

int32_t pc_attn_default_partition_blocks(void) { return kDefaultPartitionBlocks; }

int64_t pc_attn_workspace_bytes(int32_t batch, int32_t max_blocks, int32_t partition_blocks) {
  if (check_attn_shape(batch, max_blocks, partition_blocks) != PC_OK) return 0;
  return workspace_layout(batch, max_blocks, partition_blocks).bytes;
}

int64_t pc_attn_plan_capacity(int32_t batch, int32_t max_blocks, int32_t partition_blocks) {
  if (check_attn_shape(batch, max_blocks, partition_blocks) != PC_OK) return -1;
  return static_cast<int64_t>(batch) * max_items(max_blocks, partition_blocks);
}

int32_t pc_attn_plan_record_ints(int32_t partition_blocks) {
  if (!valid_partition(partition_blocks)) {
    return -set_error(PC_ERR_ARGUMENT, "partition_blocks %d is not 1, 2, 4 or 8", partition_blocks);
  }
  return plan_fields(partition_blocks);
}

int32_t pc_attn_plan(const int32_t* context_lens, const int32_t* block_tables, int32_t batch,
                     int32_t max_blocks, int32_t partition_blocks, int32_t* work_items, int64_t capacity) {
  if (int rc = check_attn_shape(batch, max_blocks, partition_blocks)) return -rc;
  if (batch > 0 && (!context_lens || !block_tables || !work_items)) {
    return -set_error(PC_ERR_ARGUMENT, "null pointer");
  }
  const int fields = plan_fields(partition_blocks);
  int64_t total = 0;
  for (int32_t b = 0; b < batch; ++b) {
    const int32_t len = context_lens[b];
    if (len > 0) total += max_items(std::min((len - 1) / kSlots + 1, max_blocks), partition_blocks);
  }
  if (total > capacity) {
    return -set_error(PC_ERR_ARGUMENT, "work item capacity %lld too small (%lld items)",
                      static_cast<long long>(capacity), static_cast<long long>(total));
  }
  // Workgroups are dispatched in record order. A multi-item sequence's closer -- its last
  // item, the one with the fewest blocks -- goes after every other item of every
  // sequence, so when it finishes its own blocks its siblings have long published their
  // partials; before the closers, items with fewer blocks go later.
  int64_t n = 0;
  for (int pass = 0; pass < 2; ++pass) {
    const bool closers = pass == 1;
    for (int32_t count = partition_blocks; count >= 1; --count) {
      for (int32_t b = 0; b < batch; ++b) {
        const int32_t len = context_lens[b];
        if (len <= 0) continue;
        const int32_t nblk = std::min((len - 1) / kSlots + 1, max_blocks);
        const int32_t items = max_items(nblk, partition_blocks);
        const int32_t* row = block_tables + static_cast<int64_t>(b) * max_blocks;
        for (int32_t i = 0; i < items; ++i) {
          const bool closer = items > 1 && i == items - 1;
          if (closer != closers || std::min(nblk - i * partition_blocks, partition_blocks) != count) continue;
          int32_t* rec = work_items + n * fields;
          rec[0] = b;
          rec[1] = i;
          rec[2] = len;
          rec[3] = closer ? 1 : 0;
          for (int32_t j = 0; j < fields - kPlanHeader; ++j) {
            const int32_t blk = i * partition_blocks + j;
            rec[kPlanHeader + j] = (j < count) ? row[blk] : 0;
          }
          ++n;
        }
      }
    }
  }
  ok();
  return static_cast<int32_t>(n);
}

int pc_kv_append(void* pool, int64_t num_blocks, int32_t layer_begin, int32_t num_layers,
                 const void* key, int64_t key_layer_stride, int64_t key_token_stride,
                 const void* value, int64_t value_layer_stride, int64_t value_token_stride,
                 const int64_t* slot_mapping, int64_t num_tokens, void* stream) {
  if (!pool || !key || !value || !slot_mapping) return set_error(PC_ERR_ARGUMENT, "null pointer");
  if (num_blocks < 1 || num_blocks > (INT64_MAX / (kLayers * 2 * kBlockElems * 2))) {
    return set_error(PC_ERR_ARGUMENT, "num_blocks %lld out of range", static_cast<long long>(num_blocks));
  }
  if (num_layers < 1 || layer_begin < 0 || layer_begin + num_layers > kLayers) {
    return set_error(PC_ERR_ARGUMENT, "layers [%d, %d) outside [0, %d)", layer_begin,
                     layer_begin + num_layers, kLayers);
  }
  if (num_tokens < 0) return set_error(PC_ERR_ARGUMENT, "negative token count");
  if (num_tokens == 0) return ok();
  const uint64_t rows = static_cast<uint64_t>(num_layers) * num_tokens * 2;
  if (rows * kRowElems > (uint64_t{1} << 40) || rows * kRowChunks > UINT32_MAX) {
    return set_error(PC_ERR_ARGUMENT, "append of %lld tokens too large", static_cast<long long>(num_tokens));
  }
  if (!aligned(pool, 16)) return set_error(PC_ERR_ARGUMENT, "pool must be 16-byte aligned");
  const int64_t kl = key_layer_stride * 2, kt = key_token_stride * 2;
  const int64_t vl = value_layer_stride * 2, vt = value_token_stride * 2;
  hipStream_t s = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  const bool vec = aligned(key, 16) && aligned(value, 16) && kl % 16 == 0 && kt % 16 == 0 &&
                   vl % 16 == 0 && vt % 16 == 0;
  if (vec) {
    const uint64_t chunks = rows * kRowChunks;
    const uint64_t per_block = kAppendThreads * kAppendChunksPerThread;
    const unsigned grid = static_cast<unsigned>((chunks + per_block - 1) / per_block);
    AppendArgs a;
    a.key = static_cast<const char*>(key);
    a.value = static_cast<const char*>(value);
    a.slot_mapping = slot_mapping;
    a.key_layer_bytes = kl;
    a.key_token_bytes = kt;
    a.value_layer_bytes = vl;
    a.value_token_bytes = vt;
    a.slot_limit = num_blocks * kSlots;
    a.layer_begin = layer_begin;
    a.num_tokens = static_cast<uint32_t>(num_tokens);
    a.total_rows = static_cast<uint32_t>(rows);
    hipLaunchKernelGGL(kv_append_vec_kernel, dim3(grid), dim3(kAppendThreads), 0, s,
                       static_cast<uint4*>(pool), a);
  } else {
    if (!aligned(key, 2) || !aligned(value, 2)) return set_error(PC_ERR_ARGUMENT, "K/V must be 2-byte aligned");
    const uint64_t words = rows * kRowElems;
    const unsigned grid = static_cast<unsigned>((words + kAppendThreads - 1) / kAppendThreads);
    hipLaunchKernelGGL(kv_append_word_kernel, dim3(grid), dim3(kAppendThreads), 0, s,
                       static_cast<uint16_t*>(pool), num_blocks, layer_begin,
                       static_cast<uint32_t>(num_tokens), words, static_cast<const char*>(key), kl, kt,
                       static_cast<const char*>(value), vl, vt, slot_mapping);
  }
  return check_launch("kv_append");
}

int pc_paged_decode_attn(void* out, const void* query, const void* pool, int64_t num_blocks,
                         int32_t layer, const int32_t* block_tables, int32_t max_blocks,
                         const int32_t* context_lens, int32_t batch, int32_t partition_blocks,
                         const int32_t* work_items, int32_t num_work_items, void* workspace,
                         int32_t* tickets, int32_t flags, void* stream) {
  if (!out || !query || !pool || !block_tables || !context_lens) {
    return set_error(PC_ERR_ARGUMENT, "null pointer");
  }
  if (num_blocks < 1 || num_blocks > INT32_MAX) return set_error(PC_ERR_ARGUMENT, "num_blocks out of range");
  if (layer < 0 || layer >= kLayers) return set_error(PC_ERR_ARGUMENT, "layer %d outside [0, 22)", layer);
  if (int rc = check_attn_shape(batch, max_blocks, partition_blocks)) return rc;
  if (flags & ~PC_ATTN_SEPARATE_REDUCE) return set_error(PC_ERR_ARGUMENT, "unknown flags 0x%x", flags);
  const int items = max_items(max_blocks, partition_blocks);
  if (items > 1 && !workspace) return set_error(PC_ERR_ARGUMENT, "workspace required");
  if (items > 1 && !(flags & PC_ATTN_SEPARATE_REDUCE) && !tickets) {
    return set_error(PC_ERR_ARGUMENT, "tickets required for the fused merge");
  }
  if (!aligned(query, 16) || !aligned(out, 16) || !aligned(pool, 16) || !aligned(workspace, 256) ||
      !aligned(tickets, 4) || !aligned(work_items, 4)) {
    return set_error(PC_ERR_ARGUMENT,
                     "query/out/pool must be 16-byte, tickets/work_items 4-byte, workspace 256-byte aligned");
  }
  if (work_items && (num_work_items < 0 || num_work_items > static_cast<int64_t>(batch) * items)) {
    return set_error(PC_ERR_ARGUMENT, "num_work_items %d outside [0, batch * items]", num_work_items);
  }
  if (batch == 0 || (work_items && num_work_items == 0)) return ok();
  const WorkspaceLayout w = workspace_layout(batch, max_blocks, partition_blocks);
  char* base = static_cast<char*>(workspace);
  AttnArgs a;
  a.out = static_cast<_Float16*>(out);
  a.query = static_cast<const _Float16*>(query);
  a.pool = static_cast<const _Float16*>(pool);
  a.num_blocks = num_blocks;
  a.block_tables = block_tables;
  a.context_lens = context_lens;
  a.ws_out = base ? reinterpret_cast<float*>(base + w.out_offset) : nullptr;
  a.ws_ml = base ? reinterpret_cast<float*>(base + w.ml_offset) : nullptr;
  a.tickets = tickets;
  a.work_items = work_items;
  a.layer = layer;
  a.max_blocks = max_blocks;
  a.batch = batch;
  a.max_items = items;
  a.fused_merge = (flags & PC_ATTN_SEPARATE_REDUCE) ? 0 : 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  const unsigned grid = static_cast<unsigned>(work_items ? static_cast<int64_t>(num_work_items) : static_cast<int64_t>(batch) * items);
  switch (partition_blocks) {
    case 1: launch_items<1>(a, grid, s); break;
    case 2: launch_items<2>(a, grid, s); break;
    case 4: launch_items<4>(a, grid, s); break;
    default: launch_items<8>(a, grid, s); break;
  }
  if (int rc = check_launch("paged_decode_item")) return rc;
  if (items > 1 && !a.fused_merge) {
    hipLaunchKernelGGL(paged_decode_merge_kernel, dim3(static_cast<unsigned>(batch) * kKVHeads),
                       dim3(kMergeThreads), 0, s, a, static_cast<int>(partition_blocks));
    return check_launch("paged_decode_merge");
  }
  return PC_OK;
}

}  // extern "C"
