// Paged KV-cache hot path for MI355X (gfx950): KV append; paged decode attention in balanced
// bins, one workgroup each, with the split-K merge of a cut sequence's parts inside the same
// kernel (optionally also appending each sequence's newest token); and the host planner
// that cuts a batch into those bins. Exposed through the C ABI declared in
// include/pagedcore_hip.h. No device memory is allocated at run time: every buffer comes from
// the caller, except the fixed per-GPU split-K array of the allocation-free entry point.
//
// Pool layout (fixed by the reference allocator, src/pagedcore/kv_cache.py:39-43):
//   fp16 [22 layers][2 kinds][num_blocks][16 slots][4 kv heads][64 dims]
// One (layer, kind, block) is 8 KiB contiguous; one (block, kv head) is 16 rows of 128 B
// at a 512 B stride.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <vector>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "pagedcore_hip.h"
#include "pc_device.h"
#include "pc_internal.h"

namespace pc_internal {

namespace {
thread_local char g_error[512] = "";
}  // namespace

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

const char* last_error() { return g_error; }

}  // namespace pc_internal

namespace {

using namespace pc_device;
using pc_internal::aligned;
using pc_internal::check_launch;
using pc_internal::ok;
using pc_internal::set_error;

constexpr int kAbiVersion = 13;
constexpr int kLayers = 22;
constexpr int kSlots = 16;
constexpr int kKVHeads = 4;
constexpr int kQHeads = 32;
constexpr int kGroup = kQHeads / kKVHeads;  // 8 query heads per kv head
constexpr int kHeadDim = 64;
constexpr int64_t kRowElems = kKVHeads * kHeadDim;  // 256 fp16 per token row
constexpr int64_t kBlockElems = kSlots * kRowElems;  // 4096 fp16 per (layer, kind, block)
constexpr int kRowChunks = kRowElems * 2 / 16;       // 32 chunks of 16 B per token row

// ---------------------------------------------------------------------------------------
// KV append: token rows -> pool slots. Raw 16-bit moves only, so the copy is bit-exact.
// ---------------------------------------------------------------------------------------

constexpr int kAppendThreads = 256;
constexpr int kAppendChunksPerThread = 4;  // loads issued before stores for memory-level parallelism

struct AppendChunk {
  uint4 data;
  int64_t dst;  // destination in 16 B units, -1 = nothing to store
};

// The kernel's arguments. The first 56 bytes (pointers, layer strides, token strides,
// counts: everything the first loads need) are the ones the compiler preloads into SGPRs.
struct AppendArgs {
  const char* key;
  const char* value;
  const int64_t* slot_mapping;
  int64_t key_layer_bytes, value_layer_bytes;
  int32_t key_token_bytes, value_token_bytes;
  uint32_t num_tokens, total_rows;
  uint4* pool;
  int64_t slot_limit;
  int layer_begin;
};

// Chunk q (16 B) of the flattened work: q = ((l * T + t) * 2 + kind) * 32 + c. The source
// chunk and the slot are loaded together (the source address does not depend on the slot),
// so the chunk costs one memory round trip before its store.
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
    const char* src = kind ? a.value + l * a.value_layer_bytes + static_cast<int64_t>(t) * a.value_token_bytes
                           : a.key + l * a.key_layer_bytes + static_cast<int64_t>(t) * a.key_token_bytes;
    out.data = *reinterpret_cast<const uint4*>(src + c * 16);
    const int64_t slot = a.slot_mapping[t];
    if (slot >= 0 && slot < a.slot_limit) {
      // pool row (layer, kind, slot) in units of one 512 B row, then the chunk.
      out.dst = ((static_cast<int64_t>(a.layer_begin + l) * 2 + kind) * a.slot_limit + slot) *
                    kRowChunks + c;
    }
  }
  return out;
}

// Each thread moves four 16 B chunks, issuing all loads before any store. Scalar parameters
// in the order of AppendArgs, so that the leading ones are preloaded.
__global__ __launch_bounds__(kAppendThreads) void kv_append_vec_kernel(
    const char* key, const char* value, const int64_t* slot_mapping, int64_t key_layer_bytes,
    int64_t value_layer_bytes, int32_t key_token_bytes, int32_t value_token_bytes, uint32_t num_tokens,
    uint32_t total_rows, uint4* __restrict__ pool, int64_t slot_limit, int layer_begin) {
  const AppendArgs a{key, value, slot_mapping, key_layer_bytes, value_layer_bytes, key_token_bytes, value_token_bytes,
                     num_tokens, total_rows, pool, slot_limit, layer_begin};
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
// Paged decode attention over balanced bins.
//
// Work split. The host plan (pc_attn_plan) lays every sequence's blocks end to end and cuts
// them into bins of nearly equal block counts, one workgroup per bin, so that every CU
// streams the same number of bytes whatever the context lengths. Sequences are first dealt
// to 8 groups (longest first, to the group with the fewest blocks); each group is cut into
// its own bins, and bin i of group x is workgroup x + 8 i. The hardware dispatches
// workgroup j to XCD (j + s) mod 8 for one s per launch, so all bins of one sequence run on
// one XCD and share its L2. A bin holds at most kMaxSegs sequences (segments) and
// kMaxUnits blocks; a sequence longer than the rest of a bin continues in the group's next
// bin(s) (a cut sequence, spanning nspan bins). A bin that starts with the last part of a
// cut sequence merges the others after its stream and is given a few blocks fewer.
//
// Each of the four waves streams one kv head's K and V of the bin's blocks, in bin order,
// through a two-unit LDS ring filled by LDS DMA (global_load_lds_dwordx4, non-temporal: the
// pool planes are read once per pass and are far larger than the caches). Q of each segment
// is staged in LDS before the first unit. A (block, head) unit is 4 KiB: K as 16 rows of
// 128 B, 16 B chunk q of row r at position q ^ (r & 7) (the reads below are free of bank
// conflicts), then V with 32 B dim group u of row r at position u ^ row_sel(r) (for the
// transposing reads).
//
// Per block (online softmax, fp32):
//   * S^T[16 tokens][16] = K . Q^T on the matrix core (columns 8..15 repeat q heads 0..7):
//     lane (c, g) holds the raw dots of q head c % 8 for tokens 4g..4g+3;
//   * tokens past the context become -inf and their V rows are zeroed in the B operand, so
//     poisoned tail slots never reach a product (0 x NaN would);
//   * the running max is raised only when a score exceeds it by 2^8 in probability (a
//     ballot over the wave); otherwise p = 2^((dot - max) log2(e) / 8) needs no cross-lane
//     reduction;
//   * O[16][64] += P . V with v_mfma_f32_16x16x16f16: rows 0..7 carry the fp16 rounding of
//     p, rows 8..15 the remainder scaled by 2^18, so the product keeps fp32 accuracy over
//     the range p in [2^-32, 2^8]; V reaches the B layout through ds_read_b64_tr_b16.
//
// Outputs. A sequence complete within the bin is normalized into LDS during the stream and
// written after it (no store shares the wave's memory counter with the ring's loads). A cut
// sequence leaves one fp32 partial per bin and kv head in the workspace: every part but the
// last is stored by its bin, which then raises the part's flag (after the stores are
// acknowledged); the bin holding the last part (dispatched after all the others, so waiting
// cannot deadlock) stages each part in LDS as its flag rises, combines them in span order
// with its own last (their max first, then the weighted sums), lowers the flags and writes
// the output rows from registers. Partials and flags stay in the XCD's L2 (plain stores and
// loads are coherent there); the flag carries the plan's epoch, the layer and
// the writer's XCD id: a flag of another epoch or layer is not this call's and is waited
// past, and a merge that sees this call's flag with another XCD's id writes NaN rows
// instead of reading stale partials and records the fault in the workspace.
// ---------------------------------------------------------------------------------------

constexpr int kBinThreads = 64 * kKVHeads;         // one wave per kv head
constexpr int kRing = 2;                           // (block, head) units in flight per wave
constexpr int kMaxSegs = 4;                        // sequences per bin
constexpr int kMaxUnits = 256;                     // blocks per bin
constexpr int kUnitBytes = 4096;                   // K (2 KiB) then V (2 KiB) of one head of one block
constexpr int kWaveLds = kRing * kUnitBytes + 2 * kMaxSegs * 1024;  // ring, Q and output per segment
constexpr int kHeaderInts = 8;                     // {segments, blocks, plan epoch, 0 x 5}
constexpr int kSegInts = 8;                        // {sequence, length, first block, blocks, first bin, part, parts, first slot}
constexpr int kRecordInts = kHeaderInts + kMaxSegs * kSegInts;
constexpr int kRowInts = kRecordInts + kMaxUnits;  // one plan row: the record, then the block ids
constexpr int kGroups = 8;                         // XCDs of an MI355X
constexpr int kTargetBins = 256;                   // CUs of an MI355X
constexpr int kMinBinBlocks = 8;                   // smaller workloads use fewer bins
constexpr int kSlotBytes = 2176;                   // partial: O (2 KiB, lane-major), (m, l) x 8, flag; 17 lines
constexpr int kFlagOffset = 2112;
constexpr int kMaxSpins = 100000;                  // bounded wait for a part's flag
constexpr int kWorkspaceHeader = PC_ATTN_WORKSPACE_HEADER_BYTES;  // the fault word, then reserved
constexpr uint32_t kEpochMask = (1u << 22) - 1;    // plan epochs occupy flag bits 9..30
static_assert(kWorkspaceHeader % 256 == 0, "partial slots keep the workspace's 256-byte alignment");

// A raised part flag: the plan's epoch in bits 9..30, the layer in bits 4..8 and the
// writer's XCD id + 1 in bits 0..3. A flag counts for a call only if its epoch and layer
// are the call's, so a flag left raised by an earlier call (a producer whose merge gave up
// waiting, or a plan without a merging row) is never taken for this call's partial: the
// merge keeps waiting until this call's producer overwrites it.
__device__ __forceinline__ int flag_key(int epoch, int layer) {
  return static_cast<int>(((static_cast<uint32_t>(epoch) & kEpochMask) << 9) | (static_cast<uint32_t>(layer) << 4));
}
__device__ __forceinline__ bool flag_of_call(int f, int key) { return (f & 0xF) != 0 && (f & ~0xF) == key; }
// Scale of the low (remainder) part of p in the PV product (2^18).
constexpr float kLowScale = 262144.0f;
// Headroom (log2 of p) before the running max is raised.
constexpr float kLazyLog2 = 8.0f;
static_assert(kMaxUnits == 256, "the kernel reads a bin's block ids as four 64-lane vectors");
static_assert(kRing == 2, "wait_ring covers one later unit");

// Blocks holding `len` tokens, without the int32 overflow of len + 15.
__device__ __host__ __forceinline__ int blocks_of(int len) { return len / kSlots + (len % kSlots != 0); }

// One uniform int32 by a scalar load that bypasses the scalar cache (sees L2; waits on
// lgkmcnt only, so the ring's loads stay counted).
__device__ __forceinline__ int xcc_id() {
  int v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xff;
}

// The ring's unit u has landed: at most `later` units (4 DMAs each) issued after it may be
// outstanding. Loads return in order; a store among them (the fused append's, one per
// sequence) only raises the count, so the wait never ends before unit u has landed.
__device__ __forceinline__ void wait_ring(int later) {
  if (later > 0) {
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

// Reduce-scatter of a PV tile pair over the wave halves: lanes < 32 get x[l] + x[l + 32] / 2^18,
// lanes >= 32 get y[l - 32] + y[l] / 2^18 (high rows of a tile in lanes 0..31, scaled low rows
// in lanes 32..63).
__device__ __forceinline__ float fold_low_rows(float x, float y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return fmaf(__uint_as_float(r[1]), 1.0f / kLowScale, __uint_as_float(r[0]));
}

// LDS ordering inside one wave.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float lane_value(float x, int k) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), k));
}

// x of lane q (hi false) or of lane 4 + q (hi true). Both lanes are read in uniform control
// flow and each lane then selects one: a readlane written inside the two arms of a per-lane
// condition compiles to exec-masked branches around each read.
__device__ __forceinline__ float lane_value_of_half(float x, int q, bool hi) {
  const float lo_value = lane_value(x, q);
  const float hi_value = lane_value(x, 4 + q);
  return hi ? hi_value : lo_value;
}

// Partial of one (sequence, kv head) in the PV layout: lane (c, g) holds q heads 4(g&1)+r,
// dims 16(2k + g/2) + c (k = 0, 1): unnormalized O, and the max and sum of each q head.
struct Part {
  float o[2][4];
  float m[4], l[4];
};

// acc <- acc (+) p, the online-softmax fold. Explicit fmaf: every fold rounds the same way
// wherever it runs.
__device__ __forceinline__ void fold_part(Part& acc, const Part& p) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float mn = fmaxf(acc.m[r], p.m[r]);
    const float so = exp2_fast((acc.m[r] - mn) * kScoreToLog2);
    const float sn = exp2_fast((p.m[r] - mn) * kScoreToLog2);
    acc.l[r] = fmaf(p.l[r], sn, acc.l[r] * so);
    acc.o[0][r] = fmaf(p.o[0][r], sn, acc.o[0][r] * so);
    acc.o[1][r] = fmaf(p.o[1][r], sn, acc.o[1][r] * so);
    acc.m[r] = mn;
  }
}

// fp16 output rows [8 q heads][64] of a partial, normalized, in natural order into `area`
// (LDS or the output rows themselves).
__device__ __forceinline__ void put_output(char* area, int lane, const Part& p) {
  const int c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int idx = (4 * (g & 1) + r) * kHeadDim + 16 * (2 * k + (g >> 1)) + c;
      reinterpret_cast<_Float16*>(area)[idx] = static_cast<_Float16>(p.o[k][r] * (1.0f / p.l[r]));
    }
}

// A partial in a workspace slot: lane L's 8 O values at byte 32 L, then (m[4], l[4]) of q
// heads 0..3 at 2048 and of q heads 4..7 at 2080; the part's flag word at kFlagOffset.
__device__ __forceinline__ void store_part(char* slot, int lane, const Part& p) {
  float4_t* d = reinterpret_cast<float4_t*>(slot + lane * 32);
  d[0] = float4_t{p.o[0][0], p.o[0][1], p.o[0][2], p.o[0][3]};
  d[1] = float4_t{p.o[1][0], p.o[1][1], p.o[1][2], p.o[1][3]};
  if (lane == 0 || lane == 16) {
    float4_t* e = reinterpret_cast<float4_t*>(slot + 2048 + (lane >> 4) * 32);
    e[0] = float4_t{p.m[0], p.m[1], p.m[2], p.m[3]};
    e[1] = float4_t{p.l[0], p.l[1], p.l[2], p.l[3]};
  }
}

// A partial staged in LDS by stage_part: lane L's O at 16 L and 1024 + 16 L, lane L's
// copy of (m, l) word L % 16 at 2048 + 4 L (words 0-3 m of q heads 0-3, 4-7 their l, 8-11 m
// of q heads 4-7, 12-15 their l).
constexpr int kStageBytes = 2048 + 256;
constexpr int kStageParts = kWaveLds / kStageBytes;  // partials per round trip of a merge (7)

__device__ __forceinline__ void stage_part(const char* slot, int lane, char* dst) {
  __builtin_amdgcn_global_load_lds(static_cast<const void*>(slot + lane * 32), lds_ptr(dst), 16, 0, 0);
  __builtin_amdgcn_global_load_lds(static_cast<const void*>(slot + lane * 32 + 16), lds_ptr(dst + 1024), 16, 0, 0);
  __builtin_amdgcn_global_load_lds(static_cast<const void*>(slot + 2048 + 4 * (lane & 15)), lds_ptr(dst + 2048), 4, 0, 0);
}

// The staged partials [0, n) of one chunk, and the merging bin's own part last when
// `with_own`, combined into one: their max M first (all reads issued at once), then, in part
// order, each part's sum and O weighted by
// 2^(m log2(e) / 8 - M log2(e) / 8). One wave per SIMD issues a VALU instruction every 4
// cycles and waits out every LDS latency it does not overlap: this form costs about a third
// of a pairwise online fold.
__device__ __forceinline__ Part combine_staged(const char* stage, int n, int lane, const Part& own, bool with_own) {
  const int ml = 2048 + 32 * ((lane >> 4) & 1);
  float4_t mk[kStageParts];
#pragma unroll
  for (int i = 0; i < kStageParts; ++i) mk[i] = *reinterpret_cast<const float4_t*>(stage + min(i, n - 1) * kStageBytes + ml);
  float4_t mx = mk[0];
#pragma unroll
  for (int i = 1; i < kStageParts; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx[r] = fmaxf(mx[r], mk[i][r]);
  if (with_own) {
#pragma unroll
    for (int r = 0; r < 4; ++r) mx[r] = fmaxf(mx[r], own.m[r]);
  }
  Part c;
  float neg[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    c.m[r] = mx[r];
    c.l[r] = 0.f;
    c.o[0][r] = 0.f;
    c.o[1][r] = 0.f;
    neg[r] = -mx[r] * kScoreToLog2;
  }
  // Two parts per iteration (the second one's weight is 0 past the chunk): their eight LDS
  // reads share one latency.
#pragma nounroll
  for (int i = 0; i < n; i += 2) {
    const char* p0 = stage + i * kStageBytes;
    const char* p1 = stage + min(i + 1, n - 1) * kStageBytes;
    const float4_t a0 = *reinterpret_cast<const float4_t*>(p0 + lane * 16);
    const float4_t b0 = *reinterpret_cast<const float4_t*>(p0 + 1024 + lane * 16);
    const float4_t m0 = *reinterpret_cast<const float4_t*>(p0 + ml);
    const float4_t l0 = *reinterpret_cast<const float4_t*>(p0 + ml + 16);
    const float4_t a1 = *reinterpret_cast<const float4_t*>(p1 + lane * 16);
    const float4_t b1 = *reinterpret_cast<const float4_t*>(p1 + 1024 + lane * 16);
    const float4_t m1 = *reinterpret_cast<const float4_t*>(p1 + ml);
    const float4_t l1 = *reinterpret_cast<const float4_t*>(p1 + ml + 16);
    const bool second = i + 1 < n;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float s0 = exp2_fast(fmaf(m0[r], kScoreToLog2, neg[r]));
      const float s1 = second ? exp2_fast(fmaf(m1[r], kScoreToLog2, neg[r])) : 0.f;
      c.l[r] = fmaf(l1[r], s1, fmaf(l0[r], s0, c.l[r]));
      c.o[0][r] = fmaf(a1[r], s1, fmaf(a0[r], s0, c.o[0][r]));
      c.o[1][r] = fmaf(b1[r], s1, fmaf(b0[r], s0, c.o[1][r]));
    }
  }
  if (with_own) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float s = exp2_fast(fmaf(own.m[r], kScoreToLog2, neg[r]));
      c.l[r] = fmaf(own.l[r], s, c.l[r]);
      c.o[0][r] = fmaf(own.o[0][r], s, c.o[0][r]);
      c.o[1][r] = fmaf(own.o[1][r], s, c.o[1][r]);
    }
  }
  return c;
}

// Workspace slot of part k of a cut sequence whose parts start at slot `first` (the plan
// numbers the parts of all cut sequences densely; the last part has no slot). `slots` is
// the workspace past its header.
__device__ __forceinline__ char* part_slot(char* slots, int first, int k, int h) {
  return slots + ((static_cast<int64_t>(first) + k) * kKVHeads + h) * kSlotBytes;
}

// Scalar parameters in an order whose leading ones (plan, query, pool, num_blocks, layer)
// the compiler preloads into SGPRs at wave launch.
//
// APPEND: the newest token of each sequence (position length - 1), given as new_key and
// new_value [batch][4][64], is written into the pool row its block table gives. The bin
// holding the sequence's last block stages the row in LDS with the Q DMAs, and once that
// block's DMA has landed copies the row into its ring slot (so this pass already reads it)
// and stores it to the pool.
//
// Faults. A merge that gives up waiting (PC_ATTN_FAULT_MERGE_TIMEOUT), a part flag raised
// on another XCD (PC_ATTN_FAULT_FOREIGN_XCD) and a block id outside the pool
// (PC_ATTN_FAULT_BLOCK_ID) turn the affected rows into NaN and are ORed into the
// workspace's fault word by one lane's vector atomic. The kernel never clears the word.
template <bool APPEND>
__global__ __launch_bounds__(kBinThreads) void paged_decode_bin_kernel(const int32_t* plan, const _Float16* query,
                                                                      _Float16* pool, int64_t num_blocks,
                                                                      int layer, int batch, int nslots, _Float16* out,
                                                                      char* workspace, const _Float16* new_key,
                                                                      const _Float16* new_value) {
  __shared__ __attribute__((aligned(16))) char lds[kKVHeads * kWaveLds];
  const int h = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = lane & 15, g = lane >> 4;
  const int32_t* row = plan + static_cast<int64_t>(blockIdx.x) * kRowInts;
  char* const slots = workspace + kWorkspaceHeader;

  // The record (scalar loads) and the bin's block ids (lane L of vector k holds id 64 k + L)
  // in one round trip: the id addresses do not depend on the record.
  int32_t rec[kRecordInts];
#pragma unroll
  for (int i = 0; i < kRecordInts; ++i) rec[i] = row[i];
  int32_t idv[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) idv[k] = row[kRecordInts + 64 * k + lane];
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" : "+v"(idv[0]), "+v"(idv[1]), "+v"(idv[2]), "+v"(idv[3]) :: "memory");
  const int nseg = rec[0], nunits = rec[1];
  if (nseg <= 0 || nseg > kMaxSegs || nunits <= 0 || nunits > kMaxUnits) return;  // padding rows do nothing
  // This call's flag values (the plan's epoch and the layer; the XCD id is added where a flag
  // is raised), held in a VGPR: the stream loop needs every SGPR it has.
  int key;
  asm volatile("v_mov_b32 %0, %1" : "=v"(key) : "s"(flag_key(rec[2], layer)));

  char* wl = lds + h * kWaveLds;
  char* ring = wl;
  char* qarea = wl + kRing * kUnitBytes;
  char* oarea = qarea + kMaxSegs * 1024;
  const int64_t kind_elems = num_blocks * kBlockElems;
  const _Float16* lbase = pool + static_cast<int64_t>(layer) * 2 * kind_elems + h * kHeadDim;

  // Q of every segment into its LDS area: lane L loads q head L / 8, 16 B chunk
  // (L % 8) ^ (L / 8). A sequence index outside the batch reads row 0 (its rows are never
  // written).
#pragma unroll
  for (int s = 0; s < kMaxSegs; ++s) {
    if (s < nseg) {
      int b = rec[kHeaderInts + s * kSegInts];
      b = (b < 0 || b >= batch) ? 0 : b;
      const int qh = lane >> 3, pos = lane & 7;
      const _Float16* src = query + (static_cast<int64_t>(b) * kQHeads + kGroup * h + qh) * kHeadDim + 8 * (pos ^ qh);
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src), lds_ptr(qarea + s * 1024), 16, 0, 0);
    }
  }
  // APPEND: the new K row (lane L < 8: 16 B chunk L) and V row (lanes 8-15: chunk L - 8) of
  // this wave's kv head into the segment's output area (unused until the segment ends);
  // lanes 16-63 repeat lanes 0-15. Issued before the ring, so the first ring wait covers them.
  if constexpr (APPEND) {
#pragma unroll
    for (int s = 0; s < kMaxSegs; ++s) {
      if (s < nseg) {
        int b = rec[kHeaderInts + s * kSegInts];
        b = (b < 0 || b >= batch) ? 0 : b;
        const _Float16* src = (c < 8 ? new_key : new_value) + (static_cast<int64_t>(b) * kKVHeads + h) * kHeadDim + 8 * (c & 7);
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(src), lds_ptr(oarea + s * 1024), 16, 0, 0);
      }
    }
  }
  auto block_id = [&](int u) -> uint32_t {
    const int32_t v = u < 64 ? idv[0] : u < 128 ? idv[1] : u < 192 ? idv[2] : idv[3];
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(v, u & 63));
  };
  // K DMA: lane L -> row L / 8 (+ 8), position L % 8 holds chunk (L % 8) ^ (row & 7).
  const int kr = lane >> 3, kp = lane & 7;
  const int koffA = kr * kRowElems + 8 * (kp ^ kr), koffB = (kr + 8) * kRowElems + 8 * (kp ^ kr);
  // V DMA: lane L -> row L / 8 (+ 8), the chunk stored at position L % 8.
  const int voffA = kr * kRowElems + 8 * (2 * ((kp >> 1) ^ row_sel(kr)) + (kp & 1));
  const int voffB = (kr + 8) * kRowElems + 8 * (2 * ((kp >> 1) ^ row_sel(kr + 8)) + (kp & 1));
  auto issue = [&](int u) {
    uint32_t id = block_id(u);
    if (id >= static_cast<uint64_t>(num_blocks)) id = 0;  // never dereferenced out of the pool
    const _Float16* kb = lbase + static_cast<int64_t>(id) * kBlockElems;
    const _Float16* vb = kb + kind_elems;
    char* dst = ring + (u & (kRing - 1)) * kUnitBytes;
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(kb + koffA), lds_ptr(dst), 16, 0, kStreamAux);
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(kb + koffB), lds_ptr(dst + 1024), 16, 0, kStreamAux);
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(vb + voffA), lds_ptr(dst + 2048), 16, 0, kStreamAux);
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(vb + voffB), lds_ptr(dst + 3072), 16, 0, kStreamAux);
  };
  int issued = 0;
  for (; issued < kRing && issued < nunits; ++issued) issue(issued);

  // K reads: lane (c, g) takes row c, chunks g and 4 + g; Q reads the same chunks of row c % 8.
  const uint32_t kaddr0 = c * 128 + ((g ^ (c & 7)) * 16), kaddr1 = c * 128 + (((4 + g) ^ (c & 7)) * 16);
  const uint32_t qaddr0 = (c & 7) * 128 + ((g ^ (c & 7)) * 16), qaddr1 = (c & 7) * 128 + (((4 + g) ^ (c & 7)) * 16);
  // Transposing reads: lane (c, g) supplies row 4g + c/4, 8 B piece c % 4 of a dim group.
  const int rr = 4 * g + (c >> 2);
  const uint32_t tsel = row_sel(rr);
  const uint32_t ring_base = lds_offset(ring);

  Part first_part, last_part;  // partials of segment 0 and of the last segment (cut sequences)
  int patch_u = -1;  // APPEND: the segment's unit holding the new token, or -1
  int seg = -1, seg_end = 0, len = 0, j0 = 0, nblk = 0, nspan = 1;
  half8_t qa, qb;
  float m = 0.f, mc = 0.f, lsum = 0.f;
  float4_t acc[4];
  bool bad = false, first_block = true;

  auto finish_segment = [&]() {
    Part p;
    const float l = sum_over_groups(lsum);
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int q = 0; q < 4; ++q) p.o[k][q] = bad ? NAN : fold_low_rows(acc[2 * k][q], acc[2 * k + 1][q]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      p.m[q] = lane_value_of_half(m, q, (g & 1) != 0);
      p.l[q] = lane_value_of_half(l, q, (g & 1) != 0);
    }
    if (nspan == 1) {
      wave_lds_fence();
      put_output(oarea + seg * 1024, lane, p);
    } else {
      if (seg == 0) first_part = p;
      if (seg == nseg - 1) last_part = p;
    }
  };

  for (int u = 0; u < nunits; ++u) {
    if (u == seg_end) {
      if (seg >= 0) finish_segment();
      if (++seg >= nseg) break;  // malformed record: blocks beyond the segments are not processed
      len = seg == 0 ? rec[9] : seg == 1 ? rec[17] : seg == 2 ? rec[25] : rec[33];
      j0 = seg == 0 ? rec[10] : seg == 1 ? rec[18] : seg == 2 ? rec[26] : rec[34];
      nblk = seg == 0 ? rec[11] : seg == 1 ? rec[19] : seg == 2 ? rec[27] : rec[35];
      nspan = seg == 0 ? rec[14] : seg == 1 ? rec[22] : seg == 2 ? rec[30] : rec[38];
      seg_end = u + max(nblk, 1);
      if constexpr (APPEND) {
        const int sb = seg == 0 ? rec[8] : seg == 1 ? rec[16] : seg == 2 ? rec[24] : rec[32];
        const bool ends = nblk > 0 && len > 0 && j0 + nblk == blocks_of(len) && sb >= 0 && sb < batch;
        patch_u = ends ? seg_end - 1 : -1;
      }
      bad = false;
      first_block = true;
      lsum = 0.f;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) acc[nt] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
    wait_ring(issued - u - 1);  // also covers the Q DMAs, issued before every unit
    if constexpr (APPEND) {
      if (u == patch_u) {
        // The block holding the new token has landed: its staged row replaces the pool's
        // (stale) row in the ring slot (K chunk c at c ^ (r & 7), V chunk c at
        // 2 ((c / 2) ^ row_sel(r)) + c % 2 of row r) and goes to the pool, K by lanes 0-7, V
        // by lanes 8-15. LDS accesses as assembly, so the compiler adds no wait for the ring's
        // DMAs still in flight; the one store only lengthens later ring waits (loads return
        // in order, so an extra count never lets a wait end early).
        const int r = (len - 1) % kSlots, ch = c & 7;
        const int pos = c < 8 ? (ch ^ (r & 7)) : 128 + 2 * ((ch >> 1) ^ row_sel(r)) + (ch & 1);
        half8_t v;
        asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                     : "=v"(v)
                     : "v"(lds_offset(oarea + seg * 1024 + c * 16))
                     : "memory");
        // The id is read with every lane active: block_id selects its vector per lane, and
        // readlane of a lane outside a branch's exec mask would see a stale register.
        const uint32_t id = block_id(u);
        if (lane < 16) {
          asm volatile("ds_write_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                       :
                       : "v"(ring_base + (u & (kRing - 1)) * kUnitBytes + r * 128 + pos * 16), "v"(v)
                       : "memory");
          if (id < static_cast<uint64_t>(num_blocks)) {
            *reinterpret_cast<half8_t*>(pool + ((static_cast<int64_t>(layer) * 2 + (c >> 3)) * num_blocks + id) *
                                                   kBlockElems + r * kRowElems + h * kHeadDim + 8 * ch) = v;
          }
        }
      }
    }
    if (first_block) {
      const uint32_t qbase = lds_offset(qarea + seg * 1024);
      asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                   : "=&v"(qa), "=&v"(qb)
                   : "v"(qbase + qaddr0), "v"(qbase + qaddr1)
                   : "memory");
    }
    if (block_id(u) >= static_cast<uint64_t>(num_blocks)) bad = true;
    const uint32_t slot = ring_base + (u & (kRing - 1)) * kUnitBytes;
    half8_t k0v, k1v;
    short4_t v0, v1, v2, v3;
    {
      const uint32_t vbase = slot + rr * 128 + 8 * (c & 3);
      asm volatile(
          "ds_read_b128 %0, %6\n\t"
          "ds_read_b128 %1, %7\n\t"
          "ds_read_b64_tr_b16 %2, %8 offset:2048\n\t"
          "ds_read_b64_tr_b16 %3, %9 offset:2048\n\t"
          "ds_read_b64_tr_b16 %4, %10 offset:2048\n\t"
          "ds_read_b64_tr_b16 %5, %11 offset:2048\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(k0v), "=&v"(k1v), "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3)
          : "v"(slot + kaddr0), "v"(slot + kaddr1), "v"(vbase + 32 * (0 ^ tsel)), "v"(vbase + 32 * (1 ^ tsel)),
            "v"(vbase + 32 * (2 ^ tsel)), "v"(vbase + 32 * (3 ^ tsel))
          : "memory");
    }
    // The slot's LDS reads are complete: refill it with the unit kRing ahead.
    if (issued < nunits) {
      issue(issued);
      ++issued;
    }
    float4_t sv = {0.f, 0.f, 0.f, 0.f};
    sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0v, qa, sv, 0, 0, 0);
    sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1v, qb, sv, 0, 0, 0);
    const int valid = len - (j0 + (u - (seg_end - nblk))) * kSlots;
    float sc[4] = {sv[0], sv[1], sv[2], sv[3]};
    if (valid < kSlots) {
#pragma unroll
      for (int q = 0; q < 4; ++q) sc[q] = 4 * g + q < valid ? sc[q] : -INFINITY;
    }
    const float bm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    if (first_block) {
      m = max_over_groups(bm);  // finite: token 0 of a segment's first block is valid
      mc = m * kScoreToLog2;
      first_block = false;
    } else if (__builtin_amdgcn_ballot_w64(bm * kScoreToLog2 > mc + kLazyLog2) != 0) {
      const float mn = fmaxf(m, max_over_groups(bm));
      const float alpha = exp2_fast((m - mn) * kScoreToLog2);
      lsum *= alpha;
      float al[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) al[q] = lane_value_of_half(alpha, q, (g & 1) != 0);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[nt][q] *= al[q];
      m = mn;
      mc = m * kScoreToLog2;
    }
    float p[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) p[q] = exp2_fast(fmaf(sc[q], kScoreToLog2, -mc));
    lsum += (p[0] + p[1]) + (p[2] + p[3]);
    // A operand: row c holds p of q head c % 8 for tokens 4g..4g+3: the fp16 rounding of p
    // for c < 8, the exact remainder scaled by 2^18 for c >= 8.
    half4_t pa;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float hi = static_cast<float>(static_cast<_Float16>(p[q]));
      pa[q] = static_cast<_Float16>(c < kGroup ? p[q] : (p[q] - hi) * kLowScale);
    }
    if (valid < kSlots) {
      // lane (c, g) holds V of tokens 4g..4g+3: zero the ones past the context
      const int keep = valid - 4 * g;
      const uint32_t mlo = (keep > 0 ? 0xFFFFu : 0u) | (keep > 1 ? 0xFFFF0000u : 0u);
      const uint32_t mhi = (keep > 2 ? 0xFFFFu : 0u) | (keep > 3 ? 0xFFFF0000u : 0u);
      uint2_t x;
      x = __builtin_bit_cast(uint2_t, v0); x[0] &= mlo; x[1] &= mhi; v0 = __builtin_bit_cast(short4_t, x);
      x = __builtin_bit_cast(uint2_t, v1); x[0] &= mlo; x[1] &= mhi; v1 = __builtin_bit_cast(short4_t, x);
      x = __builtin_bit_cast(uint2_t, v2); x[0] &= mlo; x[1] &= mhi; v2 = __builtin_bit_cast(short4_t, x);
      x = __builtin_bit_cast(uint2_t, v3); x[0] &= mlo; x[1] &= mhi; v3 = __builtin_bit_cast(short4_t, x);
    }
    acc[0] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4_t, v0), acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4_t, v1), acc[1], 0, 0, 0);
    acc[2] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4_t, v2), acc[2], 0, 0, 0);
    acc[3] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4_t, v3), acc[3], 0, 0, 0);
  }
  if (seg < nseg) finish_segment();
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // every DMA has landed (also after a malformed record)
  const bool complete = seg == nseg - 1 && seg_end == nunits;  // the record's segments cover its blocks

  // Segment fields of the first and the last segment.
  const int b0 = rec[8], k00 = rec[12], kidx0 = rec[13], nspan0 = rec[14], slot0 = rec[15];
  const int sl = nseg - 1;
  const int kidxl = sl == 0 ? rec[13] : sl == 1 ? rec[21] : sl == 2 ? rec[29] : rec[37];
  const int nspanl = sl == 0 ? rec[14] : sl == 1 ? rec[22] : sl == 2 ? rec[30] : rec[38];
  const int slotl = sl == 0 ? rec[15] : sl == 1 ? rec[23] : sl == 2 ? rec[31] : rec[39];
  // The span's slots [first, first + parts - 1) lie in the workspace.
  auto slots_ok = [&](int first, int parts) { return first >= 0 && parts >= 2 && first + static_cast<int64_t>(parts) - 1 <= nslots; };

  // A part that is not the last of its span: store it, wait for the acknowledgement, then
  // raise the part's flag.
  if (complete && nspanl > 1 && kidxl < nspanl - 1 && kidxl >= 0 && slots_ok(slotl, nspanl)) {
    char* slot = part_slot(slots, slotl, kidxl, h);
    store_part(slot, lane, last_part);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane == 0) {
      __hip_atomic_store(reinterpret_cast<int32_t*>(slot + kFlagOffset), key | (xcc_id() + 1), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // Sequences complete within the bin: their fp16 rows from LDS (before the merge, which
  // stages partials over the whole wave area).
  wave_lds_fence();
#pragma unroll
  for (int s = 0; s < kMaxSegs; ++s) {
    const int sb = rec[kHeaderInts + s * kSegInts];
    if (complete && s < nseg && rec[kHeaderInts + s * kSegInts + 6] == 1 && sb >= 0 && sb < batch) {
      *reinterpret_cast<uint4*>(out + (static_cast<int64_t>(sb) * kQHeads + kGroup * h) * kHeadDim + lane * 8) =
          *reinterpret_cast<const uint4*>(oarea + s * 1024 + lane * 16);
    }
  }
  // The last part of a cut sequence: wait for the other parts' flags, fold them in span
  // order and this bin's part last, lower the flags, write the rows. This code stays small
  // and its loops rolled: it runs once per merge, cold in the instruction cache, where every
  // 64-byte line fetched costs an L2 round trip.
  // A block id outside the pool anywhere in the bin (lane L of vector k holds id 64 k + L).
  bool any_bad = false;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    any_bad |= __builtin_amdgcn_ballot_w64(64 * k + lane < nunits && static_cast<uint32_t>(idv[k]) >= num_blocks) != 0;
  }
  int fault = any_bad ? PC_ATTN_FAULT_BLOCK_ID : 0;
  if (complete && nspan0 > 1 && kidx0 == nspan0 - 1 && slots_ok(slot0, nspan0) &&
      k00 + static_cast<int64_t>(kGroups) * kidx0 == static_cast<int64_t>(blockIdx.x) && k00 >= 0) {
    const int want = key | (xcc_id() + 1);
    const int nparts = nspan0 - 1;  // parts 0 .. nspan0 - 2 are in the workspace
    bool timeout = false, foreign = false;
    Part acc_p;
    if (nparts <= kStageParts) {
      // One chunk: lane k polls part k's flag (lanes past the span repeat the last part's),
      // and every part whose flag is up is staged right away, by DMA into its LDS slot
      // (the wave's area is free after the stream), while the others are still awaited.
      const int32_t* flag =
          reinterpret_cast<const int32_t*>(part_slot(slots, slot0, min(lane, nparts - 1), h) + kFlagOffset);
      uint64_t pending = (nparts == 64 ? ~0ull : (1ull << nparts) - 1);
      int spins = 0;
#pragma nounroll
      while (pending != 0) {
        const int f = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool raised = flag_of_call(f, key);
        // raised on another XCD: its partial is not visible here
        if (__builtin_amdgcn_ballot_w64(lane < nparts && raised && f != want) != 0) foreign = true;
        uint64_t ready = __builtin_amdgcn_ballot_w64(raised) & pending;
        if (ready == 0) {
          if (++spins >= kMaxSpins) {  // never raised: the rows become NaN
            timeout = true;
            break;
          }
          __builtin_amdgcn_s_sleep(2);
          continue;
        }
        pending &= ~ready;
#pragma nounroll
        while (ready != 0) {
          const int k = __builtin_ctzll(ready);
          ready &= ready - 1;
          stage_part(part_slot(slots, slot0, k, h), lane, wl + k * kStageBytes);
        }
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      acc_p = combine_staged(wl, nparts, lane, first_part, true);
    } else {
      // Longer spans: the flags, 64 per load, until all are raised; then the partials,
      // kStageParts per round trip, each chunk combined and folded in span order, and the
      // own part last.
      for (int base = 0; base < nparts; base += 64) {
        const int32_t* flag =
            reinterpret_cast<const int32_t*>(part_slot(slots, slot0, min(base + lane, nparts - 1), h) + kFlagOffset);
        int f = 0;
#pragma nounroll
        for (int spins = 0; spins < kMaxSpins; ++spins) {
          f = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (__builtin_amdgcn_ballot_w64(!flag_of_call(f, key)) == 0) break;
          __builtin_amdgcn_s_sleep(2);
        }
        if (__builtin_amdgcn_ballot_w64(!flag_of_call(f, key)) != 0) timeout = true;
        if (__builtin_amdgcn_ballot_w64(flag_of_call(f, key) && f != want) != 0) foreign = true;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc_p.m[r] = -INFINITY;
        acc_p.l[r] = 0.f;
        acc_p.o[0][r] = 0.f;
        acc_p.o[1][r] = 0.f;
      }
      for (int c0 = 0; c0 < nparts; c0 += kStageParts) {
        const int cn = min(kStageParts, nparts - c0);
#pragma nounroll
        for (int i = 0; i < cn; ++i) stage_part(part_slot(slots, slot0, c0 + i, h), lane, wl + i * kStageBytes);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        fold_part(acc_p, combine_staged(wl, cn, lane, first_part, false));
        wave_lds_fence();  // the chunk's LDS reads are done before the next chunk's DMA
      }
      fold_part(acc_p, first_part);
    }
    if (timeout || foreign) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc_p.o[0][r] = NAN;
        acc_p.o[1][r] = NAN;
      }
      fault |= (timeout ? PC_ATTN_FAULT_MERGE_TIMEOUT : 0) | (foreign ? PC_ATTN_FAULT_FOREIGN_XCD : 0);
    }
    for (int k = lane; k < nspan0 - 1; k += 64) {
      __hip_atomic_store(reinterpret_cast<int32_t*>(part_slot(slots, slot0, k, h) + kFlagOffset), 0, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    if (b0 >= 0 && b0 < batch) {
      // Straight from registers (16 lanes per 32-byte run of a row): no LDS round trip.
      put_output(reinterpret_cast<char*>(out + (static_cast<int64_t>(b0) * kQHeads + kGroup * h) * kHeadDim), lane,
                 acc_p);
    }
  }
  // `fault` is uniform over the wave; one lane ORs it into the fault word.
  if (fault != 0 && lane == 0) {
    __hip_atomic_fetch_or(reinterpret_cast<int32_t*>(workspace), fault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------------------
// Host-side validation, plan and workspace layout.
// ---------------------------------------------------------------------------------------

int check_attn_shape(int32_t batch, int32_t max_blocks) {
  if (batch < 0 || batch > (1 << 20)) return set_error(PC_ERR_ARGUMENT, "batch %d out of range", batch);
  if (max_blocks < 1 || max_blocks > (1 << 16)) {
    return set_error(PC_ERR_ARGUMENT, "max_blocks %d out of range [1, 65536]", max_blocks);
  }
  return PC_OK;
}

// Bins of one group the planner may create for a batch of `batch` sequences of at most
// `max_blocks` blocks: the nominal cut (at most the whole target, or one bin per kMaxUnits
// blocks when that is more), plus one early close per kMaxSegs - 1 complete sequences (a bin
// closed at kMaxSegs segments holds at least that many), plus one.
int64_t group_bins_bound(int32_t batch, int32_t max_blocks) {
  const int64_t total = static_cast<int64_t>(batch) * max_blocks;
  const int64_t nominal = std::max<int64_t>(kTargetBins, (total + kMaxUnits - 1) / kMaxUnits);
  return nominal + 1 + (batch + kMaxSegs - 2) / (kMaxSegs - 1) + 1;
}

// Plan rows (workgroups) that always suffice for the shape.
int64_t plan_rows_bound(int32_t batch, int32_t max_blocks) {
  return static_cast<int64_t>(kGroups) * group_bins_bound(batch, max_blocks);
}

// Partial slots that always suffice: one per bin at most (a bin ends at most one cut part
// that is not a sequence's last). The bins over all groups number at most the target plus
// one per kMaxUnits blocks plus rounding (kGroups x 1.5), plus the early closes.
int64_t slots_bound(int32_t batch, int32_t max_blocks) {
  const int64_t total = static_cast<int64_t>(batch) * max_blocks;
  return kTargetBins + (total + kMaxUnits - 1) / kMaxUnits + 2 * kGroups + (batch + kMaxSegs - 2) / (kMaxSegs - 1);
}

// The header (fault word), then the partial slots.
int64_t workspace_bytes_for(int64_t slots) { return kWorkspaceHeader + slots * kKVHeads * kSlotBytes; }

// Split-K scratch of pc_paged_decode_attn_noalloc: a file-scope device array, one copy per
// GPU, held until the process ends. Host code never passes `scratch` itself to a kernel (in
// host code the name is a stand-in, not a device address); it uses the address
// hipGetSymbolAddress returns for the device, looked up once per device. Its contents start
// at zero (part flags must) and every call leaves them so.
constexpr int64_t kNoAllocScratchBytes = PC_ATTN_NOALLOC_SCRATCH_BYTES;
static_assert(kNoAllocScratchBytes % 256 == 0, "the scratch keeps the workspace's 256-byte alignment");
__device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on `device` (which must be current), or null with the error
// recorded.
void* scratch_address(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr) {
      set_error(PC_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", device, hipGetErrorString(err));
      return nullptr;
    }
    g_scratch_ptr[device] = ptr;
  }
  return g_scratch_ptr[device];
}

// Argument checks and the launch of pc_paged_decode_attn (APPEND false) and
// pc_kv_append_paged_decode_attn (APPEND true, new_key and new_value checked by the caller).
template <bool APPEND>
int launch_decode_attn(void* out, const void* query, void* pool, int64_t num_blocks, int32_t layer,
                       const int32_t* context_lens, int32_t batch, int32_t max_blocks, const int32_t* plan,
                       int32_t num_records, const void* new_key, const void* new_value, void* workspace,
                       void* stream) {
  if (!out || !query || !pool || !context_lens || !plan) return set_error(PC_ERR_ARGUMENT, "null pointer");
  if (!workspace) return set_error(PC_ERR_ARGUMENT, "workspace required (null pointer)");
  if (num_blocks < 1 || num_blocks > INT32_MAX) return set_error(PC_ERR_ARGUMENT, "num_blocks out of range");
  if (layer < 0 || layer >= kLayers) return set_error(PC_ERR_ARGUMENT, "layer %d outside [0, 22)", layer);
  if (int rc = check_attn_shape(batch, max_blocks)) return rc;
  if (!aligned(query, 16) || !aligned(out, 16) || !aligned(pool, 16) || !aligned(workspace, 256) ||
      !aligned(plan, 16) || !aligned(context_lens, 4)) {
    return set_error(PC_ERR_ARGUMENT, "query/out/pool/plan must be 16-byte, workspace 256-byte aligned");
  }
  if (num_records < 0 || num_records > plan_rows_bound(batch, max_blocks)) {
    return set_error(PC_ERR_ARGUMENT, "num_records %d outside [0, pc_attn_plan_capacity]", num_records);
  }
  const int64_t nslots = slots_bound(batch, max_blocks);
  if (batch == 0 || num_records == 0) return ok();
  hipStream_t s = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  hipLaunchKernelGGL(paged_decode_bin_kernel<APPEND>, dim3(static_cast<unsigned>(num_records)), dim3(kBinThreads), 0, s,
                     plan, static_cast<const _Float16*>(query), static_cast<_Float16*>(pool), num_blocks, layer, batch,
                     static_cast<int>(nslots), static_cast<_Float16*>(out), static_cast<char*>(workspace),
                     static_cast<const _Float16*>(new_key), static_cast<const _Float16*>(new_value));
  return check_launch(APPEND ? "kv_append_paged_decode_bin" : "paged_decode_bin");
}

// Plan epochs: every plan gets the next nonzero 22-bit value, stamped into each of its rows
// (header int 2). Part flags carry it, so a flag raised under another plan is never taken
// for this plan's.
std::atomic<uint32_t> g_plan_epoch{0};

uint32_t next_plan_epoch() {
  uint32_t e;
  do {
    e = (g_plan_epoch.fetch_add(1, std::memory_order_relaxed) + 1) & kEpochMask;
  } while (e == 0);
  return e;
}

// One bin while it is being cut: its segments {sequence, first block, blocks}.
struct BinSegs {
  int32_t seg[kMaxSegs][3];
  int nseg = 0;
  int blocks = 0;
};

}  // namespace

extern "C" {

int pc_abi_version(void) { return kAbiVersion; }

const char* pc_last_error(void) { return pc_internal::last_error(); }

int32_t pc_attn_plan_record_ints(void) { return kRowInts; }

int64_t pc_attn_plan_capacity(int32_t batch, int32_t max_blocks) {
  if (check_attn_shape(batch, max_blocks) != PC_OK) return -1;
  return plan_rows_bound(batch, max_blocks);
}

int64_t pc_attn_workspace_bytes(int32_t batch, int32_t max_blocks) {
  if (check_attn_shape(batch, max_blocks) != PC_OK) return 0;
  return workspace_bytes_for(slots_bound(batch, max_blocks));
}

int32_t pc_attn_plan(const int32_t* context_lens, const int32_t* block_tables, int32_t batch, int32_t max_blocks,
                     int32_t* plan, int64_t capacity) {
  if (int rc = check_attn_shape(batch, max_blocks)) return -rc;
  if (batch > 0 && (!context_lens || !block_tables || !plan)) return -set_error(PC_ERR_ARGUMENT, "null pointer");
  std::vector<int32_t> order;
  order.reserve(batch);
  int64_t total = 0;
  for (int32_t b = 0; b < batch; ++b) {
    if (context_lens[b] > static_cast<int64_t>(max_blocks) * kSlots) {
      return -set_error(PC_ERR_ARGUMENT, "context length %d of sequence %d exceeds its %d-block table", context_lens[b], b,
                        max_blocks);
    }
    if (context_lens[b] > 0) {
      order.push_back(b);
      total += blocks_of(context_lens[b]);
    }
  }
  if (total == 0) return (ok(), 0);
  // Sequences, longest first, go to the group with the fewest blocks so far.
  std::stable_sort(order.begin(), order.end(),
                   [&](int32_t x, int32_t y) { return blocks_of(context_lens[x]) > blocks_of(context_lens[y]); });
  std::vector<std::vector<int32_t>> members(kGroups);
  std::vector<int64_t> load(kGroups, 0);
  for (int32_t b : order) {
    const int x = static_cast<int>(std::min_element(load.begin(), load.end()) - load.begin());
    members[x].push_back(b);
    load[x] += blocks_of(context_lens[b]);
  }
  // Bins over the whole batch: one per CU, fewer for small workloads, more when a bin would
  // exceed kMaxUnits blocks; each group gets its share, cut at equal block counts.
  const int64_t target = std::max<int64_t>(std::min<int64_t>(kTargetBins, std::max<int64_t>(1, total / kMinBinBlocks)),
                                           (total + kMaxUnits - 1) / kMaxUnits);
  std::vector<std::vector<BinSegs>> bins(kGroups);
  for (int x = 0; x < kGroups; ++x) {
    if (load[x] == 0) continue;
    int64_t nb = (target * load[x] + total / 2) / total;
    nb = std::max<int64_t>(nb, (load[x] + kMaxUnits - 1) / kMaxUnits);
    nb = std::max<int64_t>(1, std::min<int64_t>(nb, load[x]));
    // Each bin takes the group's remaining blocks over its remaining bins (at most
    // kMaxUnits); a bin also closes when it holds kMaxSegs segments and the next block starts
    // another sequence. A bin that starts with the last part of a cut sequence merges that
    // sequence's earlier parts after its own stream (about a third of a block's stream time
    // per part, measured), so it takes (parts + 3) / 4 blocks fewer and the other bins share
    // them.
    std::vector<BinSegs>& out = bins[x];
    auto bin_end = [&](int64_t pos, int32_t seq_blocks, int32_t done, int32_t parts) {
      const int64_t left = std::max<int64_t>(1, nb - static_cast<int64_t>(out.size()));
      int64_t cap = (load[x] - pos + left - 1) / left;
      if (done > 0 && seq_blocks - done <= cap) cap = std::max<int64_t>(seq_blocks - done, cap - (parts + 3) / 4);
      return pos + std::min<int64_t>(std::max<int64_t>(cap, 1), kMaxUnits);
    };
    BinSegs cur;
    int64_t pos = 0, end = -1;
    for (int32_t b : members[x]) {
      const int32_t n = blocks_of(context_lens[b]);
      int32_t j = 0, parts = 0;
      if (end < 0) end = bin_end(0, n, 0, 0);
      while (j < n) {
        if (cur.blocks > 0 && (pos == end || cur.nseg == kMaxSegs)) {
          out.push_back(cur);
          cur = BinSegs();
          end = bin_end(pos, n, j, parts);
        }
        const int32_t take = static_cast<int32_t>(std::min<int64_t>(n - j, end - pos));
        cur.seg[cur.nseg][0] = b;
        cur.seg[cur.nseg][1] = j;
        cur.seg[cur.nseg][2] = take;
        ++cur.nseg;
        ++parts;
        cur.blocks += take;
        j += take;
        pos += take;
      }
    }
    if (cur.blocks > 0) out.push_back(cur);
  }
  size_t most = 0;
  for (const auto& v : bins) most = std::max(most, v.size());
  const int64_t rows = static_cast<int64_t>(most) * kGroups;
  if (rows > capacity || rows > INT32_MAX) {
    return -set_error(PC_ERR_ARGUMENT, "plan capacity %lld too small (%lld rows)", static_cast<long long>(capacity),
                      static_cast<long long>(rows));
  }
  // Each sequence's bins (rows), in order, and the first slot of each cut sequence.
  std::vector<int32_t> first_row(batch, -1), nspan(batch, 0), first_slot(batch, -1);
  for (int x = 0; x < kGroups; ++x) {
    for (size_t i = 0; i < bins[x].size(); ++i) {
      const BinSegs& bs = bins[x][i];
      for (int s = 0; s < bs.nseg; ++s) {
        const int32_t b = bs.seg[s][0];
        if (first_row[b] < 0) first_row[b] = static_cast<int32_t>(x + kGroups * i);
        ++nspan[b];
      }
    }
  }
  int64_t slots = 0;
  for (int32_t b = 0; b < batch; ++b) {
    if (nspan[b] > 1) {
      first_slot[b] = static_cast<int32_t>(slots);
      slots += nspan[b] - 1;
    }
  }
  if (slots > slots_bound(batch, max_blocks)) {
    return -set_error(PC_ERR_ARGUMENT, "plan needs %lld partial slots, above the workspace's %lld",
                      static_cast<long long>(slots), static_cast<long long>(slots_bound(batch, max_blocks)));
  }
  std::fill(plan, plan + rows * kRowInts, 0);
  const int32_t epoch = static_cast<int32_t>(next_plan_epoch());
  for (int x = 0; x < kGroups; ++x) {
    for (size_t i = 0; i < bins[x].size(); ++i) {
      const BinSegs& bs = bins[x][i];
      const int32_t r = static_cast<int32_t>(x + kGroups * i);
      int32_t* row = plan + static_cast<int64_t>(r) * kRowInts;
      row[0] = bs.nseg;
      row[1] = bs.blocks;
      row[2] = epoch;
      int u = 0;
      for (int s = 0; s < bs.nseg; ++s) {
        const int32_t b = bs.seg[s][0], j0 = bs.seg[s][1], n = bs.seg[s][2];
        int32_t* seg = row + kHeaderInts + s * kSegInts;
        seg[0] = b;
        seg[1] = context_lens[b];
        seg[2] = j0;
        seg[3] = n;
        seg[4] = first_row[b];
        seg[5] = (r - first_row[b]) / kGroups;
        seg[6] = nspan[b];
        seg[7] = first_slot[b];
        const int32_t* table = block_tables + static_cast<int64_t>(b) * max_blocks;
        for (int32_t j = 0; j < n; ++j) row[kRecordInts + u++] = table[j0 + j];
      }
    }
  }
  ok();
  return static_cast<int32_t>(rows);
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
                   vl % 16 == 0 && vt % 16 == 0 && kt >= INT32_MIN && kt <= INT32_MAX && vt >= INT32_MIN &&
                   vt <= INT32_MAX;
  if (vec) {
    const uint64_t chunks = rows * kRowChunks;
    const uint64_t per_block = kAppendThreads * kAppendChunksPerThread;
    const unsigned grid = static_cast<unsigned>((chunks + per_block - 1) / per_block);
    hipLaunchKernelGGL(kv_append_vec_kernel, dim3(grid), dim3(kAppendThreads), 0, s, static_cast<const char*>(key),
                       static_cast<const char*>(value), slot_mapping, kl, vl, static_cast<int32_t>(kt),
                       static_cast<int32_t>(vt), static_cast<uint32_t>(num_tokens), static_cast<uint32_t>(rows),
                       static_cast<uint4*>(pool), num_blocks * kSlots, layer_begin);
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

int pc_paged_decode_attn(void* out, const void* query, const void* pool, int64_t num_blocks, int32_t layer,
                         const int32_t* context_lens, int32_t batch, int32_t max_blocks, const int32_t* plan,
                         int32_t num_records, void* workspace, void* stream) {
  return launch_decode_attn<false>(out, query, const_cast<void*>(pool), num_blocks, layer, context_lens, batch,
                                   max_blocks, plan, num_records, nullptr, nullptr, workspace, stream);
}

int pc_kv_append_paged_decode_attn(void* out, const void* query, void* pool, int64_t num_blocks, int32_t layer,
                                   const int32_t* context_lens, int32_t batch, int32_t max_blocks,
                                   const int32_t* plan, int32_t num_records, const void* new_key,
                                   const void* new_value, void* workspace, void* stream) {
  if (!new_key || !new_value) return set_error(PC_ERR_ARGUMENT, "null pointer");
  if (!aligned(new_key, 16) || !aligned(new_value, 16)) {
    return set_error(PC_ERR_ARGUMENT, "new_key/new_value must be 16-byte aligned");
  }
  return launch_decode_attn<true>(out, query, pool, num_blocks, layer, context_lens, batch, max_blocks, plan,
                                  num_records, new_key, new_value, workspace, stream);
}

int pc_paged_decode_attn_noalloc(void* out, const void* query, const void* pool, int64_t num_blocks, int32_t layer,
                                 const int32_t* context_lens, int32_t batch, int32_t max_blocks, const int32_t* plan,
                                 int32_t num_records, void* stream) {
  // The size check comes first: a call beyond the scratch is refused before any HIP call.
  if (int rc = check_attn_shape(batch, max_blocks)) return rc;
  const int64_t need = workspace_bytes_for(slots_bound(batch, max_blocks));
  if (need > kNoAllocScratchBytes) {
    return set_error(PC_ERR_ARGUMENT,
                     "batch %d with %d-block tables needs %lld bytes of split-K scratch; the allocation-free entry "
                     "point holds %lld (use pc_paged_decode_attn with a workspace)",
                     batch, max_blocks, static_cast<long long>(need), static_cast<long long>(kNoAllocScratchBytes));
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  int device = -1, current = -1;
  if (hipStreamGetDevice(s, &device) != hipSuccess || hipGetDevice(&current) != hipSuccess) {
    return set_error(PC_ERR_LAUNCH, "cannot determine the stream's device");
  }
  if (device != current) {
    return set_error(PC_ERR_ARGUMENT, "stream is on device %d but device %d is current", device, current);
  }
  if (device < 0 || device >= kMaxDevices) return set_error(PC_ERR_ARGUMENT, "device %d out of range", device);
  void* workspace = scratch_address(device);
  if (!workspace) return PC_ERR_LAUNCH;
  return pc_paged_decode_attn(out, query, pool, num_blocks, layer, context_lens, batch, max_blocks, plan, num_records,
                              workspace, stream);
}

}  // extern "C"
