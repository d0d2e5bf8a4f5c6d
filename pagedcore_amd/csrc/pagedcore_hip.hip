// Paged KV-cache hot path for MI355X (gfx950): KV append, paged decode attention over split-K
// work items, and the merge of the items' partials. Exposed through the C ABI declared in
// include/pagedcore_hip.h. No device memory is allocated here; every buffer comes from the
// caller.
//
// Pool layout (fixed by the reference allocator, src/pagedcore/kv_cache.py:39-43):
//   fp16 [22 layers][2 kinds][num_blocks][16 slots][4 kv heads][64 dims]
// One (layer, kind, block) is 8 KiB contiguous; one (block, kv head) is 16 rows of 128 B
// at a 512 B stride.

#include <hip/hip_runtime.h>

#include <algorithm>
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

constexpr int kAbiVersion = 10;
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
// Paged decode attention.
//
// Work split. A work item is 9 consecutive blocks of one sequence (the last item of a
// sequence may hold fewer) and runs as one workgroup of 12 waves: wave w serves kv head
// h = w % 4 for sub-chunk s = w / 4, i.e. blocks [9 item + 3 s, 9 item + 3 s + 3). Every
// load of a wave is issued before its first block is processed:
//   * Q of the head's 8 query heads (1 KiB, from L2 after the first item of the sequence);
//   * K, per block 16 rows x 128 B: lane (c = lane % 16, g = lane / 16) loads row c, dims
//     8g..8g+7 and 32+8g..39+8g -- the A operand of v_mfma_f32_16x16x32_f16 -- into VGPRs;
//   * V, per block 16 rows x 128 B, straight into the wave's LDS area by LDS DMA
//     (global_load_lds_dwordx4), each 32 B dim group of row r stored at group position
//     u ^ sel(r) so that the transposing reads below are free of bank conflicts.
// K and V are read once per pass, so both use the non-temporal cache policy (the pool's
// planes are far larger than the caches). A CU holds two such workgroups (72 KiB of LDS and
// 77 VGPRs each), so a 64-sequence decode batch is in flight in one round.
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
// The three sub-chunk waves of a head then merge through LDS: each leaves (max, sum,
// unnormalized O) in its area and takes an LDS ticket; the last one folds them in
// sub-chunk order. A sequence that is one item writes its fp16 output directly; otherwise
// the item's partial goes to the workspace and paged_decode_merge_kernel folds the items of
// each (sequence, kv head) in item order.
// ---------------------------------------------------------------------------------------


constexpr int kSubBlocks = 3;                              // blocks per wave
constexpr int kSubs = 3;                                   // sub-chunk waves per kv head
constexpr int kItemBlocks = kSubBlocks * kSubs;            // 9 blocks per work item
constexpr int kItemWaves = kKVHeads * kSubs;               // 12 waves per workgroup
constexpr int kItemThreads = 64 * kItemWaves;
constexpr int kHeadBlockBytes = kSlots * kHeadDim * 2;     // one kv head of one block: 2 KiB
constexpr int kAreaBytes = kSubBlocks * kHeadBlockBytes;   // LDS per wave: 6 KiB
constexpr int kPlanInts = 16;                              // {seq, item, len, items, 9 ids, 3 x 0}
constexpr int kPlanBins = 8;                               // XCDs of an MI355X
constexpr int kPartFloats = kGroup * kHeadDim + 2 * kGroup;  // item partial: O [8][64], (m, l) x 8
constexpr int kMergeThreads = 256;
constexpr int kMergeItems = 16;                            // items per merge round trip
// Scale of the low (remainder) part of p in the PV product (2^18).
constexpr float kLowScale = 262144.0f;
// Headroom (log2 of p) before the running max is raised.
constexpr float kLazyLog2 = 8.0f;

struct AttnArgs {
  _Float16* out;
  const _Float16* query;
  const _Float16* pool;
  int64_t num_blocks;
  const int32_t* plan;
  const int32_t* context_lens;
  float* partials;  // [batch][4 kv heads][max_items][kPartFloats]
  int layer, batch, max_blocks, max_items;
};

// Blocks holding `len` tokens, without the int32 overflow of len + 15.
__device__ __host__ __forceinline__ int blocks_of(int len) { return len / kSlots + (len % kSlots != 0); }

__device__ __forceinline__ int items_of(int len, int max_blocks) {
  return len > 0 ? (min(blocks_of(len), max_blocks) + kItemBlocks - 1) / kItemBlocks : 0;
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


// Every load of the wave has returned. The K registers are named so that none of them is
// reused while a load of an unused block slot could still land in it.
__device__ __forceinline__ void wait_all_loads(half8_t (&k0)[kSubBlocks], half8_t (&k1)[kSubBlocks]) {
  asm volatile("s_waitcnt vmcnt(0)"
               : "+v"(k0[0]), "+v"(k1[0]), "+v"(k0[1]), "+v"(k1[1]), "+v"(k0[2]), "+v"(k1[2])
               :
               : "memory");
}

__device__ __forceinline__ float lane_value(float x, int k) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), k));
}

// x of lane q (hi false) or of lane 4 + q (hi true). Both lanes are read in uniform control
// flow and each lane then selects one: a readlane written inside the two arms of a per-lane
// condition compiles to exec-masked branches around each read (about 0.3 us of the tail).
__device__ __forceinline__ float lane_value_of_half(float x, int q, bool hi) {
  const float lo_value = lane_value(x, q);
  const float hi_value = lane_value(x, 4 + q);
  return hi ? hi_value : lo_value;
}

// Online-softmax state of the 4 q heads a lane holds in the PV layout (q head 4(g&1) + r,
// dims 16(2k + g/2) + c), with the fold of one more partial. Explicit fmaf: every fold
// rounds the same way wherever it runs. The state starts as the first partial itself, which
// is what folding that partial into the empty state (m = -inf, l = 0, O = 0) gives for any
// partial with a finite m: scales exp2(-inf) = 0 and exp2(0) = 1, and fmaf(x, 1, 0) = x.
struct Fold {
  float M[4], L[4], O[2][4];
  __device__ __forceinline__ void set(const float (&m)[4], const float (&l)[4], const float (&x)[2][4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      M[r] = m[r];
      L[r] = l[r];
      O[0][r] = x[0][r];
      O[1][r] = x[1][r];
    }
  }
  __device__ __forceinline__ void add(const float (&m)[4], const float (&l)[4], const float (&x)[2][4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float mn = fmaxf(M[r], m[r]);
      const float so = exp2_fast((M[r] - mn) * kScoreToLog2);
      const float sn = exp2_fast((m[r] - mn) * kScoreToLog2);
      L[r] = fmaf(l[r], sn, L[r] * so);
      O[0][r] = fmaf(x[0][r], sn, O[0][r] * so);
      O[1][r] = fmaf(x[1][r], sn, O[1][r] * so);
      M[r] = mn;
    }
  }
};

// A sub-chunk partial in its wave's LDS area: lane L's 8 O values at [L][8] floats (value
// (k, r) at 4k + r), then (m, l) of q head j at byte 2048 + 8j.
__device__ __forceinline__ void put_sub(char* area, int lane, int g, const float (&x)[2][4], const float (&m)[4],
                                        const float (&l)[4]) {
  *reinterpret_cast<float4_t*>(area + lane * 32) = float4_t{x[0][0], x[0][1], x[0][2], x[0][3]};
  *reinterpret_cast<float4_t*>(area + lane * 32 + 16) = float4_t{x[1][0], x[1][1], x[1][2], x[1][3]};
  if (lane == 0 || lane == 16) {
    *reinterpret_cast<float4_t*>(area + 2048 + (g & 1) * 32) = float4_t{m[0], l[0], m[1], l[1]};
    *reinterpret_cast<float4_t*>(area + 2048 + (g & 1) * 32 + 16) = float4_t{m[2], l[2], m[3], l[3]};
  }
}

__device__ __forceinline__ void get_sub(const char* area, int lane, int g, float (&x)[2][4], float (&m)[4], float (&l)[4]) {
  const float4_t x0 = *reinterpret_cast<const float4_t*>(area + lane * 32);
  const float4_t x1 = *reinterpret_cast<const float4_t*>(area + lane * 32 + 16);
  const float4_t y0 = *reinterpret_cast<const float4_t*>(area + 2048 + (g & 1) * 32);
  const float4_t y1 = *reinterpret_cast<const float4_t*>(area + 2048 + (g & 1) * 32 + 16);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    x[0][r] = x0[r];
    x[1][r] = x1[r];
  }
  m[0] = y0[0]; l[0] = y0[1]; m[1] = y0[2]; l[1] = y0[3];
  m[2] = y1[0]; l[2] = y1[1]; m[3] = y1[2]; l[3] = y1[3];
}

// PV-layout values to natural order [8 q heads][64] through `area`: the fp16 output rows
// (scaled by inv[r]) or the fp32 item partial; each lane then stores 16 or 32 contiguous bytes.
template <bool kHalf>
__device__ __forceinline__ void store_natural(void* dst, char* area, int lane, const float (&x)[2][4], const float (&inv)[4]) {
  const int c = lane & 15, g = lane >> 4;
  wave_lds_fence();
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int idx = (4 * (g & 1) + r) * kHeadDim + 16 * (2 * k + (g >> 1)) + c;
      if constexpr (kHalf) {
        reinterpret_cast<_Float16*>(area)[idx] = static_cast<_Float16>(x[k][r] * inv[r]);
      } else {
        reinterpret_cast<float*>(area)[idx] = x[k][r];
      }
    }
  wave_lds_fence();
  char* d = static_cast<char*>(dst);
  if constexpr (kHalf) {
    *reinterpret_cast<uint4*>(d + lane * 16) = *reinterpret_cast<const uint4*>(area + lane * 16);
  } else {
    *reinterpret_cast<uint4*>(d + lane * 32) = *reinterpret_cast<const uint4*>(area + lane * 32);
    *reinterpret_cast<uint4*>(d + lane * 32 + 16) = *reinterpret_cast<const uint4*>(area + lane * 32 + 16);
  }
}

__global__ __launch_bounds__(kItemThreads) __attribute__((amdgpu_waves_per_eu(6, 8))) void paged_decode_item_kernel(
    const int32_t* plan, const _Float16* query, const _Float16* pool, int64_t num_blocks, int layer, int batch,
    int max_blocks, int max_items, _Float16* out, float* partials) {
  // Scalar parameters, those the first loads need leading: the compiler preloads the leading
  // ones into SGPRs at wave launch (no kernel-argument round trip before the plan record).
  AttnArgs a;
  a.out = out;
  a.query = query;
  a.pool = pool;
  a.num_blocks = num_blocks;
  a.plan = plan;
  a.context_lens = nullptr;
  a.partials = partials;
  a.layer = layer;
  a.batch = batch;
  a.max_blocks = max_blocks;
  a.max_items = max_items;
  __shared__ __attribute__((aligned(16))) char lds[kItemWaves * kAreaBytes];
  __shared__ int32_t sub_tickets[kKVHeads];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = w & 3;
  const int s = w >> 2;
  const int lane = threadIdx.x & 63;
  const int c = lane & 15;
  const int g = lane >> 4;

  // The whole plan record in one round trip; this wave's block ids are selected from it.
  // The empty asm makes every word (and every kernel argument the loads below need) an
  // input before the first branch: otherwise those loads sink below the early exits, and
  // each becomes one more dependent round trip, queued behind the K/V loads of the
  // workgroups already running (microseconds each).
  const int32_t* rec = a.plan + static_cast<int64_t>(blockIdx.x) * kPlanInts;
  int32_t r[kPlanInts];
#pragma unroll
  for (int i = 0; i < kPlanInts; ++i) r[i] = rec[i];
  asm volatile("" ::"s"(r[0]), "s"(r[1]), "s"(r[2]), "s"(r[4]), "s"(r[5]), "s"(r[6]), "s"(r[7]), "s"(r[8]), "s"(r[9]),
               "s"(r[10]), "s"(r[11]), "s"(r[12]), "s"(a.batch), "s"(a.max_blocks), "s"(a.max_items), "s"(a.pool),
               "s"(a.query), "s"(a.num_blocks), "s"(a.layer));
  const int b = r[0];
  const int item = r[1];
  const int len = r[2];
  // Padding records (b < 0) and records that do not fit the call's shapes do nothing: the
  // whole workgroup leaves before the barrier.
  if (b < 0 || b >= a.batch || item < 0 || item >= items_of(len, a.max_blocks) || item >= a.max_items) return;
  const int nitems = items_of(len, a.max_blocks);
  int32_t ids[kSubBlocks];
#pragma unroll
  for (int t = 0; t < kSubBlocks; ++t) ids[t] = s == 0 ? r[4 + t] : (s == 1 ? r[4 + kSubBlocks + t] : r[4 + 2 * kSubBlocks + t]);
  const int nblk = min(blocks_of(len), a.max_blocks);
  const int count = min(kItemBlocks, nblk - item * kItemBlocks);  // blocks of this item, >= 1
  const int nsub = (count + kSubBlocks - 1) / kSubBlocks;
  const int first = item * kItemBlocks + s * kSubBlocks;          // first block of this wave
  const int mine = min(kSubBlocks, count - s * kSubBlocks);       // its blocks (if s < nsub)
  char* area = lds + (h * kSubs + s) * kAreaBytes;

  // The LDS tickets are zeroed before any wave can take one. The waves of a workgroup start
  // together, and the record is in registers first, so no load waits behind this barrier.
  if (w == 0 && lane < kKVHeads) sub_tickets[lane] = 0;
  asm volatile("" ::"s"(item), "s"(len), "s"(ids[0]), "s"(ids[1]), "s"(ids[2]));
  __syncthreads();
  if (s >= nsub) return;

  half8_t qa, qb, k0[kSubBlocks], k1[kSubBlocks];
  bool bad = false;
  {
    const int64_t kind_elems = a.num_blocks * kBlockElems;
    const _Float16* qrow = a.query + (static_cast<int64_t>(b) * kQHeads + kGroup * h + (c & 7)) * kHeadDim + 8 * g;
    load_pair(qa, qb, qrow);
    const _Float16* lbase = a.pool + static_cast<int64_t>(a.layer) * 2 * kind_elems + h * kHeadDim;
    // LDS DMA slots: instruction 0 fills rows 0..7, instruction 1 rows 8..15; lane holds the
    // 16 B chunk stored at position lane % 8 of row lane / 8 (+ 8).
    const int qs = lane & 7;
    const int rA = lane >> 3, rB = rA + 8;
    const int offA = rA * kRowElems + 8 * (2 * ((qs >> 1) ^ row_sel(rA)) + (qs & 1));
    const int offB = rB * kRowElems + 8 * (2 * ((qs >> 1) ^ row_sel(rB)) + (qs & 1));
#pragma unroll
    for (int t = 0; t < kSubBlocks; ++t) {
      uint32_t id = static_cast<uint32_t>(ids[t]);
      if (id >= static_cast<uint64_t>(a.num_blocks)) {  // negative ids wrap to huge values
        if (t < mine) bad = true;
        id = 0;  // never dereferenced out of the pool
      }
      const _Float16* kb = lbase + static_cast<int64_t>(id) * kBlockElems;
      load_pair_stream(k0[t], k1[t], kb + c * kRowElems + 8 * g);
      const _Float16* vb = kb + kind_elems;
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(vb + offA), lds_ptr(area + t * kHeadBlockBytes), 16, 0,
                                       kStreamAux);
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(vb + offB), lds_ptr(area + t * kHeadBlockBytes + 1024), 16,
                                       0, kStreamAux);
      __builtin_amdgcn_sched_barrier(0);  // keep the issue order the waits below count on
    }
  }

  // Transposing reads: lane (c, g) supplies row 4g + c/4, 8 B piece c % 4 of a dim group.
  const int rr = 4 * g + (c >> 2);
  const uint32_t tbase = lds_offset(area) + rr * 128 + 8 * (c & 3);
  const uint32_t tsel = row_sel(rr);
  float m = 0.f, mc = 0.f, lsum = 0.f;
  float4_t acc[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) acc[nt] = float4_t{0.f, 0.f, 0.f, 0.f};

#define PC_PROCESS_BLOCK(I)                                                                                     \
  if (I < mine) {                                                                                               \
    wait_loads<4 * (kSubBlocks - 1 - I)>(k0[I], k1[I]);                                                          \
    if (I == 0) wait_loads<4 * (kSubBlocks - 1)>(qa, qb);                                                       \
    float4_t sv = {0.f, 0.f, 0.f, 0.f};                                                                          \
    sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0[I], qa, sv, 0, 0, 0);                                          \
    sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1[I], qb, sv, 0, 0, 0);                                          \
    const int valid = len - (first + I) * kSlots;                                                               \
    float sc[4] = {sv[0], sv[1], sv[2], sv[3]};                                                                 \
    if (valid < kSlots) {                                                                                       \
      _Pragma("unroll") for (int q = 0; q < 4; ++q) sc[q] = 4 * g + q < valid ? sc[q] : -INFINITY;              \
    }                                                                                                           \
    const float bm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));                                           \
    if (I == 0) {                                                                                               \
      m = max_over_groups(bm); /* finite: token 0 of a wave's first block is valid */                            \
      mc = m * kScoreToLog2;                                                                                    \
    } else if (__builtin_amdgcn_ballot_w64(bm * kScoreToLog2 > mc + kLazyLog2) != 0) {                         \
      const float mn = fmaxf(m, max_over_groups(bm));                                                           \
      const float alpha = exp2_fast((m - mn) * kScoreToLog2);                                                   \
      lsum *= alpha;                                                                                            \
      float al[4];                                                                                              \
      _Pragma("unroll") for (int q = 0; q < 4; ++q) al[q] = lane_value_of_half(alpha, q, (g & 1) != 0); \
      _Pragma("unroll") for (int nt = 0; nt < 4; ++nt) _Pragma("unroll") for (int q = 0; q < 4; ++q) acc[nt][q] *= al[q]; \
      m = mn;                                                                                                   \
      mc = m * kScoreToLog2;                                                                                    \
    }                                                                                                           \
    float p[4];                                                                                                 \
    _Pragma("unroll") for (int q = 0; q < 4; ++q) p[q] = exp2_fast(fmaf(sc[q], kScoreToLog2, -mc));             \
    lsum += (p[0] + p[1]) + (p[2] + p[3]);                                                                      \
    /* A operand: row c holds p of q head c % 8 for tokens 4g..4g+3: the fp16 rounding of */                    \
    /* p for c < 8, the exact remainder scaled by 2^18 for c >= 8 */                                             \
    half4_t pa;                                                                                                 \
    _Pragma("unroll") for (int q = 0; q < 4; ++q) {                                                             \
      const float hi = static_cast<float>(static_cast<_Float16>(p[q]));                                         \
      pa[q] = static_cast<_Float16>(c < kGroup ? p[q] : (p[q] - hi) * kLowScale);                               \
    }                                                                                                           \
    short4_t v0, v1, v2, v3;                                                                                    \
    read_v_tiles<I * kHeadBlockBytes>(tbase, tsel, v0, v1, v2, v3);                                             \
    if (valid < kSlots) {                                                                                       \
      /* lane (c, g) holds V of tokens 4g..4g+3: zero the ones past the context */                             \
      const int keep = valid - 4 * g;                                                                           \
      const uint32_t mlo = (keep > 0 ? 0xFFFFu : 0u) | (keep > 1 ? 0xFFFF0000u : 0u);                           \
      const uint32_t mhi = (keep > 2 ? 0xFFFFu : 0u) | (keep > 3 ? 0xFFFF0000u : 0u);                           \
      uint2_t u;                                                                                                \
      u = __builtin_bit_cast(uint2_t, v0); u[0] &= mlo; u[1] &= mhi; v0 = __builtin_bit_cast(short4_t, u);        \
      u = __builtin_bit_cast(uint2_t, v1); u[0] &= mlo; u[1] &= mhi; v1 = __builtin_bit_cast(short4_t, u);        \
      u = __builtin_bit_cast(uint2_t, v2); u[0] &= mlo; u[1] &= mhi; v2 = __builtin_bit_cast(short4_t, u);        \
      u = __builtin_bit_cast(uint2_t, v3); u[0] &= mlo; u[1] &= mhi; v3 = __builtin_bit_cast(short4_t, u);        \
    }                                                                                                           \
    acc[0] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4_t, v0), acc[0], 0, 0, 0);        \
    acc[1] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4_t, v1), acc[1], 0, 0, 0);        \
    acc[2] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4_t, v2), acc[2], 0, 0, 0);        \
    acc[3] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4_t, v3), acc[3], 0, 0, 0);        \
  }

  PC_PROCESS_BLOCK(0)
  PC_PROCESS_BLOCK(1)
  PC_PROCESS_BLOCK(2)
#undef PC_PROCESS_BLOCK
  static_assert(kSubBlocks == 3, "three PC_PROCESS_BLOCK expansions");
  wait_all_loads(k0, k1);

  // This wave's partial in the PV layout: (m, l) per q head and the folded O.
  const float l = sum_over_groups(lsum);
  float ox[2][4], om[4], ol[4];
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int q = 0; q < 4; ++q) ox[k][q] = bad ? NAN : fold_low_rows(acc[2 * k][q], acc[2 * k + 1][q]);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    om[q] = lane_value_of_half(m, q, (g & 1) != 0);
    ol[q] = lane_value_of_half(l, q, (g & 1) != 0);
  }

  Fold f;
  if (nsub > 1) {
    // Sub-chunk merge: every wave of kv head h leaves its partial in its own LDS area and
    // takes a ticket; the last one folds the head's sub-chunks in order.
    wave_lds_fence();
    put_sub(area, lane, g, ox, om, ol);
    int old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(&sub_tickets[h], 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old != nsub - 1) return;
    // Every sub-chunk's partial is read before the first fold (one LDS round trip; the
    // area of a sub-chunk past nsub is read and not folded).
    float px[kSubs][2][4], pm[kSubs][4], pl[kSubs][4];
#pragma unroll
    for (int s2 = 0; s2 < kSubs; ++s2) get_sub(lds + (h * kSubs + s2) * kAreaBytes, lane, g, px[s2], pm[s2], pl[s2]);
    f.set(pm[0], pl[0], px[0]);
#pragma unroll
    for (int s2 = 1; s2 < kSubs; ++s2) {
      if (s2 < nsub) f.add(pm[s2], pl[s2], px[s2]);
    }
  } else {
    f.set(om, ol, ox);
  }

  if (nitems == 1) {
    float inv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) inv[q] = 1.0f / f.L[q];
    store_natural<true>(a.out + (static_cast<int64_t>(b) * kQHeads + kGroup * h) * kHeadDim, area, lane, f.O, inv);
    return;
  }
  float* part = a.partials + ((static_cast<int64_t>(b) * kKVHeads + h) * a.max_items + item) * kPartFloats;
  store_natural<false>(part, area, lane, f.O, f.L);
  if (lane == 0 || lane == 16) {
    *reinterpret_cast<float4_t*>(part + 512 + (g & 1) * 8) = float4_t{f.M[0], f.L[0], f.M[1], f.L[1]};
    *reinterpret_cast<float4_t*>(part + 512 + (g & 1) * 8 + 4) = float4_t{f.M[2], f.L[2], f.M[3], f.L[3]};
  }
}

// Merge of multi-item sequences: one workgroup per (sequence, kv head); thread t owns dims
// 2(t % 32), +1 of q head t / 32 and folds the items' partials in item order, the loads of
// up to kMergeItems items issued at once.
__global__ __launch_bounds__(kMergeThreads) void paged_decode_merge_kernel(const int32_t* context_lens, int max_blocks,
                                                                         int max_items, const float* partials,
                                                                         _Float16* out) {
  AttnArgs a;
  a.out = out;
  a.context_lens = context_lens;
  a.partials = const_cast<float*>(partials);
  a.max_blocks = max_blocks;
  a.max_items = max_items;
  const int grp = blockIdx.x;
  const int b = grp / kKVHeads, h = grp % kKVHeads;
  const int t = threadIdx.x;
  const int qh = t >> 5;
  const int d = 2 * (t & 31);
  const int nitems = min(items_of(a.context_lens[b], a.max_blocks), a.max_items);
  if (nitems <= 1) return;
  const float* gpart = a.partials + static_cast<int64_t>(grp) * a.max_items * kPartFloats;
  float M = -INFINITY, L = 0.f, O0 = 0.f, O1 = 0.f;
#pragma unroll 1
  for (int i0 = 0; i0 < nitems; i0 += kMergeItems) {
    float2_t x[kMergeItems], ml[kMergeItems];
#pragma unroll
    for (int i = 0; i < kMergeItems; ++i) {
      const float* p = gpart + static_cast<int64_t>(min(i0 + i, nitems - 1)) * kPartFloats;  // clamped: in bounds
      x[i] = *reinterpret_cast<const float2_t*>(p + qh * kHeadDim + d);
      ml[i] = *reinterpret_cast<const float2_t*>(p + 512 + 2 * qh);
    }
#pragma unroll
    for (int i = 0; i < kMergeItems; ++i) {
      // Branch-free: a clamped duplicate gets weight 0 (m stays finite from the first item).
      const bool used = i0 + i < nitems;
      const float mp = used ? ml[i][0] : -INFINITY;
      const float lp = used ? ml[i][1] : 0.f;
      const float mn = fmaxf(M, mp);
      const float so = exp2_fast((M - mn) * kScoreToLog2);
      const float sn = exp2_fast((mp - mn) * kScoreToLog2);
      L = fmaf(lp, sn, L * so);
      O0 = fmaf(used ? x[i][0] : 0.f, sn, O0 * so);
      O1 = fmaf(used ? x[i][1] : 0.f, sn, O1 * so);
      M = mn;
    }
  }
  const float inv = 1.0f / L;
  *reinterpret_cast<half2_t*>(a.out + (static_cast<int64_t>(b) * kQHeads + kGroup * h + qh) * kHeadDim + d) =
      half2_t{static_cast<_Float16>(O0 * inv), static_cast<_Float16>(O1 * inv)};
}

// ---------------------------------------------------------------------------------------
// Host-side validation, plan and workspace layout.
// ---------------------------------------------------------------------------------------

int64_t items_per_sequence(int32_t max_blocks) { return (static_cast<int64_t>(max_blocks) + kItemBlocks - 1) / kItemBlocks; }

int check_attn_shape(int32_t batch, int32_t max_blocks) {
  if (batch < 0 || batch > (1 << 20)) return set_error(PC_ERR_ARGUMENT, "batch %d out of range", batch);
  if (max_blocks < 1 || max_blocks > (1 << 16)) {
    return set_error(PC_ERR_ARGUMENT, "max_blocks %d out of range [1, 65536]", max_blocks);
  }
  if ((static_cast<int64_t>(batch) + kPlanBins) * items_per_sequence(max_blocks) > INT32_MAX) {
    return set_error(PC_ERR_ARGUMENT, "attention grid too large");
  }
  return PC_OK;
}

// Split-K scratch of pc_paged_decode_attn_noalloc: a file-scope device array, one copy per
// GPU, held until the process ends. Host code never passes `scratch` itself to a kernel (in
// host code the name is a stand-in, not a device address); it uses the address
// hipGetSymbolAddress returns for the device, looked up once per device.
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

}  // namespace

extern "C" {

int pc_abi_version(void) { return kAbiVersion; }

const char* pc_last_error(void) { return pc_internal::last_error(); }

int32_t pc_attn_plan_record_ints(void) { return kPlanInts; }

int64_t pc_attn_plan_capacity(int32_t batch, int32_t max_blocks) {
  if (check_attn_shape(batch, max_blocks) != PC_OK) return -1;
  // Greedy binning leaves no bin more than one sequence's items above the average.
  return (static_cast<int64_t>(batch) + kPlanBins) * items_per_sequence(max_blocks);
}

int64_t pc_attn_workspace_bytes(int32_t batch, int32_t max_blocks) {
  if (check_attn_shape(batch, max_blocks) != PC_OK) return 0;
  return static_cast<int64_t>(batch) * kKVHeads * items_per_sequence(max_blocks) * kPartFloats * 4;
}

int32_t pc_attn_plan(const int32_t* context_lens, const int32_t* block_tables, int32_t batch, int32_t max_blocks,
                     int32_t* plan, int64_t capacity) {
  if (int rc = check_attn_shape(batch, max_blocks)) return -rc;
  if (batch > 0 && (!context_lens || !block_tables || !plan)) return -set_error(PC_ERR_ARGUMENT, "null pointer");
  // Sequences, longest first, go to the bin (XCD) with the fewest items so far; work item k
  // of bin x becomes record k * kPlanBins + x, and the hardware dispatches workgroup i to XCD
  // (i + start) % 8, so the items of one sequence share an XCD and its L2. Bins shorter than
  // the longest are padded with empty records.
  std::vector<int32_t> order;
  order.reserve(batch);
  for (int32_t b = 0; b < batch; ++b) {
    if (context_lens[b] > static_cast<int64_t>(max_blocks) * kSlots) {
      return -set_error(PC_ERR_ARGUMENT, "context length %d of sequence %d exceeds its %d-block table", context_lens[b], b,
                        max_blocks);
    }
    if (context_lens[b] > 0) order.push_back(b);
  }
  std::stable_sort(order.begin(), order.end(), [&](int32_t x, int32_t y) { return context_lens[x] > context_lens[y]; });
  std::vector<std::vector<int32_t>> bins(kPlanBins);
  std::vector<int64_t> load(kPlanBins, 0);
  for (int32_t b : order) {
    const int32_t len = context_lens[b];
    const int32_t nblk = blocks_of(len);  // <= max_blocks, checked above
    const int32_t nitems = (nblk + kItemBlocks - 1) / kItemBlocks;
    const int bin = static_cast<int>(std::min_element(load.begin(), load.end()) - load.begin());
    load[bin] += nitems;
    const int32_t* row = block_tables + static_cast<int64_t>(b) * max_blocks;
    for (int32_t item = 0; item < nitems; ++item) {
      int32_t rec[kPlanInts] = {b, item, len, nitems};
      for (int i = 0; i < kItemBlocks; ++i) rec[4 + i] = row[std::min(item * kItemBlocks + i, nblk - 1)];
      bins[bin].insert(bins[bin].end(), rec, rec + kPlanInts);
    }
  }
  int64_t most = 0;
  for (const auto& v : bins) most = std::max<int64_t>(most, static_cast<int64_t>(v.size()) / kPlanInts);
  const int64_t total = most * kPlanBins;
  if (total > capacity) {
    return -set_error(PC_ERR_ARGUMENT, "plan capacity %lld too small (%lld records)", static_cast<long long>(capacity),
                      static_cast<long long>(total));
  }
  for (int64_t pos = 0; pos < most; ++pos) {
    for (int x = 0; x < kPlanBins; ++x) {
      int32_t* dst = plan + (pos * kPlanBins + x) * kPlanInts;
      if (pos < static_cast<int64_t>(bins[x].size()) / kPlanInts) {
        std::copy(bins[x].begin() + pos * kPlanInts, bins[x].begin() + (pos + 1) * kPlanInts, dst);
      } else {
        std::fill(dst, dst + kPlanInts, 0);
        dst[0] = -1;
      }
    }
  }
  ok();
  return static_cast<int32_t>(total);
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
  if (!out || !query || !pool || !context_lens || !plan) return set_error(PC_ERR_ARGUMENT, "null pointer");
  if (num_blocks < 1 || num_blocks > INT32_MAX) return set_error(PC_ERR_ARGUMENT, "num_blocks out of range");
  if (layer < 0 || layer >= kLayers) return set_error(PC_ERR_ARGUMENT, "layer %d outside [0, 22)", layer);
  if (int rc = check_attn_shape(batch, max_blocks)) return rc;
  const int64_t max_items = items_per_sequence(max_blocks);
  if (max_items > 1 && !workspace) return set_error(PC_ERR_ARGUMENT, "workspace required");
  if (!aligned(query, 16) || !aligned(out, 16) || !aligned(pool, 16) || !aligned(workspace, 256) ||
      !aligned(plan, 16) || !aligned(context_lens, 4)) {
    return set_error(PC_ERR_ARGUMENT, "query/out/pool/plan must be 16-byte, workspace 256-byte aligned");
  }
  if (num_records < 0 || num_records > (static_cast<int64_t>(batch) + kPlanBins) * max_items) {
    return set_error(PC_ERR_ARGUMENT, "num_records %d outside [0, (batch + 8) * items per sequence]", num_records);
  }
  if (batch == 0 || num_records == 0) return ok();
  AttnArgs a;
  a.out = static_cast<_Float16*>(out);
  a.query = static_cast<const _Float16*>(query);
  a.pool = static_cast<const _Float16*>(pool);
  a.num_blocks = num_blocks;
  a.plan = plan;
  a.context_lens = context_lens;
  a.partials = static_cast<float*>(workspace);
  a.layer = layer;
  a.batch = batch;
  a.max_blocks = max_blocks;
  a.max_items = static_cast<int>(max_items);
  hipStream_t s = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  hipLaunchKernelGGL(paged_decode_item_kernel, dim3(static_cast<unsigned>(num_records)), dim3(kItemThreads), 0, s, a.plan,
                     a.query, a.pool, a.num_blocks, a.layer, a.batch, a.max_blocks, a.max_items, a.out, a.partials);
  if (int rc = check_launch("paged_decode_item")) return rc;
  if (max_items > 1) {
    hipLaunchKernelGGL(paged_decode_merge_kernel, dim3(static_cast<unsigned>(batch) * kKVHeads), dim3(kMergeThreads), 0,
                       s, a.context_lens, a.max_blocks, a.max_items, static_cast<const float*>(a.partials), a.out);
    return check_launch("paged_decode_merge");
  }
  return PC_OK;
}

int pc_paged_decode_attn_noalloc(void* out, const void* query, const void* pool, int64_t num_blocks, int32_t layer,
                                 const int32_t* context_lens, int32_t batch, int32_t max_blocks, const int32_t* plan,
                                 int32_t num_records, void* stream) {
  // The size check comes first: a call beyond the scratch is refused before any HIP call.
  if (int rc = check_attn_shape(batch, max_blocks)) return rc;
  const int64_t need = static_cast<int64_t>(batch) * kKVHeads * items_per_sequence(max_blocks) * kPartFloats * 4;
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
