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

constexpr int kAbiVersion = 5;
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
// One wave per (sequence b, kv head h, partition p); the partition's blocks are walked in
// order with the next block's loads in flight. Nothing is shared between waves, so there
// is no barrier and LDS holds only the p exchange (1.25 KiB per wave). Per 16-token block:
//   * QK on the matrix core: S^T[16 tokens][16] = K[16][64] . Q^T[64][16] with two
//     v_mfma_f32_16x16x32_f16 (q heads 8..15 are zero padding). K fragments come straight
//     from HBM with 16 B loads, rows = tokens; fp16 x fp16 products are exact in fp32.
//     Lane (c = lane % 16, g = lane / 16) receives the scores of q head c for tokens
//     4g..4g+3.
//   * online softmax in fp32 in the raw-dot domain (m = max q.k); p = 2^((dot - m) * C)
//     with C = log2(e)/8, so the 1/8 scale is applied after the exact difference. The
//     block max of each q head is taken over the 4 token groups with two permlane swaps,
//     so all groups share one running max, and that max only moves when a block beats it
//     by more than 2^8 (so rescales are rare and p <= 256).
//   * p goes through LDS to the PV layout; PV is fp32 FMA on the VALU with fp16 V
//     operands (v_fma_mix). Lane (c, g) owns dims 4c..4c+3 of all 8 q heads for tokens
//     4g..4g+3 (8 B V loads; one load instruction covers 4 rows of 128 B).
// At the end the 4 token groups are summed in registers by a permlane reduce-scatter, and
// each lane holds one dim of every q head. A single-partition sequence writes fp16 output
// directly. Otherwise the partial (m, l, o) goes to the workspace and the last wave of the
// (sequence, head) to finish -- found with an atomic ticket -- merges all partitions, so
// split-K needs no second launch (a separate reduce kernel is kept behind
// PC_ATTN_SEPARATE_REDUCE).
// ---------------------------------------------------------------------------------------

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef short short4_t __attribute__((ext_vector_type(4)));

constexpr int kAttnThreads = 64;   // one wave per (sequence, kv head, partition)
constexpr int kMergeThreads = 64;  // separate merge kernel: one wave per (sequence, kv head)
constexpr int kDefaultPartitionBlocks = 16;
constexpr int kRing = 4;  // K/V blocks per wave whose loads are in flight together
constexpr int kMaxPartitionBlocks = 64;  // one block id per lane
constexpr int kVRowBytes = 136;  // LDS row of staged V: 64 fp16 dims + 8 B pad (spreads banks)
constexpr int kMergeBatch = 8;   // partitions whose partials one merge round trip loads
// log2(e) / sqrt(64): turns a raw q.k difference into a base-2 exponent.
constexpr float kScoreToLog2 = 0.18033688011112042f;
// Lazy-rescale threshold in raw-dot units (2^8 in probability terms).
constexpr float kRescaleDot = 8.0f / kScoreToLog2;
// Scale of the low (remainder) part of p in the PV product (2^18).
constexpr float kLowScale = 262144.0f;

struct BlockFrag {
  half8_t k0, k1;  // K[token c][dims 8g..8g+7] and [32+8g..32+8g+7]
  half4_t v[4];    // V[token 4g+j][dims 4c..4c+3]
};

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float lane_value(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

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

// Reduce-scatter over the wave halves: lanes < 32 get x[l] + x[l + 32], lanes >= 32 get
// y[l - 32] + y[l].
__device__ __forceinline__ float add_swap32(float x, float y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

struct WaveState {
  float m_run;      // running max of raw q.k, q head c % 8 (the same in every lane of that head)
  float l_part;     // sum of p over this lane's 4 tokens of every block, q head c % 8
  float4_t acc[4];  // PV tiles: acc[nt][r] = sum over tokens of A[row 4g + r] * V[dim 16nt + c],
                    // rows 0..7 from the fp16 roundings of p, rows 8..15 from the scaled remainders
};

struct BlockSource {
  const _Float16* kpool;  // K plane of the layer
  const _Float16* vpool;  // V plane of the layer
  uint32_t num_blocks;
  int kofs, vofs;  // lane offsets inside a block
};

// Loads one block's K/V fragments. `ids` holds the partition's block ids, one per lane;
// `i` is wave-uniform, so the id lands in an SGPR and the block base is scalar
// arithmetic. Returns 1 if the block id is out of range (the fragments then come from
// block 0 so that no access leaves the pool).
__device__ __forceinline__ int load_block(BlockFrag& f, const BlockSource& src, int ids, int i) {
  uint32_t phys = static_cast<uint32_t>(__builtin_amdgcn_readlane(ids, i));
  int bad = 0;
  if (phys >= src.num_blocks) {  // negative ids wrap to huge values
    bad = 1;
    phys = 0;
  }
  const _Float16* kblk = src.kpool + static_cast<int64_t>(phys) * kBlockElems;
  const _Float16* vblk = src.vpool + static_cast<int64_t>(phys) * kBlockElems;
  f.k0 = *reinterpret_cast<const half8_t*>(kblk + src.kofs);
  f.k1 = *reinterpret_cast<const half8_t*>(kblk + src.kofs + 32);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f.v[j] = *reinterpret_cast<const half4_t*>(vblk + src.vofs + j * kRowElems);
  }
  return bad;
}

// Value of head-indexed lane data for rows 4(g & 1) + r (r = 0..3) of this lane.
__device__ __forceinline__ float row_head_value(float x, int r, int g) {
  return (g & 1) ? lane_value(x, 4 + r) : lane_value(x, r);
}

// One block: S = K Q^T on MFMA (lanes c and c + 8 compute the same q head), online
// softmax, then O += P V on MFMA with P split into its fp16 rounding (rows 0..7) and the
// scaled remainder (rows 8..15), so that the product keeps fp32 accuracy and range. V
// reaches the MFMA B layout through LDS: row-major stores, transposing reads.
__device__ __forceinline__ void process_block(WaveState& st, const BlockFrag& f, half8_t qa,
                                              half8_t qb, int valid, int c, int g,
                                              char* __restrict__ vlds) {
  float4_t s = {0.f, 0.f, 0.f, 0.f};
  s = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.k0, qa, s, 0, 0, 0);
  s = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.k1, qb, s, 0, 0, 0);
  // s[r] = q[head c % 8] . k[token 4g + r]
  float sc[4] = {s[0], s[1], s[2], s[3]};
  half4_t v[4] = {f.v[0], f.v[1], f.v[2], f.v[3]};
  if (valid < kSlots) {  // last, partial block: masked slots never enter a product
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (4 * g + r >= valid) {
        sc[r] = -INFINITY;
        v[r] = half4_t{};
      }
    }
  }
  // V rows to LDS early: the stores overlap the softmax arithmetic.
#pragma unroll
  for (int j = 0; j < 4; ++j) *reinterpret_cast<half4_t*>(vlds + (4 * g + j) * kVRowBytes + 8 * c) = v[j];

  // Block max over all 16 tokens (finite: every block has a valid token).
  const float mblk = max_over_groups(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
  if (__any(mblk > st.m_run + kRescaleDot)) {
    const float m_new = fmaxf(st.m_run, mblk);
    const float alpha = exp2_fast((st.m_run - m_new) * kScoreToLog2);  // 0 when m_run = -inf
    st.l_part *= alpha;
    st.m_run = m_new;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float a = row_head_value(alpha, r, g);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) st.acc[nt][r] *= a;
    }
  }
  float p[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    p[r] = (sc[r] == -INFINITY) ? 0.f : exp2_fast((sc[r] - st.m_run) * kScoreToLog2);
  }
  st.l_part += (p[0] + p[1]) + (p[2] + p[3]);
  // A operand: row c holds p of head c % 8 for tokens 4g..4g+3: for c < 8 the fp16
  // rounding of p, for c >= 8 the remainder scaled by 2^18. p <= 2^8 (lazy rescale)
  // bounds the scaled remainder by 2^15, and the scale keeps p down to 2^-32 in fp16's
  // normal range, so tiny probabilities still reach the value products.
  half4_t hi, pa;
#pragma unroll
  for (int r = 0; r < 4; ++r) hi[r] = static_cast<_Float16>(p[r]);
  pa = hi;
  if (c >= kGroup) {
#pragma unroll
    for (int r = 0; r < 4; ++r) pa[r] = static_cast<_Float16>((p[r] - static_cast<float>(hi[r])) * kLowScale);
  }

  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // Lane (c, g) reads row 4g + c/4, dims 16nt + 4(c%4)..+3; the transposing read hands
  // it V[tokens 4g..4g+3][dim 16nt + c], the B operand of the 16x16x16 MFMA.
  const char* vrow = vlds + (4 * g + (c >> 2)) * kVRowBytes + 8 * (c & 3);
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const short4_t raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        reinterpret_cast<__attribute__((address_space(3))) short4_t*>(
            reinterpret_cast<uintptr_t>(vrow + 32 * nt)));
    st.acc[nt] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4_t, raw), st.acc[nt], 0, 0, 0);
  }
  // The next block rewrites vlds; LDS ops of one wave complete in order, and this fence
  // keeps the compiler from hoisting those stores above these reads.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Partition count of a sequence.
__device__ __forceinline__ int partitions_of(int len, int max_blocks, int partition_blocks, int& nblk) {
  nblk = min((len + kSlots - 1) / kSlots, max_blocks);
  return (nblk + partition_blocks - 1) / partition_blocks;
}

struct AttnArgs {
  _Float16* out;
  const _Float16* query;
  const _Float16* pool;
  int64_t num_blocks;
  const int32_t* block_tables;
  const int32_t* context_lens;
  float* ws_out;     // [batch*4][max_parts][8 q heads][64] unnormalized partial outputs
  float* ws_ml;      // [batch*4][max_parts][8 q heads][2] (running max, sum of p)
  int32_t* tickets;  // [batch*4] merge tickets, zero between calls
  const int32_t* work_items;  // (sequence, partition) pairs, or null: every (sequence, partition slot)
  int layer, max_blocks, batch, partition_blocks, max_parts, fused_merge;
};

// Agent-coherent accesses (global_store / global_load ... sc1): they bypass this XCD's L2,
// so partials published by one wave are visible to a wave on any XCD without a cache
// writeback or invalidate. The plain variants serve the separate merge kernel, which
// runs after the partition kernel has completed.
template <bool kCoherent>
__device__ __forceinline__ void store_partial(float* p, float x) {
  if constexpr (kCoherent) {
    __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *p = x;
  }
}

template <bool kCoherent>
__device__ __forceinline__ void store_partial2(float* p, float x, float y) {
  if constexpr (kCoherent) {
    const uint64_t bits = (static_cast<uint64_t>(__float_as_uint(y)) << 32) | __float_as_uint(x);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *reinterpret_cast<float2_t*>(p) = float2_t{x, y};
  }
}

template <bool kCoherent>
__device__ __forceinline__ float2_t load_partial2(const float* p) {
  if constexpr (kCoherent) {
    const uint64_t x = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    return float2_t{__uint_as_float(static_cast<uint32_t>(x)), __uint_as_float(static_cast<uint32_t>(x >> 32))};
  } else {
    return *reinterpret_cast<const float2_t*>(p);
  }
}

template <bool kCoherent>
__device__ __forceinline__ float4_t load_partial4(const float* p) {
  if constexpr (kCoherent) {
    const float2_t lo = load_partial2<true>(p);
    const float2_t hi = load_partial2<true>(p + 2);
    return float4_t{lo[0], lo[1], hi[0], hi[1]};
  } else {
    return *reinterpret_cast<const float4_t*>(p);
  }
}

// Merges the nparts partials of one (sequence, kv head) and writes its 8 output rows.
// Lane (qh = lane / 8, dl = lane % 8) folds every partition's dims 8dl..8dl+7 of q head
// qh with the online softmax rule; the loads of kMergeBatch partitions are issued
// before any of them is used, so a merge of up to kMergeBatch partitions costs one
// round trip.
template <bool kCoherent>
__device__ __forceinline__ void merge_partitions(const AttnArgs& a, int bh, int nparts, int lane) {
  const int qh = lane >> 3;
  const int dl = lane & 7;
  float m = -INFINITY, l = 0.f, o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = 0.f;
  const int64_t first = static_cast<int64_t>(bh) * a.max_parts;
#pragma unroll 1
  for (int p0 = 0; p0 < nparts; p0 += kMergeBatch) {
    float2_t ml[kMergeBatch];
    float4_t x0[kMergeBatch], x1[kMergeBatch];
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j) {
      const int64_t p = first + min(p0 + j, nparts - 1);  // clamped: always in bounds
      ml[j] = load_partial2<kCoherent>(a.ws_ml + (p * kGroup + qh) * 2);
      const float* xp = a.ws_out + (p * kGroup + qh) * kHeadDim + 8 * dl;
      x0[j] = load_partial4<kCoherent>(xp);
      x1[j] = load_partial4<kCoherent>(xp + 4);
    }
    // Branch-free fold (a branch would let the compiler sink each load to its use): a
    // clamped duplicate gets weight 0; m is finite from partition 0 on, so m_new is too.
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j) {
      const float mp = (p0 + j < nparts) ? ml[j][0] : -INFINITY;
      const float m_new = fmaxf(m, mp);
      const float s_old = exp2_fast((m - m_new) * kScoreToLog2);  // 0 while m = -inf
      const float s_new = exp2_fast((mp - m_new) * kScoreToLog2);  // 0 for a duplicate
      l = l * s_old + ml[j][1] * s_new;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] = o[i] * s_old + x0[j][i] * s_new;
        o[4 + i] = o[4 + i] * s_old + x1[j][i] * s_new;
      }
      m = m_new;
    }
  }
  half8_t r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = static_cast<_Float16>(o[i] / l);
  *reinterpret_cast<half8_t*>(a.out + (static_cast<int64_t>(bh) * kGroup + qh) * kHeadDim + 8 * dl) = r;
}

__global__ __launch_bounds__(kAttnThreads) void paged_decode_partition_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char lds_v[kSlots * kVRowBytes];  // V rows of one block

  const int h = blockIdx.x % kKVHeads;
  const int rest = blockIdx.x / kKVHeads;
  int b, part;
  if (a.work_items) {  // planned grid: one item per existing partition
    b = a.work_items[2 * rest];
    part = a.work_items[2 * rest + 1];
    if (static_cast<uint32_t>(b) >= static_cast<uint32_t>(a.batch) || part < 0) return;
  } else {  // full grid: partition slots past a sequence's length exit below
    b = rest % a.batch;
    part = rest / a.batch;
  }
  const int lane = threadIdx.x;
  const int c = lane & 15;
  const int g = lane >> 4;

  // One round trip: the length, this partition's block ids and Q are requested together.
  const int pbeg = part * a.partition_blocks;
  const int32_t* table = a.block_tables + static_cast<int64_t>(b) * a.max_blocks;
  const int id_index = pbeg + lane;
  const int ids = (lane < a.partition_blocks && id_index < a.max_blocks) ? table[id_index] : 0;
  // MFMA B operand = Q^T: column c is q head h*8 + c % 8 (columns 8..15 repeat 0..7).
  const _Float16* qrow = a.query + (static_cast<int64_t>(b) * kQHeads + h * kGroup + (c & 7)) * kHeadDim;
  const half8_t qa = *reinterpret_cast<const half8_t*>(qrow + 8 * g);
  const half8_t qb = *reinterpret_cast<const half8_t*>(qrow + 32 + 8 * g);
  const int len = a.context_lens[b];
  if (len <= 0) return;
  int nblk;
  const int nparts = partitions_of(len, a.max_blocks, a.partition_blocks, nblk);
  if (part >= nparts) return;
  const int count = min(nblk - pbeg, a.partition_blocks);

  BlockSource src;
  const int64_t kind_elems = a.num_blocks * kBlockElems;
  src.kpool = a.pool + static_cast<int64_t>(a.layer) * 2 * kind_elems;
  src.vpool = src.kpool + kind_elems;
  src.num_blocks = static_cast<uint32_t>(a.num_blocks);  // host checks num_blocks < 2^31
  src.kofs = c * kRowElems + h * kHeadDim + 8 * g;
  src.vofs = 4 * g * kRowElems + h * kHeadDim + 4 * c;

  WaveState st;
  st.m_run = -INFINITY;
  st.l_part = 0.f;
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) st.acc[nt] = float4_t{0.f, 0.f, 0.f, 0.f};
  int bad = 0;

  // Ring of kRing fragment buffers: while one block is processed, the loads of the next
  // kRing - 1 blocks are in flight. Loads are unconditional (indices past the last block
  // re-read it: in bounds, served by L2) so each block waits only for its own loads.
  {
    BlockFrag f[kRing];
#pragma unroll
    for (int j = 0; j < kRing; ++j) {
      bad |= load_block(f[j], src, ids, min(j, count - 1));
      __builtin_amdgcn_sched_barrier(0);  // issue order = use order
    }
    for (int i = 0; i < count; i += kRing) {
#pragma unroll
      for (int j = 0; j < kRing; ++j) {
        __builtin_amdgcn_sched_barrier(0);  // keep the refills ahead of the next block's waits
        if (i + j < count) process_block(st, f[j], qa, qb, len - (pbeg + i + j) * kSlots, c, g, lds_v);
        bad |= load_block(f[j], src, ids, min(i + j + kRing, count - 1));
      }
    }
  }

  // Add the high rows and the unscaled low rows: afterwards lane (c, g) holds o[k][r] =
  // output of q head 4(g & 1) + r, dim 16(2k + g / 2) + c (lanes g < 2 from tile 2k,
  // g >= 2 from 2k + 1).
  const float l_sum = sum_over_groups(st.l_part);  // lane c < 8: q head c
  const float row_scale = g >= 2 ? 1.0f / kLowScale : 1.0f;
  float o[2][4];
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      o[k][r] = add_swap32(st.acc[2 * k][r] * row_scale, st.acc[2 * k + 1][r] * row_scale);
    }
  const int bh = b * kKVHeads + h;
  const int64_t row0 = static_cast<int64_t>(bh) * kGroup;  // output row of q head 0
  const int head0 = 4 * (g & 1);
  const int dim0 = 16 * (g >> 1) + c;  // + 32k

  if (nparts == 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float inv = 1.0f / row_head_value(l_sum, r, g);
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const float x = bad ? NAN : o[k][r] * inv;
        a.out[(row0 + head0 + r) * kHeadDim + dim0 + 32 * k] = static_cast<_Float16>(x);
      }
    }
    return;
  }
  const int64_t pidx = static_cast<int64_t>(bh) * a.max_parts + part;
  float* ws_out = a.ws_out + pidx * kGroup * kHeadDim;
  float* ws_ml = a.ws_ml + pidx * kGroup * 2;
  if (!a.fused_merge) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        store_partial<false>(ws_out + (head0 + r) * kHeadDim + dim0 + 32 * k, bad ? NAN : o[k][r]);
      }
    if (lane < kGroup) store_partial2<false>(ws_ml + lane * 2, st.m_run, l_sum);
    return;
  }

  // Last-arriver merge: publish the partial with agent-coherent stores, wait until they
  // have completed, then take a ticket; the wave that draws nparts - 1 sees every other
  // partial through agent-coherent loads, writes the output and re-arms the ticket.
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      store_partial<true>(ws_out + (head0 + r) * kHeadDim + dim0 + 32 * k, bad ? NAN : o[k][r]);
    }
  if (lane < kGroup) store_partial2<true>(ws_ml + lane * 2, st.m_run, l_sum);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): every store of this wave has completed
  int ticket = 0;
  if (lane == 0) {
    ticket = __hip_atomic_fetch_add(&a.tickets[bh], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  ticket = __builtin_amdgcn_readfirstlane(ticket);
  if (ticket != nparts - 1) return;
  merge_partitions<true>(a, bh, nparts, lane);
  if (lane == 0) __hip_atomic_store(&a.tickets[bh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Separate merge of every multi-partition (sequence, kv head): one wave each.
__global__ __launch_bounds__(kMergeThreads) void paged_decode_reduce_kernel(AttnArgs a) {
  const int bh = blockIdx.x;
  const int len = a.context_lens[bh / kKVHeads];
  if (len <= 0) return;
  int nblk;
  const int nparts = partitions_of(len, a.max_blocks, a.partition_blocks, nblk);
  if (nparts <= 1) return;
  merge_partitions<false>(a, bh, nparts, threadIdx.x);
}
// ---------------------------------------------------------------------------------------
// Host-side validation and workspace layout.
// ---------------------------------------------------------------------------------------

int max_partitions(int32_t max_blocks, int32_t partition_blocks) {
  return (max_blocks + partition_blocks - 1) / partition_blocks;
}

int check_attn_shape(int32_t batch, int32_t max_blocks, int32_t partition_blocks) {
  if (batch < 0 || batch > (1 << 20)) return set_error(PC_ERR_ARGUMENT, "batch %d out of range", batch);
  if (max_blocks < 1 || max_blocks > (1 << 16)) {
    return set_error(PC_ERR_ARGUMENT, "max_blocks %d out of range [1, 65536]", max_blocks);
  }
  if (partition_blocks < 1 || partition_blocks > kMaxPartitionBlocks) {
    return set_error(PC_ERR_ARGUMENT, "partition_blocks %d outside [1, %d]", partition_blocks,
                     kMaxPartitionBlocks);
  }
  const int64_t grid = static_cast<int64_t>(batch) * kKVHeads * max_partitions(max_blocks, partition_blocks);
  if (grid > INT32_MAX) return set_error(PC_ERR_ARGUMENT, "attention grid too large");
  return PC_OK;
}

// Workspace = ws_out floats | ws_ml floats, each region 256 B aligned.
struct WorkspaceLayout {
  int64_t out_offset, ml_offset, bytes;
};

WorkspaceLayout workspace_layout(int32_t batch, int32_t max_blocks, int32_t partition_blocks) {
  auto round_up = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int64_t rows = static_cast<int64_t>(batch) * kQHeads * max_partitions(max_blocks, partition_blocks);
  WorkspaceLayout w;
  w.out_offset = 0;
  w.ml_offset = round_up(rows * kHeadDim * 4);
  w.bytes = w.ml_offset + round_up(rows * 2 * 4);
  return w;
}

bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

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
  return static_cast<int64_t>(batch) * max_partitions(max_blocks, partition_blocks);
}

int32_t pc_attn_plan(const int32_t* context_lens, int32_t batch, int32_t max_blocks,
                     int32_t partition_blocks, int32_t* work_items, int64_t capacity) {
  if (int rc = check_attn_shape(batch, max_blocks, partition_blocks)) return -rc;
  if (batch > 0 && (!context_lens || !work_items)) return -set_error(PC_ERR_ARGUMENT, "null pointer");
  int64_t n = 0;
  for (int32_t b = 0; b < batch; ++b) {
    const int32_t len = context_lens[b];
    if (len <= 0) continue;
    const int32_t nblk = static_cast<int32_t>(std::min<int64_t>((static_cast<int64_t>(len) + kSlots - 1) / kSlots, max_blocks));
    const int32_t parts = max_partitions(nblk, partition_blocks);
    if (n + parts > capacity) return -set_error(PC_ERR_ARGUMENT, "work item capacity %lld too small", static_cast<long long>(capacity));
    for (int32_t p = 0; p < parts; ++p, ++n) {
      work_items[2 * n] = b;
      work_items[2 * n + 1] = p;
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
  const int parts = max_partitions(max_blocks, partition_blocks);
  if (parts > 1 && !workspace) return set_error(PC_ERR_ARGUMENT, "workspace required");
  if (parts > 1 && !(flags & PC_ATTN_SEPARATE_REDUCE) && !tickets) {
    return set_error(PC_ERR_ARGUMENT, "tickets required for the fused merge");
  }
  if (!aligned(query, 16) || !aligned(out, 16) || !aligned(pool, 16) || !aligned(workspace, 256) ||
      !aligned(tickets, 4) || !aligned(work_items, 4)) {
    return set_error(PC_ERR_ARGUMENT,
                     "query/out/pool must be 16-byte, tickets/work_items 4-byte, workspace 256-byte aligned");
  }
  if (work_items && (num_work_items < 0 || num_work_items > static_cast<int64_t>(batch) * parts)) {
    return set_error(PC_ERR_ARGUMENT, "num_work_items %d outside [0, batch * partitions]", num_work_items);
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
  a.partition_blocks = partition_blocks;
  a.max_parts = parts;
  a.fused_merge = (flags & PC_ATTN_SEPARATE_REDUCE) ? 0 : 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  const unsigned grid = static_cast<unsigned>(work_items ? static_cast<int64_t>(num_work_items) : static_cast<int64_t>(batch) * parts) * kKVHeads;
  hipLaunchKernelGGL(paged_decode_partition_kernel, dim3(grid), dim3(kAttnThreads), 0, s, a);
  if (int rc = check_launch("paged_decode_partition")) return rc;
  if (parts > 1 && !a.fused_merge) {
    hipLaunchKernelGGL(paged_decode_reduce_kernel, dim3(static_cast<unsigned>(batch) * kKVHeads),
                       dim3(kMergeThreads), 0, s, a);
    return check_launch("paged_decode_reduce");
  }
  return PC_OK;
}

}  // extern "C"
