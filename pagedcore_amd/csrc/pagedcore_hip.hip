// Paged KV-cache hot path for MI355X (gfx950): KV append, paged decode attention with
// split-K partitions, and the partition reduce. Exposed through the C ABI declared in
// include/pagedcore_hip.h. No allocation happens here; every buffer comes from the caller.
//
// Pool layout (fixed by the reference allocator, src/pagedcore/kv_cache.py:39-43):
//   fp16 [22 layers][2 kinds][num_blocks][16 slots][4 kv heads][64 dims]
// One (layer, kind, block) is 8 KiB contiguous; one (block, kv head) is 16 rows of 128 B
// at a 512 B stride.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "pagedcore_hip.h"

namespace {

constexpr int kAbiVersion = 1;
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
// One workgroup = (sequence b, kv head h, partition p) with 4 waves; wave w walks blocks
// p*P + w, p*P + w + 4, ... of the partition. Per 16-token block and wave:
//   * QK on the matrix core: S^T[16 tokens][16] = K[16][64] . Q^T[64][16] with two
//     v_mfma_f32_16x16x32_f16 (q heads 8..15 are zero padding). K fragments come straight
//     from HBM with 16 B loads, rows = tokens; fp16 x fp16 products are exact in fp32.
//     Lane (c = lane % 16, g = lane / 16) receives the scores of q head c for tokens
//     4g..4g+3.
//   * online softmax in fp32 in the raw-dot domain (m = max q.k); p = 2^((dot - m) * C)
//     with C = log2(e)/8, so the 1/8 scale is applied after the exact difference. Each
//     (q head, token group g) is its own softmax stream; a stream's running max only moves
//     when a block beats it by more than 2^8 (so rescales are rare and p <= 256).
//   * p goes through 1 KiB of LDS to the PV layout; PV is fp32 FMA on the VALU with fp16 V
//     operands (v_fma_mix). Lane (c, g) owns dims 4c..4c+3 of all 8 q heads for tokens
//     4g..4g+3 (8 B V loads; one load instruction covers 4 rows of 128 B).
// The 16 streams (4 waves x 4 token groups) are merged through LDS at the end; a
// single-partition sequence writes fp16 output, otherwise (m, l, o) partials go to the
// workspace for the reduce kernel.
// ---------------------------------------------------------------------------------------

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));

constexpr int kAttnWaves = 4;
constexpr int kAttnThreads = 64 * kAttnWaves;
constexpr int kStreams = kAttnWaves * 4;  // softmax streams per workgroup
constexpr int kDefaultPartitionBlocks = 32;
constexpr int kMaxPartitionBlocks = 128;
// log2(e) / sqrt(64): turns a raw q.k difference into a base-2 exponent.
constexpr float kScoreToLog2 = 0.18033688011112042f;
// Lazy-rescale threshold in raw-dot units (2^8 in probability terms).
constexpr float kRescaleDot = 8.0f / kScoreToLog2;

struct BlockFrag {
  half8_t k0, k1;  // K[token c][dims 8g..8g+7] and [32+8g..32+8g+7]
  half4_t v[4];    // V[token 4g+j][dims 4c..4c+3]
};

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Per-wave streaming state for one (sequence, kv head, partition).
struct WaveState {
  float m_run;  // running max of raw q.k, stream (q head c, token group g)
  float l_part; // sum of p of that stream
  float acc[kGroup][4];  // sum of p * v for q heads 0..7, dims 4c..4c+3, token group g
};

struct BlockSource {
  const _Float16* kpool;  // K plane of the layer
  const _Float16* vpool;  // V plane of the layer
  const int32_t* table;   // block ids of the sequence
  uint32_t num_blocks;
  int kofs, vofs;         // lane offsets inside a block
};

// Loads one block's K/V fragments. `ids` holds the wave's block ids, one per lane; `i` is
// wave-uniform, so the id lands in an SGPR and the block base is scalar arithmetic.
// Returns 1 if the block id is out of range (the fragments then come from block 0 so that
// no access leaves the pool).
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

__device__ __forceinline__ void process_block(WaveState& st, const BlockFrag& f, half8_t qa,
                                              half8_t qb, int valid, int c, int g,
                                              float* __restrict__ plds) {
  float4_t s = {0.f, 0.f, 0.f, 0.f};
  s = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.k0, qa, s, 0, 0, 0);
  s = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.k1, qb, s, 0, 0, 0);
  // s[r] = q[head c] . k[token 4g + r]
  float sc[4] = {s[0], s[1], s[2], s[3]};
  half4_t v[4] = {f.v[0], f.v[1], f.v[2], f.v[3]};
  if (valid < kSlots) {  // last, partial block: masked slots never enter an FMA
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (4 * g + r >= valid) {
        sc[r] = -INFINITY;
        v[r] = half4_t{};
      }
    }
  }
  const float mloc = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
  if (__any((c < kGroup) && (mloc > st.m_run + kRescaleDot))) {
    // A stream whose tokens are all masked keeps m_run = -inf; alpha is then irrelevant.
    const float m_new = fmaxf(st.m_run, mloc);
    const float alpha = (m_new == -INFINITY) ? 1.f : exp2_fast((st.m_run - m_new) * kScoreToLog2);
    st.l_part *= alpha;
    st.m_run = m_new;
#pragma unroll
    for (int qh = 0; qh < kGroup; ++qh) {
      const float a = __shfl(alpha, qh + 16 * g);
#pragma unroll
      for (int i = 0; i < 4; ++i) st.acc[qh][i] *= a;
    }
  }
  float p[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    p[r] = (sc[r] == -INFINITY) ? 0.f : exp2_fast((sc[r] - st.m_run) * kScoreToLog2);
  }
  st.l_part += (p[0] + p[1]) + (p[2] + p[3]);

  *reinterpret_cast<float4_t*>(plds + c * 16 + 4 * g) = float4_t{p[0], p[1], p[2], p[3]};
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float4_t pv[kGroup];
#pragma unroll
  for (int qh = 0; qh < kGroup; ++qh) pv[qh] = *reinterpret_cast<const float4_t*>(plds + qh * 16 + 4 * g);
  // The next block rewrites plds; LDS ops of one wave complete in order, and this fence
  // keeps the compiler from hoisting that store above these loads.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();

#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float v0 = static_cast<float>(v[j][0]);
    const float v1 = static_cast<float>(v[j][1]);
    const float v2 = static_cast<float>(v[j][2]);
    const float v3 = static_cast<float>(v[j][3]);
#pragma unroll
    for (int qh = 0; qh < kGroup; ++qh) {
      const float pj = pv[qh][j];
      st.acc[qh][0] = fmaf(pj, v0, st.acc[qh][0]);
      st.acc[qh][1] = fmaf(pj, v1, st.acc[qh][1]);
      st.acc[qh][2] = fmaf(pj, v2, st.acc[qh][2]);
      st.acc[qh][3] = fmaf(pj, v3, st.acc[qh][3]);
    }
  }
}

__global__ __launch_bounds__(kAttnThreads) void paged_decode_partition_kernel(
    _Float16* __restrict__ out, const _Float16* __restrict__ query,
    const _Float16* __restrict__ pool, int64_t num_blocks, int layer,
    const int32_t* __restrict__ block_tables, int max_blocks,
    const int32_t* __restrict__ context_lens, int batch, int partition_blocks, int max_parts,
    float* __restrict__ ws_out, float* __restrict__ ws_ml) {
  __shared__ float lds_p[kAttnWaves][16 * 16];             // [q head][token] per wave
  __shared__ float lds_acc[kStreams][kGroup][kHeadDim];    // [wave*4+g][q head][dim]
  __shared__ float lds_l[kStreams][kGroup];
  __shared__ float lds_m[kStreams][kGroup];
  __shared__ int lds_bad[kAttnWaves];

  const int h = blockIdx.x % kKVHeads;
  const int rest = blockIdx.x / kKVHeads;
  const int b = rest % batch;
  const int part = rest / batch;

  const int len = context_lens[b];
  if (len <= 0) return;
  const int nblk = min((len + kSlots - 1) / kSlots, max_blocks);
  const int nparts = (nblk + partition_blocks - 1) / partition_blocks;
  if (part >= nparts) return;  // the whole workgroup leaves together

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;

  BlockSource src;
  const int64_t kind_elems = num_blocks * kBlockElems;
  src.kpool = pool + static_cast<int64_t>(layer) * 2 * kind_elems;
  src.vpool = src.kpool + kind_elems;
  src.table = block_tables + static_cast<int64_t>(b) * max_blocks;
  src.num_blocks = static_cast<uint32_t>(num_blocks);  // host checks num_blocks < 2^31
  src.kofs = c * kRowElems + h * kHeadDim + 8 * g;
  src.vofs = 4 * g * kRowElems + h * kHeadDim + 4 * c;

  // MFMA B operand = Q^T: column c is q head h*8+c (zero for the 8 padding columns).
  half8_t qa = {}, qb = {};
  if (c < kGroup) {
    const _Float16* qrow = query + (static_cast<int64_t>(b) * kQHeads + h * kGroup + c) * kHeadDim;
    qa = *reinterpret_cast<const half8_t*>(qrow + 8 * g);
    qb = *reinterpret_cast<const half8_t*>(qrow + 32 + 8 * g);
  }

  WaveState st;
  st.m_run = -INFINITY;
  st.l_part = 0.f;
#pragma unroll
  for (int qh = 0; qh < kGroup; ++qh)
#pragma unroll
    for (int i = 0; i < 4; ++i) st.acc[qh][i] = 0.f;
  int bad = 0;

  const int blk_begin = part * partition_blocks;
  const int blk_end = min(nblk, blk_begin + partition_blocks);
  float* plds = lds_p[wave];

  // Ping-pong over two fragment buffers: the next block's loads are in flight while the
  // current block is processed. The prefetch is unconditional (clamped to the wave's last
  // block, an in-bounds re-read served by L2) so that the wait before each block covers
  // only that block's loads.
  // The wave's blocks are blk_begin + wave + 4 i for i < count; lane i holds the id of
  // block i, read once up front so the loop never waits on the table.
  const int first = blk_begin + wave;
  const int count = first < blk_end ? (blk_end - first + kAttnWaves - 1) / kAttnWaves : 0;
  const int ids = lane < count ? src.table[first + kAttnWaves * lane] : 0;
  BlockFrag fa, fb;
  bad |= load_block(fa, src, ids, 0);  // count may be 0: block 0's id is then 0, in bounds
  for (int i = 0; i < count; i += 2) {
    bad |= load_block(fb, src, ids, min(i + 1, count - 1));
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of this block's waits
    process_block(st, fa, qa, qb, len - (first + kAttnWaves * i) * kSlots, c, g, plds);
    bad |= load_block(fa, src, ids, min(i + 2, count - 1));
    __builtin_amdgcn_sched_barrier(0);
    if (i + 1 < count) {
      process_block(st, fb, qa, qb, len - (first + kAttnWaves * (i + 1)) * kSlots, c, g, plds);
    }
  }

  // Merge the 16 streams.
  const int stream = wave * 4 + g;
  float* la = &lds_acc[stream][0][0];
#pragma unroll
  for (int qh = 0; qh < kGroup; ++qh) {
    *reinterpret_cast<float4_t*>(la + qh * kHeadDim + 4 * c) =
        float4_t{st.acc[qh][0], st.acc[qh][1], st.acc[qh][2], st.acc[qh][3]};
  }
  if (c < kGroup) {
    lds_l[stream][c] = st.l_part;
    lds_m[stream][c] = st.m_run;
  }
  if (lane == 0) lds_bad[wave] = bad;
  __syncthreads();

  const int t = threadIdx.x;
  const int qh = t >> 5;
  const int d = (t & 31) * 2;
  float m_all = -INFINITY;
#pragma unroll
  for (int sidx = 0; sidx < kStreams; ++sidx) m_all = fmaxf(m_all, lds_m[sidx][qh]);
  float l_all = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int sidx = 0; sidx < kStreams; ++sidx) {
    const float ms = lds_m[sidx][qh];
    // Streams that saw no unmasked token have m = -inf and contribute nothing.
    const float a = (ms == -INFINITY) ? 0.f : exp2_fast((ms - m_all) * kScoreToLog2);
    const float2_t x = *reinterpret_cast<const float2_t*>(&lds_acc[sidx][qh][d]);
    l_all += a * lds_l[sidx][qh];
    o0 += a * x[0];
    o1 += a * x[1];
  }
  int any_bad = 0;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) any_bad |= lds_bad[w];
  if (any_bad) {  // an out-of-range block id poisons the row instead of reading out of bounds
    o0 = NAN;
    o1 = NAN;
  }
  const int64_t row = static_cast<int64_t>(b) * kQHeads + h * kGroup + qh;
  if (nparts == 1) {
    *reinterpret_cast<half2_t*>(out + row * kHeadDim + d) =
        half2_t{static_cast<_Float16>(o0 / l_all), static_cast<_Float16>(o1 / l_all)};
  } else {
    const int64_t slot = row * max_parts + part;
    *reinterpret_cast<float2_t*>(ws_out + slot * kHeadDim + d) = float2_t{o0, o1};
    if ((t & 31) == 0) *reinterpret_cast<float2_t*>(ws_ml + slot * 2) = float2_t{m_all, l_all};
  }
}

// Merge the partitions of every multi-partition (sequence, kv head): one workgroup each.
__global__ __launch_bounds__(kAttnThreads) void paged_decode_reduce_kernel(
    _Float16* __restrict__ out, const int32_t* __restrict__ context_lens, int max_blocks,
    int partition_blocks, int max_parts, const float* __restrict__ ws_out,
    const float* __restrict__ ws_ml) {
  const int h = blockIdx.x % kKVHeads;
  const int b = blockIdx.x / kKVHeads;
  const int len = context_lens[b];
  if (len <= 0) return;
  const int nblk = min((len + kSlots - 1) / kSlots, max_blocks);
  const int nparts = (nblk + partition_blocks - 1) / partition_blocks;
  if (nparts <= 1) return;

  const int t = threadIdx.x;
  const int qh = t >> 5;
  const int d = (t & 31) * 2;
  const int64_t row = static_cast<int64_t>(b) * kQHeads + h * kGroup + qh;
  const float* ml = ws_ml + row * max_parts * 2;
  float m_all = -INFINITY;
  for (int p = 0; p < nparts; ++p) m_all = fmaxf(m_all, ml[2 * p]);
  float l_all = 0.f, o0 = 0.f, o1 = 0.f;
  for (int p = 0; p < nparts; ++p) {
    const float a = exp2_fast((ml[2 * p] - m_all) * kScoreToLog2);
    l_all += a * ml[2 * p + 1];
    const float2_t x =
        *reinterpret_cast<const float2_t*>(ws_out + (row * max_parts + p) * kHeadDim + d);
    o0 += a * x[0];
    o1 += a * x[1];
  }
  *reinterpret_cast<half2_t*>(out + row * kHeadDim + d) =
      half2_t{static_cast<_Float16>(o0 / l_all), static_cast<_Float16>(o1 / l_all)};
}

// ---------------------------------------------------------------------------------------
// Host-side validation shared by the attention entry points.
// ---------------------------------------------------------------------------------------

int max_partitions(int32_t max_blocks, int32_t partition_blocks) {
  return (max_blocks + partition_blocks - 1) / partition_blocks;
}

int check_attn_shape(int32_t batch, int32_t max_blocks, int32_t partition_blocks) {
  if (batch < 0 || batch > (1 << 20)) return set_error(PC_ERR_ARGUMENT, "batch %d out of range", batch);
  if (max_blocks < 1 || max_blocks > (1 << 16)) {
    return set_error(PC_ERR_ARGUMENT, "max_blocks %d out of range [1, 65536]", max_blocks);
  }
  if (partition_blocks < 4 || partition_blocks > kMaxPartitionBlocks || partition_blocks % 4 != 0) {
    return set_error(PC_ERR_ARGUMENT, "partition_blocks %d must be a multiple of 4 in [4, %d]",
                     partition_blocks, kMaxPartitionBlocks);
  }
  const int64_t grid = static_cast<int64_t>(batch) * kKVHeads * max_partitions(max_blocks, partition_blocks);
  if (grid > INT32_MAX) return set_error(PC_ERR_ARGUMENT, "attention grid too large");
  return PC_OK;
}

bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

}  // namespace

extern "C" {

int pc_abi_version(void) { return kAbiVersion; }

const char* pc_last_error(void) { return g_error; }

int32_t pc_attn_default_partition_blocks(void) { return kDefaultPartitionBlocks; }

int64_t pc_attn_workspace_floats(int32_t batch, int32_t max_blocks, int32_t partition_blocks) {
  if (check_attn_shape(batch, max_blocks, partition_blocks) != PC_OK) return 0;
  const int64_t rows = static_cast<int64_t>(batch) * kQHeads * max_partitions(max_blocks, partition_blocks);
  return rows * kHeadDim + rows * 2;
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

int pc_paged_decode_attn_partitions(void* out, const void* query, const void* pool,
                                    int64_t num_blocks, int32_t layer,
                                    const int32_t* block_tables, int32_t max_blocks,
                                    const int32_t* context_lens, int32_t batch,
                                    int32_t partition_blocks, float* ws_out, float* ws_ml,
                                    void* stream) {
  if (!out || !query || !pool || !block_tables || !context_lens) {
    return set_error(PC_ERR_ARGUMENT, "null pointer");
  }
  if (num_blocks < 1 || num_blocks > INT32_MAX) {
    return set_error(PC_ERR_ARGUMENT, "num_blocks out of range");
  }
  if (layer < 0 || layer >= kLayers) return set_error(PC_ERR_ARGUMENT, "layer %d outside [0, 22)", layer);
  if (int rc = check_attn_shape(batch, max_blocks, partition_blocks)) return rc;
  const int parts = max_partitions(max_blocks, partition_blocks);
  if (parts > 1 && (!ws_out || !ws_ml)) return set_error(PC_ERR_ARGUMENT, "workspace required");
  if (!aligned(query, 16) || !aligned(out, 4) || !aligned(pool, 16)) {
    return set_error(PC_ERR_ARGUMENT, "query/pool must be 16-byte and out 4-byte aligned");
  }
  if (parts > 1 && (!aligned(ws_out, 8) || !aligned(ws_ml, 8))) {
    return set_error(PC_ERR_ARGUMENT, "workspace must be 8-byte aligned");
  }
  if (batch == 0) return ok();
  hipStream_t s = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  const unsigned grid = static_cast<unsigned>(batch) * kKVHeads * parts;
  hipLaunchKernelGGL(paged_decode_partition_kernel, dim3(grid), dim3(kAttnThreads), 0, s,
                     static_cast<_Float16*>(out), static_cast<const _Float16*>(query),
                     static_cast<const _Float16*>(pool), num_blocks, layer, block_tables, max_blocks,
                     context_lens, batch, partition_blocks, parts, ws_out, ws_ml);
  return check_launch("paged_decode_partition");
}

int pc_paged_decode_attn_reduce(void* out, const int32_t* context_lens, int32_t batch,
                                int32_t max_blocks, int32_t partition_blocks,
                                const float* ws_out, const float* ws_ml, void* stream) {
  if (!out || !context_lens) return set_error(PC_ERR_ARGUMENT, "null pointer");
  if (int rc = check_attn_shape(batch, max_blocks, partition_blocks)) return rc;
  const int parts = max_partitions(max_blocks, partition_blocks);
  if (parts <= 1 || batch == 0) return ok();  // nothing was split
  if (!ws_out || !ws_ml) return set_error(PC_ERR_ARGUMENT, "workspace required");
  hipStream_t s = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  hipLaunchKernelGGL(paged_decode_reduce_kernel, dim3(static_cast<unsigned>(batch) * kKVHeads),
                     dim3(kAttnThreads), 0, s, static_cast<_Float16*>(out), context_lens, max_blocks,
                     partition_blocks, parts, ws_out, ws_ml);
  return check_launch("paged_decode_reduce");
}

int pc_paged_decode_attn(void* out, const void* query, const void* pool, int64_t num_blocks,
                         int32_t layer, const int32_t* block_tables, int32_t max_blocks,
                         const int32_t* context_lens, int32_t batch, int32_t partition_blocks,
                         float* ws_out, float* ws_ml, void* stream) {
  if (int rc = pc_paged_decode_attn_partitions(out, query, pool, num_blocks, layer, block_tables,
                                               max_blocks, context_lens, batch, partition_blocks,
                                               ws_out, ws_ml, stream)) {
    return rc;
  }
  return pc_paged_decode_attn_reduce(out, context_lens, batch, max_blocks, partition_blocks, ws_out,
                                     ws_ml, stream);
}

}  // extern "C"
