// Causal prompt attention over contiguous K/V (the prefill of one sequence).
//
// o[t][h] = softmax_{j <= t}(q[t][h] . k[j][h / 8] / 8) . v[j][h / 8] for a prompt of T tokens,
// with q [T][32][64], k and v [T][4][64] (the rotated keys and the values that
// pc_rope_kv_append wrote), o [T][32][64], all fp16.
//
// Work split: one workgroup per (16-query block, kv head), longest (latest) blocks first; its
// 8 waves are the 8 query heads of the kv head. Each 16-key block of K and V is staged in
// LDS once per workgroup (LDS DMA by four of the waves, two buffers, one barrier per block)
// and read by all eight waves. A wave walks key blocks 0 .. its query block with an online
// softmax in fp32:
//   S^T = K_blk . Q^T   on v_mfma_f32_16x16x32_f16 (lane (c, g): keys 4g..4g+3 of position c)
//   O^T += V^T . P^T    on v_mfma_f32_16x16x16f16, V^T from the decode kernel's transposing
//                       LDS reads, P^T straight from the S^T registers
//   l   += 1 . P^T      one more v_mfma_f32_16x16x16f16 with an all-ones A operand: the
//                       softmax denominator of every position, summed on the matrix core
// so every per-position quantity (running max, sum, rescale) stays in the lane that owns
// the position. Only the diagonal block needs the causal mask. Probabilities enter the PV
// product as fp16 (relative error 2^-11) and the denominator sums those same fp16 weights;
// everything else is fp32 with one final fp16 rounding.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "pagedcore_hip.h"
#include "pc_device.h"
#include "pc_internal.h"

namespace {

using namespace pc_device;
using pc_internal::aligned;
using pc_internal::check_launch;
using pc_internal::ok;
using pc_internal::set_error;

constexpr int kKVHeads = 4;
constexpr int kQHeads = 32;
constexpr int kHeadDim = 64;
constexpr int kWaves = kQHeads / kKVHeads;  // 8 query heads per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kBlock = 16;                   // positions per query block and keys per key block
constexpr int kTileBytes = kBlock * kHeadDim * 2;  // 16 rows of one kv head: 2 KiB
constexpr int kBufBytes = 2 * kTileBytes;           // one key block: K tile, then V tile
constexpr int kStepBlocks = 4;                      // key blocks per step (a multiple of 2)
constexpr int kStageBytes = kStepBlocks * kBufBytes;
constexpr int kMaxTokens = 1 << 16;
constexpr float kLazyLog2 = 8.0f;            // headroom (log2 of p) before the running max is raised

// f(integral_constant<int, p>) for every pair p of key blocks of a step, in order.
template <typename F, int... P>
__device__ __forceinline__ void for_pairs_impl(F&& f, std::integer_sequence<int, P...>) {
  (f(std::integral_constant<int, P>{}), ...);
}
template <typename F>
__device__ __forceinline__ void for_pairs(F&& f) {
  for_pairs_impl(f, std::make_integer_sequence<int, kStepBlocks / 2>{});
}

// Two 16-key tiles as one 32-key MFMA operand (first tile's keys first).
__device__ __forceinline__ half8_t join(short4_t x, short4_t y) {
  const half4_t a = __builtin_bit_cast(half4_t, x), b = __builtin_bit_cast(half4_t, y);
  return half8_t{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

struct PrefillArgs {
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  int tokens;
  _Float16* out;
};

// Scalar parameters in the order of PrefillArgs: all are preloaded into SGPRs at wave
// launch.
__global__ __launch_bounds__(kThreads) void prefill_attention_kernel(const _Float16* q, const _Float16* k,
                                                                     const _Float16* v, int tokens, _Float16* out) {
  const PrefillArgs a{q, k, v, tokens, out};
  // Two stages of kStepBlocks key blocks each: stage s, block b: K tile at s * kStageBytes +
  // b * kBufBytes, its V tile kTileBytes after it.
  __shared__ __attribute__((aligned(16))) char lds[2][kStageBytes];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int qblocks = (a.tokens + kBlock - 1) / kBlock;
  const int h = blockIdx.x % kKVHeads;
  const int qb = qblocks - 1 - static_cast<int>(blockIdx.x / kKVHeads);
  const int head = kWaves * h + w;
  const int pos = kBlock * qb + c;  // this lane's query position (column of S^T)
  const int last = a.tokens - 1;

  const _Float16* qrow = a.q + (static_cast<int64_t>(min(pos, last)) * kQHeads + head) * kHeadDim + 8 * g;
  half8_t qa = *reinterpret_cast<const half8_t*>(qrow);
  half8_t qc = *reinterpret_cast<const half8_t*>(qrow + 32);

  // Staging: every wave issues kStepBlocks / 2 LDS DMA instructions per stage (each 64 lanes
  // x 16 B = rows srow .. srow + 7 of one tile): wave w stages blocks w / 4, w / 4 + 2, ...
  // of the step, the K (w & 2 = 0) or V tile, rows 8 (w & 1) .. 8 (w & 1) + 7. K piece p of
  // row r sits at position p ^ (r & 7) (the A-operand reads of 16 rows then hit 8 different
  // 16 B bank groups); V uses the decode kernel's 32 B-group swizzle for its transposing
  // reads.
  const bool stage_v = (w & 2) != 0;
  const int sblock = w >> 2;
  const int qs = lane & 7;
  const int srow = 8 * (w & 1) + (lane >> 3);
  const int piece = stage_v ? 2 * ((qs >> 1) ^ row_sel(srow)) + (qs & 1) : qs ^ (srow & 7);
  const _Float16* ssrc = (stage_v ? a.v : a.k) + h * kHeadDim + 8 * piece;
  const int sdst = sblock * kBufBytes + (stage_v ? kTileBytes : 0) + 1024 * (w & 1);
  const uint32_t lds0 = lds_offset(lds[0]);
  // K reads: lane (c, g) takes row c, pieces g and 4 + g
  const uint32_t kaddr0 = lds0 + c * 128 + 16 * (g ^ (c & 7));
  const uint32_t kaddr1 = lds0 + c * 128 + 16 * ((4 + g) ^ (c & 7));
  // V transposing reads: lane (c, g) supplies row 4g + c/4, 8 B piece c % 4
  const int rr = 4 * g + (c >> 2);
  const uint32_t vbase = lds0 + kTileBytes + rr * 128 + 8 * (c & 3);
  const uint32_t tsel = row_sel(rr);

  // Key blocks kStepBlocks * j .. + kStepBlocks - 1 into stage `buf` (rows past the prompt
  // repeat its last row; their scores are masked).
  auto stage = [&](int j, int buf) {
#pragma unroll
    for (int i = 0; i < kStepBlocks / 2; ++i) {
      const int row = min(kBlock * (kStepBlocks * j + sblock + 2 * i) + srow, last);
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(ssrc + static_cast<int64_t>(row) * kKVHeads * kHeadDim),
                                       lds_ptr(lds[buf] + sdst + 2 * i * kBufBytes), 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  const half8_t ones = {1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16};
  float m = 0.f, mc = 0.f;
  float4_t acc[4], lacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < 4; ++u) acc[u] = float4_t{0.f, 0.f, 0.f, 0.f};
  const int steps = (qb + kStepBlocks) / kStepBlocks;  // causal: key blocks 0 .. qb

  // One step over the key blocks of step j, staged in stage B (a compile-time constant, so
  // every LDS address below is a fixed base plus an immediate offset).
  auto step = [&](int j, auto stage_index) {
    constexpr int B = decltype(stage_index)::value;
    constexpr uint32_t so = B * kStageBytes;
    // This wave's staging of step j (and, before the first step, Q) has landed; after the
    // barrier every wave's has, and every wave has finished reading the other stage (its
    // reads of step j - 1 waited for lgkmcnt(0)), which the next staging refills. Q is named
    // so that the compiler does not add a wait of its own for it, which would also wait for
    // the staging issued below.
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(qa), "+v"(qc) : : "memory");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < steps) stage(j + 1, B ^ 1);
    // sc[4 b + e]: key 4g + e of block kStepBlocks * j + b
    float sc[4 * kStepBlocks];
    auto scores = [&](auto pair) {
      constexpr int b = 2 * decltype(pair)::value;
      half8_t k00, k01, k10, k11;
      asm volatile(
          "ds_read_b128 %0, %4 offset:%6\n\tds_read_b128 %1, %5 offset:%6\n\tds_read_b128 %2, %4 offset:%7\n\t"
          "ds_read_b128 %3, %5 offset:%7\n\ts_waitcnt lgkmcnt(0)"
          : "=&v"(k00), "=&v"(k01), "=&v"(k10), "=&v"(k11)
          : "v"(kaddr0), "v"(kaddr1), "i"(so + b * kBufBytes), "i"(so + (b + 1) * kBufBytes)
          : "memory");
      float4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k00, qa, s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k10, qa, s1, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k01, qc, s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k11, qc, s1, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sc[4 * b + e] = s0[e];
        sc[4 * b + 4 + e] = s1[e];
      }
    };
    for_pairs(scores);
    if (kStepBlocks * j + kStepBlocks - 1 >= qb) {  // the diagonal step: keys after the position, or past the prompt, are masked
#pragma unroll
      for (int e = 0; e < 4 * kStepBlocks; ++e) {
        const int key = kBlock * (kStepBlocks * j + (e >> 2)) + 4 * g + (e & 3);
        sc[e] = (key <= pos && key <= last) ? sc[e] : -INFINITY;
      }
    }
    float bm = sc[0];
#pragma unroll
    for (int e = 1; e < 4 * kStepBlocks; ++e) bm = fmaxf(bm, sc[e]);
    if (j == 0) {
      m = max_over_groups(bm);  // finite: key 0 is visible to every position
      mc = m * kScoreToLog2;
    } else if (__builtin_amdgcn_ballot_w64(bm * kScoreToLog2 > mc + kLazyLog2) != 0) {
      const float mn = fmaxf(m, max_over_groups(bm));
      const float alpha = exp2_fast((m - mn) * kScoreToLog2);
      lacc *= alpha;
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] *= alpha;
      m = mn;
      mc = m * kScoreToLog2;
    }
    // Per pair of blocks, P^T as one 32-key B operand: element e is key 4g + (e & 3) of
    // the pair's block e / 4; the V^T A operands concatenate the two blocks in the same
    // order.
    auto accumulate = [&](auto pair) {
      constexpr int b = 2 * decltype(pair)::value;
      half8_t pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = static_cast<_Float16>(exp2_fast(fmaf(sc[4 * b + e], kScoreToLog2, -mc)));
      short4_t a0, a1, a2, a3, b0, b1, b2, b3;
      read_v_tiles<so + b * kBufBytes>(vbase, tsel, a0, a1, a2, a3);
      read_v_tiles<so + (b + 1) * kBufBytes>(vbase, tsel, b0, b1, b2, b3);
      acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(join(a0, b0), pb, acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(join(a1, b1), pb, acc[1], 0, 0, 0);
      acc[2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(join(a2, b2), pb, acc[2], 0, 0, 0);
      acc[3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(join(a3, b3), pb, acc[3], 0, 0, 0);
      lacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pb, lacc, 0, 0, 0);
    };
    for_pairs(accumulate);
  };

  stage(0, 0);
  for (int j = 0; j < steps; j += 2) {
    step(j, std::integral_constant<int, 0>{});
    if (j + 1 < steps) step(j + 1, std::integral_constant<int, 1>{});
  }

  // lane (c, g) of tile u holds O^T[dims 16u + 4g .. + 3][position c]; every row of lacc
  // holds the denominator of position c
  const float inv = 1.0f / lacc[0];
  if (pos <= last) {
    _Float16* dst = a.out + (static_cast<int64_t>(pos) * kQHeads + head) * kHeadDim + 4 * g;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      half4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = static_cast<_Float16>(acc[u][e] * inv);
      *reinterpret_cast<half4_t*>(dst + 16 * u) = o;
    }
  }
}

}  // namespace

extern "C" int pc_prefill_attention(void* out, const void* query, const void* key, const void* value, int32_t tokens,
                                    void* stream) {
  if (tokens < 0 || tokens > kMaxTokens) return set_error(PC_ERR_ARGUMENT, "tokens %d outside [0, %d]", tokens, kMaxTokens);
  if (tokens == 0) return ok();
  if (!out || !query || !key || !value) return set_error(PC_ERR_ARGUMENT, "null pointer");
  if (!aligned(out, 16) || !aligned(query, 16) || !aligned(key, 16) || !aligned(value, 16))
    return set_error(PC_ERR_ARGUMENT, "buffers must be 16-byte aligned");
  const unsigned grid = static_cast<unsigned>((tokens + kBlock - 1) / kBlock) * kKVHeads;
  hipLaunchKernelGGL(prefill_attention_kernel, dim3(grid), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const _Float16*>(query), static_cast<const _Float16*>(key),
                     static_cast<const _Float16*>(value), static_cast<int>(tokens), static_cast<_Float16*>(out));
  return check_launch("prefill_attention");
}
