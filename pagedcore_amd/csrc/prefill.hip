// Causal prompt attention over contiguous K/V (the prefill of one sequence).
//
// o[t][h] = softmax_{j <= t}(q[t][h] . k[j][h / 8] / 8) . v[j][h / 8] for a prompt of T tokens,
// with q [T][32][64], k and v [T][4][64] (the rotated keys and the values that
// pc_rope_kv_append wrote), o [T][32][64], all fp16.
//
// Work split: one workgroup per (16-query block, kv head), longest (latest) blocks first; its
// 8 waves are the 8 query heads of the kv head, so each K/V block is fetched once per
// workgroup (the waves share it through L1). A wave walks key blocks 0 .. its query block
// with an online softmax in fp32:
//   S^T = K_blk . Q^T   on v_mfma_f32_16x16x32_f16 (lane (c, g): keys 4g..4g+3 of position c)
//   O^T += V^T . P^T    on v_mfma_f32_16x16x16f16, V^T from the transposing LDS reads of the
//                       decode kernel's V layout, P^T straight from the S^T registers
// so every per-position quantity (running max, sum, rescale) stays in the lane that owns
// the position. K and V of the next block move to LDS by DMA while the current block is
// processed (two buffers per wave). Probabilities enter the PV
// product as fp16 (relative error 2^-11) and the normalising sum adds those same fp16
// weights; everything else is fp32 with one final fp16 rounding.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

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
constexpr int kBufBytes = 2 * kTileBytes;           // K tile, then V tile
constexpr int kMaxTokens = 1 << 16;
constexpr float kLazyLog2 = 8.0f;            // headroom (log2 of p) before the running max is raised

struct PrefillArgs {
  _Float16* out;
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  int tokens;
};

__global__ __launch_bounds__(kThreads) void prefill_attention_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[kWaves][2][kBufBytes];
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

  // Q is loaded once with ordinary loads. K and V of each key block arrive by LDS DMA into
  // one of two buffers (waited for explicitly), so no register is ever the target of a load
  // still in flight across loop iterations.
  const _Float16* qrow = a.q + (static_cast<int64_t>(min(pos, last)) * kQHeads + head) * kHeadDim + 8 * g;
  const half8_t qa = *reinterpret_cast<const half8_t*>(qrow);
  const half8_t qc = *reinterpret_cast<const half8_t*>(qrow + 32);

  // DMA lane mapping (64 lanes x 16 B = 8 rows of 128 B per instruction): lane moves piece
  // qs of rows r8 and r8 + 8. K piece p of row r sits at position p ^ (r & 7) (the A-operand
  // reads of 16 rows then hit 8 different 16 B bank groups); V uses the decode kernel's
  // 32 B-group swizzle for its transposing reads.
  const int qs = lane & 7, r8 = lane >> 3;
  const int kpieceA = qs ^ (r8 & 7), kpieceB = qs ^ ((r8 + 8) & 7);
  const int vpieceA = 2 * ((qs >> 1) ^ row_sel(r8)) + (qs & 1);
  const int vpieceB = 2 * ((qs >> 1) ^ row_sel(r8 + 8)) + (qs & 1);
  const uint32_t buf0 = lds_offset(lds[w][0]);
  // K reads: lane (c, g) takes row c, pieces g and 4 + g
  const uint32_t kaddr0 = buf0 + c * 128 + 16 * (g ^ (c & 7));
  const uint32_t kaddr1 = buf0 + c * 128 + 16 * ((4 + g) ^ (c & 7));
  // V transposing reads: lane (c, g) supplies row 4g + c/4, 8 B piece c % 4
  const int rr = 4 * g + (c >> 2);
  const uint32_t vbase = buf0 + kTileBytes + rr * 128 + 8 * (c & 3);
  const uint32_t tsel = row_sel(rr);

  auto issue = [&](int kb, int buf) {
    char* dst = lds[w][buf];
    const int ra = min(kBlock * kb + r8, last), rb = min(kBlock * kb + r8 + 8, last);
    const _Float16* ka = a.k + (static_cast<int64_t>(ra) * kKVHeads + h) * kHeadDim;
    const _Float16* kb8 = a.k + (static_cast<int64_t>(rb) * kKVHeads + h) * kHeadDim;
    const _Float16* va = a.v + (static_cast<int64_t>(ra) * kKVHeads + h) * kHeadDim;
    const _Float16* vb8 = a.v + (static_cast<int64_t>(rb) * kKVHeads + h) * kHeadDim;
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(ka + 8 * kpieceA), lds_ptr(dst), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(kb8 + 8 * kpieceB), lds_ptr(dst + 1024), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(va + 8 * vpieceA), lds_ptr(dst + kTileBytes), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(vb8 + 8 * vpieceB), lds_ptr(dst + kTileBytes + 1024), 16,
                                     0, 0);
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order the waits count on
  };

  float m = 0.f, mc = 0.f, lsum = 0.f;
  float4_t acc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) acc[u] = float4_t{0.f, 0.f, 0.f, 0.f};
  const int nkb = qb + 1;  // causal: key blocks 0 .. qb

  issue(0, 0);
  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
    const bool more = kb + 1 < nkb;
    // The other buffer was last read in the previous iteration (its reads waited for
    // lgkmcnt(0)), so it can be refilled; then this block's four DMAs are complete once at
    // most the next block's four are pending.
    if (more) {
      issue(kb + 1, buf ^ 1);
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    half8_t k0, k1;
    asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(k0), "=&v"(k1)
                 : "v"(kaddr0 + buf * kBufBytes), "v"(kaddr1 + buf * kBufBytes)
                 : "memory");
    float4_t sv = {0.f, 0.f, 0.f, 0.f};
    sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, qa, sv, 0, 0, 0);
    sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, qc, sv, 0, 0, 0);
    float sc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int key = kBlock * kb + 4 * g + e;
      sc[e] = (key <= pos && key <= last) ? sv[e] : -INFINITY;
    }
    const float bm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    if (kb == 0) {
      m = max_over_groups(bm);  // finite: key 0 is visible to every position
      mc = m * kScoreToLog2;
    } else if (__builtin_amdgcn_ballot_w64(bm * kScoreToLog2 > mc + kLazyLog2) != 0) {
      const float mn = fmaxf(m, max_over_groups(bm));
      const float alpha = exp2_fast((m - mn) * kScoreToLog2);
      lsum *= alpha;
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] *= alpha;
      m = mn;
      mc = m * kScoreToLog2;
    }
    half4_t pb;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // the sum takes the fp16 weights the PV product uses, so constant V comes back exactly
      pb[e] = static_cast<_Float16>(exp2_fast(fmaf(sc[e], kScoreToLog2, -mc)));
      lsum += static_cast<float>(pb[e]);
    }
    short4_t v0, v1, v2, v3;
    read_v_tiles<0>(vbase + buf * kBufBytes, tsel, v0, v1, v2, v3);
    acc[0] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, v0), pb, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, v1), pb, acc[1], 0, 0, 0);
    acc[2] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, v2), pb, acc[2], 0, 0, 0);
    acc[3] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, v3), pb, acc[3], 0, 0, 0);
  }

  // lane (c, g) of tile u holds O^T[dims 16u + 4g .. + 3][position c]
  const float inv = 1.0f / sum_over_groups(lsum);
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
  PrefillArgs a{static_cast<_Float16*>(out), static_cast<const _Float16*>(query), static_cast<const _Float16*>(key),
                static_cast<const _Float16*>(value), tokens};
  const unsigned grid = static_cast<unsigned>((tokens + kBlock - 1) / kBlock) * kKVHeads;
  hipLaunchKernelGGL(prefill_attention_kernel, dim3(grid), dim3(kThreads), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("prefill_attention");
}
