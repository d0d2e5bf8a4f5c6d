// Elementwise kernels of the batched decode step around paged attention: RoPE fused with the
// KV append, residual add fused with RMSNorm, and SiLU fused with the up-projection product.
// The first two also take their projection input as fp32 split-K partial sums (the output of
// pc_gemm_m128's partials epilogue), added in split order and rounded to fp16 once: the
// value the reference's fp16 GEMM output holds, up to the order of fp32 accumulation.
//
// Each one reproduces the fp16 rounding points of the reference's torch expressions
// (src/pagedcore/dense.py:17-21, 33-61, 102-104): every torch op on fp16 tensors computes
// in fp32 and rounds its result to fp16 once, so a kernel rounds exactly where the
// reference expression materialises an fp16 tensor and nowhere else. Contraction of a
// multiply into a following add is switched off wherever that would skip a rounding.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "pagedcore_hip.h"
#include "pc_internal.h"

namespace {

using pc_internal::aligned;
using pc_internal::check_launch;
using pc_internal::ok;
using pc_internal::set_error;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

constexpr int kLayers = 22;
constexpr int kSlots = 16;
constexpr int kKVHeads = 4;
constexpr int kQHeads = 32;
constexpr int kHeadDim = 64;
constexpr int kHalfDim = kHeadDim / 2;                 // 32 rotation frequencies
constexpr int64_t kRowElems = kKVHeads * kHeadDim;     // 256 fp16 per pool token row
constexpr int kQElems = kQHeads * kHeadDim;            // 2048
constexpr int kQkvElems = kQElems + 2 * kRowElems;     // 2560: q | k | v of one token
constexpr int kRopeThreads = 192;                      // 128 q tasks, 16 k tasks, 32 v tasks
constexpr int kNormThreads = 256;
constexpr int kNormMaxChunks = 4;                      // rows of up to 4 * 256 * 8 = 8192
constexpr int kSiluThreads = 256;

__device__ __forceinline__ _Float16 round_h(float x) { return static_cast<_Float16>(x); }

typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kUnrolledSplits = 8;  // split counts up to this load all their parts at once

// fp16(sum over the splits of parts[s * split_stride + offset + 0..7]), added in split order.
// Up to kUnrolledSplits splits, every load is issued before the first add (one memory round
// trip, not one per split); a split past `splits` reloads split 0 and is not added.
__device__ __forceinline__ half8_t sum_parts8(const float* parts, int64_t offset, int splits, int64_t split_stride) {
  float4_t lo, hi;
  if (splits <= kUnrolledSplits) {
    float4_t l[kUnrolledSplits], h[kUnrolledSplits];
#pragma unroll
    for (int s = 0; s < kUnrolledSplits; ++s) {
      const float* p = parts + (s < splits ? s : 0) * split_stride + offset;
      l[s] = *reinterpret_cast<const float4_t*>(p);
      h[s] = *reinterpret_cast<const float4_t*>(p + 4);
    }
    lo = l[0];
    hi = h[0];
#pragma unroll
    for (int s = 1; s < kUnrolledSplits; ++s) {
      lo = s < splits ? lo + l[s] : lo;
      hi = s < splits ? hi + h[s] : hi;
    }
  } else {
    lo = *reinterpret_cast<const float4_t*>(parts + offset);
    hi = *reinterpret_cast<const float4_t*>(parts + offset + 4);
    for (int s = 1; s < splits; ++s) {
      const float* p = parts + s * split_stride + offset;
      lo += *reinterpret_cast<const float4_t*>(p);
      hi += *reinterpret_cast<const float4_t*>(p + 4);
    }
  }
  half8_t out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[i] = round_h(lo[i]);
    out[i + 4] = round_h(hi[i]);
  }
  return out;
}

// ---------------------------------------------------------------------------------------
// RoPE + KV append.
//
// One workgroup per token row t. Task layout (one 16 B chunk pair each):
//   threads   0..127  q head tid / 4, dims [8c, 8c + 8) with their partners 32 further on
//   threads 128..143  k head (tid - 128) / 4, same dims
//   threads 144..175  v dims [8j, 8j + 8) over the 4 heads' 256 values, copied unrotated
// The reference rotation (dense.py:56-59) is x * cos + cat(-x2, x1) * sin with cos/sin the
// fp16 tables of the position; for d < 32 that is x[d] * c[d] + (-x[d + 32]) * s[d], for
// d >= 32 x[d] * c[d - 32] + x[d - 32] * s[d - 32], each product and the sum rounded to fp16.
// ---------------------------------------------------------------------------------------

struct RopeArgs {
  _Float16* query_out;        // [T][32][64]
  _Float16* key_out;          // [T][4][64] or null
  _Float16* value_out;        // [T][4][64] or null
  const _Float16* qkv;        // [T][qkv_stride]: q (2048) | k (256) | v (256); or null and
  const float* qkv_parts;     // [splits][T][2560] fp32 partial sums of the same columns
  int32_t splits;
  const int64_t* positions;   // [T]
  const _Float16* rope;       // [rope_positions][2][32]: cos, then sin
  _Float16* pool;             // or null
  const int64_t* slot_mapping;  // [T] or null
  int64_t qkv_stride;         // qkv's row stride, or qkv_parts' split stride (T * 2560)
  int64_t slot_limit;         // num_blocks * 16
  int64_t kind_elems;         // num_blocks * 16 * 256: one (layer, kind) plane
  int32_t layer;
  int32_t rope_positions;
};

__device__ __forceinline__ void rotate_pair(half8_t& lo, half8_t& hi, const half8_t c, const half8_t s) {
#pragma clang fp contract(off)
  half8_t out_lo, out_hi;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float x1 = static_cast<float>(lo[i]);
    const float x2 = static_cast<float>(hi[i]);
    const float cf = static_cast<float>(c[i]);
    const float sf = static_cast<float>(s[i]);
    const float a1 = static_cast<float>(round_h(x1 * cf));
    // fp16(-a * b) == -fp16(a * b): round-to-nearest-even is symmetric.
    const float b1 = static_cast<float>(-round_h(x2 * sf));
    const float a2 = static_cast<float>(round_h(x2 * cf));
    const float b2 = static_cast<float>(round_h(x1 * sf));
    out_lo[i] = round_h(a1 + b1);
    out_hi[i] = round_h(a2 + b2);
  }
  lo = out_lo;
  hi = out_hi;
}

// 8 columns of token t's q | k | v row, from the fp16 row or the partial sums.
__device__ __forceinline__ half8_t load_qkv8(const RopeArgs& a, int64_t t, int col) {
  if (a.qkv_parts != nullptr) return sum_parts8(a.qkv_parts, t * kQkvElems + col, a.splits, a.qkv_stride);
  return *reinterpret_cast<const half8_t*>(a.qkv + t * a.qkv_stride + col);
}

// Scalar parameters, those the first loads need leading (the compiler preloads the leading
// 56 bytes into SGPRs at wave launch: no kernel-argument round trip before them).
__global__ __launch_bounds__(kRopeThreads) void rope_kv_append_kernel(
    const int64_t* positions, const float* qkv_parts, const _Float16* qkv, int64_t qkv_stride, const _Float16* rope,
    const int64_t* slot_mapping, int32_t splits, int32_t rope_positions, _Float16* pool, int64_t slot_limit,
    int64_t kind_elems, _Float16* query_out, _Float16* key_out, _Float16* value_out, int32_t layer) {
  RopeArgs a;
  a.query_out = query_out;
  a.key_out = key_out;
  a.value_out = value_out;
  a.qkv = qkv;
  a.qkv_parts = qkv_parts;
  a.splits = splits;
  a.positions = positions;
  a.rope = rope;
  a.pool = pool;
  a.slot_mapping = slot_mapping;
  a.qkv_stride = qkv_stride;
  a.slot_limit = slot_limit;
  a.kind_elems = kind_elems;
  a.layer = layer;
  a.rope_positions = rope_positions;
  const int64_t t = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t position = a.positions[t];
  const bool valid_position = position >= 0 && position < a.rope_positions;
  int64_t slot = -1;
  if (a.pool != nullptr && a.slot_mapping != nullptr) {
    slot = a.slot_mapping[t];
    if (slot >= a.slot_limit) slot = -1;  // outside the pool: never written
  }
  const int64_t pool_row = static_cast<int64_t>(a.layer) * 2 * a.kind_elems + slot * kRowElems;

  if (tid < 144) {
    const bool is_q = tid < 128;
    const int task = is_q ? tid : tid - 128;
    const int head = task >> 2;
    const int c = task & 3;
    const int col = (is_q ? 0 : kQElems) + head * kHeadDim + 8 * c;
    half8_t lo = load_qkv8(a, t, col);
    half8_t hi = load_qkv8(a, t, col + kHalfDim);
    if (valid_position) {
      const _Float16* table = a.rope + position * kHeadDim + 8 * c;
      const half8_t cs = *reinterpret_cast<const half8_t*>(table);
      const half8_t sn = *reinterpret_cast<const half8_t*>(table + kHalfDim);
      rotate_pair(lo, hi, cs, sn);
    } else {
      // Never reached through the host API (positions are checked there); a bad position
      // yields NaN rows instead of a read outside the table.
      lo = static_cast<half8_t>(__builtin_nanf16(""));
      hi = lo;
    }
    if (is_q) {
      _Float16* dst = a.query_out + t * kQElems + head * kHeadDim + 8 * c;
      *reinterpret_cast<half8_t*>(dst) = lo;
      *reinterpret_cast<half8_t*>(dst + kHalfDim) = hi;
    } else {
      const int64_t offset = head * kHeadDim + 8 * c;
      if (a.key_out != nullptr) {
        *reinterpret_cast<half8_t*>(a.key_out + t * kRowElems + offset) = lo;
        *reinterpret_cast<half8_t*>(a.key_out + t * kRowElems + offset + kHalfDim) = hi;
      }
      if (slot >= 0 && valid_position) {
        *reinterpret_cast<half8_t*>(a.pool + pool_row + offset) = lo;
        *reinterpret_cast<half8_t*>(a.pool + pool_row + offset + kHalfDim) = hi;
      }
    }
  } else if (tid < 176) {
    const int j = tid - 144;
    const half8_t v = load_qkv8(a, t, kQElems + kRowElems + 8 * j);
    if (a.value_out != nullptr) *reinterpret_cast<half8_t*>(a.value_out + t * kRowElems + 8 * j) = v;
    if (slot >= 0 && valid_position) *reinterpret_cast<half8_t*>(a.pool + pool_row + a.kind_elems + 8 * j) = v;
  }
}

// ---------------------------------------------------------------------------------------
// Residual add + RMSNorm (dense.py:17-21 after the residual sum of decoder.py:191-192).
//
// One workgroup per row; thread i owns 16 B chunks i, i + 256, ... of the row.
//   h   = fp16(hidden + delta)                     (only when delta is given; stored back)
//   r   = 1 / sqrt(sum(h * h) / width + eps)       (fp32)
//   out = fp16(weight * fp16(h * r))
// ---------------------------------------------------------------------------------------

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) x += __shfl_xor(x, offset, 64);
  return x;
}

// delta, when given, is fp16 [rows][width] or (delta_parts, splits) fp32 partial sums
// [splits][rows][width], rounded to fp16 before the add. The parameters the first loads need
// lead (they are preloaded into SGPRs).
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(_Float16* __restrict__ hidden,
                                                                    const float* __restrict__ delta_parts,
                                                                    const _Float16* __restrict__ delta,
                                                                    int64_t parts_stride, int32_t splits,
                                                                    int32_t width, float eps,
                                                                    const _Float16* __restrict__ weight,
                                                                    _Float16* __restrict__ out) {
#pragma clang fp contract(off)
  __shared__ float wave_sums[kNormThreads / 64];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * width;
  const int tid = threadIdx.x;
  const int chunks = width / 8;
  // The weight chunks are loaded first, with the same guards as their use below, so that
  // their round trip overlaps the residual's instead of following the reduction.
  half8_t wt[kNormMaxChunks];
#pragma unroll
  for (int k = 0; k < kNormMaxChunks; ++k) {
    const int chunk = tid + k * kNormThreads;
    if (chunk < chunks) wt[k] = *reinterpret_cast<const half8_t*>(weight + 8 * chunk);
  }
  half8_t h[kNormMaxChunks];
  float squares = 0.0f;
#pragma unroll
  for (int k = 0; k < kNormMaxChunks; ++k) {
    const int chunk = tid + k * kNormThreads;
    if (chunk < chunks) {
      _Float16* p = hidden + base + 8 * chunk;
      h[k] = *reinterpret_cast<const half8_t*>(p);
      if (delta != nullptr || delta_parts != nullptr) {
        const half8_t d = delta_parts != nullptr ? sum_parts8(delta_parts, base + 8 * chunk, splits, parts_stride)
                                                 : *reinterpret_cast<const half8_t*>(delta + base + 8 * chunk);
#pragma unroll
        for (int i = 0; i < 8; ++i) h[k][i] = round_h(static_cast<float>(h[k][i]) + static_cast<float>(d[i]));
        *reinterpret_cast<half8_t*>(p) = h[k];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = static_cast<float>(h[k][i]);
        squares += x * x;
      }
    }
  }
  squares = wave_sum(squares);
  if ((tid & 63) == 0) wave_sums[tid >> 6] = squares;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int w = 0; w < kNormThreads / 64; ++w) total += wave_sums[w];
  const float scale = 1.0f / sqrtf(total / static_cast<float>(width) + eps);
#pragma unroll
  for (int k = 0; k < kNormMaxChunks; ++k) {
    const int chunk = tid + k * kNormThreads;
    if (chunk < chunks) {
      half8_t o;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float normalized = static_cast<float>(round_h(static_cast<float>(h[k][i]) * scale));
        o[i] = round_h(static_cast<float>(wt[k][i]) * normalized);
      }
      *reinterpret_cast<half8_t*>(out + base + 8 * chunk) = o;
    }
  }
}

// ---------------------------------------------------------------------------------------
// SwiGLU activation (dense.py:102-104): out = fp16(fp16(silu(gate)) * up), where
// gate_up row r is [gate (width) | up (width)], silu(x) = x / (1 + exp(-x)) in fp32.
// ---------------------------------------------------------------------------------------

__global__ __launch_bounds__(kSiluThreads) void silu_mul_kernel(_Float16* __restrict__ out,
                                                                const _Float16* __restrict__ gate_up,
                                                                int64_t rows, int32_t width) {
#pragma clang fp contract(off)
  const int64_t chunks_per_row = width / 8;
  const int64_t chunk = static_cast<int64_t>(blockIdx.x) * kSiluThreads + threadIdx.x;
  if (chunk >= rows * chunks_per_row) return;
  const int64_t r = chunk / chunks_per_row;
  const int64_t c = chunk % chunks_per_row;
  const _Float16* src = gate_up + r * 2 * width + 8 * c;
  const half8_t g = *reinterpret_cast<const half8_t*>(src);
  const half8_t u = *reinterpret_cast<const half8_t*>(src + width);
  half8_t o;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float x = static_cast<float>(g[i]);
    const float activated = static_cast<float>(round_h(x / (1.0f + expf(-x))));
    o[i] = round_h(activated * static_cast<float>(u[i]));
  }
  *reinterpret_cast<half8_t*>(out + r * width + 8 * c) = o;
}

}  // namespace

extern "C" {

}  // extern "C"

namespace {

// Shared by both RoPE entry points: exactly one of qkv / qkv_parts is given (checked by the
// callers), with qkv_stride its row stride or split stride.
int rope_kv_append(void* query_out, void* key_out, void* value_out, const void* qkv, const float* qkv_parts,
                   int32_t splits, int64_t qkv_stride, const int64_t* positions, const void* rope_table,
                   int32_t rope_positions, void* pool, int64_t num_blocks, int32_t layer,
                   const int64_t* slot_mapping, int64_t num_tokens, void* stream) {
  if (!query_out || !positions || !rope_table) return set_error(PC_ERR_ARGUMENT, "null pointer");
  if (rope_positions < 1) return set_error(PC_ERR_ARGUMENT, "rope_positions must be positive");
  if ((pool == nullptr) != (slot_mapping == nullptr))
    return set_error(PC_ERR_ARGUMENT, "pool and slot_mapping must both be given or both be null");
  if (pool != nullptr) {
    if (num_blocks < 1 || num_blocks > INT32_MAX)
      return set_error(PC_ERR_ARGUMENT, "num_blocks %lld out of range", static_cast<long long>(num_blocks));
    if (layer < 0 || layer >= kLayers) return set_error(PC_ERR_ARGUMENT, "layer %d outside [0, 22)", layer);
  }
  if (!aligned(query_out, 16) || !aligned(qkv, 16) || !aligned(qkv_parts, 16) || !aligned(rope_table, 16) ||
      !aligned(pool, 16) || !aligned(key_out, 16) || !aligned(value_out, 16))
    return set_error(PC_ERR_ARGUMENT, "buffers must be 16-byte aligned");
  hipLaunchKernelGGL(rope_kv_append_kernel, dim3(static_cast<uint32_t>(num_tokens)), dim3(kRopeThreads), 0,
                     static_cast<hipStream_t>(stream), positions, qkv_parts, static_cast<const _Float16*>(qkv),
                     qkv_stride, static_cast<const _Float16*>(rope_table), slot_mapping, splits, rope_positions,
                     static_cast<_Float16*>(pool), pool ? num_blocks * kSlots : int64_t{0},
                     pool ? num_blocks * kSlots * kRowElems : int64_t{0}, static_cast<_Float16*>(query_out),
                     static_cast<_Float16*>(key_out), static_cast<_Float16*>(value_out), pool ? layer : 0);
  return check_launch("rope_kv_append");
}

int add_rms_norm(void* out, void* hidden, const void* delta, const float* delta_parts, int32_t splits,
                 const void* weight, int64_t rows, int32_t width, float eps, void* stream) {
  if (rows < 0 || rows > INT32_MAX) return set_error(PC_ERR_ARGUMENT, "rows %lld out of range", static_cast<long long>(rows));
  if (width < 8 || width % 8 != 0 || width > kNormThreads * kNormMaxChunks * 8)
    return set_error(PC_ERR_ARGUMENT, "width %d must be a multiple of 8 in [8, %d]", width,
                     kNormThreads * kNormMaxChunks * 8);
  if (rows == 0) return ok();  // nothing to read or write (empty buffers may be null)
  if (!out || !hidden || !weight) return set_error(PC_ERR_ARGUMENT, "null pointer");
  if (!(eps >= 0.0f)) return set_error(PC_ERR_ARGUMENT, "eps must be non-negative");
  if (!aligned(out, 16) || !aligned(hidden, 16) || !aligned(delta, 16) || !aligned(delta_parts, 16) ||
      !aligned(weight, 16))
    return set_error(PC_ERR_ARGUMENT, "buffers must be 16-byte aligned");
  hipLaunchKernelGGL(add_rms_norm_kernel, dim3(static_cast<uint32_t>(rows)), dim3(kNormThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<_Float16*>(hidden), delta_parts,
                     static_cast<const _Float16*>(delta), rows * width, splits, width, eps,
                     static_cast<const _Float16*>(weight), static_cast<_Float16*>(out));
  return check_launch("add_rms_norm");
}

}  // namespace

extern "C" {

int pc_rope_kv_append(void* query_out, void* key_out, void* value_out, const void* qkv, int64_t qkv_stride,
                      const int64_t* positions, const void* rope_table, int32_t rope_positions, void* pool,
                      int64_t num_blocks, int32_t layer, const int64_t* slot_mapping, int64_t num_tokens,
                      void* stream) {
  if (num_tokens < 0) return set_error(PC_ERR_ARGUMENT, "negative token count");
  if (num_tokens > INT32_MAX) return set_error(PC_ERR_ARGUMENT, "too many tokens");
  if (num_tokens == 0) return ok();  // nothing to read or write (empty buffers may be null)
  if (!qkv) return set_error(PC_ERR_ARGUMENT, "null pointer");
  if (qkv_stride < kQkvElems || qkv_stride % 8 != 0)
    return set_error(PC_ERR_ARGUMENT, "qkv_stride %lld must be >= %d and a multiple of 8",
                     static_cast<long long>(qkv_stride), kQkvElems);
  return rope_kv_append(query_out, key_out, value_out, qkv, nullptr, 1, qkv_stride, positions, rope_table,
                        rope_positions, pool, num_blocks, layer, slot_mapping, num_tokens, stream);
}

int pc_rope_kv_append_parts(void* query_out, void* key_out, void* value_out, const float* qkv_parts, int32_t splits,
                            const int64_t* positions, const void* rope_table, int32_t rope_positions, void* pool,
                            int64_t num_blocks, int32_t layer, const int64_t* slot_mapping, int64_t num_tokens,
                            void* stream) {
  if (num_tokens < 0) return set_error(PC_ERR_ARGUMENT, "negative token count");
  if (num_tokens > INT32_MAX / kQkvElems) return set_error(PC_ERR_ARGUMENT, "too many tokens");
  if (num_tokens == 0) return ok();
  if (!qkv_parts) return set_error(PC_ERR_ARGUMENT, "null pointer");
  if (splits < 1 || splits > 64) return set_error(PC_ERR_ARGUMENT, "splits %d outside [1, 64]", splits);
  return rope_kv_append(query_out, key_out, value_out, nullptr, qkv_parts, splits, num_tokens * kQkvElems, positions,
                        rope_table, rope_positions, pool, num_blocks, layer, slot_mapping, num_tokens, stream);
}

int pc_add_rms_norm(void* out, void* hidden, const void* delta, const void* weight, int64_t rows, int32_t width,
                    float eps, void* stream) {
  return add_rms_norm(out, hidden, delta, nullptr, 1, weight, rows, width, eps, stream);
}

int pc_add_rms_norm_parts(void* out, void* hidden, const float* delta_parts, int32_t splits, const void* weight,
                          int64_t rows, int32_t width, float eps, void* stream) {
  if (rows > 0 && !delta_parts) return set_error(PC_ERR_ARGUMENT, "null pointer");
  if (splits < 1 || splits > 64) return set_error(PC_ERR_ARGUMENT, "splits %d outside [1, 64]", splits);
  if (rows > INT32_MAX / 8192) return set_error(PC_ERR_ARGUMENT, "rows %lld out of range", static_cast<long long>(rows));
  return add_rms_norm(out, hidden, nullptr, delta_parts, splits, weight, rows, width, eps, stream);
}

int pc_silu_mul(void* out, const void* gate_up, int64_t rows, int32_t width, void* stream) {
  if (rows < 0) return set_error(PC_ERR_ARGUMENT, "negative row count");
  if (width < 8 || width % 8 != 0) return set_error(PC_ERR_ARGUMENT, "width %d must be a positive multiple of 8", width);
  if (rows == 0) return ok();  // nothing to read or write (empty buffers may be null)
  if (!out || !gate_up) return set_error(PC_ERR_ARGUMENT, "null pointer");
  if (!aligned(out, 16) || !aligned(gate_up, 16)) return set_error(PC_ERR_ARGUMENT, "buffers must be 16-byte aligned");
  const int64_t chunks = rows * (width / 8);
  const int64_t blocks = (chunks + kSiluThreads - 1) / kSiluThreads;
  if (blocks > INT32_MAX) return set_error(PC_ERR_ARGUMENT, "silu_mul too large");
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kSiluThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<_Float16*>(out),
                     static_cast<const _Float16*>(gate_up), rows, width);
  return check_launch("silu_mul");
}

}  // extern "C"
