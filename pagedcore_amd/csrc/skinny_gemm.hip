// Projection GEMMs of the batched decode step at up to 128 rows: Y = X W^T with X fp16
// [m <= 128][k] (the step's activations) and W fp16 [n][k] (a weight, row-major as stored),
// fp32 accumulation. The reference computes these with torch.nn.functional.linear on fp16
// tensors (src/pagedcore/dense.py:91-104 via decoder.py:156-199): fp32 accumulation and one
// rounding to fp16 per output element. Here the rounding stays where the reference has it:
// the split-K consumers (pc_rope_kv_append_parts, pc_add_rms_norm_parts) add the fp32
// partial sums in split order and round once.
//
// Design for decode shapes (m = batch, n and k in the thousands): the weight is read once
// from HBM and is the only large stream, so one workgroup computes ALL m rows of an NT-row
// slice of W over a range of K (split-K when n alone gives too few workgroups to fill the
// 256 CUs). X and W chunks stream through a ring of LDS stages filled by LDS DMA
// (global_load_lds_dwordx4, 16 B per lane, rows swizzled so that the MFMA operand reads are
// bank-conflict free); the waves read 16x32 operand fragments from LDS and issue
// v_mfma_f32_16x16x32_f16 with W as the A operand (16 weight rows) and X as the B operand
// (16 activation rows), so each lane ends with 4 consecutive output columns of one row.
//
// Epilogues: fp32 partials [splits][m][n]; fp16 [m][n] (one split); or SwiGLU (one split):
// a tile's W rows are 32 gate_proj rows and the 32 matching up_proj rows of the stacked
// [gate | up] weight, and the tile writes fp16(fp16(silu(fp16 gate)) * fp16 up) for its 32
// columns (dense.py:102-104 with the roundings of silu_mul_kernel).

#include <hip/hip_runtime.h>

#include <atomic>

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
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kMaxRows = 128;
constexpr int kSwiGLUHalf = 32;  // gate (and up) rows per SwiGLU tile

enum Epilogue : int32_t { kPartials = PC_GEMM_PARTIALS, kHalf = PC_GEMM_HALF, kSwiGLU = PC_GEMM_SWIGLU };

__device__ __forceinline__ __attribute__((address_space(3))) void* lds_ptr(char* p) {
  return (__attribute__((address_space(3))) void*)(p);
}
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}
__device__ __forceinline__ half8_t lds_read(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) half8_t*>(static_cast<uintptr_t>(addr));
}
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory");
}
// Workgroup barrier without a memory fence (a fence would wait for every DMA in flight);
// the empty asm statements keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

struct GemmArgs {
  const _Float16* x;
  const _Float16* w;
  int m, n, k, ksplit;  // ksplit: K range of one split
  int tiles;            // workgroups per split
  int half_rows;        // SwiGLU: rows of gate_proj (up_proj starts there)
  void* out;
};

template <int NT, int KC, int STAGES, int WAVES>
struct Shape {
  static constexpr int CH = KC / 8;        // 16-byte chunks per LDS row
  static constexpr int XB = kMaxRows * KC * 2;
  static constexpr int WB = NT * KC * 2;
  static constexpr int SB = XB + WB;       // bytes per ring stage
  static constexpr int XI = XB / 1024;     // 1 KiB DMA instructions per stage
  static constexpr int WI = WB / 1024;
  static_assert(XI % WAVES == 0 && WI % WAVES == 0, "each wave issues the same number of DMA instructions");
  static constexpr int PER = (XI + WI) / WAVES;
  static constexpr int MT = kMaxRows / 16 / WAVES;  // 16-row X tiles per wave
  static constexpr int NTL = NT / 16;               // 16-row W tiles
  static constexpr int LDS = STAGES * SB;
  static_assert(LDS <= 160 * 1024, "ring fits the CU's LDS");
};

// Position of 16-byte chunk c of LDS row r (an involution): the 16 rows one operand read
// touches at one chunk land on distinct banks.
template <int CH>
__device__ __forceinline__ int swizzle(int r, int c) {
  if constexpr (CH == 16) {
    return c ^ (r & 15);
  } else {
    static_assert(CH == 8, "KC of 64 or 128");
    return c ^ ((r >> 1) & 7);
  }
}

// Weight row held in LDS row r of tile `tile`.
template <int NT, Epilogue E>
__device__ __forceinline__ int weight_row(const GemmArgs& a, int tile, int r) {
  if constexpr (E == kSwiGLU) {
    return (r < kSwiGLUHalf ? 0 : a.half_rows - kSwiGLUHalf) + tile * kSwiGLUHalf + r;
  } else {
    return tile * NT + r;
  }
}

// DMA of one ring stage: X rows 0..127 (rows past m repeat row m - 1) and the tile's W rows,
// K columns [kbase, kbase + KC).
template <int NT, int KC, int STAGES, int WAVES, Epilogue E>
__device__ __forceinline__ void issue_stage(char* stage, const GemmArgs& a, int tile, int kbase, int wave, int lane) {
  using S = Shape<NT, KC, STAGES, WAVES>;
#pragma unroll
  for (int i = 0; i < S::XI / WAVES; ++i) {
    const int j = i * WAVES + wave;
    const int p = j * 64 + lane;
    const int r = p / S::CH;
    const int c = swizzle<S::CH>(r, p % S::CH);
    const int xr = r < a.m ? r : a.m - 1;
    const _Float16* src = a.x + static_cast<int64_t>(xr) * a.k + kbase + 8 * c;
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(src), lds_ptr(stage + j * 1024), 16, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < S::WI / WAVES; ++i) {
    const int j = i * WAVES + wave;
    const int p = j * 64 + lane;
    const int r = p / S::CH;
    const int c = swizzle<S::CH>(r, p % S::CH);
    const _Float16* src = a.w + static_cast<int64_t>(weight_row<NT, E>(a, tile, r)) * a.k + kbase + 8 * c;
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(src), lds_ptr(stage + S::XB + j * 1024), 16, 0, 0);
  }
}

__device__ __forceinline__ _Float16 round_h(float x) { return static_cast<_Float16>(x); }

// Scalar parameters in the order of GemmArgs: all of them are preloaded into SGPRs at wave
// launch (no kernel-argument round trip before the first DMA).
template <int NT, int KC, int STAGES, int WAVES, Epilogue E>
__global__ __launch_bounds__(64 * WAVES) void gemm_m128_kernel(const _Float16* x, const _Float16* w, int m, int n, int k,
                                                               int ksplit, int tiles, int half_rows, void* out) {
  const GemmArgs a{x, w, m, n, k, ksplit, tiles, half_rows, out};
  using S = Shape<NT, KC, STAGES, WAVES>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int tile = blockIdx.x % a.tiles;
  const int split = blockIdx.x / a.tiles;
  const int k0 = split * a.ksplit;
  const int steps = a.ksplit / KC;
  float4_t acc[S::NTL][S::MT];
#pragma unroll
  for (int i = 0; i < S::NTL; ++i)
#pragma unroll
    for (int j = 0; j < S::MT; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int t = 0; t < STAGES - 1; ++t) {
    if (t < steps) issue_stage<NT, KC, STAGES, WAVES, E>(smem + t * S::SB, a, tile, k0 + t * KC, wave, lane);
  }

  const uint32_t lds0 = lds_offset(smem);
  const int r16 = lane & 15, g = lane >> 4;
  for (int t = 0; t < steps; ++t) {
    // This wave's DMA of stage t has landed once at most the later stages already issued
    // (min(STAGES - 2, steps - 1 - t) of them, PER instructions each) are outstanding.
    if constexpr (STAGES == 4) {
      if (t + 2 < steps) wait_vm<2 * S::PER>();
      else if (t + 1 < steps) wait_vm<S::PER>();
      else wait_vm<0>();
    } else {
      static_assert(STAGES == 3, "three or four stages");
      if (t + 1 < steps) wait_vm<S::PER>();
      else wait_vm<0>();
    }
    // Every wave's DMA of stage t has landed, and every wave has finished reading stage
    // t - 1 (its LDS reads were consumed by its MFMAs), which the next DMA overwrites. A
    // bare barrier: a fence here would wait for the DMAs still in flight.
    stage_barrier();
    if (t + STAGES - 1 < steps) {
      issue_stage<NT, KC, STAGES, WAVES, E>(smem + ((t + STAGES - 1) % STAGES) * S::SB, a, tile,
                                            k0 + (t + STAGES - 1) * KC, wave, lane);
    }
    const uint32_t xs = lds0 + (t % STAGES) * S::SB;
    const uint32_t ws = xs + S::XB;
#pragma unroll
    for (int ks = 0; ks < KC / 32; ++ks) {
      // Lane (r16, g) supplies row r16 of each 16-row tile at K columns 32 ks + 8 g .. + 7.
      const int chunk = 4 * ks + g;
      half8_t wf[S::NTL], xf[S::MT];
#pragma unroll
      for (int i = 0; i < S::NTL; ++i) {
        const int r = 16 * i + r16;
        wf[i] = lds_read(ws + (r * S::CH + swizzle<S::CH>(r, chunk)) * 16);
      }
#pragma unroll
      for (int j = 0; j < S::MT; ++j) {
        const int r = 16 * (wave * S::MT + j) + r16;
        xf[j] = lds_read(xs + (r * S::CH + swizzle<S::CH>(r, chunk)) * 16);
      }
#pragma unroll
      for (int i = 0; i < S::NTL; ++i)
#pragma unroll
        for (int j = 0; j < S::MT; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[i], xf[j], acc[i][j], 0, 0, 0);
    }
  }

  // acc[i][j], lane (r16, g), element e: output row m = 16 (wave MT + j) + r16, column
  // (LDS W row) 16 i + 4 g + e of the tile.
#pragma unroll
  for (int j = 0; j < S::MT; ++j) {
    const int m = 16 * (wave * S::MT + j) + r16;
    if (m >= a.m) continue;
    if constexpr (E == kSwiGLU) {
#pragma clang fp contract(off)
      const int width = a.half_rows;
#pragma unroll
      for (int i = 0; i < kSwiGLUHalf / 16; ++i) {
        half4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = static_cast<float>(round_h(acc[i][j][e]));
          const float up = static_cast<float>(round_h(acc[i + kSwiGLUHalf / 16][j][e]));
          const float activated = static_cast<float>(round_h(x / (1.0f + expf(-x))));
          o[e] = round_h(activated * up);
        }
        const int col = tile * kSwiGLUHalf + 16 * i + 4 * g;
        *reinterpret_cast<half4_t*>(static_cast<_Float16*>(a.out) + static_cast<int64_t>(m) * width + col) = o;
      }
    } else {
#pragma unroll
      for (int i = 0; i < S::NTL; ++i) {
        const int col = tile * NT + 16 * i + 4 * g;
        if constexpr (E == kHalf) {
          half4_t o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = round_h(acc[i][j][e]);
          *reinterpret_cast<half4_t*>(static_cast<_Float16*>(a.out) + static_cast<int64_t>(m) * a.n + col) = o;
        } else {
          float* y = static_cast<float*>(a.out) + (static_cast<int64_t>(split) * a.m + m) * a.n;
          *reinterpret_cast<float4_t*>(y + col) = acc[i][j];
        }
      }
    }
  }
}

constexpr int kMaxDevices = 64;

// Raises a kernel's dynamic LDS limit once per device (on the current one), remembering
// the devices done in `done` (one bit each).
int raise_lds_limit(const void* kernel, int bytes, std::atomic<uint64_t>& done) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) {
    return set_error(PC_ERR_LAUNCH, "cannot determine the current device");
  }
  const uint64_t bit = uint64_t{1} << device;
  if (done.load(std::memory_order_acquire) & bit) return PC_OK;
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess) {
    return set_error(PC_ERR_LAUNCH, "cannot raise the GEMM's LDS limit to %d bytes", bytes);
  }
  done.fetch_or(bit, std::memory_order_acq_rel);
  return PC_OK;
}

template <int NT, int KC, int STAGES, int WAVES, Epilogue E>
int launch(GemmArgs a, int splits, hipStream_t s) {
  using S = Shape<NT, KC, STAGES, WAVES>;
  if (a.ksplit % KC != 0) {
    return set_error(PC_ERR_ARGUMENT, "k per split (%d) must be a multiple of %d", a.ksplit, KC);
  }
  auto kernel = gemm_m128_kernel<NT, KC, STAGES, WAVES, E>;
  static std::atomic<uint64_t> raised{0};
  if (int rc = raise_lds_limit(reinterpret_cast<const void*>(kernel), S::LDS, raised)) return rc;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(a.tiles * splits)), dim3(64 * WAVES), S::LDS, s, a.x, a.w, a.m,
                     a.n, a.k, a.ksplit, a.tiles, a.half_rows, a.out);
  return check_launch("gemm_m128");
}

}  // namespace

extern "C" {

int pc_gemm_m128(void* out, const void* x, const void* w, int32_t m, int32_t n, int32_t k, int32_t splits,
                 int32_t epilogue, void* stream) {
  if (!out || !x || !w) return set_error(PC_ERR_ARGUMENT, "null pointer");
  if (m < 1 || m > kMaxRows) return set_error(PC_ERR_ARGUMENT, "m = %d outside [1, %d]", m, kMaxRows);
  if (n < 1 || k < 1 || splits < 1) return set_error(PC_ERR_ARGUMENT, "n, k and splits must be positive");
  if (k % splits != 0) return set_error(PC_ERR_ARGUMENT, "k = %d not divisible into %d splits", k, splits);
  if (static_cast<int64_t>(n) * k > (int64_t{1} << 31) || static_cast<int64_t>(splits) * m * n > (int64_t{1} << 31)) {
    return set_error(PC_ERR_ARGUMENT, "GEMM of %d x %d x %d with %d splits too large", m, n, k, splits);
  }
  if (!aligned(out, 16) || !aligned(x, 16) || !aligned(w, 16)) {
    return set_error(PC_ERR_ARGUMENT, "out, x and w must be 16-byte aligned");
  }
  GemmArgs a;
  a.x = static_cast<const _Float16*>(x);
  a.w = static_cast<const _Float16*>(w);
  a.out = out;
  a.m = m;
  a.n = n;
  a.k = k;
  a.ksplit = k / splits;
  a.half_rows = 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  switch (epilogue) {
    case kPartials:
    case kHalf:
      if (epilogue == kHalf && splits != 1) return set_error(PC_ERR_ARGUMENT, "fp16 output needs one split");
      // 64-row tiles with eight waves when they alone fill the GPU's workgroup slots; with
      // four waves (2 x 4 register tiles per wave) when they give 160 to 175 workgroups, where
      // 32-row tiles would need more workgroups than one round on the CUs (q|k|v at 4
      // splits: 7.5 vs 8.3 us); else 32-row tiles with four waves.
      if (n % 64 == 0 && (n / 64) * splits >= 176) {
        a.tiles = n / 64;
        return epilogue == kHalf ? launch<64, 64, 4, 8, kHalf>(a, splits, s) : launch<64, 64, 4, 8, kPartials>(a, splits, s);
      }
      if (n % 64 == 0 && (n / 64) * splits >= 160 && (n / 32) * splits > 256) {
        a.tiles = n / 64;
        return epilogue == kHalf ? launch<64, 64, 4, 4, kHalf>(a, splits, s) : launch<64, 64, 4, 4, kPartials>(a, splits, s);
      }
      if (n % 32 != 0) return set_error(PC_ERR_ARGUMENT, "n = %d must be a multiple of 32", n);
      a.tiles = n / 32;
      return epilogue == kHalf ? launch<32, 64, 4, 4, kHalf>(a, splits, s) : launch<32, 64, 4, 4, kPartials>(a, splits, s);
    case kSwiGLU:
      if (splits != 1) return set_error(PC_ERR_ARGUMENT, "the SwiGLU epilogue needs one split");
      if (n % (2 * kSwiGLUHalf) != 0) return set_error(PC_ERR_ARGUMENT, "n = %d must be a multiple of 64", n);
      a.half_rows = n / 2;
      a.tiles = n / (2 * kSwiGLUHalf);
      return launch<64, 64, 4, 8, kSwiGLU>(a, splits, s);
    default:
      return set_error(PC_ERR_ARGUMENT, "unknown epilogue %d", epilogue);
  }
}

}  // extern "C"
