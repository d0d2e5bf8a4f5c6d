// Device helpers shared by the library's kernels (not part of the C ABI): vector types,
// cross-lane reductions over the four 16-lane groups of a wave, loads issued without
// compiler tracking, and the transposing LDS reads of 16-token V tiles.
#ifndef PAGEDCORE_PC_DEVICE_H
#define PAGEDCORE_PC_DEVICE_H

#include <hip/hip_runtime.h>

#include <stdint.h>

namespace pc_device {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));

// log2(e) / sqrt(64): turns a raw q.k difference into a base-2 exponent.
constexpr float kScoreToLog2 = 0.18033688011112042f;

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Max / sum over the 4 lanes l, l^16, l^32, l^48 (one q head's 4 token groups).
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

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

__device__ __forceinline__ __attribute__((address_space(3))) void* lds_ptr(char* p) {
  return (__attribute__((address_space(3))) void*)p;
}

// Dim group u (dims 16u..16u+15) of staged V row r sits at group position u ^ row_sel(r):
// the four rows one transposing read touches per 16 lanes land in four different 32 B bank
// groups, and so do the even and the odd rows of any eight.
__device__ __forceinline__ int row_sel(int r) { return (r + (r >> 2)) & 3; }

// The four transposing reads of one staged block (B operands of the four 16-dim tiles). The
// loads are written out so that the compiler does not treat them as waiting on the LDS DMA
// (it would wait for every outstanding load); the wave has waited for this block's DMA.
template <int kOff>
__device__ __forceinline__ void read_v_tiles(uint32_t base, uint32_t sel, short4_t& r0, short4_t& r1, short4_t& r2,
                                             short4_t& r3) {
  const uint32_t a0 = base + 32 * (0 ^ sel), a1 = base + 32 * (1 ^ sel), a2 = base + 32 * (2 ^ sel),
                 a3 = base + 32 * (3 ^ sel);
  asm volatile(
      "ds_read_b64_tr_b16 %0, %4 offset:%8\n\t"
      "ds_read_b64_tr_b16 %1, %5 offset:%8\n\t"
      "ds_read_b64_tr_b16 %2, %6 offset:%8\n\t"
      "ds_read_b64_tr_b16 %3, %7 offset:%8\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
      : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "i"(kOff)
      : "memory");
}

// 16 B at p and p + 64 B, issued without compiler tracking; wait_loads<N>() on the same
// registers (N = loads issued after them) makes them available.
__device__ __forceinline__ void load_pair(half8_t& x, half8_t& y, const _Float16* p) {
  asm volatile("global_load_dwordx4 %0, %2, off\n\tglobal_load_dwordx4 %1, %2, off offset:64"
               : "=&v"(x), "=&v"(y)
               : "v"(p)
               : "memory");
}

// Cache policy of loads that stream data read once per pass (the KV pool, decode weights):
// non-temporal (`nt`). Such streams are far larger than the caches; allocating them there
// only costs bandwidth (a load-only pass over the paged KV layout measured 11.9 us with `nt`
// against 13.2 us with the default policy, on the VGPR and the LDS DMA path alike).
// kStreamAux is the same bit as the cache-policy operand of __builtin_amdgcn_global_load_lds.
constexpr int kStreamAux = 2;

// load_pair with the streaming policy.
__device__ __forceinline__ void load_pair_stream(half8_t& x, half8_t& y, const _Float16* p) {
  asm volatile("global_load_dwordx4 %0, %2, off nt\n\tglobal_load_dwordx4 %1, %2, off offset:64 nt"
               : "=&v"(x), "=&v"(y)
               : "v"(p)
               : "memory");
}

template <int N>
__device__ __forceinline__ void wait_loads(half8_t& x, half8_t& y) {
  asm volatile("s_waitcnt vmcnt(%2)" : "+v"(x), "+v"(y) : "i"(N) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_loads4(half8_t& x, half8_t& y, half8_t& z, half8_t& t) {
  asm volatile("s_waitcnt vmcnt(%4)" : "+v"(x), "+v"(y), "+v"(z), "+v"(t) : "i"(N) : "memory");
}

}  // namespace pc_device

#endif  // PAGEDCORE_PC_DEVICE_H
