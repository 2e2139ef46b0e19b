// Device helpers shared by the gfx950 kernels: 16-byte vector types, bf16 <-> fp32,
// wave64 reductions, and the launch-status plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/cpu_attention_hip.h"

namespace ca {

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

constexpr float kLog2e = 1.4426950408889634f;  // the reference's LOG2E (isa.mojo:58-62)
constexpr int kWave = 64;

// A 32-bit word as a bf16 pair.  Taking the word by value matters: hipcc (ROCm 7.2)
// folds __builtin_bit_cast applied directly to an ext_vector element expression
// (v.y, v.z, ...) onto element 0.
__device__ __forceinline__ bf16x2 as_bf16x2(uint32_t w) { return __builtin_bit_cast(bf16x2, w); }

// bf16 held as the high half of an fp32: widening is exact.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16, round to nearest even (the fptrunc the hardware implements as
// v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// Orders this wave's LDS writes before its later LDS reads by other lanes of the
// same wave (no other wave takes part).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__host__ __device__ constexpr int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Hardware dispatches workgroup i to XCD i % 8.  Remap so each XCD walks a
// contiguous range of the logical work ids: neighbouring work (one head's K/V,
// or neighbouring heads that share cache lines) then meets in one XCD's L2.
__host__ __device__ inline int64_t xcd_remap(int64_t bid, int64_t nb) {
  const int64_t x = bid & 7, slot = bid >> 3;
  const int64_t per = nb >> 3, rem = nb & 7;
  return x * per + (x < rem ? x : rem) + slot;
}

}  // namespace ca

// Host: turn the last launch's status into the ABI's return code.
static inline int ca_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? CA_OK : CA_HIP_ERROR - (int)e;
}
