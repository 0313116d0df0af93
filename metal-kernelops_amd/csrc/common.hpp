// Shared device helpers for the gfx950 SSM scan kernels.
//
// Storage types: float, _Float16 and bf16 (raw 16-bit pattern).  Every kernel
// computes in float32 and rounds once on the store.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/mko.h"

namespace mko {

constexpr int kWave = 64;

struct bf16 {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(_Float16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f32(bf16 v) {
  return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float v) { return static_cast<_Float16>(v); }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) {
  // Round to nearest even; NaN stays a quiet NaN.
  uint32_t u = __float_as_uint(v);
  bf16 r;
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    r.bits = static_cast<uint16_t>((u >> 16) | 0x40u);
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    r.bits = static_cast<uint16_t>(u >> 16);
  }
  return r;
}

// 2^x on the transcendental unit (v_exp_f32).  Underflows to 0 for very negative
// x, which is the value every decay below wants.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

// torch's softplus rule (beta 1, threshold 20) in float32.  log1p(exp(v)) is
// evaluated with the library routines so a step of 1e-3 keeps its relative
// accuracy.
__device__ __forceinline__ float softplus(float v) {
  return v > 20.0f ? v : log1pf(expf(v));
}

// d softplus / dv with the same threshold: sigmoid(v), or 1 above 20.
__device__ __forceinline__ float softplus_grad(float v) {
  return v > 20.0f ? 1.0f : 1.0f / (1.0f + expf(-v));
}

__device__ __forceinline__ float sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

// Wave-uniform copy of a value (makes the compiler keep it in an SGPR).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Order this wave's LDS writes before its later LDS reads of other lanes' data.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace mko

// Error reporting for the C ABI (defined in abi.hip).
void mko_set_error(const char* fmt, ...);
int mko_check_launch(const char* what);
