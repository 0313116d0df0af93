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

// v as a finished fp32 value.  Every rounding to float16 in these kernels goes through it: it
// is rounded to fp32 first, then to float16.  Without it the compiler folds a product of
// a float16 and an fp32 value into one mixed-precision multiply-add (v_fma_mixlo_f16) that
// rounds the exact product once, and does so in some kernels and not in others.  The two
// roundings differ by one float16 unit where the fp32 product falls on a float16 tie, so the
// SSD backward's row and column sums that must cancel (gy . y~ against u . du, from the same
// rounded u, K and gy) would then not.
__device__ __forceinline__ float fp32_value(float v) {
  asm("" : "+v"(v));
  return v;
}

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float v) { return static_cast<_Float16>(fp32_value(v)); }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) {
  // Round to nearest even (v_cvt_pk_bf16_f32); NaN stays NaN.
  bf16 r;
  r.bits = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
  return r;
}

// ---- raw words
// Consecutive elements kept as the 32-bit words they occupy in memory: a 16-bit type holds
// elements 2i (low half) and 2i + 1 (high half) in word i, fp32 one element per word.  The
// kernels' vector loads, stores and conversions all go through these.

template <typename T, int NE>
constexpr int kWordsOf = NE * static_cast<int>(sizeof(T)) / 4;

// W words at p: 16-byte vectors when W is a multiple of 4, else one 8- or 4-byte access.
template <int W>
__device__ __forceinline__ void load_words(const void* p, uint32_t (&w)[W]) {
  if constexpr (W % 4 == 0) {
    const uint4* q = static_cast<const uint4*>(p);
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      const uint4 t = q[i];
      w[4 * i + 0] = t.x;
      w[4 * i + 1] = t.y;
      w[4 * i + 2] = t.z;
      w[4 * i + 3] = t.w;
    }
  } else if constexpr (W == 2) {
    const uint2 t = *static_cast<const uint2*>(p);
    w[0] = t.x;
    w[1] = t.y;
  } else {
    static_assert(W == 1, "16-byte vectors, or one 8- or 4-byte access");
    w[0] = *static_cast<const uint32_t*>(p);
  }
}

template <int W>
__device__ __forceinline__ void store_words(void* p, const uint32_t (&w)[W]) {
  if constexpr (W % 4 == 0) {
    uint4* q = static_cast<uint4*>(p);
#pragma unroll
    for (int i = 0; i < W / 4; ++i) q[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
  } else if constexpr (W == 2) {
    *static_cast<uint2*>(p) = make_uint2(w[0], w[1]);
  } else {
    static_assert(W == 1, "16-byte vectors, or one 8- or 4-byte access");
    *static_cast<uint32_t*>(p) = w[0];
  }
}

// The same accesses with the nontemporal hint (global_load/store ... nt): for streams that are
// read or written once and not reused from the caches, such as a decode step's state.  On
// this part a read-and-write stream runs about 8% faster with them (6.2 against 5.7 TB/s for
// a device copy at four 16-byte vectors per lane).
typedef uint32_t mko_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t mko_u32x2 __attribute__((ext_vector_type(2)));

template <int W>
__device__ __forceinline__ void load_words_nt(const void* p, uint32_t (&w)[W]) {
  if constexpr (W % 4 == 0) {
    const mko_u32x4* q = static_cast<const mko_u32x4*>(p);
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      const mko_u32x4 t = __builtin_nontemporal_load(q + i);
      w[4 * i + 0] = t.x;
      w[4 * i + 1] = t.y;
      w[4 * i + 2] = t.z;
      w[4 * i + 3] = t.w;
    }
  } else if constexpr (W == 2) {
    const mko_u32x2 t = __builtin_nontemporal_load(static_cast<const mko_u32x2*>(p));
    w[0] = t.x;
    w[1] = t.y;
  } else {
    static_assert(W == 1, "16-byte vectors, or one 8- or 4-byte access");
    w[0] = __builtin_nontemporal_load(static_cast<const uint32_t*>(p));
  }
}

template <int W>
__device__ __forceinline__ void store_words_nt(void* p, const uint32_t (&w)[W]) {
  if constexpr (W % 4 == 0) {
    mko_u32x4* q = static_cast<mko_u32x4*>(p);
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      const mko_u32x4 t = {w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
      __builtin_nontemporal_store(t, q + i);
    }
  } else if constexpr (W == 2) {
    const mko_u32x2 t = {w[0], w[1]};
    __builtin_nontemporal_store(t, static_cast<mko_u32x2*>(p));
  } else {
    static_assert(W == 1, "16-byte vectors, or one 8- or 4-byte access");
    __builtin_nontemporal_store(w[0], static_cast<uint32_t*>(p));
  }
}

// One element (2 or 4 bytes) with the nontemporal hint.
template <typename T>
__device__ __forceinline__ T load_nt(const T* p) {
  static_assert(sizeof(T) == 2 || sizeof(T) == 4, "16- or 32-bit elements");
  if constexpr (sizeof(T) == 2)
    return __builtin_bit_cast(T, __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(p)));
  else
    return __builtin_bit_cast(T, __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p)));
}
template <typename T>
__device__ __forceinline__ void store_nt(T* p, T v) {
  static_assert(sizeof(T) == 2 || sizeof(T) == 4, "16- or 32-bit elements");
  if constexpr (sizeof(T) == 2)
    __builtin_nontemporal_store(__builtin_bit_cast(uint16_t, v), reinterpret_cast<uint16_t*>(p));
  else
    __builtin_nontemporal_store(__builtin_bit_cast(uint32_t, v), reinterpret_cast<uint32_t*>(p));
}

// p advanced by off bytes.  With a wave-uniform p the access compiles to the scalar-base
// form of the global loads and stores (64-bit base in SGPRs, one 32-bit offset VGPR per
// lane) instead of a 64-bit address pair per lane.
template <typename T>
__device__ __forceinline__ T* at_bytes(T* p, uint32_t off) {
  return reinterpret_cast<T*>(reinterpret_cast<char*>(p) + off);
}
template <typename T>
__device__ __forceinline__ const T* at_bytes(const T* p, uint32_t off) {
  return reinterpret_cast<const T*>(reinterpret_cast<const char*>(p) + off);
}

// v, unchanged, as a value the optimiser cannot see through.  A byte offset passed through it
// stays a 32-bit value in one VGPR (the scalar-base form of at_bytes), where a select or a
// mask folded into it would otherwise be widened to a 64-bit address per lane.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm("" : "+v"(v));
  return v;
}

// The two 16-bit elements of a word as fp32 (exact).
template <typename T>
__device__ __forceinline__ void unpack2(uint32_t w, float& lo, float& hi) {
  if constexpr (__is_same(T, bf16)) {
    lo = __uint_as_float(w << 16);
    hi = __uint_as_float(w & 0xffff0000u);
  } else {
    lo = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
    hi = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
  }
}

// Two values rounded to nearest even in a 16-bit type, packed low first.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (__is_same(T, bf16)) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t t = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
    return __builtin_bit_cast(uint32_t, t);
  } else {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t t = {static_cast<_Float16>(fp32_value(a)), static_cast<_Float16>(fp32_value(b))};
    return __builtin_bit_cast(uint32_t, t);
  }
}

// NE elements of T from their words.
template <typename T, int NE>
__device__ __forceinline__ void unpack_words(const uint32_t* w, float (&f)[NE]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < NE; ++i) f[i] = __uint_as_float(w[i]);
  } else {
    static_assert(NE % 2 == 0, "16-bit elements come in word pairs");
#pragma unroll
    for (int i = 0; i < NE / 2; ++i) unpack2<T>(w[i], f[2 * i], f[2 * i + 1]);
  }
}

// NE fp32 values rounded to T, as words.
template <typename T, int NE>
__device__ __forceinline__ void pack_words(const float (&f)[NE], uint32_t* w) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < NE; ++i) w[i] = __float_as_uint(f[i]);
  } else {
    static_assert(NE % 2 == 0, "16-bit elements come in word pairs");
#pragma unroll
    for (int i = 0; i < NE / 2; ++i) w[i] = pack2<T>(f[2 * i], f[2 * i + 1]);
  }
}

// 2^x on the transcendental unit (v_exp_f32).  Underflows to 0 for very negative
// x, which is the value every decay below wants.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// exp(v) on the transcendental unit; relative error a few ulp for |v| <= 80.
__device__ __forceinline__ float fast_exp(float v) { return fast_exp2(v * kLog2e); }

// torch's softplus rule (beta 1, threshold 20): v above 20, else log1p(exp(v)).
// log1p(e) is Goldberg's log(u) * e / (u - 1) with u = fl(1 + e), which keeps the
// relative accuracy of small steps (v = -7 gives 1e-3) to a few ulp using the
// hardware log2/rcp.
__device__ __forceinline__ float softplus(float v) {
  const float e = fast_exp(v);
  const float u = 1.0f + e;
  const float r = (u == 1.0f) ? e : fast_log2(u) * kLn2 * (e * fast_rcp(u - 1.0f));
  return v > 20.0f ? v : r;
}

__device__ __forceinline__ float sigmoid(float v) { return fast_rcp(1.0f + fast_exp(-v)); }

// d softplus / dv with the same threshold: sigmoid(v), or 1 above 20.
__device__ __forceinline__ float softplus_grad(float v) { return v > 20.0f ? 1.0f : sigmoid(v); }

// The same derivative from the softplus value s = softplus(v): sigmoid(v) = 1 - e^{-s}
// exactly (and s = v > 20 gives 1 - e^{-20} = 1 in float).  Below 1/8 a 4-term series
// of 1 - e^{-s} avoids the cancellation (truncation s^4/120 relative).
__device__ __forceinline__ float softplus_grad_from_value(float s) {
  if (s < 0.125f) return s * (1.0f - s * (0.5f - s * (1.0f / 6.0f - s * (1.0f / 24.0f))));
  return 1.0f - fast_exp(-s);
}

// Pointer into the constant address space: loads through it with a wave-uniform
// address compile to scalar (SMEM) loads.
typedef const float __attribute__((address_space(4)))* cfptr;
__device__ __forceinline__ cfptr as_const(const float* p) { return (cfptr)(p); }

// s_waitcnt lgkmcnt(0) with vmcnt/expcnt left alone: retires outstanding scalar
// and LDS loads.  Issued before a prefetch, it keeps the compiler's own wait for
// the data in use from also waiting on the prefetch that follows.
__device__ __forceinline__ void wait_lgkm() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Wave-uniform copy of a value (makes the compiler keep it in an SGPR).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Order this wave's LDS writes before its later LDS reads of other lanes' data.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Sum over each 16-lane row of the wave; every lane of the row gets the same bits
// (each DPP step adds a value and its mirror, and float addition commutes).
// quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror.
__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xf, 0xf, false));
  return v;
}

// Sum over the whole wave, wave-uniform: the four row sums added in a fixed order.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}

// Records HIP events around the launches in its scope when kernel timing is on
// (mko_profile_enable); a no-op otherwise.
class ProfScope {
 public:
  ProfScope(const char* name, hipStream_t stream);
  ~ProfScope();
  ProfScope(const ProfScope&) = delete;
  ProfScope& operator=(const ProfScope&) = delete;

 private:
  hipStream_t stream_;
  hipEvent_t start_ = nullptr, stop_ = nullptr;
  int slot_ = -1;
};

}  // namespace mko

// Launch statement(s) timed under `name` when kernel timing is enabled.
#define MKO_TIMED(name, stream, ...)        \
  do {                                      \
    ::mko::ProfScope mko_scope_(name, stream); \
    __VA_ARGS__;                            \
  } while (0)

// Coordinates of a 3-D problem launched as a 1-D grid of nx * ny * nz workgroups.
// The dispatcher deals consecutive workgroups round-robin to the 8 XCDs of the
// chip, each with its own L2; the workgroup index is permuted so that
// consecutive logical indices (x fastest) run on one XCD and share its L2.
struct WgId {
  int x, y;
  int64_t z;
};
constexpr int kXcds = 8;
__device__ __forceinline__ WgId wg_id(int nx, int ny) {
  const int64_t total = gridDim.x, w = blockIdx.x;
  const int64_t per = total / kXcds;
  const int64_t lid = (w < per * kXcds) ? (w % kXcds) * per + w / kXcds : w;
  WgId r;
  r.x = static_cast<int>(lid % nx);
  const int64_t rest = lid / nx;
  r.y = static_cast<int>(rest % ny);
  r.z = rest / ny;
  return r;
}

// Error reporting for the C ABI (defined in abi.hip).
void mko_set_error(const char* fmt, ...);
int mko_check_launch(const char* what);
