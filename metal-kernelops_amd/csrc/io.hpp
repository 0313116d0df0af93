// Per-lane runs of consecutive elements: a lane owns one row and reads or writes
// NB consecutive steps of it, as 16-byte vectors when the run is whole and
// aligned, element by element (masked) otherwise.  The element dtype is a
// runtime, wave-uniform value, so one kernel serves float32/float16/bfloat16.
#pragma once

#include "common.hpp"

namespace mko {

template <typename T, int NB>
__device__ __forceinline__ void load_run_t(const T* __restrict__ p, int nvalid, bool vec,
                                           float (&out)[NB]) {
  if (vec && nvalid >= NB) {
    constexpr int kWords = kWordsOf<T, NB>;
    static_assert(kWords % 4 == 0, "run must be a whole number of 16-byte vectors");
    uint32_t w[kWords];
    load_words(p, w);
    unpack_words<T, NB>(w, out);
  } else {
#pragma unroll
    for (int i = 0; i < NB; ++i) out[i] = (i < nvalid) ? to_f32(p[i]) : 0.0f;
  }
}

template <typename T, int NB>
__device__ __forceinline__ void store_run_t(T* __restrict__ p, int nvalid, bool vec,
                                            const float (&in)[NB]) {
  if (vec && nvalid >= NB) {
    uint32_t w[kWordsOf<T, NB>];
    pack_words<T, NB>(in, w);
    store_words(p, w);
  } else {
#pragma unroll
    for (int i = 0; i < NB; ++i)
      if (i < nvalid) p[i] = from_f32<T>(in[i]);
  }
}

// Runtime-dtype front ends.  `off` is an element offset into the array.
template <int NB>
__device__ __forceinline__ void load_run(const void* p, int dtype, int64_t off, int nvalid,
                                         bool vec, float (&out)[NB]) {
  if (dtype == MKO_F32)
    load_run_t<float, NB>(static_cast<const float*>(p) + off, nvalid, vec, out);
  else if (dtype == MKO_BF16)
    load_run_t<bf16, NB>(static_cast<const bf16*>(p) + off, nvalid, vec, out);
  else
    load_run_t<_Float16, NB>(static_cast<const _Float16*>(p) + off, nvalid, vec, out);
}

template <int NB>
__device__ __forceinline__ void store_run(void* p, int dtype, int64_t off, int nvalid, bool vec,
                                          const float (&in)[NB]) {
  if (dtype == MKO_F32)
    store_run_t<float, NB>(static_cast<float*>(p) + off, nvalid, vec, in);
  else if (dtype == MKO_BF16)
    store_run_t<bf16, NB>(static_cast<bf16*>(p) + off, nvalid, vec, in);
  else
    store_run_t<_Float16, NB>(static_cast<_Float16*>(p) + off, nvalid, vec, in);
}

__device__ __forceinline__ float load_one(const void* p, int dtype, int64_t i) {
  if (dtype == MKO_F32) return static_cast<const float*>(p)[i];
  if (dtype == MKO_BF16) return to_f32(static_cast<const bf16*>(p)[i]);
  return to_f32(static_cast<const _Float16*>(p)[i]);
}

__device__ __forceinline__ void store_one(void* p, int dtype, int64_t i, float v) {
  if (dtype == MKO_F32)
    static_cast<float*>(p)[i] = v;
  else if (dtype == MKO_BF16)
    static_cast<bf16*>(p)[i] = from_f32<bf16>(v);
  else
    static_cast<_Float16*>(p)[i] = from_f32<_Float16>(v);
}

inline int dtype_size(int dtype) { return dtype == MKO_F32 ? 4 : 2; }

}  // namespace mko
