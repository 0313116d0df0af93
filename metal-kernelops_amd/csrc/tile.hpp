// Staging of 64x64 operand tiles from HBM into LDS for the mma.hpp tile products.
//
// A thread of the 256-thread workgroup owns a 2-row x 8-column block of a tile:
// rows r0 = 2*(tid/8) and r0+1, columns c0 = 8*(tid%8) .. c0+7.  Eight lanes cover a
// 64-element row, so a wavefront's loads are whole 128-byte lines of 16-bit data.
// A block is loaded as raw 16-byte vectors (V8), converted to fp32 in registers,
// transformed (scaled, decayed, masked), then rounded to the operand type and
// written to LDS either as is ([row][col]) or transposed ([col][row], one word per
// row pair) -- the transposed form turns token-major HBM data into the
// K-contiguous layout the matrix cores read when the contraction runs over tokens.
#pragma once

#include "mma.hpp"

namespace mko {

__device__ __forceinline__ int blk_r0() { return 2 * static_cast<int>(threadIdx.x >> 3); }
__device__ __forceinline__ int blk_c0() { return 8 * static_cast<int>(threadIdx.x & 7); }

// Eight consecutive elements of T, raw.
// `mask` is all ones when the row lies inside its window and zero otherwise; every
// consumer applies it, so a load can be issued unconditionally and its result masked
// only when it is used (after the wait it needs anyway).
template <typename T>
struct V8 {
  static constexpr int kWords = static_cast<int>(sizeof(T)) * 2;
  uint32_t w[kWords];
  uint32_t mask;
};

template <typename T>
__device__ __forceinline__ void v8_zero(V8<T>& v) {
#pragma unroll
  for (int i = 0; i < V8<T>::kWords; ++i) v.w[i] = 0u;
  v.mask = 0u;
}

// Loads elements p[0 .. min(n, 8)) (zero beyond): 16-byte vectors when `vec` and the
// run is whole (p is then 16-byte aligned), element by element otherwise.
template <typename T>
__device__ __forceinline__ void v8_load(V8<T>& v, const T* p, int n, bool vec) {
  constexpr int W = V8<T>::kWords;
  v.mask = ~0u;
  if (vec && n >= 8) {
    load_words(p, v.w);
  } else {
#pragma unroll
    for (int i = 0; i < W; ++i) v.w[i] = 0u;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (e < n) {
        if constexpr (sizeof(T) == 4)
          v.w[e] = __builtin_bit_cast(uint32_t, p[e]);
        else
          v.w[e >> 1] |= static_cast<uint32_t>(__builtin_bit_cast(uint16_t, p[e])) << (16 * (e & 1));
      }
    }
  }
}

template <typename T>
__device__ __forceinline__ void v8_f32(const V8<T>& v, float (&f)[8]) {
  uint32_t w[V8<T>::kWords];
#pragma unroll
  for (int i = 0; i < V8<T>::kWords; ++i) w[i] = v.w[i] & v.mask;
  unpack_words<T, 8>(w, f);
}

// Stores 8 fp32 values as T at p (16-byte aligned when `vec`), or the first n of them.
template <typename T, bool NT = false>
__device__ __forceinline__ void v8_store(T* p, int n, bool vec, const float (&f)[8]) {
  if (vec && n >= 8) {
    uint32_t w[V8<T>::kWords];
    pack_words<T, 8>(f, w);
    if constexpr (NT)
      store_words_nt(p, w);
    else
      store_words(p, w);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e < n) p[e] = from_f32<T>(f[e]);
  }
}

// Writes the thread's block (row r0 = a, row r0+1 = b, columns c0..c0+7) into an LDS
// operand tile, as is or transposed.
template <typename TM, bool TRANS, int LD = tile_ld<TM>()>
__device__ __forceinline__ void put2x8(TM* dst, int r0, int c0, const float (&a)[8], const float (&b)[8]) {
  constexpr int ld = LD;
  if constexpr (sizeof(TM) == 2) {
    if constexpr (!TRANS) {
      *reinterpret_cast<uint4*>(dst + lds_idx<TM, LD>(r0, c0)) =
          make_uint4(pack2<TM>(a[0], a[1]), pack2<TM>(a[2], a[3]), pack2<TM>(a[4], a[5]), pack2<TM>(a[6], a[7]));
      *reinterpret_cast<uint4*>(dst + lds_idx<TM, LD>(r0 + 1, c0)) =
          make_uint4(pack2<TM>(b[0], b[1]), pack2<TM>(b[2], b[3]), pack2<TM>(b[4], b[5]), pack2<TM>(b[6], b[7]));
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        *reinterpret_cast<uint32_t*>(dst + lds_idx<TM, LD>(c0 + k, r0)) = pack2<TM>(a[k], b[k]);
    }
  } else {
    if constexpr (!TRANS) {
#pragma unroll
      for (int k = 0; k < 8; k += 2) {
        *reinterpret_cast<float2*>(dst + r0 * ld + c0 + k) = make_float2(a[k], a[k + 1]);
        *reinterpret_cast<float2*>(dst + (r0 + 1) * ld + c0 + k) = make_float2(b[k], b[k + 1]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) *reinterpret_cast<float2*>(dst + (c0 + k) * ld + r0) = make_float2(a[k], b[k]);
    }
  }
}

// Loads the thread's 2x8 block of a 64x64 window of a row-major view: window element
// (r, c) is base[r * ld + c] (base and ld uniform, (63 * ld + 63) * sizeof(T) < 2^32, so
// each lane's byte offset is one 32-bit value added to the scalar base); rows >= nrows and
// columns >= ncols read as zero.  VEC: whole 8-element runs, 16-byte aligned, and the
// loads are unconditional (a lane outside the window reads at offset 0 of the window, or
// of `safe`, any valid aligned address, when the window is empty, and discards it), so the
// number of loads in flight is static and the compiler can wait for exactly the ones it
// needs.  NT: with the nontemporal hint, for a window that no other workgroup reads again.
template <typename T, bool VEC, bool NT = false>
__device__ __forceinline__ void load_win(const T* base, int ld, int nrows, int ncols, V8<T> (&v)[2],
                                         const T* safe) {
  const int r0 = blk_r0(), c0 = blk_c0();
  // a window with no element starts anywhere: its lanes all read `safe`
  const T* wb = nrows > 0 && ncols > 0 ? base : safe;
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int r = r0 + rr;
    if constexpr (VEC) {
      const bool ok = r < nrows && c0 < ncols;
      const T* at = at_bytes(wb, opaque(ok ? static_cast<uint32_t>((r * ld + c0) * sizeof(T)) : 0u));
      if constexpr (NT)
        load_words_nt(at, v[rr].w);
      else
        load_words(at, v[rr].w);
      v[rr].mask = ok ? ~0u : 0u;
    } else {
      const int n = r < nrows ? ncols - c0 : 0;
      if (n > 0)
        v8_load(v[rr], base + (r * ld + c0), n, false);
      else
        v8_zero(v[rr]);
    }
  }
}

// Stores the thread's block (rows r0, r0+1 of a 64x64 window at base with row stride
// ld, under load_win's offset bound) as T, inside nrows x ncols.
template <typename T, bool VEC, bool NT = false>
__device__ __forceinline__ void store_win(T* base, int ld, int nrows, int ncols, const float (&a)[8],
                                          const float (&b)[8]) {
  const int r0 = blk_r0(), c0 = blk_c0();
  const int n = ncols - c0;
  if (r0 < nrows && n > 0) v8_store<T, NT>(at_bytes(base, static_cast<uint32_t>((r0 * ld + c0) * sizeof(T))), n, VEC, a);
  if (r0 + 1 < nrows && n > 0)
    v8_store<T, NT>(at_bytes(base, static_cast<uint32_t>(((r0 + 1) * ld + c0) * sizeof(T))), n, VEC, b);
}

// Stores row r0 + rr of the thread's block only.
template <typename T, bool VEC, bool NT = false>
__device__ __forceinline__ void store_win_row(T* base, int ld, int nrows, int ncols, int rr, const float (&a)[8]) {
  const int r = blk_r0() + rr, c0 = blk_c0();
  const int n = ncols - c0;
  if (r < nrows && n > 0) v8_store<T, NT>(at_bytes(base, static_cast<uint32_t>((r * ld + c0) * sizeof(T))), n, VEC, a);
}

// Writes the thread's raw block (rows a, b) into an LDS operand tile without conversion.
template <typename TM, bool TRANS, int LD = tile_ld<TM>()>
__device__ __forceinline__ void put_raw(TM* dst, int r0, int c0, const V8<TM>& a, const V8<TM>& b) {
  constexpr int ld = LD;
  constexpr int W = V8<TM>::kWords;
  uint32_t aw[W], bw[W];
#pragma unroll
  for (int i = 0; i < W; ++i) {
    aw[i] = a.w[i] & a.mask;
    bw[i] = b.w[i] & b.mask;
  }
  if constexpr (sizeof(TM) == 2) {
    if constexpr (!TRANS) {
      *reinterpret_cast<uint4*>(dst + lds_idx<TM, LD>(r0, c0)) = make_uint4(aw[0], aw[1], aw[2], aw[3]);
      *reinterpret_cast<uint4*>(dst + lds_idx<TM, LD>(r0 + 1, c0)) = make_uint4(bw[0], bw[1], bw[2], bw[3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // column 2i: low halves of a and b; column 2i+1: high halves
        *reinterpret_cast<uint32_t*>(dst + lds_idx<TM, LD>(c0 + 2 * i, r0)) = __builtin_amdgcn_perm(bw[i], aw[i], 0x05040100u);
        *reinterpret_cast<uint32_t*>(dst + lds_idx<TM, LD>(c0 + 2 * i + 1, r0)) =
            __builtin_amdgcn_perm(bw[i], aw[i], 0x07060302u);
      }
    }
  } else {
    if constexpr (!TRANS) {
#pragma unroll
      for (int k = 0; k < 8; k += 2) {
        *reinterpret_cast<uint2*>(dst + r0 * ld + c0 + k) = make_uint2(aw[k], aw[k + 1]);
        *reinterpret_cast<uint2*>(dst + (r0 + 1) * ld + c0 + k) = make_uint2(bw[k], bw[k + 1]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) *reinterpret_cast<uint2*>(dst + (c0 + k) * ld + r0) = make_uint2(aw[k], bw[k]);
    }
  }
}

// Runs n >= 1 stages of a tile product with two register sets of prefetched operands
// (the loads of stage k+2 are issued while stage k is multiplied) and a double-buffered
// LDS tile (one barrier per stage).  fetch(k, regs) issues the loads of stage k,
// put(k, regs) writes them to LDS buffer k & 1, mma(k) multiplies from that buffer.
// Prefetches are unconditional (past the end they repeat the last stage's loads), so
// the loads in flight at each put are the same on every path.
template <class Regs, class Fetch, class Put, class Mma>
__device__ __forceinline__ void pipeline2(int n, Regs& ra, Regs& rb, Fetch&& fetch, Put&& put, Mma&& mma) {
  const int last = n - 1;
  fetch(0, ra);
  fetch(1 < last ? 1 : last, rb);
  int k = 0;
  for (; k + 1 < n; k += 2) {
    put(k, ra);
    __syncthreads();
    fetch(k + 2 < last ? k + 2 : last, ra);
    mma(k);
    put(k + 1, rb);
    __syncthreads();
    fetch(k + 3 < last ? k + 3 : last, rb);
    mma(k + 1);
  }
  if (k < n) {
    put(k, ra);
    __syncthreads();
    mma(k);
  }
}

// f(Int<K>{}) for K = B .. E-1, each call with K a compile-time constant.
template <int K>
struct Int {
  static constexpr int value = K;
  __device__ constexpr operator int() const { return K; }
};
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(Int<B>{});
    static_for<B + 1, E>(f);
  }
}

// pipeline2 over a stage count known at compile time: every stage index is a constant, so
// a stage schedule that depends only on it compiles to straight-line code.
template <int N, class Regs, class Fetch, class Put, class Mma>
__device__ __forceinline__ void pipeline2_static(Regs (&r)[2], Fetch&& fetch, Put&& put, Mma&& mma) {
  fetch(Int<0>{}, r[0]);
  if constexpr (N > 1) fetch(Int<1>{}, r[1]);
  static_for<0, N>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    put(kc, r[k & 1]);
    __syncthreads();
    if constexpr (k + 2 < N) fetch(Int<k + 2>{}, r[k & 1]);
    mma(kc);
  });
}

// The same with D register sets: the loads of stage k + D are issued while stage k is
// multiplied, so each load has D stages of work to arrive.  For kernels whose occupancy
// LDS bounds at a few waves per SIMD, the registers are there and the latency is not
// otherwise hidden.
template <int N, int D, class Regs, class Fetch, class Put, class Mma>
__device__ __forceinline__ void pipeline_static(Regs (&r)[D], Fetch&& fetch, Put&& put, Mma&& mma) {
  static_for<0, (D < N ? D : N)>([&](auto kc) { fetch(kc, r[decltype(kc)::value]); });
  static_for<0, N>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    put(kc, r[k % D]);
    __syncthreads();
    if constexpr (k + D < N) fetch(Int<k + D>{}, r[k % D]);
    mma(kc);
  });
}

// As pipeline2, but the fetches past the last stage load stage n -- the epilogue's
// inputs -- instead of repeating stage n-1, and epi(regs) is called at the end with the
// set that holds them (even n: both do; odd n: rb).  Two call sites instead of a select
// keep both sets in registers.
template <class Regs, class Fetch, class Put, class Mma, class Epi>
__device__ __forceinline__ void pipeline2e(int n, Regs& ra, Regs& rb, Fetch&& fetch, Put&& put, Mma&& mma, Epi&& epi) {
  fetch(0, ra);
  fetch(1 < n ? 1 : n, rb);
  int k = 0;
  for (; k + 1 < n; k += 2) {
    put(k, ra);
    __syncthreads();
    fetch(k + 2 < n ? k + 2 : n, ra);
    mma(k);
    put(k + 1, rb);
    __syncthreads();
    fetch(k + 3 < n ? k + 3 : n, rb);
    mma(k + 1);
  }
  if (k < n) {
    put(k, ra);
    __syncthreads();
    mma(k);
    epi(rb);
  } else {
    epi(ra);
  }
}

// Reads the thread's block back from a 64x65 fp32 LDS tile written in the accumulator
// layout (acc_to_lds): a = row r0, b = row r0+1.
__device__ __forceinline__ void lds_block(const float* red, int r0, int c0, float (&a)[8], float (&b)[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    a[k] = red[r0 * 65 + c0 + k];
    b[k] = red[(r0 + 1) * 65 + c0 + k];
  }
}

// Lane exchange within rows of 16 lanes by a DPP control word (no LDS round trip).
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xf, 0xf, false));
}

// Sum over the 8 lanes that share a row pair (tid%8 varies): every one of them gets it,
// summed as ((v0+v1)+(v2+v3))+((v4+v5)+(v6+v7)).  DPP: quad_perm [1,0,3,2] and
// [2,3,0,1] swap neighbours and pairs, row_half_mirror (lane 7-i of each 8) brings in
// the other quad's sum.
__device__ __forceinline__ float row8_sum(float v) {
  v += dpp_f32<0xb1>(v);
  v += dpp_f32<0x4e>(v);
  v += dpp_f32<0x141>(v);
  return v;
}

}  // namespace mko
