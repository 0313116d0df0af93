// Mamba-2 decode step (selective state update), forward and backward, for gfx950.
//
// One workgroup per (batch, head): its headdim rows of dstate states are one
// contiguous block of the state tensor.  TPR lanes share a row and stride over
// it in 4-element vectors, so a wavefront's loads are contiguous 16-byte runs;
// the row's <new_state, C> is a butterfly over those TPR lanes.  delta and the
// decay are per (batch, head) (or per row when dt has a headdim axis).
//
// Backward: the same workgroup recomputes the new state (instead of re-reading it
// from memory), writes the row-local gradients, and reduces dB/dC over its rows
// and dA/dD/ddt over its rows in a fixed order; two more kernels sum the per-head
// partials over heads (dB/dC) and over batch (dA/dD/ddt_bias, one workgroup per head).  Every output
// has one writer, so the backward is bit-deterministic.
#include <mutex>
#include <vector>

#include "common.hpp"

namespace mko {
namespace su {

constexpr int kThreads = 256;
constexpr int kMaxPerThread = 16;  // states per lane: dstate / TPR <= 16

struct Geo {
  int64_t batch, nheads, headdim, dstate, ngroups;
  int tpr;  // lanes per row (power of two, <= 64)
  int vec;  // 4 if rows can use 4-element vector accesses, else 1
  int state_dtype, x_dtype, dt_dtype, bc_dtype;
  int softplus, dt_per_row, d_per_row;
};

struct Args {
  Geo g;
  const void* state;
  const void* x;
  const void* dt;
  const float* A;
  const void* B;
  const void* C;
  const float* D;
  const void* z;
  const float* dt_bias;
  void* new_state;
  void* y;
  const float* dy;
  const float* dnew;
  float* gstate;
  float* dx;
  float* ddt;
  float* dz;
  float* pb;    // (batch, nheads, dstate) dB partials per head
  float* pc;    // (batch, nheads, dstate) dC partials
  float* pa;    // (batch, nheads) dA partials
  float* pd;    // (batch, nheads) or (batch, nheads, headdim) dD partials
  float* pbias; // (batch, nheads) ddt_bias partials
};

template <typename T>
__device__ __forceinline__ void load4(const void* base, int64_t i, float (&v)[4]) {
  uint32_t w[kWordsOf<T, 4>];
  load_words(static_cast<const T*>(base) + i, w);
  unpack_words<T, 4>(w, v);
}

template <typename T>
__device__ __forceinline__ void store4(void* base, int64_t i, const float (&v)[4]) {
  uint32_t w[kWordsOf<T, 4>];
  pack_words<T, 4>(v, w);
  store_words(static_cast<T*>(base) + i, w);
}

template <typename T>
__device__ __forceinline__ float ld(const void* base, int64_t i) {
  return to_f32(static_cast<const T*>(base)[i]);
}

__device__ __forceinline__ float ld_any(const void* base, int dtype, int64_t i) {
  if (dtype == MKO_F32) return static_cast<const float*>(base)[i];
  if (dtype == MKO_BF16) return to_f32(static_cast<const bf16*>(base)[i]);
  return to_f32(static_cast<const _Float16*>(base)[i]);
}

// Element i of a float32, float16 or bfloat16 array chosen at run time, read without a branch
// and converted later: two 16-bit loads (the element's low half, and for float32 its high
// half; a 16-bit element is read twice rather than reading past it), and the conversion by
// selects.  A load under a run-time dtype branch makes the compiler wait at the join for every
// load in flight, and converting each value right after its load serialises the loads.
struct RawAny {
  uint32_t lo, hi;
};
__device__ __forceinline__ RawAny load_any_raw(const void* base, int dtype, int64_t i) {
  const bool f32 = dtype == MKO_F32;
  const uint16_t* p = reinterpret_cast<const uint16_t*>(static_cast<const char*>(base) + i * (f32 ? 4 : 2));
  return {p[0], p[f32 ? 1 : 0]};
}
__device__ __forceinline__ float raw_any_f32(RawAny r, int dtype) {
  const float as_f32 = __uint_as_float(r.lo | (r.hi << 16));
  const float as_bf16 = __uint_as_float(r.lo << 16);
  const float as_f16 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.lo)));
  return dtype == MKO_F32 ? as_f32 : (dtype == MKO_BF16 ? as_bf16 : as_f16);
}

// Elements of a row handled by lane j of its TPR lanes: vector chunks j, j+TPR, ...
// (VEC = 4) or single elements (VEC = 1), at most SPL of them.
template <int VEC, int SPL = kMaxPerThread, typename F>
__device__ __forceinline__ void for_row_chunks(int n_states, int tpr, int j, F&& f) {
#pragma unroll
  for (int k = 0; k < SPL / VEC; ++k) {
    const int n0 = (j + k * tpr) * VEC;
    if (n0 < n_states) f(k, n0);
  }
}

__device__ __forceinline__ float row_sum(float v, int tpr) {
  for (int off = tpr >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

template <typename T>
__device__ __forceinline__ void load4_nt(const void* base, int64_t i, float (&v)[4]) {
  uint32_t w[kWordsOf<T, 4>];
  load_words_nt(static_cast<const T*>(base) + i, w);
  unpack_words<T, 4>(w, v);
}

template <typename T>
__device__ __forceinline__ void store4_nt(void* base, int64_t i, const float (&v)[4]) {
  uint32_t w[kWordsOf<T, 4>];
  pack_words<T, 4>(v, w);
  store_words_nt(static_cast<T*>(base) + i, w);
}

// Passes (of kThreads / tpr rows) per forward workgroup: a workgroup streams 2 x 4 KB of an
// fp32 state.  One workgroup per whole (batch, head) (8 passes at d_state 128) streamed at
// 5.4 TB/s; two passes with their state rows requested before any arithmetic and the state
// read and written with the nontemporal hint, at 6.3 TB/s.
constexpr int kFwdPasses = 2;

// Sum over the tpr lanes of a row (tpr a power of two <= 64, uniform): an unrolled butterfly.
__device__ __forceinline__ float row_sum_pow2(float v, int tpr) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    if (off < tpr) v += __shfl_xor(v, off);
  return v;
}

// The forward when one 4-element vector per lane covers a row (tpr * 4 >= dstate).  Grid (row
// blocks of kFwdPasses passes, nheads, batch), so the head and batch need no division; lane
// arithmetic is shifts and masks of the power-of-two tpr; every array is addressed from a
// wave-uniform 64-bit base with a 32-bit lane offset.  Every load is issued unconditionally,
// from a clamped row and state (a lane past the row's states reads chunk 0, a pass past the
// head's rows reads its first row) and masked at use, and the per-row scalars are read
// without a dtype branch (load_any_raw): a load under a run-time condition makes the compiler
// wait for each load before the next, and 64-bit index division cost several hundred
// instructions per workgroup.  At c5 this runs at 6.3 TB/s, the rate of a nontemporal device
// copy, against 5.4 TB/s for one workgroup per (batch, head).
template <typename TS, typename TB>
__global__ void __launch_bounds__(kThreads) fwd_v4(Args a, int tpr_shift) {
  const Geo& g = a.g;
  const int h = static_cast<int>(blockIdx.y), b = static_cast<int>(blockIdx.z);
  const int H = static_cast<int>(g.nheads), P = static_cast<int>(g.headdim), N = static_cast<int>(g.dstate);
  const int gg = g.ngroups == 1 ? 0 : h / (H / static_cast<int>(g.ngroups));
  const int tpr = 1 << tpr_shift;
  const int j = static_cast<int>(threadIdx.x) & (tpr - 1);
  const int rows_per_pass = kThreads >> tpr_shift;
  const int prow0 = static_cast<int>(blockIdx.x) * kFwdPasses * rows_per_pass;  // the block's first row
  const int slot = static_cast<int>(threadIdx.x) >> tpr_shift;
  const int64_t head_row0 = (static_cast<int64_t>(b) * H + h) * P;  // the head's first row
  const bool nok = 4 * j < N;
  const int n0 = nok ? 4 * j : 0;
  const TB* Bb = static_cast<const TB*>(a.B) + (static_cast<int64_t>(b) * g.ngroups + gg) * N;
  const TB* Cb = static_cast<const TB*>(a.C) + (static_cast<int64_t>(b) * g.ngroups + gg) * N;
  const TS* sb = static_cast<const TS*>(a.state) + (head_row0 + prow0) * N;
  TS* nb = static_cast<TS*>(a.new_state) + (head_row0 + prow0) * N;
  float bv[4], cv[4];
  load4<TB>(Bb, n0, bv);
  load4<TB>(Cb, n0, cv);
  int prel[kFwdPasses];  // the pass's row within the block, clamped to a row of the head
  float sv[kFwdPasses][4];
#pragma unroll
  for (int q = 0; q < kFwdPasses; ++q) {
    const int r = q * rows_per_pass + slot;
    prel[q] = prow0 + r < P ? r : -prow0;
    load4_nt<TS>(sb, static_cast<uint32_t>(prel[q] * N + n0), sv[q]);
  }
  // the per-row scalars: every raw load issued before any of them is converted
  // (D as well: loaded in the epilogue it would wait for the previous pass's stores too, which
  // the vector memory counter also counts)
  const void* zsrc = a.z ? a.z : a.x;
  const float* dsrc = a.D ? a.D : a.A;
  RawAny rdt[kFwdPasses], rx[kFwdPasses], rz[kFwdPasses];
  float dv[kFwdPasses];
#pragma unroll
  for (int q = 0; q < kFwdPasses; ++q) {
    const int64_t row = head_row0 + prow0 + prel[q];
    rdt[q] = load_any_raw(a.dt, g.dt_dtype, g.dt_per_row ? row : static_cast<int64_t>(b) * H + h);
    rx[q] = load_any_raw(a.x, g.x_dtype, row);
    rz[q] = load_any_raw(zsrc, g.x_dtype, row);
    dv[q] = dsrc[a.D && g.d_per_row ? h * P + prow0 + prel[q] : h];
  }
  const float Ah = a.A[h];
  const float bias = a.dt_bias ? a.dt_bias[h] : 0.0f;
  float decay[kFwdPasses], dx[kFwdPasses], xv[kFwdPasses], zv[kFwdPasses];
#pragma unroll
  for (int q = 0; q < kFwdPasses; ++q) {
    float del = raw_any_f32(rdt[q], g.dt_dtype) + bias;
    if (g.softplus) del = softplus(del);
    decay[q] = expf(Ah * del);
    xv[q] = raw_any_f32(rx[q], g.x_dtype);
    dx[q] = del * xv[q];
    zv[q] = raw_any_f32(rz[q], g.x_dtype);
  }
#pragma unroll
  for (int q = 0; q < kFwdPasses; ++q) {
    const int r = q * rows_per_pass + slot;
    const bool pok = prow0 + r < P;
    float nv[4];
    float acc = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      nv[e] = fmaf(decay[q], sv[q][e], dx[q] * bv[e]);
      acc = fmaf(nv[e], cv[e], acc);
    }
    if (pok && nok) store4_nt<TS>(nb, static_cast<uint32_t>(r * N + n0), nv);
    acc = row_sum_pow2(nok ? acc : 0.0f, tpr);
    if (pok && j == 0) {
      const int p = prow0 + r;
      float out = acc;
      if (a.D) out = fmaf(dv[q], xv[q], out);
      if (a.z) out *= zv[q] * sigmoid(zv[q]);
      static_cast<TS*>(a.y)[head_row0 + p] = from_f32<TS>(out);
    }
  }
}

// Grid (batch * nheads, row blocks of kFwdPasses passes).  SPL: states per lane (tpr * SPL
// >= dstate); 4 when one 4-element vector per lane covers a row.
template <typename TS, int VEC, int SPL>
__global__ void __launch_bounds__(kThreads) fwd(Args a) {
  const Geo& g = a.g;
  const int64_t bh = blockIdx.x;
  const int64_t b = bh / g.nheads, h = bh % g.nheads;
  const int64_t bg = b * g.ngroups + h / (g.nheads / g.ngroups);
  const int N = static_cast<int>(g.dstate);
  const int tpr = g.tpr;
  const int j = threadIdx.x % tpr;
  const int rows_per_pass = kThreads / tpr;
  const int pfirst = static_cast<int>(blockIdx.y) * kFwdPasses * rows_per_pass + static_cast<int>(threadIdx.x) / tpr;
  const float Ah = a.A[h];
  const float bias = a.dt_bias ? a.dt_bias[h] : 0.0f;
  // this lane's B and C: the same for every row of the head
  float bvs[SPL], cvs[SPL];
  for_row_chunks<VEC, SPL>(N, tpr, j, [&](int k, int n0) {
    if constexpr (VEC == 4) {
      float b4[4], c4[4];
      if (g.bc_dtype == MKO_F32) { load4<float>(a.B, bg * N + n0, b4); load4<float>(a.C, bg * N + n0, c4); }
      else if (g.bc_dtype == MKO_BF16) { load4<bf16>(a.B, bg * N + n0, b4); load4<bf16>(a.C, bg * N + n0, c4); }
      else { load4<_Float16>(a.B, bg * N + n0, b4); load4<_Float16>(a.C, bg * N + n0, c4); }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bvs[k * 4 + e] = b4[e];
        cvs[k * 4 + e] = c4[e];
      }
    } else {
      bvs[k] = ld_any(a.B, g.bc_dtype, bg * N + n0);
      cvs[k] = ld_any(a.C, g.bc_dtype, bg * N + n0);
    }
  });
  // the state rows of every pass, requested before any arithmetic
  float sv[kFwdPasses][SPL];
#pragma unroll
  for (int q = 0; q < kFwdPasses; ++q) {
    const int p = pfirst + q * rows_per_pass;
    if (p >= g.headdim) continue;
    const int64_t row = bh * g.headdim + p;
    for_row_chunks<VEC, SPL>(N, tpr, j, [&](int k, int n0) {
      if constexpr (VEC == 4) {
        float s4[4];
        load4_nt<TS>(a.state, row * N + n0, s4);
#pragma unroll
        for (int e = 0; e < 4; ++e) sv[q][k * 4 + e] = s4[e];
      } else {
        sv[q][k] = ld<TS>(a.state, row * N + n0);
      }
    });
  }
#pragma unroll
  for (int q = 0; q < kFwdPasses; ++q) {
    const int p = pfirst + q * rows_per_pass;
    if (p >= g.headdim) continue;  // uniform over the row's tpr lanes (a row is whole in a wavefront)
    const int64_t row = bh * g.headdim + p;
    float del = ld_any(a.dt, g.dt_dtype, g.dt_per_row ? row : bh) + bias;
    if (g.softplus) del = softplus(del);
    const float decay = expf(Ah * del);
    const float xv = ld_any(a.x, g.x_dtype, row);
    const float dx = del * xv;
    float acc = 0.0f;
    for_row_chunks<VEC, SPL>(N, tpr, j, [&](int k, int n0) {
      if constexpr (VEC == 4) {
        float nv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          nv[e] = fmaf(decay, sv[q][k * 4 + e], dx * bvs[k * 4 + e]);
          acc = fmaf(nv[e], cvs[k * 4 + e], acc);
        }
        store4_nt<TS>(a.new_state, row * N + n0, nv);
      } else {
        const float nv = fmaf(decay, sv[q][k], dx * bvs[k]);
        static_cast<TS*>(a.new_state)[row * N + n0] = from_f32<TS>(nv);
        acc = fmaf(nv, cvs[k], acc);
      }
    });
    acc = row_sum(acc, tpr);
    if (j == 0) {
      float out = acc;
      if (a.D) out = fmaf(g.d_per_row ? a.D[h * g.headdim + p] : a.D[h], xv, out);
      if (a.z) {
        const float zv = ld_any(a.z, g.x_dtype, row);
        out *= zv * sigmoid(zv);
      }
      static_cast<TS*>(a.y)[row] = from_f32<TS>(out);
    }
  }
}

// SPL: states per lane (tpr * SPL >= dstate).  With 8 (two 4-element vectors per lane and
// row) the dB/dC accumulators take 16 registers instead of 32, so more waves share a SIMD,
// and each pass's rows are requested a pass ahead.
template <typename TS, int VEC, int SPL>
__global__ void __launch_bounds__(kThreads) bwd(Args a) {
  __shared__ float red[kThreads * SPL];  // [rows_per_pass][tpr * SPL] fold buffer
  __shared__ float rowv[3][kThreads];  // per-row dA, dD, ddt terms of the current 256-row window
  const Geo& g = a.g;
  // 32-bit index arithmetic (the grid is batch * nheads < 2^31 workgroups; tpr is a power of two)
  const uint32_t bh32 = blockIdx.x, H32 = static_cast<uint32_t>(g.nheads);
  const int64_t bh = bh32;
  const int64_t b = bh32 / H32, h = bh32 - static_cast<uint32_t>(b) * H32;
  const int64_t bg = b * g.ngroups + (g.ngroups == 1 ? 0 : static_cast<uint32_t>(h) / (H32 / static_cast<uint32_t>(g.ngroups)));
  const int N = static_cast<int>(g.dstate);
  const int tpr = g.tpr;
  const int tpr_shift = __builtin_ctz(static_cast<unsigned>(tpr));
  const int j = static_cast<int>(threadIdx.x) & (tpr - 1);
  const int slot = static_cast<int>(threadIdx.x) >> tpr_shift;
  const int rows_per_pass = kThreads >> tpr_shift;
  const float Ah = a.A[h];
  const float bias = a.dt_bias ? a.dt_bias[h] : 0.0f;
  float pb[SPL], pc[SPL];
#pragma unroll
  for (int k = 0; k < SPL; ++k) pb[k] = pc[k] = 0.0f;
  float sum_a = 0.0f, sum_d = 0.0f, sum_t = 0.0f;  // thread 0: per-head folds

  // This lane's elements of a row (chunk k of VEC at n0 = (j + k tpr) VEC, present when
  // n0 < N): B and C are the same for every row of the head and are loaded once; a row's
  // state and new-state adjoint are requested a pass ahead when a lane holds at most 8.
  constexpr bool kAhead = SPL <= 8;
  float bvs[SPL], cvs[SPL];
  // A pass's inputs: the state and new-state adjoint rows, and the row's raw scalars.  They are
  // all loaded unconditionally (from the last row for a slot past the head's rows, from chunk 0
  // for a chunk past the row's states; an absent optional input is read from an array of the
  // same shape and masked at use): a load under a run-time condition, or a scalar load issued
  // after the next pass's rows, makes the compiler wait for every load issued before it, which
  // drains the look-ahead.
  struct Row {
    float s[SPL], dn[SPL];
    RawAny dt, x, z;
    float dy, dv;
  };
  for_row_chunks<VEC, SPL>(N, tpr, j, [&](int k, int n0) {
    float* bv = bvs + k * VEC;
    float* cv = cvs + k * VEC;
    if constexpr (VEC == 4) {
      float b4[4], c4[4];
      if (g.bc_dtype == MKO_F32) { load4<float>(a.B, bg * N + n0, b4); load4<float>(a.C, bg * N + n0, c4); }
      else if (g.bc_dtype == MKO_BF16) { load4<bf16>(a.B, bg * N + n0, b4); load4<bf16>(a.C, bg * N + n0, c4); }
      else { load4<_Float16>(a.B, bg * N + n0, b4); load4<_Float16>(a.C, bg * N + n0, c4); }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bv[e] = b4[e];
        cv[e] = c4[e];
      }
    } else {
      bv[0] = ld_any(a.B, g.bc_dtype, bg * N + n0);
      cv[0] = ld_any(a.C, g.bc_dtype, bg * N + n0);
    }
  });
  const int P = static_cast<int>(g.headdim);
  const void* zsrc = a.z ? a.z : a.x;                // same shape and dtype as z
  const float* dysrc = a.dy ? a.dy : a.dx;           // same shape as dy (an output; masked)
  const float* dnsrc = a.dnew ? a.dnew : a.gstate;   // same shape as dnew (an output; masked)
  const float* dsrc = a.D ? a.D : a.A;
  // The state and the new-state adjoint stream through once, read with the nontemporal hint.
  auto fetch = [&](int p, Row& r) {
    const int pc = p < P ? p : P - 1;
    const int64_t row = bh * g.headdim + pc;
    r.dt = load_any_raw(a.dt, g.dt_dtype, g.dt_per_row ? row : bh);
    r.x = load_any_raw(a.x, g.x_dtype, row);
    r.z = load_any_raw(zsrc, g.x_dtype, row);
    r.dy = dysrc[row];
    r.dv = dsrc[a.D ? (g.d_per_row ? h * g.headdim + pc : h) : 0];
#pragma unroll
    for (int k = 0; k < SPL / VEC; ++k) {
      const int n0 = (j + k * tpr) * VEC;
      const int nc = n0 < N ? n0 : 0;
      float* s = r.s + k * VEC;
      float* dn = r.dn + k * VEC;
      if constexpr (VEC == 4) {
        load4_nt<TS>(a.state, row * N + nc, *reinterpret_cast<float(*)[4]>(s));
        load4_nt<float>(dnsrc, row * N + nc, *reinterpret_cast<float(*)[4]>(dn));
      } else {
        s[0] = ld<TS>(a.state, row * N + nc);
        dn[0] = dnsrc[row * N + nc];
      }
    }
  };
  Row cur, nxt;
  if constexpr (kAhead) fetch(slot, cur);

  // Passes are uniform over the workgroup (every thread runs every pass), so the
  // barriers below are reached by all threads.
  for (int p0 = 0; p0 < g.headdim; p0 += rows_per_pass) {
    const int p = p0 + slot;
    if constexpr (kAhead) {
      fetch(p + rows_per_pass, nxt);
    } else {
      fetch(p, cur);
    }
    if (p < g.headdim) {
      const int64_t row = bh * g.headdim + p;
      const float raw = raw_any_f32(cur.dt, g.dt_dtype) + bias;
      const float del = g.softplus ? softplus(raw) : raw;
      const float decay = expf(Ah * del);
      const float xv = raw_any_f32(cur.x, g.x_dtype);
      const float dxv = del * xv;
      const float dv = a.D ? cur.dv : 0.0f;
      const float dyv = a.dy ? cur.dy : 0.0f;
      float zv = 0.0f, sg = 1.0f, gate = 1.0f;
      if (a.z) {
        zv = raw_any_f32(cur.z, g.x_dtype);
        sg = sigmoid(zv);
        gate = zv * sg;
      }
      const float dyp = dyv * gate;  // grad of the pre-gate output
      float sx = 0.0f, sa = 0.0f, sy = 0.0f;
      for_row_chunks<VEC, SPL>(N, tpr, j, [&](int k, int n0) {
        const float* s = cur.s + k * VEC;
        float dn[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) dn[e] = a.dnew ? cur.dn[k * VEC + e] : 0.0f;
        const float* bv = bvs + k * VEC;
        const float* cv = cvs + k * VEC;
        float gs[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float nv = fmaf(decay, s[e], dxv * bv[e]);
          const float q = fmaf(dyp, cv[e], dn[e]);  // grad of the new state
          gs[e] = q * decay;
          pb[k * VEC + e] = fmaf(q, dxv, pb[k * VEC + e]);
          pc[k * VEC + e] = fmaf(dyp, nv, pc[k * VEC + e]);
          sx = fmaf(q, bv[e], sx);
          sa = fmaf(q, s[e], sa);
          sy = fmaf(nv, cv[e], sy);
        }
        if constexpr (VEC == 4) {
          store4_nt<float>(a.gstate, row * N + n0, gs);
        } else {
          a.gstate[row * N + n0] = gs[0];
        }
      });
      sx = row_sum_pow2(sx, tpr);
      sa = row_sum_pow2(sa, tpr);
      sy = row_sum_pow2(sy, tpr);
      if (j == 0) {
        a.dx[row] = fmaf(del, sx, dyp * dv);
        // delta enters through the drive (del x B) and the decay (exp(A del)).
        float dd = fmaf(xv, sx, sa * decay * Ah);
        if (g.softplus) dd *= softplus_grad(raw);
        if (g.dt_per_row) a.ddt[row] = dd;
        if (a.z && a.dz) {
          const float ypre = fmaf(xv, dv, sy);
          a.dz[row] = dyv * ypre * sg * (1.0f + zv * (1.0f - sg));
        }
        const float dD = dyp * xv;
        if (a.D && g.d_per_row) a.pd[row] = dD;
        const int rw = p % kThreads;  // the row's slot in its window
        rowv[0][rw] = sa * decay * del;  // dA contribution
        rowv[1][rw] = dD;
        rowv[2][rw] = dd;
      }
    }
    // At the end of a 256-row window (or of the rows), fold its per-row values: lane r of
    // the first wavefront adds rows r, r + 64, ... in order, then a fixed butterfly.
    const int pnext = p0 + rows_per_pass;
    if (pnext % kThreads == 0 || pnext >= g.headdim) {
      __syncthreads();
      if (threadIdx.x < kWave) {
        const int wbase = p0 - p0 % kThreads;
        const int nrows = min(static_cast<int>(g.headdim) - wbase, kThreads);
        float va = 0.0f, vd = 0.0f, vt = 0.0f;
        for (int r = threadIdx.x; r < nrows; r += kWave) {
          va += rowv[0][r];
          vd += rowv[1][r];
          vt += rowv[2][r];
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
          va += __shfl_xor(va, m);
          vd += __shfl_xor(vd, m);
          vt += __shfl_xor(vt, m);
        }
        if (threadIdx.x == 0) {
          sum_a += va;
          sum_d += vd;
          sum_t += vt;
        }
      }
      __syncthreads();
    }
    if constexpr (kAhead) cur = nxt;
  }
  // dB/dC: fold the lanes' per-state partials over the row slots in a fixed order.
  for (int which = 0; which < 2; ++which) {
    float* src = which == 0 ? pb : pc;
#pragma unroll
    for (int k = 0; k < SPL; ++k) red[slot * SPL * tpr + k * tpr + j] = src[k];
    __syncthreads();
    for (int n = threadIdx.x; n < N; n += kThreads) {
      // state n lives at chunk k = n / (tpr*VEC), lane j = (n / VEC) % tpr, element e = n % VEC
      const int k = n / (tpr * VEC);
      const int jj = (n / VEC) % tpr;
      const int e = n % VEC;
      float s = 0.0f;
      const int nslots = min(rows_per_pass, static_cast<int>(g.headdim));
      for (int r = 0; r < nslots; ++r) s += red[r * SPL * tpr + (k * VEC + e) * tpr + jj];
      (which == 0 ? a.pb : a.pc)[bh * N + n] = s;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    a.pa[bh] = sum_a;
    if (a.D && !g.d_per_row) a.pd[bh] = sum_d;
    if (a.pbias) a.pbias[bh] = sum_t;
    if (!g.dt_per_row) a.ddt[bh] = sum_t;
  }
}

// dB/dC: the per-head partials summed over the heads of a group.  A workgroup takes 64 states
// of one (batch, group); its four wavefronts each add a quarter of the group's heads in order
// (the loads issued eight at a time), and the quarters meet in a fixed order.
__global__ void __launch_bounds__(256) reduce_bc(Args a, float* dB, float* dC) {
  __shared__ float qs[2][4][64];
  const Geo& g = a.g;
  const int64_t N = g.dstate;
  const int64_t hpg = g.nheads / g.ngroups;
  const int64_t ntile = (N + 63) / 64;
  const int64_t bgi = blockIdx.x / ntile;
  const int64_t b = bgi / g.ngroups, gi = bgi % g.ngroups;
  const int nl = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int64_t n = (blockIdx.x % ntile) * 64 + nl;
  const int64_t k0 = q * hpg / 4, k1 = (q + 1) * hpg / 4;
  float sb = 0.0f, sc = 0.0f;
  if (n < N) {
    const int64_t base = (b * g.nheads + gi * hpg) * N + n;
    int64_t k = k0;
    for (; k + 8 <= k1; k += 8) {
      float vb[8], vc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        vb[e] = a.pb[base + (k + e) * N];
        vc[e] = a.pc[base + (k + e) * N];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sb += vb[e];
        sc += vc[e];
      }
    }
    for (; k < k1; ++k) {
      sb += a.pb[base + k * N];
      sc += a.pc[base + k * N];
    }
  }
  qs[0][q][nl] = sb;
  qs[1][q][nl] = sc;
  __syncthreads();
  if (q == 0 && n < N) {
    const int64_t i = bgi * N + n;
    dB[i] = (qs[0][0][nl] + qs[0][1][nl]) + (qs[0][2][nl] + qs[0][3][nl]);
    dC[i] = (qs[1][0][nl] + qs[1][1][nl]) + (qs[1][2][nl] + qs[1][3][nl]);
  }
}

// Sum over the workgroup's 256 threads in a fixed order (lane butterflies, then the four
// wavefronts in order); every thread gets the result.
__device__ __forceinline__ float block_sum(float v, float* wsum) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = v;
  __syncthreads();
  return (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
}

// dA, ddt_bias and dD: the per-(batch, head) partials summed over the batch, one workgroup
// per head.  Thread t adds batches t, t + 256, ... in order; the threads' sums then meet in
// a fixed tree.  A per-row D takes headdim columns x 4 batch quarters per pass.
__global__ void __launch_bounds__(256) reduce_heads(Args a, float* dA, float* dD, float* dbias) {
  __shared__ float wsum[4];
  __shared__ float part[4][64];
  const Geo& g = a.g;
  const int64_t h = blockIdx.x;
  const int t = threadIdx.x;
  float s = 0.0f, u = 0.0f, d = 0.0f;
  for (int64_t b = t; b < g.batch; b += 256) {
    s += a.pa[b * g.nheads + h];
    if (a.pbias) u += a.pbias[b * g.nheads + h];
    if (a.D && !g.d_per_row) d += a.pd[b * g.nheads + h];
  }
  s = block_sum(s, wsum);
  if (t == 0) dA[h] = s;
  if (dbias) {
    u = block_sum(u, wsum);
    if (t == 0) dbias[h] = u;
  }
  if (a.D && !g.d_per_row && dD) {
    d = block_sum(d, wsum);
    if (t == 0) dD[h] = d;
  }
  if (a.D && g.d_per_row && dD) {
    const int col = t & 63, quarter = t >> 6;
    for (int64_t p0 = 0; p0 < g.headdim; p0 += 64) {
      const int64_t pp = p0 + col;
      float v = 0.0f;
      if (pp < g.headdim)
        for (int64_t b = quarter; b < g.batch; b += 4) v += a.pd[(b * g.nheads + h) * g.headdim + pp];
      __syncthreads();
      part[quarter][col] = v;
      __syncthreads();
      if (quarter == 0 && pp < g.headdim)
        dD[h * g.headdim + pp] = (part[0][col] + part[1][col]) + (part[2][col] + part[3][col]);
    }
  }
}

inline size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

static int make_geo(const mko_state_update_params* p, Geo* g) {
  if (!p) {
    mko_set_error("state_update: null params");
    return MKO_EINVAL;
  }
  g->batch = p->batch;
  g->nheads = p->nheads;
  g->headdim = p->headdim;
  g->dstate = p->dstate;
  g->ngroups = p->ngroups;
  if (g->batch < 0 || g->nheads < 1 || g->headdim < 0 || g->dstate < 1 || g->ngroups < 1 ||
      g->nheads % g->ngroups) {
    mko_set_error("state_update: bad sizes");
    return MKO_EINVAL;
  }
  if (g->headdim > 65535 * 8) {  // the forward's row blocks of at least 8 rows are a grid axis
    mko_set_error("state_update: headdim=%lld > %d is not supported", (long long)g->headdim, 65535 * 8);
    return MKO_EUNSUPPORTED;
  }
  if (g->dstate > kMaxPerThread * 64) {
    mko_set_error("state_update: dstate=%lld > %d is not supported", (long long)g->dstate, kMaxPerThread * 64);
    return MKO_EUNSUPPORTED;
  }
  for (int dt : {p->state_dtype, p->x_dtype, p->dt_dtype, p->bc_dtype}) {
    if (dt != MKO_F32 && dt != MKO_F16 && dt != MKO_BF16) {
      mko_set_error("state_update: unknown dtype %d", dt);
      return MKO_EINVAL;
    }
  }
  int tpr = 1;
  while (tpr < 64 && tpr * kMaxPerThread < g->dstate) tpr <<= 1;
  g->tpr = tpr;
  g->state_dtype = p->state_dtype;
  g->x_dtype = p->x_dtype;
  g->dt_dtype = p->dt_dtype;
  g->bc_dtype = p->bc_dtype;
  g->softplus = (p->flags & MKO_SU_SOFTPLUS) ? 1 : 0;
  g->dt_per_row = (p->flags & MKO_SU_DT_PER_ROW) ? 1 : 0;
  g->d_per_row = (p->flags & MKO_SU_D_PER_ROW) ? 1 : 0;
  return MKO_OK;
}

static bool al(const void* q, int bytes) { return (reinterpret_cast<uintptr_t>(q) % bytes) == 0; }

static int pick_vec(const Geo& g, const mko_state_update_params* p, bool bwd) {
  const int ss = g.state_dtype == MKO_F32 ? 4 : 2;
  const int bs = g.bc_dtype == MKO_F32 ? 4 : 2;
  if (g.dstate % 4) return 1;
  if (!al(p->state, 4 * ss) || !al(p->B, 4 * bs) || !al(p->C, 4 * bs)) return 1;
  if (!bwd && !al(p->new_state, 4 * ss)) return 1;
  if (bwd && (!al(p->grad_state, 16) || (p->dnew_state && !al(p->dnew_state, 16)))) return 1;
  return 4;
}

}  // namespace su
}  // namespace mko

using namespace mko;
using namespace mko::su;

namespace {

// Lanes per row for one 4-element vector per lane, when a row needs at most 64 lanes.
static int tpr_one_vector(const Geo& g) {
  int tpr = 1;
  while (tpr < 64 && tpr * 4 < g.dstate) tpr <<= 1;
  return tpr * 4 >= g.dstate ? tpr : 0;
}

template <typename TS>
void launch_fwd_t(const Args& a, int vec, hipStream_t s, unsigned bh) {
  const int tpr4 = tpr_one_vector(a.g);
  Args f = a;
  // fwd_v4's grid has the heads and the batch as its y and z axes
  const bool v4 = vec == 4 && tpr4 && a.g.nheads <= 65535 && a.g.batch <= 65535;
  if (v4) f.g.tpr = tpr4;
  const int64_t rows_per_wg = static_cast<int64_t>(kFwdPasses) * (kThreads / f.g.tpr);
  const unsigned nrb = static_cast<unsigned>((a.g.headdim + rows_per_wg - 1) / rows_per_wg);
  if (v4) {
    const dim3 grid(nrb, static_cast<unsigned>(a.g.nheads), static_cast<unsigned>(a.g.batch));
    const int shift = __builtin_ctz(static_cast<unsigned>(tpr4));
    MKO_TIMED("state_update_fwd", s,
              if (a.g.bc_dtype == MKO_F32) fwd_v4<TS, float><<<grid, kThreads, 0, s>>>(f, shift);
              else if (a.g.bc_dtype == MKO_BF16) fwd_v4<TS, bf16><<<grid, kThreads, 0, s>>>(f, shift);
              else fwd_v4<TS, _Float16><<<grid, kThreads, 0, s>>>(f, shift));
    return;
  }
  const dim3 grid(bh, nrb);
  MKO_TIMED("state_update_fwd", s,
            if (vec == 4) fwd<TS, 4, kMaxPerThread><<<grid, kThreads, 0, s>>>(f);
            else fwd<TS, 1, kMaxPerThread><<<grid, kThreads, 0, s>>>(f));
}

// Lanes per row for two 4-element vectors per lane, when a row needs at most 64 lanes.
static int tpr_two_vectors(const Geo& g) {
  int tpr = 1;
  while (tpr < 64 && tpr * 8 < g.dstate) tpr <<= 1;
  return tpr * 8 >= g.dstate ? tpr : 0;
}

template <typename TS>
void launch_bwd_t(const Args& a, int vec, hipStream_t s, unsigned grid) {
  const int tpr8 = tpr_two_vectors(a.g);
  if (vec == 4 && tpr8) {
    Args b = a;
    b.g.tpr = tpr8;
    MKO_TIMED("state_update_bwd", s, bwd<TS, 4, 8><<<grid, kThreads, 0, s>>>(b));
  } else {
    MKO_TIMED("state_update_bwd", s,
              if (vec == 4) bwd<TS, 4, kMaxPerThread><<<grid, kThreads, 0, s>>>(a);
              else bwd<TS, 1, kMaxPerThread><<<grid, kThreads, 0, s>>>(a));
  }
}

Args base_args(const mko_state_update_params* p, const Geo& g) {
  Args a{};
  a.g = g;
  a.state = p->state;
  a.x = p->x;
  a.dt = p->dt;
  a.A = p->A;
  a.B = p->B;
  a.C = p->C;
  a.D = p->D;
  a.z = p->z;
  a.dt_bias = p->dt_bias;
  return a;
}

struct BwdLayout {
  size_t pb, pc, pa, pd, pbias, total;
};

BwdLayout bwd_layout(const Geo& g) {
  BwdLayout l{};
  const size_t bh = static_cast<size_t>(g.batch * g.nheads);
  size_t o = 0;
  l.pb = o; o = align_up(o + bh * g.dstate * 4);
  l.pc = o; o = align_up(o + bh * g.dstate * 4);
  l.pa = o; o = align_up(o + bh * 4);
  l.pd = o; o = align_up(o + bh * (g.headdim > 0 ? g.headdim : 1) * 4);
  l.pbias = o; o = align_up(o + bh * 4);
  l.total = o;
  return l;
}

}  // namespace

extern "C" int mko_state_update_fwd(const mko_state_update_params* p, void* stream) {
  Geo g;
  int st = make_geo(p, &g);
  if (st != MKO_OK) return st;
  if (g.batch == 0 || g.headdim == 0) return MKO_OK;
  if (!p->state || !p->x || !p->dt || !p->A || !p->B || !p->C || !p->new_state || !p->y) {
    mko_set_error("state_update_fwd: state, x, dt, A, B, C, new_state and y are required");
    return MKO_EINVAL;
  }
  g.vec = pick_vec(g, p, false);
  Args a = base_args(p, g);
  a.new_state = p->new_state;
  a.y = p->y;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>(g.batch * g.nheads);
  if (g.state_dtype == MKO_F32) launch_fwd_t<float>(a, g.vec, s, grid);
  else if (g.state_dtype == MKO_BF16) launch_fwd_t<bf16>(a, g.vec, s, grid);
  else launch_fwd_t<_Float16>(a, g.vec, s, grid);
  return mko_check_launch("state_update_fwd");
}

extern "C" size_t mko_state_update_bwd_workspace_size(const mko_state_update_params* p) {
  Geo g;
  if (make_geo(p, &g) != MKO_OK) return 0;
  return bwd_layout(g).total;
}

namespace {

// The checks and launches of the backward, with the per-head partials in `ws` (at least
// bwd_layout(g).total bytes of device memory on the stream's device).
int run_bwd(const mko_state_update_params* p, void* stream, char* ws, const Geo& geo) {
  Geo g = geo;
  const BwdLayout l = bwd_layout(g);
  g.vec = pick_vec(g, p, true);
  Args a = base_args(p, g);
  a.dy = p->dy;
  a.dnew = p->dnew_state;
  a.gstate = p->grad_state;
  a.dx = p->dx;
  a.ddt = p->ddt;
  a.dz = p->dz;
  a.pb = reinterpret_cast<float*>(ws + l.pb);
  a.pc = reinterpret_cast<float*>(ws + l.pc);
  a.pa = reinterpret_cast<float*>(ws + l.pa);
  a.pd = reinterpret_cast<float*>(ws + l.pd);
  a.pbias = p->dt_bias ? reinterpret_cast<float*>(ws + l.pbias) : nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>(g.batch * g.nheads);
  if (g.state_dtype == MKO_F32) launch_bwd_t<float>(a, g.vec, s, grid);
  else if (g.state_dtype == MKO_BF16) launch_bwd_t<bf16>(a, g.vec, s, grid);
  else launch_bwd_t<_Float16>(a, g.vec, s, grid);
  const int64_t nred = g.batch * g.ngroups * ((g.dstate + 63) / 64);
  if (nred > 0)
    MKO_TIMED("state_update_bwd_reduce", s,
              reduce_bc<<<static_cast<unsigned>(nred), 256, 0, s>>>(a, p->dB, p->dC));
  MKO_TIMED("state_update_bwd_reduce", s,
            reduce_heads<<<static_cast<unsigned>(g.nheads), 256, 0, s>>>(a, p->dA, p->dD, p->ddt_bias));
  return mko_check_launch("state_update_bwd");
}

// Sizes and pointers every backward call needs; MKO_OK with *empty set when there is
// nothing to launch.
int check_bwd(const mko_state_update_params* p, Geo* g, bool* empty) {
  int st = make_geo(p, g);
  if (st != MKO_OK) return st;
  if (!p->grad_state || !p->dx || !p->ddt || !p->dA || !p->dB || !p->dC) {
    mko_set_error("state_update_bwd: grad_state, dx, ddt, dA, dB and dC are required");
    return MKO_EINVAL;
  }
  if ((p->D && !p->dD) || (p->z && !p->dz) || (p->dt_bias && !p->ddt_bias)) {
    mko_set_error("state_update_bwd: dD/dz/ddt_bias are required when D/z/dt_bias are given");
    return MKO_EINVAL;
  }
  *empty = g->batch == 0 || g->headdim == 0;  // the caller zero-fills
  return MKO_OK;
}

// The partials of mko_state_update_bwd_static: one copy of this array per GPU, held until
// the process ends.  In host code `scratch` only names the symbol; its device address on
// each GPU comes from hipGetSymbolAddress (scratch_address) and is what kernels receive.
__device__ __align__(256) unsigned char scratch[MKO_SU_STATIC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
std::vector<void*> g_scratch_at;  // per device ordinal; null until first resolved

// The device address of `scratch` on the current device (resolved once per device).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess || dev < 0) {
    mko_set_error("state_update_bwd_static: no current device: %s", hipGetErrorString(err));
    return MKO_ELAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (static_cast<size_t>(dev) >= g_scratch_at.size()) g_scratch_at.resize(dev + 1, nullptr);
  if (!g_scratch_at[dev]) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr) {
      mko_set_error("state_update_bwd_static: scratch address on device %d: %s", dev, hipGetErrorString(err));
      return MKO_ELAUNCH;
    }
    g_scratch_at[dev] = ptr;
  }
  *out = g_scratch_at[dev];
  return MKO_OK;
}

}  // namespace

extern "C" int mko_state_update_bwd(const mko_state_update_params* p, void* stream) {
  Geo g;
  bool empty = false;
  int st = check_bwd(p, &g, &empty);
  if (st != MKO_OK || empty) return st;
  const size_t need = bwd_layout(g).total;
  if (!p->workspace || p->workspace_bytes < need) {
    mko_set_error("state_update_bwd: workspace of %zu bytes needed, %zu given", need, p->workspace_bytes);
    return MKO_EWORKSPACE;
  }
  return run_bwd(p, stream, static_cast<char*>(p->workspace), g);
}

extern "C" int mko_state_update_bwd_static(const mko_state_update_params* p, void* stream) {
  Geo g;
  bool empty = false;
  int st = check_bwd(p, &g, &empty);
  if (st != MKO_OK || empty) return st;
  const size_t need = bwd_layout(g).total;
  if (need > MKO_SU_STATIC_SCRATCH_BYTES) {
    mko_set_error("state_update_bwd_static: this problem needs %zu bytes of partials, more than the %zu-byte "
                  "static scratch (batch x nheads x (2 dstate + headdim + 2) floats must fit); call "
                  "mko_state_update_bwd with a workspace instead",
                  need, static_cast<size_t>(MKO_SU_STATIC_SCRATCH_BYTES));
    return MKO_EWORKSPACE;
  }
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) {
    mko_set_error("state_update_bwd_static: no current device");
    return MKO_ELAUNCH;
  }
  if (stream) {
    int sdev = -1;
    if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev) != hipSuccess || sdev != dev) {
      mko_set_error("state_update_bwd_static: the stream belongs to device %d, device %d is current", sdev, dev);
      return MKO_EINVAL;
    }
  }
  void* ws = nullptr;
  st = scratch_address(&ws);
  if (st != MKO_OK) return st;
  return run_bwd(p, stream, static_cast<char*>(ws), g);
}
