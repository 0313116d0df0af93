// Mamba-2 SSD chunk scan backward for gfx950.
//
// With u_s = step_s x_s, K[l][s] = e^{cs_l - cs_s} CB[l][s] (s <= l), gy = dy * silu(z),
// S_in / S_out the states entering / leaving a chunk and G the adjoint of S_out:
//   gate        y~ = K u + e^{cs} C S_in^T recomputed; dz; gy; gy.y~ per token; dD partials
//   chunk_state local adjoint of S_in: sum_l e^{cs_l} gy_l (x) C_l
//   state_rev   per state element, backwards over chunks: G, dinitial and e^T <G, S_in>
//               (the transfer's part of the derivative with respect to the chunk's total decay T)
//   du          du = K^T gy + e^{T - cs_s} B_s G^T; dx = step du + D gy; per token x.du,
//               u.du and tau = u.du_state (the rest of the derivative with respect to T)
//   dcb         adjoint of C.B^T: sum over the heads of a group of (gy u^T) o e^{cs_l - cs_s}
//   dbc_state   state terms of dC (e^{cs} gy S_in) and dB (e^{T - cs} u G) summed over heads
//   dbc_final   dC = dCB B + state term, dB = dCB^T C + state term
//   finish      d cs = gy.y~ - u.du (+ sum tau + e^T <G, S_in> at the chunk end), reverse
//               cumsum, d step = A rcs + x.du, ddt, dA and ddt_bias partials
// d cs is a difference of row and column sums of the same pairwise terms, so both
// sides use the same rounded operands (gy and u as the matrix cores see them) and
// the cancellation between them is exact up to fp32 accumulation.
//   reduce      dA, ddt_bias, dD
// Every partial sum is reduced in a fixed order: the backward is deterministic.
#include <algorithm>

#include "ssd.hpp"

namespace mko {
namespace ssd {
namespace {

struct BwdLayout {
  size_t gy, dstates, dT, ya, dsx, ut, tau, pdD, dcb, pbc, pA, pbias, total;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

// Sum over the workgroup (256 threads); every thread gets the result.
__device__ __forceinline__ float block_sum(float v, float* wsum) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = v;
  __syncthreads();
  return (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
}

__device__ __forceinline__ int64_t xidx(const Geo& g, int64_t b, int64_t t, int64_t h, int64_t pc) {
  return ((b * g.length + t) * g.nheads + h) * g.headdim + pc;
}
__device__ __forceinline__ int64_t bcidx(const Geo& g, int64_t b, int64_t t, int64_t gg, int64_t n) {
  return ((b * g.length + t) * g.ngroups + gg) * g.dstate + n;
}

template <typename TM>
__global__ void __launch_bounds__(256) gate(Geo g, BwdPlan pl, Ptrs p) {
  __shared__ TM sa[LdsTile<TM>::elems], sb[LdsTile<TM>::elems];
  __shared__ float csr[64], css[64], eo[64];
  __shared__ float red[64 * 65];
  const int i = blockIdx.x % g.qb, pt = blockIdx.x / g.qb;
  const int c = blockIdx.y;
  const int64_t bh = blockIdx.z, b = bh / g.nheads, h = bh % g.nheads;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  f32x16 acc;
  chunk_out<TM>(g, p, acc, sa, sb, csr, css, eo, i, pt, c, bh);
  const int64_t tl0 = static_cast<int64_t>(c) * g.q + 64 * i;
  float va[16], vd[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t t = tl0 + acc_row(wm, lane, r);
    const int64_t pc = static_cast<int64_t>(pt) * 64 + acc_col(wn, lane);
    va[r] = vd[r] = 0.0f;
    if (t >= g.length || pc >= g.headdim) continue;
    const int64_t xi = xidx(g, b, t, h, pc);
    const float xv = load_one(p.x, g.x_dtype, xi);
    const float dyv = load_one(p.dy, g.x_dtype, xi);
    const float yt = acc[r];
    float gyv = dyv;
    if (p.z) {
      const float zv = load_one(p.z, g.x_dtype, xi);
      const float sg = sigmoid(zv);
      gyv = to_f32(from_f32<TM>(dyv * zv * sg));  // as stored for the other kernels
      float ypre = yt;
      if (p.D) ypre = fmaf(g.d_per_row ? p.D[h * g.headdim + pc] : p.D[h], xv, ypre);
      store_one(p.dz, g.x_dtype, xi, dyv * ypre * sg * fmaf(zv, 1.0f - sg, 1.0f));
      store_one(p.gyw, g.x_dtype, xi, gyv);
    }
    va[r] = gyv * yt;
    vd[r] = gyv * xv;
  }
  acc_to_lds(red, va, wm, wn, lane);
  __syncthreads();
  if (threadIdx.x < 64) {
    float s = 0.0f;
    for (int k = 0; k < 64; ++k) s += red[threadIdx.x * 65 + k];
    p.ya[((bh * g.nc + c) * pl.npt + pt) * g.q + 64 * i + threadIdx.x] = s;
  }
  if (p.D) {
    __syncthreads();
    acc_to_lds(red, vd, wm, wn, lane);
    __syncthreads();
    const int64_t pc = static_cast<int64_t>(pt) * 64 + threadIdx.x;
    if (threadIdx.x < 64 && pc < g.headdim) {
      float s = 0.0f;
      for (int k = 0; k < 64; ++k) s += red[k * 65 + threadIdx.x];
      p.pdD[(((b * g.nc + c) * g.qb + i) * g.nheads + h) * g.headdim + pc] = s;
    }
  }
}

// Backwards over the chunks, one thread per state element: G (the adjoint of the
// state leaving each chunk) over the local adjoints in dstates, e^T <G, S_in> per
// state block, and the adjoint of the initial state.
__global__ void __launch_bounds__(256) state_rev(Geo g, BwdPlan pl, Ptrs p) {
  __shared__ float wsum[4];
  const int64_t pn = g.headdim * g.dstate;
  const int blk = blockIdx.x;
  const int64_t e = static_cast<int64_t>(blk) * 256 + threadIdx.x;
  const bool valid = e < pn;
  const int64_t bh = blockIdx.y;
  float gv = (valid && p.dfinal) ? load_one(p.dfinal, g.x_dtype, bh * pn + e) : 0.0f;
  for (int c = g.nc - 1; c >= 0; --c) {
    const int64_t o = (bh * g.nc + c) * pn + e;
    const float eT = fast_exp(p.cs[(bh * g.nc + c) * g.q + g.q - 1]);
    const float dt = block_sum(valid ? gv * p.states[o] : 0.0f, wsum);
    if (threadIdx.x == 0) p.dT[(bh * g.nc + c) * pl.nblk + blk] = eT * dt;
    if (valid) {
      const float loc = p.dstates[o];
      p.dstates[o] = gv;
      gv = fmaf(eT, gv, loc);
    }
  }
  if (valid && p.dinit) store_one(p.dinit, g.x_dtype, bh * pn + e, gv);
}

// Row sums over the 64 columns of an accumulator-layout tile, through LDS; thread
// t < 64 returns row t.  Brackets its LDS use with workgroup barriers.
__device__ __forceinline__ float row_sums(float* red, const float* v, int wm, int wn, int lane) {
  __syncthreads();
  acc_to_lds(red, v, wm, wn, lane);
  __syncthreads();
  float s = 0.0f;
  if (threadIdx.x < 64)
    for (int k = 0; k < 64; ++k) s += red[threadIdx.x * 65 + k];
  return s;
}

template <typename TM>
__global__ void __launch_bounds__(256) du_kernel(Geo g, BwdPlan pl, Ptrs p) {
  __shared__ TM sa[LdsTile<TM>::elems], sb[LdsTile<TM>::elems];
  __shared__ float csr[64], css[64], ws[64], dls[64];
  __shared__ float red[64 * 65];
  const int j = blockIdx.x % g.qb, pt = blockIdx.x / g.qb;
  const int c = blockIdx.y;
  const int64_t bh = blockIdx.z, b = bh / g.nheads, h = bh % g.nheads, gg = h / g.hpg;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int64_t so = (bh * g.nc + c) * g.q;
  const int64_t ts0 = static_cast<int64_t>(c) * g.q + 64 * j;
  const float* cbt = p.cb + ((b * g.nc + c) * g.ngroups + gg) * g.q * g.q;
  if (threadIdx.x < 64) {
    const float T = p.cs[so + g.q - 1];
    css[threadIdx.x] = p.cs[so + 64 * j + threadIdx.x];
    ws[threadIdx.x] = fast_exp(T - css[threadIdx.x]);
    dls[threadIdx.x] = p.dl[so + 64 * j + threadIdx.x];
  }
  // u_s[p] as the matrix cores see it (rounded like the forward's operand) and x_s[p]
  float uv[16], xv[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t t = ts0 + acc_row(wm, lane, r);
    const int64_t pc = static_cast<int64_t>(pt) * 64 + acc_col(wn, lane);
    xv[r] = (t < g.length && pc < g.headdim) ? load_one(p.x, g.x_dtype, xidx(g, b, t, h, pc)) : 0.0f;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 16; ++r) uv[r] = to_f32(from_f32<TM>(dls[acc_row(wm, lane, r)] * xv[r]));
  f32x16 acc;
  zero(acc);
  // state part: du_state[s][p] = e^{T - cs_s} sum_n B_s[n] G[p][n]
  const float* gc = p.dstates + (bh * g.nc + c) * g.headdim * g.dstate;
  for (int n0 = 0; n0 < g.dstate; n0 += 64) {
    __syncthreads();
    stage<TM, false>(sa, [&](int s, int k) {  // A[s][n] = e^{T - cs_s} B_s[n]
      const int64_t t = ts0 + s;
      const int n = n0 + k;
      if (t >= g.length || n >= g.dstate) return 0.0f;
      return ws[s] * load_one(p.B, g.bc_dtype, bcidx(g, b, t, gg, n));
    });
    stage<TM, false>(sb, [&](int pp, int k) {  // Bt[p][n] = G[p][n]
      const int64_t pc = static_cast<int64_t>(pt) * 64 + pp;
      const int n = n0 + k;
      if (pc >= g.headdim || n >= g.dstate) return 0.0f;
      return gc[pc * g.dstate + n];
    });
    __syncthreads();
    mma_tile<TM>(acc, sa, sb, wm, wn, lane, 64);
  }
  const int64_t po = ((bh * g.nc + c) * pl.npt + pt) * g.q + 64 * j;
  {
    float v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = uv[r] * acc[r];
    const float tau = row_sums(red, v, wm, wn, lane);
    if (threadIdx.x < 64) p.tau[po + threadIdx.x] = tau;
  }
  // intra-chunk part: du[s][p] += sum_{l >= s} K[l][s] gy_l[p]
  for (int i = j; i < g.qb; ++i) {
    const int64_t tl0 = static_cast<int64_t>(c) * g.q + 64 * i;
    __syncthreads();
    if (threadIdx.x < 64) csr[threadIdx.x] = p.cs[so + 64 * i + threadIdx.x];
    __syncthreads();
    stage<TM, true>(sa, [&](int l, int s) {  // A[s][l] = K[l][s]
      if (64 * j + s > 64 * i + l) return 0.0f;
      return cbt[(64 * i + l) * g.q + 64 * j + s] * fast_exp(csr[l] - css[s]);
    });
    stage<TM, true>(sb, [&](int l, int pp) {  // Bt[p][l] = gy_l[p]
      const int64_t t = tl0 + l;
      const int64_t pc = static_cast<int64_t>(pt) * 64 + pp;
      if (t >= g.length || pc >= g.headdim) return 0.0f;
      return load_one(p.gy, g.x_dtype, xidx(g, b, t, h, pc));
    });
    __syncthreads();
    mma_tile<TM>(acc, sa, sb, wm, wn, lane, 64);
  }
  float vx[16], vu[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int s = acc_row(wm, lane, r);
    const int64_t t = ts0 + s;
    const int64_t pc = static_cast<int64_t>(pt) * 64 + acc_col(wn, lane);
    const float du = acc[r];
    vx[r] = xv[r] * du;
    vu[r] = uv[r] * du;
    if (t >= g.length || pc >= g.headdim) continue;
    const int64_t xi = xidx(g, b, t, h, pc);
    float dxv = dls[s] * du;
    if (p.D) dxv = fmaf(g.d_per_row ? p.D[h * g.headdim + pc] : p.D[h], load_one(p.gy, g.x_dtype, xi), dxv);
    store_one(p.dx, g.x_dtype, xi, dxv);
  }
  const float sx = row_sums(red, vx, wm, wn, lane);
  if (threadIdx.x < 64) p.dsx[po + threadIdx.x] = sx;
  const float su = row_sums(red, vu, wm, wn, lane);
  if (threadIdx.x < 64) p.ut[po + threadIdx.x] = su;
}

// Adjoint of C.B^T for one lower tile (i, j) of a chunk, summed over a block of the
// group's heads: sum_h (gy_i u_j^T) o e^{cs_l - cs_s}.
template <typename TM>
__global__ void __launch_bounds__(256) dcb_kernel(Geo g, BwdPlan pl, Ptrs p) {
  __shared__ TM sa[LdsTile<TM>::elems], sb[LdsTile<TM>::elems];
  __shared__ float csr[64], css[64], dls[64];
  const int pair = blockIdx.x / pl.hb1, hb = blockIdx.x % pl.hb1;
  int i = 0;
  while ((i + 1) * (i + 2) / 2 <= pair) ++i;
  const int j = pair - i * (i + 1) / 2;
  const int c = blockIdx.y / g.ngroups;
  const int64_t gg = blockIdx.y % g.ngroups, b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int64_t tl0 = static_cast<int64_t>(c) * g.q + 64 * i, ts0 = static_cast<int64_t>(c) * g.q + 64 * j;
  const int64_t h0 = gg * g.hpg + static_cast<int64_t>(hb) * pl.hpb1;
  const int64_t hend = (gg + 1) * g.hpg, h1 = h0 + pl.hpb1 < hend ? h0 + pl.hpb1 : hend;
  f32x16 dacc;
  zero(dacc);
  for (int64_t h = h0; h < h1; ++h) {
    const int64_t so = ((b * g.nheads + h) * g.nc + c) * g.q;
    __syncthreads();
    if (threadIdx.x < 64) {
      csr[threadIdx.x] = p.cs[so + 64 * i + threadIdx.x];
      css[threadIdx.x] = p.cs[so + 64 * j + threadIdx.x];
      dls[threadIdx.x] = p.dl[so + 64 * j + threadIdx.x];
    }
    f32x16 w;
    zero(w);
    for (int pt = 0; pt < pl.npt; ++pt) {
      __syncthreads();
      stage<TM, false>(sa, [&](int l, int pp) {  // A[l][p] = gy_l[p]
        const int64_t t = tl0 + l;
        const int64_t pc = static_cast<int64_t>(pt) * 64 + pp;
        if (t >= g.length || pc >= g.headdim) return 0.0f;
        return load_one(p.gy, g.x_dtype, xidx(g, b, t, h, pc));
      });
      stage<TM, false>(sb, [&](int s, int pp) {  // Bt[s][p] = step_s x_s[p]
        const int64_t t = ts0 + s;
        const int64_t pc = static_cast<int64_t>(pt) * 64 + pp;
        if (t >= g.length || pc >= g.headdim) return 0.0f;
        return dls[s] * load_one(p.x, g.x_dtype, xidx(g, b, t, h, pc));
      });
      __syncthreads();
      mma_tile<TM>(w, sa, sb, wm, wn, lane, 64);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int l = acc_row(wm, lane, r), s = acc_col(wn, lane);
      if (i != j || s <= l) dacc[r] = fmaf(w[r], fast_exp(csr[l] - css[s]), dacc[r]);
    }
  }
  float* out = p.dcb + (((b * g.nc + c) * g.ngroups + gg) * pl.hb1 + hb) * g.q * g.q;
#pragma unroll
  for (int r = 0; r < 16; ++r)
    out[(64 * i + acc_row(wm, lane, r)) * g.q + 64 * j + acc_col(wn, lane)] = dacc[r];
}

// State terms of dB (which 0: sum_h e^{T - cs_s} step_s x_s G) and dC (which 1:
// sum_h e^{cs_l} gy_l S_in) for one 64-token tile and one d_state tile, over a
// block of the group's heads.
template <typename TM>
__global__ void __launch_bounds__(256) dbc_state(Geo g, BwdPlan pl, Ptrs p) {
  __shared__ TM sa[LdsTile<TM>::elems], sb[LdsTile<TM>::elems];
  __shared__ float sc[64];
  int idx = blockIdx.x;
  const int hb = idx % pl.hb2;
  idx /= pl.hb2;
  const int which = idx % 2;
  idx /= 2;
  const int nt = idx % pl.nnt, tt = idx / pl.nnt;
  const int c = blockIdx.y / g.ngroups;
  const int64_t gg = blockIdx.y % g.ngroups, b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int64_t tl0 = static_cast<int64_t>(c) * g.q + 64 * tt;
  const int64_t h0 = gg * g.hpg + static_cast<int64_t>(hb) * pl.hpb2;
  const int64_t hend = (gg + 1) * g.hpg, h1 = h0 + pl.hpb2 < hend ? h0 + pl.hpb2 : hend;
  f32x16 acc;
  zero(acc);
  for (int64_t h = h0; h < h1; ++h) {
    const int64_t bh = b * g.nheads + h;
    const int64_t so = (bh * g.nc + c) * g.q;
    __syncthreads();
    if (threadIdx.x < 64) {
      const float cl = p.cs[so + 64 * tt + threadIdx.x];
      sc[threadIdx.x] = which ? fast_exp(cl) : p.dl[so + 64 * tt + threadIdx.x] * fast_exp(p.cs[so + g.q - 1] - cl);
    }
    const void* src = which ? p.gy : p.x;
    const float* st = (which ? p.states : p.dstates) + (bh * g.nc + c) * g.headdim * g.dstate;
    for (int pt = 0; pt < pl.npt; ++pt) {
      __syncthreads();
      stage<TM, false>(sa, [&](int l, int pp) {  // A[l][p]
        const int64_t t = tl0 + l;
        const int64_t pc = static_cast<int64_t>(pt) * 64 + pp;
        if (t >= g.length || pc >= g.headdim) return 0.0f;
        return sc[l] * load_one(src, g.x_dtype, xidx(g, b, t, h, pc));
      });
      stage<TM, true>(sb, [&](int pp, int n) {  // Bt[n][p] = S[p][n]
        const int64_t pc = static_cast<int64_t>(pt) * 64 + pp;
        const int64_t nn = static_cast<int64_t>(nt) * 64 + n;
        if (pc >= g.headdim || nn >= g.dstate) return 0.0f;
        return st[pc * g.dstate + nn];
      });
      __syncthreads();
      mma_tile<TM>(acc, sa, sb, wm, wn, lane, 64);
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t t = tl0 + acc_row(wm, lane, r);
    const int64_t nn = static_cast<int64_t>(nt) * 64 + acc_col(wn, lane);
    if (t >= g.length || nn >= g.dstate) continue;
    p.pbc[((((b * g.length + t) * g.ngroups + gg) * pl.hb2 + hb) * 2 + which) * g.dstate + nn] = acc[r];
  }
}

// dC = dCB B (which 1) and dB = dCB^T C (which 0) for one 64-token tile and one
// d_state tile, plus the head-block partials of the state terms.
template <typename TM>
__global__ void __launch_bounds__(256) dbc_final(Geo g, BwdPlan pl, Ptrs p) {
  __shared__ TM sa[LdsTile<TM>::elems], sb[LdsTile<TM>::elems];
  int idx = blockIdx.x;
  const int which = idx % 2;
  idx /= 2;
  const int nt = idx % pl.nnt, tt = idx / pl.nnt;
  const int c = blockIdx.y / g.ngroups;
  const int64_t gg = blockIdx.y % g.ngroups, b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int64_t qq = static_cast<int64_t>(g.q) * g.q;
  const float* dcb = p.dcb + ((b * g.nc + c) * g.ngroups + gg) * pl.hb1 * qq;
  auto dcb_at = [&](int l, int s) {  // sum over head blocks of dCB[l][s]
    float v = 0.0f;
    for (int k = 0; k < pl.hb1; ++k) v += dcb[k * qq + static_cast<int64_t>(l) * g.q + s];
    return v;
  };
  const int64_t nn0 = static_cast<int64_t>(nt) * 64;
  f32x16 acc;
  zero(acc);
  if (which) {
    for (int j = 0; j <= tt; ++j) {
      const int64_t ts0 = static_cast<int64_t>(c) * g.q + 64 * j;
      __syncthreads();
      stage<TM, false>(sa, [&](int l, int s) {  // A[l][s] = dCB[l][s]
        if (64 * j + s > 64 * tt + l) return 0.0f;
        return dcb_at(64 * tt + l, 64 * j + s);
      });
      stage<TM, true>(sb, [&](int s, int n) {  // Bt[n][s] = B_s[n]
        const int64_t t = ts0 + s;
        if (t >= g.length || nn0 + n >= g.dstate) return 0.0f;
        return load_one(p.B, g.bc_dtype, bcidx(g, b, t, gg, nn0 + n));
      });
      __syncthreads();
      mma_tile<TM>(acc, sa, sb, wm, wn, lane, 64);
    }
  } else {
    for (int i = tt; i < g.qb; ++i) {
      const int64_t tl0 = static_cast<int64_t>(c) * g.q + 64 * i;
      __syncthreads();
      stage<TM, true>(sa, [&](int l, int s) {  // A[s][l] = dCB[l][s]
        if (64 * tt + s > 64 * i + l) return 0.0f;
        return dcb_at(64 * i + l, 64 * tt + s);
      });
      stage<TM, true>(sb, [&](int l, int n) {  // Bt[n][l] = C_l[n]
        const int64_t t = tl0 + l;
        if (t >= g.length || nn0 + n >= g.dstate) return 0.0f;
        return load_one(p.C, g.bc_dtype, bcidx(g, b, t, gg, nn0 + n));
      });
      __syncthreads();
      mma_tile<TM>(acc, sa, sb, wm, wn, lane, 64);
    }
  }
  const int64_t t0 = static_cast<int64_t>(c) * g.q + 64 * tt;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t t = t0 + acc_row(wm, lane, r);
    const int64_t nn = nn0 + acc_col(wn, lane);
    if (t >= g.length || nn >= g.dstate) continue;
    float v = acc[r];
    const float* part = p.pbc + (((b * g.length + t) * g.ngroups + gg) * pl.hb2 * 2 + which) * g.dstate + nn;
    for (int k = 0; k < pl.hb2; ++k) v += part[static_cast<int64_t>(k) * 2 * g.dstate];
    store_one(which ? p.dC : p.dB, g.bc_dtype, bcidx(g, b, t, gg, nn), v);
  }
}

// Per (b, h, chunk), one thread per token in reverse order: d cs, its reverse
// cumulative sum, d step, ddt, and the dA / ddt_bias partials.
__global__ void __launch_bounds__(256) finish(Geo g, BwdPlan pl, Ptrs p) {
  __shared__ float wsum[4];
  const int c = blockIdx.x;
  const int64_t h = blockIdx.y, b = blockIdx.z, bh = b * g.nheads + h;
  const int tid = threadIdx.x;
  const bool active = tid < g.q;
  const int l = g.q - 1 - tid;
  const int64_t so = (bh * g.nc + c) * g.q;
  float dcs = 0.0f, dsxv = 0.0f, del = 0.0f, tau = 0.0f;
  if (active) {
    for (int pt = 0; pt < pl.npt; ++pt) {
      const int64_t o = ((bh * g.nc + c) * pl.npt + pt) * g.q + l;
      dcs += p.ya[o] - p.ut[o];
      dsxv += p.dsx[o];
      tau += p.tau[o];
    }
    del = p.dl[so + l];
  }
  // d T = sum_s tau_s + e^T <G, S_in>, at the chunk's last position
  const float tau_sum = block_sum(tau, wsum);
  if (active && l == g.q - 1) {
    dcs += tau_sum;
    for (int k = 0; k < pl.nblk; ++k) dcs += p.dT[(bh * g.nc + c) * pl.nblk + k];
  }
  __syncthreads();
  // inclusive scan in thread order = suffix sum over the chunk positions
  float v = dcs;
  for (int off = 1; off < kWave; off <<= 1) {
    const float n = __shfl_up(v, off);
    if ((tid & 63) >= off) v += n;
  }
  if ((tid & 63) == 63) wsum[tid >> 6] = v;
  __syncthreads();
  for (int w = 0; w < (tid >> 6); ++w) v += wsum[w];
  const float rcs = v;
  const float ddel = fmaf(p.A[h], rcs, dsxv);
  const int64_t t = static_cast<int64_t>(c) * g.q + l;
  float dd = 0.0f;
  if (active && t < g.length) {
    const int64_t o = (b * g.length + t) * g.nheads + h;
    float raw = load_one(p.dt, g.dt_dtype, o);
    if (p.bias) raw += p.bias[h];
    dd = g.softplus ? ddel * softplus_grad(raw) : ddel;
    store_one(p.ddt, g.dt_dtype, o, dd);
  }
  __syncthreads();
  const float sa = block_sum(del * rcs, wsum);
  const float sb = block_sum(dd, wsum);
  if (tid == 0) {
    p.pA[bh * g.nc + c] = sa;
    p.pbias[bh * g.nc + c] = sb;
  }
}

__global__ void __launch_bounds__(256) reduce_params(Geo g, BwdPlan pl, Ptrs p) {
  __shared__ float wsum[4];
  const int64_t h = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t nbc = g.batch * g.nc;
  float sa = 0.0f, sb = 0.0f;
  for (int64_t k = tid; k < nbc; k += 256) {
    const int64_t o = ((k / g.nc) * g.nheads + h) * g.nc + k % g.nc;
    sa += p.pA[o];
    sb += p.pbias[o];
  }
  sa = block_sum(sa, wsum);
  sb = block_sum(sb, wsum);
  if (tid == 0) {
    p.dA[h] = sa;
    if (p.dbias) p.dbias[h] = sb;
  }
  if (!p.dD) return;
  const int64_t nrow = nbc * g.qb;  // (b, chunk, tile) partial rows
  if (g.d_per_row) {
    for (int64_t pc = tid; pc < g.headdim; pc += 256) {
      float s = 0.0f;
      for (int64_t k = 0; k < nrow; ++k) s += p.pdD[(k * g.nheads + h) * g.headdim + pc];
      p.dD[h * g.headdim + pc] = s;
    }
  } else {
    float s = 0.0f;
    for (int64_t pc = tid; pc < g.headdim; pc += 256)
      for (int64_t k = 0; k < nrow; ++k) s += p.pdD[(k * g.nheads + h) * g.headdim + pc];
    s = block_sum(s, wsum);
    if (tid == 0) p.dD[h] = s;
  }
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

BwdPlan make_plan(const Geo& g) {
  BwdPlan pl{};
  pl.npt = static_cast<int>(cdiv(g.headdim, 64));
  pl.nnt = static_cast<int>(cdiv(g.dstate, 64));
  pl.nblk = static_cast<int>(cdiv(g.headdim * g.dstate, 256));
  pl.npairs = g.qb * (g.qb + 1) / 2;
  // Split the head sums so each launch has about 2048 workgroups.
  const int64_t base1 = std::max<int64_t>(1, g.batch * g.nc * g.ngroups * pl.npairs);
  pl.hb1 = static_cast<int>(std::min<int64_t>(g.hpg, std::max<int64_t>(1, cdiv(2048, base1))));
  pl.hpb1 = static_cast<int>(cdiv(g.hpg, pl.hb1));
  pl.hb1 = static_cast<int>(cdiv(g.hpg, pl.hpb1));
  const int64_t base2 = std::max<int64_t>(1, g.batch * g.nc * g.ngroups * g.qb * pl.nnt * 2);
  pl.hb2 = static_cast<int>(std::min<int64_t>(g.hpg, std::max<int64_t>(1, cdiv(2048, base2))));
  pl.hpb2 = static_cast<int>(cdiv(g.hpg, pl.hb2));
  pl.hb2 = static_cast<int>(cdiv(g.hpg, pl.hpb2));
  return pl;
}

BwdLayout bwd_layout(const Geo& g, const BwdPlan& pl, bool has_z) {
  BwdLayout l{};
  const size_t bh = static_cast<size_t>(g.batch * g.nheads);
  const size_t chunks = bh * g.nc;
  size_t o = 0;
  l.gy = o; o = align256(o + (has_z ? static_cast<size_t>(g.batch * g.length * g.nheads * g.headdim) * dtype_size(g.x_dtype) : 0));
  l.dstates = o; o = align256(o + chunks * g.headdim * g.dstate * 4);
  l.dT = o; o = align256(o + chunks * pl.nblk * 4);
  l.ya = o; o = align256(o + chunks * pl.npt * g.q * 4);
  l.dsx = o; o = align256(o + chunks * pl.npt * g.q * 4);
  l.ut = o; o = align256(o + chunks * pl.npt * g.q * 4);
  l.tau = o; o = align256(o + chunks * pl.npt * g.q * 4);
  l.pdD = o; o = align256(o + chunks * g.qb * g.headdim * 4);
  l.dcb = o; o = align256(o + static_cast<size_t>(g.batch) * g.nc * g.ngroups * pl.hb1 * g.q * g.q * 4);
  l.pbc = o; o = align256(o + static_cast<size_t>(g.batch * g.length * g.ngroups) * pl.hb2 * 2 * g.dstate * 4);
  l.pA = o; o = align256(o + chunks * 4);
  l.pbias = o; o = align256(o + chunks * 4);
  l.total = o;
  return l;
}

template <typename TM>
void launch_bwd_t(const Geo& g, const BwdPlan& pl, const Ptrs& q, hipStream_t s) {
  const unsigned bh = static_cast<unsigned>(g.batch * g.nheads);
  const unsigned ncg = static_cast<unsigned>(g.nc * g.ngroups);
  MKO_TIMED("ssd_gate", s, gate<TM><<<dim3(g.qb * pl.npt, g.nc, bh), 256, 0, s>>>(g, pl, q));
  MKO_TIMED("ssd_chunk_state_bwd", s,
            chunk_state<TM, true><<<dim3(pl.npt * pl.nnt, g.nc, bh), 256, 0, s>>>(g, q, q.dstates));
  MKO_TIMED("ssd_state_rev", s, state_rev<<<dim3(pl.nblk, bh), 256, 0, s>>>(g, pl, q));
  MKO_TIMED("ssd_du", s, du_kernel<TM><<<dim3(g.qb * pl.npt, g.nc, bh), 256, 0, s>>>(g, pl, q));
  MKO_TIMED("ssd_dcb", s,
            dcb_kernel<TM><<<dim3(pl.npairs * pl.hb1, ncg, static_cast<unsigned>(g.batch)), 256, 0, s>>>(g, pl, q));
  MKO_TIMED("ssd_dbc_state", s,
            dbc_state<TM><<<dim3(g.qb * pl.nnt * 2 * pl.hb2, ncg, static_cast<unsigned>(g.batch)), 256, 0, s>>>(
                g, pl, q));
  MKO_TIMED("ssd_dbc_final", s,
            dbc_final<TM><<<dim3(g.qb * pl.nnt * 2, ncg, static_cast<unsigned>(g.batch)), 256, 0, s>>>(g, pl, q));
  MKO_TIMED("ssd_finish", s,
            finish<<<dim3(g.nc, static_cast<unsigned>(g.nheads), static_cast<unsigned>(g.batch)), 256, 0, s>>>(g, pl, q));
  MKO_TIMED("ssd_reduce", s, reduce_params<<<dim3(static_cast<unsigned>(g.nheads)), 256, 0, s>>>(g, pl, q));
}

}  // namespace
}  // namespace ssd
}  // namespace mko

using namespace mko;
using namespace mko::ssd;

extern "C" size_t mko_ssd_bwd_workspace_size(const mko_ssd_params* prm) {
  Geo g;
  if (make_geo(prm, &g) != MKO_OK) return 0;
  return bwd_layout(g, make_plan(g), prm->z != nullptr).total;
}

extern "C" int mko_ssd_bwd(const mko_ssd_params* prm, void* stream) {
  Geo g;
  int st = make_geo(prm, &g);
  if (st != MKO_OK) return st;
  const bool tokens = g.batch > 0 && g.length > 0;
  if (!prm->A || !prm->dA ||
      (tokens && (!prm->x || !prm->dt || !prm->B || !prm->C || !prm->saved || !prm->dy || !prm->dx || !prm->ddt ||
                  !prm->dB || !prm->dC))) {
    mko_set_error("ssd_bwd: x, dt, A, B, C, saved, dy, dx, ddt, dA, dB and dC are required");
    return MKO_EINVAL;
  }
  if ((prm->D && !prm->dD) || (tokens && prm->z && !prm->dz) || (prm->dt_bias && !prm->ddt_bias)) {
    mko_set_error("ssd_bwd: dD, dz and ddt_bias are required with D, z and dt_bias");
    return MKO_EINVAL;
  }
  const BwdPlan pl = make_plan(g);
  const BwdLayout lay = bwd_layout(g, pl, prm->z != nullptr);
  if (prm->workspace_bytes < lay.total || (lay.total && !prm->workspace)) {
    mko_set_error("ssd_bwd: workspace of %zu bytes needed, %zu given", lay.total, prm->workspace_bytes);
    return MKO_EWORKSPACE;
  }
  Ptrs q = base_ptrs(prm);
  bind_saved(g, prm->saved, &q);
  char* ws = static_cast<char*>(prm->workspace);
  q.gyw = prm->z ? ws + lay.gy : nullptr;
  q.gy = prm->z ? static_cast<const void*>(ws + lay.gy) : prm->dy;
  q.dstates = reinterpret_cast<float*>(ws + lay.dstates);
  q.dT = reinterpret_cast<float*>(ws + lay.dT);
  q.ya = reinterpret_cast<float*>(ws + lay.ya);
  q.dsx = reinterpret_cast<float*>(ws + lay.dsx);
  q.ut = reinterpret_cast<float*>(ws + lay.ut);
  q.tau = reinterpret_cast<float*>(ws + lay.tau);
  q.pdD = reinterpret_cast<float*>(ws + lay.pdD);
  q.dcb = reinterpret_cast<float*>(ws + lay.dcb);
  q.pbc = reinterpret_cast<float*>(ws + lay.pbc);
  q.pA = reinterpret_cast<float*>(ws + lay.pA);
  q.pbias = reinterpret_cast<float*>(ws + lay.pbias);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (tokens) {
    if (g.x_dtype == MKO_F32) launch_bwd_t<float>(g, pl, q, s);
    else if (g.x_dtype == MKO_BF16) launch_bwd_t<bf16>(g, pl, q, s);
    else launch_bwd_t<_Float16>(g, pl, q, s);
  } else {
    // no tokens: dinitial = dfinal (zero without it); the parameter gradients are zero
    if (g.batch > 0 && q.dinit)
      MKO_TIMED("ssd_state_rev", s,
                state_rev<<<dim3(pl.nblk, static_cast<unsigned>(g.batch * g.nheads)), 256, 0, s>>>(g, pl, q));
    MKO_TIMED("ssd_reduce", s, reduce_params<<<dim3(static_cast<unsigned>(g.nheads)), 256, 0, s>>>(g, pl, q));
  }
  return mko_check_launch("ssd_bwd");
}
