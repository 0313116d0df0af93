// Mamba-2 SSD chunk scan backward for gfx950.
//
// With u_s = step_s x_s, K[l][s] = e^{cs_l - cs_s} CB[l][s] (s <= l), gy = dy * silu(z),
// S_in / S_out the states entering / leaving a chunk and G the adjoint of S_out:
//   gate        y~ = K u + e^{cs} C S_in^T (saved or recomputed); dz; gy; gy.y~ per token;
//               dD partials
//   chunk_state local adjoint of S_in: sum_l e^{cs_l} gy_l (x) C_l
//   (16-bit inputs with d_state <= 128 run gate and chunk_state as one kernel per chunk and
//   head, gate_state_mt, and du as du_mt, or du_cm at 256-token chunks with d_state 128; see
//   multi_tile() in ssd.hpp)
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
// Every partial sum is reduced in a fixed order: the backward is deterministic.  dcb runs on
// a second stream beside state_rev, du, dbc_state, finish and reduce (launch_bwd_t), and
// dbc_final, which reads its partials, runs last.
#include <algorithm>
#include <mutex>
#include <vector>

#include "ssd.hpp"
#include "ssd64.hpp"

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

// The gate's backward on row r0 + rr and columns c0 .. c0 + 7 of the token tile at tl0, from
// yt = that row of the chunk output before the skip and the gate, y~.  With z: dz = dy (D x +
// y~) d silu(z) and gy = dy silu(z) rounded to the storage type (the value the other kernels
// read), both stored; without z, gy = dy.  gy gets gy, ya[po + r0 + rr] the row sum gy . y~,
// and dd accumulates the column partials gy x.
template <typename TM, bool VEC>
__device__ __forceinline__ void gate_row(const Geo& g, const Ptrs& p, int rr, const float (&yt)[8], const V8<TM>& xv,
                                         const V8<TM>& zv, const V8<TM>& dyv, const float (&dv)[8], int64_t b,
                                         int64_t tl0, int64_t h, int64_t pc0, int64_t po, float (&gy)[8],
                                         float (&dd)[8]) {
  float xf[8];
  v8_f32(xv, xf);
  v8_f32(dyv, gy);
  if (p.z) {
    float zf[8], dz[8];
    v8_f32(zv, zf);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float sgm = sigmoid(zf[e]);
      const float ypre = fmaf(dv[e], xf[e], yt[e]);
      dz[e] = gy[e] * ypre * sgm * fmaf(zf[e], 1.0f - sgm, 1.0f);
      gy[e] = to_f32(from_f32<TM>(gy[e] * zf[e] * sgm));
    }
    store_xw_row<TM, VEC, true>(g, static_cast<TM*>(p.dz), b, tl0, h, pc0, rr, dz);
    store_xw_row<TM, VEC>(g, static_cast<TM*>(p.gyw), b, tl0, h, pc0, rr, gy);
  }
  float ya = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    ya = fmaf(gy[e], yt[e], ya);
    dd[e] = fmaf(gy[e], xf[e], dd[e]);
  }
  ya = row8_sum(ya);
  if ((threadIdx.x & 7) == 0) p.ya[po + blk_r0() + rr] = ya;
}

// Column sums of the threads' dd over a tile's 64 rows (lanes sharing tid % 8, then the four
// wavefronts in a fixed order through colred, 256 floats of LDS) into out[col] for col <
// ncol.  colred must be free on entry; it is read by the first 64 threads on exit.
__device__ __forceinline__ void dd_columns(float (&dd)[8], float* colred, float* out, int ncol) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, c0 = blk_c0();
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float v = dd[e];
    v += __shfl_xor(v, 8);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    dd[e] = v;
  }
  if (lane < 8) {
#pragma unroll
    for (int e = 0; e < 8; ++e) colred[64 * wave + c0 + e] = dd[e];
  }
  __syncthreads();
  const int col = threadIdx.x;
  if (col < 64 && col < ncol) out[col] = (colred[col] + colred[64 + col]) + (colred[128 + col] + colred[192 + col]);
}

// SAVED: the forward saved the chunk output (p.yt); otherwise it is recomputed here.
template <typename TM, bool VEC, bool SAVED>
__global__ void __launch_bounds__(256) gate(Geo g, BwdPlan pl, Ptrs p) {
  constexpr int TE = LdsTile<TM>::elems;
  __shared__ __align__(16) TM sbuf[2][2 * TE];
  __shared__ __align__(16) float csc[256], dlc[256], ecol[256];
  __shared__ float colred[4][64];
  // Heads fastest: the workgroups that run together cover whole token rows (a row's
  // heads are adjacent in x, dy, z and the outputs) instead of one head's columns of
  // many rows.
  const WgId id = wg_id(g.nheads, g.qb * g.npt);
  const int64_t h = id.x, b = id.z / g.nc;
  const int i = id.y % g.qb, pt = id.y / g.qb;
  const int c = static_cast<int>(id.z % g.nc);
  const int64_t bh = b * g.nheads + h;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int wm, wn;
  quadrant(wave, wm, wn);
  const int r0 = blk_r0(), c0 = blk_c0();
  const int64_t tl0 = static_cast<int64_t>(c) * g.q + 64 * i, pc0 = static_cast<int64_t>(pt) * 64, pc = pc0 + c0;
  // epilogue inputs, in flight during the products
  V8<TM> xv[2], dyv[2], zv[2];
  load_xw<TM, VEC>(g, static_cast<const TM*>(p.x), b, tl0, h, pc0, xv);
  load_xw<TM, VEC>(g, static_cast<const TM*>(p.dy), b, tl0, h, pc0, dyv);
  if (p.z) load_xw<TM, VEC>(g, static_cast<const TM*>(p.z), b, tl0, h, pc0, zv);
  float dv[8];
  load_d8(g, p, h, pc, dv);
  float yt[2][8];
  if constexpr (SAVED) {
    V8<float> yv[2];
    load_xw<float, VEC>(g, p.yt, b, tl0, h, pc0, yv);
    v8_f32(yv[0], yt[0]);
    v8_f32(yv[1], yt[1]);
  } else {
    load_chunk_cs(g, p, bh, c, csc, dlc, ecol);
    __syncthreads();
    f32x16 acc;
    chunk_out<TM, VEC>(g, p, acc, sbuf, csc, dlc, ecol, i, pt, c, bh);
    float* red = reinterpret_cast<float*>(&sbuf[0][0]);
    acc_to_lds(red, acc, wm, wn, lane);
    __syncthreads();
    lds_block(red, r0, c0, yt[0], yt[1]);
  }
  const int64_t po = ((bh * g.nc + c) * g.npt + pt) * g.q + 64 * i;
  float dd[8] = {};
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    float gy[8];
    gate_row<TM, VEC>(g, p, rr, yt[rr], xv[rr], zv[rr], dyv[rr], dv, b, tl0, h, pc0, po, gy, dd);
  }
  if (p.D)
    dd_columns(dd, &colred[0][0], p.pdD + (((b * g.nc + c) * g.qb + i) * g.nheads + h) * g.headdim + pc0,
               clamp64(g.headdim - pc0));
}

// Stage k of gate_state_mt: first the chunk output of each token tile, the tiles in
// descending order (tile i: nnt state stages, then intra stages over the s-tiles 0 .. i);
// then qb * nnt stages of the local state adjoint (l-tile i, n-tile kk).
struct GsStage {
  bool adj;
  int i, kk;
};
constexpr GsStage gs_stage(int k, int nnt, int qb) {
  const int ny = qb * nnt + qb * (qb + 1) / 2;
  if (k >= ny) return GsStage{true, (k - ny) / nnt, (k - ny) % nnt};
  int ti = 0, base = 0;
  while (k >= base + nnt + (qb - 1 - ti) + 1) {
    base += nnt + (qb - 1 - ti) + 1;
    ++ti;
  }
  return GsStage{false, qb - 1 - ti, k - base};
}

// gate and the local state adjoint in one pass over a (b, h, chunk, d_head tile), 16-bit
// operands, d_state <= 64 * NNT.  The chunk output before the skip and the gate,
//   y~[l][p] = sum_{s<=l} K[l][s] u_s[p] + e^{cs_l} sum_n C_l[n] S_in[p][n],
// is recomputed in fp32 exactly as the forward's multi-tile scan forms it (same operands,
// same stage order), so the forward saves no copy of it.  Per token tile, from y~: dz, gy =
// dy silu(z) (stored in the input dtype, which is what the other kernels read), the row
// sums gy.y~ and the dD column partials.  The tiles run in descending order, so once tile i
// is done its u slot in LDS is free and takes (e^{cs} gy)^T, the left operand of the local
// adjoint sum_l e^{cs_l} gy_l (x) C_l that the last stages accumulate; the adjoint leaves
// through LDS as 16-byte rows.
template <typename TM, bool VEC, int QB, int NNT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) gate_state_mt(Geo g, BwdPlan pl,
                                                                                             Ptrs p) {
  static_assert(sizeof(TM) == 2, "16-bit operands");
  constexpr int TE = LdsTile<TM>::elems;
  constexpr int NY = QB * NNT + QB * (QB + 1) / 2;
  constexpr int N = NY + QB * NNT;
  constexpr int Q = 64 * QB;
  __shared__ __align__(16) TM ut[QB][TE];   // u_j^T [p][s]; after token tile i, slot i holds (e^{cs} gy)^T [p][l]
  __shared__ __align__(16) TM st[NNT][TE];  // S_in [p][n]
  __shared__ __align__(16) TM ab[2][TE];    // right/left operand per stage; the epilogue's fp32 tile
  __shared__ __align__(16) float csc[Q], dlc[Q], ecol[Q], ecs[Q], dcol[64];
  __shared__ float colred[4][64];
  const WgId id = wg_id(g.nheads, g.npt);
  const int64_t h = id.x;
  const int pt = id.y;
  const int64_t b = id.z / g.nc;
  const int c = static_cast<int>(id.z % g.nc);
  const int64_t bh = b * g.nheads + h, gg = h / g.hpg;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int wm, wn;
  quadrant(wave, wm, wn);
  const int r0 = blk_r0(), c0 = blk_c0();
  const int64_t tc = static_cast<int64_t>(c) * Q, pc0 = static_cast<int64_t>(pt) * 64;
  const TM* X = static_cast<const TM*>(p.x);
  const TM* Z = p.z ? static_cast<const TM*>(p.z) : X;
  const TM* DY = static_cast<const TM*>(p.dy);
  const TM* Cm = static_cast<const TM*>(p.C);
  const TM* cbt = static_cast<const TM*>(p.cb) + ((b * g.nc + c) * g.ngroups + gg) * Q * Q;
  const TM* S = static_cast<const TM*>(p.states) + (bh * g.nc + c) * g.headdim * g.dstate;
  {
    V8<TM> xr[QB][2], sr[NNT][2];
#pragma unroll
    for (int j = 0; j < QB; ++j) load_xw<TM, VEC>(g, X, b, tc + 64 * j, h, pc0, xr[j]);
#pragma unroll
    for (int k = 0; k < NNT; ++k) load_sw<TM, VEC>(g, S, pc0, 64 * k, sr[k]);
    load_chunk_cs(g, p, bh, c, csc, dlc, ecol);
    if (threadIdx.x < Q) ecs[threadIdx.x] = fast_exp(csc[threadIdx.x]);
    if (threadIdx.x < 64) {
      const int64_t pp = pc0 + threadIdx.x;
      dcol[threadIdx.x] = !p.D ? 0.0f : g.d_per_row ? (pp < g.headdim ? p.D[h * g.headdim + pp] : 0.0f) : p.D[h];
    }
    __syncthreads();  // csc, dlc
#pragma unroll
    for (int j = 0; j < QB; ++j) {
      float a[8], bb[8];
      scale8(xr[j][0], dlc[64 * j + r0], a);
      scale8(xr[j][1], dlc[64 * j + r0 + 1], bb);
      put2x8<TM, true>(ut[j], r0, c0, a, bb);  // Bt[p][s] = step_s x_s[p]
    }
#pragma unroll
    for (int k = 0; k < NNT; ++k) put_raw<TM, false>(st[k], r0, c0, sr[k][0], sr[k][1]);  // Bt[p][n] = S_in[p][n]
  }
  struct Regs {
    V8<TM> a[2];
  };
  auto fetch = [&](auto kc, Regs& r) {
    constexpr GsStage sg = gs_stage(decltype(kc)::value, NNT, QB);
    if constexpr (sg.adj || sg.kk < NNT)
      load_bw<TM, VEC>(g, Cm, b, tc + 64 * sg.i, gg, 64 * sg.kk, r.a);  // C rows l
    else
      load_win<TM, true>(cbt + (64 * sg.i) * Q + 64 * (sg.kk - NNT), Q, 64, 64, r.a, cbt);  // cb rows l
  };
  auto put = [&](auto kc, Regs& r) {
    constexpr int k = decltype(kc)::value;
    constexpr GsStage sg = gs_stage(k, NNT, QB);
    if constexpr (sg.adj) {
      put_raw<TM, true>(ab[k & 1], r0, c0, r.a[0], r.a[1]);  // Bt[n][l] = C_l[n]
    } else if constexpr (sg.kk < NNT) {
      put_raw<TM, false>(ab[k & 1], r0, c0, r.a[0], r.a[1]);  // A[l][n] = C_l[n]
    } else {
      float a[8], bb[8];
      k_block<TM>(r.a[0], r.a[1], csc, ecol, sg.i, sg.kk - NNT, r0, c0, a, bb);
      put2x8<TM, false>(ab[k & 1], r0, c0, a, bb);  // A[l][s] = K[l][s]
    }
  };
  f32x16 acc, acc1;
  zero(acc);
  zero(acc1);
  V8<TM> xv[2], zv[2], dyv[2];
  constexpr int D = N < 6 ? N : 6;
  Regs regs[D];
  pipeline_static<N, D>(regs, fetch, put, [&](auto kc) {
    constexpr int k = decltype(kc)::value;
    constexpr GsStage sg = gs_stage(k, NNT, QB);
    if constexpr (sg.adj) {
      // A[p][l] = e^{cs_l} gy_l[p] (slot i), Bt[n][l] = C_l[n]
      mma_tile<TM>(sg.kk == 0 ? acc : acc1, ut[sg.i], ab[k & 1], wm, wn, lane, 64);
      return;
    } else {
      const int i = sg.i;
      const int64_t tl0 = tc + 64 * i;
      if constexpr (sg.kk == 0) {  // epilogue inputs of tile i
        load_xw<TM, VEC>(g, X, b, tl0, h, pc0, xv);
        load_xw<TM, VEC>(g, Z, b, tl0, h, pc0, zv);
        load_xw<TM, VEC>(g, DY, b, tl0, h, pc0, dyv);
      }
      if constexpr (sg.kk < NNT) {
        mma_tile<TM>(acc, ab[k & 1], st[sg.kk], wm, wn, lane, 64);
        if constexpr (sg.kk == NNT - 1) {
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[r] *= ecs[64 * i + acc_row(wm, lane, r)];
        }
        return;
      }
      mma_tile<TM>(acc, ab[k & 1], ut[sg.kk - NNT], wm, wn, lane, 64);
      if constexpr (sg.kk == NNT + sg.i) {
        float* red = reinterpret_cast<float*>(&ab[0][0]);
        __syncthreads();
        acc_to_lds(red, acc, wm, wn, lane);
        zero(acc);
        __syncthreads();
        float yt[2][8];
        lds_block(red, r0, c0, yt[0], yt[1]);
        const float4 da = *reinterpret_cast<const float4*>(dcol + c0);
        const float4 db = *reinterpret_cast<const float4*>(dcol + c0 + 4);
        const float dv[8] = {da.x, da.y, da.z, da.w, db.x, db.y, db.z, db.w};
        const int64_t po = ((bh * g.nc + c) * g.npt + pt) * Q + 64 * i;
        float dd[8] = {};
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          float gy[8];
          gate_row<TM, VEC>(g, p, rr, yt[rr], xv[rr], zv[rr], dyv[rr], dv, b, tl0, h, pc0, po, gy, dd);
          const float el = ecs[64 * i + r0 + rr];
#pragma unroll
          for (int e = 0; e < 8; ++e) yt[rr][e] = gy[e] * el;  // the adjoint's operand, e^{cs_l} gy_l
        }
        put2x8<TM, true>(ut[i], r0, c0, yt[0], yt[1]);  // A[p][l] = e^{cs_l} gy_l[p]
        if (p.D)
          dd_columns(dd, &colred[0][0], p.pdD + (((b * g.nc + c) * g.qb + i) * g.nheads + h) * g.headdim + pc0,
                     clamp64(g.headdim - pc0));
        __syncthreads();  // the next stage refills the operand buffers; colred is reused
      }
    }
  });
  // the local adjoint [p][n], one 64-wide n-tile at a time through the fp32 tile
  TM* out = static_cast<TM*>(p.dstates) + (bh * g.nc + c) * g.headdim * g.dstate + pc0 * g.dstate;
  float* red = reinterpret_cast<float*>(&ab[0][0]);
#pragma unroll
  for (int kk = 0; kk < NNT; ++kk) {
    __syncthreads();
    acc_to_lds(red, kk == 0 ? acc : acc1, wm, wn, lane);
    __syncthreads();
    float v[2][8];
    lds_block(red, r0, c0, v[0], v[1]);
    store_win<TM, VEC>(out + 64 * kk, static_cast<int>(g.dstate), clamp64(g.headdim - pc0),
                       static_cast<int>(g.dstate - 64 * kk), v[0], v[1]);
  }
}

// Backwards over the chunks, 8 state elements per thread: G (the adjoint of the
// state leaving each chunk) over the local adjoints in dstates, e^T <G, S_in> per
// 2048-element state block, and the adjoint of the initial state.
template <typename TM>
__global__ void __launch_bounds__(256) state_rev(Geo g, BwdPlan pl, Ptrs p) {
  __shared__ float wsum[4];
  const int64_t pn = g.headdim * g.dstate;
  const int blk = blockIdx.x;
  const int64_t e0 = (static_cast<int64_t>(blk) * 256 + threadIdx.x) * 8;
  const int n = e0 < pn ? static_cast<int>(pn - e0 < 8 ? pn - e0 : 8) : 0;
  const int64_t bh = blockIdx.y;
  TM* ds = static_cast<TM*>(p.dstates);
  const TM* st = static_cast<const TM*>(p.states);
  float gv[8];
  if (n > 0 && p.dfinal) {
    V8<TM> v;
    v8_load(v, static_cast<const TM*>(p.dfinal) + bh * pn + e0, n, g.vec);
    v8_f32(v, gv);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) gv[k] = 0.0f;
  }
  for (int c = g.nc - 1; c >= 0; --c) {
    const int64_t o = (bh * g.nc + c) * pn + e0;
    const float eT = fast_exp(p.cs[(bh * g.nc + c) * g.q + g.q - 1]);
    float part = 0.0f, loc[8];
    if (n > 0) {
      V8<TM> v;
      v8_load(v, st + o, n, g.vec);
      float sf[8];
      v8_f32(v, sf);
#pragma unroll
      for (int k = 0; k < 8; ++k) part = fmaf(gv[k], sf[k], part);
      v8_load(v, ds + o, n, g.vec);
      v8_f32(v, loc);
      v8_store(ds + o, n, g.vec, gv);
    }
    const float dt = block_sum(part, wsum);
    if (threadIdx.x == 0) p.dT[(bh * g.nc + c) * pl.nblk + blk] = eT * dt;
    if (n > 0) {
#pragma unroll
      for (int k = 0; k < 8; ++k) gv[k] = fmaf(eT, gv[k], loc[k]);
    }
  }
  if (n > 0 && p.dinit) v8_store(static_cast<TM*>(p.dinit) + bh * pn + e0, n, g.vec, gv);
}

// du for the 64-token tiles ja = jx and jb = qb-1-jx (one tile when they coincide) and
// d_head tile pt of one (b, h, chunk):
//   du[s][p] = e^{T - cs_s} sum_n B_s[n] G[p][n]  +  sum_{l >= s} K[l][s] gy_l[p]
// Tile j takes nnt state stages, then qb - j intra stages, so a pair takes
// 2 nnt + qb + 1 stages whichever jx it is; both tiles run through one pipeline.  The
// state part of a tile runs first and its u.du_state is taken before the intra part
// is added.  Between stages the LDS buffer the next stage will fill is free, so the
// snapshots and epilogues go through it.
template <typename TM, bool VEC>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) du_kernel(Geo g, BwdPlan pl, Ptrs p) {
  constexpr int TE = LdsTile<TM>::elems;
  __shared__ __align__(16) TM sbuf[2][2 * TE];
  __shared__ __align__(16) float csc[256], dlc[256], ecol[256], dcol[64];
  const int nj = (g.qb + 1) / 2;
  // heads fastest, as in the forward's chunk_scan
  const WgId id = wg_id(g.nheads, nj * g.npt);
  const int jx = id.y % nj, pt = id.y / nj;
  const int ja = jx, jb = g.qb - 1 - jx;
  const int c = static_cast<int>(id.z % g.nc);
  const int64_t h = id.x, b = id.z / g.nc, gg = h / g.hpg;
  const int64_t bh = b * g.nheads + h;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int r0 = blk_r0(), c0 = blk_c0();
  load_chunk_cs(g, p, bh, c, csc, dlc, ecol);
  const int64_t tc = static_cast<int64_t>(c) * g.q;
  const int64_t pc0 = static_cast<int64_t>(pt) * 64;
  if (threadIdx.x < 64) {
    const int64_t pp = pc0 + threadIdx.x;
    dcol[threadIdx.x] = !p.D ? 0.0f : g.d_per_row ? (pp < g.headdim ? p.D[h * g.headdim + pp] : 0.0f) : p.D[h];
  }
  const TM* cbt = static_cast<const TM*>(p.cb) + ((b * g.nc + c) * g.ngroups + gg) * g.q * g.q;
  const TM* Bm = static_cast<const TM*>(p.B);
  const TM* gy = static_cast<const TM*>(p.gy);
  const TM* G = static_cast<const TM*>(p.dstates) + (bh * g.nc + c) * g.headdim * g.dstate;
  const int na = g.nnt + g.qb - ja;
  const int n = na + (jb != ja ? g.nnt + g.qb - jb : 0);
  // stage k -> tile j and its stage kk within the tile
  auto tile_of = [&](int k, int& j, int& kk) {
    j = k < na ? ja : jb;
    kk = k < na ? k : k - na;
  };
  // x of the tile in progress (for tau and the epilogue) and gy of its epilogue, issued
  // stages ahead of their use so that waiting for them does not drain the prefetches
  V8<TM> xv[2], gv[2];
  load_xw<TM, VEC>(g, static_cast<const TM*>(p.x), b, tc + 64 * ja, h, pc0, xv);
  f32x16 acc;
  zero(acc);
  __syncthreads();  // csc, dlc, ecol, dcol
  const float T = csc[g.q - 1];
  // x of the thread's block (rows s = r0, r0+1 of tile j) and u_s = R(dt_s x_s), the
  // rounded input of the forward's products
  auto u8 = [&](int j, const V8<TM> (&xv)[2], int rr, float (&xf)[8], float (&uf)[8]) {
    v8_f32(xv[rr], xf);
    const float d = dlc[64 * j + r0 + rr];
#pragma unroll
    for (int k = 0; k < 8; ++k) uf[k] = to_f32(from_f32<TM>(d * xf[k]));
  };
  const int64_t po0 = ((bh * g.nc + c) * g.npt + pt) * g.q;
  // Per tile: stages 0 .. nnt-1: state part, A = e^{T - cs_s} B_s[n], Bt = G[p][n];
  // then tau_s = u_s . du_state_s; stages nnt .. : intra-chunk tiles i >= j,
  // A = K[l][s] (transposed), Bt = gy_l[p] (transposed).  Both kinds load two rows
  // of two 64-wide windows.
  struct Regs {
    V8<TM> a[2], b[2];
  };
  auto fetch = [&](int k, Regs& r) {
    int j, kk;
    tile_of(k, j, kk);
    if (kk < g.nnt) {
      load_bw<TM, VEC>(g, Bm, b, tc + 64 * j, gg, 64 * kk, r.a);  // B rows s
      load_sw<TM, VEC>(g, G, pc0, 64 * kk, r.b);                  // G rows p
    } else {
      const int i = j + kk - g.nnt;
      load_win<TM, true>(cbt + (64 * i) * g.q + 64 * j, g.q, 64, 64, r.a, cbt);  // cb rows l
      load_xw<TM, VEC>(g, gy, b, tc + 64 * i, h, pc0, r.b);                     // gy rows l
    }
  };
  auto put = [&](int k, Regs& r) {
    int j, kk;
    tile_of(k, j, kk);
    TM* buf = sbuf[k & 1];
    float a[8], bb[8];
    if (kk < g.nnt) {
      const float w0 = fast_exp(T - csc[64 * j + r0]), w1 = fast_exp(T - csc[64 * j + r0 + 1]);
      scale8(r.a[0], w0, a);
      scale8(r.a[1], w1, bb);
      put2x8<TM, false>(buf, r0, c0, a, bb);                  // A[s][n] = e^{T - cs_s} B_s[n]
      put_raw<TM, false>(buf + TE, r0, c0, r.b[0], r.b[1]);  // Bt[p][n] = G[p][n]
    } else {
      const int i = j + kk - g.nnt;
      k_block<TM>(r.a[0], r.a[1], csc, ecol, i, j, r0, c0, a, bb);
      put2x8<TM, true>(buf, r0, c0, a, bb);                  // A[s][l] = K[l][s]
      put_raw<TM, true>(buf + TE, r0, c0, r.b[0], r.b[1]);  // Bt[p][l] = gy_l[p]
    }
  };
  // tau_s = u_s . du_state_s for tile j; red is the free buffer
  auto tau_snapshot = [&](int j, float* red) {
    acc_to_lds(red, acc, wm, wn, lane);
    __syncthreads();
    float v[2][8];
    lds_block(red, r0, c0, v[0], v[1]);
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      float xf[8], uf[8];
      u8(j, xv, rr, xf, uf);
      float tau = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) tau = fmaf(uf[e], v[rr][e], tau);
      tau = row8_sum(tau);
      if ((threadIdx.x & 7) == 0) p.tau[po0 + 64 * j + r0 + rr] = tau;
    }
    load_xw<TM, VEC>(g, gy, b, tc + 64 * j, h, pc0, gv);
    __syncthreads();  // red is refilled by the next stage
  };
  // dx = dt du + D gy, and the row sums x.du and u.du of tile j; red is the free buffer
  auto epilogue = [&](int j, float* red) {
    acc_to_lds(red, acc, wm, wn, lane);
    __syncthreads();
    float du[2][8], dxo[2][8];
    lds_block(red, r0, c0, du[0], du[1]);
    const float4 da = *reinterpret_cast<const float4*>(dcol + c0);
    const float4 db = *reinterpret_cast<const float4*>(dcol + c0 + 4);
    const float dv[8] = {da.x, da.y, da.z, da.w, db.x, db.y, db.z, db.w};
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      float gf[8], xf[8], uf[8];
      v8_f32(gv[rr], gf);
      u8(j, xv, rr, xf, uf);
      const float d = dlc[64 * j + r0 + rr];
      float sx = 0.0f, su = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = d * du[rr][e];
        v = fmaf(dv[e], gf[e], v);
        dxo[rr][e] = v;
        sx = fmaf(xf[e], du[rr][e], sx);
        su = fmaf(uf[e], du[rr][e], su);
      }
      sx = row8_sum(sx);
      su = row8_sum(su);
      if ((threadIdx.x & 7) == 0) {
        p.dsx[po0 + 64 * j + r0 + rr] = sx;
        p.ut[po0 + 64 * j + r0 + rr] = su;
      }
    }
    store_xw<TM, VEC, true>(g, static_cast<TM*>(p.dx), b, tc + 64 * j, h, pc0, dxo[0], dxo[1]);
    if (j != jb) load_xw<TM, VEC>(g, static_cast<const TM*>(p.x), b, tc + 64 * jb, h, pc0, xv);
    __syncthreads();  // red is refilled by the next stage
  };
  Regs ra, rb;
  pipeline2(n, ra, rb, fetch, put, [&](int k) {
    mma_tile<TM>(acc, sbuf[k & 1], sbuf[k & 1] + TE, wm, wn, lane, 64);
    int j, kk;
    tile_of(k, j, kk);
    // buffer (k+1)&1 was last read by stage k-1, which every wave finished before the
    // barrier that published stage k
    float* red = reinterpret_cast<float*>(&sbuf[(k + 1) & 1][0]);
    if (kk == g.nnt - 1) tau_snapshot(j, red);
    if (kk == g.nnt + g.qb - j - 1) {
      epilogue(j, red);
      zero(acc);
    }
  });
}

// Stage k of du_mt's schedule: s-tile j, then its state stages kk < nnt and its intra
// stages kk = nnt + m over the l-tiles i = j + m, m = 0 .. qb-1-j (nnt + qb - j stages).
struct DuStage {
  int j, kk;
};
constexpr DuStage du_stage(int k, int nnt, int qb) {
  int j = 0, base = 0;
  while (k >= base + nnt + qb - j) {
    base += nnt + qb - j;
    ++j;
  }
  return DuStage{j, k - base};
}

// du for all QB 64-token tiles of one (b, h, chunk, d_head tile), 16-bit operands and
// d_state <= 64 * NNT:
//   du[s][p] = e^{T - cs_s} sum_n B_s[n] G[p][n]  +  sum_{l >= s} K[l][s] gy_l[p]
// gy (transposed) and G of the chunk are staged into LDS once; per stage only the left
// operand is: B rows as they are in memory for the state stages (the row factor
// e^{T - cs_s}, at most 1, is applied to the accumulator after the last of them), K^T from
// the C.B^T tile for the intra stages.  The schedule is fixed at compile time and each
// left operand is requested six stages ahead.  Per s-tile: tau_s = u_s . du_state_s after
// the state stages, then dx = step du + D gy and the row sums x.du and u.du.
template <typename TM, bool VEC, int QB, int NNT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) du_mt(Geo g, BwdPlan pl, Ptrs p) {
  static_assert(sizeof(TM) == 2, "16-bit operands");
  constexpr int TE = LdsTile<TM>::elems;
  constexpr int N = QB * NNT + QB * (QB + 1) / 2;
  constexpr int Q = 64 * QB;
  __shared__ __align__(16) TM gyt[QB][TE];  // gy_l^T [p][l]
  __shared__ __align__(16) TM gt[NNT][TE];  // G [p][n]
  __shared__ __align__(16) TM ab[2][TE];    // left operand, double-buffered; the fp32 tile of the epilogues
  __shared__ __align__(16) float csc[Q], dlc[Q], ecol[Q], ew[Q], dcol[64];
  const WgId id = wg_id(g.nheads, g.npt);
  const int64_t h = id.x;
  const int pt = id.y;
  const int64_t b = id.z / g.nc;
  const int c = static_cast<int>(id.z % g.nc);
  const int64_t bh = b * g.nheads + h, gg = h / g.hpg;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int r0 = blk_r0(), c0 = blk_c0();
  const int64_t tc = static_cast<int64_t>(c) * Q, pc0 = static_cast<int64_t>(pt) * 64;
  const TM* X = static_cast<const TM*>(p.x);
  const TM* gy = static_cast<const TM*>(p.gy);
  const TM* Bm = static_cast<const TM*>(p.B);
  const TM* cbt = static_cast<const TM*>(p.cb) + ((b * g.nc + c) * g.ngroups + gg) * Q * Q;
  const TM* G = static_cast<const TM*>(p.dstates) + (bh * g.nc + c) * g.headdim * g.dstate;
  const int64_t so = (bh * g.nc + c) * Q;
  {
    V8<TM> gr[QB][2], sr[NNT][2];
#pragma unroll
    for (int i = 0; i < QB; ++i) load_xw<TM, VEC>(g, gy, b, tc + 64 * i, h, pc0, gr[i]);
#pragma unroll
    for (int k = 0; k < NNT; ++k) load_sw<TM, VEC>(g, G, pc0, 64 * k, sr[k]);
    load_chunk_cs(g, p, bh, c, csc, dlc, ecol);
    if (threadIdx.x < Q) ew[threadIdx.x] = fast_exp(p.cs[so + Q - 1] - p.cs[so + threadIdx.x]);
    if (threadIdx.x < 64) {
      const int64_t pp = pc0 + threadIdx.x;
      dcol[threadIdx.x] = !p.D ? 0.0f : g.d_per_row ? (pp < g.headdim ? p.D[h * g.headdim + pp] : 0.0f) : p.D[h];
    }
#pragma unroll
    for (int i = 0; i < QB; ++i) put_raw<TM, true>(gyt[i], r0, c0, gr[i][0], gr[i][1]);  // Bt[p][l] = gy_l[p]
#pragma unroll
    for (int k = 0; k < NNT; ++k) put_raw<TM, false>(gt[k], r0, c0, sr[k][0], sr[k][1]);  // Bt[p][n] = G[p][n]
    __syncthreads();  // csc, dlc, ecol, ew, dcol (the tiles are published by the first stage's barrier)
  }
  struct Regs {
    V8<TM> a[2];
  };
  auto fetch = [&](auto kc, Regs& r) {
    constexpr DuStage sg = du_stage(decltype(kc)::value, NNT, QB);
    if constexpr (sg.kk < NNT) {
      load_bw<TM, VEC>(g, Bm, b, tc + 64 * sg.j, gg, 64 * sg.kk, r.a);  // B rows s
    } else {
      constexpr int i = sg.j + sg.kk - NNT;
      load_win<TM, true>(cbt + (64 * i) * Q + 64 * sg.j, Q, 64, 64, r.a, cbt);  // cb rows l
    }
  };
  auto put = [&](auto kc, Regs& r) {
    constexpr int k = decltype(kc)::value;
    constexpr DuStage sg = du_stage(k, NNT, QB);
    if constexpr (sg.kk < NNT) {
      put_raw<TM, false>(ab[k & 1], r0, c0, r.a[0], r.a[1]);  // A[s][n] = B_s[n]
    } else {
      float a[8], bb[8];
      k_block<TM>(r.a[0], r.a[1], csc, ecol, sg.j + sg.kk - NNT, sg.j, r0, c0, a, bb);
      put2x8<TM, true>(ab[k & 1], r0, c0, a, bb);  // A[s][l] = K[l][s]
    }
  };
  // x of tile j's rows s = r0, r0+1 and u_s = R(step_s x_s), the rounded input of the forward's products
  auto u8 = [&](int j, const V8<TM> (&xv)[2], int rr, float (&xf)[8], float (&uf)[8]) {
    v8_f32(xv[rr], xf);
    const float d = dlc[64 * j + r0 + rr];
#pragma unroll
    for (int e = 0; e < 8; ++e) uf[e] = to_f32(from_f32<TM>(d * xf[e]));
  };
  const int64_t po0 = ((bh * g.nc + c) * g.npt + pt) * Q;
  float* red = reinterpret_cast<float*>(&ab[0][0]);
  f32x16 acc;
  zero(acc);
  V8<TM> xv[2], gv[2];
  constexpr int D = N < 6 ? N : 6;
  Regs regs[D];
  pipeline_static<N, D>(regs, fetch, put, [&](auto kc) {
    constexpr int k = decltype(kc)::value;
    constexpr DuStage sg = du_stage(k, NNT, QB);
    constexpr int j = sg.j;
    const int64_t ts0 = tc + 64 * j;
    if constexpr (sg.kk == 0) {  // tile j's x (tau, epilogue) and gy (epilogue)
      load_xw<TM, VEC>(g, X, b, ts0, h, pc0, xv);
      load_xw<TM, VEC>(g, gy, b, ts0, h, pc0, gv);
    }
    if constexpr (sg.kk < NNT) {
      mma_tile<TM>(acc, ab[k & 1], gt[sg.kk], wm, wn, lane, 64);
      if constexpr (sg.kk == NNT - 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] *= ew[64 * j + acc_row(wm, lane, r)];
        // tau_s = u_s . du_state_s
        __syncthreads();
        acc_to_lds(red, acc, wm, wn, lane);
        __syncthreads();
        float v[2][8];
        lds_block(red, r0, c0, v[0], v[1]);
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          float xf[8], uf[8];
          u8(j, xv, rr, xf, uf);
          float tau = 0.0f;
#pragma unroll
          for (int e = 0; e < 8; ++e) tau = fmaf(uf[e], v[rr][e], tau);
          tau = row8_sum(tau);
          if ((threadIdx.x & 7) == 0) p.tau[po0 + 64 * j + r0 + rr] = tau;
        }
        __syncthreads();  // the next stage refills the operand buffers
      }
    } else {
      mma_tile<TM>(acc, ab[k & 1], gyt[j + sg.kk - NNT], wm, wn, lane, 64);
      if constexpr (j + sg.kk - NNT == QB - 1) {
        // dx = step du + D gy, and the row sums x.du and u.du of tile j
        __syncthreads();
        acc_to_lds(red, acc, wm, wn, lane);
        zero(acc);
        __syncthreads();
        float du[2][8], dxo[2][8];
        lds_block(red, r0, c0, du[0], du[1]);
        const float4 da = *reinterpret_cast<const float4*>(dcol + c0);
        const float4 db = *reinterpret_cast<const float4*>(dcol + c0 + 4);
        const float dv[8] = {da.x, da.y, da.z, da.w, db.x, db.y, db.z, db.w};
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          float gf[8], xf[8], uf[8];
          v8_f32(gv[rr], gf);
          u8(j, xv, rr, xf, uf);
          const float d = dlc[64 * j + r0 + rr];
          float sx = 0.0f, su = 0.0f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            dxo[rr][e] = fmaf(dv[e], gf[e], d * du[rr][e]);
            sx = fmaf(xf[e], du[rr][e], sx);
            su = fmaf(uf[e], du[rr][e], su);
          }
          sx = row8_sum(sx);
          su = row8_sum(su);
          if ((threadIdx.x & 7) == 0) {
            p.dsx[po0 + 64 * j + r0 + rr] = sx;
            p.ut[po0 + 64 * j + r0 + rr] = su;
          }
        }
        store_xw<TM, VEC, true>(g, static_cast<TM*>(p.dx), b, ts0, h, pc0, dxo[0], dxo[1]);
        if constexpr (k + 1 < N) __syncthreads();  // the next stage refills the operand buffers
      }
    }
  });
}

// The schedule of du_cm at qb = 4 and two state tiles (d_state 128).  The output tiles run in
// two halves, {3, 2} and {1, 0}, each with its own two accumulators: the half's state stages
// (right operand: G's n-tiles; tau after a tile's last one), then its intra pairs (l-tile i,
// s-tile j) by l-tile in descending order, gy_i staged with the first pair of its l-tile.  A
// tile is complete after its pair with i = j, where its epilogue runs.  Two LDS slots hold the
// right operands: G's n-tile k in slot k, gy_i in slot (i + 1) & 1; every slot is rewritten at
// least two stages after its last reader, so the stage barriers cover it.
struct DuCmStage {
  bool state;
  int i, j;   // state stages: i = output tile, j = n-tile; pairs: l-tile i, s-tile j
  int stage;  // this stage's put also stages gy_i (pairs) or G's n-tile j (state), when set
  int load;   // after this stage's products: 1 = gy_2, 2 = gy_3, x_1 and x_0, 3 = gy_2,
              // 4 = gy_1, 5 = gy_0 (G's n-tiles stay in registers from the start)
};
constexpr DuCmStage kDuCmSchedule[18] = {
    {true, 3, 0, 0, 0},  {true, 2, 0, 0, 0},  {true, 3, 1, 0, 0},  {true, 2, 1, 0, 0},
    {false, 3, 3, 1, 1}, {false, 3, 2, 0, 6}, {false, 2, 2, 1, 2},
    {true, 1, 0, 1, 0},  {true, 0, 0, 0, 0},  {true, 1, 1, 1, 0},  {true, 0, 1, 0, 0},
    {false, 3, 1, 1, 3}, {false, 3, 0, 0, 0}, {false, 2, 1, 1, 4}, {false, 2, 0, 0, 0},
    {false, 1, 1, 1, 5}, {false, 1, 0, 0, 0}, {false, 0, 0, 1, 0}};

// du_mt at qb = 4, d_state 128 with three workgroups per CU (16-bit operands): the same
// products in the order of kDuCmSchedule, two right-operand slots in LDS instead of all of a
// chunk's gy tiles and G, two accumulators live instead of one per tile.  Compact 64-element
// operand tiles; 53.8 KB of LDS.
template <typename TM, bool VEC>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) du_cm(Geo g, BwdPlan pl, Ptrs p) {
  static_assert(sizeof(TM) == 2, "16-bit operands");
  constexpr int LD = compact_ld<TM>();
  constexpr int TE = LdsTile<TM, LD>::elems;
  constexpr int N = 18;
  constexpr int Q = 256;
  __shared__ __align__(16) TM ab[2][TE];  // left operand, double-buffered
  __shared__ __align__(16) TM ub[2][TE];  // right operand slots
  __shared__ __align__(16) float red[64 * 65];
  __shared__ __align__(16) float csc[Q], dlc[Q], ecol[Q], ew[Q], dcol[64];
  const WgId id = wg_id(g.nheads, g.npt);
  const int64_t h = id.x;
  const int pt = id.y;
  const int64_t b = id.z / g.nc;
  const int c = static_cast<int>(id.z % g.nc);
  const int64_t bh = b * g.nheads + h, gg = h / g.hpg;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int r0 = blk_r0(), c0 = blk_c0();
  const int64_t tc = static_cast<int64_t>(c) * Q, pc0 = static_cast<int64_t>(pt) * 64;
  const TM* X = static_cast<const TM*>(p.x);
  const TM* gy = static_cast<const TM*>(p.gy);
  const TM* Bm = static_cast<const TM*>(p.B);
  const TM* cbt = static_cast<const TM*>(p.cb) + ((b * g.nc + c) * g.ngroups + gg) * Q * Q;
  const TM* G = static_cast<const TM*>(p.dstates) + (bh * g.nc + c) * g.headdim * g.dstate;
  const int64_t so = (bh * g.nc + c) * Q;
  V8<TM> xs[2][2];  // x rows of the output tiles, tile j in set j & 1
  V8<TM> gv[2];     // gy rows of the l-tile staged next (its epilogue's too when i = j)
  V8<TM> sv[2][2];  // G's n-tiles, for the second half
  {
#pragma unroll
    for (int k = 0; k < 2; ++k) load_sw<TM, VEC>(g, G, pc0, 64 * k, sv[k]);
    load_xw<TM, VEC>(g, X, b, tc + 192, h, pc0, xs[1]);
    load_xw<TM, VEC>(g, X, b, tc + 128, h, pc0, xs[0]);
    load_xw<TM, VEC>(g, gy, b, tc + 192, h, pc0, gv);
    load_chunk_cs(g, p, bh, c, csc, dlc, ecol);
    if (threadIdx.x < Q) ew[threadIdx.x] = fast_exp(p.cs[so + Q - 1] - p.cs[so + threadIdx.x]);
    if (threadIdx.x < 64) {
      const int64_t pp = pc0 + threadIdx.x;
      dcol[threadIdx.x] = !p.D ? 0.0f : g.d_per_row ? (pp < g.headdim ? p.D[h * g.headdim + pp] : 0.0f) : p.D[h];
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) put_raw<TM, false, LD>(ub[k], r0, c0, sv[k][0], sv[k][1]);  // Bt[p][n] = G[p][n]
  }
  struct Regs {
    V8<TM> a[2];
  };
  auto fetch = [&](auto kc, Regs& r) {
    constexpr DuCmStage sg = kDuCmSchedule[decltype(kc)::value];
    if constexpr (sg.state)
      load_bw<TM, VEC>(g, Bm, b, tc + 64 * sg.i, gg, 64 * sg.j, r.a);  // B rows s
    else
      load_win<TM, true>(cbt + (64 * sg.i) * Q + 64 * sg.j, Q, 64, 64, r.a, cbt);  // cb rows l
  };
  auto put = [&](auto kc, Regs& r) {
    constexpr int k = decltype(kc)::value;
    constexpr DuCmStage sg = kDuCmSchedule[k];
    if constexpr (sg.state) {
      put_raw<TM, false, LD>(ab[k & 1], r0, c0, r.a[0], r.a[1]);  // A[s][n] = B_s[n]
      if constexpr (sg.stage) put_raw<TM, false, LD>(ub[sg.j], r0, c0, sv[sg.j][0], sv[sg.j][1]);
    } else {
      float a[8], bb[8];
      k_block<TM>(r.a[0], r.a[1], csc, ecol, sg.i, sg.j, r0, c0, a, bb);
      put2x8<TM, true, LD>(ab[k & 1], r0, c0, a, bb);  // A[s][l] = K[l][s]
      if constexpr (sg.stage) put_raw<TM, true, LD>(ub[(sg.i + 1) & 1], r0, c0, gv[0], gv[1]);  // Bt[p][l] = gy_l[p]
    }
  };
  // x of tile j's rows s and u_s = R(step_s x_s), the rounded input of the forward's products
  auto u8 = [&](int j, const V8<TM> (&xv)[2], int rr, float (&xf)[8], float (&uf)[8]) {
    v8_f32(xv[rr], xf);
    const float d = dlc[64 * j + r0 + rr];
#pragma unroll
    for (int e = 0; e < 8; ++e) uf[e] = to_f32(from_f32<TM>(d * xf[e]));
  };
  const int64_t po0 = ((bh * g.nc + c) * g.npt + pt) * Q;
  f32x16 acc[2];
  zero(acc[0]);
  zero(acc[1]);
  constexpr int D = 2;
  Regs regs[D];
  __syncthreads();  // csc, dlc, ecol, ew, dcol, G
  pipeline_static<N, D>(regs, fetch, put, [&](auto kc) {
    constexpr int k = decltype(kc)::value;
    constexpr DuCmStage sg = kDuCmSchedule[k];
    if constexpr (sg.state) {
      constexpr int j = sg.i;
      f32x16& ac = acc[j & 1];
      mma_tile<TM, LD>(ac, ab[k & 1], ub[sg.j], wm, wn, lane, 64);
      if constexpr (sg.j == 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) ac[r] *= ew[64 * j + acc_row(wm, lane, r)];
        // tau_s = u_s . du_state_s
        acc_to_lds(red, ac, wm, wn, lane);
        __syncthreads();
        float v[2][8];
        lds_block(red, r0, c0, v[0], v[1]);
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          float xf[8], uf[8];
          u8(j, xs[j & 1], rr, xf, uf);
          float tau = 0.0f;
#pragma unroll
          for (int e = 0; e < 8; ++e) tau = fmaf(uf[e], v[rr][e], tau);
          tau = row8_sum(tau);
          if ((threadIdx.x & 7) == 0) p.tau[po0 + 64 * j + r0 + rr] = tau;
        }
      }
    } else {
      constexpr int j = sg.j;
      f32x16& ac = acc[j & 1];
      mma_tile<TM, LD>(ac, ab[k & 1], ub[(sg.i + 1) & 1], wm, wn, lane, 64);
      if constexpr (sg.i == sg.j) {
        // dx = step du + D gy, and the row sums x.du and u.du of tile j
        const int64_t ts0 = tc + 64 * j;
        acc_to_lds(red, ac, wm, wn, lane);
        zero(ac);
        __syncthreads();
        float du[2][8], dxo[2][8];
        lds_block(red, r0, c0, du[0], du[1]);
        const float4 da = *reinterpret_cast<const float4*>(dcol + c0);
        const float4 db = *reinterpret_cast<const float4*>(dcol + c0 + 4);
        const float dv[8] = {da.x, da.y, da.z, da.w, db.x, db.y, db.z, db.w};
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          float gf[8], xf[8], uf[8];
          v8_f32(gv[rr], gf);
          u8(j, xs[j & 1], rr, xf, uf);
          const float d = dlc[64 * j + r0 + rr];
          float sx = 0.0f, su = 0.0f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            dxo[rr][e] = fmaf(dv[e], gf[e], d * du[rr][e]);
            sx = fmaf(xf[e], du[rr][e], sx);
            su = fmaf(uf[e], du[rr][e], su);
          }
          sx = row8_sum(sx);
          su = row8_sum(su);
          if ((threadIdx.x & 7) == 0) {
            p.dsx[po0 + 64 * j + r0 + rr] = sx;
            p.ut[po0 + 64 * j + r0 + rr] = su;
          }
        }
        store_xw<TM, VEC, true>(g, static_cast<TM*>(p.dx), b, ts0, h, pc0, dxo[0], dxo[1]);
      }
    }
    if constexpr (sg.load == 1) {
      load_xw<TM, VEC>(g, gy, b, tc + 128, h, pc0, gv);
    } else if constexpr (sg.load == 2) {
      load_xw<TM, VEC>(g, gy, b, tc + 192, h, pc0, gv);
      load_xw<TM, VEC>(g, X, b, tc + 64, h, pc0, xs[1]);
      load_xw<TM, VEC>(g, X, b, tc, h, pc0, xs[0]);
    } else if constexpr (sg.load == 3) {
      load_xw<TM, VEC>(g, gy, b, tc + 128, h, pc0, gv);
    } else if constexpr (sg.load == 4) {
      load_xw<TM, VEC>(g, gy, b, tc + 64, h, pc0, gv);
    } else if constexpr (sg.load == 5) {
      load_xw<TM, VEC>(g, gy, b, tc, h, pc0, gv);
    } else if constexpr (sg.load == 6) {
#pragma unroll
      for (int k = 0; k < 2; ++k) load_sw<TM, VEC>(g, G, pc0, 64 * k, sv[k]);
    }
  });
}

// Adjoint of C.B^T for one lower tile (i, j) of a chunk, summed over a block of the
// group's heads: sum_h (gy_i u_j^T) o e^{cs_l - cs_s}.
template <typename TM, bool VEC>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) dcb_kernel(Geo g, BwdPlan pl, Ptrs p) {
  constexpr int TE = LdsTile<TM>::elems;
  __shared__ __align__(16) TM sbuf[2][2 * TE];
  __shared__ float csr[2][64], css[2][64];
  const WgId id = wg_id(pl.npairs * pl.hb1, g.nc * g.ngroups);
  const int pair = id.x / pl.hb1, hb = id.x % pl.hb1;
  int i = 0;
  while ((i + 1) * (i + 2) / 2 <= pair) ++i;
  const int j = pair - i * (i + 1) / 2;
  const int c = id.y / g.ngroups;
  const int64_t gg = id.y % g.ngroups, b = id.z;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int r0 = blk_r0(), c0 = blk_c0();
  const int64_t tc = static_cast<int64_t>(c) * g.q;
  const int64_t h0 = gg * g.hpg + static_cast<int64_t>(hb) * pl.hpb1;
  const int64_t hend = (gg + 1) * g.hpg;
  const int nh = static_cast<int>((h0 + pl.hpb1 < hend ? h0 + pl.hpb1 : hend) - h0);
  const int nst = nh * g.npt;
  const TM* gy = static_cast<const TM*>(p.gy);
  const TM* X = static_cast<const TM*>(p.x);
  struct Regs {
    V8<TM> gm[2], xm[2];
    float dls[2], cr, cc;
  };
  auto fetch = [&](int k, Regs& r) {
    const int hh = k / g.npt, pt = k % g.npt;
    const int64_t h = h0 + hh;
    const int64_t so = ((b * g.nheads + h) * g.nc + c) * g.q;
    load_xw<TM, VEC>(g, gy, b, tc + 64 * i, h, pt * 64, r.gm);  // gy rows l
    load_xw<TM, VEC>(g, X, b, tc + 64 * j, h, pt * 64, r.xm);   // x rows s
    r.dls[0] = p.dl[so + 64 * j + r0];
    r.dls[1] = p.dl[so + 64 * j + r0 + 1];
    r.cr = p.cs[so + 64 * i + lane];
    r.cc = p.cs[so + 64 * j + lane];
  };
  auto put = [&](int k, Regs& r) {
    const int hh = k / g.npt, pt = k % g.npt;
    TM* buf = sbuf[k & 1];
    float a[8], bb[8];
    put_raw<TM, false>(buf, r0, c0, r.gm[0], r.gm[1]);  // A[l][p] = gy_l[p]
    scale8(r.xm[0], r.dls[0], a);
    scale8(r.xm[1], r.dls[1], bb);
    put2x8<TM, false>(buf + TE, r0, c0, a, bb);  // Bt[s][p] = step_s x_s[p]
    if (pt == 0 && threadIdx.x < 64) {
      csr[hh & 1][threadIdx.x] = r.cr;
      css[hh & 1][threadIdx.x] = r.cc;
    }
  };
  f32x16 dacc;
  zero(dacc);
  if (i == j) {
    // diagonal tile: per head, the product times e^{cs_l - cs_s} below the diagonal
    f32x16 w;
    zero(w);
    Regs ra, rb;
    pipeline2(nst, ra, rb, fetch, put, [&](int k) {
      const int hh = k / g.npt, pt = k % g.npt;
      mma_tile<TM>(w, sbuf[k & 1], sbuf[k & 1] + TE, wm, wn, lane, 64);
      if (pt == g.npt - 1) {
        const float cs_s = css[hh & 1][acc_col(wn, lane)];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int l = acc_row(wm, lane, r), s = acc_col(wn, lane);
          if (s <= l) dacc[r] = fmaf(w[r], fast_exp(csr[hh & 1][l] - cs_s), dacc[r]);
        }
        zero(w);
      }
    });
  } else {
    // i > j: e^{cs_l - cs_s} = e^{cs_l - cs_e} e^{cs_e - cs_s} (e = the last token of
    // tile j, both factors at most 1 for a non-increasing cs) goes into the operands'
    // rows, and the products of all heads accumulate in the matrix cores.
    struct RegsO {
      V8<TM> gm[2], xm[2];
      float dls[2], ci[2], cj[2], ce;
    };
    auto fetch_o = [&](int k, RegsO& r) {
      const int hh = k / g.npt, pt = k % g.npt;
      const int64_t h = h0 + hh;
      const int64_t so = ((b * g.nheads + h) * g.nc + c) * g.q;
      load_xw<TM, VEC>(g, gy, b, tc + 64 * i, h, pt * 64, r.gm);  // gy rows l
      load_xw<TM, VEC>(g, X, b, tc + 64 * j, h, pt * 64, r.xm);   // x rows s
      r.dls[0] = p.dl[so + 64 * j + r0];
      r.dls[1] = p.dl[so + 64 * j + r0 + 1];
      r.ci[0] = p.cs[so + 64 * i + r0];
      r.ci[1] = p.cs[so + 64 * i + r0 + 1];
      r.cj[0] = p.cs[so + 64 * j + r0];
      r.cj[1] = p.cs[so + 64 * j + r0 + 1];
      r.ce = p.cs[so + 64 * j + 63];
    };
    auto put_o = [&](int k, RegsO& r) {
      TM* buf = sbuf[k & 1];
      float a[8], bb[8];
      scale8(r.gm[0], fast_exp(r.ci[0] - r.ce), a);
      scale8(r.gm[1], fast_exp(r.ci[1] - r.ce), bb);
      put2x8<TM, false>(buf, r0, c0, a, bb);  // A[l][p] = e^{cs_l - cs_e} gy_l[p]
      scale8(r.xm[0], r.dls[0] * fast_exp(r.ce - r.cj[0]), a);
      scale8(r.xm[1], r.dls[1] * fast_exp(r.ce - r.cj[1]), bb);
      put2x8<TM, false>(buf + TE, r0, c0, a, bb);  // Bt[s][p] = e^{cs_e - cs_s} step_s x_s[p]
    };
    RegsO ra, rb;
    pipeline2(nst, ra, rb, fetch_o, put_o,
              [&](int k) { mma_tile<TM>(dacc, sbuf[k & 1], sbuf[k & 1] + TE, wm, wn, lane, 64); });
  }
  float* out = p.dcb + (((b * g.nc + c) * g.ngroups + gg) * pl.hb1 + hb) * g.q * g.q;
#pragma unroll
  for (int r = 0; r < 16; ++r)
    out[(64 * i + acc_row(wm, lane, r)) * g.q + 64 * j + acc_col(wn, lane)] = dacc[r];
}

// State terms of dB (which 0: sum_h e^{T - cs_s} step_s x_s G) and dC (which 1:
// sum_h e^{cs_l} gy_l S_in) for one 64-token tile and two d_state tiles, over a
// block of the group's heads.
template <typename TM, bool VEC>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(sizeof(TM) == 2 ? 3 : 1)))
dbc_state(Geo g, BwdPlan pl, Ptrs p) {
  constexpr int LD = compact_ld<TM>();  // LDS bounds this kernel: the compact tiles
  constexpr int TE = LdsTile<TM, LD>::elems;
  __shared__ __align__(16) TM sbuf[2][3 * TE];
  const WgId id = wg_id(g.qb * g.nnp * 2 * pl.hb2, g.nc * g.ngroups);
  int idx = id.x;
  const int hb = idx % pl.hb2;
  idx /= pl.hb2;
  const int which = idx % 2;
  idx /= 2;
  const int np = idx % g.nnp, tt = idx / g.nnp;
  const int c = id.y / g.ngroups;
  const int64_t gg = id.y % g.ngroups, b = id.z;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int r0 = blk_r0(), c0 = blk_c0();
  const int64_t tl0 = static_cast<int64_t>(c) * g.q + 64 * tt;
  const int64_t nn0 = static_cast<int64_t>(np) * 128;
  const int64_t h0 = gg * g.hpg + static_cast<int64_t>(hb) * pl.hpb2;
  const int64_t hend = (gg + 1) * g.hpg;
  const int nh = static_cast<int>((h0 + pl.hpb2 < hend ? h0 + pl.hpb2 : hend) - h0);
  const int nst = nh * g.npt;
  const TM* src = static_cast<const TM*>(which ? p.gy : p.x);
  const TM* stm = static_cast<const TM*>(which ? p.states : p.dstates);
  struct Regs {
    V8<TM> src[2], s0[2], s1[2];
    float cl[2], dl[2], T;
  };
  auto fetch = [&](int k, Regs& r) {
    const int hh = k / g.npt, pt = k % g.npt;
    const int64_t h = h0 + hh, bh = b * g.nheads + h;
    const int64_t so = (bh * g.nc + c) * g.q;
    // x / gy and the states stream through once (no later kernel reads them again): nontemporal
    load_xw<TM, VEC, true>(g, src, b, tl0, h, pt * 64, r.src);  // rows l
    const TM* st = stm + (bh * g.nc + c) * g.headdim * g.dstate;
    load_sw<TM, VEC, true>(g, st, pt * 64, nn0, r.s0);  // rows p
    load_sw<TM, VEC, true>(g, st, pt * 64, nn0 + 64, r.s1);
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      r.cl[rr] = p.cs[so + 64 * tt + r0 + rr];
      r.dl[rr] = p.dl[so + 64 * tt + r0 + rr];
    }
    r.T = p.cs[so + g.q - 1];
  };
  auto put = [&](int k, Regs& r) {
    TM* buf = sbuf[k & 1];
    float a[8], bb[8];
    const float sc0 = which ? fast_exp(r.cl[0]) : r.dl[0] * fast_exp(r.T - r.cl[0]);
    const float sc1 = which ? fast_exp(r.cl[1]) : r.dl[1] * fast_exp(r.T - r.cl[1]);
    scale8(r.src[0], sc0, a);
    scale8(r.src[1], sc1, bb);
    put2x8<TM, false, LD>(buf, r0, c0, a, bb);                    // A[l][p]
    put_raw<TM, true, LD>(buf + TE, r0, c0, r.s0[0], r.s0[1]);      // Bt[n][p] = S[p][n]
    put_raw<TM, true, LD>(buf + 2 * TE, r0, c0, r.s1[0], r.s1[1]);
  };
  f32x16 acc0, acc1;
  zero(acc0);
  zero(acc1);
  Regs ra, rb;
  pipeline2(nst, ra, rb, fetch, put, [&](int k) {
    TM* buf = sbuf[k & 1];
    mma_tile<TM, LD>(acc0, buf, buf + TE, wm, wn, lane, 64);
    mma_tile<TM, LD>(acc1, buf, buf + 2 * TE, wm, wn, lane, 64);
  });
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t t = tl0 + acc_row(wm, lane, r);
    const int64_t nn = nn0 + acc_col(wn, lane);
    if (t >= g.length) continue;
    float* out = p.pbc + ((((b * g.length + t) * g.ngroups + gg) * pl.hb2 + hb) * 2 + which) * g.dstate;
    if (nn < g.dstate) out[nn] = acc0[r];
    if (nn + 64 < g.dstate) out[nn + 64] = acc1[r];
  }
}

// dC = dCB B (which 1) and dB = dCB^T C (which 0) for one 64-token tile and two
// d_state tiles, plus the head-block partials of the state terms.
template <typename TM, bool VEC>
__global__ void __launch_bounds__(256) dbc_final(Geo g, BwdPlan pl, Ptrs p) {
  constexpr int TE = LdsTile<TM>::elems;
  __shared__ __align__(16) TM sbuf[2][3 * TE];
  const WgId id = wg_id(g.qb * g.nnp * 2, g.nc * g.ngroups);
  int idx = id.x;
  const int which = idx % 2;
  idx /= 2;
  const int np = idx % g.nnp, tt = idx / g.nnp;
  const int c = id.y / g.ngroups;
  const int64_t gg = id.y % g.ngroups, b = id.z;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int r0 = blk_r0(), c0 = blk_c0();
  const int64_t tc = static_cast<int64_t>(c) * g.q;
  const int64_t nn0 = static_cast<int64_t>(np) * 128;
  const int64_t qq = static_cast<int64_t>(g.q) * g.q;
  const float* dcb = p.dcb + ((b * g.nc + c) * g.ngroups + gg) * pl.hb1 * qq;
  const TM* Om = static_cast<const TM*>(which ? p.B : p.C);  // the other operand
  const int nst = which ? tt + 1 : g.qb - tt;
  struct Regs {
    float kf[2][8];
    V8<TM> o0[2], o1[2];
  };
  auto fetch = [&](int k, Regs& r) {
    // which 1: rows l of tile tt, columns s of tile k;  which 0: rows l of tile tt + k, columns s of tile tt
    const int lt = which ? tt : tt + k, st = which ? k : tt;
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const float* row = dcb + (64 * lt + r0 + rr) * g.q + 64 * st + c0;
      load_f8(row, r.kf[rr]);
      for (int hb = 1; hb < pl.hb1; ++hb) {
        float f[8];
        load_f8(row + hb * qq, f);
#pragma unroll
        for (int e = 0; e < 8; ++e) r.kf[rr][e] += f[e];
      }
    }
    const int64_t ot0 = tc + 64 * (which ? st : lt);  // token rows of the other operand
    load_bw<TM, VEC>(g, Om, b, ot0, gg, nn0, r.o0);
    load_bw<TM, VEC>(g, Om, b, ot0, gg, nn0 + 64, r.o1);
  };
  auto put = [&](int k, Regs& r) {
    TM* buf = sbuf[k & 1];
    if (which)
      put2x8<TM, false>(buf, r0, c0, r.kf[0], r.kf[1]);  // A[l][s] = dCB[l][s]
    else
      put2x8<TM, true>(buf, r0, c0, r.kf[0], r.kf[1]);   // A[s][l] = dCB[l][s]
    put_raw<TM, true>(buf + TE, r0, c0, r.o0[0], r.o0[1]);  // Bt[n][token] of B (which 1) or C (which 0)
    put_raw<TM, true>(buf + 2 * TE, r0, c0, r.o1[0], r.o1[1]);
  };
  f32x16 acc0, acc1;
  zero(acc0);
  zero(acc1);
  Regs ra, rb;
  pipeline2(nst, ra, rb, fetch, put, [&](int k) {
    TM* buf = sbuf[k & 1];
    mma_tile<TM>(acc0, buf, buf + TE, wm, wn, lane, 64);
    mma_tile<TM>(acc1, buf, buf + 2 * TE, wm, wn, lane, 64);
  });
  __syncthreads();
  float* red = reinterpret_cast<float*>(&sbuf[0][0]);
  TM* out = static_cast<TM*>(which ? p.dC : p.dB);
  const int64_t t0 = tc + 64 * tt;
  for (int half = 0; half < 2; ++half) {
    if (half) __syncthreads();
    acc_to_lds(red, half ? acc1 : acc0, wm, wn, lane);
    __syncthreads();
    float v[2][8];
    lds_block(red, r0, c0, v[0], v[1]);
    const int64_t nn = nn0 + 64 * half + c0;
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int64_t t = t0 + r0 + rr;
      const int n = t < g.length ? static_cast<int>(g.dstate - nn) : 0;
      if (n <= 0) continue;
      const float* part = p.pbc + (((b * g.length + t) * g.ngroups + gg) * pl.hb2 * 2 + which) * g.dstate + nn;
      for (int hb = 0; hb < pl.hb2; ++hb) {
        float f[8];
        if (VEC) {
          load_f8(part + static_cast<int64_t>(hb) * 2 * g.dstate, f);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) f[e] = e < n ? part[static_cast<int64_t>(hb) * 2 * g.dstate + e] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) v[rr][e] += f[e];
      }
    }
    store_bw<TM, VEC>(g, out, b, t0, gg, nn0 + 64 * half, v[0], v[1]);
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
    for (int pt = 0; pt < g.npt; ++pt) {
      const int64_t o = ((bh * g.nc + c) * g.npt + pt) * g.q + l;
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
  // dD: (b, chunk, tile) partial rows; 64 columns x 4 row groups per pass
  __shared__ float part[4][64];
  const int64_t nrow = nbc * g.qb;
  const int col = tid & 63, grp = tid >> 6;
  float hsum = 0.0f;
  for (int pt = 0; pt < g.npt; ++pt) {
    const int64_t pc = static_cast<int64_t>(pt) * 64 + col;
    // rows grp, grp + 4, ... in 16 chains, so that 16 loads are in flight per thread
    float sv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) sv[e] = 0.0f;
    if (pc < g.headdim) {
      const float* q = p.pdD + h * g.headdim + pc;
      const int64_t stride = g.nheads * g.headdim;
      int64_t k = grp;
      for (; k + 60 < nrow; k += 64) {
        float v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = q[(k + 4 * e) * stride];
#pragma unroll
        for (int e = 0; e < 16; ++e) sv[e] += v[e];
      }
      for (; k < nrow; k += 4) sv[0] += q[k * stride];
    }
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
      for (int e = 0; e < w; ++e) sv[e] += sv[e + w];
    __syncthreads();
    part[grp][col] = sv[0];
    __syncthreads();
    if (tid < 64 && pc < g.headdim) {
      const float tot = (part[0][col] + part[1][col]) + (part[2][col] + part[3][col]);
      if (g.d_per_row)
        p.dD[h * g.headdim + pc] = tot;
      else
        hsum += tot;
    }
  }
  if (!g.d_per_row) {
    hsum = block_sum(hsum, wsum);
    if (tid == 0) p.dD[h] = hsum;
  }
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

BwdPlan make_plan(const Geo& g) {
  BwdPlan pl{};
  pl.nblk = static_cast<int>(cdiv(g.headdim * g.dstate, 2048));
  pl.npairs = g.qb * (g.qb + 1) / 2;
  // Split the head sums only as far as each launch needs to reach about 512 workgroups: every
  // split adds a partial that dbc_final reads back (at 4 x 4096 tokens, 64 heads, d_state 128,
  // splitting to 2048 workgroups cost 0.025 ms more in dbc_final and dbc_state than it saved
  // in dcb).
  const int64_t base1 = std::max<int64_t>(1, g.batch * g.nc * g.ngroups * pl.npairs);
  pl.hb1 = static_cast<int>(std::min<int64_t>(g.hpg, std::max<int64_t>(1, cdiv(512, base1))));
  pl.hpb1 = static_cast<int>(cdiv(g.hpg, pl.hb1));
  pl.hb1 = static_cast<int>(cdiv(g.hpg, pl.hpb1));
  const int64_t base2 = std::max<int64_t>(1, g.batch * g.nc * g.ngroups * g.qb * g.nnp * 2);
  pl.hb2 = static_cast<int>(std::min<int64_t>(g.hpg, std::max<int64_t>(1, cdiv(512, base2))));
  pl.hpb2 = static_cast<int>(cdiv(g.hpg, pl.hb2));
  pl.hb2 = static_cast<int>(cdiv(g.hpg, pl.hpb2));
  return pl;
}

BwdLayout bwd_layout(const Geo& g, const BwdPlan& pl, bool has_z) {
  BwdLayout l{};
  const size_t bh = static_cast<size_t>(g.batch * g.nheads);
  const size_t chunks = bh * g.nc;
  size_t o = 0;
  const size_t es = dtype_size(g.x_dtype);
  l.gy = o; o = align256(o + (has_z ? static_cast<size_t>(g.batch * g.length * g.nheads * g.headdim) * es : 0));
  l.dstates = o; o = align256(o + chunks * g.headdim * g.dstate * es);
  l.dT = o; o = align256(o + chunks * pl.nblk * 4);
  l.ya = o; o = align256(o + chunks * g.npt * g.q * 4);
  l.dsx = o; o = align256(o + chunks * g.npt * g.q * 4);
  l.ut = o; o = align256(o + chunks * g.npt * g.q * 4);
  l.tau = o; o = align256(o + chunks * g.npt * g.q * 4);
  l.pdD = o; o = align256(o + chunks * g.qb * g.headdim * 4);
  l.dcb = o; o = align256(o + static_cast<size_t>(g.batch) * g.nc * g.ngroups * pl.hb1 * g.q * g.q * 4);
  l.pbc = o; o = align256(o + static_cast<size_t>(g.batch * g.length * g.ngroups) * pl.hb2 * 2 * g.dstate * 4);
  l.pA = o; o = align256(o + chunks * 4);
  l.pbias = o; o = align256(o + chunks * 4);
  l.total = o;
  return l;
}

// The fused gate and local state adjoint (multi-tile geometries); false if the geometry
// takes the separate kernels.
template <typename TM, bool VEC>
bool launch_gate_state(const Geo& g, const BwdPlan& pl, const Ptrs& q, hipStream_t s) {
  if constexpr (sizeof(TM) == 2) {
    if (!multi_tile(g)) return false;
    const dim3 grid(static_cast<unsigned>(g.npt * g.nc * g.batch * g.nheads));
    if (g.qb == 4 && g.nnt == 2) MKO_TIMED("ssd_gate_state", s, gate_state_mt<TM, VEC, 4, 2><<<grid, 256, 0, s>>>(g, pl, q));
    else if (g.qb == 4) MKO_TIMED("ssd_gate_state", s, gate_state_mt<TM, VEC, 4, 1><<<grid, 256, 0, s>>>(g, pl, q));
    else if (g.qb == 2 && g.nnt == 2) MKO_TIMED("ssd_gate_state", s, gate_state_mt<TM, VEC, 2, 2><<<grid, 256, 0, s>>>(g, pl, q));
    else if (g.qb == 2) MKO_TIMED("ssd_gate_state", s, gate_state_mt<TM, VEC, 2, 1><<<grid, 256, 0, s>>>(g, pl, q));
    else if (g.nnt == 2) MKO_TIMED("ssd_gate_state", s, gate_state_mt<TM, VEC, 1, 2><<<grid, 256, 0, s>>>(g, pl, q));
    else MKO_TIMED("ssd_gate_state", s, gate_state_mt<TM, VEC, 1, 1><<<grid, 256, 0, s>>>(g, pl, q));
    return true;
  }
  return false;
}

template <typename TM, bool VEC>
void launch_du(const Geo& g, const BwdPlan& pl, const Ptrs& q, hipStream_t s) {
  const unsigned bh = static_cast<unsigned>(g.batch * g.nheads);
  if constexpr (sizeof(TM) == 2) {
    const dim3 grid(g.npt * g.nc * bh);
    if (multi_tile(g) && g.qb == 4 && g.nnt == 2 && g.dstate == 128) {
      MKO_TIMED("ssd_du", s, du_cm<TM, VEC><<<grid, 256, 0, s>>>(g, pl, q));
      return;
    }
    if (multi_tile(g)) {
      if (g.qb == 4 && g.nnt == 2) MKO_TIMED("ssd_du", s, du_mt<TM, VEC, 4, 2><<<grid, 256, 0, s>>>(g, pl, q));
      else if (g.qb == 4) MKO_TIMED("ssd_du", s, du_mt<TM, VEC, 4, 1><<<grid, 256, 0, s>>>(g, pl, q));
      else if (g.qb == 2 && g.nnt == 2) MKO_TIMED("ssd_du", s, du_mt<TM, VEC, 2, 2><<<grid, 256, 0, s>>>(g, pl, q));
      else if (g.qb == 2) MKO_TIMED("ssd_du", s, du_mt<TM, VEC, 2, 1><<<grid, 256, 0, s>>>(g, pl, q));
      else if (g.nnt == 2) MKO_TIMED("ssd_du", s, du_mt<TM, VEC, 1, 2><<<grid, 256, 0, s>>>(g, pl, q));
      else MKO_TIMED("ssd_du", s, du_mt<TM, VEC, 1, 1><<<grid, 256, 0, s>>>(g, pl, q));
      return;
    }
  }
  MKO_TIMED("ssd_du", s, du_kernel<TM, VEC><<<dim3((g.qb + 1) / 2 * g.npt * g.nc * bh), 256, 0, s>>>(g, pl, q));
}

// The backward's second stream on each device: one non-blocking stream at the default
// priority and its events, created on first use and kept until the process ends.
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
std::mutex g_side_mu;  // guards g_side and keeps each call's event records next to their waits
std::vector<SideStream> g_side;  // per device ordinal

// The current device's side stream in *out (created on first use), or null while s is being
// captured into a graph, where creating it is not allowed: the caller then runs everything
// on s.  Call with g_side_mu held.
int side_stream(hipStream_t s, SideStream** out) {
  *out = nullptr;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t err = hipStreamIsCapturing(s, &cap);
  if (err != hipSuccess) {
    mko_set_error("ssd_bwd: stream capture status: %s", hipGetErrorString(err));
    return MKO_ELAUNCH;
  }
  if (cap != hipStreamCaptureStatusNone) return MKO_OK;
  int dev = -1;
  err = hipGetDevice(&dev);
  if (err != hipSuccess || dev < 0) {
    mko_set_error("ssd_bwd: no current device: %s", hipGetErrorString(err));
    return MKO_ELAUNCH;
  }
  if (static_cast<size_t>(dev) >= g_side.size()) g_side.resize(dev + 1);
  SideStream& sd = g_side[dev];
  if (!sd.stream) {
    SideStream made;
    err = hipStreamCreateWithFlags(&made.stream, hipStreamNonBlocking);
    for (hipEvent_t* e : {&made.fork, &made.join})
      if (err == hipSuccess) err = hipEventCreateWithFlags(e, hipEventDisableTiming);
    if (err != hipSuccess) {
      mko_set_error("ssd_bwd: second stream on device %d: %s", dev, hipGetErrorString(err));
      for (hipEvent_t e : {made.fork, made.join})
        if (e) (void)hipEventDestroy(e);
      if (made.stream) (void)hipStreamDestroy(made.stream);
      return MKO_ELAUNCH;
    }
    sd = made;
  }
  *out = &sd;
  return MKO_OK;
}

// Makes `to` wait for the work queued on `from` so far, through event e.
int stream_wait(hipStream_t from, hipStream_t to, hipEvent_t e) {
  hipError_t err = hipEventRecord(e, from);
  if (err == hipSuccess) err = hipStreamWaitEvent(to, e, 0);
  if (err != hipSuccess) {
    mko_set_error("ssd_bwd: ordering of the two streams: %s", hipGetErrorString(err));
    return MKO_ELAUNCH;
  }
  return MKO_OK;
}

// The kernels after the gate, in two streams.  dcb reads only gy and the forward's inputs
// and writes only partials that dbc_final reads, so the side stream runs it as soon as the
// gate is done, beside state_rev, du, dbc_state, finish and reduce_params on s, and s waits
// for it just before dbc_final.  Alone at 4 x 4096 tokens and 64 heads, dcb's 640 long
// workgroups leave about 40% of the workgroup slots empty for 0.12 ms.  (dbc_state could
// follow it there once state_rev is done; it runs faster on s, where it does not compete with
// du.)  Calls from several host threads share the side stream: the lock keeps each fork
// record next to its wait, and a join that waits for a later call's work on the same stream
// also waits for its own.
template <typename TM, bool VEC>
int launch_bwd_t(const Geo& g, const BwdPlan& pl, const Ptrs& q, hipStream_t s) {
  const unsigned bh = static_cast<unsigned>(g.batch * g.nheads);
  const unsigned ncg = static_cast<unsigned>(g.nc * g.ngroups);
  const unsigned nb = static_cast<unsigned>(g.batch);
  if (!launch_gate_state<TM, VEC>(g, pl, q, s)) {
    if (q.yt)
      MKO_TIMED("ssd_gate", s, gate<TM, VEC, true><<<dim3(g.qb * g.npt * g.nc * bh), 256, 0, s>>>(g, pl, q));
    else
      MKO_TIMED("ssd_gate", s, gate<TM, VEC, false><<<dim3(g.qb * g.npt * g.nc * bh), 256, 0, s>>>(g, pl, q));
    const dim3 cs_grid(g.npt * g.nnp * g.nc * bh);
    if (g.qb == 4)
      MKO_TIMED("ssd_chunk_state_bwd", s, chunk_state<TM, VEC, true, 4><<<cs_grid, 256, 0, s>>>(g, q, q.dstates));
    else
      MKO_TIMED("ssd_chunk_state_bwd", s, chunk_state<TM, VEC, true><<<cs_grid, 256, 0, s>>>(g, q, q.dstates));
  }
  auto dcb = [&](hipStream_t st) {
    MKO_TIMED("ssd_dcb", st, dcb_kernel<TM, VEC><<<dim3(pl.npairs * pl.hb1 * ncg * nb), 256, 0, st>>>(g, pl, q));
  };
  hipEvent_t join = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_side_mu);
    SideStream* sd = nullptr;
    int err = side_stream(s, &sd);
    if (err != MKO_OK) return err;
    if (sd) {
      if ((err = stream_wait(s, sd->stream, sd->fork)) != MKO_OK) return err;
      dcb(sd->stream);
      const hipError_t e = hipEventRecord(sd->join, sd->stream);
      if (e != hipSuccess) {
        mko_set_error("ssd_bwd: join event of the second stream: %s", hipGetErrorString(e));
        return MKO_ELAUNCH;
      }
      join = sd->join;
    }
  }
  MKO_TIMED("ssd_state_rev", s, state_rev<TM><<<dim3(pl.nblk, bh), 256, 0, s>>>(g, pl, q));
  launch_du<TM, VEC>(g, pl, q, s);
  if (!join) dcb(s);
  MKO_TIMED("ssd_dbc_state", s,
            dbc_state<TM, VEC><<<dim3(g.qb * g.nnp * 2 * pl.hb2 * ncg * nb), 256, 0, s>>>(g, pl, q));
  MKO_TIMED("ssd_finish", s,
            finish<<<dim3(g.nc, static_cast<unsigned>(g.nheads), nb), 256, 0, s>>>(g, pl, q));
  MKO_TIMED("ssd_reduce", s, reduce_params<<<dim3(static_cast<unsigned>(g.nheads)), 256, 0, s>>>(g, pl, q));
  if (join) {
    const hipError_t e = hipStreamWaitEvent(s, join, 0);
    if (e != hipSuccess) {
      mko_set_error("ssd_bwd: join of the second stream: %s", hipGetErrorString(e));
      return MKO_ELAUNCH;
    }
  }
  MKO_TIMED("ssd_dbc_final", s, dbc_final<TM, VEC><<<dim3(g.qb * g.nnp * 2 * ncg * nb), 256, 0, s>>>(g, pl, q));
  return MKO_OK;
}

template <typename TM>
int launch_bwd_t(const Geo& g, const BwdPlan& pl, const Ptrs& q, hipStream_t s) {
  return g.vec ? launch_bwd_t<TM, true>(g, pl, q, s) : launch_bwd_t<TM, false>(g, pl, q, s);
}

}  // namespace
}  // namespace ssd
}  // namespace mko

using namespace mko;
using namespace mko::ssd;

extern "C" size_t mko_ssd_bwd_workspace_size(const mko_ssd_params* prm) {
  if (prm && prm->x_dtype == MKO_F64) return ssd64_bwd_workspace_size(prm);
  Geo g;
  if (make_geo(prm, &g) != MKO_OK) return 0;
  return bwd_layout(g, make_plan(g), prm->z != nullptr).total;
}

extern "C" int mko_ssd_bwd(const mko_ssd_params* prm, void* stream) {
  if (prm && prm->x_dtype == MKO_F64) return ssd64_bwd(prm, static_cast<hipStream_t>(stream));
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
  q.dstates = ws + lay.dstates;
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
    if (g.x_dtype == MKO_F32) st = launch_bwd_t<float>(g, pl, q, s);
    else if (g.x_dtype == MKO_BF16) st = launch_bwd_t<bf16>(g, pl, q, s);
    else st = launch_bwd_t<_Float16>(g, pl, q, s);
    if (st != MKO_OK) return st;
  } else {
    // no tokens: dinitial = dfinal (zero without it); the parameter gradients are zero
    if (g.batch > 0 && q.dinit) {
      const dim3 grid(pl.nblk, static_cast<unsigned>(g.batch * g.nheads));
      if (g.x_dtype == MKO_F32) MKO_TIMED("ssd_state_rev", s, state_rev<float><<<grid, 256, 0, s>>>(g, pl, q));
      else if (g.x_dtype == MKO_BF16) MKO_TIMED("ssd_state_rev", s, state_rev<bf16><<<grid, 256, 0, s>>>(g, pl, q));
      else MKO_TIMED("ssd_state_rev", s, state_rev<_Float16><<<grid, 256, 0, s>>>(g, pl, q));
    }
    MKO_TIMED("ssd_reduce", s, reduce_params<<<dim3(static_cast<unsigned>(g.nheads)), 256, 0, s>>>(g, pl, q));
  }
  return mko_check_launch("ssd_bwd");
}
