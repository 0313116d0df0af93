// Shared declarations and device code of the SSD chunk-scan kernels
// (ssd.hip: forward, ssd_bwd.hip: backward).
//
// All activation-like tensors (x, z, dy, B, C, initial/final states and their
// gradients) share one storage type TM, the operand type of the matrix cores
// (float32, float16 or bfloat16); dt may differ.  Chunk states are stored in TM
// too: they are matrix-core operands and the reference rounds them the same way.
#pragma once

#include "common.hpp"
#include "io.hpp"
#include "mma.hpp"
#include "tile.hpp"

namespace mko {
namespace ssd {

struct Geo {
  int64_t batch, length, nheads, headdim, ngroups, dstate;
  int qb;   // 64-token tiles per chunk
  int q;    // chunk length, 64 * qb
  int nc;   // number of chunks
  int hpg;  // heads per group
  int npt;  // 64-wide d_head tiles
  int nnt;  // 64-wide d_state tiles
  int nnp;  // pairs of d_state tiles (a workgroup covers up to 128 states)
  int x_dtype, dt_dtype;
  int softplus, d_per_row, save_y;
  int vec;  // 16-byte vector access of 8-element runs is valid (P, N multiples of 8, aligned)
};

// Backward work split (ssd_bwd.hip).
struct BwdPlan {
  int nblk;       // 2048-element blocks of a (d_head x d_state) state
  int npairs;     // lower (l-tile, s-tile) pairs of a chunk
  int hb1, hpb1;  // head blocks (and heads per block) of the C.B^T adjoint
  int hb2, hpb2;  // head blocks (and heads per block) of the state terms of dB/dC
};

struct Ptrs {
  const void* x;
  const void* dt;
  const float* A;
  const void* B;
  const void* C;
  const float* D;
  const void* z;
  const float* bias;
  const void* init;
  void* y;
  void* final_state;
  const void* dy;
  const void* dfinal;
  void* dx;
  void* ddt;
  void* dz;
  void* dinit;
  float* dA;
  void* dB;
  void* dC;
  float* dD;
  float* dbias;
  // forward save area
  void* states;  // (b, H, nc, P, N) TM: state entering each chunk
  float* dl;     // (b, H, nc, q) step sizes (0 past the end)
  float* cs;     // (b, H, nc, q) cumulative step * A inside the chunk
  void* cb;      // (b, nc, G, q, q) TM: C . B^T, lower tiles
  float* yt;     // (b, L, H, P) chunk output before the skip and the gate (save_y), else null
  // backward workspace
  const void* gy;  // (b, L, H, P) TM: dy * silu(z) (dy itself without z)
  void* gyw;       // writable alias of gy when it is materialised
  void* dstates;   // (b, H, nc, P, N) TM: local state adjoints, then G, the adjoint of the state leaving each chunk
  float* dT;       // (b, H, nc, nblk) partial e^T <G, S_in> per state block
  float* ya;       // (b, H, nc, npt, q) partial gy . (y - D x) per d_head tile
  float* dsx;      // (b, H, nc, npt, q) partial x . du
  float* ut;       // (b, H, nc, npt, q) partial u . du (u as the matrix cores see it)
  float* tau;      // (b, H, nc, npt, q) partial u . du_state
  float* pdD;      // (b, nc, qb, H, P) dD partials per 64-token tile
  float* dcb;      // (b, nc, G, hb1, q, q) head-block partials of the C.B^T adjoint
  float* pbc;      // (b, L, G, hb2, 2, N) head-block partials of the state terms of dB (0) and dC (1)
  float* pA;       // (b, H, nc) dA partials
  float* pbias;    // (b, H, nc) ddt_bias partials
};

struct SavedLayout {
  size_t states, dl, cs, cb, yt, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

// 16-bit operands with d_state <= 128: one workgroup per (b, h, chunk, d_head tile) runs
// all of a chunk's token tiles (chunk_scan_mt, gate_state_mt, du_mt; at 256-token chunks
// with d_state 128 the scan and du run as chunk_scan_cm and du_cm), and the backward
// recomputes the chunk output instead of reading a saved copy.
inline bool multi_tile(const Geo& g) {
  return g.x_dtype != MKO_F32 && g.nnt <= 2 && (g.qb == 1 || g.qb == 2 || g.qb == 4);
}

int make_geo(const mko_ssd_params* prm, Geo* g);
SavedLayout saved_layout(const Geo& g);
void bind_saved(const Geo& g, void* saved, Ptrs* q);
Ptrs base_ptrs(const mko_ssd_params* prm);

// ------------------------------------------------------------ device helpers

__device__ __forceinline__ int64_t xidx(const Geo& g, int64_t b, int64_t t, int64_t h, int64_t pc) {
  return ((b * g.length + t) * g.nheads + h) * g.headdim + pc;
}
__device__ __forceinline__ int64_t bcidx(const Geo& g, int64_t b, int64_t t, int64_t gg, int64_t n) {
  return ((b * g.length + t) * g.ngroups + gg) * g.dstate + n;
}
__device__ __forceinline__ int clamp64(int64_t v) { return v >= 64 ? 64 : (v < 0 ? 0 : static_cast<int>(v)); }

// Writes an accumulator tile (value v[r] at (acc_row, acc_col)) to a 64x65 fp32 LDS tile.
template <typename V>
__device__ __forceinline__ void acc_to_lds(float* red, const V& v, int wm, int wn, int lane) {
#pragma unroll
  for (int r = 0; r < 16; ++r) red[acc_row(wm, lane, r) * 65 + acc_col(wn, lane)] = v[r];
}

// 64x64 windows of the problem's tensors; the base is uniform, each lane adds a
// 32-bit offset (load_win / store_win).
//   x-like (b, L, H, P): rows = tokens t0 .., columns = d_head pc0 ..
template <typename TM, bool VEC, bool NT = false>
__device__ __forceinline__ void load_xw(const Geo& g, const TM* src, int64_t b, int64_t t0, int64_t h, int64_t pc0,
                                        V8<TM> (&v)[2]) {
  load_win<TM, VEC, NT>(src + xidx(g, b, t0, h, pc0), static_cast<int>(g.nheads * g.headdim), clamp64(g.length - t0),
                    static_cast<int>(g.headdim - pc0), v, src);
}
template <typename TM, bool VEC, bool NT = false>
__device__ __forceinline__ void store_xw(const Geo& g, TM* dst, int64_t b, int64_t t0, int64_t h, int64_t pc0,
                                         const float (&a)[8], const float (&bb)[8]) {
  store_win<TM, VEC, NT>(dst + xidx(g, b, t0, h, pc0), static_cast<int>(g.nheads * g.headdim), clamp64(g.length - t0),
                     static_cast<int>(g.headdim - pc0), a, bb);
}
template <typename TM, bool VEC, bool NT = false>
__device__ __forceinline__ void store_xw_row(const Geo& g, TM* dst, int64_t b, int64_t t0, int64_t h, int64_t pc0,
                                             int rr, const float (&a)[8]) {
  store_win_row<TM, VEC, NT>(dst + xidx(g, b, t0, h, pc0), static_cast<int>(g.nheads * g.headdim),
                         clamp64(g.length - t0), static_cast<int>(g.headdim - pc0), rr, a);
}
//   B/C-like (b, L, G, N): rows = tokens t0 .., columns = d_state nn0 ..
template <typename TM, bool VEC, bool NT = false>
__device__ __forceinline__ void load_bw(const Geo& g, const TM* src, int64_t b, int64_t t0, int64_t gg, int64_t nn0,
                                        V8<TM> (&v)[2]) {
  load_win<TM, VEC, NT>(src + bcidx(g, b, t0, gg, nn0), static_cast<int>(g.ngroups * g.dstate), clamp64(g.length - t0),
                    static_cast<int>(g.dstate - nn0), v, src);
}
template <typename TM, bool VEC>
__device__ __forceinline__ void store_bw(const Geo& g, TM* dst, int64_t b, int64_t t0, int64_t gg, int64_t nn0,
                                         const float (&a)[8], const float (&bb)[8]) {
  store_win<TM, VEC>(dst + bcidx(g, b, t0, gg, nn0), static_cast<int>(g.ngroups * g.dstate), clamp64(g.length - t0),
                     static_cast<int>(g.dstate - nn0), a, bb);
}
//   a (P, N) state matrix: rows = d_head pc0 .., columns = d_state nn0 ..
template <typename TM, bool VEC, bool NT = false>
__device__ __forceinline__ void load_sw(const Geo& g, const TM* st, int64_t pc0, int64_t nn0, V8<TM> (&v)[2]) {
  load_win<TM, VEC, NT>(st + pc0 * g.dstate + nn0, static_cast<int>(g.dstate), clamp64(g.headdim - pc0),
                    static_cast<int>(g.dstate - nn0), v, st);
}

// 8 fp32 at p (32-byte aligned).
__device__ __forceinline__ void load_f8(const float* p, float (&f)[8]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

template <typename TM>
__device__ __forceinline__ void scale8(const V8<TM>& v, float s, float (&f)[8]) {
  v8_f32(v, f);
#pragma unroll
  for (int k = 0; k < 8; ++k) f[k] *= s;
}

// out[p][n] = sum_l s1(l) X(l, p) Y(l, n) over the chunk, for one 64-row d_head tile
// and two 64-column d_state tiles, stored in TM.
//   FWD: X = x, s1 = step e^{T - cs}, Y = B  -> local chunk state
//   BWD: X = gy, s1 = e^{cs}, Y = C          -> the chunk's own contribution to the
//        adjoint of its entering state
// Both operands are token-major in HBM and the contraction runs over tokens, so both
// are staged transposed.  Double-buffered: the loads of the next 64 tokens are in
// flight during the products of the current ones.
// QB > 0: the chunk has QB 64-token tiles (a compile-time stage count, with the loads of
// up to three stages in flight); QB = 0: qb at run time, two stages in flight.
template <typename TM, bool VEC, bool BWD, int QB = 0>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(sizeof(TM) == 2 ? 3 : 1)))
chunk_state(Geo g, Ptrs p, void* out_) {
  constexpr int LD = compact_ld<TM>();  // LDS bounds this kernel: the compact tiles
  constexpr int TE = LdsTile<TM, LD>::elems;
  __shared__ __align__(16) TM sbuf[2][3 * TE];
  __shared__ float s1[256];
  const WgId id = wg_id(g.npt * g.nnp, g.nc);
  const int pt = id.x / g.nnp, np = id.x % g.nnp;
  const int c = id.y;
  const int64_t bh = id.z, b = bh / g.nheads, h = bh % g.nheads, gg = h / g.hpg;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int r0 = blk_r0(), c0 = blk_c0();
  const int64_t so = (bh * g.nc + c) * g.q;
  const float T = p.cs[so + g.q - 1];
  for (int l = threadIdx.x; l < g.q; l += 256) {
    const bool ok = static_cast<int64_t>(c) * g.q + l < g.length;
    s1[l] = !ok ? 0.0f : (BWD ? fast_exp(p.cs[so + l]) : p.dl[so + l] * fast_exp(T - p.cs[so + l]));
  }
  const TM* X = static_cast<const TM*>(BWD ? p.gy : p.x);
  const TM* Y = static_cast<const TM*>(BWD ? p.C : p.B);
  const int64_t pc0 = static_cast<int64_t>(pt) * 64, nn0 = static_cast<int64_t>(np) * 128;
  struct Regs {
    V8<TM> x[2], y0[2], y1[2];
  };
  auto fetch = [&](auto kc, Regs& r) {
    const int kb = kc;
    const int64_t t0 = static_cast<int64_t>(c) * g.q + 64 * kb;
    load_xw<TM, VEC>(g, X, b, t0, h, pc0, r.x);
    load_bw<TM, VEC>(g, Y, b, t0, gg, nn0, r.y0);
    load_bw<TM, VEC>(g, Y, b, t0, gg, nn0 + 64, r.y1);
  };
  auto put = [&](auto kc, Regs& r) {
    const int kb = kc;
    TM* buf = sbuf[kb & 1];
    float a[8], bb[8];
    scale8(r.x[0], s1[64 * kb + r0], a);
    scale8(r.x[1], s1[64 * kb + r0 + 1], bb);
    put2x8<TM, true, LD>(buf, r0, c0, a, bb);                     // A[p][l]
    put_raw<TM, true, LD>(buf + TE, r0, c0, r.y0[0], r.y0[1]);      // Bt[n][l]
    put_raw<TM, true, LD>(buf + 2 * TE, r0, c0, r.y1[0], r.y1[1]);
  };
  f32x16 acc0, acc1;
  zero(acc0);
  zero(acc1);
  __syncthreads();  // s1
  auto mma = [&](auto kc) {
    TM* buf = sbuf[static_cast<int>(kc) & 1];
    mma_tile<TM, LD>(acc0, buf, buf + TE, wm, wn, lane, 64);
    mma_tile<TM, LD>(acc1, buf, buf + 2 * TE, wm, wn, lane, 64);
  };
  if constexpr (QB > 0) {
    constexpr int D = QB < 3 ? QB : 3;
    Regs regs[D];
    pipeline_static<QB, D>(regs, fetch, put, mma);
  } else {
    Regs ra, rb;
    pipeline2(g.qb, ra, rb, fetch, put, mma);
  }
  // the [p][n] tile leaves through LDS as 16-byte row runs, one 64-wide n-tile at a time
  TM* out = static_cast<TM*>(out_) + (bh * g.nc + c) * g.headdim * g.dstate + pc0 * g.dstate + nn0;
  float* red = reinterpret_cast<float*>(&sbuf[0][0]);
  static_assert(sizeof(sbuf) >= 64 * 65 * sizeof(float), "the fp32 tile fits the operand buffers");
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    __syncthreads();  // the last stage's products (kk 0), or the reads of the previous tile, are done
    acc_to_lds(red, kk == 0 ? acc0 : acc1, wm, wn, lane);
    __syncthreads();
    float v[2][8];
    lds_block(red, blk_r0(), blk_c0(), v[0], v[1]);
    store_win<TM, VEC>(out + 64 * kk, static_cast<int>(g.dstate), clamp64(g.headdim - pc0),
                       static_cast<int>(g.dstate - nn0 - 64 * kk), v[0], v[1]);
  }
}

// Loads cs and step of a whole chunk into LDS (q <= 256 values each), and the column
// decay factors ecol[s] = e^{cs_e - cs_s}, e = the last token of s's 64-token tile.
__device__ __forceinline__ void load_chunk_cs(const Geo& g, const Ptrs& p, int64_t bh, int c, float* csc, float* dlc,
                                              float* ecol) {
  const int64_t so = (bh * g.nc + c) * g.q;
  const int l = threadIdx.x;  // q <= 256
  if (l < g.q) {
    const float cs = p.cs[so + l];
    csc[l] = cs;
    dlc[l] = p.dl[so + l];
    ecol[l] = fast_exp(p.cs[so + (l | 63)] - cs);
  }
}

// The thread's block of K[l][s] = cb[l][s] e^{cs_l - cs_s} for rows l = 64i + r0, r0+1
// (a, bb) and columns s = 64j + c0 .. +7, from the raw cb block (ra, rb); zero above
// the diagonal of the diagonal tile.  Off the diagonal (i > j) the decay splits at the
// last token e of tile j, e^{cs_l - cs_e} e^{cs_e - cs_s}: one exponential per row and
// the column factors from ecol instead of one per element.  With a non-increasing cs
// (A step <= 0) both factors are at most 1, and one underflows only where the whole
// product does.  Every kernel that multiplies by K uses this routine, so the forward
// and the backward round the same K.
template <typename TM>
__device__ __forceinline__ void k_block(const V8<TM>& ra, const V8<TM>& rb, const float* csc, const float* ecol, int i,
                                        int j, int r0, int c0, float (&a)[8], float (&bb)[8]) {
  const float cl0 = csc[64 * i + r0], cl1 = csc[64 * i + r0 + 1];
  v8_f32(ra, a);
  v8_f32(rb, bb);
  if (i != j) {
    const float ref = csc[64 * j + 63];
    const float e0 = fast_exp(cl0 - ref), e1 = fast_exp(cl1 - ref);
    const float4 ea = *reinterpret_cast<const float4*>(ecol + 64 * j + c0);
    const float4 eb = *reinterpret_cast<const float4*>(ecol + 64 * j + c0 + 4);
    const float ec[8] = {ea.x, ea.y, ea.z, ea.w, eb.x, eb.y, eb.z, eb.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] = (a[e] * ec[e]) * e0;
      bb[e] = (bb[e] * ec[e]) * e1;
    }
  } else {
    const float4 cs_a = *reinterpret_cast<const float4*>(csc + 64 * j + c0);
    const float4 cs_b = *reinterpret_cast<const float4*>(csc + 64 * j + c0 + 4);
    const float css[8] = {cs_a.x, cs_a.y, cs_a.z, cs_a.w, cs_b.x, cs_b.y, cs_b.z, cs_b.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] *= fast_exp(cl0 - css[e]);
      bb[e] *= fast_exp(cl1 - css[e]);
      if (c0 + e > r0) a[e] = 0.0f;
      if (c0 + e > r0 + 1) bb[e] = 0.0f;
    }
  }
}

// Chunk output before the skip and the gate, for the 64-token tile i and d_head
// tile pt of head (bh) in chunk c:
//   acc[l][p] = sum_{s<=l} e^{cs_l - cs_s} CB[l][s] step_s x_s[p] + e^{cs_l} sum_n C_l[n] S_in[p][n]
// Stages 0..i are the intra-chunk tiles, then one stage per d_state tile.  csc/dlc/ecol
// hold the chunk's cs, step and column decay factors (load_chunk_cs, visible before the
// call).
// Ends with a barrier, so the caller may reuse sbuf.  With EPI the fetches past the last
// stage load the epilogue's inputs instead, x rows l and z rows l (x again without z), so
// that they arrive during the products, and epi(x, z) runs after that barrier.
struct NoEpi {
  template <class V>
  __device__ void operator()(const V&, const V&) const {}
};
template <typename TM, bool VEC, bool EPI = false, class Epi = NoEpi>
__device__ __forceinline__ void chunk_out(const Geo& g, const Ptrs& p, f32x16& acc, TM (*sbuf)[2 * LdsTile<TM>::elems],
                                          const float* csc, const float* dlc, const float* ecol, int i, int pt, int c,
                                          int64_t bh, Epi&& epi = NoEpi{}) {
  constexpr int TE = LdsTile<TM>::elems;
  const int64_t b = bh / g.nheads, h = bh % g.nheads, gg = h / g.hpg;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int r0 = blk_r0(), c0 = blk_c0();
  const int64_t tc = static_cast<int64_t>(c) * g.q;
  const int64_t pc0 = static_cast<int64_t>(pt) * 64;
  const TM* cbt = static_cast<const TM*>(p.cb) + ((b * g.nc + c) * g.ngroups + gg) * g.q * g.q;
  const TM* X = static_cast<const TM*>(p.x);
  const TM* Cm = static_cast<const TM*>(p.C);
  const TM* S = static_cast<const TM*>(p.states) + (bh * g.nc + c) * g.headdim * g.dstate;
  const float cl0 = csc[64 * i + r0], cl1 = csc[64 * i + r0 + 1];
  const float e0 = fast_exp(cl0), e1 = fast_exp(cl1);
  // Stages 0 .. nnt-1: state part, A = e^{cs_l} C_l[n], Bt = S_in[p][n];
  // stages nnt .. nnt+i: intra-chunk tiles j, A = K[l][s], Bt = step_s x_s[p].
  // Both kinds load two rows of two 64-wide windows, so the loads in flight are the
  // same on every path.
  struct Regs {
    V8<TM> a[2], b[2];
  };
  const int n = g.nnt + i + 1;
  auto fetch = [&](int k, Regs& r) {
    if (EPI && k == n) {
      load_xw<TM, VEC>(g, X, b, tc + 64 * i, h, pc0, r.a);                                   // x rows l
      load_xw<TM, VEC>(g, p.z ? static_cast<const TM*>(p.z) : X, b, tc + 64 * i, h, pc0, r.b);  // z rows l
    } else if (k < g.nnt) {
      load_bw<TM, VEC>(g, Cm, b, tc + 64 * i, gg, 64 * k, r.a);  // C rows l
      load_sw<TM, VEC>(g, S, pc0, 64 * k, r.b);                  // S rows p
    } else {
      const int j = k - g.nnt;
      load_win<TM, true>(cbt + (64 * i) * g.q + 64 * j, g.q, 64, 64, r.a, cbt);  // cb rows l
      load_xw<TM, VEC>(g, X, b, tc + 64 * j, h, pc0, r.b);                      // x rows s
    }
  };
  auto put = [&](int k, Regs& r) {
    TM* buf = sbuf[k & 1];
    float a[8], bb[8];
    if (k < g.nnt) {
      scale8(r.a[0], e0, a);
      scale8(r.a[1], e1, bb);
      put2x8<TM, false>(buf, r0, c0, a, bb);                  // A[l][n] = e^{cs_l} C_l[n]
      put_raw<TM, false>(buf + TE, r0, c0, r.b[0], r.b[1]);  // Bt[p][n] = S_in[p][n]
    } else {
      const int j = k - g.nnt;
      k_block<TM>(r.a[0], r.a[1], csc, ecol, i, j, r0, c0, a, bb);
      put2x8<TM, false>(buf, r0, c0, a, bb);  // A[l][s] = K
      scale8(r.b[0], dlc[64 * j + r0], a);
      scale8(r.b[1], dlc[64 * j + r0 + 1], bb);
      put2x8<TM, true>(buf + TE, r0, c0, a, bb);  // Bt[p][s] = step_s x_s[p]
    }
  };
  zero(acc);
  Regs ra, rb;
  auto mma = [&](int k) { mma_tile<TM>(acc, sbuf[k & 1], sbuf[k & 1] + TE, wm, wn, lane, 64); };
  if constexpr (EPI) {
    pipeline2e(n, ra, rb, fetch, put, mma, [&](const Regs& r) {
      __syncthreads();
      epi(r.a, r.b);
    });
  } else {
    pipeline2(n, ra, rb, fetch, put, mma);
    __syncthreads();
  }
}

// The skip weights D of the thread's 8 d_head columns (zero without D).
__device__ __forceinline__ void load_d8(const Geo& g, const Ptrs& p, int64_t h, int64_t pc, float (&d)[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float v = 0.0f;
    if (p.D) v = g.d_per_row ? (pc + k < g.headdim ? p.D[h * g.headdim + pc + k] : 0.0f) : p.D[h];
    d[k] = v;
  }
}

}  // namespace ssd
}  // namespace mko
