// Shared declarations and device helpers of the SSD chunk-scan kernels
// (ssd.hip: forward, ssd_bwd.hip: backward).
#pragma once

#include "common.hpp"
#include "io.hpp"
#include "mma.hpp"

namespace mko {
namespace ssd {

struct Geo {
  int64_t batch, length, nheads, headdim, ngroups, dstate;
  int qb;   // 64-token tiles per chunk
  int q;    // chunk length, 64 * qb
  int nc;   // number of chunks
  int hpg;  // heads per group
  int x_dtype, dt_dtype, bc_dtype;
  int softplus, d_per_row;
};

// Backward work split (ssd_bwd.hip).
struct BwdPlan {
  int npt;     // 64-wide d_head tiles
  int nnt;     // 64-wide d_state tiles
  int nblk;    // 256-element blocks of a (d_head x d_state) state
  int npairs;  // lower (l-tile, s-tile) pairs of a chunk
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
  float* states;  // (b, H, nc, P, N) state entering each chunk
  float* dl;      // (b, H, nc, q) step sizes (0 past the end)
  float* cs;      // (b, H, nc, q) cumulative step * A inside the chunk
  float* cb;      // (b, nc, G, q, q) C . B^T, lower tiles
  // backward workspace
  const void* gy;  // (b, L, H, P) x dtype: dy * silu(z) (dy itself without z)
  void* gyw;       // writable alias of gy when it is materialised
  float* dstates;  // (b, H, nc, P, N) local state adjoints, then the adjoint of the state leaving each chunk
  float* dT;       // (b, H, nc, nblk) partial e^T <G, S_in> per state block
  float* ya;       // (b, H, nc, npt, q) partial gy . (y - D x) per d_head tile
  float* dsx;      // (b, H, nc, npt, q) partial x . du per d_head tile
  float* ut;       // (b, H, nc, npt, q) partial u . du per d_head tile (u as the matrix cores see it)
  float* tau;      // (b, H, nc, npt, q) partial u . du_state per d_head tile
  float* pdD;      // (b, nc, qb, H, P) dD partials per 64-token tile
  float* dcb;      // (b, nc, G, hb1, q, q) head-block partials of the C.B^T adjoint
  float* pbc;      // (b, L, G, hb2, 2, N) head-block partials of the state terms of dB (0) and dC (1)
  float* pA;       // (b, H, nc) dA partials
  float* pbias;    // (b, H, nc) ddt_bias partials
};

struct SavedLayout {
  size_t states, dl, cs, cb, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

int make_geo(const mko_ssd_params* prm, Geo* g);
SavedLayout saved_layout(const Geo& g);
void bind_saved(const Geo& g, void* saved, Ptrs* q);
Ptrs base_ptrs(const mko_ssd_params* prm);

// ------------------------------------------------------------ device helpers

// Stages a 64x64 operand tile into LDS, row-major ([row][col]) or transposed
// ([col][row]); `val(row, col)` gives the fp32 value (0 outside the problem).
// 256 threads, 16 elements each, the column index fastest so global reads are
// contiguous along the source row.
template <typename TM, bool TRANS, typename F>
__device__ __forceinline__ void stage(TM* dst, F&& val) {
  constexpr int ld = tile_ld<TM>();
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int e = k * 256 + tid;
    const int row = e >> 6, col = e & 63;
    const float v = val(row, col);
    if (TRANS)
      dst[col * ld + row] = from_f32<TM>(v);
    else
      dst[row * ld + col] = from_f32<TM>(v);
  }
}

// Writes an accumulator tile (value v[r] at (acc_row, acc_col)) to a 64x65 fp32 LDS tile.
__device__ __forceinline__ void acc_to_lds(float* red, const float* v, int wm, int wn, int lane) {
#pragma unroll
  for (int r = 0; r < 16; ++r) red[acc_row(wm, lane, r) * 65 + acc_col(wn, lane)] = v[r];
}

// out[p][n] = sum_l s1(l) X(l, p) Y(l, n) over the chunk, for one 64x64 (p, n) tile.
//   FWD: X = x, s1 = step e^{T - cs}, Y = B  -> local chunk state
//   BWD: X = gy, s1 = e^{cs}, Y = C          -> the chunk's own contribution to the
//        adjoint of its entering state
template <typename TM, bool BWD>
__global__ void __launch_bounds__(256) chunk_state(Geo g, Ptrs p, float* out) {
  __shared__ TM sa[LdsTile<TM>::elems], sb[LdsTile<TM>::elems];
  __shared__ float s1[64];
  const int ntiles = static_cast<int>((g.dstate + 63) / 64);
  const int pt = blockIdx.x / ntiles, nt = blockIdx.x % ntiles;
  const int c = blockIdx.y;
  const int64_t bh = blockIdx.z, b = bh / g.nheads, h = bh % g.nheads, gg = h / g.hpg;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int64_t so = (bh * g.nc + c) * g.q;
  const float T = p.cs[so + g.q - 1];
  f32x16 acc;
  zero(acc);
  for (int kb = 0; kb < g.qb; ++kb) {
    const int64_t t0 = static_cast<int64_t>(c) * g.q + 64 * kb;
    if (threadIdx.x < 64) {
      const int64_t o = so + 64 * kb + threadIdx.x;
      const bool ok = t0 + threadIdx.x < g.length;
      s1[threadIdx.x] = !ok ? 0.0f : (BWD ? fast_exp(p.cs[o]) : p.dl[o] * fast_exp(T - p.cs[o]));
    }
    __syncthreads();
    stage<TM, true>(sa, [&](int l, int pp) {  // A[p][l]
      const int64_t t = t0 + l;
      const int64_t pc = static_cast<int64_t>(pt) * 64 + pp;
      if (t >= g.length || pc >= g.headdim) return 0.0f;
      const int64_t xi = ((b * g.length + t) * g.nheads + h) * g.headdim + pc;
      return s1[l] * load_one(BWD ? p.gy : p.x, g.x_dtype, xi);
    });
    stage<TM, true>(sb, [&](int l, int n) {  // Bt[n][l]
      const int64_t t = t0 + l;
      const int64_t nn = static_cast<int64_t>(nt) * 64 + n;
      if (t >= g.length || nn >= g.dstate) return 0.0f;
      return load_one(BWD ? p.C : p.B, g.bc_dtype, ((b * g.length + t) * g.ngroups + gg) * g.dstate + nn);
    });
    __syncthreads();
    mma_tile<TM>(acc, sa, sb, wm, wn, lane, 64);
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t pp = static_cast<int64_t>(pt) * 64 + acc_row(wm, lane, r);
    const int64_t nn = static_cast<int64_t>(nt) * 64 + acc_col(wn, lane);
    if (pp < g.headdim && nn < g.dstate) out[((bh * g.nc + c) * g.headdim + pp) * g.dstate + nn] = acc[r];
  }
}

// Chunk output before the skip and the gate, for the 64-token tile i and d_head
// tile pt of head (bh) in chunk c:
//   acc[l][p] = sum_{s<=l} e^{cs_l - cs_s} CB[l][s] step_s x_s[p] + e^{cs_l} sum_n C_l[n] S_in[p][n]
// csr/eo receive cs and e^{cs} of the tile's rows.  Leaves the workgroup synchronised
// only on the LDS operand tiles; the caller owns the epilogue.
template <typename TM>
__device__ __forceinline__ void chunk_out(const Geo& g, const Ptrs& p, f32x16& acc, TM* sa, TM* sb, float* csr,
                                          float* css, float* eo, int i, int pt, int c, int64_t bh) {
  const int64_t b = bh / g.nheads, h = bh % g.nheads, gg = h / g.hpg;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int64_t so = (bh * g.nc + c) * g.q;
  const int64_t tl0 = static_cast<int64_t>(c) * g.q + 64 * i;
  const float* cbt = p.cb + ((b * g.nc + c) * g.ngroups + gg) * g.q * g.q;
  if (threadIdx.x < 64) {
    csr[threadIdx.x] = p.cs[so + 64 * i + threadIdx.x];
    eo[threadIdx.x] = fast_exp(csr[threadIdx.x]);
  }
  zero(acc);
  for (int j = 0; j <= i; ++j) {
    const int64_t ts0 = static_cast<int64_t>(c) * g.q + 64 * j;
    __syncthreads();
    if (threadIdx.x < 64) css[threadIdx.x] = p.cs[so + 64 * j + threadIdx.x];
    __syncthreads();
    stage<TM, false>(sa, [&](int r, int s) {  // K[l][s]
      if (64 * j + s > 64 * i + r) return 0.0f;
      return cbt[(64 * i + r) * g.q + 64 * j + s] * fast_exp(csr[r] - css[s]);
    });
    stage<TM, true>(sb, [&](int s, int pp) {  // Bt[p][s] = step_s x_s[p]
      const int64_t t = ts0 + s;
      const int64_t pc = static_cast<int64_t>(pt) * 64 + pp;
      if (t >= g.length || pc >= g.headdim) return 0.0f;
      return p.dl[so + 64 * j + s] * load_one(p.x, g.x_dtype, ((b * g.length + t) * g.nheads + h) * g.headdim + pc);
    });
    __syncthreads();
    mma_tile<TM>(acc, sa, sb, wm, wn, lane, 64);
  }
  const float* st = p.states + (bh * g.nc + c) * g.headdim * g.dstate;
  for (int n0 = 0; n0 < g.dstate; n0 += 64) {
    __syncthreads();
    stage<TM, false>(sa, [&](int r, int k) {  // e^{cs_l} C_l[n]
      const int64_t t = tl0 + r;
      const int n = n0 + k;
      if (t >= g.length || n >= g.dstate) return 0.0f;
      return eo[r] * load_one(p.C, g.bc_dtype, ((b * g.length + t) * g.ngroups + gg) * g.dstate + n);
    });
    stage<TM, false>(sb, [&](int pp, int k) {  // Bt[p][n] = S_in[p][n]
      const int64_t pc = static_cast<int64_t>(pt) * 64 + pp;
      const int n = n0 + k;
      if (pc >= g.headdim || n >= g.dstate) return 0.0f;
      return st[pc * g.dstate + n];
    });
    __syncthreads();
    mma_tile<TM>(acc, sa, sb, wm, wn, lane, 64);
  }
}

}  // namespace ssd
}  // namespace mko
