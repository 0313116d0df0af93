// Mamba-2 SSD chunk scan (forward and backward) for gfx950.
//
// The sequence is cut into chunks of q = 64*qb tokens; inside a chunk every
// contraction is done on 64x64 tiles on the matrix cores (mma.hpp):
//   prep        per (b, h, chunk): step = softplus(dt + bias), cs = cumsum(step * A)
//   cb          per (b, chunk, group), lower tiles: CB = C . B^T      (shared by the heads)
//   chunk_state per (b, h, chunk): S = sum_l step_l e^{T - cs_l} x_l (x) B_l   (P x N)
//   state_pass  per (b, h), element-wise over P x N, sequential over chunks:
//               entering state of every chunk, and the final state
//   chunk_scan  per (b, h, chunk, 64-token tile), or per (b, h, chunk) for 16-bit inputs
//               with d_state <= 128 (chunk_scan_mt; chunk_scan_cm at 256-token chunks with
//               d_state 128):
//               y = tril(e^{cs_l - cs_s} CB) (step x) + e^{cs_l} C S_in^T + D x, * silu(z)
// The backward mirrors these (see ssd_bwd.hip).  Operands of the products are
// rounded to the input dtype (bf16/f16 products on the bf16/f16 matrix cores,
// fp32 inputs on the fp32 ones); accumulation, decays and states are fp32.
#include "ssd.hpp"
#include "ssd64.hpp"

namespace mko {
namespace ssd {

// ---------------------------------------------------------------- kernels

__global__ void __launch_bounds__(256) prep(Geo g, Ptrs p) {
  __shared__ float wsum[4];
  const int c = blockIdx.x;
  const int64_t h = blockIdx.y, b = blockIdx.z;
  const int l = threadIdx.x;
  const int64_t t = static_cast<int64_t>(c) * g.q + l;
  float del = 0.0f;
  if (l < g.q && t < g.length) {
    float raw = load_one(p.dt, g.dt_dtype, (b * g.length + t) * g.nheads + h);
    if (p.bias) raw += p.bias[h];
    del = g.softplus ? softplus(raw) : raw;
  }
  float v = del * p.A[h];
  // inclusive scan over the workgroup: wavefront butterflies, then wavefront offsets
  for (int off = 1; off < kWave; off <<= 1) {
    const float n = __shfl_up(v, off);
    if ((l & 63) >= off) v += n;
  }
  if ((l & 63) == 63) wsum[l >> 6] = v;
  __syncthreads();
  for (int w = 0; w < (l >> 6); ++w) v += wsum[w];
  if (l < g.q) {
    const int64_t o = ((b * g.nheads + h) * g.nc + c) * g.q + l;
    p.dl[o] = del;
    p.cs[o] = v;
  }
}

template <typename TM, bool VEC>
__global__ void __launch_bounds__(256) cb_kernel(Geo g, Ptrs p) {
  constexpr int TE = LdsTile<TM>::elems;
  __shared__ __align__(16) TM sbuf[2][2 * TE];
  // lower-triangular tile (i, j), j <= i
  const WgId id = wg_id(g.qb * (g.qb + 1) / 2, g.nc * g.ngroups);
  const int idx = id.x;
  int i = 0;
  while ((i + 1) * (i + 2) / 2 <= idx) ++i;
  const int j = idx - i * (i + 1) / 2;
  const int c = id.y / g.ngroups;
  const int64_t gg = id.y % g.ngroups, b = id.z;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int r0 = blk_r0(), c0 = blk_c0();
  const int64_t tc = static_cast<int64_t>(c) * g.q;
  const TM* Cm = static_cast<const TM*>(p.C);
  const TM* Bm = static_cast<const TM*>(p.B);
  struct Regs {
    V8<TM> c[2], b[2];
  };
  auto fetch = [&](int k, Regs& r) {
    load_bw<TM, VEC>(g, Cm, b, tc + 64 * i, gg, 64 * k, r.c);
    load_bw<TM, VEC>(g, Bm, b, tc + 64 * j, gg, 64 * k, r.b);
  };
  auto put = [&](int k, Regs& r) {
    TM* buf = sbuf[k & 1];
    put_raw<TM, false>(buf, r0, c0, r.c[0], r.c[1]);       // A[l][n] = C_l[n]
    put_raw<TM, false>(buf + TE, r0, c0, r.b[0], r.b[1]);  // Bt[s][n] = B_s[n]
  };
  f32x16 acc;
  zero(acc);
  Regs ra, rb;
  pipeline2(g.nnt, ra, rb, fetch, put,
            [&](int k) { mma_tile<TM>(acc, sbuf[k & 1], sbuf[k & 1] + TE, wm, wn, lane, 64); });
  TM* out = static_cast<TM*>(p.cb) + ((b * g.nc + c) * g.ngroups + gg) * g.q * g.q;
#pragma unroll
  for (int r = 0; r < 16; ++r)
    out[(64 * i + acc_row(wm, lane, r)) * g.q + 64 * j + acc_col(wn, lane)] = from_f32<TM>(acc[r]);
}

// Entering state of every chunk (in place over the local states) and the final
// state, 8 consecutive state elements per thread, sequential over the chunks.
template <typename TM>
__global__ void __launch_bounds__(256) state_pass(Geo g, Ptrs p) {
  const int64_t pn = g.headdim * g.dstate;
  const int64_t e0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (e0 >= pn) return;
  const int n = static_cast<int>(pn - e0 < 8 ? pn - e0 : 8);
  const int64_t bh = blockIdx.y;
  TM* st = static_cast<TM*>(p.states);
  float s[8];
  if (p.init) {
    V8<TM> v;
    v8_load(v, static_cast<const TM*>(p.init) + bh * pn + e0, n, g.vec);
    v8_f32(v, s);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) s[k] = 0.0f;
  }
  for (int c = 0; c < g.nc; ++c) {
    TM* o = st + (bh * g.nc + c) * pn + e0;
    V8<TM> v;
    v8_load(v, o, n, g.vec);
    float loc[8];
    v8_f32(v, loc);
    v8_store(o, n, g.vec, s);
    const float eT = fast_exp(p.cs[(bh * g.nc + c) * g.q + g.q - 1]);
#pragma unroll
    for (int k = 0; k < 8; ++k) s[k] = fmaf(eT, s[k], loc[k]);
  }
  v8_store(static_cast<TM*>(p.final_state) + bh * pn + e0, n, g.vec, s);
}

template <typename TM, bool VEC>
__global__ void __launch_bounds__(256) chunk_scan(Geo g, Ptrs p) {
  constexpr int TE = LdsTile<TM>::elems;
  __shared__ __align__(16) TM sbuf[2][2 * TE];
  __shared__ __align__(16) float csc[256], dlc[256], ecol[256], dcol[64];
  // Heads fastest: the workgroups that run together share the group's C and C B^T
  // tiles and cover whole token rows of x and the outputs.
  const WgId id = wg_id(g.nheads, g.qb * g.npt);
  const int64_t h = id.x, b = id.z / g.nc;
  const int i = id.y % g.qb, pt = id.y / g.qb;
  const int c = static_cast<int>(id.z % g.nc);
  const int64_t bh = b * g.nheads + h;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int r0 = blk_r0(), c0 = blk_c0();
  const int64_t tl0 = static_cast<int64_t>(c) * g.q + 64 * i, pc0 = static_cast<int64_t>(pt) * 64;
  load_chunk_cs(g, p, bh, c, csc, dlc, ecol);
  if (threadIdx.x < 64) {
    const int64_t pp = pc0 + threadIdx.x;
    dcol[threadIdx.x] = !p.D ? 0.0f : g.d_per_row ? (pp < g.headdim ? p.D[h * g.headdim + pp] : 0.0f) : p.D[h];
  }
  __syncthreads();
  f32x16 acc;
  // epilogue through LDS: each thread owns rows r0, r0+1 and 8 consecutive d_head columns;
  // x and z of the block come from the pipeline's last loads
  chunk_out<TM, VEC, true>(g, p, acc, sbuf, csc, dlc, ecol, i, pt, c, bh,
                           [&](const V8<TM> (&xv)[2], const V8<TM> (&zv)[2]) {
    float* red = reinterpret_cast<float*>(&sbuf[0][0]);
    acc_to_lds(red, acc, wm, wn, lane);
    __syncthreads();
    float v[2][8];
    lds_block(red, r0, c0, v[0], v[1]);
    const float4 da = *reinterpret_cast<const float4*>(dcol + c0);
    const float4 db = *reinterpret_cast<const float4*>(dcol + c0 + 4);
    const float dv[8] = {da.x, da.y, da.z, da.w, db.x, db.y, db.z, db.w};
    if (p.yt) store_xw<float, VEC>(g, p.yt, b, tl0, h, pc0, v[0], v[1]);
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      float xf[8], zf[8];
      v8_f32(xv[rr], xf);
      if (p.z) v8_f32(zv[rr], zf);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        float y = v[rr][k];
        y = fmaf(dv[k], xf[k], y);
        if (p.z) y *= zf[k] * sigmoid(zf[k]);
        v[rr][k] = y;
      }
    }
    store_xw<TM, VEC, true>(g, static_cast<TM*>(p.y), b, tl0, h, pc0, v[0], v[1]);
  });
}

// Stage k of a chunk's schedule: token tile i, then its state stages kk < nnt and its
// intra stages kk = nnt + j, j = 0 .. i (nnt + i + 1 stages for tile i).
struct ScanStage {
  int i, kk;
};
constexpr ScanStage scan_stage(int k, int nnt) {
  int i = 0, base = 0;
  while (k >= base + nnt + i + 1) {
    base += nnt + i + 1;
    ++i;
  }
  return ScanStage{i, k - base};
}

// One workgroup per (b, h, chunk, d_head tile) for all QB 64-token tiles of the chunk
// (16-bit operands, d_state <= 64 * NNT).  The chunk's u = step x tiles (transposed) and
// its entering state tiles are staged into LDS once and serve every token tile; only the
// left operand is staged per stage:
//   state stages (kk < NNT): C rows of tile i as they are in memory, times S_in; the row
//     factor e^{cs_l} (at most 1) is applied to the accumulator after the last of them
//   intra stages (kk = NNT + j, j = 0 .. i): K[l][s] from the C.B^T tile (k_block), times u_j.
// The schedule is fixed at compile time, and each stage's left operand is requested six
// stages ahead (LDS holds the workgroup to two per CU, so the latency must be hidden by the
// prefetch).  Tile i's x and z rows are requested at its first stage, for its epilogue.
template <typename TM, bool VEC, int QB, int NNT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) chunk_scan_mt(Geo g, Ptrs p) {
  static_assert(sizeof(TM) == 2, "16-bit operands");
  constexpr int TE = LdsTile<TM>::elems;
  constexpr int N = QB * NNT + QB * (QB + 1) / 2;
  constexpr int Q = 64 * QB;
  __shared__ __align__(16) TM ut[QB][TE];   // u_j^T [p][s]
  __shared__ __align__(16) TM st[NNT][TE];  // S_in [p][n], n-tile k
  __shared__ __align__(16) TM ab[2][TE];    // left operand, double-buffered; the epilogue's fp32 tile
  __shared__ __align__(16) float csc[Q], dlc[Q], ecol[Q], ecs[Q], dcol[64];
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
  const TM* Z = p.z ? static_cast<const TM*>(p.z) : X;
  const TM* Cm = static_cast<const TM*>(p.C);
  const TM* cbt = static_cast<const TM*>(p.cb) + ((b * g.nc + c) * g.ngroups + gg) * Q * Q;
  const TM* S = static_cast<const TM*>(p.states) + (bh * g.nc + c) * g.headdim * g.dstate;
  {
    // the chunk's x tiles and entering state
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
    constexpr ScanStage sg = scan_stage(decltype(kc)::value, NNT);
    if constexpr (sg.kk < NNT)
      load_bw<TM, VEC>(g, Cm, b, tc + 64 * sg.i, gg, 64 * sg.kk, r.a);  // C rows l
    else
      load_win<TM, true>(cbt + (64 * sg.i) * Q + 64 * (sg.kk - NNT), Q, 64, 64, r.a, cbt);  // cb rows l
  };
  auto put = [&](auto kc, Regs& r) {
    constexpr int k = decltype(kc)::value;
    constexpr ScanStage sg = scan_stage(k, NNT);
    if constexpr (sg.kk < NNT) {
      put_raw<TM, false>(ab[k & 1], r0, c0, r.a[0], r.a[1]);  // A[l][n] = C_l[n]
    } else {
      float a[8], bb[8];
      k_block<TM>(r.a[0], r.a[1], csc, ecol, sg.i, sg.kk - NNT, r0, c0, a, bb);
      put2x8<TM, false>(ab[k & 1], r0, c0, a, bb);  // A[l][s] = K[l][s]
    }
  };
  f32x16 acc;
  zero(acc);
  V8<TM> xv[2], zv[2];
  constexpr int D = N < 6 ? N : 6;  // stages of prefetch
  Regs regs[D];
  pipeline_static<N, D>(regs, fetch, put, [&](auto kc) {
    constexpr int k = decltype(kc)::value;
    constexpr ScanStage sg = scan_stage(k, NNT);
    const int64_t tl0 = tc + 64 * sg.i;
    if constexpr (sg.kk == 0) {  // epilogue inputs of tile i
      load_xw<TM, VEC>(g, X, b, tl0, h, pc0, xv);
      load_xw<TM, VEC>(g, Z, b, tl0, h, pc0, zv);
    }
    if constexpr (sg.kk < NNT) {
      mma_tile<TM>(acc, ab[k & 1], st[sg.kk], wm, wn, lane, 64);
      if constexpr (sg.kk == NNT - 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] *= ecs[64 * sg.i + acc_row(wm, lane, r)];
      }
    } else {
      mma_tile<TM>(acc, ab[k & 1], ut[sg.kk - NNT], wm, wn, lane, 64);
      if constexpr (sg.kk == NNT + sg.i) {
        // epilogue of tile i: both operand buffers hold the fp32 tile once every wave is done
        float* red = reinterpret_cast<float*>(&ab[0][0]);
        __syncthreads();
        acc_to_lds(red, acc, wm, wn, lane);
        zero(acc);
        __syncthreads();
        float v[2][8];
        lds_block(red, r0, c0, v[0], v[1]);
        if (p.yt) store_xw<float, VEC>(g, p.yt, b, tl0, h, pc0, v[0], v[1]);
        const float4 da = *reinterpret_cast<const float4*>(dcol + c0);
        const float4 db = *reinterpret_cast<const float4*>(dcol + c0 + 4);
        const float dv[8] = {da.x, da.y, da.z, da.w, db.x, db.y, db.z, db.w};
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          float xf[8], zf[8];
          v8_f32(xv[rr], xf);
          if (p.z) v8_f32(zv[rr], zf);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float y = fmaf(dv[e], xf[e], v[rr][e]);
            if (p.z) y *= zf[e] * sigmoid(zf[e]);
            v[rr][e] = y;
          }
        }
        store_xw<TM, VEC, true>(g, static_cast<TM*>(p.y), b, tl0, h, pc0, v[0], v[1]);
        if constexpr (k + 1 < N) __syncthreads();  // the next stage refills the operand buffers
      }
    }
  });
}

// The three-workgroups-per-CU schedule of a chunk's output at qb = 4 and two state tiles
// (d_state 128).  The chunk's four token tiles run in two halves, {0, 1} and {2, 3}, each with
// its own two accumulators: the state stages of the half's tiles (right operand: S_in's
// n-tiles), then its intra pairs (i, j) column by column, u_j staged with the first pair of
// its column.  Each tile accumulates its terms in chunk_scan_mt's order (state, then j
// ascending) and runs its epilogue after its diagonal pair.  Two LDS slots hold the right
// operands: S_in's n-tile k, or u_j, in slot (k or j) & 1; every slot is rewritten at least
// two stages after its last reader, so the stage barriers cover it.  Register operands are
// requested one or two stages before their use.
struct CmStage {
  bool state;
  int i, j;   // state stages: token tile i, n-tile j; pairs: l-tile i, s-tile j
  int stage;  // this stage's put also stages u_j (pairs) or S_in's n-tile j (state) into slot j & 1, when set
  // requested after this stage's products (-1: none): x rows of token tile x (for u_x), z rows
  // of tile z (the epilogue's inputs), S_in's n-tile s
  int x, z, s;
};
constexpr CmStage kCmSchedule[18] = {
    {true, 0, 0, 0, -1, -1, -1},  {true, 0, 1, 0, -1, -1, -1},  {true, 1, 0, 0, -1, 0, -1},
    {true, 1, 1, 0, -1, -1, -1},  {false, 0, 0, 1, 1, 1, -1},   {false, 1, 0, 0, -1, -1, 0},
    {false, 1, 1, 1, 0, -1, 1},   {true, 2, 0, 1, -1, -1, -1},  {true, 2, 1, 1, -1, -1, -1},
    {true, 3, 0, 0, -1, -1, -1},  {true, 3, 1, 0, -1, -1, -1},  {false, 2, 0, 1, 1, -1, -1},
    {false, 3, 0, 0, -1, -1, -1}, {false, 2, 1, 1, 2, 2, -1},   {false, 3, 1, 0, -1, -1, -1},
    {false, 2, 2, 1, 3, 3, -1},   {false, 3, 2, 0, -1, -1, -1}, {false, 3, 3, 1, -1, -1, -1}};

// chunk_scan_mt at qb = 4, d_state 128 with three workgroups per CU (16-bit operands): the same
// sums, bit for bit, in the order of kCmSchedule, so that LDS holds two right-operand slots
// instead of all of a chunk's u tiles, and two accumulators are live instead of one per tile.
// Compact 64-element operand tiles; 53.8 KB of LDS.
template <typename TM, bool VEC>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) chunk_scan_cm(Geo g, Ptrs p) {
  static_assert(sizeof(TM) == 2, "16-bit operands");
  constexpr int LD = compact_ld<TM>();
  constexpr int TE = LdsTile<TM, LD>::elems;
  constexpr int N = 18;
  constexpr int Q = 256;
  __shared__ __align__(16) TM ab[2][TE];  // left operand, double-buffered
  __shared__ __align__(16) TM ub[2][TE];  // right operand slots
  __shared__ __align__(16) float red[64 * 65];
  __shared__ __align__(16) float csc[Q], dlc[Q], ecol[Q], ecs[Q], dcol[64];
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
  const TM* Z = p.z ? static_cast<const TM*>(p.z) : X;
  const TM* Cm = static_cast<const TM*>(p.C);
  const TM* cbt = static_cast<const TM*>(p.cb) + ((b * g.nc + c) * g.ngroups + gg) * Q * Q;
  const TM* S = static_cast<const TM*>(p.states) + (bh * g.nc + c) * g.headdim * g.dstate;
  V8<TM> xv[2];     // x rows of the tile whose u is staged next (and whose epilogue is next)
  V8<TM> zv[2];     // z rows of the tile whose epilogue is next
  V8<TM> sv[2][2];  // S_in's n-tiles
  {
#pragma unroll
    for (int k = 0; k < 2; ++k) load_sw<TM, VEC>(g, S, pc0, 64 * k, sv[k]);
    load_xw<TM, VEC>(g, X, b, tc, h, pc0, xv);
    load_chunk_cs(g, p, bh, c, csc, dlc, ecol);
    if (threadIdx.x < Q) ecs[threadIdx.x] = fast_exp(csc[threadIdx.x]);
    if (threadIdx.x < 64) {
      const int64_t pp = pc0 + threadIdx.x;
      dcol[threadIdx.x] = !p.D ? 0.0f : g.d_per_row ? (pp < g.headdim ? p.D[h * g.headdim + pp] : 0.0f) : p.D[h];
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) put_raw<TM, false, LD>(ub[k], r0, c0, sv[k][0], sv[k][1]);  // Bt[p][n] = S_in[p][n]
  }
  struct Regs {
    V8<TM> a[2];
  };
  auto fetch = [&](auto kc, Regs& r) {
    constexpr CmStage sg = kCmSchedule[decltype(kc)::value];
    if constexpr (sg.state)
      load_bw<TM, VEC>(g, Cm, b, tc + 64 * sg.i, gg, 64 * sg.j, r.a);  // C rows l
    else
      load_win<TM, true>(cbt + (64 * sg.i) * Q + 64 * sg.j, Q, 64, 64, r.a, cbt);  // cb rows l
  };
  auto put = [&](auto kc, Regs& r) {
    constexpr int k = decltype(kc)::value;
    constexpr CmStage sg = kCmSchedule[k];
    if constexpr (sg.state) {
      put_raw<TM, false, LD>(ab[k & 1], r0, c0, r.a[0], r.a[1]);  // A[l][n] = C_l[n]
      if constexpr (sg.stage) put_raw<TM, false, LD>(ub[sg.j & 1], r0, c0, sv[sg.j][0], sv[sg.j][1]);
    } else {
      float a[8], bb[8];
      k_block<TM>(r.a[0], r.a[1], csc, ecol, sg.i, sg.j, r0, c0, a, bb);
      put2x8<TM, false, LD>(ab[k & 1], r0, c0, a, bb);  // A[l][s] = K[l][s]
      if constexpr (sg.stage) {
        scale8(xv[0], dlc[64 * sg.j + r0], a);
        scale8(xv[1], dlc[64 * sg.j + r0 + 1], bb);
        put2x8<TM, true, LD>(ub[sg.j & 1], r0, c0, a, bb);  // Bt[p][s] = step_s x_s[p]
      }
    }
  };
  f32x16 acc[2];
  zero(acc[0]);
  zero(acc[1]);
  constexpr int D = 2;
  Regs regs[D];
  __syncthreads();  // csc, dlc, S_in
  pipeline_static<N, D>(regs, fetch, put, [&](auto kc) {
    constexpr int k = decltype(kc)::value;
    constexpr CmStage sg = kCmSchedule[k];
    f32x16& ac = acc[sg.i & 1];
    if constexpr (sg.state) {
      mma_tile<TM, LD>(ac, ab[k & 1], ub[sg.j & 1], wm, wn, lane, 64);
      if constexpr (sg.j == 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) ac[r] *= ecs[64 * sg.i + acc_row(wm, lane, r)];
      }
    } else {
      mma_tile<TM, LD>(ac, ab[k & 1], ub[sg.j & 1], wm, wn, lane, 64);
      if constexpr (sg.i == sg.j) {
        // tile i is complete
        acc_to_lds(red, ac, wm, wn, lane);
        zero(ac);
        __syncthreads();
        float v[2][8];
        lds_block(red, r0, c0, v[0], v[1]);
        const float4 da = *reinterpret_cast<const float4*>(dcol + c0);
        const float4 db = *reinterpret_cast<const float4*>(dcol + c0 + 4);
        const float dv[8] = {da.x, da.y, da.z, da.w, db.x, db.y, db.z, db.w};
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          float xf[8], zf[8];
          v8_f32(xv[rr], xf);
          if (p.z) v8_f32(zv[rr], zf);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float y = fmaf(dv[e], xf[e], v[rr][e]);
            if (p.z) y *= zf[e] * sigmoid(zf[e]);
            v[rr][e] = y;
          }
        }
        store_xw<TM, VEC, true>(g, static_cast<TM*>(p.y), b, tc + 64 * sg.i, h, pc0, v[0], v[1]);
      }
    }
    if constexpr (sg.x >= 0) load_xw<TM, VEC>(g, X, b, tc + 64 * sg.x, h, pc0, xv);
    if constexpr (sg.z >= 0) load_xw<TM, VEC>(g, Z, b, tc + 64 * sg.z, h, pc0, zv);
    if constexpr (sg.s >= 0) load_sw<TM, VEC>(g, S, pc0, 64 * sg.s, sv[sg.s]);
  });
}

// ---------------------------------------------------------------- host

int make_geo(const mko_ssd_params* prm, Geo* g) {
  if (!prm) {
    mko_set_error("ssd: null params");
    return MKO_EINVAL;
  }
  g->batch = prm->batch;
  g->length = prm->length;
  g->nheads = prm->nheads;
  g->headdim = prm->headdim;
  g->ngroups = prm->ngroups;
  g->dstate = prm->dstate;
  if (g->batch < 0 || g->length < 0 || g->nheads < 1 || g->headdim < 1 || g->ngroups < 1 || g->dstate < 1 ||
      g->nheads % g->ngroups) {
    mko_set_error("ssd: bad sizes");
    return MKO_EINVAL;
  }
  for (int dt : {prm->x_dtype, prm->dt_dtype, prm->bc_dtype}) {
    if (dt != MKO_F32 && dt != MKO_F16 && dt != MKO_BF16) {
      mko_set_error("ssd: unknown dtype %d", dt);
      return MKO_EINVAL;
    }
  }
  if (prm->bc_dtype != prm->x_dtype) {
    mko_set_error("ssd: B and C must have the dtype of x");
    return MKO_EINVAL;
  }
  // Longer chunks give the matrix cores deeper products; fp32 inputs keep 64-token
  // chunks, where the in-chunk decay exponents (differences of cumulative sums) stay
  // small and the gradient with respect to them keeps fp32 accuracy.
  g->qb = prm->x_dtype == MKO_F32 ? 1 : (g->length >= 1024 ? 4 : (g->length >= 256 ? 2 : 1));
  g->q = 64 * g->qb;
  g->nc = static_cast<int>((g->length + g->q - 1) / g->q);
  g->hpg = static_cast<int>(g->nheads / g->ngroups);
  g->npt = static_cast<int>((g->headdim + 63) / 64);
  g->nnt = static_cast<int>((g->dstate + 63) / 64);
  g->nnp = (g->nnt + 1) / 2;
  // row strides below 2^24 keep every lane's byte offset in a 64-row window within 32 bits
  if (g->nheads * g->headdim >= (int64_t(1) << 24) || g->ngroups * g->dstate >= (int64_t(1) << 24)) {
    mko_set_error("ssd: nheads * headdim and ngroups * dstate must be below 2^24");
    return MKO_EUNSUPPORTED;
  }
  g->x_dtype = prm->x_dtype;
  g->dt_dtype = prm->dt_dtype;
  // 16-byte vectors of 8 elements: whole runs of d_head and d_state, aligned bases
  bool vec = g->headdim % 8 == 0 && g->dstate % 8 == 0;
  const void* ptrs[] = {prm->x,  prm->z,      prm->B,  prm->C,  prm->initial_states, prm->y,
                        prm->final_state, prm->saved, prm->dy, prm->dfinal, prm->dx, prm->dz,
                        prm->dB, prm->dC, prm->dinitial, prm->workspace};
  for (const void* q : ptrs) vec = vec && (reinterpret_cast<uintptr_t>(q) % 16 == 0);
  g->vec = vec ? 1 : 0;
  g->softplus = (prm->flags & MKO_SSD_SOFTPLUS) ? 1 : 0;
  g->d_per_row = (prm->flags & MKO_SSD_D_PER_ROW) ? 1 : 0;
  g->save_y = (prm->flags & MKO_SSD_SAVE_Y) ? 1 : 0;
  return MKO_OK;
}

SavedLayout saved_layout(const Geo& g) {
  SavedLayout l{};
  const size_t bh = static_cast<size_t>(g.batch * g.nheads);
  size_t o = 0;
  l.states = o; o = align256(o + bh * g.nc * g.headdim * g.dstate * dtype_size(g.x_dtype));
  l.dl = o; o = align256(o + bh * g.nc * g.q * 4);
  l.cs = o; o = align256(o + bh * g.nc * g.q * 4);
  l.cb = o; o = align256(o + static_cast<size_t>(g.batch) * g.nc * g.ngroups * g.q * g.q * dtype_size(g.x_dtype));
  // the multi-tile backward recomputes the chunk output instead of reading a saved copy
  const bool yt = g.save_y && !multi_tile(g);
  l.yt = o; o = align256(o + (yt ? static_cast<size_t>(g.batch * g.length * g.nheads * g.headdim) * 4 : 0));
  l.total = o;
  return l;
}

void bind_saved(const Geo& g, void* saved, Ptrs* q) {
  const SavedLayout l = saved_layout(g);
  char* s = static_cast<char*>(saved);
  q->states = s + l.states;
  q->dl = reinterpret_cast<float*>(s + l.dl);
  q->cs = reinterpret_cast<float*>(s + l.cs);
  q->cb = s + l.cb;
  q->yt = g.save_y && !multi_tile(g) ? reinterpret_cast<float*>(s + l.yt) : nullptr;
}

Ptrs base_ptrs(const mko_ssd_params* prm) {
  Ptrs q{};
  q.x = prm->x;
  q.dt = prm->dt;
  q.A = prm->A;
  q.B = prm->B;
  q.C = prm->C;
  q.D = prm->D;
  q.z = prm->z;
  q.bias = prm->dt_bias;
  q.init = prm->initial_states;
  q.y = prm->y;
  q.final_state = prm->final_state;
  q.dy = prm->dy;
  q.dfinal = prm->dfinal;
  q.dx = prm->dx;
  q.ddt = prm->ddt;
  q.dz = prm->dz;
  q.dinit = prm->dinitial;
  q.dA = prm->dA;
  q.dB = prm->dB;
  q.dC = prm->dC;
  q.dD = prm->dD;
  q.dbias = prm->ddt_bias;
  return q;
}

template <typename TM, bool VEC>
static void launch_fwd_t(const Geo& g, const Ptrs& q, hipStream_t s) {
  const unsigned bh = static_cast<unsigned>(g.batch * g.nheads);
  MKO_TIMED("ssd_prep", s, prep<<<dim3(g.nc, g.nheads, g.batch), 256, 0, s>>>(g, q));
  MKO_TIMED("ssd_cb", s,
            cb_kernel<TM, VEC><<<dim3(g.qb * (g.qb + 1) / 2 * g.nc * g.ngroups * g.batch), 256, 0, s>>>(g, q));
  const dim3 cs_grid(g.npt * g.nnp * g.nc * bh);
  if (g.qb == 4) MKO_TIMED("ssd_chunk_state", s, chunk_state<TM, VEC, false, 4><<<cs_grid, 256, 0, s>>>(g, q, q.states));
  else MKO_TIMED("ssd_chunk_state", s, chunk_state<TM, VEC, false><<<cs_grid, 256, 0, s>>>(g, q, q.states));
  MKO_TIMED("ssd_state_pass", s,
            state_pass<TM><<<dim3(static_cast<unsigned>((g.headdim * g.dstate + 2047) / 2048), bh), 256, 0, s>>>(
                g, q));
  if constexpr (sizeof(TM) == 2) {
    const dim3 grid(g.npt * g.nc * bh);
    if (multi_tile(g) && g.qb == 4 && g.nnt == 2 && g.dstate == 128) {
      MKO_TIMED("ssd_chunk_scan", s, chunk_scan_cm<TM, VEC><<<grid, 256, 0, s>>>(g, q));
      return;
    }
    if (multi_tile(g)) {
      if (g.qb == 4 && g.nnt == 2) MKO_TIMED("ssd_chunk_scan", s, chunk_scan_mt<TM, VEC, 4, 2><<<grid, 256, 0, s>>>(g, q));
      else if (g.qb == 4) MKO_TIMED("ssd_chunk_scan", s, chunk_scan_mt<TM, VEC, 4, 1><<<grid, 256, 0, s>>>(g, q));
      else if (g.qb == 2 && g.nnt == 2) MKO_TIMED("ssd_chunk_scan", s, chunk_scan_mt<TM, VEC, 2, 2><<<grid, 256, 0, s>>>(g, q));
      else if (g.qb == 2) MKO_TIMED("ssd_chunk_scan", s, chunk_scan_mt<TM, VEC, 2, 1><<<grid, 256, 0, s>>>(g, q));
      else if (g.nnt == 2) MKO_TIMED("ssd_chunk_scan", s, chunk_scan_mt<TM, VEC, 1, 2><<<grid, 256, 0, s>>>(g, q));
      else MKO_TIMED("ssd_chunk_scan", s, chunk_scan_mt<TM, VEC, 1, 1><<<grid, 256, 0, s>>>(g, q));
      return;
    }
  }
  MKO_TIMED("ssd_chunk_scan", s, chunk_scan<TM, VEC><<<dim3(g.qb * g.npt * g.nc * bh), 256, 0, s>>>(g, q));
}

template <typename TM>
static void launch_fwd_t(const Geo& g, const Ptrs& q, hipStream_t s) {
  if (g.vec) launch_fwd_t<TM, true>(g, q, s);
  else launch_fwd_t<TM, false>(g, q, s);
}

}  // namespace ssd
}  // namespace mko

using namespace mko;
using namespace mko::ssd;

extern "C" size_t mko_ssd_saved_bytes(const mko_ssd_params* prm) {
  if (prm && prm->x_dtype == MKO_F64) return ssd64_saved_bytes(prm);
  Geo g;
  if (make_geo(prm, &g) != MKO_OK) return 0;
  return saved_layout(g).total;
}

extern "C" size_t mko_ssd_fwd_workspace_size(const mko_ssd_params* prm) {
  if (prm && prm->x_dtype == MKO_F64) return 0;
  Geo g;
  if (make_geo(prm, &g) != MKO_OK) return 0;
  return 0;
}

extern "C" int mko_ssd_fwd(const mko_ssd_params* prm, void* stream) {
  if (prm && prm->x_dtype == MKO_F64) return ssd64_fwd(prm, static_cast<hipStream_t>(stream));
  Geo g;
  int st = make_geo(prm, &g);
  if (st != MKO_OK) return st;
  if (g.batch == 0) return MKO_OK;
  if (!prm->A || !prm->final_state ||
      (g.length > 0 && (!prm->x || !prm->dt || !prm->B || !prm->C || !prm->y || !prm->saved))) {
    mko_set_error("ssd_fwd: x, dt, A, B, C, y, final_state and saved are required");
    return MKO_EINVAL;
  }
  Ptrs q = base_ptrs(prm);
  bind_saved(g, prm->saved, &q);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (g.length == 0) {
    // no tokens: the final state is the initial state (or zero)
    const dim3 grid(static_cast<unsigned>((g.headdim * g.dstate + 2047) / 2048),
                    static_cast<unsigned>(g.batch * g.nheads));
    if (g.x_dtype == MKO_F32) MKO_TIMED("ssd_state_pass", s, state_pass<float><<<grid, 256, 0, s>>>(g, q));
    else if (g.x_dtype == MKO_BF16) MKO_TIMED("ssd_state_pass", s, state_pass<bf16><<<grid, 256, 0, s>>>(g, q));
    else MKO_TIMED("ssd_state_pass", s, state_pass<_Float16><<<grid, 256, 0, s>>>(g, q));
    return mko_check_launch("ssd_fwd");
  }
  if (g.x_dtype == MKO_F32) launch_fwd_t<float>(g, q, s);
  else if (g.x_dtype == MKO_BF16) launch_fwd_t<bf16>(g, q, s);
  else launch_fwd_t<_Float16>(g, q, s);
  return mko_check_launch("ssd_fwd");
}
