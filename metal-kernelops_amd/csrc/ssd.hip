// Mamba-2 SSD chunk scan (forward and backward) for gfx950.
//
// The sequence is cut into chunks of q = 64*qb tokens; inside a chunk every
// contraction is done on 64x64 tiles on the matrix cores (mma.hpp):
//   prep        per (b, h, chunk): step = softplus(dt + bias), cs = cumsum(step * A)
//   cb          per (b, chunk, group), lower tiles: CB = C . B^T      (shared by the heads)
//   chunk_state per (b, h, chunk): S = sum_l step_l e^{T - cs_l} x_l (x) B_l   (P x N)
//   state_pass  per (b, h), element-wise over P x N, sequential over chunks:
//               entering state of every chunk, and the final state
//   chunk_scan  per (b, h, chunk, 64-token tile):
//               y = tril(e^{cs_l - cs_s} CB) (step x) + e^{cs_l} C S_in^T + D x, * silu(z)
// The backward mirrors these (see ssd_bwd.hip).  Operands of the products are
// rounded to the input dtype (bf16/f16 products on the bf16/f16 matrix cores,
// fp32 inputs on the fp32 ones); accumulation, decays and states are fp32.
#include "ssd.hpp"

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

template <typename TM>
__global__ void __launch_bounds__(256) cb_kernel(Geo g, Ptrs p) {
  __shared__ TM sa[LdsTile<TM>::elems], sb[LdsTile<TM>::elems];
  // lower-triangular tile (i, j), j <= i
  const int idx = blockIdx.x;
  int i = 0;
  while ((i + 1) * (i + 2) / 2 <= idx) ++i;
  const int j = idx - i * (i + 1) / 2;
  const int c = blockIdx.y / g.ngroups;
  const int64_t gg = blockIdx.y % g.ngroups, b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  const int64_t tc0 = static_cast<int64_t>(c) * g.q + 64 * i, tb0 = static_cast<int64_t>(c) * g.q + 64 * j;
  f32x16 acc;
  zero(acc);
  for (int n0 = 0; n0 < g.dstate; n0 += 64) {
    stage<TM, false>(sa, [&](int r, int k) {
      const int64_t t = tc0 + r;
      const int n = n0 + k;
      return (t < g.length && n < g.dstate) ? load_one(p.C, g.bc_dtype, ((b * g.length + t) * g.ngroups + gg) * g.dstate + n) : 0.0f;
    });
    stage<TM, false>(sb, [&](int s, int k) {
      const int64_t t = tb0 + s;
      const int n = n0 + k;
      return (t < g.length && n < g.dstate) ? load_one(p.B, g.bc_dtype, ((b * g.length + t) * g.ngroups + gg) * g.dstate + n) : 0.0f;
    });
    __syncthreads();
    mma_tile<TM>(acc, sa, sb, wm, wn, lane, 64);
    __syncthreads();
  }
  float* out = p.cb + ((b * g.nc + c) * g.ngroups + gg) * g.q * g.q;
#pragma unroll
  for (int r = 0; r < 16; ++r) out[(64 * i + acc_row(wm, lane, r)) * g.q + 64 * j + acc_col(wn, lane)] = acc[r];
}

// Entering state of every chunk (in place over the local states) and the final state.
__global__ void __launch_bounds__(256) state_pass(Geo g, Ptrs p) {
  const int64_t pn = g.headdim * g.dstate;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= pn) return;
  const int64_t bh = blockIdx.y;
  float s = p.init ? load_one(p.init, g.x_dtype, bh * pn + e) : 0.0f;
  for (int c = 0; c < g.nc; ++c) {
    const int64_t o = (bh * g.nc + c) * pn + e;
    const float loc = p.states[o];
    p.states[o] = s;
    s = fmaf(fast_exp(p.cs[(bh * g.nc + c) * g.q + g.q - 1]), s, loc);
  }
  store_one(p.final_state, g.x_dtype, bh * pn + e, s);
}

template <typename TM>
__global__ void __launch_bounds__(256) chunk_scan(Geo g, Ptrs p) {
  __shared__ TM sa[LdsTile<TM>::elems], sb[LdsTile<TM>::elems];
  __shared__ float csr[64], css[64], eo[64];
  const int i = blockIdx.x % g.qb, pt = blockIdx.x / g.qb;
  const int c = blockIdx.y;
  const int64_t bh = blockIdx.z, b = bh / g.nheads, h = bh % g.nheads;
  const int lane = threadIdx.x & 63;
  int wm, wn;
  quadrant(threadIdx.x >> 6, wm, wn);
  f32x16 acc;
  chunk_out<TM>(g, p, acc, sa, sb, csr, css, eo, i, pt, c, bh);
  const int64_t tl0 = static_cast<int64_t>(c) * g.q + 64 * i;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t t = tl0 + acc_row(wm, lane, r);
    const int64_t pc = static_cast<int64_t>(pt) * 64 + acc_col(wn, lane);
    if (t >= g.length || pc >= g.headdim) continue;
    const int64_t xi = ((b * g.length + t) * g.nheads + h) * g.headdim + pc;
    float v = acc[r];
    if (p.D) v = fmaf(g.d_per_row ? p.D[h * g.headdim + pc] : p.D[h], load_one(p.x, g.x_dtype, xi), v);
    if (p.z) {
      const float zv = load_one(p.z, g.x_dtype, xi);
      v *= zv * sigmoid(zv);
    }
    store_one(p.y, g.x_dtype, xi, v);
  }
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
  // Longer chunks give the matrix cores deeper products; fp32 inputs keep 64-token
  // chunks, where the in-chunk decay exponents (differences of cumulative sums) stay
  // small and the gradient with respect to them keeps fp32 accuracy.
  g->qb = prm->x_dtype == MKO_F32 ? 1 : (g->length >= 1024 ? 4 : (g->length >= 256 ? 2 : 1));
  g->q = 64 * g->qb;
  g->nc = static_cast<int>((g->length + g->q - 1) / g->q);
  g->hpg = static_cast<int>(g->nheads / g->ngroups);
  g->x_dtype = prm->x_dtype;
  g->dt_dtype = prm->dt_dtype;
  g->bc_dtype = prm->bc_dtype;
  g->softplus = (prm->flags & MKO_SSD_SOFTPLUS) ? 1 : 0;
  g->d_per_row = (prm->flags & MKO_SSD_D_PER_ROW) ? 1 : 0;
  return MKO_OK;
}

SavedLayout saved_layout(const Geo& g) {
  SavedLayout l{};
  const size_t bh = static_cast<size_t>(g.batch * g.nheads);
  size_t o = 0;
  l.states = o; o = align256(o + bh * g.nc * g.headdim * g.dstate * 4);
  l.dl = o; o = align256(o + bh * g.nc * g.q * 4);
  l.cs = o; o = align256(o + bh * g.nc * g.q * 4);
  l.cb = o; o = align256(o + static_cast<size_t>(g.batch) * g.nc * g.ngroups * g.q * g.q * 4);
  l.total = o;
  return l;
}

void bind_saved(const Geo& g, void* saved, Ptrs* q) {
  const SavedLayout l = saved_layout(g);
  char* s = static_cast<char*>(saved);
  q->states = reinterpret_cast<float*>(s + l.states);
  q->dl = reinterpret_cast<float*>(s + l.dl);
  q->cs = reinterpret_cast<float*>(s + l.cs);
  q->cb = reinterpret_cast<float*>(s + l.cb);
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

template <typename TM>
static void launch_fwd_t(const Geo& g, const Ptrs& q, hipStream_t s) {
  const unsigned bh = static_cast<unsigned>(g.batch * g.nheads);
  const unsigned pt = static_cast<unsigned>((g.headdim + 63) / 64), nt = static_cast<unsigned>((g.dstate + 63) / 64);
  MKO_TIMED("ssd_prep", s, prep<<<dim3(g.nc, g.nheads, g.batch), 256, 0, s>>>(g, q));
  MKO_TIMED("ssd_cb", s,
            cb_kernel<TM><<<dim3(g.qb * (g.qb + 1) / 2, g.nc * g.ngroups, g.batch), 256, 0, s>>>(g, q));
  MKO_TIMED("ssd_chunk_state", s, chunk_state<TM, false><<<dim3(pt * nt, g.nc, bh), 256, 0, s>>>(g, q, q.states));
  MKO_TIMED("ssd_state_pass", s,
            state_pass<<<dim3(static_cast<unsigned>((g.headdim * g.dstate + 255) / 256), bh), 256, 0, s>>>(g, q));
  MKO_TIMED("ssd_chunk_scan", s, chunk_scan<TM><<<dim3(g.qb * pt, g.nc, bh), 256, 0, s>>>(g, q));
}

}  // namespace ssd
}  // namespace mko

using namespace mko;
using namespace mko::ssd;

extern "C" size_t mko_ssd_saved_bytes(const mko_ssd_params* prm) {
  Geo g;
  if (make_geo(prm, &g) != MKO_OK) return 0;
  return saved_layout(g).total;
}

extern "C" size_t mko_ssd_fwd_workspace_size(const mko_ssd_params* prm) {
  Geo g;
  if (make_geo(prm, &g) != MKO_OK) return 0;
  return 0;
}

extern "C" int mko_ssd_fwd(const mko_ssd_params* prm, void* stream) {
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
    MKO_TIMED("ssd_state_pass", s,
              state_pass<<<dim3(static_cast<unsigned>((g.headdim * g.dstate + 255) / 256),
                                static_cast<unsigned>(g.batch * g.nheads)), 256, 0, s>>>(g, q));
    return mko_check_launch("ssd_fwd");
  }
  if (g.x_dtype == MKO_F32) launch_fwd_t<float>(g, q, s);
  else if (g.x_dtype == MKO_BF16) launch_fwd_t<bf16>(g, q, s);
  else launch_fwd_t<_Float16>(g, q, s);
  return mko_check_launch("ssd_fwd");
}
