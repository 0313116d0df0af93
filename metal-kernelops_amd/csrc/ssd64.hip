// Mamba-2 SSD chunk scan in float64 (x_dtype MKO_F64), forward and backward, for gfx950.
//
// The reference's torch composition accepts float64 inputs and computes in float64
// (cv/mamba2_chunk.py:439-440, 447-462); its verifier checks the scan that way against
// ssd_minimal_discrete (benchmarks/verify_mamba2_chunk.py:214-233).  The matrix-core kernels
// of ssd.hip take 32- and 16-bit operands, so float64 runs here: the per-token recurrence on
// the fp64 vector units, which computes what the chunked composition does up to float64
// rounding (the chunk length only regroups the same sums).
//
//   s_t = exp(dt_t A) s_{t-1} + dt_t x_t (x) B_t,   y_t = <C_t, s_t> + D x_t, y_t *= silu(z_t)
//
// Layout: one workgroup of 256 lanes per (batch, head, block of rows p of the (P, N) state).
// TN lanes (a power of two, at most 64) share a row and hold its states n = lane + k TN,
// k < 4, so d_state <= 256; a row's <C, s> is a butterfly over its TN lanes.  The forward
// saves the state entering every 16-step block; the backward walks the blocks in reverse,
// recomputes a block's 16 states into LDS from its saved entering state, and carries the
// state adjoint q backwards:
//   q_t += gy_t C_t;  dC_t += gy_t s_t;  dB_t += q_t dt_t x_t;  dx_t = dt_t <q_t, B_t> + D gy_t;
//   d dt_t = sum q_t (A a_t s_{t-1} + x_t B_t);  dA += sum q_t dt_t a_t s_{t-1};  q_{t-1} = a_t q_t
// dB, dC, d dt and dA leave as per-(row block) partials that fixed-order kernels sum over the
// row blocks and the heads of a group, so the backward is deterministic.  With x_dtype MKO_F64
// every floating-point array of mko_ssd_params is float64, A, D and dt_bias and their
// gradients included.
#include "common.hpp"
#include "ssd64.hpp"

namespace mko {
namespace ssd64 {

constexpr int kLanes = 256;
constexpr int kPerLane = 4;  // states per lane
constexpr int kBlock = 16;   // steps between saved states

struct Geo {
  int64_t batch, length, nheads, headdim, ngroups, dstate;
  int hpg;    // heads per group
  int tn;     // lanes per row
  int rows;   // rows per workgroup (kLanes / tn)
  int nrb;    // row blocks per head
  int nblk;   // 16-step blocks
  int softplus, d_per_row;
};

struct Ptrs {
  const double *x, *dt, *A, *B, *C, *D, *z, *bias, *init, *dy, *dfinal;
  double *y, *final_state, *dx, *ddt, *dA, *dB, *dC, *dD, *dz, *dbias, *dinit;
  double* ckpt;  // (b, H, nblk, P, N): the state entering each block (saved area)
  // backward partials (workspace)
  double* pbc;   // (b, L, H, nrb, 2, N): the row block's dB (0) and dC (1) terms
  double* pdel;  // (b, L, H, nrb): the row block's d dt terms (before the softplus derivative)
  double* pA;    // (b, H, nrb)
  double* pD;    // (b, H, P): sum over time of gy x per row
};

__device__ __forceinline__ double softplus64(double v) { return v > 20.0 ? v : log1p(exp(v)); }
__device__ __forceinline__ double sigmoid64(double v) { return 1.0 / (1.0 + exp(-v)); }
__device__ __forceinline__ double softplus64_grad(double v) { return v > 20.0 ? 1.0 : sigmoid64(v); }

// Sum over the tn lanes of a row (tn a power of two <= 64); every lane gets it.
__device__ __forceinline__ double row_sum64(double v, int tn) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    if (off < tn) v += __shfl_xor(v, off);
  return v;
}

struct Lane {
  int64_t b, h, gg;
  int p;      // this lane's row
  bool prow;  // the row exists
  int j;      // lane within the row
};

__device__ __forceinline__ Lane lane_of(const Geo& g) {
  Lane l;
  l.b = blockIdx.z;
  l.h = blockIdx.y;
  l.gg = l.h / g.hpg;
  const int r = static_cast<int>(threadIdx.x) / g.tn;
  l.j = static_cast<int>(threadIdx.x) % g.tn;
  l.p = static_cast<int>(blockIdx.x) * g.rows + r;
  l.prow = l.p < g.headdim;
  return l;
}

// The step size of (b, t, h): raw dt plus bias, through softplus when asked.
__device__ __forceinline__ double step_raw(const Geo& g, const Ptrs& q, int64_t b, int64_t t, int64_t h) {
  double raw = q.dt[(b * g.length + t) * g.nheads + h];
  if (q.bias) raw += q.bias[h];
  return raw;
}

__global__ void __launch_bounds__(kLanes) fwd(Geo g, Ptrs q) {
  const Lane l = lane_of(g);
  const int64_t N = g.dstate, P = g.headdim;
  const int64_t bh = l.b * g.nheads + l.h;
  const int pr = l.prow ? l.p : 0;
  double s[kPerLane];
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) {
    const int64_t n = l.j + k * g.tn;
    s[k] = (q.init && l.prow && n < N) ? q.init[(bh * P + pr) * N + n] : 0.0;
  }
  const double Ah = q.A[l.h];
  const double Dv = q.D ? (g.d_per_row ? q.D[l.h * P + pr] : q.D[l.h]) : 0.0;
  for (int64_t t = 0; t < g.length; ++t) {
    if (t % kBlock == 0 && l.prow) {
      double* ck = q.ckpt + ((bh * g.nblk + t / kBlock) * P + pr) * N;
#pragma unroll
      for (int k = 0; k < kPerLane; ++k) {
        const int64_t n = l.j + k * g.tn;
        if (n < N) ck[n] = s[k];
      }
    }
    const double raw = step_raw(g, q, l.b, t, l.h);
    const double del = g.softplus ? softplus64(raw) : raw;
    const double a = exp(del * Ah);
    const int64_t xo = ((l.b * g.length + t) * g.nheads + l.h) * P + pr;
    const double xv = q.x[xo];
    const double dxv = del * xv;
    const int64_t bo = ((l.b * g.length + t) * g.ngroups + l.gg) * N;
    double yp = 0.0;
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) {
      const int64_t n = l.j + k * g.tn;
      if (n < N) {
        s[k] = a * s[k] + dxv * q.B[bo + n];
        yp += q.C[bo + n] * s[k];
      }
    }
    const double yv = row_sum64(yp, g.tn);
    if (l.j == 0 && l.prow) {
      double out = yv + Dv * xv;
      if (q.z) {
        const double zv = q.z[xo];
        out *= zv * sigmoid64(zv);
      }
      q.y[xo] = out;
    }
  }
  if (l.prow) {
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) {
      const int64_t n = l.j + k * g.tn;
      if (n < N) q.final_state[(bh * P + pr) * N + n] = s[k];
    }
  }
}

// The backward of fwd: the states of a 16-step block are recomputed into LDS (hs[step][lane]),
// then the block is walked backwards.
__global__ void __launch_bounds__(kLanes) bwd(Geo g, Ptrs q) {
  __shared__ double hs[kBlock][kLanes * kPerLane];
  __shared__ double cred[kLanes * 2 * kPerLane];  // the row block's dB/dC terms, reduced over rows
  __shared__ double rred[kLanes];                 // per row: d dt
  const Lane l = lane_of(g);
  const int64_t N = g.dstate, P = g.headdim;
  const int64_t bh = l.b * g.nheads + l.h;
  const int pr = l.prow ? l.p : 0;
  const int row = static_cast<int>(threadIdx.x) / g.tn;
  double qa[kPerLane];
#pragma unroll
  for (int k = 0; k < kPerLane; ++k) {
    const int64_t n = l.j + k * g.tn;
    qa[k] = (q.dfinal && l.prow && n < N) ? q.dfinal[(bh * P + pr) * N + n] : 0.0;
  }
  const double Ah = q.A[l.h];
  const double Dv = q.D ? (g.d_per_row ? q.D[l.h * P + pr] : q.D[l.h]) : 0.0;
  double dA_acc = 0.0, dD_acc = 0.0;
  for (int blk = g.nblk - 1; blk >= 0; --blk) {
    const int64_t t0 = static_cast<int64_t>(blk) * kBlock;
    const int nt = static_cast<int>(g.length - t0 < kBlock ? g.length - t0 : kBlock);
    // the block's entering state and its recomputed states
    double s0[kPerLane], s[kPerLane];
    const double* ck = q.ckpt + ((bh * g.nblk + blk) * P + pr) * N;
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) {
      const int64_t n = l.j + k * g.tn;
      s0[k] = (l.prow && n < N) ? ck[n] : 0.0;
      s[k] = s0[k];
    }
    for (int i = 0; i < nt; ++i) {
      const int64_t t = t0 + i;
      const double raw = step_raw(g, q, l.b, t, l.h);
      const double del = g.softplus ? softplus64(raw) : raw;
      const double a = exp(del * Ah);
      const double dxv = del * q.x[((l.b * g.length + t) * g.nheads + l.h) * P + pr];
      const int64_t bo = ((l.b * g.length + t) * g.ngroups + l.gg) * N;
#pragma unroll
      for (int k = 0; k < kPerLane; ++k) {
        const int64_t n = l.j + k * g.tn;
        s[k] = n < N ? a * s[k] + dxv * q.B[bo + n] : 0.0;
        hs[i][threadIdx.x * kPerLane + k] = s[k];
      }
    }
    for (int i = nt - 1; i >= 0; --i) {
      const int64_t t = t0 + i;
      const double raw = step_raw(g, q, l.b, t, l.h);
      const double del = g.softplus ? softplus64(raw) : raw;
      const double a = exp(del * Ah);
      const int64_t xo = ((l.b * g.length + t) * g.nheads + l.h) * P + pr;
      const double xv = q.x[xo];
      const double dyv = l.prow ? q.dy[xo] : 0.0;  // a row past the head's adds nothing
      const int64_t bo = ((l.b * g.length + t) * g.ngroups + l.gg) * N;
      double st[kPerLane], sp[kPerLane], bv[kPerLane], cv[kPerLane];
      double yp = 0.0;
#pragma unroll
      for (int k = 0; k < kPerLane; ++k) {
        const int64_t n = l.j + k * g.tn;
        const bool ok = n < N;
        st[k] = hs[i][threadIdx.x * kPerLane + k];
        sp[k] = i > 0 ? hs[i - 1][threadIdx.x * kPerLane + k] : s0[k];
        bv[k] = ok ? q.B[bo + n] : 0.0;
        cv[k] = ok ? q.C[bo + n] : 0.0;
        yp += cv[k] * st[k];
      }
      const double yt = row_sum64(yp, g.tn);  // the output before the skip and the gate
      double gy = dyv;
      if (q.z) {
        const double zv = q.z[xo];
        const double sg = sigmoid64(zv);
        gy = dyv * zv * sg;
        if (l.j == 0 && l.prow) q.dz[xo] = dyv * (yt + Dv * xv) * sg * (1.0 + zv * (1.0 - sg));
      }
      dD_acc += gy * xv;
      double dxs = 0.0, dd = 0.0;
#pragma unroll
      for (int k = 0; k < kPerLane; ++k) {
        qa[k] += gy * cv[k];
        cred[threadIdx.x * 2 * kPerLane + k] = qa[k] * del * xv;           // dB term
        cred[threadIdx.x * 2 * kPerLane + kPerLane + k] = gy * st[k];      // dC term
        dxs += qa[k] * bv[k];
        dd += qa[k] * (Ah * a * sp[k] + xv * bv[k]);
        dA_acc += qa[k] * del * a * sp[k];
        qa[k] *= a;
      }
      dxs = row_sum64(dxs, g.tn);
      dd = row_sum64(dd, g.tn);
      if (l.j == 0) {
        if (l.prow) q.dx[xo] = del * dxs + Dv * gy;
        rred[row] = l.prow ? dd : 0.0;
      }
      __syncthreads();
      // the row block's sums over its rows, in row order: dB/dC per state, d dt
      const int64_t po = ((l.b * g.length + t) * g.nheads + l.h) * g.nrb + blockIdx.x;
      for (int c = threadIdx.x; c < 2 * g.tn * kPerLane; c += kLanes) {
        const int which = c / (g.tn * kPerLane), jk = c % (g.tn * kPerLane);
        const int jj = jk / kPerLane, k = jk % kPerLane;
        const int64_t n = jj + static_cast<int64_t>(k) * g.tn;
        if (n < N) {
          double v = 0.0;
          for (int r = 0; r < g.rows; ++r) v += cred[(r * g.tn + jj) * 2 * kPerLane + which * kPerLane + k];
          q.pbc[(po * 2 + which) * N + n] = v;
        }
      }
      if (threadIdx.x == 0) {
        double v = 0.0;
        for (int r = 0; r < g.rows; ++r) v += rred[r];
        q.pdel[po] = v;
      }
      __syncthreads();
    }
  }
  // the adjoint of the initial state; dA and dD partials
  if (q.dinit && l.prow) {
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) {
      const int64_t n = l.j + k * g.tn;
      if (n < N) q.dinit[(bh * P + pr) * N + n] = qa[k];
    }
  }
  dA_acc = row_sum64(dA_acc, g.tn);
  if (l.j == 0) rred[row] = l.prow ? dA_acc : 0.0;
  if (l.j == 0 && l.prow) q.pD[bh * P + pr] = dD_acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double v = 0.0;
    for (int r = 0; r < g.rows; ++r) v += rred[r];
    q.pA[bh * g.nrb + blockIdx.x] = v;
  }
}

// dB and dC: one thread per (b, t, group, state), summing the heads of the group and their row
// blocks in order.
__global__ void __launch_bounds__(kLanes) reduce_bc(Geo g, Ptrs q) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kLanes + threadIdx.x;
  const int64_t N = g.dstate;
  const int64_t total = g.batch * g.length * g.ngroups * N;
  if (i >= total) return;
  const int64_t n = i % N, btg = i / N, gg = btg % g.ngroups, bt = btg / g.ngroups;
  double sb = 0.0, sc = 0.0;
  for (int64_t hh = 0; hh < g.hpg; ++hh) {
    const int64_t h = gg * g.hpg + hh;
    for (int rb = 0; rb < g.nrb; ++rb) {
      const int64_t po = (bt * g.nheads + h) * g.nrb + rb;
      sb += q.pbc[(po * 2 + 0) * N + n];
      sc += q.pbc[(po * 2 + 1) * N + n];
    }
  }
  q.dB[i] = sb;
  q.dC[i] = sc;
}

// ddt: one thread per (b, t, h), the row blocks in order, times the softplus derivative.
__global__ void __launch_bounds__(kLanes) reduce_dt(Geo g, Ptrs q) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kLanes + threadIdx.x;
  const int64_t total = g.batch * g.length * g.nheads;
  if (i >= total) return;
  double v = 0.0;
  for (int rb = 0; rb < g.nrb; ++rb) v += q.pdel[i * g.nrb + rb];
  const int64_t h = i % g.nheads, bt = i / g.nheads, b = bt / g.length, t = bt % g.length;
  if (g.softplus) v *= softplus64_grad(step_raw(g, q, b, t, h));
  q.ddt[i] = v;
}

// dA, dD and ddt_bias: one workgroup per head, each thread summing a strided share in order,
// then a fixed tree.
__device__ __forceinline__ double block_sum64(double v, double* ws) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = v;
  __syncthreads();
  return (ws[0] + ws[1]) + (ws[2] + ws[3]);
}

__global__ void __launch_bounds__(kLanes) reduce_params(Geo g, Ptrs q) {
  __shared__ double ws[4];
  const int64_t h = blockIdx.x, P = g.headdim;
  double va = 0.0;
  for (int64_t k = threadIdx.x; k < g.batch * g.nrb; k += kLanes) {
    const int64_t b = k / g.nrb, rb = k % g.nrb;
    va += q.pA[(b * g.nheads + h) * g.nrb + rb];
  }
  va = block_sum64(va, ws);
  if (threadIdx.x == 0) q.dA[h] = va;
  if (q.dbias) {
    double vb = 0.0;
    for (int64_t k = threadIdx.x; k < g.batch * g.length; k += kLanes) vb += q.ddt[k * g.nheads + h];
    vb = block_sum64(vb, ws);
    if (threadIdx.x == 0) q.dbias[h] = vb;
  }
  if (q.dD) {
    if (g.d_per_row) {
      for (int64_t pp = threadIdx.x; pp < P; pp += kLanes) {
        double v = 0.0;
        for (int64_t b = 0; b < g.batch; ++b) v += q.pD[(b * g.nheads + h) * P + pp];
        q.dD[h * P + pp] = v;
      }
    } else {
      double v = 0.0;
      for (int64_t k = threadIdx.x; k < g.batch * P; k += kLanes) {
        const int64_t b = k / P, pp = k % P;
        v += q.pD[(b * g.nheads + h) * P + pp];
      }
      v = block_sum64(v, ws);
      if (threadIdx.x == 0) q.dD[h] = v;
    }
  }
}

// ---------------------------------------------------------------- host

int make_geo(const mko_ssd_params* prm, Geo* g) {
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
  if (prm->dt_dtype != MKO_F64 || prm->bc_dtype != MKO_F64) {
    mko_set_error("ssd: with float64 x, dt, B and C are float64 too");
    return MKO_EINVAL;
  }
  if (g->dstate > 64 * kPerLane) {
    mko_set_error("ssd: float64 runs d_state <= %d, got %lld", 64 * kPerLane, static_cast<long long>(g->dstate));
    return MKO_EUNSUPPORTED;
  }
  int tn = 1;
  while (tn * kPerLane < g->dstate) tn <<= 1;
  g->tn = tn;
  g->rows = kLanes / tn;
  g->nrb = static_cast<int>((g->headdim + g->rows - 1) / g->rows);
  g->nblk = static_cast<int>((g->length + kBlock - 1) / kBlock);
  g->hpg = static_cast<int>(g->nheads / g->ngroups);
  if (g->nrb > 65535 || g->nheads > 65535 || g->batch > 65535) {
    mko_set_error("ssd: float64 grid too large (row blocks, heads and batch at most 65535 each)");
    return MKO_EUNSUPPORTED;
  }
  g->softplus = (prm->flags & MKO_SSD_SOFTPLUS) ? 1 : 0;
  g->d_per_row = (prm->flags & MKO_SSD_D_PER_ROW) ? 1 : 0;
  return MKO_OK;
}

static size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

static size_t saved_bytes(const Geo& g) {
  return align256(static_cast<size_t>(g.batch * g.nheads) * g.nblk * g.headdim * g.dstate * 8);
}

struct BwdLayout {
  size_t pbc, pdel, pA, pD, total;
};

static BwdLayout bwd_layout(const Geo& g) {
  BwdLayout l{};
  const size_t rows = static_cast<size_t>(g.batch * g.length * g.nheads) * g.nrb;
  size_t o = 0;
  l.pbc = o; o = align256(o + rows * 2 * g.dstate * 8);
  l.pdel = o; o = align256(o + rows * 8);
  l.pA = o; o = align256(o + static_cast<size_t>(g.batch * g.nheads) * g.nrb * 8);
  l.pD = o; o = align256(o + static_cast<size_t>(g.batch * g.nheads * g.headdim) * 8);
  l.total = o;
  return l;
}

static Ptrs ptrs(const mko_ssd_params* prm) {
  Ptrs q{};
  q.x = static_cast<const double*>(prm->x);
  q.dt = static_cast<const double*>(prm->dt);
  q.A = reinterpret_cast<const double*>(prm->A);
  q.B = static_cast<const double*>(prm->B);
  q.C = static_cast<const double*>(prm->C);
  q.D = reinterpret_cast<const double*>(prm->D);
  q.z = static_cast<const double*>(prm->z);
  q.bias = reinterpret_cast<const double*>(prm->dt_bias);
  q.init = static_cast<const double*>(prm->initial_states);
  q.dy = static_cast<const double*>(prm->dy);
  q.dfinal = static_cast<const double*>(prm->dfinal);
  q.y = static_cast<double*>(prm->y);
  q.final_state = static_cast<double*>(prm->final_state);
  q.dx = static_cast<double*>(prm->dx);
  q.ddt = static_cast<double*>(prm->ddt);
  q.dA = reinterpret_cast<double*>(prm->dA);
  q.dB = static_cast<double*>(prm->dB);
  q.dC = static_cast<double*>(prm->dC);
  q.dD = reinterpret_cast<double*>(prm->dD);
  q.dz = static_cast<double*>(prm->dz);
  q.dbias = reinterpret_cast<double*>(prm->ddt_bias);
  q.dinit = static_cast<double*>(prm->dinitial);
  q.ckpt = static_cast<double*>(prm->saved);
  return q;
}

static dim3 grid_of(const Geo& g) {
  return dim3(static_cast<unsigned>(g.nrb), static_cast<unsigned>(g.nheads), static_cast<unsigned>(g.batch));
}

}  // namespace ssd64

size_t ssd64_saved_bytes(const mko_ssd_params* prm) {
  ssd64::Geo g;
  if (ssd64::make_geo(prm, &g) != MKO_OK) return 0;
  return ssd64::saved_bytes(g);
}

size_t ssd64_bwd_workspace_size(const mko_ssd_params* prm) {
  ssd64::Geo g;
  if (ssd64::make_geo(prm, &g) != MKO_OK) return 0;
  return ssd64::bwd_layout(g).total;
}

int ssd64_fwd(const mko_ssd_params* prm, hipStream_t s) {
  ssd64::Geo g;
  const int st = ssd64::make_geo(prm, &g);
  if (st != MKO_OK) return st;
  if (g.batch == 0) return MKO_OK;
  if (!prm->A || !prm->final_state ||
      (g.length > 0 && (!prm->x || !prm->dt || !prm->B || !prm->C || !prm->y || !prm->saved))) {
    mko_set_error("ssd_fwd: x, dt, A, B, C, y, final_state and saved are required");
    return MKO_EINVAL;
  }
  MKO_TIMED("ssd64_fwd", s, ssd64::fwd<<<ssd64::grid_of(g), ssd64::kLanes, 0, s>>>(g, ssd64::ptrs(prm)));
  return mko_check_launch("ssd_fwd (float64)");
}

int ssd64_bwd(const mko_ssd_params* prm, hipStream_t s) {
  ssd64::Geo g;
  const int st = ssd64::make_geo(prm, &g);
  if (st != MKO_OK) return st;
  const bool tokens = g.batch > 0 && g.length > 0;
  if (!prm->A || !prm->dA || !prm->dy ||
      (tokens && (!prm->x || !prm->dt || !prm->B || !prm->C || !prm->saved || !prm->dx || !prm->ddt || !prm->dB ||
                  !prm->dC))) {
    mko_set_error("ssd_bwd: x, dt, A, B, C, saved, dy, dx, ddt, dA, dB and dC are required");
    return MKO_EINVAL;
  }
  if ((prm->D && !prm->dD) || (tokens && prm->z && !prm->dz) || (prm->dt_bias && !prm->ddt_bias)) {
    mko_set_error("ssd_bwd: dD, dz and ddt_bias are required with D, z and dt_bias");
    return MKO_EINVAL;
  }
  if (g.batch == 0) return MKO_OK;
  const ssd64::BwdLayout lay = ssd64::bwd_layout(g);
  if (prm->workspace_bytes < lay.total || !prm->workspace) {
    mko_set_error("ssd_bwd: workspace of %zu bytes needed, %zu given", lay.total, prm->workspace_bytes);
    return MKO_EWORKSPACE;
  }
  ssd64::Ptrs q = ssd64::ptrs(prm);
  char* ws = static_cast<char*>(prm->workspace);
  q.pbc = reinterpret_cast<double*>(ws + lay.pbc);
  q.pdel = reinterpret_cast<double*>(ws + lay.pdel);
  q.pA = reinterpret_cast<double*>(ws + lay.pA);
  q.pD = reinterpret_cast<double*>(ws + lay.pD);
  using ssd64::kLanes;
  MKO_TIMED("ssd64_bwd", s, ssd64::bwd<<<ssd64::grid_of(g), kLanes, 0, s>>>(g, q));
  const int64_t nbc = g.batch * g.length * g.ngroups * g.dstate;
  const int64_t ndt = g.batch * g.length * g.nheads;
  if (nbc > 0)
    MKO_TIMED("ssd64_reduce", s,
              ssd64::reduce_bc<<<static_cast<unsigned>((nbc + kLanes - 1) / kLanes), kLanes, 0, s>>>(g, q));
  if (ndt > 0)
    MKO_TIMED("ssd64_reduce", s,
              ssd64::reduce_dt<<<static_cast<unsigned>((ndt + kLanes - 1) / kLanes), kLanes, 0, s>>>(g, q));
  MKO_TIMED("ssd64_reduce", s, ssd64::reduce_params<<<static_cast<unsigned>(g.nheads), kLanes, 0, s>>>(g, q));
  return mko_check_launch("ssd_bwd (float64)");
}

}  // namespace mko
