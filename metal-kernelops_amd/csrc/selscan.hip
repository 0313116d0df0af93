// Mamba-1 selective scan, forward and backward, for gfx950.
//
// Mapping: one lane per channel row (batch, d).  A wavefront holds 64 channels of
// one (batch, group) whenever dim/ngroups is a multiple of 64 ("uniform" mode), so
// B_t and C_t are wave-uniform and the dB/dC sums over channels are cross-lane
// reductions.  Each lane walks time sequentially with its N states in registers.
//
// Time parallelism: the sequence is cut into `nchunks` coarse chunks of `lc`
// steps (a multiple of 64).  The forward is three launches:
//   1. fwd_summary: per chunk, the state it leaves from a zero entry and the sum
//      of its steps (its decay is exp(A * sum));
//   2. chain: per (row, state), the exact entering state of every chunk;
//   3. fwd_replay: replays every chunk from its entering state, writes
//      out = (C.x + D u) * silu(z) and the state entering every 16-step block.
// The backward mirrors it: bwd_summary (each chunk's adjoint from a zero exit),
// a reverse chain, then bwd_main, which walks every chunk backwards one 16-step
// block at a time, recomputing the block's forward states from the saved state,
// and finally small reduction kernels for dB/dC, dA, dD and ddelta_bias.
//
// Per-step inputs of the state-inner loops (one lane, all states, one step at a
// time) are staged through LDS so the step loop is a real loop and B_t/C_t are
// fetched one step at a time.
#include <type_traits>

#include "common.hpp"
#include "io.hpp"

namespace mko {
namespace ss {

constexpr int CK = MKO_SS_CHECKPOINT;  // steps between saved states
constexpr int HS = 16;                 // steps held in registers / staged at a time

struct Geo {
  int64_t batch, dim, length, dstate, ngroups;
  int64_t rows;      // batch * dim
  int64_t dg;        // channels per group
  int64_t nwr;       // wave rows = ceil(rows / 64)
  int lc;            // coarse chunk length (multiple of CK)
  int nchunks;       // number of coarse chunks
  int nck;           // saved states per row = ceil(length / CK)
  int wpg;           // wavefronts per workgroup
  int ncb;           // channel blocks (of 64*wpg channels) per group, uniform mode
  int u_dtype, d_dtype, bc_dtype;
  int softplus;
  int vec;           // per-element rows may use 16-byte vector accesses
};

struct Ptrs {
  const void* u;
  const void* delta;
  const float* A;
  const void* B;
  const void* C;
  const float* D;
  const void* z;
  const float* bias;
  const void* dout;
  void* out;
  float* states;
  void* du;
  void* ddelta;
  void* dz;
  // workspace
  float* bt;     // (batch*G, L, NS) B, time-major, fp32, zero-padded states
  float* ct;     // (batch*G, L, NS) C
  float* bn;     // (batch*G, NS, L) B, state-major (backward)
  float* cn;     // (batch*G, NS, L) C
  float* drive;  // (rows, nchunks, N) chunk summaries
  float* sumd;   // (rows, nchunks) sum of steps per chunk
  float* adj;    // (rows, nchunks, N) adjoint entering each chunk from the right
  float* pbc;    // (batch*G, ncb, L, NS, 2) dB/dC partial sums
  float* dap;    // (nchunks, NS, rows) dA partials
  float* ddp;    // (nchunks, rows) dD partials
  float* dbp;    // (nchunks, rows) ddelta_bias partials
};

struct LaneInfo {
  int64_t row;   // clamped to a valid row
  bool active;
  int64_t d;
  int64_t bg;    // batch * G + group
  int64_t wave_row;
};

__device__ __forceinline__ LaneInfo lane_info(const Geo& g, bool uni) {
  LaneInfo li;
  const int wave = uniform(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  li.wave_row = static_cast<int64_t>(blockIdx.x) * g.wpg + wave;
  const int64_t row = li.wave_row * kWave + lane;
  li.active = row < g.rows;
  li.row = li.active ? row : g.rows - 1;
  li.d = li.row % g.dim;
  if (uni) {
    const int64_t r0 = li.wave_row * kWave;
    const int64_t b0 = r0 / g.dim;
    const int64_t g0 = (r0 % g.dim) / g.dg;
    li.bg = __builtin_amdgcn_readfirstlane(static_cast<int>(b0 * g.ngroups + g0));
  } else {
    li.bg = (li.row / g.dim) * g.ngroups + li.d / g.dg;
  }
  return li;
}

__device__ __forceinline__ float step_of(const Geo& g, float raw, float bias) {
  const float v = raw + bias;
  return g.softplus ? softplus(v) : v;
}

// Saved scan states, (batch, checkpoint, dim, state): a channel's states are contiguous, so
// a lane-per-channel wavefront reads or writes 64 consecutive channels' states as one run,
// and the lane-per-state kernels' 4 channels x 16 states are 256 contiguous bytes.
__device__ __forceinline__ int64_t ck_index(const Geo& g, int64_t row, int64_t k, int64_t n) {
  const int64_t b = row / g.dim, d = row - b * g.dim;
  return ((b * g.nck + k) * g.dim + d) * g.dstate + n;
}

// ---------------------------------------------------------------- layout prep

// B, C (bg, N, L) any dtype -> the fp32 copies the scan kernels read: time-major
// (bg, L, NS) in bt/ct and state-major (bg, NS, L) in bn/cn, states >= N zeroed. Any
// output may be null. A workgroup converts one kPrepSteps-step tile of one (batch,
// group): the loads and the state-major stores run along L, and the time-major stores
// go through an LDS transpose so that they run along the states.
constexpr int kPrepSteps = 64;

template <int NS>
__global__ void __launch_bounds__(256) prep_layouts(Geo g, int64_t ntiles, const void* B, const void* C,
                                                    float* bt, float* ct, float* bn, float* cn) {
  __shared__ float tile[2][kPrepSteps][NS + 1];
  const int64_t bg = blockIdx.x / ntiles;
  const int64_t t0 = (blockIdx.x % ntiles) * kPrepSteps;
  const int tl = threadIdx.x & (kPrepSteps - 1);
  const int64_t t = t0 + tl;
  const bool in_t = t < g.length;
  const int N = static_cast<int>(g.dstate);
  for (int n = static_cast<int>(threadIdx.x) / kPrepSteps; n < NS; n += 256 / kPrepSteps) {
    float vb = 0.0f, vc = 0.0f;
    if (in_t && n < N) {
      const int64_t src = (bg * N + n) * g.length + t;
      if (B) vb = load_one(B, g.bc_dtype, src);
      if (C) vc = load_one(C, g.bc_dtype, src);
    }
    tile[0][tl][n] = vb;
    tile[1][tl][n] = vc;
    if (in_t) {
      const int64_t dst = (bg * NS + n) * g.length + t;
      if (bn) bn[dst] = vb;
      if (cn) cn[dst] = vc;
    }
  }
  if (!bt && !ct) return;  // the same for the whole grid
  __syncthreads();
  const int64_t base = (bg * g.length + t0) * NS;
  const int nt = static_cast<int>(min(static_cast<int64_t>(kPrepSteps), g.length - t0));
  for (int e = threadIdx.x; e < nt * NS; e += 256) {
    const int tt = e / NS, n = e % NS;
    if (bt) bt[base + e] = tile[0][tt][n];
    if (ct) ct[base + e] = tile[1][tt][n];
  }
}

// ---------------------------------------------------------------- forward

// One step's B_t (and C_t) for a lane: scalar loads when the wavefront shares
// (batch, group), vector loads otherwise.  WITH_B / WITH_C select the rows.
template <int NS, bool UNI, bool WITH_B, bool WITH_C>
struct StepBC {
  float b[NS], c[NS];
  __device__ __forceinline__ void load(const float* __restrict__ bt, const float* __restrict__ ct,
                                       int64_t off) {
    if (UNI) {
      if (WITH_B) {
        const cfptr pb = as_const(bt + off);
#pragma unroll
        for (int n = 0; n < NS; ++n) b[n] = pb[n];
      }
      if (WITH_C) {
        const cfptr pc = as_const(ct + off);
#pragma unroll
        for (int n = 0; n < NS; ++n) c[n] = pc[n];
      }
    } else {
      if (WITH_B) {
        const float4* qb = reinterpret_cast<const float4*>(bt + off);
#pragma unroll
        for (int v = 0; v < NS / 4; ++v) {
          const float4 w = qb[v];
          b[4 * v] = w.x; b[4 * v + 1] = w.y; b[4 * v + 2] = w.z; b[4 * v + 3] = w.w;
        }
      }
      if (WITH_C) {
        const float4* qc = reinterpret_cast<const float4*>(ct + off);
#pragma unroll
        for (int v = 0; v < NS / 4; ++v) {
          const float4 w = qc[v];
          c[4 * v] = w.x; c[4 * v + 1] = w.y; c[4 * v + 2] = w.z; c[4 * v + 3] = w.w;
        }
      }
    }
  }
};

// One state-inner step: x <- exp(A del) x + du B; returns <C, x> when WITH_Y.
template <int NS, bool WITH_Y>
__device__ __forceinline__ float advance(const float (&A2)[NS], float del, float du, const float (&b)[NS],
                                         const float (&c)[NS], float (&x)[NS]) {
  float acc = 0.0f;
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    x[n] = fmaf(fast_exp2(A2[n] * del), x[n], du * b[n]);
    if (WITH_Y) acc = fmaf(c[n], x[n], acc);
  }
  return acc;
}

// Advances the states over the first nv steps of a block starting at t0 (per-step
// del/du in registers, indexed by the wave-uniform step).  Two B/C buffers
// alternate: each half-iteration retires the outstanding loads, requests the
// next step's B/C, then computes the current step, so a load has a whole step of
// work to arrive.  With WITH_Y, y[i] = <C_t, x_t>.
template <int NS, bool UNI, bool WITH_Y>
__device__ __forceinline__ void forward_block(const float* __restrict__ bt, const float* __restrict__ ct,
                                              int64_t row0, int t0, int nv, const float (&del)[HS],
                                              const float (&du)[HS], const float (&A2)[NS], float (&x)[NS],
                                              float (&y)[HS]) {
  StepBC<NS, UNI, true, WITH_Y> e0, e1;
  e0.load(bt, ct, (row0 + t0) * NS);
  for (int i = 0; i < nv; i += 2) {
    const bool two = i + 1 < nv;
    wait_lgkm();
    if (two) e1.load(bt, ct, (row0 + t0 + i + 1) * NS);
    float acc = advance<NS, WITH_Y>(A2, del[i], du[i], e0.b, e0.c, x);
    if (WITH_Y) y[i] = acc;
    if (two) {
      wait_lgkm();
      if (i + 2 < nv) e0.load(bt, ct, (row0 + t0 + i + 2) * NS);
      acc = advance<NS, WITH_Y>(A2, del[i + 1], du[i + 1], e1.b, e1.c, x);
      if (WITH_Y) y[i + 1] = acc;
    }
  }
}

// One 16-step block of the time-major B (and C) rows of a wavefront's (batch, group),
// staged through the wavefront's own LDS: each lane fetches HS*NS/64 floats per
// matrix (coalesced) one block ahead, then writes them to the idle buffer.  The step
// loop reads a step's row with broadcast LDS loads, whose waits are exact (unlike
// scalar loads, which can only be waited for all together).
template <int NS, bool WB, bool WC>
struct WaveBC {
  static constexpr int PER = HS * NS / kWave;
  float rb[PER], rc[PER];
  __device__ __forceinline__ void fetch(const float* __restrict__ bt, const float* __restrict__ ct, int64_t off) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      if (WB) rb[k] = bt[off + lane + k * kWave];
      if (WC) rc[k] = ct[off + lane + k * kWave];
    }
  }
  __device__ __forceinline__ void put(float* sb, float* sc) const {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      if (WB) sb[lane + k * kWave] = rb[k];
      if (WC) sc[lane + k * kWave] = rc[k];
    }
  }
};

template <int NS>
__device__ __forceinline__ void lds_row(const float* src, float (&v)[NS]) {
#pragma unroll
  for (int q = 0; q < NS / 4; ++q) {
    const float4 w = reinterpret_cast<const float4*>(src)[q];
    v[4 * q] = w.x;
    v[4 * q + 1] = w.y;
    v[4 * q + 2] = w.z;
    v[4 * q + 3] = w.w;
  }
}

// forward_block over a whole block with B/C rows from LDS (sb/sc: [HS][NS]).
template <int NS, bool WITH_Y>
__device__ __forceinline__ void forward_block_lds(const float* sb, const float* sc, const float (&del)[HS],
                                                  const float (&du)[HS], const float (&A2)[NS], float (&x)[NS],
                                                  float (&y)[HS]) {
#pragma unroll
  for (int i = 0; i < HS; ++i) {
    float b[NS], c[NS];
    lds_row<NS>(sb + i * NS, b);
    if (WITH_Y) lds_row<NS>(sc + i * NS, c);
    const float acc = advance<NS, WITH_Y>(A2, del[i], du[i], b, c, x);
    if (WITH_Y) y[i] = acc;
  }
}

// The element type of u / z / dout / du / dz.  Dyn: read from Geo at run time (any
// length, any alignment, any delta dtype); float / _Float16 / bf16: the typed path
// (delta float32, whole 16-step blocks, 16-byte aligned rows), whose loads keep the
// raw words in registers until they are used, so a block's inputs can be requested
// while the previous block is computed.
struct Dyn {};

template <class T, int NE = HS>
struct RawRun {  // NE consecutive elements of a row, raw
  static constexpr int W = NE * static_cast<int>(sizeof(T)) / 4;
  uint32_t w[W];
  __device__ __forceinline__ void load(const Geo&, const void* base, int, int64_t off, int) {
    load_words(static_cast<const T*>(base) + off, w);
  }
  __device__ __forceinline__ void get(float (&f)[NE]) const { unpack_words<T, NE>(w, f); }
};

template <>
struct RawRun<Dyn, HS> {
  float f[HS];
  __device__ __forceinline__ void load(const Geo& g, const void* base, int dtype, int64_t off, int nv) {
    load_run<HS>(base, dtype, off, nv, g.vec, f);
  }
  __device__ __forceinline__ void get(float (&o)[HS]) const {
#pragma unroll
    for (int i = 0; i < HS; ++i) o[i] = f[i];
  }
};

// delta's type in each path
template <class TU>
using DeltaT = typename std::conditional<__is_same(TU, Dyn), Dyn, float>::type;

template <class TU>
__device__ __forceinline__ void store_u(const Geo& g, void* base, int64_t off, int nv, const float (&v)[HS]) {
  if constexpr (__is_same(TU, Dyn))
    store_run<HS>(base, g.u_dtype, off, nv, g.vec, v);
  else
    store_run_t<TU, HS>(static_cast<TU*>(base) + off, HS, true, v);
}
template <class TU>
__device__ __forceinline__ void store_d(const Geo& g, void* base, int64_t off, int nv, const float (&v)[HS]) {
  if constexpr (__is_same(TU, Dyn))
    store_run<HS>(base, g.d_dtype, off, nv, g.vec, v);
  else
    store_run_t<float, HS>(static_cast<float*>(base) + off, HS, true, v);
}

// Step sizes and du = step * u of one block from raw runs; returns the sum of steps.
__device__ __forceinline__ float steps_from(const Geo& g, const float (&raw)[HS], const float (&uu)[HS], int nv,
                                            float bias, float (&del)[HS], float (&du)[HS]) {
  float sd = 0.0f;
#pragma unroll
  for (int i = 0; i < HS; ++i) {
    del[i] = i < nv ? step_of(g, raw[i], bias) : 0.0f;
    du[i] = del[i] * uu[i];
    sd += del[i];
  }
  return sd;
}

template <int NS, bool UNI, class TU>
__global__ void __launch_bounds__(256) fwd_summary(Geo g, Ptrs p) {
  const LaneInfo li = lane_info(g, UNI);
  const int N = static_cast<int>(g.dstate);
  const int c = blockIdx.y;
  const int t_begin = c * g.lc;
  const int t_end = min(t_begin + g.lc, static_cast<int>(g.length));
  float A2[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) A2[n] = n < N ? p.A[li.d * N + n] * kLog2e : 0.0f;
  const float bias = p.bias ? p.bias[li.d] : 0.0f;
  float x[NS], unused[HS];
#pragma unroll
  for (int n = 0; n < NS; ++n) x[n] = 0.0f;
  float sd = 0.0f;
  const int64_t rbase = li.row * g.length;
  const int t_last = t_begin + ((t_end - t_begin - 1) / HS) * HS;
  RawRun<DeltaT<TU>> rd;
  RawRun<TU> ru;
  rd.load(g, p.delta, g.d_dtype, rbase + t_begin, min(HS, t_end - t_begin));
  ru.load(g, p.u, g.u_dtype, rbase + t_begin, min(HS, t_end - t_begin));
  constexpr bool kLds = UNI && !__is_same(TU, Dyn);
  __shared__ float sbc[kLds ? 4 * 2 * HS * NS : 1];  // per wavefront: two buffers of [HS][NS] B rows
  float* wb = sbc + (kLds ? (threadIdx.x >> 6) * 2 * HS * NS : 0);
  WaveBC<NS, true, false> st;
  const int64_t brow = li.bg * g.length;
  if constexpr (kLds) {
    st.fetch(p.bt, nullptr, (brow + t_begin) * NS);
    st.put(wb, nullptr);
    wave_lds_sync();
  }
  int cur = 0;
  for (int t0 = t_begin; t0 < t_end; t0 += HS) {
    const int nv = min(HS, t_end - t0);
    float raw[HS], uu[HS], del[HS], du[HS];
    rd.get(raw);
    ru.get(uu);
    const int tn = t0 + HS < t_last ? t0 + HS : t_last;  // next block (the last one repeats)
    rd.load(g, p.delta, g.d_dtype, rbase + tn, min(HS, t_end - tn));
    ru.load(g, p.u, g.u_dtype, rbase + tn, min(HS, t_end - tn));
    sd += steps_from(g, raw, uu, nv, bias, del, du);
    if constexpr (kLds) {
      st.fetch(p.bt, nullptr, (brow + tn) * NS);
      forward_block_lds<NS, false>(wb + cur * HS * NS, nullptr, del, du, A2, x, unused);
      cur ^= 1;
      st.put(wb + cur * HS * NS, nullptr);
      wave_lds_sync();
    } else {
      forward_block<NS, UNI, false>(p.bt, nullptr, brow, t0, nv, del, du, A2, x, unused);
    }
  }
  if (li.active) {
    const int64_t o = (li.row * g.nchunks + c) * N;
#pragma unroll
    for (int n = 0; n < NS; ++n)
      if (n < N) p.drive[o + n] = x[n];
    p.sumd[li.row * g.nchunks + c] = sd;
  }
}

// Forward: state entering chunk c (written at saved-state slot c*lc/CK).
// Reverse: adjoint entering chunk c from the right.
template <bool REV>
__global__ void __launch_bounds__(256) chain(Geo g, const float* __restrict__ A,
                                             const float* __restrict__ drive,
                                             const float* __restrict__ sumd, float* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int N = static_cast<int>(g.dstate);
  if (i >= g.rows * N) return;
  const int64_t row = i / N;
  const int n = static_cast<int>(i % N);
  const float a2 = A[(row % g.dim) * N + n] * kLog2e;
  const int k = g.nchunks;
  // The chunk maps (decay, drive) do not depend on the carried state: they are fetched
  // PB chunks at a time (clamped indices, so every load is issued), then composed.
  constexpr int PB = 16;
  float dec[PB], drv[PB];
  auto fetch = [&](int c0, int dir) {
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      int c = c0 + dir * q;
      c = c < 0 ? 0 : (c >= k ? k - 1 : c);
      dec[q] = sumd[row * k + c];
      drv[q] = drive[(row * k + c) * N + n];
    }
  };
  if (!REV) {
    const int per = g.lc / CK;
    float x = 0.0f;
    for (int c0 = 0; c0 < k; c0 += PB) {
      fetch(c0, 1);
#pragma unroll
      for (int q = 0; q < PB; ++q) {
        const int c = c0 + q;
        if (c >= k) break;
        out[ck_index(g, row, static_cast<int64_t>(c) * per, n)] = x;
        if (c + 1 < k) x = fmaf(fast_exp2(a2 * dec[q]), x, drv[q]);
      }
    }
  } else {
    float h = 0.0f;
    for (int c0 = k - 1; c0 >= 0; c0 -= PB) {
      fetch(c0, -1);
#pragma unroll
      for (int q = 0; q < PB; ++q) {
        const int c = c0 - q;
        if (c < 0) break;
        out[(row * k + c) * N + n] = h;
        if (c > 0) h = fmaf(fast_exp2(a2 * dec[q]), h, drv[q]);
      }
    }
  }
}

// FULL: dstate == NS (no padded states), so the saved-state stores need no guards.
// The same chain with one wavefront per (row, state), for problems of few rows and many
// chunks, where one thread per pair walking the chunks in turn leaves most of the chip
// idle. Each lane composes the maps x -> e x + d of a run of consecutive chunks (in walk
// order), a scan across the wavefront composes the runs before each lane, and each lane
// walks its run again from that entering value to write the states. The map of the last
// chunk in walk order is never applied (its summary is not computed), so no run reads it.
template <bool REV>
__global__ void __launch_bounds__(256) chain_wave(Geo g, const float* __restrict__ A,
                                                  const float* __restrict__ drive,
                                                  const float* __restrict__ sumd, float* __restrict__ out) {
  const int64_t pair = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int N = static_cast<int>(g.dstate);
  if (pair >= g.rows * N) return;  // the same for the whole wavefront
  const int lane = threadIdx.x & 63;
  const int64_t row = pair / N;
  const int n = static_cast<int>(pair % N);
  const float a2 = A[(row % g.dim) * N + n] * kLog2e;
  const int k = g.nchunks;
  const int run = (k + kWave - 1) / kWave;
  const int r0 = min(lane * run, k), r1 = min(r0 + run, k);
  // the maps of walk positions b0 .. b0 + PB - 1, fetched together (clamped positions:
  // every load is issued; values past the run are not used)
  constexpr int PB = 8;
  float e[PB], d[PB];
  auto fetch = [&](int b0) {
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      const int r = min(b0 + q, k - 1);
      const int64_t c = row * k + (REV ? k - 1 - r : r);
      e[q] = sumd[c];
      d[q] = drive[c * N + n];
    }
#pragma unroll
    for (int q = 0; q < PB; ++q) e[q] = fast_exp2(a2 * e[q]);
  };
  const int rc = min(r1, k - 1);  // the maps this run applies
  float E = 1.0f, D = 0.0f;
  for (int b0 = r0; b0 < rc; b0 += PB) {
    fetch(b0);
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      const bool use = b0 + q < rc;
      const float eq = use ? e[q] : 1.0f, dq = use ? d[q] : 0.0f;
      E *= eq;
      D = fmaf(eq, D, dq);
    }
  }
  // inclusive scan: the maps of lanes below apply first
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const float Ep = __shfl_up(E, off), Dp = __shfl_up(D, off);
    if (lane >= off) {
      D = fmaf(E, Dp, D);
      E *= Ep;
    }
  }
  float x = __shfl_up(D, 1);  // every earlier run applied to the zero entering state
  if (lane == 0) x = 0.0f;
  const int per = g.lc / CK;
  for (int b0 = r0; b0 < r1; b0 += PB) {
    if (run > PB || b0 != r0) fetch(b0);  // a run of at most PB maps is still held
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      const int r = b0 + q;
      if (r >= r1) break;
      if (REV)
        out[(row * k + (k - 1 - r)) * N + n] = x;
      else
        out[ck_index(g, row, static_cast<int64_t>(r) * per, n)] = x;
      if (r + 1 < k) x = fmaf(e[q], x, d[q]);
    }
  }
}

template <int NS, bool UNI, class TU, bool FULL>
__global__ void __launch_bounds__(256) fwd_replay(Geo g, Ptrs p) {
  const LaneInfo li = lane_info(g, UNI);
  const int N = static_cast<int>(g.dstate);
  const int c = blockIdx.y;
  const int t_begin = c * g.lc;
  const int t_end = min(t_begin + g.lc, static_cast<int>(g.length));
  float A2[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) A2[n] = n < N ? p.A[li.d * N + n] * kLog2e : 0.0f;
  const float bias = p.bias ? p.bias[li.d] : 0.0f;
  const float Dd = p.D ? p.D[li.d] : 0.0f;
  const bool has_z = p.z != nullptr;
  float x[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) x[n] = n < N ? p.states[ck_index(g, li.row, t_begin / CK, n)] : 0.0f;
  const int64_t rbase = li.row * g.length;
  const int t_last = t_begin + ((t_end - t_begin - 1) / HS) * HS;
  RawRun<DeltaT<TU>> rd;
  RawRun<TU> ru, rz;
  const void* zsrc = has_z ? p.z : p.u;  // without z the third run repeats u (unused)
  rd.load(g, p.delta, g.d_dtype, rbase + t_begin, min(HS, t_end - t_begin));
  ru.load(g, p.u, g.u_dtype, rbase + t_begin, min(HS, t_end - t_begin));
  rz.load(g, zsrc, g.u_dtype, rbase + t_begin, min(HS, t_end - t_begin));
  constexpr bool kLds = UNI && !__is_same(TU, Dyn);
  __shared__ float sbc[kLds ? 4 * 4 * HS * NS : 1];  // per wavefront: two buffers of B rows, two of C rows
  float* wb = sbc + (kLds ? (threadIdx.x >> 6) * 4 * HS * NS : 0);
  float* wc = wb + 2 * HS * NS;
  WaveBC<NS, true, true> st;
  const int64_t brow = li.bg * g.length;
  if constexpr (kLds) {
    st.fetch(p.bt, p.ct, (brow + t_begin) * NS);
    st.put(wb, wc);
    wave_lds_sync();
  }
  int cur = 0;
  for (int t0 = t_begin; t0 < t_end; t0 += HS) {
    // the state entering this block (saved every block, CK == HS; at the chunk's
    // first block it rewrites the value the chain stored).  Unconditional, so the
    // loads in flight are the same on every path; lanes past the last row hold the
    // clamped last row and store identical values.
    static_assert(CK == HS, "one saved state per block");
    {
      float* sp = p.states + ck_index(g, li.row, t0 / CK, 0);
      if constexpr (FULL) {
#pragma unroll
        for (int v = 0; v < NS / 4; ++v)
          reinterpret_cast<float4*>(sp)[v] = make_float4(x[4 * v], x[4 * v + 1], x[4 * v + 2], x[4 * v + 3]);
      } else {
#pragma unroll
        for (int n = 0; n < NS; ++n)
          if (n < N) sp[n] = x[n];
      }
    }
    const int nv = min(HS, t_end - t0);
    float raw[HS], uu[HS], zz[HS], del[HS], du[HS], y[HS];
    rd.get(raw);
    ru.get(uu);
    rz.get(zz);
    const int tn = t0 + HS < t_last ? t0 + HS : t_last;  // next block (the last one repeats)
    rd.load(g, p.delta, g.d_dtype, rbase + tn, min(HS, t_end - tn));
    ru.load(g, p.u, g.u_dtype, rbase + tn, min(HS, t_end - tn));
    rz.load(g, zsrc, g.u_dtype, rbase + tn, min(HS, t_end - tn));
    steps_from(g, raw, uu, nv, bias, del, du);
    if constexpr (kLds) {
      st.fetch(p.bt, p.ct, (brow + tn) * NS);
      forward_block_lds<NS, true>(wb + cur * HS * NS, wc + cur * HS * NS, del, du, A2, x, y);
      cur ^= 1;
      st.put(wb + cur * HS * NS, wc + cur * HS * NS);
      wave_lds_sync();
    } else {
      forward_block<NS, UNI, true>(p.bt, p.ct, brow, t0, nv, del, du, A2, x, y);
    }
#pragma unroll
    for (int i = 0; i < HS; ++i) y[i] = fmaf(Dd, uu[i], y[i]);
    if (has_z) {
#pragma unroll
      for (int i = 0; i < HS; ++i) y[i] *= zz[i] * sigmoid(zz[i]);
    }
    if (li.active) store_u<TU>(g, p.out, rbase + t0, nv, y);
  }
}

// ---------------------------------------------------------------- forward, lane per (channel, state)
//
// With dstate <= 16 and enough rows, a wavefront holds 4 channels x 16 states, lane (c, n),
// and walks the whole sequence once, 16 steps a block: no time chunks, so no summary pass
// and no replay.  Per block:
//   - lane (c, n) loads step t0 + n of its channel's delta, u and z (a wavefront reads 4 rows
//     x 16 consecutive steps) and forms that step's size and du = step * u;
//   - the 4 channels share one (batch, group), so the block's B and C (16 states x 16 steps
//     each) are fetched once per wavefront, 8 values a lane, and staged in LDS as float32;
//   - lane (c, n) advances its one state over the 16 steps, reading step i's size and du
//     from lane i of its row (DPP row_newbcast, folded into the multiplies) and B_n, C_n of
//     those steps from the staged block;
//   - the 16 states' C_n x_n per step go through a per-wavefront LDS transpose, so lane
//     (c, n) sums step t0 + n's, adds the skip, applies the gate and stores it;
//   - the state entering the block is saved (4 channels x 16 states: 256 contiguous bytes).
// A block's inputs are requested two blocks ahead.

template <int I, int END, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < END) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, END>(f);
  }
}

// The value held by lane I of each 16-lane row, in every lane of that row.
template <int I>
__device__ __forceinline__ float row_newbcast(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + I, 0xf, 0xf, false));
}

constexpr int kLaneChannels = 4;  // channels per wavefront in the lane-per-state kernels

// One 16-step block of B and C staged through LDS for a wavefront of the lane-per-state
// kernels, whose 4 channels share one (batch, group): lane l fetches 8 values of it (matrix
// l / 32, state (l / 2) mod 16, steps 8 (l mod 2) ..), stages them as float32 (zeros for
// padded states), and lane (c, n) reads its state's 16 steps back.  Rows are kBcRow floats:
// 16-byte aligned, and the 16 rows' reads fall in distinct banks.
constexpr int kBcRow = 20;

template <class TU, class TB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5))) fwd_lane(Geo g, Ptrs p) {
  constexpr int kRow = HS + 1;   // a step's 16 states, padded so the transposed reads miss no bank
  constexpr int kCS = HS * kRow; // one channel's [step][state] block (272 floats: 16 banks apart)
  __shared__ float sy[4][kLaneChannels * kCS];
  const int wave = uniform(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, cl = lane >> 4, n = lane & 15;
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * kLaneChannels + cl;
  const bool active = row < g.rows;
  const int64_t r = active ? row : g.rows - 1;
  const int64_t bb = r / g.dim, d = r - bb * g.dim;
  const int64_t bg = bb * g.ngroups + d / g.dg;
  const int N = static_cast<int>(g.dstate);
  const bool sn = n < N;
  const float a2 = sn ? p.A[d * N + n] * kLog2e : 0.0f;
  const float bias = p.bias ? p.bias[d] : 0.0f;
  const float Dd = p.D ? p.D[d] : 0.0f;
  const bool has_z = p.z != nullptr;
  const int64_t L = g.length;
  const int64_t rbase = r * L + n;  // this lane's step of every block
  const float* dp = static_cast<const float*>(p.delta) + rbase;
  const TU* up = static_cast<const TU*>(p.u) + rbase;
  const TU* zp = static_cast<const TU*>(has_z ? p.z : p.u) + rbase;
  TU* op = static_cast<TU*>(p.out) + rbase;
  float* sp = p.states + ck_index(g, r, 0, sn ? n : 0);
  const int64_t sstep = g.dim * N;  // one saved state further
  float* sw = sy[wave] + cl * kCS;
  // The wavefront's 4 channels share one (batch, group), so one 16-step block of B and C
  // serves all of them, staged through LDS (kBcRow).
  __shared__ __align__(16) float sbc[4][2][HS][kBcRow];
  const int sm = lane >> 5, sst = (lane >> 1) & 15, shf = lane & 1;
  const bool sok = sst < N;
  const TB* bcsrc = static_cast<const TB*>(sm ? p.C : p.B) + (bg * N + (sok ? sst : 0)) * L + 8 * shf;
  float* stg = &sbc[wave][sm][sst][8 * shf];
  const float* brow = &sbc[wave][0][n][0];
  const float* crow = &sbc[wave][1][n][0];

  struct In {
    float dl;
    TU u, z;
    RawRun<TB, 8> bc;
  };
  auto load = [&](int64_t t0, In& in) {
    in.dl = dp[t0];
    in.u = up[t0];
    in.z = zp[t0];
    in.bc.load(g, bcsrc, 0, t0, 8);
  };
  const int nblk = static_cast<int>(L / HS);
  // Two buffers of raw inputs: a block's raw words are unpacked first and then
  // reloaded with the block two further on (the last ones reload the last block), so
  // each load has two blocks of work to arrive.  32-bit B/C need no unpacking (the
  // raw words are the values), so their reload waits for the end of the block
  // instead of holding a second copy: one block of work, as many registers as one
  // buffer ahead.
  auto ahead = [&](int k) { return static_cast<int64_t>(k < nblk ? k : nblk - 1) * HS; };
  In ra, rb;
  load(0, ra);
  load(ahead(1), rb);
  float x = 0.0f;
  auto block = [&](int k, In& in) {
    const int64_t t0 = static_cast<int64_t>(k) * HS;
    if (active && sn) __builtin_nontemporal_store(x, sp + k * sstep);  // whole lines, read once by the backward
    const float uu = to_f32(in.u);
    const float zz = to_f32(in.z);
    const float del = step_of(g, in.dl, bias);
    {
      float sv[8];
      in.bc.get(sv);
      if (!sok) {  // a padded state adds nothing
#pragma unroll
        for (int i = 0; i < 8; ++i) sv[i] = 0.0f;
      }
      reinterpret_cast<float4*>(stg)[0] = make_float4(sv[0], sv[1], sv[2], sv[3]);
      reinterpret_cast<float4*>(stg)[1] = make_float4(sv[4], sv[5], sv[6], sv[7]);
    }
    if constexpr (sizeof(TB) == 2) load(ahead(k + 2), in);
    wave_lds_sync();
    float bv[HS], cv[HS];
    lds_row<HS>(brow, bv);
    lds_row<HS>(crow, cv);
    const float du = del * uu;
    static_for<0, HS>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      x = fmaf(fast_exp2(a2 * row_newbcast<i>(del)), x, row_newbcast<i>(du) * bv[i]);
      sw[i * kRow + n] = cv[i] * x;
    });
    wave_lds_sync();
    float s4[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) s4[m] = sw[n * kRow + m];
#pragma unroll
    for (int m = 4; m < HS; ++m) s4[m & 3] += sw[n * kRow + m];
    wave_lds_sync();
    float y = fmaf(Dd, uu, (s4[0] + s4[1]) + (s4[2] + s4[3]));
    if (has_z) y *= zz * sigmoid(zz);
    if (active) op[t0] = from_f32<TU>(y);
    if constexpr (sizeof(TB) == 4) load(ahead(k + 2), in);
  };
  for (int k = 0; k < nblk; k += 2) {
    block(k, ra);
    if (k + 1 < nblk) block(k + 1, rb);
  }
}

// ---------------------------------------------------------------- backward, lane per (channel, state)
//
// The backward in fwd_lane's mapping: a wavefront holds 4 channels x 16 states, lane (c, n), and
// walks the whole sequence once in reverse, 16 steps a block.  With every (channel, state) chain
// on its own lane there are enough wavefronts without cutting time into chunks, so the adjoint
// entering a block is simply carried over from the block to its right: no summary pass, no chain.
// Per block:
//   - lane (c, n) loads step t0 + n of its channel's delta, u, z, dout and out and forms that
//     element's step, du, gy = dout silu(z) and the factor of dz;
//   - B and C of the block come through LDS as in fwd_lane (kBcRow), lane (c, n) reading its
//     state's 16 steps of each;
//   - from the saved state entering the block, the lane recomputes the block's 16 states and
//     decays a = exp(A delta);
//   - it walks the 16 steps backwards with the adjoint h_t = gy_t C_t + a_{t+1} h_{t+1}, and per
//     step writes its state's terms of the two sums over states that du and ddelta need,
//     h_t B_t and A a_t x_{t-1} h_t, as one pair into the wavefront's LDS transpose, and adds its
//     dA term (the adjoint and dA multiply-adds take their step's gy and delta as a DPP row
//     broadcast, fmac_row);
//   - the dB and dC terms, h_t du_t and gy_t x_t, are summed over the wavefront's 4 channels
//     (one 16-lane row each) with gfx950's lane swaps: v_permlane32_swap exchanges the
//     wavefront's halves, so one add sums rows (0 + 2, 1 + 3) of a step's dB terms and, in the
//     other half, of its dC terms; v_permlane16_swap of two such registers (steps i and i + 1)
//     exchanges odd and even rows, and one more add leaves dB_i, dB_{i+1}, dC_i and dC_{i+1} as
//     the four rows of one register: 6 instructions per two steps, in a fixed order;
//   - lane (c, n) then owns step t0 + n: it sums its row of the transpose and writes du,
//     ddelta and dz.  The pre-gate output that dz needs comes back as out / silu(z); a block
//     where silu(z) is exactly zero somewhere (or out was not given) first sums a transpose
//     of C x instead;
//   - the workgroup's 4 wavefronts add their dB/dC blocks in a fixed order and write one
//     partial per 16 channels (per 4 channels when a group is not a multiple of 16 wide).
// A block's inputs are requested one block ahead.  Needs dstate <= 16, whole 16-step blocks,
// channels per group a multiple of 4, fp32 delta and 16-byte aligned rows.

// The transposes of a wavefront hold, per step, a row of 4 channels x 16 states of pairs
// (h B, A a x h): a step's two terms leave a lane as one 8-byte write at an immediate offset
// from one base address.  Rows are padded to 4 mod 32 floats, so the 16-byte reads of lanes
// (c, i..i+7), which read rows i..i+7, fall in distinct banks.
constexpr int kTrPitch = 2 * 4 * HS + 4;
constexpr int kTrFloats = HS * kTrPitch;  // one wavefront's transpose block

// The value lane I of each 16-lane row holds, in every lane of that row.  Every row and bank
// is enabled and bound_ctrl is set, so no lane keeps an old value: the move folds into the VALU
// instruction that consumes it, as its DPP source operand.
template <int I>
__device__ __forceinline__ float row_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + I, 0xf, 0xf, true));
}

// acc + (the value lane I of each 16-lane row holds in v) * m, as one v_fmac_f32 with the row
// broadcast as its DPP source (the compiler folds DPP into multiplies but not into fmac, and
// would otherwise spend a v_mov_b32_dpp on it).  A DPP source written by the instruction just
// before needs two wait states, which the compiler does not insert for inline assembly: with
// kGuard the instruction carries them itself; without it v must have been written well before
// (every caller's v is formed before the block's recompute, dozens of instructions earlier;
// tests/test_isa_hazards.py checks the built code).
template <int I, bool kGuard = false>
__device__ __forceinline__ float fmac_row(float acc, float v, float m) {
  if constexpr (kGuard)
    asm("s_nop 1\n\tv_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "+v"(acc) : "v"(v), "v"(m), "i"(I));
  else
    asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "+v"(acc) : "v"(v), "v"(m), "i"(I));
  return acc;
}

template <class TU, class TB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
bwd_lane(Geo g, Ptrs p, int cpb) {
  // per wavefront: the transposes of the pairs (h B, A a x h); in blocks that need it, the
  // first terms first transpose C x; the workgroup's dB/dC blocks reuse the buffers
  __shared__ __align__(16) float lds[4][kTrFloats];
  __shared__ __align__(16) float sbc[4][2][HS][kBcRow];  // B and C of the block (kBcRow)
  const int wave = uniform(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63, cl = lane >> 4, n = lane & 15;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * kLaneChannels;  // first row of the wave
  const bool active = row0 < g.rows;  // a wavefront's 4 rows are all valid or all past the end
  const int64_t r = active ? row0 + cl : g.rows - 1;
  const int64_t bb = r / g.dim, d = r - bb * g.dim;
  const int64_t bg = uniform(static_cast<int>((active ? row0 : g.rows - 1) / g.dg));  // (batch, group) of the wave
  const int N = static_cast<int>(g.dstate);
  const bool sn = n < N;  // states n >= N exist only as zero lanes
  const float an = sn ? p.A[d * N + n] : 0.0f;
  const float a2 = an * kLog2e;
  const float bias = p.bias ? p.bias[d] : 0.0f;
  const float Dd = p.D ? p.D[d] : 0.0f;
  const bool has_z = p.z != nullptr;
  const bool has_out = p.out != nullptr;
  const int64_t L = g.length;
  float* tr = lds[wave];
  // Lane offsets in elements (lane_bwd_shape keeps the per-row arrays and B/C below 2^31
  // elements each): this lane's
  // element of a block, its saved state, and its state's row of B and C (read straight from
  // memory: the wavefront's 4 channels read the same rows, which the vector L1 serves once).
  // Block offsets are added to wave-uniform base pointers.
  const uint32_t eoff = static_cast<uint32_t>(r * L + n);
  const uint32_t soff = static_cast<uint32_t>(ck_index(g, r, 0, sn ? n : 0));
  const int sm = lane >> 5, sst = (lane >> 1) & 15, shf = lane & 1;  // this lane's share of the B/C block
  const bool sok = sst < N;
  const uint32_t bcoff = static_cast<uint32_t>((bg * N + (sok ? sst : 0)) * L + 8 * shf);
  const TB* bcsrc = static_cast<const TB*>(sm ? p.C : p.B);
  float* stg = &sbc[wave][sm][sst][8 * shf];
  const float* brow = &sbc[wave][0][n][0];
  const float* crow = &sbc[wave][1][n][0];
  const int tw = cl * HS + n;  // this lane's column in a transpose row
  const int64_t sstep = g.dim * N;
  const TU* zsrc = static_cast<const TU*>(has_z ? p.z : p.u);
  const TU* osrc = static_cast<const TU*>(has_out ? p.out : p.u);
  // dB/dC partial slot of the wavefront (cpb 4) or workgroup (cpb 16): partial index = first row / cpb
  float2* pbc = reinterpret_cast<float2*>(p.pbc) +
                ((cpb == 16 ? row0 - wave * kLaneChannels : row0) / cpb) * L * HS;

  struct In {
    float dl, xin;
    TU u, z, go, o;
    RawRun<TB, 8> bc;
  };
  auto load = [&](int k, In& in) {
    const int64_t t0 = static_cast<int64_t>(k) * HS;
    in.dl = (static_cast<const float*>(p.delta) + t0)[eoff];
    in.u = (static_cast<const TU*>(p.u) + t0)[eoff];
    in.z = (zsrc + t0)[eoff];
    in.go = (static_cast<const TU*>(p.dout) + t0)[eoff];
    in.o = (osrc + t0)[eoff];
    in.xin = __builtin_nontemporal_load(p.states + k * sstep + soff);  // whole lines, read once
    in.bc.load(g, bcsrc + t0, 0, bcoff, 8);
  };
  const int nblk = static_cast<int>(L / HS);
  In cur;
  load(nblk - 1, cur);
  float carry = 0.0f;  // a_{t+1} h_{t+1} entering the block's last step from the right
  float dA0 = 0.0f, dA1 = 0.0f, dD_acc = 0.0f, db_acc = 0.0f;  // dA in two chains (even, odd steps)
  const float act = active ? 1.0f : 0.0f;

  for (int k = nblk - 1; k >= 0; --k) {
    const int64_t t0 = static_cast<int64_t>(k) * HS;
    // ---- this lane's element: step t0 + n of channel c
    const float uu = to_f32(cur.u);
    const float del = step_of(g, cur.dl, bias);
    const float du = del * uu;
    float gy = to_f32(cur.go) * act;
    float dzf = 0.0f, ypre = 0.0f;
    bool need_y = false;
    if (has_z) {
      const float zz = to_f32(cur.z);
      const float sg = sigmoid(zz);
      const float gate = zz * sg;
      dzf = gy * sg * (1.0f + zz * (1.0f - sg));
      if (has_out && gate != 0.0f) ypre = to_f32(cur.o) * fast_rcp(gate);
      else need_y = true;
      gy *= gate;
    }
    const bool ty = __ballot(need_y) != 0;  // wave-uniform: transpose C x in this block
    const float x0 = sn ? cur.xin : 0.0f;
    {
      float sv[8];
      cur.bc.get(sv);
      if (!sok) {  // a padded state adds nothing
#pragma unroll
        for (int i = 0; i < 8; ++i) sv[i] = 0.0f;
      }
      reinterpret_cast<float4*>(stg)[0] = make_float4(sv[0], sv[1], sv[2], sv[3]);
      reinterpret_cast<float4*>(stg)[1] = make_float4(sv[4], sv[5], sv[6], sv[7]);
    }
    load(k > 0 ? k - 1 : 0, cur);  // the next block's inputs: a block of work to arrive
    wave_lds_sync();
    float bv[HS], cv[HS];
    lds_row<HS>(brow, bv);
    lds_row<HS>(crow, cv);
    // ---- recompute the block's states from the saved one
    float xh[HS], ah[HS];
    auto recompute = [&](auto with_y) {
      float x = x0;
      static_for<0, HS>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        ah[i] = fast_exp2(row_bcast<i>(del) * a2);
        x = fmaf(ah[i], x, row_bcast<i>(du) * bv[i]);
        xh[i] = x;
        if constexpr (decltype(with_y)::value) tr[i * kTrPitch + 2 * tw] = cv[i] * x;
      });
    };
    if (ty) {
      // blocks with a zero gate somewhere: the pre-gate output from the sum of C x
      recompute(std::true_type{});
      wave_lds_sync();
      float v3[2 * HS], c4[4];
      lds_row<2 * HS>(tr + n * kTrPitch + 2 * cl * HS, v3);
#pragma unroll
      for (int m = 0; m < 4; ++m) c4[m] = v3[2 * m];
#pragma unroll
      for (int m = 4; m < HS; ++m) c4[m & 3] += v3[2 * m];
      if (need_y) ypre = fmaf(Dd, uu, (c4[0] + c4[1]) + (c4[2] + c4[3]));
      wave_lds_sync();
    } else {
      recompute(std::false_type{});
    }
    // ---- reverse walk
    float sbc[HS / 2];  // dB/dC of step pairs summed over the wavefront's 4 channels (see below)
    float rodd = 0.0f;  // the odd step's half-summed register, waiting for its even partner
    static_for<0, HS>([&](auto jc) {
      constexpr int i = HS - 1 - decltype(jc)::value;
      const float h = fmac_row<i, i == HS - 1>(carry, gy, cv[i]);
      const float hc = ah[i] * h;
      const float pr = hc * (i > 0 ? xh[i > 0 ? i - 1 : 0] : x0);
      *reinterpret_cast<float2*>(tr + i * kTrPitch + 2 * tw) = make_float2(h * bv[i], an * pr);
      if constexpr (i % 2 == 0) dA0 = fmac_row<i>(dA0, del, pr);
      else dA1 = fmac_row<i>(dA1, del, pr);
      // dB and dC terms of step i, h du_i and gy_i x_i: rows c0 + c2 and c1 + c3 of each
      // (a swap of the wavefront's halves), dB in rows 0-1 and dC in rows 2-3 ...
      const float pb = row_bcast<i>(du) * h, pc = row_bcast<i>(gy) * xh[i];
      const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(pb), __float_as_uint(pc), false, false);
      const float rr = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
      if constexpr (i % 2 == 1) {
        rodd = rr;
      } else {
        // ... and with the odd step's register, a swap of odd and even rows completes the
        // channel sums: rows dB_i, dB_{i+1}, dC_i, dC_{i+1}, each over the 16 states
        const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(rr), __float_as_uint(rodd), false, false);
        sbc[i / 2] = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
      }
      carry = hc;
    });
    wave_lds_sync();
    // ---- lane (c, n) owns step t0 + n: its row of the transpose
    float s1, s2;
    {
      float v[2 * HS];
      lds_row<2 * HS>(tr + n * kTrPitch + 2 * cl * HS, v);
      float a[4], b[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        a[m] = v[2 * m];
        b[m] = v[2 * m + 1];
      }
#pragma unroll
      for (int m = 4; m < HS; ++m) {
        a[m & 3] += v[2 * m];
        b[m & 3] += v[2 * m + 1];
      }
      s1 = (a[0] + a[1]) + (a[2] + a[3]);
      s2 = (b[0] + b[1]) + (b[2] + b[3]);
    }
    const float duo = fmaf(del, s1, Dd * gy);
    float dd = fmaf(uu, s1, s2);
    if (g.softplus) dd *= softplus_grad_from_value(del);
    dD_acc = fmaf(gy, uu, dD_acc);
    db_acc = fmaf(dd, act, db_acc);
    if (active) {
      (static_cast<TU*>(p.du) + t0)[eoff] = from_f32<TU>(duo);
      (static_cast<float*>(p.ddelta) + t0)[eoff] = dd;
      if (has_z && p.dz) (static_cast<TU*>(p.dz) + t0)[eoff] = from_f32<TU>(dzf * ypre);
    }
    // ---- dB/dC of the block: register m of lane (row q, state n) holds dB (q < 2) or dC (q >= 2)
    // of step 2m + (q mod 2)
    wave_lds_sync();  // every read of the transposes is done before they take the dB/dC block
    const int which = cl >> 1, par = cl & 1;
    if (cpb == 16) {
#pragma unroll
      for (int m = 0; m < HS / 2; ++m) tr[which * HS * HS + (2 * m + par) * HS + n] = sbc[m];
      __syncthreads();
      // thread (i, s) adds the 4 wavefronts' (step i, state s) in order
      const int o = threadIdx.x;
      float sb = 0.0f, sc = 0.0f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        sb += lds[w][o];
        sc += lds[w][HS * HS + o];
      }
      {
        // whole 2 KB runs that only reduce_bc reads back: written with the nontemporal hint
        // (the per-lane element streams above keep plain accesses: a wavefront covers half a
        // line of each per block, and the next block uses the other half)
        const mko_u32x2 w = {__float_as_uint(sb), __float_as_uint(sc)};
        __builtin_nontemporal_store(w, reinterpret_cast<mko_u32x2*>(pbc + t0 * HS) + o);
      }
      __syncthreads();
    } else if (active) {
      float* pf = reinterpret_cast<float*>(pbc + t0 * HS) + which;
#pragma unroll
      for (int m = 0; m < HS / 2; ++m) pf[((2 * m + par) * HS + n) * 2] = sbc[m];
    }
  }
  if (active && sn) p.dap[static_cast<int64_t>(n) * g.rows + row0 + cl] = dA0 + dA1;
  dD_acc = row16_sum(dD_acc);
  db_acc = row16_sum(db_acc);
  if (active && n == 0) {
    p.ddp[row0 + cl] = dD_acc;
    p.dbp[row0 + cl] = db_acc;
  }
}

// ---------------------------------------------------------------- backward

template <int NS, bool UNI, class TU>
__global__ void __launch_bounds__(256) bwd_summary(Geo g, Ptrs p) {
  const LaneInfo li = lane_info(g, UNI);
  const int N = static_cast<int>(g.dstate);
  const int c = blockIdx.y + 1;  // chunk 0's adjoint summary is never needed
  const int t_begin = c * g.lc;
  const int t_end = min(t_begin + g.lc, static_cast<int>(g.length));
  float A2[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) A2[n] = n < N ? p.A[li.d * N + n] * kLog2e : 0.0f;
  const float bias = p.bias ? p.bias[li.d] : 0.0f;
  const bool has_z = p.z != nullptr;
  float hc[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) hc[n] = 0.0f;
  float sd = 0.0f;
  const int64_t rbase = li.row * g.length;
  const int64_t row0 = li.bg * g.length;
  const int nblk = (t_end - t_begin + HS - 1) / HS;
  const void* zsrc = has_z ? p.z : p.dout;  // without z the third run repeats dout (unused)
  RawRun<DeltaT<TU>> rd;
  RawRun<TU> rg, rz;
  {
    const int t0 = t_begin + (nblk - 1) * HS, nv = min(HS, t_end - t0);
    rd.load(g, p.delta, g.d_dtype, rbase + t0, nv);
    rg.load(g, p.dout, g.u_dtype, rbase + t0, nv);
    rz.load(g, zsrc, g.u_dtype, rbase + t0, nv);
  }
  constexpr bool kLds = UNI && !__is_same(TU, Dyn);
  __shared__ float sbc[kLds ? 4 * 2 * HS * NS : 1];  // per wavefront: two buffers of [HS][NS] C rows
  float* wc = sbc + (kLds ? (threadIdx.x >> 6) * 2 * HS * NS : 0);
  WaveBC<NS, false, true> st;
  if constexpr (kLds) {
    st.fetch(nullptr, p.ct, (row0 + t_begin + (nblk - 1) * HS) * NS);
    st.put(nullptr, wc);
    wave_lds_sync();
  }
  int cur = 0;
  for (int blk = nblk - 1; blk >= 0; --blk) {
    const int t0 = t_begin + blk * HS;
    const int nv = min(HS, t_end - t0);
    float del[HS], gy[HS], zz[HS];
    rd.get(del);
    rg.get(gy);
    rz.get(zz);
    {
      const int tp = t_begin + (blk > 0 ? blk - 1 : 0) * HS, np = min(HS, t_end - tp);  // previous block
      rd.load(g, p.delta, g.d_dtype, rbase + tp, np);
      rg.load(g, p.dout, g.u_dtype, rbase + tp, np);
      rz.load(g, zsrc, g.u_dtype, rbase + tp, np);
    }
    if (has_z) {
#pragma unroll
      for (int i = 0; i < HS; ++i) gy[i] *= zz[i] * sigmoid(zz[i]);
    }
#pragma unroll
    for (int i = 0; i < HS; ++i) {
      del[i] = i < nv ? step_of(g, del[i], bias) : 0.0f;
      sd += del[i];
    }
    if constexpr (kLds) {
      st.fetch(nullptr, p.ct, (row0 + t_begin + (blk > 0 ? blk - 1 : 0) * HS) * NS);
      const float* sc = wc + cur * HS * NS;
#pragma unroll
      for (int i = HS - 1; i >= 0; --i) {
        float cv[NS];
        lds_row<NS>(sc + i * NS, cv);
        const float d = del[i], gv = gy[i];
#pragma unroll
        for (int n = 0; n < NS; ++n) hc[n] = fast_exp2(A2[n] * d) * fmaf(gv, cv[n], hc[n]);
      }
      cur ^= 1;
      st.put(nullptr, wc + cur * HS * NS);
      wave_lds_sync();
      continue;
    }
    StepBC<NS, UNI, false, true> e0, e1;
    e0.load(nullptr, p.ct, (row0 + t0 + nv - 1) * NS);
    for (int i = nv - 1; i >= 0; i -= 2) {
      const bool two = i > 0;
      wait_lgkm();
      if (two) e1.load(nullptr, p.ct, (row0 + t0 + i - 1) * NS);
      {
        const float d = del[i], gv = gy[i];
#pragma unroll
        for (int n = 0; n < NS; ++n) hc[n] = fast_exp2(A2[n] * d) * fmaf(gv, e0.c[n], hc[n]);
      }
      if (two) {
        wait_lgkm();
        if (i > 1) e0.load(nullptr, p.ct, (row0 + t0 + i - 2) * NS);
        const float d = del[i - 1], gv = gy[i - 1];
#pragma unroll
        for (int n = 0; n < NS; ++n) hc[n] = fast_exp2(A2[n] * d) * fmaf(gv, e1.c[n], hc[n]);
      }
    }
  }
  if (li.active) {
    const int64_t o = (li.row * g.nchunks + c) * N;
#pragma unroll
    for (int n = 0; n < NS; ++n)
      if (n < N) p.drive[o + n] = hc[n];
    p.sumd[li.row * g.nchunks + c] = sd;
  }
}

// bwd_main LDS (floats): per wavefront a transposition buffer [64][2*HS+1] and
// its dB/dC half-column sums [NS][64]; per workgroup the block's B and C rows
// [2][NS][HS] when the workgroup shares (batch, group).
constexpr int kTransPitch = 2 * HS + 1;

template <int NS>
struct MainLds {
  static constexpr int kWaveFloats = kWave * kTransPitch + NS * kWave;
  static constexpr int kRows = 2 * NS * HS;
};

// One state's B and C over the HS steps of a block (state-major rows).
template <bool UNI>
__device__ __forceinline__ void load_state_rows(const float* __restrict__ bn, const float* __restrict__ cn,
                                                int64_t off, float (&bv)[HS], float (&cv)[HS]) {
  if (UNI) {
    const cfptr pb = as_const(bn + off);
    const cfptr pc = as_const(cn + off);
#pragma unroll
    for (int i = 0; i < HS; ++i) {
      bv[i] = pb[i];
      cv[i] = pc[i];
    }
  } else {
    const float4* qb = reinterpret_cast<const float4*>(bn + off);
    const float4* qc = reinterpret_cast<const float4*>(cn + off);
#pragma unroll
    for (int v = 0; v < HS / 4; ++v) {
      const float4 wb = qb[v], wc = qc[v];
      bv[4 * v] = wb.x; bv[4 * v + 1] = wb.y; bv[4 * v + 2] = wb.z; bv[4 * v + 3] = wb.w;
      cv[4 * v] = wc.x; cv[4 * v + 1] = wc.y; cv[4 * v + 2] = wc.z; cv[4 * v + 3] = wc.w;
    }
  }
}

// FULL: dstate == NS, so the per-state loop has no run-time guards.
template <int NS, bool UNI, bool FULL>
__global__ void __launch_bounds__(256) bwd_main(Geo g, Ptrs p) {
  __shared__ float lds[4 * MainLds<NS>::kWaveFloats + MainLds<NS>::kRows];
  // per wavefront, the block's dz factor dy sigma(z) (1 + z (1 - sigma(z))) per step and
  // lane, computed from the block's first loads so the gradients need no second read
  __shared__ float dzs[4][HS * kWave];
  // and u's raw 16-bit values when u is 16-bit (fp32 u is read again)
  __shared__ uint16_t us16[4][HS * kWave];
  const bool u16 = g.u_dtype != MKO_F32;
  // non-uniform mode: per wavefront, the first lane and the (batch, group) of each run
  // of lanes that share a group (segment s covers lanes seg_first[s] .. seg_first[s+1])
  __shared__ int seg_first[UNI ? 1 : 4][kWave + 1], seg_bg[UNI ? 1 : 4][kWave];
  const LaneInfo li = lane_info(g, UNI);
  const int N = static_cast<int>(g.dstate);
  const int lane = threadIdx.x & 63;
  const int wave = uniform(static_cast<int>(threadIdx.x >> 6));
  int nseg = 0;
  if constexpr (!UNI) {
    const int bgi = static_cast<int>(li.bg);
    const int prev = __shfl_up(bgi, 1);
    const bool first = lane == 0 || prev != bgi;
    const unsigned long long mask = __ballot(first);
    nseg = __popcll(mask);
    if (first) {
      const int sidx = __popcll(mask & ((1ull << lane) - 1ull));
      seg_first[wave][sidx] = lane;
      seg_bg[wave][sidx] = bgi;
    }
    if (lane == 0) seg_first[wave][nseg] = kWave;
    wave_lds_sync();
  }
  float* trans = lds + wave * kWave * kTransPitch;                // [64][kTransPitch]
  float* acc_all = lds + 4 * kWave * kTransPitch;                 // [wave][NS][64]
  float* acc = acc_all + wave * NS * kWave;
  float* rows_b = lds + 4 * MainLds<NS>::kWaveFloats;  // [NS][HS]
  float* rows_c = rows_b + NS * HS;                    // [NS][HS]

  const int c = blockIdx.y;
  const int t_begin = c * g.lc;
  const int t_end = min(t_begin + g.lc, static_cast<int>(g.length));
  const float bias = p.bias ? p.bias[li.d] : 0.0f;
  const float Dd = p.D ? p.D[li.d] : 0.0f;
  const bool has_z = p.z != nullptr;
  const int64_t rbase = li.row * g.length;
  const float* arow = p.A + li.d * N;
  const float act = li.active ? 1.0f : 0.0f;
  const int64_t R = g.rows;
  // dA partials per (chunk, state, row), state-major so a wavefront's 64 lanes
  // touch 256 contiguous bytes.
  float* dap = p.dap + static_cast<int64_t>(c) * NS * R;

  // adjoint carried between blocks and the dA sums, one per state, in registers
  float hcr[NS], dar[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    hcr[n] = n < N ? p.adj[(li.row * g.nchunks + c) * N + n] : 0.0f;
    dar[n] = 0.0f;
  }

  int64_t cb = 0;
  if (UNI) {
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * g.wpg * kWave;
    cb = ((r0 % g.dim) % g.dg) / (static_cast<int64_t>(g.wpg) * kWave);
  }
  float A2[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) A2[n] = n < N ? arow[n] * kLog2e : 0.0f;
  float dD_acc = 0.0f, db_acc = 0.0f;
  const int64_t brow0 = li.bg * g.length;

  static_assert(CK == HS, "one saved state per 16-step block");
  const int jb = t_begin / CK;
  const int je = (t_end + CK - 1) / CK;
  // blocks in reverse, states one at a time
  for (int j = je - 1; j >= jb; --j) {
    const int qs = j * CK;
    // saved state entering block j, element n at srow[n]
    const float* srow = p.states + ck_index(g, li.row, j, 0);
    {
      const int nv = min(HS, t_end - qs);
      float del[HS], du[HS], gy[HS];
      {
        float uu[HS];
        load_run<HS>(p.delta, g.d_dtype, rbase + qs, nv, g.vec, del);
        load_run<HS>(p.u, g.u_dtype, rbase + qs, nv, g.vec, uu);
        if (u16) {
          // exact: the floats came from 16-bit values
#pragma unroll
          for (int i = 0; i < HS; ++i)
            us16[wave][i * kWave + lane] = g.u_dtype == MKO_BF16 ? __builtin_bit_cast(uint16_t, from_f32<bf16>(uu[i]))
                                                                 : __builtin_bit_cast(uint16_t, from_f32<_Float16>(uu[i]));
        }
        load_run<HS>(p.dout, g.u_dtype, rbase + qs, nv, g.vec, gy);
        if (has_z) {
          float zz[HS];
          load_run<HS>(p.z, g.u_dtype, rbase + qs, nv, g.vec, zz);
#pragma unroll
          for (int i = 0; i < HS; ++i) {
            const float sg = sigmoid(zz[i]);
            dzs[wave][i * kWave + lane] = gy[i] * sg * (1.0f + zz[i] * (1.0f - sg));  // gy is dy here
            gy[i] *= zz[i] * sg;
          }
        }
#pragma unroll
        for (int i = 0; i < HS; ++i) {
          del[i] = i < nv ? step_of(g, del[i], bias) : 0.0f;
          du[i] = del[i] * uu[i] * act;
          gy[i] *= act;
        }
      }
      float s1[HS], s2[HS], ya[HS];
#pragma unroll
      for (int i = 0; i < HS; ++i) s1[i] = s2[i] = ya[i] = 0.0f;

      if (UNI) {
        // The block's B/C rows, shared by the workgroup (the previous block's
        // flush barrier orders this write after every read of the old rows).
        for (int e = threadIdx.x; e < NS * HS; e += blockDim.x) {
          const int n = e / HS, i = e % HS;
          const int64_t src = (li.bg * NS + n) * g.length + qs + i;
          rows_b[e] = p.bn[src];
          rows_c[e] = p.cn[src];
        }
        __syncthreads();
      }
      const float* xin_p = srow;
      const int xin_stride = 1;
      const float* bn_p = p.bn + (li.bg * NS) * g.length + qs;
      const float* cn_p = p.cn + (li.bg * NS) * g.length + qs;
      float xin_n = xin_p[0];
#pragma unroll
      for (int n = 0; n < NS; ++n) {
        if (!FULL && n >= N) break;
        const bool more = n + 1 < (FULL ? NS : N);
        float xin_x = 0.0f;
        if (more) xin_x = xin_p[(n + 1) * xin_stride];
        float bv[HS], cv[HS];
        if (UNI) {
#pragma unroll
          for (int i = 0; i < HS; ++i) {
            bv[i] = rows_b[n * HS + i];
            cv[i] = rows_c[n * HS + i];
          }
        } else {
          load_run_t<float, HS>(bn_p + n * static_cast<int64_t>(g.length), HS, (g.length % 4) == 0, bv);
          load_run_t<float, HS>(cn_p + n * static_cast<int64_t>(g.length), HS, (g.length % 4) == 0, cv);
        }
        const float an = arow[n];
        const float a2 = an * kLog2e;
        float xh[HS], ah[HS];
        float x = xin_n;
#pragma unroll
        for (int i = 0; i < HS; ++i) {
          ah[i] = fast_exp2(a2 * del[i]);
          x = fmaf(ah[i], x, du[i] * bv[i]);
          xh[i] = x;
        }
        float hc = hcr[n];
        float dan = 0.0f;
#pragma unroll
        for (int i = HS - 1; i >= 0; --i) {
          const float h = fmaf(gy[i], cv[i], hc);
          s1[i] = fmaf(h, bv[i], s1[i]);
          const float xp = i > 0 ? xh[i - 1] : xin_n;
          const float pr = h * ah[i] * xp;
          s2[i] = fmaf(an, pr, s2[i]);
          dan = fmaf(del[i], pr, dan);
          ya[i] = fmaf(cv[i], xh[i], ya[i]);
          trans[lane * kTransPitch + i] = h * du[i];
          trans[lane * kTransPitch + HS + i] = gy[i] * xh[i];
          hc = ah[i] * h;
        }
        hcr[n] = hc;
        dar[n] += dan;
        wave_lds_sync();
        if (UNI) {
          // lane l sums column (l mod 32) over one half of the 64 rows; the
          // halves and the wavefronts are added in a fixed order at the flush.
          const int col = lane & (2 * HS - 1);
          const int r0 = (lane >> 5) * 32;
          float sum = 0.0f;
#pragma unroll 8
          for (int r = 0; r < 32; ++r) sum += trans[(r0 + r) * kTransPitch + col];
          acc[n * kWave + lane] = sum;
        } else {
          // One sum per (segment, column) over the segment's rows, stored in the partial
          // slot of its (batch, group) that belongs to this wavefront: slot k of group bg
          // is the k-th wavefront its rows [bg dg, (bg + 1) dg) meet, so every slot has one
          // writer and reduce_bc adds them in slot order.  Inactive lanes hold zeros (act =
          // 0) and sit in the last row's segment; a wavefront past the last row writes
          // nothing (its clamped rows would name a slot beyond its group's).
          const bool live = li.wave_row * kWave < g.rows;  // wave-uniform
          for (int w = lane; live && w < nseg * 2 * HS; w += kWave) {
            const int sidx = w / (2 * HS), col = w % (2 * HS);
            const int i = col % HS, k = col / HS;
            if (i >= nv) continue;
            float sum = 0.0f;
            for (int r = seg_first[wave][sidx]; r < seg_first[wave][sidx + 1]; ++r)
              sum += trans[r * kTransPitch + col];
            const int64_t bgs = seg_bg[wave][sidx];
            const int64_t slot = bgs * g.ncb + (li.wave_row - bgs * g.dg / kWave);
            p.pbc[((slot * g.length + qs + i) * NS + n) * 2 + k] = sum;
          }
        }
        wave_lds_sync();
        if (more) xin_n = xin_x;
      }
      // ---- per-step gradients of the block
      {
        float uu[HS], o1[HS], o2[HS];
        if (u16) {
#pragma unroll
          for (int i = 0; i < HS; ++i) {
            const uint16_t v = us16[wave][i * kWave + lane];
            uu[i] = g.u_dtype == MKO_BF16 ? to_f32(__builtin_bit_cast(bf16, v)) : to_f32(__builtin_bit_cast(_Float16, v));
          }
        } else {
          load_run<HS>(p.u, g.u_dtype, rbase + qs, nv, g.vec, uu);
        }
#pragma unroll
        for (int i = 0; i < HS; ++i) {
          o1[i] = fmaf(del[i], s1[i], Dd * gy[i]);  // du
          float dd = fmaf(uu[i], s1[i], s2[i]);      // d loss / d step
          if (g.softplus) dd *= softplus_grad_from_value(del[i]);
          o2[i] = dd;
          if (i < nv) {
            dD_acc = fmaf(gy[i], uu[i], dD_acc);
            db_acc += dd * act;
          }
        }
        if (li.active) {
          store_run<HS>(p.du, g.u_dtype, rbase + qs, nv, g.vec, o1);
          store_run<HS>(p.ddelta, g.d_dtype, rbase + qs, nv, g.vec, o2);
        }
        if (has_z && p.dz) {
#pragma unroll
          for (int i = 0; i < HS; ++i) o1[i] = dzs[wave][i * kWave + lane] * fmaf(Dd, uu[i], ya[i]);
          if (li.active) store_run<HS>(p.dz, g.u_dtype, rbase + qs, nv, g.vec, o1);
        }
      }
      if (UNI) {
        // The workgroup's dB/dC sums of this block, column k*HS + i of state n:
        // wavefronts in order, each as (first half of rows) + (second half).
        __syncthreads();
        float* dst = p.pbc + ((li.bg * g.ncb + cb) * g.length + qs) * NS * 2;
        for (int e = threadIdx.x; e < N * 2 * HS; e += blockDim.x) {
          const int col = e % (2 * HS);
          const int n = e / (2 * HS);
          const int i = col % HS;
          const int k = col / HS;
          float sum = 0.0f;
          for (int w = 0; w < g.wpg; ++w) {
            const float* aw = acc_all + (w * NS + n) * kWave;
            sum += aw[col] + aw[col + 2 * HS];
          }
          if (i < nv) dst[(static_cast<int64_t>(i) * NS + n) * 2 + k] = sum;
        }
        __syncthreads();
      }
    }
  }
  if (li.active) {
#pragma unroll
    for (int n = 0; n < NS; ++n)
      if (n < N) dap[n * R + li.row] = dar[n];
    p.ddp[static_cast<int64_t>(c) * g.rows + li.row] = dD_acc;
    p.dbp[static_cast<int64_t>(c) * g.rows + li.row] = db_acc;
  }
}

// dB/dC (bg, N, L) = sum over channel blocks of the partials (bg, ncb, L, NS, 2).
// A workgroup covers 256/NS steps x NS states: it reads the partials contiguously
// (state fastest) and writes through an LDS transpose so the stores run along L.
// seg_dg != 0 (groups of seg_dg channels, not a multiple of 64 wide): group bg has one
// partial per wavefront its rows meet, of the ncb slots laid out for each group.
template <int NS>
__global__ void __launch_bounds__(256) reduce_bc(Geo g, int ncb, int64_t seg_dg, const float* __restrict__ pbc,
                                                 void* dB, void* dC) {
  constexpr int TT = 256 / NS;
  __shared__ float sb[NS][TT + 1], sc[NS][TT + 1];
  const int64_t nt = (g.length + TT - 1) / TT;
  const int64_t bg = blockIdx.x / nt;
  const int nsum = seg_dg ? static_cast<int>(((bg + 1) * seg_dg - 1) / kWave - bg * seg_dg / kWave + 1) : ncb;
  const int64_t t0 = (blockIdx.x % nt) * TT;
  const int tid = threadIdx.x;
  {
    const int tl = tid / NS, n = tid % NS;
    const int64_t t = t0 + tl;
    float vb = 0.0f, vc = 0.0f;
    if (t < g.length) {
      // channel blocks in order: whole batches of sixteen issue their loads together, the
      // rest one at a time; the partials are read once, with the nontemporal hint (eight at a
      // time without it: 0.135 ms at c3; sixteen with it: 0.107 ms, thirty-two the same)
      constexpr int PF = 16;
      const float* src = pbc + ((bg * ncb * g.length + t) * NS + n) * 2;
      const int64_t stride = g.length * NS * 2;  // floats between channel blocks
      int cbk = 0;
      for (; cbk + PF <= nsum; cbk += PF) {
        uint32_t q[PF][2];
#pragma unroll
        for (int j = 0; j < PF; ++j) load_words_nt(src + (cbk + j) * stride, q[j]);
#pragma unroll
        for (int j = 0; j < PF; ++j) {
          vb += __uint_as_float(q[j][0]);
          vc += __uint_as_float(q[j][1]);
        }
      }
      for (; cbk < nsum; ++cbk) {
        uint32_t q[2];
        load_words_nt(src + cbk * stride, q);
        vb += __uint_as_float(q[0]);
        vc += __uint_as_float(q[1]);
      }
    }
    sb[n][tl] = vb;
    sc[n][tl] = vc;
  }
  __syncthreads();
  const int n = tid / TT, tl = tid % TT;
  const int64_t t = t0 + tl;
  if (n < g.dstate && t < g.length) {
    const int64_t o = (bg * g.dstate + n) * g.length + t;
    if (dB) store_one(dB, g.bc_dtype, o, sb[n][tl]);
    if (dC) store_one(dC, g.bc_dtype, o, sc[n][tl]);
  }
}

// Partials grp, grp + 4, ... of one channel (partial k = chunk k / nb, batch k % nb, at
// k / nb * cstride + k % nb * dim), added in that order. Whole batches of eight issue
// their loads together and the rest go one at a time; the bounds are wave-uniform. TWO:
// p1 is summed into s1 alongside.
template <bool TWO>
__device__ __forceinline__ void sum_partials(const Geo& g, int grp, int npart, int nb, int64_t cstride,
                                             const float* __restrict__ p0, const float* __restrict__ p1,
                                             float& s0, float& s1) {
  constexpr int PF = 8;
  auto at = [&](int k) { return (k / nb) * cstride + (k % nb) * g.dim; };
  int k = grp;
  for (; k + 4 * (PF - 1) < npart; k += 4 * PF) {
    float v0[PF], v1[PF];
#pragma unroll
    for (int q = 0; q < PF; ++q) {
      const int64_t o = at(k + 4 * q);
      v0[q] = p0[o];
      if constexpr (TWO) v1[q] = p1[o];
    }
#pragma unroll
    for (int q = 0; q < PF; ++q) {
      s0 += v0[q];
      if constexpr (TWO) s1 += v1[q];
    }
  }
  for (; k < npart; k += 4) {
    const int64_t o = at(k);
    s0 += p0[o];
    if constexpr (TWO) s1 += p1[o];
  }
}

// dA (dim, N) = sum over (chunk, batch) of partials; dD, ddelta_bias likewise.
// A workgroup covers 64 channels of one output row (a state n, or the dD / dbias
// row when n == N): 4 groups of 64 threads split the (chunk, batch) partials, read
// channel-fastest, and are added in a fixed order.
__global__ void __launch_bounds__(256) reduce_params(Geo g, int ns, const float* __restrict__ dap,
                                                     const float* __restrict__ ddp,
                                                     const float* __restrict__ dbp, float* dA,
                                                     float* dD, float* dbias) {
  __shared__ float part[2][4][64];
  const int N = static_cast<int>(g.dstate);
  const int64_t dblocks = (g.dim + 63) / 64;
  const int n = static_cast<int>(blockIdx.x / dblocks);  // 0..N (N: the dD / dbias row)
  const int64_t d = (blockIdx.x % dblocks) * 64 + (threadIdx.x & 63);
  const int grp = threadIdx.x >> 6;
  const int npart = g.nchunks * static_cast<int>(g.batch);
  const int nb = static_cast<int>(g.batch);
  float s0 = 0.0f, s1 = 0.0f;
  if (d < g.dim) {
    const int64_t cstride = static_cast<int64_t>(n < N ? ns : 1) * g.rows;  // between chunks
    if (n < N)
      sum_partials<false>(g, grp, npart, nb, cstride, dap + n * g.rows + d, nullptr, s0, s1);
    else
      sum_partials<true>(g, grp, npart, nb, cstride, ddp + d, dbp + d, s0, s1);
  }
  part[0][grp][threadIdx.x & 63] = s0;
  part[1][grp][threadIdx.x & 63] = s1;
  __syncthreads();
  if (threadIdx.x < 64 && d < g.dim) {
    const int l = threadIdx.x;
    const float t0 = (part[0][0][l] + part[0][1][l]) + (part[0][2][l] + part[0][3][l]);
    const float t1 = (part[1][0][l] + part[1][1][l]) + (part[1][2][l] + part[1][3][l]);
    if (n < N) {
      if (dA) dA[d * N + n] = t0;
    } else {
      if (dD) dD[d] = t0;
      if (dbias) dbias[d] = t1;
    }
  }
}

// ---------------------------------------------------------------- host plan

struct Plan {
  Geo g;
  int ns;
  bool uni;
  bool lane;  // forward through fwd_lane (set per call from pointer alignment and shape)
  bool lane_bwd;  // backward through bwd_lane (likewise)
  size_t off_bt, off_ct, off_bn, off_cn, off_drive, off_sumd, off_adj, off_pbc, off_dap, off_ddp,
      off_dbp;
  // bwd_lane's workspace: dB/dC partials per cpb channels, dA / dD / ddelta_bias partials per row
  int cpb;
  int64_t lncb;
  size_t loff_pbc, loff_dap, loff_ddp, loff_dbp;
  size_t fwd_bytes, bwd_bytes;
};

inline size_t align_up(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Rows from which the lane-per-state kernels have enough wavefronts (rows / 4 of them) to fill
// the chip without time chunks.
constexpr int64_t kLaneRows = 6144;

// Shapes the lane-per-state forward takes (dtypes and alignment are checked per call).
static bool lane_shape(const Geo& g, int ns) {
  return ns == 16 && g.rows >= kLaneRows && g.length % HS == 0 && g.dg % kLaneChannels == 0;
}

// The backward's too.  It indexes the per-row arrays (u, delta, z, dout, out, du, ddelta, dz,
// the saved states) and B/C with 32-bit lane offsets from a 64-bit base, so each of them must
// hold fewer than 2^31 elements: rows x length for the rows, and batch x groups x 16 states x
// length for B and C (four times the rows' count when a group is 4 channels wide).
static bool lane_bwd_shape(const Geo& g, int ns) {
  constexpr int64_t kLimit = static_cast<int64_t>(1) << 31;
  return lane_shape(g, ns) && g.rows * g.length < kLimit && g.batch * g.ngroups * HS * g.length < kLimit;
}

static int make_plan(const mko_selscan_params* p, Plan* pl) {
  if (!p) {
    mko_set_error("selscan: null params");
    return MKO_EINVAL;
  }
  Geo& g = pl->g;
  g.batch = p->batch;
  g.dim = p->dim;
  g.length = p->length;
  g.dstate = p->dstate;
  g.ngroups = p->ngroups;
  if (g.batch < 0 || g.dim < 0 || g.length < 0 || g.dstate < 1 || g.ngroups < 1) {
    mko_set_error("selscan: bad sizes batch=%lld dim=%lld length=%lld dstate=%lld ngroups=%lld",
                  (long long)g.batch, (long long)g.dim, (long long)g.length, (long long)g.dstate,
                  (long long)g.ngroups);
    return MKO_EINVAL;
  }
  if (g.dim % g.ngroups) {
    mko_set_error("selscan: dim=%lld not divisible by ngroups=%lld", (long long)g.dim, (long long)g.ngroups);
    return MKO_EINVAL;
  }
  if (g.dstate > 32) {
    mko_set_error("selscan: dstate=%lld > 32 is not supported", (long long)g.dstate);
    return MKO_EUNSUPPORTED;
  }
  if (g.length > (int64_t)1 << 30 || g.batch * g.dim > (int64_t)1 << 31) {
    mko_set_error("selscan: problem too large");
    return MKO_EUNSUPPORTED;
  }
  for (int dt : {p->u_dtype, p->delta_dtype, p->bc_dtype}) {
    if (dt != MKO_F32 && dt != MKO_F16 && dt != MKO_BF16) {
      mko_set_error("selscan: unknown dtype %d", dt);
      return MKO_EINVAL;
    }
  }
  pl->ns = g.dstate <= 16 ? 16 : 32;
  g.rows = g.batch * g.dim;
  g.dg = g.dim / g.ngroups;
  g.nwr = (g.rows + kWave - 1) / kWave;
  g.u_dtype = p->u_dtype;
  g.d_dtype = p->delta_dtype;
  g.bc_dtype = p->bc_dtype;
  g.softplus = (p->flags & MKO_SS_SOFTPLUS) ? 1 : 0;
  g.nck = static_cast<int>((g.length + CK - 1) / CK);
  pl->uni = (g.dg % kWave) == 0;
  if (pl->uni) {
    const int64_t blocks = g.dg / kWave;
    g.wpg = blocks % 4 == 0 ? 4 : (blocks % 2 == 0 ? 2 : 1);
    g.ncb = static_cast<int>(g.dg / (static_cast<int64_t>(g.wpg) * kWave));
  } else {
    g.wpg = 4;
    g.ncb = static_cast<int>((g.dg + kWave - 1) / kWave + 1);  // wavefronts a group's rows can meet
  }
  // Coarse chunks: about eight wavefronts per SIMD over the chip's 1024 SIMDs
  // (the state-inner loops hide their scalar-load waits with other waves), the
  // chunk a multiple of the save interval and, while that still leaves about 2048
  // wavefronts, at least 128 steps: shorter chunks cost more in per-chunk summaries
  // and dA partials than their parallelism buys (c2, 8 x 1536 x 2048: 64 chunks of 32
  // steps 1.07 ms, 16 of 128 0.95 ms), but a problem of few channel rows (the 2D scan's
  // 384 rows) needs the short chunks for its wavefronts.
  int64_t want = (8192 + g.nwr - 1) / (g.nwr > 0 ? g.nwr : 1);
  int64_t k = 1;
  while (k < want) k <<= 1;
  int64_t lc = (g.length + k - 1) / k;
  lc = ((lc + CK - 1) / CK) * CK;
  int64_t lmin = 128;
  while (lmin > CK && g.nwr * ((g.length + lmin - 1) / lmin) < 2048) lmin /= 2;
  if (lc < lmin) lc = lmin;
  g.lc = static_cast<int>(lc);
  g.nchunks = static_cast<int>(g.length > 0 ? (g.length + lc - 1) / lc : 0);
  g.vec = 0;
  const size_t ns = static_cast<size_t>(pl->ns);
  const size_t bgl = static_cast<size_t>(g.batch * g.ngroups * g.length);
  const size_t rk = static_cast<size_t>(g.rows) * g.nchunks;
  size_t o = 0;
  // forward workspace
  pl->off_bt = o; o = align_up(o + bgl * ns * 4);
  pl->off_ct = o; o = align_up(o + bgl * ns * 4);
  pl->off_drive = o; o = align_up(o + rk * g.dstate * 4);
  pl->off_sumd = o; o = align_up(o + rk * 4);
  pl->fwd_bytes = o;
  // backward workspace (extends the forward layout: bt/ct are used by both)
  pl->off_bn = o; o = align_up(o + (bgl * ns + HS) * 4);  // + one row tail: blocks read HS steps
  pl->off_cn = o; o = align_up(o + (bgl * ns + HS) * 4);
  pl->off_adj = o; o = align_up(o + rk * g.dstate * 4);
  pl->off_pbc = o; o = align_up(o + bgl * g.ncb * ns * 2 * 4);
  pl->off_dap = o; o = align_up(o + rk * ns * 4);
  pl->off_ddp = o; o = align_up(o + rk * 4);
  pl->off_dbp = o; o = align_up(o + rk * 4);
  pl->bwd_bytes = o;
  // bwd_lane (laid out from offset 0; the workspace is the larger of the two layouts)
  pl->cpb = (g.dg % 16) == 0 ? 16 : 4;
  pl->lncb = g.dg / pl->cpb;
  if (lane_bwd_shape(g, pl->ns)) {
    size_t q = 0;
    pl->loff_pbc = q; q = align_up(q + static_cast<size_t>(g.batch * g.ngroups) * pl->lncb * g.length * 16 * 2 * 4);
    pl->loff_dap = q; q = align_up(q + static_cast<size_t>(g.rows) * 16 * 4);
    pl->loff_ddp = q; q = align_up(q + static_cast<size_t>(g.rows) * 4);
    pl->loff_dbp = q; q = align_up(q + static_cast<size_t>(g.rows) * 4);
    if (q > pl->bwd_bytes) pl->bwd_bytes = q;
  }
  return MKO_OK;
}

static bool rows_vectorisable(const Geo& g, std::initializer_list<std::pair<const void*, int>> arrays) {
  for (auto& a : arrays) {
    if (!a.first) continue;
    const int bytes = dtype_size(a.second);
    if ((g.length * bytes) % 16 != 0) return false;
    if (!aligned16(a.first)) return false;
  }
  return true;
}

static Ptrs make_ptrs(const mko_selscan_params* p, const Plan& pl) {
  Ptrs q{};
  q.u = p->u;
  q.delta = p->delta;
  q.A = p->A;
  q.B = p->B;
  q.C = p->C;
  q.D = p->D;
  q.z = p->z;
  q.bias = p->delta_bias;
  q.dout = p->dout;
  q.out = p->out;
  q.states = p->states;
  q.du = p->du;
  q.ddelta = p->ddelta;
  q.dz = p->dz;
  char* ws = static_cast<char*>(p->workspace);
  q.bt = reinterpret_cast<float*>(ws + pl.off_bt);
  q.ct = reinterpret_cast<float*>(ws + pl.off_ct);
  q.drive = reinterpret_cast<float*>(ws + pl.off_drive);
  q.sumd = reinterpret_cast<float*>(ws + pl.off_sumd);
  q.bn = reinterpret_cast<float*>(ws + pl.off_bn);
  q.cn = reinterpret_cast<float*>(ws + pl.off_cn);
  q.adj = reinterpret_cast<float*>(ws + pl.off_adj);
  q.pbc = reinterpret_cast<float*>(ws + pl.off_pbc);
  q.dap = reinterpret_cast<float*>(ws + pl.off_dap);
  q.ddp = reinterpret_cast<float*>(ws + pl.off_ddp);
  q.dbp = reinterpret_cast<float*>(ws + pl.off_dbp);
  return q;
}

static inline unsigned blocks_for(int64_t n, int per = 256) {
  return static_cast<unsigned>((n + per - 1) / per);
}

// The wavefront-per-pair chain pays off when a thread per (row, state) would walk many
// chunks and fill fewer than 1024 workgroups.
static bool chain_by_wave(const Geo& g) {
  return g.nchunks > 32 && g.rows * g.dstate < 1024 * 256;
}


template <class TU>
static int launch_fwd_lane(const Plan& pl, const Ptrs& q, hipStream_t s) {
  const Geo& g = pl.g;
  const unsigned grid = static_cast<unsigned>((g.rows + 4 * kLaneChannels - 1) / (4 * kLaneChannels));
  if (g.bc_dtype == MKO_BF16)
    MKO_TIMED("selscan_fwd_lane", s, fwd_lane<TU, bf16><<<grid, 256, 0, s>>>(g, q));
  else if (g.bc_dtype == MKO_F16)
    MKO_TIMED("selscan_fwd_lane", s, fwd_lane<TU, _Float16><<<grid, 256, 0, s>>>(g, q));
  else
    MKO_TIMED("selscan_fwd_lane", s, fwd_lane<TU, float><<<grid, 256, 0, s>>>(g, q));
  return mko_check_launch("selscan_fwd");
}

template <int NS, bool UNI, class TU>
static int launch_fwd(const Plan& pl, const Ptrs& q, hipStream_t s) {
  const Geo& g = pl.g;
  if constexpr (NS == 16 && !__is_same(TU, Dyn)) {
    if (pl.lane) return launch_fwd_lane<TU>(pl, q, s);
  }
  const dim3 block(g.wpg * kWave);
  const unsigned gx = static_cast<unsigned>((g.nwr + g.wpg - 1) / g.wpg);
  const int64_t ntiles = (g.length + kPrepSteps - 1) / kPrepSteps;
  const unsigned gprep = static_cast<unsigned>(g.batch * g.ngroups * ntiles);
  MKO_TIMED("selscan_prep", s,
            prep_layouts<NS><<<gprep, 256, 0, s>>>(g, ntiles, q.B, q.C, q.bt, q.ct, nullptr, nullptr));
  if (g.nchunks > 1) {
    MKO_TIMED("selscan_fwd_summary", s, fwd_summary<NS, UNI, TU><<<dim3(gx, g.nchunks - 1), block, 0, s>>>(g, q));
  }
  if (chain_by_wave(g))
    MKO_TIMED("selscan_chain", s,
              chain_wave<false><<<blocks_for(g.rows * g.dstate, 4), 256, 0, s>>>(g, q.A, q.drive, q.sumd, q.states));
  else
    MKO_TIMED("selscan_chain", s, chain<false><<<blocks_for(g.rows * g.dstate), 256, 0, s>>>(g, q.A, q.drive, q.sumd, q.states));
  if (g.dstate == NS)
    MKO_TIMED("selscan_fwd_replay", s, fwd_replay<NS, UNI, TU, true><<<dim3(gx, g.nchunks), block, 0, s>>>(g, q));
  else
    MKO_TIMED("selscan_fwd_replay", s, fwd_replay<NS, UNI, TU, false><<<dim3(gx, g.nchunks), block, 0, s>>>(g, q));
  return mko_check_launch("selscan_fwd");
}

template <class TU>
static int launch_bwd_lane(const Plan& pl, const Ptrs& q0, const mko_selscan_params* p, hipStream_t s) {
  Geo g = pl.g;
  Ptrs q = q0;
  char* ws = static_cast<char*>(p->workspace);
  q.pbc = reinterpret_cast<float*>(ws + pl.loff_pbc);
  q.dap = reinterpret_cast<float*>(ws + pl.loff_dap);
  q.ddp = reinterpret_cast<float*>(ws + pl.loff_ddp);
  q.dbp = reinterpret_cast<float*>(ws + pl.loff_dbp);
  const unsigned grid = static_cast<unsigned>((g.rows + 4 * kLaneChannels - 1) / (4 * kLaneChannels));
  if (g.bc_dtype == MKO_BF16)
    MKO_TIMED("selscan_bwd_lane", s, bwd_lane<TU, bf16><<<grid, 256, 0, s>>>(g, q, pl.cpb));
  else if (g.bc_dtype == MKO_F16)
    MKO_TIMED("selscan_bwd_lane", s, bwd_lane<TU, _Float16><<<grid, 256, 0, s>>>(g, q, pl.cpb));
  else
    MKO_TIMED("selscan_bwd_lane", s, bwd_lane<TU, float><<<grid, 256, 0, s>>>(g, q, pl.cpb));
  // partials: dB/dC per cpb channels; dA / dD / ddelta_bias per row (one "chunk")
  g.nchunks = 1;
  MKO_TIMED("selscan_bwd_reduce", s,
            reduce_bc<16><<<static_cast<unsigned>(g.batch * g.ngroups * ((g.length + 256 / 16 - 1) / (256 / 16))),
                            256, 0, s>>>(g, static_cast<int>(pl.lncb), 0, q.pbc, p->dB, p->dC);
            reduce_params<<<static_cast<unsigned>((g.dstate + 1) * ((g.dim + 63) / 64)), 256, 0, s>>>(
                g, 16, q.dap, q.ddp, q.dbp, p->dA, p->dD, p->ddelta_bias));
  return mko_check_launch("selscan_bwd");
}

template <int NS, bool UNI, class TU>
static int launch_bwd(const Plan& pl, const Ptrs& q, const mko_selscan_params* p, hipStream_t s) {
  if constexpr (NS == 16 && !__is_same(TU, Dyn)) {
    if (pl.lane_bwd) return launch_bwd_lane<TU>(pl, q, p, s);
  }
  const Geo& g = pl.g;
  const dim3 block(g.wpg * kWave);
  const unsigned gx = static_cast<unsigned>((g.nwr + g.wpg - 1) / g.wpg);
  const int64_t bgl = g.batch * g.ngroups * g.length;
  const int64_t ntiles = (g.length + kPrepSteps - 1) / kPrepSteps;
  const unsigned gprep = static_cast<unsigned>(g.batch * g.ngroups * ntiles);
  // the backward reads C time-major (summaries) and B, C state-major (main pass)
  MKO_TIMED("selscan_prep", s,
            prep_layouts<NS><<<gprep, 256, 0, s>>>(g, ntiles, q.B, q.C, nullptr, q.ct, q.bn, q.cn));
  if (g.nchunks > 1) {
    MKO_TIMED("selscan_bwd_summary", s, bwd_summary<NS, UNI, TU><<<dim3(gx, g.nchunks - 1), block, 0, s>>>(g, q));
  }
  if (chain_by_wave(g))
    MKO_TIMED("selscan_chain", s,
              chain_wave<true><<<blocks_for(g.rows * g.dstate, 4), 256, 0, s>>>(g, q.A, q.drive, q.sumd, q.adj));
  else
    MKO_TIMED("selscan_chain", s, chain<true><<<blocks_for(g.rows * g.dstate), 256, 0, s>>>(g, q.A, q.drive, q.sumd, q.adj));
  if (g.dstate == NS)
    MKO_TIMED("selscan_bwd_main", s, bwd_main<NS, UNI, true><<<dim3(gx, g.nchunks), block, 0, s>>>(g, q));
  else
    MKO_TIMED("selscan_bwd_main", s, bwd_main<NS, UNI, false><<<dim3(gx, g.nchunks), block, 0, s>>>(g, q));
  MKO_TIMED("selscan_bwd_reduce", s,
            reduce_bc<NS><<<static_cast<unsigned>(g.batch * g.ngroups * ((g.length + 256 / NS - 1) / (256 / NS))),
                            256, 0, s>>>(g, g.ncb, UNI ? 0 : g.dg, q.pbc, p->dB, p->dC);
            reduce_params<<<static_cast<unsigned>((g.dstate + 1) * ((g.dim + 63) / 64)), 256, 0, s>>>(
                g, NS, q.dap, q.ddp, q.dbp, p->dA, p->dD, p->ddelta_bias));
  return mko_check_launch("selscan_bwd");
}

// Typed path when delta is float32, every 16-step block is whole and rows are aligned.
template <class F>
static int dispatch_types(const Plan& pl, int u_dtype, int d_dtype, F&& f) {
  const Geo& g = pl.g;
  const bool typed = d_dtype == MKO_F32 && g.vec && g.length % HS == 0;
  if (typed && u_dtype == MKO_BF16) return f(bf16{});
  if (typed && u_dtype == MKO_F16) return f(_Float16{});
  if (typed && u_dtype == MKO_F32) return f(float{});
  return f(Dyn{});
}

}  // namespace ss
}  // namespace mko

using namespace mko;
using namespace mko::ss;

extern "C" int64_t mko_selscan_num_checkpoints(int64_t length) {
  return length <= 0 ? 0 : (length + CK - 1) / CK;
}

extern "C" size_t mko_selscan_fwd_workspace_size(const mko_selscan_params* p) {
  Plan pl;
  if (make_plan(p, &pl) != MKO_OK) return 0;
  return pl.fwd_bytes;
}

extern "C" size_t mko_selscan_bwd_workspace_size(const mko_selscan_params* p) {
  Plan pl;
  if (make_plan(p, &pl) != MKO_OK) return 0;
  return pl.bwd_bytes;
}

extern "C" int mko_selscan_plan(const mko_selscan_params* p, int* fwd_lane, int* bwd_lane) {
  Plan pl;
  const int st = make_plan(p, &pl);
  if (st != MKO_OK) return st;
  if (fwd_lane) *fwd_lane = lane_shape(pl.g, pl.ns) ? 1 : 0;
  if (bwd_lane) *bwd_lane = lane_bwd_shape(pl.g, pl.ns) ? 1 : 0;
  return MKO_OK;
}

extern "C" int mko_selscan_fwd(const mko_selscan_params* p, void* stream) {
  Plan pl;
  int st = make_plan(p, &pl);
  if (st != MKO_OK) return st;
  if (pl.g.rows == 0 || pl.g.length == 0) return MKO_OK;
  if (!p->u || !p->delta || !p->A || !p->B || !p->C || !p->out || !p->states) {
    mko_set_error("selscan_fwd: u, delta, A, B, C, out and states are required");
    return MKO_EINVAL;
  }
  if (!p->workspace || p->workspace_bytes < pl.fwd_bytes) {
    mko_set_error("selscan_fwd: workspace of %zu bytes needed, %zu given", pl.fwd_bytes, p->workspace_bytes);
    return MKO_EWORKSPACE;
  }
  pl.g.vec = rows_vectorisable(pl.g, {{p->u, p->u_dtype}, {p->delta, p->delta_dtype}, {p->z, p->u_dtype},
                                      {p->out, p->u_dtype}}) ? 1 : 0;
  pl.lane = lane_shape(pl.g, pl.ns) &&
            rows_vectorisable(pl.g, {{p->B, p->bc_dtype}, {p->C, p->bc_dtype}});
  Ptrs q = make_ptrs(p, pl);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dispatch_types(pl, p->u_dtype, p->delta_dtype, [&](auto tag) {
    using TU = decltype(tag);
    if (pl.ns == 16) return pl.uni ? launch_fwd<16, true, TU>(pl, q, s) : launch_fwd<16, false, TU>(pl, q, s);
    return pl.uni ? launch_fwd<32, true, TU>(pl, q, s) : launch_fwd<32, false, TU>(pl, q, s);
  });
}

extern "C" int mko_selscan_bwd(const mko_selscan_params* p, void* stream) {
  Plan pl;
  int st = make_plan(p, &pl);
  if (st != MKO_OK) return st;
  if (!p->du || !p->ddelta) {
    mko_set_error("selscan_bwd: du and ddelta are required");
    return MKO_EINVAL;
  }
  if (pl.g.rows == 0 || pl.g.length == 0) return MKO_OK;  // caller zero-fills parameter grads
  if (!p->u || !p->delta || !p->A || !p->B || !p->C || !p->states || !p->dout) {
    mko_set_error("selscan_bwd: u, delta, A, B, C, states and dout are required");
    return MKO_EINVAL;
  }
  if (!p->workspace || p->workspace_bytes < pl.bwd_bytes) {
    mko_set_error("selscan_bwd: workspace of %zu bytes needed, %zu given", pl.bwd_bytes, p->workspace_bytes);
    return MKO_EWORKSPACE;
  }
  pl.g.vec = rows_vectorisable(pl.g, {{p->u, p->u_dtype}, {p->delta, p->delta_dtype}, {p->z, p->u_dtype},
                                      {p->dout, p->u_dtype}, {p->du, p->u_dtype}, {p->ddelta, p->delta_dtype},
                                      {p->dz, p->u_dtype}, {p->out, p->u_dtype}}) ? 1 : 0;
  pl.lane_bwd = lane_bwd_shape(pl.g, pl.ns) && rows_vectorisable(pl.g, {{p->B, p->bc_dtype}, {p->C, p->bc_dtype}});
  Ptrs q = make_ptrs(p, pl);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dispatch_types(pl, p->u_dtype, p->delta_dtype, [&](auto tag) {
    using TU = decltype(tag);
    if (pl.ns == 16) return pl.uni ? launch_bwd<16, true, TU>(pl, q, p, s) : launch_bwd<16, false, TU>(pl, q, p, s);
    return pl.uni ? launch_bwd<32, true, TU>(pl, q, p, s) : launch_bwd<32, false, TU>(pl, q, p, s);
  });
}
