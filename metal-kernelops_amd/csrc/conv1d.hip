// Causal depthwise conv1d (the convolution ahead of every Mamba block) for gfx950.
//
// With z = cat(initial_state or zeros(K-1), x) along time and m = K - 1:
//   pre[b, c, t] = bias[c] + sum_{j < K} w[c, j] z[b, c, t + j]      (z index t + j = time t - m + j)
//   out          = act(pre),  act = identity or silu
//   final_state  = z[..., L : L + m]
// Widths up to 8: a wavefront covers 64 * WF (forward) or 64 * WB (backward) consecutive
// 8-step blocks of one row, lane l taking blocks l, l + 64, ... (one 16-byte vector load per
// block on aligned rows, so every
// wavefront access is 64 consecutive blocks); the look-back (and, in the backward,
// look-ahead) steps come from the neighbouring lanes.  Wider kernels: the forward gives a
// lane one block; the backward walks RB consecutive blocks with sliding register windows.
// Backward: the lane recomputes pre over its window, writes dx, and sums the taps'
// gradients dw[c, j] = sum_t g[t] z[t - m + j] and dbias = sum_t g[t] (g = dout act'(pre))
// over its steps; the lanes of a wavefront (or of a 16-lane group, wider kernels) add
// theirs with DPP, and `finalize_il` / `finalize` add those partials over batch and along
// the row in a fixed order, so the sums are deterministic.
// Decode: one lane per row advances a rolling state of `span` columns by q tokens in
// place.
#include "common.hpp"
#include "io.hpp"

namespace mko {
namespace conv {
namespace {

constexpr int BS = 8;  // steps per block
constexpr int RB = 4;  // blocks per lane in the wide-kernel backward (width > 8)
constexpr int WF = 4;  // iterations of the interleaved forward: a wavefront covers 64 * WF
                       // consecutive blocks of a row, lane l taking blocks l, l + 64, ...
constexpr int WB = 8;  // iterations of the interleaved backward (more, so that its longer
                       // per-wavefront setup and tap sums are paid over more blocks)

struct Geo {
  int64_t batch, channels, length, rows;  // rows = batch * channels
  int width, taps;                          // taps = width - 1
  int64_t nblk;                             // blocks of BS steps per row
  int64_t lpr;                              // lanes per row: ceil(nblk / RB), rounded up to 16
  int64_t nseg;                             // interleaved forward: wavefronts per row
  int64_t nsegb;                            // interleaved backward: wavefronts per row
  int dtype;
  int silu;
  int vec;                                  // rows are 16-byte aligned whole blocks
};

// z at time t of row `row`: x for 0 <= t < length, the initial state (or zero padding)
// for -taps <= t < 0, zero elsewhere.
__device__ __forceinline__ float z_at(const Geo& g, const void* x, const void* init, int64_t row, int64_t t) {
  if (t >= 0) return t < g.length ? load_one(x, g.dtype, row * g.length + t) : 0.0f;
  if (!init || t < -g.taps) return 0.0f;
  return load_one(init, g.dtype, row * g.taps + (g.taps + t));
}

// The taps left-padded to KMAX: wp[j'] = w[j' - (KMAX - width)], zero below, so that
// pre(t) = bias + sum_{j' < KMAX} wp[j'] z(t - (KMAX - 1) + j') with compile-time indices.
template <int KMAX>
__device__ __forceinline__ void load_taps(const Geo& g, const void* weight, int64_t c, float (&wp)[KMAX]) {
  const int lead = KMAX - g.width;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) wp[j] = j >= lead ? load_one(weight, g.dtype, c * g.width + (j - lead)) : 0.0f;
}

// The BS steps of block `blk` of a row as floats (zero past the end of the row).
__device__ __forceinline__ void row_block(const Geo& g, const void* src, int64_t row, int64_t blk, float (&v)[BS]) {
  const int64_t t0 = blk * BS;
  if (blk >= g.nblk) {
#pragma unroll
    for (int e = 0; e < BS; ++e) v[e] = 0.0f;
  } else if (g.vec) {
    load_run<BS>(src, g.dtype, row * g.length + t0, BS, true, v);
  } else {
#pragma unroll
    for (int e = 0; e < BS; ++e) v[e] = t0 + e < g.length ? load_one(src, g.dtype, row * g.length + t0 + e) : 0.0f;
  }
}

// One BS-step block of a row of T, kept as loaded until `get`, so that a block fetched a
// step ahead stays in flight until its first use (converting at the load would wait for
// it there).  The load always reads inside the row (a block past the end reads the last
// one again) and `get` zeroes the steps past the end.  VEC: whole 16-byte aligned blocks.
template <class T, bool VEC>
struct RawBlk {
  static constexpr int W = VEC ? BS * static_cast<int>(sizeof(T)) / 4 : BS;
  static_assert(!VEC || W % 4 == 0, "a block is whole 16-byte vectors");
  uint32_t w[W];
  int nok;  // steps of the block inside the row
  __device__ __forceinline__ void load(const Geo& g, const T* __restrict__ src, int64_t row, int64_t blk) {
    const int64_t b = blk < g.nblk ? blk : g.nblk - 1;
    const int64_t t0 = b * BS;
    const T* q = src + row * g.length + t0;
    if constexpr (VEC) {
      nok = blk < g.nblk ? BS : 0;
      load_words(q, w);
    } else {
      const int64_t left = g.length - t0;  // at least 1
      nok = blk < g.nblk ? (left < BS ? static_cast<int>(left) : BS) : 0;
#pragma unroll
      for (int e = 0; e < BS; ++e) w[e] = __float_as_uint(to_f32(q[e < left ? e : left - 1]));
    }
  }
  __device__ __forceinline__ void get(float (&v)[BS]) const {
    float f[BS];
    if constexpr (VEC)
      unpack_words<T, BS>(w, f);
    else
      unpack_words<float, BS>(w, f);  // the scalar path keeps fp32 words
#pragma unroll
    for (int i = 0; i < BS; ++i) v[i] = i < nok ? f[i] : 0.0f;
  }
};

// The taps (left-padded to KMAX as in load_taps) and the bias of channel c, and the carry
// z(t_first + i), i < H (x for t >= 0, else the initial state or zero padding), in the
// element type: every load reads a valid address and is issued before any is converted,
// so they arrive together (through load_one's dtype branches they would be waited for one
// at a time).
template <int KMAX, class T>
__device__ __forceinline__ void load_setup_t(const Geo& g, const mko_conv1d_params& p, int64_t row, int64_t c,
                                             int64_t t_first, float (&wp)[KMAX], float& bias,
                                             float (&carry)[KMAX - 1]) {
  constexpr int H = KMAX - 1;
  const int lead = KMAX - g.width;
  const T* w = static_cast<const T*>(p.weight) + c * g.width;
  const T* b = p.bias ? static_cast<const T*>(p.bias) + c : w;
  const T* xr = static_cast<const T*>(p.x) + row * g.length;
  const bool has_init = p.initial_state != nullptr && g.taps > 0;  // width 1: an empty state
  const T* ir = has_init ? static_cast<const T*>(p.initial_state) + row * g.taps : xr;
  T rw[KMAX], rx[H], ri[H];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) rw[j] = w[j >= lead ? j - lead : 0];
  const T rb = *b;
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const int64_t t = t_first + i, ti = g.taps + t;
    rx[i] = xr[t < 0 ? 0 : (t < g.length ? t : g.length - 1)];
    ri[i] = ir[has_init && ti >= 0 && ti < g.taps ? ti : 0];
  }
#pragma unroll
  for (int j = 0; j < KMAX; ++j) wp[j] = j >= lead ? to_f32(rw[j]) : 0.0f;
  bias = p.bias ? to_f32(rb) : 0.0f;
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const int64_t t = t_first + i;
    carry[i] = t >= 0 ? (t < g.length ? to_f32(rx[i]) : 0.0f) : (has_init && t >= -g.taps ? to_f32(ri[i]) : 0.0f);
  }
}

// The BS steps at t0 of a typed row (those inside the row).
template <class T, bool VEC>
__device__ __forceinline__ void typed_store(const Geo& g, void* dst, int64_t row, int64_t t0, const float (&v)[BS]) {
  const int64_t left = g.length - t0;
  store_run_t<T, BS>(static_cast<T*>(dst) + row * g.length + t0, left < BS ? static_cast<int>(left) : BS, VEC, v);
}

__device__ __forceinline__ void row_store(const Geo& g, void* dst, int64_t row, int64_t t0, const float (&v)[BS]) {
  if (g.vec) {
    store_run<BS>(dst, g.dtype, row * g.length + t0, BS, true, v);
  } else {
#pragma unroll
    for (int s = 0; s < BS; ++s)
      if (t0 + s < g.length) store_one(dst, g.dtype, row * g.length + t0 + s, v[s]);
  }
}

__device__ __forceinline__ float act(const Geo& g, float v) { return g.silu ? v * sigmoid(v) : v; }
__device__ __forceinline__ float act_grad(const Geo& g, float v) {
  if (!g.silu) return 1.0f;
  const float s = sigmoid(v);
  return s * (1.0f + v * (1.0f - s));
}

template <int KMAX>
__global__ void __launch_bounds__(256) forward(Geo g, mko_conv1d_params p) {
  constexpr int H = KMAX - 1;
  constexpr int RF = 1;  // blocks per lane
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= g.rows * g.nblk) return;
  const int64_t row = e / g.nblk, blk0 = e % g.nblk, c = row % g.channels;
  float wp[KMAX];
  load_taps<KMAX>(g, p.weight, c, wp);
  const float bias = p.bias ? load_one(p.bias, g.dtype, c) : 0.0f;
  // zz[i] = z(t0 - H + i); the first H carry over from the previous block
  float zz[H + BS];
#pragma unroll
  for (int i = 0; i < H; ++i) zz[i] = i >= H - g.taps ? z_at(g, p.x, p.initial_state, row, blk0 * BS - H + i) : 0.0f;
  float nxt[BS];
  row_block(g, p.x, row, blk0, nxt);
  for (int r = 0; r < RF; ++r) {
    const int64_t blk = blk0 + r;
    if (blk >= g.nblk) break;
    const int64_t t0 = blk * BS;
#pragma unroll
    for (int i = 0; i < BS; ++i) zz[H + i] = nxt[i];
    if (r + 1 < RF) row_block(g, p.x, row, blk + 1, nxt);  // in flight during this block
    float o[BS];
#pragma unroll
    for (int s = 0; s < BS; ++s) {
      float acc = bias;
#pragma unroll
      for (int j = 0; j < KMAX; ++j) acc = fmaf(wp[j], zz[s + j], acc);
      o[s] = act(g, acc);
    }
    row_store(g, p.out, row, t0, o);
#pragma unroll
    for (int i = 0; i < H; ++i) zz[i] = zz[BS + i];
    if (p.final_state && blk == g.nblk - 1) {
      for (int m = 0; m < g.taps; ++m)
        store_one(p.final_state, g.dtype, row * g.taps + m, z_at(g, p.x, p.initial_state, row, g.length - g.taps + m));
    }
  }
}

template <int KMAX>
__global__ void __launch_bounds__(256) backward(Geo g, mko_conv1d_params p, float* partial) {
  constexpr int H = KMAX - 1;
  // The grid covers whole 16-lane groups of one row each (lpr is a multiple of 16), and
  // every lane reaches the DPP sums at the end.
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool in_grid = e < g.rows * g.lpr;
  const int64_t row = in_grid ? e / g.lpr : 0, blk0 = in_grid ? (e % g.lpr) * RB : g.nblk;
  const int64_t c = row % g.channels;
  float wp[KMAX];
  load_taps<KMAX>(g, p.weight, c, wp);
  const float bias = p.bias ? load_one(p.bias, g.dtype, c) : 0.0f;
  float dwp[KMAX], dbp = 0.0f;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) dwp[j] = 0.0f;
  if (blk0 < g.nblk) {
    // zz[i] = z(t0 - H + i) over [t0 - H, t0 + BS + H); zn, dn: the next block of x, dout
    float zz[BS + 2 * H], zn[BS], dc[BS], dn[BS];
#pragma unroll
    for (int i = 0; i < H; ++i) zz[i] = z_at(g, p.x, p.initial_state, row, blk0 * BS - H + i);
    {
      float cur[BS];
      row_block(g, p.x, row, blk0, cur);
#pragma unroll
      for (int i = 0; i < BS; ++i) zz[H + i] = cur[i];
    }
    row_block(g, p.x, row, blk0 + 1, zn);
    row_block(g, p.dout, row, blk0, dc);
    row_block(g, p.dout, row, blk0 + 1, dn);
    for (int r = 0; r < RB; ++r) {
      const int64_t blk = blk0 + r;
      if (blk >= g.nblk) break;
      const int64_t t0 = blk * BS;
      // look-ahead z: the next block, then (taps beyond a block) single steps
#pragma unroll
      for (int i = 0; i < H; ++i) zz[H + BS + i] = i < BS ? zn[i] : z_at(g, p.x, p.initial_state, row, t0 + BS + i);
      // gg[i] = g(t0 + i) = dout act'(pre), zero from the end of the row
      float gg[BS + H];
#pragma unroll
      for (int i = 0; i < BS + H; ++i) {
        float pre = bias;
#pragma unroll
        for (int j = 0; j < KMAX; ++j) pre = fmaf(wp[j], zz[i + j], pre);
        const bool in_row = t0 + i < g.length;
        const float d = i < BS ? dc[i]
                               : (i - BS < BS ? dn[i - BS] : (in_row ? load_one(p.dout, g.dtype, row * g.length + t0 + i) : 0.0f));
        gg[i] = in_row ? d * act_grad(g, pre) : 0.0f;
      }
      // dx(t) = sum_j' wp[j'] g(t + H - j')
      float dxo[BS];
#pragma unroll
      for (int s = 0; s < BS; ++s) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < KMAX; ++j) acc = fmaf(wp[j], gg[s + H - j], acc);
        dxo[s] = acc;
      }
      row_store(g, p.dx, row, t0, dxo);
      // taps (padded index) and bias over this block's own steps
#pragma unroll
      for (int s = 0; s < BS; ++s) {
        dbp += gg[s];
#pragma unroll
        for (int j = 0; j < KMAX; ++j) dwp[j] = fmaf(gg[s], zz[s + j], dwp[j]);
      }
      // initial state: z(tau), -taps <= tau < 0, feeds pre(t) at t = tau + H - j'
      if (p.dinitial && blk == 0) {
#pragma unroll
        for (int k = 1; k <= H; ++k) {
          float acc = 0.0f;
#pragma unroll
          for (int j = 0; j < KMAX; ++j) {
            const int i = H - k - j;
            if (i >= 0) acc = fmaf(wp[j], gg[i], acc);
          }
          if (k <= g.taps) store_one(p.dinitial, g.dtype, row * g.taps + (g.taps - k), acc);
        }
      }
      // slide by one block; the loads of the block after next fly during the next one
#pragma unroll
      for (int i = 0; i < H; ++i) zz[i] = zz[BS + i];
#pragma unroll
      for (int i = 0; i < BS; ++i) {
        zz[H + i] = zn[i];
        dc[i] = dn[i];
      }
      if (r + 1 < RB) {
        row_block(g, p.x, row, blk + 2, zn);
        row_block(g, p.dout, row, blk + 2, dn);
      }
    }
  }
  if (!partial) return;
  // one partial per 16-lane group of a row: the K taps, then the bias
  const int lead = KMAX - g.width;
  float* dst = partial + (in_grid ? e / 16 : 0) * (g.width + 1);
  const bool writer = in_grid && (threadIdx.x & 15) == 0;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < lead) continue;  // uniform
    const float v = row16_sum(dwp[j]);
    if (writer) dst[j - lead] = v;
  }
  const float vb = row16_sum(dbp);
  if (writer) dst[g.width] = vb;
}

// Forward for widths up to 8, blocks interleaved across lanes as in `backward_il`: a
// wavefront covers 64 * WF consecutive blocks of one row, every load and store is 64
// consecutive blocks, and the H steps before a block come from lane l - 1 (lane 0: the
// carry of lane 63's previous block, or the initial state).  The per-row setup (index
// arithmetic, taps, bias) is paid once per four blocks.
template <int KMAX, class T, bool VEC>
__global__ void __launch_bounds__(256) forward_il(Geo g, mko_conv1d_params p) {
  constexpr int H = KMAX - 1;
  static_assert(H < BS, "look-back within one neighbouring block");
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wv = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + (threadIdx.x >> 6);
  if (wv >= g.rows * g.nseg) return;  // wave-uniform: whole wavefronts leave
  const int64_t row = wv / g.nseg, seg = wv % g.nseg;
  const int64_t c = row % g.channels;
  const int64_t base = seg * kWave * WF;
  // the carry: z(t0 - H + i) of lane 0's first block
  float wp[KMAX], bias, carry[H];
  load_setup_t<KMAX, T>(g, p, row, c, base * BS - H, wp, bias, carry);
  const T* xs = static_cast<const T*>(p.x);
  RawBlk<T, VEC> cur;
  cur.load(g, xs, row, base + lane);
  for (int k = 0; k < WF; ++k) {
    const int64_t blk = base + k * kWave + lane;
    if (base + k * kWave >= g.nblk) break;  // wave-uniform: no block of this iteration exists
    RawBlk<T, VEC> nxt;
    if (k + 1 < WF) nxt.load(g, xs, row, blk + kWave);  // in flight during this block
    float xc[BS];
    cur.get(xc);
    float zz[H + BS];
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const float prev = __shfl_up(xc[BS - H + i], 1);
      zz[i] = lane == 0 ? carry[i] : prev;
    }
#pragma unroll
    for (int i = 0; i < BS; ++i) zz[H + i] = xc[i];
    if (blk < g.nblk) {
      float o[BS];
#pragma unroll
      for (int s = 0; s < BS; ++s) {
        float acc = bias;
#pragma unroll
        for (int j = 0; j < KMAX; ++j) acc = fmaf(wp[j], zz[s + j], acc);
        o[s] = act(g, acc);
      }
      typed_store<T, VEC>(g, p.out, row, blk * BS, o);
      if (p.final_state && blk == g.nblk - 1) {
        for (int m = 0; m < g.taps; ++m)
          store_one(p.final_state, g.dtype, row * g.taps + m,
                    z_at(g, p.x, p.initial_state, row, g.length - g.taps + m));
      }
    }
#pragma unroll
    for (int i = 0; i < H; ++i) carry[i] = __shfl(xc[BS - H + i], kWave - 1);
    if (k + 1 < WF) cur = nxt;
  }
}

// Backward for widths up to 8 (look-back and look-ahead shorter than a block), blocks
// interleaved across lanes: at iteration k lane l holds block base + 64 k + l, so every
// load and store of a wavefront is 64 consecutive blocks (1 KB of 16-bit x).  The H = K - 1
// steps before a block come from lane l - 1 (lane 0: the carry of lane 63's block one
// iteration earlier, or the initial state), the H steps after it from lane l + 1 (lane 63:
// from lane 0's next block, which is in flight as the next iteration's prefetch).  The
// loop stays rolled: unrolled, the four iterations' registers cost a wavefront per SIMD.
// The taps' gradients are summed over the wavefront, which
// lies in one row, and `finalize_il` adds the wavefronts' partials in order.
template <int KMAX, class T, bool VEC>
__global__ void __launch_bounds__(256) backward_il(Geo g, mko_conv1d_params p, float* partial) {
  constexpr int H = KMAX - 1;
  static_assert(H < BS, "look-back and look-ahead within one neighbouring block");
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wv = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + (threadIdx.x >> 6);
  const bool in_grid = wv < g.rows * g.nsegb;
  const int64_t row = in_grid ? wv / g.nsegb : 0, seg = in_grid ? wv % g.nsegb : 0;
  const int64_t c = row % g.channels;
  float dwp[KMAX], dbp = 0.0f;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) dwp[j] = 0.0f;
  const int64_t base = in_grid ? seg * kWave * WB : g.nblk;  // no row: every block is past the end
  // the carry: z(t0 - H + i), i < H, of lane 0's first block (the initial state or zeros for
  // block 0, else the steps before the segment)
  float wp[KMAX], bias, carry[H];
  load_setup_t<KMAX, T>(g, p, row, c, base * BS - H, wp, bias, carry);
  const T* xs = static_cast<const T*>(p.x);
  const T* ds = static_cast<const T*>(p.dout);
  RawBlk<T, VEC> xr, dr;
  xr.load(g, xs, row, base + lane);
  dr.load(g, ds, row, base + lane);
#pragma unroll 1
  for (int k = 0; k < WB; ++k) {
    const int64_t blk = base + k * kWave + lane;
    const int64_t t0 = blk * BS;
    // The next iteration's blocks, in flight during this one.  Lane 0's is also the block
    // after lane 63's, so in the last iteration lane 0 alone needs it (the other lanes'
    // loads re-read the row's last block and come out as zeros).
    RawBlk<T, VEC> xnr, dnr;
    {
      const int64_t nb = (k + 1 < WB || lane == 0) ? blk + kWave : g.nblk;
      xnr.load(g, xs, row, nb);
      dnr.load(g, ds, row, nb);
    }
    float xc[BS], dc[BS];
    xr.get(xc);
    dr.get(dc);
    // zz[i] = z(t0 - H + i) over [t0 - H, t0 + BS + H); the last H (look-ahead) further down
    float zz[BS + 2 * H];
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const float prev = __shfl_up(xc[BS - H + i], 1);
      zz[i] = lane == 0 ? carry[i] : prev;
    }
#pragma unroll
    for (int i = 0; i < BS; ++i) zz[H + i] = xc[i];
    // gg[i] = g(t0 + i) = dout act'(pre), zero from the end of the row.  The block's own
    // steps first: they and the tap and bias gradients need no look-ahead.
    float gg[BS + H];
    auto grad_at = [&](int i, float d) {
      float pre = bias;
#pragma unroll
      for (int j = 0; j < KMAX; ++j) pre = fmaf(wp[j], zz[i + j], pre);
      return t0 + i < g.length ? d * act_grad(g, pre) : 0.0f;
    };
#pragma unroll
    for (int i = 0; i < BS; ++i) gg[i] = grad_at(i, dc[i]);
    // taps (padded index) and bias over this block's own steps (zero past the row)
#pragma unroll
    for (int s = 0; s < BS; ++s) {
      dbp += gg[s];
#pragma unroll
      for (int j = 0; j < KMAX; ++j) dwp[j] = fmaf(gg[s], zz[s + j], dwp[j]);
    }
    // The next block's first H steps: from lane + 1; lane 63 takes them from lane 0's next
    // block.  Kept after the work above, so that load has had that long to arrive.
    __builtin_amdgcn_sched_barrier(0);
    {
      float xn[BS], dn[BS];
      xnr.get(xn);
      dnr.get(dn);
      const bool last = lane == kWave - 1;
#pragma unroll
      for (int i = 0; i < H; ++i) {
        const float x0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xn[i]), 0));
        const float d0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dn[i]), 0));
        const float xd = __shfl_down(xc[i], 1), dd = __shfl_down(dc[i], 1);
        zz[H + BS + i] = last ? x0 : xd;
        gg[BS + i] = last ? d0 : dd;  // dout for now, the gradient just below
      }
    }
#pragma unroll
    for (int i = BS; i < BS + H; ++i) gg[i] = grad_at(i, gg[i]);
    if (blk < g.nblk) {
      float dxo[BS];
#pragma unroll
      for (int s = 0; s < BS; ++s) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < KMAX; ++j) acc = fmaf(wp[j], gg[s + H - j], acc);
        dxo[s] = acc;
      }
      typed_store<T, VEC>(g, p.dx, row, t0, dxo);
      if (p.dinitial && blk == 0) {
#pragma unroll
        for (int kk = 1; kk <= H; ++kk) {
          float acc = 0.0f;
#pragma unroll
          for (int j = 0; j < KMAX; ++j) {
            const int i = H - kk - j;
            if (i >= 0) acc = fmaf(wp[j], gg[i], acc);
          }
          if (kk <= g.taps) store_one(p.dinitial, g.dtype, row * g.taps + (g.taps - kk), acc);
        }
      }
    }
    // lane 63's last H steps precede lane 0's next block
#pragma unroll
    for (int i = 0; i < H; ++i) carry[i] = __shfl(xc[BS - H + i], kWave - 1);
    xr = xnr;
    dr = dnr;
  }
  if (!partial) return;
  // one partial per wavefront: the K taps, then the bias
  const int lead = KMAX - g.width;
  float* dst = partial + (in_grid ? wv : 0) * (g.width + 1);
  const bool writer = in_grid && lane == 0;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < lead) continue;  // uniform
    const float v = wave_sum(dwp[j]);
    if (writer) dst[j - lead] = v;
  }
  const float vb = wave_sum(dbp);
  if (writer) dst[g.width] = vb;
}

// dweight[c, j] and dbias[c] from the interleaved backward: the wavefronts' partials summed
// over batch, then along the row, in order.
__global__ void __launch_bounds__(256) finalize_il(Geo g, mko_conv1d_params p, const float* partial) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= g.channels * (g.width + 1)) return;
  const int64_t c = e / (g.width + 1);
  const int j = static_cast<int>(e % (g.width + 1));
  float s = 0.0f;
  for (int64_t b = 0; b < g.batch; ++b) {
    const int64_t row = b * g.channels + c;
    for (int64_t k = 0; k < g.nsegb; ++k) s += partial[(row * g.nsegb + k) * (g.width + 1) + j];
  }
  if (j < g.width) {
    if (p.dweight) store_one(p.dweight, g.dtype, c * g.width + j, s);
  } else if (p.dbias) {
    store_one(p.dbias, g.dtype, c, s);
  }
}

// dweight[c, j] and dbias[c]: the 16-lane partials summed over batch, then along the
// row, in order.
__global__ void __launch_bounds__(256) finalize(Geo g, mko_conv1d_params p, const float* partial) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= g.channels * (g.width + 1)) return;
  const int64_t c = e / (g.width + 1);
  const int j = static_cast<int>(e % (g.width + 1));
  const int64_t groups = g.lpr / 16;
  float s = 0.0f;
  for (int64_t b = 0; b < g.batch; ++b) {
    const int64_t row = b * g.channels + c;
    for (int64_t k = 0; k < groups; ++k) s += partial[(row * groups + k) * (g.width + 1) + j];
  }
  if (j < g.width) {
    if (p.dweight) store_one(p.dweight, g.dtype, c * g.width + j, s);
  } else if (p.dbias) {
    store_one(p.dbias, g.dtype, c, s);
  }
}

// Decode: per row, joined = cat(state[0..span), x[0..q)); out[t] = act(bias + sum_j
// w[j] joined[span + t - taps + j]); then state = joined[q .. q + span).
__global__ void __launch_bounds__(256) update(mko_conv1d_update_params p) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (row >= p.batch * p.channels) return;
  const int64_t b = row / p.channels, c = row % p.channels;
  const int dt = p.dtype;
  const int64_t sb = b * p.state_stride_b + c * p.state_stride_c;
  const int64_t taps = p.width - 1;
  const float bias = p.bias ? load_one(p.bias, dt, c) : 0.0f;
  const bool silu = (p.flags & MKO_CONV_SILU) != 0;
  // joined index i: state column i (i < span), else token i - span
  auto joined = [&](int64_t i) -> float {
    return i < p.span ? load_one(p.state, dt, sb + i) : load_one(p.x, dt, row * p.q + (i - p.span));
  };
  for (int64_t t = 0; t < p.q; ++t) {
    float acc = bias;
    for (int64_t j = 0; j < p.width; ++j)
      acc = fmaf(load_one(p.weight, dt, c * p.width + j), joined(p.span + t - taps + j), acc);
    store_one(p.out, dt, row * p.q + t, silu ? acc * sigmoid(acc) : acc);
  }
  // shift: the new column i is joined[q + i]; ascending order never overwrites a state
  // column that a later i still reads (q + i > i)
  for (int64_t i = 0; i < p.span; ++i) store_one(p.state, dt, sb + i, joined(p.q + i));
}

int make_geo(const mko_conv1d_params* p, Geo* g) {
  if (!p) {
    mko_set_error("conv1d: null parameters");
    return MKO_EINVAL;
  }
  if (p->batch < 0 || p->channels < 0 || p->length < 0 || p->width < 1) {
    mko_set_error("conv1d: bad sizes batch=%lld channels=%lld length=%lld width=%lld",
                  static_cast<long long>(p->batch), static_cast<long long>(p->channels),
                  static_cast<long long>(p->length), static_cast<long long>(p->width));
    return MKO_EINVAL;
  }
  if (p->width > 32) {
    mko_set_error("conv1d: width=%lld > 32 is not supported", static_cast<long long>(p->width));
    return MKO_EUNSUPPORTED;
  }
  if (p->dtype != MKO_F32 && p->dtype != MKO_F16 && p->dtype != MKO_BF16) {
    mko_set_error("conv1d: unknown dtype %d", p->dtype);
    return MKO_EINVAL;
  }
  g->batch = p->batch;
  g->channels = p->channels;
  g->length = p->length;
  g->rows = p->batch * p->channels;
  g->width = static_cast<int>(p->width);
  g->taps = g->width - 1;
  g->nblk = (p->length + BS - 1) / BS;
  g->lpr = ((g->nblk + RB - 1) / RB + 15) / 16 * 16;
  g->nseg = (g->nblk + kWave * WF - 1) / (kWave * WF);
  g->nsegb = (g->nblk + kWave * WB - 1) / (kWave * WB);
  g->dtype = p->dtype;
  g->silu = (p->flags & MKO_CONV_SILU) != 0;
  const uintptr_t mask = 15u;
  g->vec = p->length % BS == 0 && (reinterpret_cast<uintptr_t>(p->x) & mask) == 0 &&
           (reinterpret_cast<uintptr_t>(p->out) & mask) == 0 && (reinterpret_cast<uintptr_t>(p->dx) & mask) == 0 &&
           (reinterpret_cast<uintptr_t>(p->dout) & mask) == 0;
  return MKO_OK;
}

template <int KMAX>
void launch_fwd(const Geo& g, const mko_conv1d_params& p, hipStream_t s) {
  if constexpr (KMAX <= BS) {
    const int64_t waves = g.rows * g.nseg;
    const unsigned grid = static_cast<unsigned>((waves + 3) / 4);
#define MKO_CONV_FWD(T, V) MKO_TIMED("conv1d_fwd", s, (forward_il<KMAX, T, V><<<grid, 256, 0, s>>>(g, p)))
    if (g.dtype == MKO_F32) {
      if (g.vec) MKO_CONV_FWD(float, true); else MKO_CONV_FWD(float, false);
    } else if (g.dtype == MKO_BF16) {
      if (g.vec) MKO_CONV_FWD(bf16, true); else MKO_CONV_FWD(bf16, false);
    } else {
      if (g.vec) MKO_CONV_FWD(_Float16, true); else MKO_CONV_FWD(_Float16, false);
    }
#undef MKO_CONV_FWD
  } else {
    const int64_t n = g.rows * g.nblk;
    MKO_TIMED("conv1d_fwd", s, forward<KMAX><<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(g, p));
  }
}

template <int KMAX>
void launch_bwd(const Geo& g, const mko_conv1d_params& p, float* partial, hipStream_t s) {
  if constexpr (KMAX <= BS) {
    const int64_t waves = g.rows * g.nsegb;
    const unsigned grid = static_cast<unsigned>((waves + 3) / 4);
#define MKO_CONV_BWD(T, V) MKO_TIMED("conv1d_bwd", s, (backward_il<KMAX, T, V><<<grid, 256, 0, s>>>(g, p, partial)))
    if (g.dtype == MKO_F32) {
      if (g.vec) MKO_CONV_BWD(float, true); else MKO_CONV_BWD(float, false);
    } else if (g.dtype == MKO_BF16) {
      if (g.vec) MKO_CONV_BWD(bf16, true); else MKO_CONV_BWD(bf16, false);
    } else {
      if (g.vec) MKO_CONV_BWD(_Float16, true); else MKO_CONV_BWD(_Float16, false);
    }
#undef MKO_CONV_BWD
  } else {
    const int64_t n = g.rows * g.lpr;
    MKO_TIMED("conv1d_bwd", s, backward<KMAX><<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(g, p, partial));
  }
}

// One partial per interleaved wavefront (width <= 8) or per 16-lane group (wider).
size_t partial_bytes(const Geo& g) {
  const int64_t parts = g.width <= BS ? g.rows * g.nsegb : g.rows * (g.lpr / 16);
  return static_cast<size_t>(parts) * (g.width + 1) * sizeof(float);
}

}  // namespace
}  // namespace conv
}  // namespace mko

using namespace mko;

extern "C" size_t mko_sizeof_conv1d_params(void) { return sizeof(mko_conv1d_params); }
extern "C" size_t mko_sizeof_conv1d_update_params(void) { return sizeof(mko_conv1d_update_params); }

extern "C" int mko_conv1d_fwd(const mko_conv1d_params* p, void* stream) {
  conv::Geo g;
  int st = conv::make_geo(p, &g);
  if (st != MKO_OK) return st;
  if (g.rows == 0 || g.length == 0) return MKO_OK;
  if (!p->x || !p->weight || !p->out) {
    mko_set_error("conv1d_fwd: x, weight and out are required");
    return MKO_EINVAL;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (g.width <= 4) conv::launch_fwd<4>(g, *p, s);
  else if (g.width <= 8) conv::launch_fwd<8>(g, *p, s);
  else conv::launch_fwd<32>(g, *p, s);
  return mko_check_launch("conv1d_fwd");
}

extern "C" size_t mko_conv1d_bwd_workspace_size(const mko_conv1d_params* p) {
  conv::Geo g;
  if (conv::make_geo(p, &g) != MKO_OK) return 0;
  return conv::partial_bytes(g);
}

extern "C" int mko_conv1d_bwd(const mko_conv1d_params* p, void* stream) {
  conv::Geo g;
  int st = conv::make_geo(p, &g);
  if (st != MKO_OK) return st;
  if (g.rows == 0 || g.length == 0) return MKO_OK;  // the caller zero-fills the gradients of an empty input
  if (!p->x || !p->weight || !p->dout || !p->dx) {
    mko_set_error("conv1d_bwd: x, weight, dout and dx are required");
    return MKO_EINVAL;
  }
  const bool params = p->dweight || p->dbias;
  const size_t need = conv::partial_bytes(g);
  if (params && (!p->workspace || p->workspace_bytes < need)) {
    mko_set_error("conv1d_bwd: workspace of %zu bytes needed, %zu given", need, p->workspace_bytes);
    return MKO_EWORKSPACE;
  }
  float* partial = params ? static_cast<float*>(p->workspace) : nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (g.width <= 4) conv::launch_bwd<4>(g, *p, partial, s);
  else if (g.width <= 8) conv::launch_bwd<8>(g, *p, partial, s);
  else conv::launch_bwd<32>(g, *p, partial, s);
  if (params) {
    const int64_t n = g.channels * (g.width + 1);
    const unsigned grid = static_cast<unsigned>((n + 255) / 256);
    if (g.width <= conv::BS)
      MKO_TIMED("conv1d_finalize", s, conv::finalize_il<<<grid, 256, 0, s>>>(g, *p, partial));
    else
      MKO_TIMED("conv1d_finalize", s, conv::finalize<<<grid, 256, 0, s>>>(g, *p, partial));
  }
  return mko_check_launch("conv1d_bwd");
}

extern "C" int mko_conv1d_update(const mko_conv1d_update_params* p, void* stream) {
  if (!p) {
    mko_set_error("conv1d_update: null parameters");
    return MKO_EINVAL;
  }
  if (p->batch < 0 || p->channels < 0 || p->q < 0 || p->width < 1 || p->span < p->width - 1) {
    mko_set_error("conv1d_update: bad sizes (span must be at least width - 1)");
    return MKO_EINVAL;
  }
  if (p->dtype != MKO_F32 && p->dtype != MKO_F16 && p->dtype != MKO_BF16) {
    mko_set_error("conv1d_update: unknown dtype %d", p->dtype);
    return MKO_EINVAL;
  }
  const int64_t rows = p->batch * p->channels;
  if (rows == 0 || p->q == 0) return MKO_OK;
  if (!p->x || !p->state || !p->weight || !p->out) {
    mko_set_error("conv1d_update: x, state, weight and out are required");
    return MKO_EINVAL;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  MKO_TIMED("conv1d_update", s, conv::update<<<static_cast<unsigned>((rows + 255) / 256), 256, 0, s>>>(*p));
  return mko_check_launch("conv1d_update");
}
