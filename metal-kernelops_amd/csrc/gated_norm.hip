// Gated RMSNorm (the normalisation between the SSM scan and the output projection of a
// Mamba-2 block) for gfx950.
//
// Per (row, group) of `group` consecutive features, with s(z) = silu(z):
//   x' = x s(z) (gate before) or x;   r = 1 / sqrt(mean(x'^2) + eps)
//   y  = (x' r w + b) s(z) (gate after) or x' r w + b
// Backward, with xh = x' r and g = dy s(z) (gate after) or dy:
//   c1 = sum(xh g w) / group,   dx' = r (g w - xh c1)
//   gate before: dx = dx' s(z), dz = dx' x s'(z);   gate after: dx = dx', dz = dy (xh w + b) s'(z)
//   dw = sum over rows of g xh,  db = sum over rows of g
//
// A team of whole waves owns one group.  Its thread lt holds the vectors lt + k * tw
// (k < NV) of VEC consecutive features -- one 16-byte load when the group is aligned,
// so a wave's loads at one k are 1 KB contiguous -- in registers from the load to the
// store.  The forward team normalises one (row, group): x and z are read once and y
// written once.  The backward team walks a block of rows of one group, prefetching
// the next row while it works on the current one, and keeps dw/db for its columns in
// registers; the teams of a workgroup add theirs in LDS in a fixed order and the
// workgroup writes one partial row that `finalize` sums over the blocks in a fixed
// order, so the gradients are deterministic.
// Groups wider than the register set stream: the forward walks the group twice (sum
// of squares, then the write); the backward computes c1 per (row, group) in one kernel
// and dx/dz and the dw/db partials with one thread per vector column in another.
#include "common.hpp"

namespace mko {
namespace gnorm {
namespace {

constexpr int kMaxWaves = 16;       // waves per team: a team fits one 1024-thread workgroup
constexpr int kStream = 1024;       // threads of the streaming kernels' team
constexpr int kFwdElems = 32;       // register elements per thread, forward
constexpr int kBwdElems = 8;        // register elements per thread, backward
constexpr int kBwdTeamWaves = 8;    // waves per backward workgroup when teams are narrow
constexpr int kBwdWaveTarget = 8192;  // backward waves across the chip without parameter gradients
constexpr int kBwdWaveTargetParams = 4096;  // ... with them (each row block adds a partial row)
constexpr int kMaxBlocks = 4096;      // row blocks per group: two column-sum passes of 64 rows
constexpr int kColThreads = 256;    // workgroup of the per-column backward kernel

struct Geo {
  int64_t rows, features, group, ngroups, units;  // units = rows * ngroups
  int64_t nvec;     // vectors per group (group / vec)
  int tw, tpw;      // threads per team, teams per workgroup
  int64_t blocks;   // backward: row blocks per group (partial rows)
  int64_t rpb;      // backward: rows per block
  int gate, bias;
  int wd;           // dtype of weight and bias
  int want_dw, want_db;
  float eps;
};

__device__ __forceinline__ float silu_of(float z, float& sig) {
  sig = sigmoid(z);
  return z * sig;
}

// d silu / dz = s (1 + z (1 - s)) with s = sigmoid(z).
__device__ __forceinline__ float silu_slope(float z, float sig) { return sig * (1.0f + z * (1.0f - sig)); }

// VEC consecutive elements as loaded: 16 bytes, or one element when VEC is 1.
template <typename T, int VEC>
struct Raw {
  static constexpr int kWords = (VEC * static_cast<int>(sizeof(T)) + 3) / 4;
  uint32_t w[kWords];
};

template <typename T, int VEC>
__device__ __forceinline__ void zero(Raw<T, VEC>& r) {
#pragma unroll
  for (int i = 0; i < Raw<T, VEC>::kWords; ++i) r.w[i] = 0;
}

// Buffer resources: a descriptor (in SGPRs) over one row's group, addressed by 32-bit
// per-lane byte offsets that x, z, dy, dx and dz share.  The hardware range check makes
// a load at or past `bytes` return zero and drops such a store, which masks the lanes
// past the group and the teams without a row (bytes = 0).
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
typedef uint32_t v2u32 __attribute__((ext_vector_type(2)));
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kRsrcWord3);
}

template <typename T, int VEC>
__device__ __forceinline__ void bload(__amdgpu_buffer_rsrc_t r, uint32_t off, Raw<T, VEC>& o) {
  if constexpr (VEC * sizeof(T) == 16) {
    const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    o.w[0] = v.x;
    o.w[1] = v.y;
    o.w[2] = v.z;
    o.w[3] = v.w;
  } else if constexpr (sizeof(T) == 4) {
    o.w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  } else {
    o.w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  }
}

template <int VEC>
__device__ __forceinline__ void bload_param(__amdgpu_buffer_rsrc_t r, uint32_t off, float (&o)[VEC]) {
  if constexpr (VEC >= 4) {
#pragma unroll
    for (int i = 0; i < VEC / 4; ++i) {
      const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * i, 0, 0);
      o[4 * i] = __uint_as_float(v.x);
      o[4 * i + 1] = __uint_as_float(v.y);
      o[4 * i + 2] = __uint_as_float(v.z);
      o[4 * i + 3] = __uint_as_float(v.w);
    }
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) o[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off + 4 * i, 0, 0));
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void load_raw(const T* p, Raw<T, VEC>& r) {
  if constexpr (VEC * sizeof(T) == 16) {
    load_words(p, r.w);
  } else {
    static_assert(VEC == 1, "vectors are 16 bytes or one element");
    if constexpr (sizeof(T) == 4)
      r.w[0] = *reinterpret_cast<const uint32_t*>(p);
    else
      r.w[0] = *reinterpret_cast<const uint16_t*>(p);
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void unpack(const Raw<T, VEC>& r, float (&o)[VEC]) {
  if constexpr (sizeof(T) == 2 && VEC == 1) {
    float hi;
    unpack2<T>(r.w[0], o[0], hi);  // one element, in the low half
  } else {
    unpack_words<T, VEC>(r.w, o);
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const T* p, float (&o)[VEC]) {
  Raw<T, VEC> r;
  load_raw<T, VEC>(p, r);
  unpack<T, VEC>(r, o);
}

template <typename T, int VEC>
__device__ __forceinline__ void store_vec(T* p, const float (&v)[VEC]) {
  if constexpr (VEC * sizeof(T) == 16) {
    uint32_t w[4];
    pack_words<T, VEC>(v, w);
    store_words(p, w);
  } else {
    p[0] = from_f32<T>(v[0]);
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void bstore(__amdgpu_buffer_rsrc_t r, uint32_t off, const float (&v)[VEC]) {
  if constexpr (VEC * sizeof(T) == 16) {
    uint32_t u[4];
    pack_words<T, VEC>(v, u);
    __builtin_amdgcn_raw_buffer_store_b128(v4u32{u[0], u[1], u[2], u[3]}, r, off, 0, 0);
  } else if constexpr (sizeof(T) == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[0]), r, off, 0, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, from_f32<T>(v[0])), r, off, 0, 0);
  }
}

// VEC float32 parameters (weight, bias) starting at p.
template <int VEC>
__device__ __forceinline__ void load_param(const float* p, float (&o)[VEC]) {
  if constexpr (VEC >= 4) {
#pragma unroll
    for (int i = 0; i < VEC / 4; ++i) {
      const float4 v = reinterpret_cast<const float4*>(p)[i];
      o[4 * i] = v.x;
      o[4 * i + 1] = v.y;
      o[4 * i + 2] = v.z;
      o[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) o[i] = p[i];
  }
}

// 16-bit weights packed two to a word, as float32.
template <int VEC>
__device__ __forceinline__ void unpack16(const uint32_t (&w)[(VEC + 1) / 2], bool bf, float (&o)[VEC]) {
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const uint32_t h = (i & 1) ? (w[i / 2] >> 16) : (w[i / 2] & 0xffffu);
    o[i] = bf ? __uint_as_float(h << 16) : static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
  }
}

// VEC consecutive weights from element `elem` of a buffer of dtype `wd`, as float32.
template <int VEC>
__device__ __forceinline__ void bload_w(__amdgpu_buffer_rsrc_t r, uint32_t elem, int wd, float (&o)[VEC]) {
  if (wd == MKO_F32) {
    bload_param<VEC>(r, elem * 4, o);
    return;
  }
  uint32_t w[(VEC + 1) / 2];
  const uint32_t off = elem * 2;
  if constexpr (VEC == 8) {
    const v4u32 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    w[0] = v.x;
    w[1] = v.y;
    w[2] = v.z;
    w[3] = v.w;
  } else if constexpr (VEC == 4) {
    const v2u32 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    w[0] = v.x;
    w[1] = v.y;
  } else {
    static_assert(VEC == 1, "weights come in 1, 4 or 8");
    w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  }
  unpack16<VEC>(w, wd == MKO_BF16, o);
}

template <int VEC>
__device__ __forceinline__ void load_w(const void* p, int wd, int64_t elem, float (&o)[VEC]) {
  if (wd == MKO_F32) {
    load_param<VEC>(static_cast<const float*>(p) + elem, o);
    return;
  }
  const uint16_t* q = static_cast<const uint16_t*>(p) + elem;
  uint32_t w[(VEC + 1) / 2];
  if constexpr (VEC >= 4)
    load_words(q, w);
  else
    w[0] = q[0];
  unpack16<VEC>(w, wd == MKO_BF16, o);
}

template <int VEC>
__device__ __forceinline__ void store_param(float* p, const float (&v)[VEC]) {
  if constexpr (VEC >= 4) {
#pragma unroll
    for (int i = 0; i < VEC / 4; ++i)
      reinterpret_cast<float4*>(p)[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) p[i] = v[i];
  }
}

// Sum over the tw / 64 waves of a team, the waves added in order.  Every wave of the
// workgroup calls it the same number of times (the barrier); `slots` holds one float
// per wave and is not written again before the next barrier of the caller.
__device__ __forceinline__ float team_sum(float v, float* slots, int tw, int team) {
  v = wave_sum(v);
  if (tw == kWave) return v;
  if ((threadIdx.x & (kWave - 1)) == 0) slots[threadIdx.x >> 6] = v;
  __syncthreads();
  const int wpt = tw >> 6;
  float t = 0.0f;
  for (int i = 0; i < wpt; ++i) t += slots[team * wpt + i];
  return t;
}

// ------------------------------------------------------------------ forward

template <typename T, int VEC, int NV, int GATE>
__global__ void __launch_bounds__(1024) forward(Geo g, mko_gated_norm_params p) {
  __shared__ float slots[kMaxWaves];
  constexpr uint32_t kVB = VEC * sizeof(T);  // bytes per vector
  const int team = uniform(static_cast<int>(threadIdx.x) / g.tw);
  const int lt = threadIdx.x - team * g.tw;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * g.tpw + team;
  const bool live = unit < g.units;
  const int64_t u = live ? unit : 0;
  const int64_t row = u / g.ngroups, gi = u - row * g.ngroups;
  const int64_t base = (row * g.features + gi * g.group) * static_cast<int64_t>(sizeof(T));
  const uint32_t bytes = live ? static_cast<uint32_t>(g.group * sizeof(T)) : 0u;
  constexpr bool gate = GATE != MKO_GATE_NONE;
  const auto rx = rsrc(static_cast<const char*>(p.x) + base, bytes);
  const auto rz = rsrc(gate ? static_cast<const char*>(p.z) + base : static_cast<const char*>(p.x), gate ? bytes : 0u);
  const int64_t wsz = g.wd == MKO_F32 ? 4 : 2;
  const auto rw = rsrc(static_cast<const char*>(p.weight) + gi * g.group * wsz, static_cast<uint32_t>(g.group * wsz));
  const auto rb = rsrc(p.bias ? static_cast<const char*>(p.bias) + gi * g.group * wsz : p.weight,
                       p.bias ? static_cast<uint32_t>(g.group * wsz) : 0u);

  float v[NV][VEC], w[NV][VEC];
  Raw<T, VEC> zr[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const uint32_t i = static_cast<uint32_t>(lt + k * g.tw);
    Raw<T, VEC> xr;
    bload<T, VEC>(rx, i * kVB, xr);
    if (gate) bload<T, VEC>(rz, i * kVB, zr[k]);
    unpack<T, VEC>(xr, v[k]);
  }
  // the weights are in flight during the reduction
#pragma unroll
  for (int k = 0; k < NV; ++k) bload_w<VEC>(rw, static_cast<uint32_t>(lt + k * g.tw) * VEC, g.wd, w[k]);
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    if (GATE == MKO_GATE_BEFORE) {
      float zf[VEC];
      unpack<T, VEC>(zr[k], zf);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float sig;
        v[k][e] *= silu_of(zf[e], sig);
      }
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) ss += v[k][e] * v[k][e];
  }
  const float r = rsqrtf(team_sum(ss, slots, g.tw, team) / static_cast<float>(g.group) + g.eps);
  if (!live) return;
  if (lt == 0 && p.rstd) p.rstd[u] = r;

  const auto ro = rsrc(static_cast<char*>(p.out) + base, bytes);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const uint32_t i = static_cast<uint32_t>(lt + k * g.tw);
    float o[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) o[e] = v[k][e] * r * w[k][e];
    if (p.bias) {
      float b[VEC];
      bload_w<VEC>(rb, i * VEC, g.wd, b);
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] += b[e];
    }
    if (GATE == MKO_GATE_AFTER) {
      float zf[VEC];
      unpack<T, VEC>(zr[k], zf);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float sig;
        o[e] *= silu_of(zf[e], sig);
      }
    }
    bstore<T, VEC>(ro, i * kVB, o);
  }
}

// One 1024-thread team per (row, group), walking the group twice.
template <typename T, int VEC>
__global__ void __launch_bounds__(kStream) forward_stream(Geo g, mko_gated_norm_params p) {
  __shared__ float slots[kMaxWaves];
  const int64_t u = blockIdx.x;
  const int64_t row = u / g.ngroups, gi = u - row * g.ngroups;
  const int64_t base = row * g.features + gi * g.group;
  const T* x = static_cast<const T*>(p.x) + base;
  const T* z = static_cast<const T*>(p.z) + base;
  float ss = 0.0f;
  for (int64_t i = threadIdx.x; i < g.nvec; i += kStream) {
    float v[VEC];
    load_vec<T, VEC>(x + i * VEC, v);
    if (g.gate == MKO_GATE_BEFORE) {
      float zf[VEC];
      load_vec<T, VEC>(z + i * VEC, zf);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float sig;
        v[e] *= silu_of(zf[e], sig);
      }
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) ss += v[e] * v[e];
  }
  const float r = rsqrtf(team_sum(ss, slots, kStream, 0) / static_cast<float>(g.group) + g.eps);
  if (threadIdx.x == 0 && p.rstd) p.rstd[u] = r;
  T* out = static_cast<T*>(p.out) + base;
  const int64_t col0 = gi * g.group;
  for (int64_t i = threadIdx.x; i < g.nvec; i += kStream) {
    float v[VEC], zf[VEC], w[VEC];
    load_vec<T, VEC>(x + i * VEC, v);
    if (g.gate != MKO_GATE_NONE) load_vec<T, VEC>(z + i * VEC, zf);
    load_w<VEC>(p.weight, g.wd, col0 + i * VEC, w);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float sig;
      const float s = g.gate != MKO_GATE_NONE ? silu_of(zf[e], sig) : 1.0f;
      if (g.gate == MKO_GATE_BEFORE) v[e] *= s;
      v[e] = v[e] * r * w[e];
    }
    if (p.bias) {
      float b[VEC];
      load_w<VEC>(p.bias, g.wd, col0 + i * VEC, b);
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] += b[e];
    }
    if (g.gate == MKO_GATE_AFTER) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float sig;
        v[e] *= silu_of(zf[e], sig);
      }
    }
    store_vec<T, VEC>(out + i * VEC, v);
  }
}

// ------------------------------------------------------------------ backward

// The per-element work of the backward before c1 is known: xh and g kept for the
// second half, c1's summand returned, dw/db accumulated, and (gate after) dz written.
// b is read with the gate after only.
template <int GATE, int VEC>
__device__ __forceinline__ float bwd_first(float r, const float (&x)[VEC], const float (&z)[VEC],
                                           const float (&dy)[VEC], const float (&w)[VEC], const float (&b)[VEC],
                                           float (&xh)[VEC], float (&gg)[VEC], float (&dw)[VEC], float (&db)[VEC],
                                           float (&dz)[VEC]) {
  float c = 0.0f;
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    float sig = 0.0f, s = 1.0f;
    if (GATE != MKO_GATE_NONE) s = silu_of(z[e], sig);
    const float xp = GATE == MKO_GATE_BEFORE ? x[e] * s : x[e];
    xh[e] = xp * r;
    gg[e] = GATE == MKO_GATE_AFTER ? dy[e] * s : dy[e];
    if (GATE == MKO_GATE_AFTER) dz[e] = dy[e] * (xh[e] * w[e] + b[e]) * silu_slope(z[e], sig);
    c += xh[e] * gg[e] * w[e];
    dw[e] += gg[e] * xh[e];
    db[e] += gg[e];
  }
  return c;
}

// dx (and, gate before, dz) once c1 is known.
template <int GATE, int VEC>
__device__ __forceinline__ void bwd_second(float r, float c1, const float (&x)[VEC],
                                           const float (&z)[VEC], const float (&w)[VEC], const float (&xh)[VEC],
                                           const float (&gg)[VEC], float (&dx)[VEC], float (&dz)[VEC]) {
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    const float dxp = (gg[e] * w[e] - xh[e] * c1) * r;
    if (GATE == MKO_GATE_BEFORE) {
      float sig;
      const float s = silu_of(z[e], sig);
      dz[e] = dxp * x[e] * silu_slope(z[e], sig);
      dx[e] = dxp * s;
    } else {
      dx[e] = dxp;
    }
  }
}

template <typename T, int VEC>
struct RowIn {
  Raw<T, VEC> x, z, dy;
};

// Workgroup = tpw teams of one group; block blockIdx.x / ngroups of rpb rows, the team
// taking rows team, team + tpw, ... of it.  Dynamic LDS: 2 * group floats when tpw > 1.
template <typename T, int VEC, int NV, int GATE>
__global__ void __launch_bounds__(1024) backward(Geo g, mko_gated_norm_params p, float* part) {
  __shared__ float slots[2][kMaxWaves];
  extern __shared__ float comb[];
  constexpr uint32_t kVB = VEC * sizeof(T);
  const int team = uniform(static_cast<int>(threadIdx.x) / g.tw);
  const int lt = threadIdx.x - team * g.tw;
  const int64_t blk = blockIdx.x / g.ngroups, gi = blockIdx.x - blk * g.ngroups;
  const int64_t r0 = blk * g.rpb;
  const int64_t r1 = r0 + g.rpb < g.rows ? r0 + g.rpb : g.rows;
  const int iters = static_cast<int>((g.rpb + g.tpw - 1) / g.tpw);
  const int64_t col0 = gi * g.group;
  const uint32_t gbytes = static_cast<uint32_t>(g.group * sizeof(T));
  constexpr bool gate = GATE != MKO_GATE_NONE;
  const float inv_group = 1.0f / static_cast<float>(g.group);

  float w[NV][VEC], b[NV][VEC], dw[NV][VEC], db[NV][VEC];
  {
    const int64_t wsz = g.wd == MKO_F32 ? 4 : 2;
    const auto rw = rsrc(static_cast<const char*>(p.weight) + col0 * wsz, static_cast<uint32_t>(g.group * wsz));
    const auto rb = rsrc(p.bias ? static_cast<const char*>(p.bias) + col0 * wsz : p.weight,
                         p.bias ? static_cast<uint32_t>(g.group * wsz) : 0u);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const uint32_t elem = static_cast<uint32_t>(lt + k * g.tw) * VEC;
      bload_w<VEC>(rw, elem, g.wd, w[k]);
      if constexpr (GATE == MKO_GATE_AFTER) bload_w<VEC>(rb, elem, g.wd, b[k]);
#pragma unroll
      for (int e = 0; e < VEC; ++e) dw[k][e] = db[k][e] = 0.0f;
    }
  }

  // the row's group in each tensor; no row: zero bytes, so loads read 0 and stores drop
  const auto row_rsrc = [&](const void* t, int64_t row, bool live) {
    const int64_t off = (live ? row * g.features + col0 : 0) * static_cast<int64_t>(sizeof(T));
    return rsrc(static_cast<const char*>(t) + off, live ? gbytes : 0u);
  };
  const auto load_row = [&](int64_t row, bool live, RowIn<T, VEC>(&in)[NV]) {
    const auto rx = row_rsrc(p.x, row, live);
    const auto rd = row_rsrc(p.dout, row, live);
    const auto rz = row_rsrc(gate ? p.z : p.x, row, live && gate);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const uint32_t off = static_cast<uint32_t>(lt + k * g.tw) * kVB;
      bload<T, VEC>(rx, off, in[k].x);
      bload<T, VEC>(rd, off, in[k].dy);
      if constexpr (gate) {
        bload<T, VEC>(rz, off, in[k].z);
      } else {
        zero(in[k].z);
      }
    }
  };

  RowIn<T, VEC> cur[NV], nxt[NV];
  int64_t row = r0 + team;
  bool live = row < r1;
  load_row(row, live, cur);
  float r = live ? p.rstd[row * g.ngroups + gi] : 0.0f;

  for (int it = 0; it < iters; ++it) {
    const int64_t nrow = row + g.tpw;
    const bool nlive = nrow < r1;
    load_row(nrow, nlive, nxt);
    const float nr = nlive ? p.rstd[nrow * g.ngroups + gi] : 0.0f;

    const auto rdx = row_rsrc(p.dx, row, live);
    const auto rdz = row_rsrc(gate ? p.dz : p.dx, row, live && gate);
    float xh[NV][VEC], gg[NV][VEC];
    float c = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      float xs[VEC], zs[VEC], dy[VEC], dz[VEC];
      unpack<T, VEC>(cur[k].x, xs);
      unpack<T, VEC>(cur[k].z, zs);
      unpack<T, VEC>(cur[k].dy, dy);
      // past the group or without a row x, z, dy (and r) are zero, so xh, g and what
      // they add to c, dw and db are too
      c += bwd_first<GATE, VEC>(r, xs, zs, dy, w[k], b[k], xh[k], gg[k], dw[k], db[k], dz);
      if (GATE == MKO_GATE_AFTER) bstore<T, VEC>(rdz, static_cast<uint32_t>(lt + k * g.tw) * kVB, dz);
    }
    const float c1 = team_sum(c, slots[it & 1], g.tw, team) * inv_group;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const uint32_t off = static_cast<uint32_t>(lt + k * g.tw) * kVB;
      // x and z again from the loaded row (fewer live registers than keeping floats)
      float xs[VEC], zs[VEC], dx[VEC], dz[VEC];
      unpack<T, VEC>(cur[k].x, xs);
      unpack<T, VEC>(cur[k].z, zs);
      bwd_second<GATE, VEC>(r, c1, xs, zs, w[k], xh[k], gg[k], dx, dz);
      bstore<T, VEC>(rdx, off, dx);
      if (GATE == MKO_GATE_BEFORE) bstore<T, VEC>(rdz, off, dz);
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) cur[k] = nxt[k];
    row = nrow;
    live = nlive;
    r = nr;
  }

  if (!g.want_dw && !g.want_db) return;
  float* pw = part + blk * g.features + col0;
  float* pb = part + (g.blocks + blk) * g.features + col0;
  if (g.tpw == 1) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int64_t i = lt + static_cast<int64_t>(k) * g.tw;
      if (i >= g.nvec) continue;
      if (g.want_dw) store_param<VEC>(pw + i * VEC, dw[k]);
      if (g.want_db) store_param<VEC>(pb + i * VEC, db[k]);
    }
    return;
  }
  // teams add into LDS one after another, team 0 first
  float* cw = comb;
  float* cb = comb + g.group;
  for (int t = 0; t < g.tpw; ++t) {
    if (team == t) {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int64_t i = lt + static_cast<int64_t>(k) * g.tw;
        if (i >= g.nvec) continue;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const int64_t j = i * VEC + e;
          cw[j] = t == 0 ? dw[k][e] : cw[j] + dw[k][e];
          cb[j] = t == 0 ? db[k][e] : cb[j] + db[k][e];
        }
      }
    }
    __syncthreads();
  }
  for (int64_t j = threadIdx.x; j < g.group; j += blockDim.x) {
    if (g.want_dw) pw[j] = cw[j];
    if (g.want_db) pb[j] = cb[j];
  }
}

// Wide groups, first kernel: c1 of one (row, group) per 1024-thread team.
template <typename T, int VEC>
__global__ void __launch_bounds__(kStream) c1_stream(Geo g, mko_gated_norm_params p, float* c1out) {
  __shared__ float slots[kMaxWaves];
  const int64_t u = blockIdx.x;
  const int64_t row = u / g.ngroups, gi = u - row * g.ngroups;
  const int64_t base = row * g.features + gi * g.group;
  const float r = p.rstd[u];
  float c = 0.0f;
  for (int64_t i = threadIdx.x; i < g.nvec; i += kStream) {
    float x[VEC], z[VEC], dy[VEC], w[VEC];
    load_vec<T, VEC>(static_cast<const T*>(p.x) + base + i * VEC, x);
    load_vec<T, VEC>(static_cast<const T*>(p.dout) + base + i * VEC, dy);
    if (g.gate != MKO_GATE_NONE) load_vec<T, VEC>(static_cast<const T*>(p.z) + base + i * VEC, z);
    load_w<VEC>(p.weight, g.wd, gi * g.group + i * VEC, w);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float sig;
      const float s = g.gate != MKO_GATE_NONE ? silu_of(z[e], sig) : 1.0f;
      const float xh = (g.gate == MKO_GATE_BEFORE ? x[e] * s : x[e]) * r;
      const float gv = g.gate == MKO_GATE_AFTER ? dy[e] * s : dy[e];
      c += xh * gv * w[e];
    }
  }
  const float t = team_sum(c, slots, kStream, 0);
  if (threadIdx.x == 0) c1out[u] = t / static_cast<float>(g.group);
}

// Wide groups, second kernel: one thread per vector column of one row block writes dx
// and dz down the block and one dw/db partial.
template <typename T, int VEC>
__global__ void __launch_bounds__(kColThreads) columns(Geo g, mko_gated_norm_params p, const float* c1v,
                                                       float* part) {
  const int64_t cols = g.features / VEC;
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kColThreads + threadIdx.x;
  const int64_t blk = e0 / cols, j = e0 - blk * cols;
  if (blk >= g.blocks) return;
  const int64_t f0 = j * VEC, gi = f0 / g.group;
  float w[VEC], b[VEC], dw[VEC], db[VEC];
  load_w<VEC>(p.weight, g.wd, f0, w);
#pragma unroll
  for (int e = 0; e < VEC; ++e) b[e] = dw[e] = db[e] = 0.0f;
  if (p.bias) load_w<VEC>(p.bias, g.wd, f0, b);
  const int64_t r0 = blk * g.rpb;
  const int64_t r1 = r0 + g.rpb < g.rows ? r0 + g.rpb : g.rows;
  for (int64_t row = r0; row < r1; ++row) {
    const int64_t off = row * g.features + f0;
    const float r = p.rstd[row * g.ngroups + gi];
    const float c1 = c1v[row * g.ngroups + gi];
    float x[VEC], z[VEC], dy[VEC], xh[VEC], gg[VEC], dx[VEC], dz[VEC];
    load_vec<T, VEC>(static_cast<const T*>(p.x) + off, x);
    load_vec<T, VEC>(static_cast<const T*>(p.dout) + off, dy);
    if (g.gate != MKO_GATE_NONE) {
      load_vec<T, VEC>(static_cast<const T*>(p.z) + off, z);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) z[e] = 0.0f;
    }
    if (g.gate == MKO_GATE_NONE)
      bwd_first<MKO_GATE_NONE, VEC>(r, x, z, dy, w, b, xh, gg, dw, db, dz);
    else if (g.gate == MKO_GATE_BEFORE)
      bwd_first<MKO_GATE_BEFORE, VEC>(r, x, z, dy, w, b, xh, gg, dw, db, dz);
    else
      bwd_first<MKO_GATE_AFTER, VEC>(r, x, z, dy, w, b, xh, gg, dw, db, dz);
    if (g.gate == MKO_GATE_AFTER) store_vec<T, VEC>(static_cast<T*>(p.dz) + off, dz);
    if (g.gate == MKO_GATE_BEFORE)
      bwd_second<MKO_GATE_BEFORE, VEC>(r, c1, x, z, w, xh, gg, dx, dz);
    else
      bwd_second<MKO_GATE_NONE, VEC>(r, c1, x, z, w, xh, gg, dx, dz);
    store_vec<T, VEC>(static_cast<T*>(p.dx) + off, dx);
    if (g.gate == MKO_GATE_BEFORE) store_vec<T, VEC>(static_cast<T*>(p.dz) + off, dz);
  }
  if (g.want_dw) store_param<VEC>(part + blk * g.features + f0, dw);
  if (g.want_db) store_param<VEC>(part + (g.blocks + blk) * g.features + f0, db);
}

// dweight and dbias from the partial rows: column sums of a (rows, cols) float32 matrix,
// 64 rows by 64 columns per workgroup.  Wave v adds rows 16 v .. 16 v + 15 of the
// workgroup's 64 in order (the 16 loads issued together), then the four wave sums are
// added in order into out[blockIdx.y][col]; a second pass over the per-64-row sums
// finishes blocks > 64.  The order is fixed, so the sums are deterministic.
constexpr int kSumRows = 64;

__global__ void __launch_bounds__(256) colsum(const float* in, int64_t rows, int64_t cols, float* out) {
  __shared__ float s[4][kWave];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * kWave + lane;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * kSumRows + wave * 16;
  float a = 0.0f;
  if (col < cols) {
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = r0 + j < rows ? in[(r0 + j) * cols + col] : 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) a += v[j];
  }
  s[wave][lane] = a;
  __syncthreads();
  if (wave == 0 && col < cols) out[blockIdx.y * cols + col] = (s[0][lane] + s[1][lane]) + (s[2][lane] + s[3][lane]);
}

// ------------------------------------------------------------------ host side

enum Path { kDense = 0, kWide = 1 };

struct Plan {
  Geo g;
  int vec, nv, path;
};

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

int pow2_at_least(int64_t v) {
  int p = 1;
  while (p < v) p *= 2;
  return p;
}

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

int check_common(const mko_gated_norm_params* p, const char* what) {
  if (!p) {
    mko_set_error("%s: null parameters", what);
    return MKO_EINVAL;
  }
  if (p->rows < 0 || p->features < 0 || p->group < 1 || (p->features > 0 && p->features % p->group != 0)) {
    mko_set_error("%s: bad sizes rows=%lld features=%lld group=%lld (group must divide features)", what,
                  static_cast<long long>(p->rows), static_cast<long long>(p->features),
                  static_cast<long long>(p->group));
    return MKO_EINVAL;
  }
  if (p->dtype != MKO_F32 && p->dtype != MKO_F16 && p->dtype != MKO_BF16) {
    mko_set_error("%s: unknown dtype %d", what, p->dtype);
    return MKO_EINVAL;
  }
  if (p->wdtype != MKO_F32 && p->wdtype != MKO_F16 && p->wdtype != MKO_BF16) {
    mko_set_error("%s: unknown weight dtype %d", what, p->wdtype);
    return MKO_EINVAL;
  }
  if (p->gate != MKO_GATE_NONE && p->gate != MKO_GATE_BEFORE && p->gate != MKO_GATE_AFTER) {
    mko_set_error("%s: unknown gate %d", what, p->gate);
    return MKO_EINVAL;
  }
  if (!(p->eps >= 0.0f)) {
    mko_set_error("%s: eps must be a non-negative number", what);
    return MKO_EINVAL;
  }
  return MKO_OK;
}

// Vector width, register depth and team shape for one direction.
Plan make_plan(const mko_gated_norm_params* p, bool bwd) {
  Plan pl{};
  Geo& g = pl.g;
  const int esize = p->dtype == MKO_F32 ? 4 : 2;
  g.rows = p->rows;
  g.features = p->features;
  g.group = p->group;
  g.ngroups = p->features / p->group;
  g.units = g.rows * g.ngroups;
  g.gate = p->gate;
  g.bias = p->bias != nullptr;
  g.wd = p->wdtype;
  g.eps = p->eps;
  g.want_dw = bwd && p->dweight != nullptr;
  g.want_db = bwd && p->dbias != nullptr;

  const int vmax = 16 / esize;
  bool vec = p->group % vmax == 0 && aligned16(p->x) && aligned16(p->weight) && (!p->bias || aligned16(p->bias)) &&
             (p->gate == MKO_GATE_NONE || aligned16(p->z));
  if (bwd)
    vec = vec && aligned16(p->dout) && aligned16(p->dx) && (p->gate == MKO_GATE_NONE || aligned16(p->dz));
  else
    vec = vec && aligned16(p->out);
  pl.vec = vec ? vmax : 1;
  g.nvec = g.group / pl.vec;

  // vectors per thread: VEC * NV register elements at most, and (one element per
  // vector, one offset register each) at most 8 forward, 4 backward
  const int elems = bwd ? kBwdElems : kFwdElems;
  const int nvcap = bwd ? 4 : 8;
  const int nvmax = elems / pl.vec < nvcap ? (elems / pl.vec < 1 ? 1 : elems / pl.vec) : nvcap;
  if (g.nvec > static_cast<int64_t>(kMaxWaves) * kWave * nvmax) {
    pl.path = kWide;
    g.tw = kStream;
    g.tpw = 1;
  } else {
    pl.path = kDense;
    // aim at two vectors per thread, then as few vectors as cover the group evenly
    int64_t waves = cdiv(g.nvec, static_cast<int64_t>(kWave) * (nvmax < 2 ? nvmax : 2));
    waves = waves < 1 ? 1 : (waves > kMaxWaves ? kMaxWaves : waves);
    pl.nv = pow2_at_least(cdiv(g.nvec, kWave * waves));
    waves = cdiv(g.nvec, static_cast<int64_t>(kWave) * pl.nv);
    g.tw = static_cast<int>(waves) * kWave;
    const int wg_waves = bwd ? kBwdTeamWaves : 4;
    g.tpw = waves >= wg_waves ? 1 : static_cast<int>(wg_waves / waves);
  }
  if (bwd) {
    if (pl.path == kDense) {
      const int64_t wg_waves = static_cast<int64_t>(g.tpw) * (g.tw / kWave);
      const int64_t target = g.want_dw || g.want_db ? kBwdWaveTargetParams : kBwdWaveTarget;
      int64_t blocks = cdiv(cdiv(target, wg_waves), g.ngroups);
      blocks = blocks > kMaxBlocks ? kMaxBlocks : blocks;
      const int64_t most = cdiv(g.rows, g.tpw);
      blocks = blocks > most ? most : blocks;
      blocks = blocks < 1 ? 1 : blocks;
      g.rpb = cdiv(g.rows, blocks);
      g.blocks = cdiv(g.rows, g.rpb);
    } else {
      // one thread per vector column: enough row blocks for ~64K threads
      const int64_t cols = g.features / pl.vec;
      int64_t blocks = cdiv(65536, cols);
      blocks = blocks > g.rows ? g.rows : blocks;
      blocks = blocks > kMaxBlocks ? kMaxBlocks : blocks;
      blocks = blocks < 1 ? 1 : blocks;
      g.rpb = cdiv(g.rows, blocks);
      g.blocks = cdiv(g.rows, g.rpb);
    }
  }
  return pl;
}

// Workspace: the dw/db partial rows (2 x blocks x features), their per-64-row sums when
// blocks > 64 (2 x sums x features), and c1 per (row, group) on the wide path.
int64_t sum_rows(const Geo& g) { return g.blocks > kSumRows ? cdiv(g.blocks, kSumRows) : 0; }

size_t workspace_bytes(const Plan& pl) {
  const Geo& g = pl.g;
  size_t n = 0;
  if (g.want_dw || g.want_db) n += static_cast<size_t>(2 * (g.blocks + sum_rows(g)) * g.features) * sizeof(float);
  if (pl.path == kWide) n += static_cast<size_t>(g.units) * sizeof(float);
  return n;
}

// dst = column sums of the (rows, features) partials: one colsum pass for rows <= 64,
// two (through `tmp`, cdiv(rows, 64) rows) otherwise.
void column_sums(const float* part, int64_t rows, int64_t features, float* tmp, float* dst, hipStream_t s) {
  const unsigned gx = static_cast<unsigned>(cdiv(features, kWave));
  if (rows <= kSumRows) {
    colsum<<<dim3(gx, 1), 256, 0, s>>>(part, rows, features, dst);
    return;
  }
  const int64_t mid = cdiv(rows, kSumRows);
  colsum<<<dim3(gx, static_cast<unsigned>(mid)), 256, 0, s>>>(part, rows, features, tmp);
  colsum<<<dim3(gx, 1), 256, 0, s>>>(tmp, mid, features, dst);
}

template <typename T, int VEC, int NV>
int launch_fwd_t(const Plan& pl, const mko_gated_norm_params& p, hipStream_t s) {
  const Geo& g = pl.g;
  const unsigned grid = static_cast<unsigned>(cdiv(g.units, g.tpw));
  const unsigned block = static_cast<unsigned>(g.tw * g.tpw);
  if (g.gate == MKO_GATE_NONE)
    MKO_TIMED("gated_norm_fwd", s, forward<T, VEC, NV, MKO_GATE_NONE><<<grid, block, 0, s>>>(g, p));
  else if (g.gate == MKO_GATE_BEFORE)
    MKO_TIMED("gated_norm_fwd", s, forward<T, VEC, NV, MKO_GATE_BEFORE><<<grid, block, 0, s>>>(g, p));
  else
    MKO_TIMED("gated_norm_fwd", s, forward<T, VEC, NV, MKO_GATE_AFTER><<<grid, block, 0, s>>>(g, p));
  return MKO_OK;
}

int bad_plan(const Plan& pl) {
  mko_set_error("gated_norm: no kernel for vec=%d nv=%d", pl.vec, pl.nv);
  return MKO_EUNSUPPORTED;
}

template <typename T, int VEC>
int launch_fwd_v(const Plan& pl, const mko_gated_norm_params& p, hipStream_t s) {
  if (pl.path == kWide) {
    MKO_TIMED("gated_norm_fwd_stream", s,
              forward_stream<T, VEC><<<static_cast<unsigned>(pl.g.units), kStream, 0, s>>>(pl.g, p));
    return MKO_OK;
  }
  // register depth: VEC * NV <= kFwdElems, NV <= 8
  if (pl.nv == 1) return launch_fwd_t<T, VEC, 1>(pl, p, s);
  if (pl.nv == 2) return launch_fwd_t<T, VEC, 2>(pl, p, s);
  if (pl.nv == 4) return launch_fwd_t<T, VEC, 4>(pl, p, s);
  if constexpr (VEC * 8 <= kFwdElems) {
    if (pl.nv == 8) return launch_fwd_t<T, VEC, 8>(pl, p, s);
  }
  return bad_plan(pl);
}

template <typename T>
int launch_fwd(const Plan& pl, const mko_gated_norm_params& p, hipStream_t s) {
  if (pl.vec == 1) return launch_fwd_v<T, 1>(pl, p, s);
  return launch_fwd_v<T, 16 / sizeof(T)>(pl, p, s);
}

template <typename T, int VEC, int NV>
int launch_bwd_t(const Plan& pl, const mko_gated_norm_params& p, float* part, hipStream_t s) {
  const Geo& g = pl.g;
  const unsigned grid = static_cast<unsigned>(g.blocks * g.ngroups);
  const unsigned block = static_cast<unsigned>(g.tw * g.tpw);
  const size_t lds = g.tpw > 1 ? static_cast<size_t>(2 * g.group) * sizeof(float) : 0;
  if (g.gate == MKO_GATE_NONE)
    MKO_TIMED("gated_norm_bwd", s, backward<T, VEC, NV, MKO_GATE_NONE><<<grid, block, lds, s>>>(g, p, part));
  else if (g.gate == MKO_GATE_BEFORE)
    MKO_TIMED("gated_norm_bwd", s, backward<T, VEC, NV, MKO_GATE_BEFORE><<<grid, block, lds, s>>>(g, p, part));
  else
    MKO_TIMED("gated_norm_bwd", s, backward<T, VEC, NV, MKO_GATE_AFTER><<<grid, block, lds, s>>>(g, p, part));
  return MKO_OK;
}

template <typename T, int VEC>
int launch_bwd_v(const Plan& pl, const mko_gated_norm_params& p, float* part, float* c1, hipStream_t s) {
  const Geo& g = pl.g;
  if (pl.path == kWide) {
    MKO_TIMED("gated_norm_bwd_c1", s,
              c1_stream<T, VEC><<<static_cast<unsigned>(g.units), kStream, 0, s>>>(g, p, c1));
    const int64_t n = g.blocks * (g.features / VEC);
    MKO_TIMED("gated_norm_bwd_columns", s,
              columns<T, VEC><<<static_cast<unsigned>(cdiv(n, kColThreads)), kColThreads, 0, s>>>(g, p, c1, part));
    return MKO_OK;
  }
  // register depth: VEC * NV <= kBwdElems
  if (pl.nv == 1) return launch_bwd_t<T, VEC, 1>(pl, p, part, s);
  if constexpr (VEC * 2 <= kBwdElems) {
    if (pl.nv == 2) return launch_bwd_t<T, VEC, 2>(pl, p, part, s);
  }
  if constexpr (VEC * 4 <= kBwdElems) {
    if (pl.nv == 4) return launch_bwd_t<T, VEC, 4>(pl, p, part, s);
  }
  return bad_plan(pl);
}

template <typename T>
int launch_bwd(const Plan& pl, const mko_gated_norm_params& p, float* part, float* c1, hipStream_t s) {
  if (pl.vec == 1) return launch_bwd_v<T, 1>(pl, p, part, c1, s);
  return launch_bwd_v<T, 16 / sizeof(T)>(pl, p, part, c1, s);
}

}  // namespace
}  // namespace gnorm
}  // namespace mko

using namespace mko;

extern "C" size_t mko_sizeof_gated_norm_params(void) { return sizeof(mko_gated_norm_params); }

extern "C" int mko_gated_norm_fwd(const mko_gated_norm_params* p, void* stream) {
  int st = gnorm::check_common(p, "gated_norm_fwd");
  if (st != MKO_OK) return st;
  if (p->rows == 0 || p->features == 0) return MKO_OK;
  if (!p->x || !p->weight || !p->out || (p->gate != MKO_GATE_NONE && !p->z)) {
    mko_set_error("gated_norm_fwd: x, weight, out (and z with a gate) are required");
    return MKO_EINVAL;
  }
  const gnorm::Plan pl = gnorm::make_plan(p, false);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (p->dtype == MKO_F32)
    st = gnorm::launch_fwd<float>(pl, *p, s);
  else if (p->dtype == MKO_BF16)
    st = gnorm::launch_fwd<bf16>(pl, *p, s);
  else
    st = gnorm::launch_fwd<_Float16>(pl, *p, s);
  if (st != MKO_OK) return st;
  return mko_check_launch("gated_norm_fwd");
}

extern "C" size_t mko_gated_norm_bwd_workspace_size(const mko_gated_norm_params* p) {
  if (gnorm::check_common(p, "gated_norm_bwd") != MKO_OK) return 0;
  if (p->rows == 0 || p->features == 0) return 0;
  return gnorm::workspace_bytes(gnorm::make_plan(p, true));
}

extern "C" int mko_gated_norm_bwd(const mko_gated_norm_params* p, void* stream) {
  int st = gnorm::check_common(p, "gated_norm_bwd");
  if (st != MKO_OK) return st;
  if (p->rows == 0 || p->features == 0) return MKO_OK;  // the caller zero-fills dweight/dbias
  if (!p->x || !p->weight || !p->rstd || !p->dout || !p->dx ||
      (p->gate != MKO_GATE_NONE && (!p->z || !p->dz))) {
    mko_set_error("gated_norm_bwd: x, weight, rstd, dout, dx (and z, dz with a gate) are required");
    return MKO_EINVAL;
  }
  const gnorm::Plan pl = gnorm::make_plan(p, true);
  const size_t need = gnorm::workspace_bytes(pl);
  if (need && (!p->workspace || p->workspace_bytes < need)) {
    mko_set_error("gated_norm_bwd: workspace of %zu bytes needed, %zu given", need, p->workspace_bytes);
    return MKO_EWORKSPACE;
  }
  const gnorm::Geo& g = pl.g;
  const bool params = g.want_dw || g.want_db;
  float* part = static_cast<float*>(p->workspace);
  float* sums = part + 2 * g.blocks * g.features;
  float* c1 = params ? sums + 2 * gnorm::sum_rows(g) * g.features : part;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (p->dtype == MKO_F32)
    st = gnorm::launch_bwd<float>(pl, *p, part, c1, s);
  else if (p->dtype == MKO_BF16)
    st = gnorm::launch_bwd<bf16>(pl, *p, part, c1, s);
  else
    st = gnorm::launch_bwd<_Float16>(pl, *p, part, c1, s);
  if (st != MKO_OK) return st;
  if (params) {
    const int64_t mid = gnorm::sum_rows(g) * g.features;
    MKO_TIMED("gated_norm_bwd_sums", s, {
      if (g.want_dw) gnorm::column_sums(part, g.blocks, g.features, sums, p->dweight, s);
      if (g.want_db) gnorm::column_sums(part + g.blocks * g.features, g.blocks, g.features, sums + mid, p->dbias, s);
    });
  }
  return mko_check_launch("gated_norm_bwd");
}
