// Shared declarations of the SSD chunk-scan kernels (ssd.hip, ssd_bwd.hip).
#pragma once

#include "common.hpp"

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
  // forward save area
  float* states;  // (b, H, nc, P, N) state entering each chunk
  float* dl;      // (b, H, nc, q) step sizes (0 past the end)
  float* cs;      // (b, H, nc, q) cumulative step * A inside the chunk
  float* cb;      // (b, nc, G, q, q) C . B^T, lower tiles
  // backward workspace
  float* dstates;  // (b, H, nc, P, N) adjoint of the state leaving each chunk
  float* dT;       // (b, H, nc, tiles) partial e^T <dS_out, S_in>
  float* dcs;      // (b, H, nc, q) d loss / d cs
  float* dsx;      // (b, H, nc, q) sum_p du * x (direct step gradient)
  float* pbc;      // (b, L, G, hblocks, N, 2) dB/dC partial sums over head blocks
  float* pdD;      // (b, nc, H, P) dD partials
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

}  // namespace ssd
}  // namespace mko
