// Four-path layout of the 2D selective scan (VMamba's ss2d) for gfx950.
//
// A (batch, rows, H, W) map is read along four paths; path k visits pixel pos_k(i)
// at step i of L = H * W:
//   k = 0: i                         row-major
//   k = 1: (i % H) * W + i / H       column-major: down each column, columns left to right
//   k = 2: L - 1 - i                 path 0 reversed
//   k = 3: pos_1(L - 1 - i)          path 1 reversed
// `stack` writes the four paths of every row in step order, (batch, 4 rows, L), the
// layout the 1-D scan kernels take (4x the channels, or 4x the groups of B/C); `merge`
// adds the four step-ordered slices back at each pixel, (s0 + s2) + (s1 + s3), the
// order of the reference's merge_paths (cv/path_scan.py:372-404).
//
// One lane per (batch, row, step) or (batch, row, pixel): the contiguous side is the
// one the lane index walks, the transposed paths gather with stride W (stack) or H
// (merge).  Every operand is L2-resident at the map sizes this layer sees.
#include "common.hpp"
#include "io.hpp"

namespace mko {
namespace path {
namespace {

struct Geo {
  int64_t batch, rows, height, width, length, total;  // total = batch * rows * length
  int dtype;
  float scale;
};

__global__ void __launch_bounds__(256) stack(Geo g, const void* __restrict__ src, void* __restrict__ dst) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= g.total) return;
  const int64_t i = e % g.length, br = e / g.length;
  const int64_t r = br % g.rows, b = br / g.rows;
  const int64_t L = g.length;
  const int64_t col = (i % g.height) * g.width + i / g.height;           // pos_1(i)
  const int64_t j = L - 1 - i;
  const int64_t rcol = (j % g.height) * g.width + j / g.height;          // pos_1(L - 1 - i)
  const int64_t in = br * L;
  const int64_t out = (b * 4 * g.rows + r) * L + i;
  const int64_t slice = g.rows * L;
  store_one(dst, g.dtype, out, g.scale * load_one(src, g.dtype, in + i));
  store_one(dst, g.dtype, out + slice, g.scale * load_one(src, g.dtype, in + col));
  store_one(dst, g.dtype, out + 2 * slice, g.scale * load_one(src, g.dtype, in + j));
  store_one(dst, g.dtype, out + 3 * slice, g.scale * load_one(src, g.dtype, in + rcol));
}

__global__ void __launch_bounds__(256) merge(Geo g, const void* __restrict__ src, void* __restrict__ dst) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= g.total) return;
  const int64_t pix = e % g.length, br = e / g.length;
  const int64_t r = br % g.rows, b = br / g.rows;
  const int64_t L = g.length;
  const int64_t h = pix / g.width, w = pix - h * g.width;
  const int64_t col = w * g.height + h;  // the step at which path 1 stands on pix
  const int64_t base = (b * 4 * g.rows + r) * L;
  const int64_t slice = g.rows * L;
  const float s0 = load_one(src, g.dtype, base + pix);
  const float s1 = load_one(src, g.dtype, base + slice + col);
  const float s2 = load_one(src, g.dtype, base + 2 * slice + (L - 1 - pix));
  const float s3 = load_one(src, g.dtype, base + 3 * slice + (L - 1 - col));
  store_one(dst, g.dtype, e, ((s0 + s2) + (s1 + s3)) * g.scale);
}

int make_geo(const mko_path_params* p, Geo* g, const char* what) {
  if (!p) {
    mko_set_error("%s: null parameters", what);
    return MKO_EINVAL;
  }
  if (p->batch < 0 || p->rows < 0 || p->height < 0 || p->width < 0) {
    mko_set_error("%s: negative extent", what);
    return MKO_EINVAL;
  }
  if (p->dtype != MKO_F32 && p->dtype != MKO_F16 && p->dtype != MKO_BF16) {
    mko_set_error("%s: unknown dtype %d", what, p->dtype);
    return MKO_EINVAL;
  }
  g->batch = p->batch;
  g->rows = p->rows;
  g->height = p->height;
  g->width = p->width;
  g->length = p->height * p->width;
  g->total = p->batch * p->rows * g->length;
  g->dtype = p->dtype;
  g->scale = p->scale;
  if (g->total > 0 && (!p->src || !p->dst)) {
    mko_set_error("%s: src and dst are required", what);
    return MKO_EINVAL;
  }
  if (g->total > (int64_t{1} << 40)) {
    mko_set_error("%s: %lld elements is beyond the supported size", what, static_cast<long long>(g->total));
    return MKO_EUNSUPPORTED;
  }
  return MKO_OK;
}

unsigned blocks(int64_t n) { return static_cast<unsigned>((n + 255) / 256); }

}  // namespace
}  // namespace path
}  // namespace mko

using namespace mko;

extern "C" size_t mko_sizeof_path_params(void) { return sizeof(mko_path_params); }

extern "C" int mko_path_stack(const mko_path_params* p, void* stream) {
  path::Geo g;
  const int st = path::make_geo(p, &g, "path_stack");
  if (st != MKO_OK || g.total == 0) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  MKO_TIMED("path_stack", s, path::stack<<<path::blocks(g.total), 256, 0, s>>>(g, p->src, p->dst));
  return mko_check_launch("path_stack");
}

extern "C" int mko_path_merge(const mko_path_params* p, void* stream) {
  path::Geo g;
  const int st = path::make_geo(p, &g, "path_merge");
  if (st != MKO_OK || g.total == 0) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  MKO_TIMED("path_merge", s, path::merge<<<path::blocks(g.total), 256, 0, s>>>(g, p->src, p->dst));
  return mko_check_launch("path_merge");
}
