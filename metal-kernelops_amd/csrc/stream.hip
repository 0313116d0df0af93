// A streaming device copy: the read-and-write rate of this part that the state-sized kernels
// are measured against, and the known-size traffic that calibrates the PMC byte counters.
//
// One workgroup of 256 lanes copies 16 KB: each lane issues its four 16-byte loads before any
// store, a wavefront's accesses are whole 1 KB runs, and the grid has a workgroup per 16 KB.
// On one MI355X, with 1 GiB copied: 6.25 TB/s of reads plus writes with the nontemporal hint on
// both, 5.74 TB/s without it; 4.2-4.3 TB/s at eight vectors per lane, 5.3-5.5 TB/s as a
// persistent grid of 1024-4096 workgroups, and torch's copy_ 5.0 TB/s.
#include "common.hpp"

namespace mko {
namespace stream {

constexpr int kLanes = 256;
constexpr int kVecs = 4;  // 16-byte vectors per lane

template <bool NT>
__global__ void __launch_bounds__(kLanes) copy16(const mko_u32x4* __restrict__ src, mko_u32x4* __restrict__ dst,
                                                  size_t nvec) {
  const size_t base = static_cast<size_t>(blockIdx.x) * (kLanes * kVecs) + threadIdx.x;
  mko_u32x4 v[kVecs];
#pragma unroll
  for (int i = 0; i < kVecs; ++i) {
    const size_t k = base + static_cast<size_t>(i) * kLanes;
    if (k < nvec) v[i] = NT ? __builtin_nontemporal_load(src + k) : src[k];
  }
#pragma unroll
  for (int i = 0; i < kVecs; ++i) {
    const size_t k = base + static_cast<size_t>(i) * kLanes;
    if (k < nvec) {
      if constexpr (NT)
        __builtin_nontemporal_store(v[i], dst + k);
      else
        dst[k] = v[i];
    }
  }
}

// The bytes past the last whole 16-byte vector (fewer than 16).
__global__ void copy_tail(const unsigned char* src, unsigned char* dst, size_t n) {
  if (threadIdx.x < n) dst[threadIdx.x] = src[threadIdx.x];
}

}  // namespace stream
}  // namespace mko

using namespace mko;

extern "C" int mko_stream_copy(const void* src, void* dst, size_t bytes, uint32_t flags, void* stream) {
  if (bytes == 0) return MKO_OK;
  if (!src || !dst) {
    mko_set_error("stream_copy: null pointer");
    return MKO_EINVAL;
  }
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) {
    mko_set_error("stream_copy: src and dst must be 16-byte aligned");
    return MKO_EINVAL;
  }
  if (flags & ~static_cast<uint32_t>(MKO_STREAM_NONTEMPORAL)) {
    mko_set_error("stream_copy: unknown flags 0x%x", flags);
    return MKO_EINVAL;
  }
  const char* s8 = static_cast<const char*>(src);
  char* d8 = static_cast<char*>(dst);
  if ((s8 < d8 + bytes) && (d8 < s8 + bytes)) {
    mko_set_error("stream_copy: src and dst overlap");
    return MKO_EINVAL;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t nvec = bytes / 16;
  const size_t per = static_cast<size_t>(stream::kLanes) * stream::kVecs;
  const size_t blocks = (nvec + per - 1) / per;
  if (blocks > 0x7fffffffu) {
    mko_set_error("stream_copy: %zu bytes is more than one launch covers", bytes);
    return MKO_EUNSUPPORTED;
  }
  if (nvec) {
    const auto* sv = static_cast<const mko_u32x4*>(src);
    auto* dv = static_cast<mko_u32x4*>(dst);
    MKO_TIMED("stream_copy", s,
              if (flags & MKO_STREAM_NONTEMPORAL) stream::copy16<true><<<static_cast<unsigned>(blocks), stream::kLanes, 0, s>>>(sv, dv, nvec);
              else stream::copy16<false><<<static_cast<unsigned>(blocks), stream::kLanes, 0, s>>>(sv, dv, nvec));
  }
  if (bytes % 16)
    stream::copy_tail<<<1, 16, 0, s>>>(static_cast<const unsigned char*>(src) + nvec * 16,
                                      static_cast<unsigned char*>(dst) + nvec * 16, bytes % 16);
  return mko_check_launch("stream_copy");
}
