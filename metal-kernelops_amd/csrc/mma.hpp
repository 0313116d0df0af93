// 64x64 output tiles on CDNA4 matrix cores for a 256-thread workgroup.
//
// Each of the four wavefronts owns a 32x32 quadrant (wm = wave / 2 rows,
// wn = wave % 2 columns) accumulated in 16 fp32 registers with the MFMA 32x32
// output layout: register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4 and
// column l%32 of the quadrant.  Operands come from LDS, both stored K-contiguous:
// A as [row][k], B transposed as [col][k], so a lane's operand slice is one
// 16-byte read (bf16/f16) or one float (fp32).
//
// Operand types: bf16 and f16 use v_mfma_f32_32x32x16_{bf16,f16}; float uses
// v_mfma_f32_32x32x2_f32, which keeps fp32 products (used for fp32 inputs).
//
// 16-bit tiles are XOR-swizzled in 8-element (16-byte) units: element (row, k) lives
// at row * 72 + (k ^ (row & 0x38)).  Rows 8 apart are 288 words apart, the same bank
// with 32 banks, so the transposed stores of a staging pass (eight lanes writing rows
// 8m + j, m = 0..7, at one k) would all hit one bank; the swizzle spreads them over
// eight 4-bank groups and leaves 16-byte runs whole and aligned for the operand reads.
#pragma once

#include "common.hpp"

namespace mko {

typedef __bf16 mfma_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 mfma_f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Leading dimension (elements) of a 64-wide K-contiguous LDS operand tile: padded so
// the 16-byte (16-bit types) or 4-byte (fp32) operand reads of consecutive rows fall in
// distinct banks, and even so that row pairs can be written as one word.
template <typename TM>
constexpr int tile_ld() { return sizeof(TM) == 2 ? 72 : 66; }

// A compact 16-bit tile, 64 elements a row, for kernels whose LDS bounds their
// occupancy.  Every row is 0 mod 32 banks, so the 16-byte units of row r are XOR-swizzled
// by (r mod 8) ^ (r / 8 mod 8): the operand reads (32 consecutive rows at one k) and the
// transposed staging stores (rows 8m + j at one k) both spread over eight 4-bank groups.
// fp32 tiles keep their padded pitch.
template <typename TM>
constexpr int compact_ld() { return sizeof(TM) == 2 ? 64 : tile_ld<TM>(); }

template <typename TM, int LD = tile_ld<TM>()>
struct LdsTile {
  static constexpr int ld = LD;
  static constexpr int elems = 64 * ld;
};

// Element offset of (row, k) in an LDS operand tile (k: the contiguous dimension).
template <typename TM, int LD = tile_ld<TM>()>
__device__ __forceinline__ int lds_idx(int row, int k) {
  if constexpr (sizeof(TM) == 2) {
    if constexpr (LD == 64)
      return row * 64 + (k ^ (((row & 7) ^ ((row >> 3) & 7)) << 3));
    else
      return row * LD + (k ^ (row & 0x38));
  } else {
    return row * LD + k;
  }
}

__device__ __forceinline__ void quadrant(int lane_wave, int& wm, int& wn) {
  wm = lane_wave >> 1;
  wn = lane_wave & 1;
}

// Row (within the 64x64 tile) of accumulator register r for this lane.
__device__ __forceinline__ int acc_row(int wm, int lane, int r) {
  return wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}
__device__ __forceinline__ int acc_col(int wn, int lane) { return wn * 32 + (lane & 31); }

// acc += A[wm*32 .. +32][0..k_len) * B[0..k_len)[wn*32 .. +32], with A and B^T in LDS.
template <typename TM, int LD = tile_ld<TM>()>
__device__ __forceinline__ void mma_tile(f32x16& acc, const TM* A, const TM* Bt, int wm, int wn, int lane,
                                         int k_len) {
  constexpr int ld = LD;
  if constexpr (sizeof(TM) == 2) {
    const int ra = wm * 32 + (lane & 31), rb = wn * 32 + (lane & 31), kh = (lane >> 5) * 8;
    for (int k = 0; k < k_len; k += 16) {
      const uint4 av = *reinterpret_cast<const uint4*>(A + lds_idx<TM, LD>(ra, k + kh));
      const uint4 bv = *reinterpret_cast<const uint4*>(Bt + lds_idx<TM, LD>(rb, k + kh));
      if constexpr (__is_same(TM, bf16)) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(mfma_bf16x8, av),
                                                      __builtin_bit_cast(mfma_bf16x8, bv), acc, 0, 0, 0);
      } else {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(mfma_f16x8, av),
                                                     __builtin_bit_cast(mfma_f16x8, bv), acc, 0, 0, 0);
      }
    }
  } else {
    const float* a = A + (wm * 32 + (lane & 31)) * ld + (lane >> 5);
    const float* b = Bt + (wn * 32 + (lane & 31)) * ld + (lane >> 5);
    for (int k = 0; k < k_len; k += 2) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[k], b[k], acc, 0, 0, 0);
  }
}

__device__ __forceinline__ void zero(f32x16& acc) {
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
}

}  // namespace mko
