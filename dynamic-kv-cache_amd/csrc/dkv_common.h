// Shared device/host helpers of libdkv: arena geometry, bf16 bit conversions,
// argument checking and the thread-local error message.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "dkv.h"

namespace dkv {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int D = DKV_HEAD_DIM;      // elements per (token, head) row
constexpr int TILE = DKV_TILE_TOKENS;  // tokens per tile

__host__ __device__ inline int64_t row_bytes(int bits) {
  return bits == 4 ? 32 : (bits == 8 ? 64 : 128);
}

// One (layer, kv, head) sub-block of a tile: payload rows, then (a, s) fp32
// pairs for 4/8-bit, rounded up to 16 bytes so every row and every sub-block
// start is 128-bit aligned.
__host__ __device__ inline int64_t subblock_bytes(int rows, int bits) {
  int64_t b = (int64_t)rows * row_bytes(bits) + (bits < 16 ? (int64_t)rows * 8 : 0);
  return (b + 15) & ~int64_t(15);
}

__host__ __device__ inline int64_t slab_bytes(int rows, int bits, int layers, int heads) {
  return subblock_bytes(rows, bits) * (int64_t)layers * 2 * heads;
}

// Tile descriptors of one segment, written by the lanes of one wave.
__device__ __forceinline__ void write_tile_descriptors(int64_t seg_offset, int seg_rows, int seg_token_start,
                                                      int bits, int tile_index0, int layers, int heads,
                                                      dkv_tile* tiles) {
  const int ntiles = (seg_rows + TILE - 1) / TILE;
  const int64_t full = slab_bytes(TILE, bits, layers, heads);
  for (int t = threadIdx.x & 63; t < ntiles; t += 64) {
    dkv_tile d;
    d.offset = seg_offset + (int64_t)t * full;
    d.token_start = seg_token_start + t * TILE;
    const int r = seg_rows - t * TILE;
    d.rows = (uint16_t)(r < TILE ? r : TILE);
    d.bits = (uint8_t)bits;
    d.reserved = 0;
    tiles[tile_index0 + t] = d;
  }
}

// Byte span [seg_offset, end) of a segment of seg_rows rows in the arena.
__host__ __device__ inline int64_t segment_end(int64_t seg_offset, int seg_rows, int bits, int layers,
                                               int heads) {
  const int ntiles = (seg_rows + TILE - 1) / TILE;
  return seg_offset + (int64_t)(ntiles - 1) * slab_bytes(TILE, bits, layers, heads) +
         slab_bytes(seg_rows - (ntiles - 1) * TILE, bits, layers, heads);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even (finite inputs; NaN stays NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two fp32 values -> packed bf16 pair (low half = lo), round to nearest even
// (v_cvt_pk_bf16_f32).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}
// x rounded to the nearest bf16 value, as fp32.
__device__ __forceinline__ float round_bf16(float x) { return bf16_lo(pack_bf16(x, 0.f)); }

// Thread-local message for DKV_EINVAL returns.
void set_error(const char* fmt, ...);
void clear_error();

}  // namespace dkv
