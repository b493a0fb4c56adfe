// Segment export and import between the arena and the reference's serialized
// layout: per layer and K/V, one PackedTensor of a [1, heads, rows, 64] tensor
// (src/kv_quantization.py:12-77), that is a contiguous payload of rows and
// separate fp32 offset and scale arrays with one group per row.
//
// Both directions are byte moves, bound by HBM bandwidth (payload loads are
// nontemporal: 61-63 -> 55-56 us for the 320 MB pack volume). A wave moves
// IO_UNITS (layer, kv, head, tile) sub-blocks. Per sub-block that is up to 64
// payload rows as 16-byte vectors (the rows are contiguous on both sides) and
// one (offset, scale) pair per lane, split into or joined from the two metadata
// arrays.
#include "dkv_common.h"

namespace dkv {
namespace {

constexpr int IO_THREADS = 256;
constexpr int IO_WAVES = IO_THREADS / 64;
constexpr int IO_VECS = TILE * 128 / 16 / 64;  // 16-byte vectors per lane for a full 16-bit sub-block
#ifndef DKV_IO_UNITS
#define DKV_IO_UNITS 2
#endif
// Sub-blocks per wave, all loaded before any store. With nontemporal loads 2 is
// best for the pack volume (export / import 53.3 / 53.8 us; 1: 95 us, 3: 55 us,
// 4: 56 us, 8: 63-64 us).
constexpr int IO_UNITS = DKV_IO_UNITS;

// Sub-blocks of one segment: one per (layer, kv, head, tile).
__host__ __device__ inline int io_units(int seg_rows, int n_layers, int heads) {
  return n_layers * 2 * heads * ((seg_rows + TILE - 1) / TILE);
}

__host__ __device__ inline int io_waves(int seg_rows, int n_layers, int heads) {
  return (io_units(seg_rows, n_layers, heads) + IO_UNITS - 1) / IO_UNITS;
}

// Wave w of a segment moves sub-blocks [w*IO_UNITS, (w+1)*IO_UNITS): every load of every
// sub-block is issued before the first store, so a wave keeps up to IO_UNITS * 8 KB in flight.
template <bool IMPORT>
__device__ __forceinline__ void io_wave(const dkv_segment_io& s, int w, uint8_t* __restrict__ arena,
                                        dkv_tile* __restrict__ tiles, int layers, int heads) {
  const int units = io_units(s.seg_rows, s.n_layers, heads);
  const int u0 = w * IO_UNITS;
  if (u0 >= units) return;
  if (IMPORT && s.write_tiles && w == 0)
    write_tile_descriptors(s.seg_offset, s.seg_rows, s.seg_token_start, s.bits, s.tile_index0, layers, heads,
                           tiles);
  const int ntiles = (s.seg_rows + TILE - 1) / TILE;
  const int bits = s.bits;
  const int rb = (int)row_bytes(bits);
  const int64_t slab = slab_bytes(TILE, bits, layers, heads);
  const int lane = threadIdx.x & 63;
  u32x4 v[IO_UNITS][IO_VECS];
  float2 m[IO_UNITS];
  uint8_t* arow[IO_UNITS];
  uint8_t* pay[IO_UNITS];
  float2* meta[IO_UNITS];
  float* offp[IO_UNITS];
  float* sclp[IO_UNITS];
  int64_t buf_row[IO_UNITS];
  int nrows[IO_UNITS];
#pragma unroll
  for (int q = 0; q < IO_UNITS; ++q) {
    const int u = u0 + q;
    const int t = u % ntiles;
    const int rest = u / ntiles;
    const int h = rest % heads;
    const int kv = (rest / heads) & 1;
    const int li = rest / heads >> 1;
    const int tile_rows = min(TILE, s.seg_rows - t * TILE);
    const int lo = max(t * TILE, s.row0);  // segment rows this sub-block moves: [lo, hi)
    const int hi = min(t * TILE + tile_rows, s.row0 + s.rows);
    nrows[q] = u < units ? max(hi - lo, 0) : 0;
    uint8_t* sub = arena + s.seg_offset + (int64_t)t * slab +
                   ((int64_t)((s.layer0 + li) * 2 + kv) * heads + h) * subblock_bytes(tile_rows, bits);
    buf_row[q] = ((int64_t)li * heads + h) * s.rows + (lo - s.row0);
    // (fields picked with selects, not a runtime index: an indexed copy of the
    // table entry would live in scratch memory)
    pay[q] = static_cast<uint8_t*>(kv ? s.payload[1] : s.payload[0]) + buf_row[q] * rb;
    arow[q] = sub + (int64_t)(lo - t * TILE) * rb;
    meta[q] = reinterpret_cast<float2*>(sub + (int64_t)tile_rows * rb) + (lo - t * TILE);
    offp[q] = (kv ? s.offsets[1] : s.offsets[0]) + buf_row[q];
    sclp[q] = (kv ? s.scales[1] : s.scales[0]) + buf_row[q];
    const int nvec = nrows[q] * rb / 16;
    const u32x4* src = reinterpret_cast<const u32x4*>(IMPORT ? pay[q] : arow[q]);
#pragma unroll
    for (int k = 0; k < IO_VECS; ++k) {
      const int i = lane + 64 * k;
      if (i < nvec) v[q][k] = __builtin_nontemporal_load(src + i);  // read once: streamed past the caches
    }
    if (bits < 16 && lane < nrows[q]) {
      if (IMPORT)
        m[q] = make_float2(offp[q][lane], sclp[q][lane]);
      else
        m[q] = meta[q][lane];
    }
  }
#pragma unroll
  for (int q = 0; q < IO_UNITS; ++q) {
    const int nvec = nrows[q] * rb / 16;
    u32x4* dst = reinterpret_cast<u32x4*>(IMPORT ? arow[q] : pay[q]);
#pragma unroll
    for (int k = 0; k < IO_VECS; ++k) {
      const int i = lane + 64 * k;
      if (i < nvec) dst[i] = v[q][k];
    }
    if (bits < 16 && lane < nrows[q]) {
      if (IMPORT) {
        meta[q][lane] = m[q];
      } else {
        offp[q][lane] = m[q].x;
        sclp[q][lane] = m[q].y;
      }
    }
  }
}

template <bool IMPORT>
__global__ void __launch_bounds__(IO_THREADS)
segment_one_kernel(dkv_segment_io s, uint8_t* arena, dkv_tile* tiles, int layers, int heads) {
  const int w = (int)blockIdx.x * IO_WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  io_wave<IMPORT>(s, w, arena, tiles, layers, heads);
}

template <bool IMPORT>
__global__ void __launch_bounds__(IO_THREADS)
segment_batch_kernel(const dkv_segment_io* __restrict__ ios, int n_ios, int waves_per_io, uint8_t* arena,
                     dkv_tile* tiles, int layers, int heads) {
  const int w = (int)blockIdx.x * IO_WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = w / waves_per_io;
  if (i >= n_ios) return;
  const dkv_segment_io s = ios[i];
  io_wave<IMPORT>(s, w - i * waves_per_io, arena, tiles, layers, heads);
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

int check_io(const dkv_segment_io& s, int direction, int64_t arena_bytes, int layers, int heads, const char* who) {
  if (s.bits != 4 && s.bits != 8 && s.bits != 16) {
    set_error("%s: bits must be 4, 8 or 16 (got %d)", who, s.bits);
    return DKV_EINVAL;
  }
  if (layers <= 0 || heads <= 0 || s.n_layers <= 0 || s.layer0 < 0 || s.layer0 + s.n_layers > layers) {
    set_error("%s: layers [%d, %d) outside [0, %d) or heads %d", who, s.layer0, s.layer0 + s.n_layers, layers,
              heads);
    return DKV_EINVAL;
  }
  if (s.seg_rows <= 0 || s.row0 < 0 || s.rows < 0 || s.row0 + s.rows > s.seg_rows) {
    set_error("%s: rows [%d, %d) outside a segment of %d rows", who, s.row0, s.row0 + s.rows, s.seg_rows);
    return DKV_EINVAL;
  }
  const int64_t end = segment_end(s.seg_offset, s.seg_rows, s.bits, layers, heads);
  if (s.seg_offset < 0 || (s.seg_offset & 15) || end > arena_bytes) {
    set_error("%s: segment [%lld, %lld) outside the %lld-byte arena or misaligned", who, (long long)s.seg_offset,
              (long long)end, (long long)arena_bytes);
    return DKV_EINVAL;
  }
  if (s.rows > 0) {
    for (int kv = 0; kv < 2; ++kv) {
      if (!s.payload[kv] || !aligned(s.payload[kv], 16)) {
        set_error("%s: payload buffers must be non-null and 16-byte aligned", who);
        return DKV_EINVAL;
      }
      if (s.bits < 16 && (!s.offsets[kv] || !s.scales[kv] || !aligned(s.offsets[kv], 4) ||
                          !aligned(s.scales[kv], 4))) {
        set_error("%s: 4/8-bit segments need fp32 offset and scale buffers", who);
        return DKV_EINVAL;
      }
    }
  }
  if (direction == 1 && s.write_tiles && s.tile_index0 < 0) {
    set_error("%s: write_tiles needs a non-negative tile index", who);
    return DKV_EINVAL;
  }
  return 0;
}

int launch_one(const dkv_segment_io& s, bool import, uint8_t* arena, dkv_tile* tiles, int layers, int heads,
               void* stream) {
  const int waves = io_waves(s.seg_rows, s.n_layers, heads);
  if (s.rows == 0 && !(import && s.write_tiles)) return 0;
  const unsigned grid = (unsigned)((waves + IO_WAVES - 1) / IO_WAVES);
  if (import)
    hipLaunchKernelGGL(segment_one_kernel<true>, dim3(grid), dim3(IO_THREADS), 0, (hipStream_t)stream, s, arena,
                       tiles, layers, heads);
  else
    hipLaunchKernelGGL(segment_one_kernel<false>, dim3(grid), dim3(IO_THREADS), 0, (hipStream_t)stream, s, arena,
                       tiles, layers, heads);
  return (int)hipGetLastError();
}

}  // namespace
}  // namespace dkv

using namespace dkv;

extern "C" {

int dkv_export(const dkv_segment_io* io, const void* arena, int64_t arena_bytes, int32_t layers, int32_t heads,
               void* stream) {
  clear_error();
  if (!io || !arena) {
    set_error("dkv_export: null segment or arena");
    return DKV_EINVAL;
  }
  if (int rc = check_io(*io, 0, arena_bytes, layers, heads, "dkv_export")) return rc;
  return launch_one(*io, false, const_cast<uint8_t*>(static_cast<const uint8_t*>(arena)), nullptr, layers, heads,
                    stream);
}

int dkv_import(const dkv_segment_io* io, void* arena, int64_t arena_bytes, dkv_tile* tiles, int32_t layers,
               int32_t heads, void* stream) {
  clear_error();
  if (!io || !arena) {
    set_error("dkv_import: null segment or arena");
    return DKV_EINVAL;
  }
  if (int rc = check_io(*io, 1, arena_bytes, layers, heads, "dkv_import")) return rc;
  if (io->write_tiles && !tiles) {
    set_error("dkv_import: write_tiles needs a tile table");
    return DKV_EINVAL;
  }
  return launch_one(*io, true, static_cast<uint8_t*>(arena), tiles, layers, heads, stream);
}

int dkv_segment_batch(const dkv_segment_io* ios, int32_t n_ios, int32_t max_rows, int32_t max_layers,
                      int32_t direction, void* arena, int64_t arena_bytes, dkv_tile* tiles, int32_t layers,
                      int32_t heads, void* stream) {
  clear_error();
  (void)arena_bytes;  // the table lives in device memory; the host validated it when it built it
  if (!ios || !arena || n_ios < 0 || max_rows <= 0 || max_layers <= 0 || max_layers > layers || heads <= 0 ||
      (direction != 0 && direction != 1) || (direction == 1 && !tiles)) {
    set_error("dkv_segment_batch: bad arguments (n_ios %d, max_rows %d, max_layers %d, direction %d)", n_ios,
              max_rows, max_layers, direction);
    return DKV_EINVAL;
  }
  if (n_ios == 0) return 0;
  const int wps = io_waves(max_rows, max_layers, heads);
  const int64_t blocks = ((int64_t)n_ios * wps + IO_WAVES - 1) / IO_WAVES;
  if ((int64_t)n_ios * wps > INT32_MAX / 2) {
    set_error("dkv_segment_batch: %lld blocks exceed one launch", (long long)blocks);
    return DKV_EINVAL;
  }
  if (direction == 1)
    hipLaunchKernelGGL(segment_batch_kernel<true>, dim3((unsigned)blocks), dim3(IO_THREADS), 0,
                       (hipStream_t)stream, ios, n_ios, wps, static_cast<uint8_t*>(arena), tiles, layers, heads);
  else
    hipLaunchKernelGGL(segment_batch_kernel<false>, dim3((unsigned)blocks), dim3(IO_THREADS), 0,
                       (hipStream_t)stream, ios, n_ios, wps, static_cast<uint8_t*>(arena), tiles, layers, heads);
  return (int)hipGetLastError();
}

int dkv_segment_validate(const dkv_segment_io* ios, int32_t n_ios, int32_t direction, int64_t arena_bytes,
                         int32_t layers, int32_t heads) {
  clear_error();
  if ((!ios && n_ios > 0) || n_ios < 0 || (direction != 0 && direction != 1)) {
    set_error("dkv_segment_validate: bad segment table or direction");
    return DKV_EINVAL;
  }
  for (int i = 0; i < n_ios; ++i)
    if (int rc = check_io(ios[i], direction, arena_bytes, layers, heads, "dkv_segment_validate")) return rc;
  return 0;
}

}  // extern "C"
