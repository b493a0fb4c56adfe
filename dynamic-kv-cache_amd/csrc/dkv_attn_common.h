// Helpers shared by the vector and MFMA attention kernels: the unit walk over
// history tiles and chunk pieces, chunk segment bounds, the execution plan and
// the launchers each kernel file provides.
#pragma once
#include "dkv_common.h"
#include <math.h>

namespace dkv {

constexpr float LOG2E = 1.4426950408889634f;

// Timeline probe, a build option (-DDKV_TIMELINE; off in the library build):
// lane 0 of each workgroup records wall_clock64() (a 100 MHz counter shared by
// all CUs) at numbered points of a kernel into its source file's device array,
// which that build's dkv_timeline_*() export copies out and clears. Used to see
// where a launch's time goes (which memory round trips sit on the critical path).
#ifdef DKV_TIMELINE
constexpr int TL_EVENTS = 10;  // 8 and 9: the in-kernel merge build's
constexpr int TL_SLOTS = 1 << 14;  // workgroups recorded per launch
#define DKV_TL(buf, ev)                                                                        \
  do {                                                                                         \
    if (threadIdx.x == 0) {                                                                    \
      const int tl_wg = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);        \
      if (tl_wg < TL_SLOTS) buf[tl_wg * TL_EVENTS + (ev)] = wall_clock64();                    \
    }                                                                                          \
  } while (0)
// Copies a kernel's stamp array to the host and zeroes it, so that a later read holds only the
// workgroups of later launches (a smaller grid leaves no stale slots behind).
inline int timeline_take(const uint64_t (&stamps)[TL_SLOTS * TL_EVENTS], void* host, int64_t bytes) {
  const int64_t n = (int64_t)sizeof(stamps) < bytes ? (int64_t)sizeof(stamps) : bytes;
  hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(stamps), n, 0, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return (int)e;
  static const uint64_t zeros[TL_SLOTS * TL_EVENTS] = {};
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(stamps), zeros, sizeof(stamps), 0, hipMemcpyHostToDevice);
}
#else
#define DKV_TL(buf, ev) \
  do {                  \
  } while (0)
#endif

// A unit is 64 keys of one KV head: a history tile of the arena, or a 64-row
// piece of the chunk's own native K/V.
struct Unit {
  bool chunk;
  int first;  // first logical token (history) or chunk row (chunk)
  int valid;  // keys present in this unit
  int bits;   // 4, 8 or 16 (chunk pieces are 16)
  int rows;   // rows of the tile: the sub-block's row stride basis
  const uint8_t* ksub;
  const uint8_t* vsub;
};

// The history a launch attends to: the args' own bounds, or (graph replays)
// the device step pair. Kept apart from the by-value kernel args, which the
// kernels never write (a written copy would be spilled to scratch).
struct Hist {
  int past, n_tiles;
};

__device__ __forceinline__ Unit get_unit(const dkv_attn_args& a, const Hist& hs, int u, int h) {
  Unit un;
  if (u < hs.n_tiles) {
    const dkv_tile t = a.tiles[u];
    un.chunk = false;
    un.first = t.token_start;
    un.valid = min((int)t.rows, hs.past - t.token_start);
    un.bits = t.bits;
    un.rows = t.rows;
    const int64_t sb = subblock_bytes(t.rows, t.bits);
    const uint8_t* base = static_cast<const uint8_t*>(a.arena) + t.offset;
    un.ksub = base + ((int64_t)(a.layer * 2 + 0) * a.heads + h) * sb;
    un.vsub = base + ((int64_t)(a.layer * 2 + 1) * a.heads + h) * sb;
  } else {
    const int c = u - hs.n_tiles;
    un.chunk = true;
    un.first = c * TILE;
    un.valid = min(TILE, a.nq - c * TILE);
    un.bits = 16;
    un.rows = TILE;
    un.ksub = un.vsub = nullptr;
  }
  return un;
}

// History unit of KV head h from its tile descriptor's four dwords (offset low and high,
// token_start, rows | bits << 16).
__device__ __forceinline__ Unit history_unit(const dkv_attn_args& a, const Hist& hs, uint32_t w0, uint32_t w1,
                                             uint32_t w2, uint32_t w3, int h) {
  Unit un;
  un.chunk = false;
  un.first = (int)w2;
  un.rows = (int)(w3 & 0xffffu);
  un.bits = (int)((w3 >> 16) & 0xffu);
  un.valid = min(un.rows, hs.past - un.first);
  const int64_t sb = subblock_bytes(un.rows, un.bits);
  const uint8_t* base = static_cast<const uint8_t*>(a.arena) + (int64_t)((uint64_t)w1 << 32 | w0);
  un.ksub = base + ((int64_t)(a.layer * 2 + 0) * a.heads + h) * sb;
  un.vsub = base + ((int64_t)(a.layer * 2 + 1) * a.heads + h) * sb;
  return un;
}

// Tile descriptors carried in a launch's argument block (dkv_attn_args.tiles_host): a kernel that
// takes them has this as its first parameter, so it starts the kernarg segment, and reads
// descriptor u with one scalar load beside the arguments instead of waiting on the device table.
struct ArgTiles {
  dkv_tile t[DKV_ARG_TILES];
};
// The first parameter of a kernel variant that does not carry them: 4 bytes, not 2 KB (a larger
// argument block slows every launch that has to fetch it, including those reading the table).
struct NoArgTiles {
  int unused;
};
typedef const __attribute__((address_space(4))) uint32_t* kernarg_u32_ptr;
__device__ __forceinline__ uint4 arg_tile(int u) {
  const kernarg_u32_ptr p = (kernarg_u32_ptr)__builtin_amdgcn_kernarg_segment_ptr() + 4 * u;
  return make_uint4(p[0], p[1], p[2], p[3]);
}
// Host: whether a launch carries its descriptors (at.t[0, n_tiles) filled from tiles_host).
inline bool fill_arg_tiles(const dkv_attn_args& a, ArgTiles& at) {
  if (!a.tiles_host || a.step || a.n_tiles <= 0 || a.n_tiles > DKV_ARG_TILES) return false;
  for (int i = 0; i < a.n_tiles; ++i) at.t[i] = a.tiles_host[i];
  for (int i = a.n_tiles; i < DKV_ARG_TILES; ++i) at.t[i] = dkv_tile{};  // unused, but defined bytes
  return true;
}

// The default split count of a history of `units` units: at most `cap` splits
// (the count that keeps every workgroup resident), each of at most
// ceil(units / cap) units, and no more splits than that needs. So the
// critical path is as short as with `cap` splits while the partials (and the
// merge's reads) shrink: 65 units at cap 51 run as 33 splits of two units.
__host__ __device__ inline int balanced_splits(int units, int cap) {
  if (units <= cap) return units < 1 ? 1 : units;
  const int per = (units + cap - 1) / cap;
  return (units + per - 1) / per;
}

// Graph replays: the history bounds the kernels run with come from the device
// step pair when one is given, and the launch-time `units` and `splits` are
// bounds only (such launches are sized for `cap` splits). The splits that run
// are then the ones a direct call on the same history runs,
// balanced_splits(units, cap), or min(explicit splits, units) when the caller
// chose the count (cap 0), so a replay partitions the history exactly like a
// direct call; the other workgroups exit at once and the partials keep the
// launch's split stride. Returns the splits that run.
__device__ __forceinline__ int runtime_plan(const dkv_attn_args& a, Hist& hs, int& units, int splits, int cap) {
  hs.past = a.past;
  hs.n_tiles = a.n_tiles;
  if (!a.step) return splits;
  hs.past = a.step[0];
  hs.n_tiles = a.step[1];
  units = hs.n_tiles + (a.nq + TILE - 1) / TILE;
  return min(splits, cap > 0 ? balanced_splits(units, cap) : units);
}

// The same for the short-chunk kernel, whose default split count is
// short_default_splits(units) workgroups per KV head rather than the launch's
// count: the splits that run for the runtime history are the ones a direct
// call on that history runs (an explicit args.splits keeps its meaning), never
// more than the launch's grid (nwg). The merge kernel that reads the short
// kernel's partials applies the same rule.
__device__ __forceinline__ int short_runtime_plan(const dkv_attn_args& a, Hist& hs, int& units, int nwg);

// max(a, b) of values that are never NaN (scores, running maxima, -inf masks) in one
// instruction, v_med3_f32(a, b, +inf). fmaxf has to quiet signalling NaN operands first, an extra
// v_max_f32 x, x, x per operand the compiler cannot prove canonical (MFMA results, lane swaps);
// so would med3 with a literal +inf, which the optimizer folds back into fmaxf. The empty asm
// makes +inf an SGPR value it cannot see through (it emits no instruction).
__device__ __forceinline__ float max_nn(float a, float b) {
  float inf;
  asm("" : "=s"(inf) : "0"(INFINITY));
  return __builtin_amdgcn_fmed3f(a, b, inf);
}

// First chunk row of the segment holding chunk row j (0 when n_segs <= 1).
__device__ __forceinline__ int chunk_seg_start(const dkv_attn_args& a, int j) {
  int start = 0;
  for (int s = 1; s < a.n_segs; ++s)
    if (j >= a.seg_bounds[s]) start = a.seg_bounds[s];
  return start;
}

// Workspace of a split call: partial outputs [heads, splits, R, 64] (fp32 O
// for precision 1, fp16 O / sum for precision 0), then partial (max, sum)
// [heads, splits, R] float2.
// The short-chunk kernel writes fp32 partials (precision-1 layout) in both
// precisions.
//
// The in-kernel merge build (-DDKV_INKERNEL_MERGE=1, _build.py --in-kernel-merge;
// a measurement build, not the library the package loads): the auto path's
// precision-0 calls skip the merge kernel, and the last workgroup of each (KV
// head, row group) to store its partials merges all of them. Its workspaces
// start with INKERNEL_COUNTER_BYTES of arrival counters, zero before first use
// and left zero by every call.
#ifndef DKV_INKERNEL_MERGE
#define DKV_INKERNEL_MERGE 0
#endif
constexpr int INKERNEL_COUNTER_BYTES = DKV_INKERNEL_MERGE ? 4096 : 0;
struct Plan {
  int path;       // 1 vector, 2 MFMA, 3 short chunk
  int precision;  // 0 bf16 operands (reference rounding), 1 fp32-accurate
  int units;
  int splits;
  int row_groups;
  int rows_per_group;
  int cap;        // default split cap (0: the caller's explicit split count)
  int fused;      // the in-kernel merge build: the frame-chunk kernel merges its own splits
  int plain_parts;  // MFMA split partials of the one-block-per-wave variant: plain stores and loads
  int small;      // MFMA decode-step variant: 4-wave workgroups, four per CU (MFMA_SMALL_ROWS)
  int wide_merge; // split merge with MERGE_WAVES waves per query row (combine_wide_*_kernel)
  int64_t part_o_bytes, part_ml_bytes;
};

// Launchers (return hipGetLastError()).
int launch_attn_vec(const dkv_attn_args& a, const Plan& p, float* part_o, float2* part_ml,
                    hipStream_t s);
int launch_attn_mfma(const dkv_attn_args& a, const Plan& p, float* part_o, float2* part_ml, uint32_t* counters,
                     hipStream_t s);
int launch_attn_short(const dkv_attn_args& a, const Plan& p, float* part_o, float2* part_ml, hipStream_t s);

// The MFMA kernel's workgroup: two key groups of MFMA_KG_WAVES waves; a wave owns the 16-row query
// blocks w and w + MFMA_KG_WAVES of its group, so a group of rows_per_group rows gives its busiest
// wave this many blocks (1 or 2; the kernel's NBW variant).
constexpr int MFMA_KG_WAVES = 6;
inline int mfma_blocks_per_wave(int rows_per_group) { return (rows_per_group / 16 + MFMA_KG_WAVES - 1) / MFMA_KG_WAVES; }
constexpr int SHORT_ROWS = 16;  // query rows per KV head the short-chunk kernel takes (one MFMA block)
constexpr int SHORT_UNITS = 4;  // 64-key units per short-chunk workgroup (one per wave) by default
// Most short-chunk workgroups per KV head by default: histories past 4 * 64 units (16k tokens) give
// each workgroup more than SHORT_UNITS units instead of growing the grid. It also bounds the grid of a
// launch sized for a device step pair, whose bound is the cache's whole tile table.
constexpr int SHORT_MAX_SPLITS = 64;
// Default split count of the short-chunk kernel over `units` units.
__host__ __device__ inline int short_default_splits(int units) {
  const int s = (units + SHORT_UNITS - 1) / SHORT_UNITS;
  return s < 1 ? 1 : (s > SHORT_MAX_SPLITS ? SHORT_MAX_SPLITS : s);
}
constexpr int VEC_ROWS = 64;    // query rows per vector-path workgroup

__device__ __forceinline__ int short_runtime_plan(const dkv_attn_args& a, Hist& hs, int& units, int nwg) {
  hs.past = a.past;
  hs.n_tiles = a.n_tiles;
  if (a.step) {
    hs.past = a.step[0];
    hs.n_tiles = a.step[1];
    units = hs.n_tiles + (a.nq + TILE - 1) / TILE;
  }
  const int want = a.splits > 0 ? min(a.splits, units) : short_default_splits(units);
  return max(1, min(nwg, want));
}
constexpr int MFMA_ROWS = 192;  // query rows per MFMA-path workgroup (6 waves x 2 blocks x 16)
// The auto path's decode-step variant of the MFMA kernel (precision 0, at most this many query rows
// per KV head): 4-wave workgroups with one buffer of raw bytes and tiles, four per CU.
constexpr int MFMA_SMALL_ROWS = 32;
// Workgroups of it per CU (36 KB of LDS each). Precision 1 needs 54 KB (hi and lo tiles), two
// per CU, and two units per workgroup ran slower than the 12-wave kernel (12.24 vs 11.24 us for
// a decode step at past 8128), so only precision 0 takes this variant.
constexpr int MFMA_SMALL_PER_CU = 4;

// Waves per query row of the split merge (combine_wide_kernel, combine_half_wide_kernel); 1 keeps
// the one-wave-per-row merge kernels (a build option for comparisons).
#ifndef DKV_MERGE_WAVES
#define DKV_MERGE_WAVES 4
#endif
constexpr int MERGE_WAVES = DKV_MERGE_WAVES;

// Precision-0 split partials hold O / sum in fp16, 64 values per row (128
// bytes) in the order the MFMA kernel's lanes store them: the lane of 16-byte
// chunk c < 4 holds columns 4c + [0, 4) of 16-column blocks 0 and 1, chunk
// c >= 4 columns 4(c - 4) + [0, 4) of blocks 2 and 3. Slot of column d:
__host__ __device__ inline int half_slot(int d) {
  const int db = d >> 4, g = (d >> 2) & 3, e = d & 3;
  return (db < 2 ? 0 : 32) + 8 * g + 4 * (db & 1) + e;
}
// Column of slot i (the inverse of half_slot).
__host__ __device__ inline int half_column(int i) {
  const int c = i >> 3, k = i & 7;
  return 16 * ((c < 4 ? 0 : 2) + (k >> 2)) + 4 * (c & 3) + (k & 3);
}

// fp16 partials hold O / sum, bounded by the row's largest |V|, which can pass
// the fp16 range (65504) where bf16 K/V do not. A row whose largest |O / sum|
// reaches 2^15 is stored scaled by 2^-e (e >= 1, the largest stored value then
// below 2^15), and its sum is stored with the sign bit set and e in the low 8
// bits of its mantissa (a relative change below 2^-15); every other row keeps
// e = 0 and its sum as is.
__device__ __forceinline__ int half_partial_exponent(float amax) {
  if (!(amax >= 32768.f)) return 0;  // NaN stays unscaled
  return (int)((__float_as_uint(amax) >> 23) & 0xffu) - 127 - 14;
}
__device__ __forceinline__ float half_partial_sum(float l, int e) {
  return e ? __uint_as_float(0x80000000u | (__float_as_uint(l) & 0x7fffff00u) | (uint32_t)e) : l;
}
// The stored sum of a row and its exponent e (the row's values are O / sum / 2^e).
__device__ __forceinline__ float half_partial_decode(float stored, int& e) {
  const uint32_t b = __float_as_uint(stored);
  const bool scaled = b >> 31;
  e = scaled ? (int)(b & 0xffu) : 0;
  return scaled ? __uint_as_float(b & 0x7fffff00u) : stored;
}

}  // namespace dkv
