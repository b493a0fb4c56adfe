// Pack and reconstruct kernels of libdkv (gfx950).
//
// Pack: bf16 K/V rows of 64 elements -> 4-bit (two codes per byte, low nibble =
// even element), 8-bit or unchanged 16-bit rows, plus one fp32 (offset, scale)
// pair per 4/8-bit row. The arithmetic is the reference quantizer's, one group
// per (head, token) row because head_dim == group_size == 64
// (src/kv_quantization.py:57-71, src/gpu_kernels.py:19-46):
//   a = min(x); span = max(x) - a; s = span > 0 ? span / (2^b - 1) : 1
//   q = clamp(rint((x - a) / s), 0, 2^b - 1)
// with IEEE fp32 subtraction and correctly rounded division (the build passes
// -ffp-contract=off and -fhip-fp32-correctly-rounded-divide-sqrt).
//
// Launch shape: two threads per row, 32 elements (64 bytes, four 128-bit loads)
// each, so one 256-thread workgroup streams 128 rows. The only cross-lane step
// is one min/max exchange between the two halves of a row. Stores are 128-bit:
// a half row of 4-bit codes is exactly 16 bytes, of 8-bit codes 2 x 16 bytes.
#include "dkv_common.h"
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

namespace dkv {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}
void clear_error() { g_err[0] = 0; }

constexpr int PACK_THREADS = 256;
constexpr int PACK_ROWS_PER_BLOCK = PACK_THREADS / 2;

struct Half32 {
  float x[32];
};

__device__ __forceinline__ void load_half_row(const uint16_t* src, Half32& h) {
  const u32x4* p = reinterpret_cast<const u32x4*>(src);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 w = __builtin_nontemporal_load(p + i);
    h.x[8 * i + 0] = bf16_lo(w.x);
    h.x[8 * i + 1] = bf16_hi(w.x);
    h.x[8 * i + 2] = bf16_lo(w.y);
    h.x[8 * i + 3] = bf16_hi(w.y);
    h.x[8 * i + 4] = bf16_lo(w.z);
    h.x[8 * i + 5] = bf16_hi(w.z);
    h.x[8 * i + 6] = bf16_lo(w.w);
    h.x[8 * i + 7] = bf16_hi(w.w);
  }
}

// Packs one 64-element row, of which this thread holds half `half` (0/1).
// `src` points at the thread's 32 input elements; the partner thread is the
// adjacent lane (lane ^ 1).
__device__ __forceinline__ void pack_half_row(const uint16_t* src, int half, int bits,
                                              uint8_t* payload_row, float2* meta_row) {
  if (bits == 16) {
    const u32x4* p = reinterpret_cast<const u32x4*>(src);
    u32x4* o = reinterpret_cast<u32x4*>(payload_row + half * 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = __builtin_nontemporal_load(p + i);
    return;
  }
  Half32 h;
  load_half_row(src, h);
  float lo = h.x[0], hi = h.x[0];
#pragma unroll
  for (int i = 1; i < 32; ++i) {
    lo = fminf(lo, h.x[i]);
    hi = fmaxf(hi, h.x[i]);
  }
  lo = fminf(lo, __shfl_xor(lo, 1));
  hi = fmaxf(hi, __shfl_xor(hi, 1));
  const float a = lo;
  const float span = hi - a;
  const float levels = bits == 4 ? 15.0f : 255.0f;
  const float s = span > 0.0f ? span / levels : 1.0f;
  uint32_t q[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    float v = rintf((h.x[i] - a) / s);
    v = fminf(fmaxf(v, 0.0f), levels);
    q[i] = (uint32_t)v;
  }
  if (bits == 4) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t acc = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc |= q[8 * i + j] << (4 * j);
      w[i] = acc;
    }
    *reinterpret_cast<uint4*>(payload_row + half * 16) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      w[i] = q[4 * i] | (q[4 * i + 1] << 8) | (q[4 * i + 2] << 16) | (q[4 * i + 3] << 24);
    uint4* o = reinterpret_cast<uint4*>(payload_row + half * 32);
    o[0] = make_uint4(w[0], w[1], w[2], w[3]);
    o[1] = make_uint4(w[4], w[5], w[6], w[7]);
  }
  if (half == 0) *meta_row = make_float2(a, s);
}

__device__ __forceinline__ void write_segment_tiles(const dkv_pack_job& j, int layers, int heads,
                                                    dkv_tile* tiles) {
  const int ntiles = (j.seg_rows + TILE - 1) / TILE;
  const int64_t full = slab_bytes(TILE, j.bits, layers, heads);
  for (int t = threadIdx.x; t < ntiles; t += blockDim.x) {
    dkv_tile d;
    d.offset = j.seg_offset + (int64_t)t * full;
    d.token_start = j.seg_token_start + t * TILE;
    const int r = j.seg_rows - t * TILE;
    d.rows = (uint16_t)(r < TILE ? r : TILE);
    d.bits = (uint8_t)j.bits;
    d.reserved = 0;
    tiles[j.tile_index0 + t] = d;
  }
}

__device__ __forceinline__ void pack_job_rows(const dkv_pack_job& j, int block, uint8_t* arena,
                                              int layers, int heads) {
  const int rows_total = 2 * heads * j.n;
  const int row = block * PACK_ROWS_PER_BLOCK + (threadIdx.x >> 1);
  const int half = threadIdx.x & 1;
  if (row >= rows_total) return;  // both halves of a row exit together
  const int per_kv = heads * j.n;
  const int kv = row / per_kv;
  const int rem = row - kv * per_kv;
  const int head = rem / j.n;
  const int tok = rem - head * j.n;
  const uint16_t* src = kv == 0
      ? static_cast<const uint16_t*>(j.k) + head * j.k_head_stride + (int64_t)tok * j.k_tok_stride
      : static_cast<const uint16_t*>(j.v) + head * j.v_head_stride + (int64_t)tok * j.v_tok_stride;
  src += half * 32;
  const int r_seg = j.row0 + tok;
  const int ti = r_seg / TILE;
  const int rt = r_seg - ti * TILE;
  const int rows_i = min(TILE, j.seg_rows - ti * TILE);
  const int64_t sb = subblock_bytes(rows_i, j.bits);
  uint8_t* sub = arena + j.seg_offset + (int64_t)ti * slab_bytes(TILE, j.bits, layers, heads) +
                 ((int64_t)(j.layer * 2 + kv) * heads + head) * sb;
  uint8_t* payload_row = sub + (int64_t)rt * row_bytes(j.bits);
  float2* meta_row = reinterpret_cast<float2*>(sub + (int64_t)rows_i * row_bytes(j.bits)) + rt;
  pack_half_row(src, half, j.bits, payload_row, meta_row);
}

__global__ void __launch_bounds__(PACK_THREADS)
pack_one_kernel(dkv_pack_job j, uint8_t* arena, dkv_tile* tiles, int layers, int heads) {
  if (j.write_tiles && blockIdx.x == 0) write_segment_tiles(j, layers, heads, tiles);
  pack_job_rows(j, blockIdx.x, arena, layers, heads);
}

__global__ void __launch_bounds__(PACK_THREADS)
pack_batch_kernel(const dkv_pack_job* __restrict__ jobs, uint8_t* arena, dkv_tile* tiles,
                  int layers, int heads) {
  const dkv_pack_job j = jobs[blockIdx.y];
  if (j.write_tiles && blockIdx.x == 0) write_segment_tiles(j, layers, heads, tiles);
  pack_job_rows(j, blockIdx.x, arena, layers, heads);
}

// Reconstruct: one 256-thread block per (tile, kv*heads + head); four threads
// per row, 16 elements each. x = q*s + a with a separately rounded multiply and
// add, exactly as the reference's unpack (src/kv_quantization.py:90-91).
__global__ void __launch_bounds__(256)
reconstruct_kernel(const uint8_t* __restrict__ arena, const dkv_tile* __restrict__ tiles,
                   int n_tokens, int layer, int layers, int heads, void* out, int out_dtype) {
  const dkv_tile t = tiles[blockIdx.x];
  const int kvh = blockIdx.y;  // kv * heads + head
  const int valid = min((int)t.rows, n_tokens - t.token_start);
  const int r = threadIdx.x >> 2;
  const int c = threadIdx.x & 3;
  if (r >= valid) return;
  const int bits = t.bits;
  const int64_t sb = subblock_bytes(t.rows, bits);
  const uint8_t* sub = arena + t.offset + ((int64_t)layer * 2 * heads + kvh) * sb;
  const uint8_t* prow = sub + (int64_t)r * row_bytes(bits);
  float x[16];
  if (bits == 16) {
    const uint4* p = reinterpret_cast<const uint4*>(prow + c * 32);
    uint4 w0 = p[0], w1 = p[1];
    uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[2 * i] = bf16_lo(w[i]);
      x[2 * i + 1] = bf16_hi(w[i]);
    }
  } else {
    const float2 as = reinterpret_cast<const float2*>(sub + (int64_t)t.rows * row_bytes(bits))[r];
    uint32_t code[16];
    if (bits == 4) {
      uint2 w = *reinterpret_cast<const uint2*>(prow + c * 8);
#pragma unroll
      for (int i = 0; i < 8; ++i) code[i] = (w.x >> (4 * i)) & 15u;
#pragma unroll
      for (int i = 0; i < 8; ++i) code[8 + i] = (w.y >> (4 * i)) & 15u;
    } else {
      uint4 w = *reinterpret_cast<const uint4*>(prow + c * 16);
      uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < 16; ++i) code[i] = (ww[i >> 2] >> (8 * (i & 3))) & 255u;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = __fadd_rn(__fmul_rn((float)code[i], as.y), as.x);
  }
  const int kv = kvh / heads, head = kvh - kv * heads;
  const int64_t o = (((int64_t)kv * heads + head) * n_tokens + t.token_start + r) * D + c * 16;
  if (out_dtype == 1) {
    float4* dst = reinterpret_cast<float4*>(static_cast<float*>(out) + o);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = make_float4(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
  } else {
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = f32_to_bf16_rne(x[2 * i]) | (f32_to_bf16_rne(x[2 * i + 1]) << 16);
    uint4* dst = reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + o);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
  }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static int check_job(const dkv_pack_job& j, int64_t arena_bytes, int layers, int heads) {
  if (j.bits != 4 && j.bits != 8 && j.bits != 16) {
    set_error("dkv_pack: bits must be 4, 8 or 16 (got %d)", j.bits);
    return DKV_EINVAL;
  }
  if (j.n < 0 || j.row0 < 0 || j.row0 + j.n > j.seg_rows || j.seg_rows <= 0) {
    set_error("dkv_pack: rows [%d, %d) outside a segment of %d rows", j.row0, j.row0 + j.n, j.seg_rows);
    return DKV_EINVAL;
  }
  if (j.layer < 0 || j.layer >= layers || heads <= 0) {
    set_error("dkv_pack: layer %d outside [0, %d) or heads %d", j.layer, layers, heads);
    return DKV_EINVAL;
  }
  const int ntiles = (j.seg_rows + TILE - 1) / TILE;
  const int64_t end = j.seg_offset + (int64_t)(ntiles - 1) * slab_bytes(TILE, j.bits, layers, heads) +
                      slab_bytes(j.seg_rows - (ntiles - 1) * TILE, j.bits, layers, heads);
  if (j.seg_offset < 0 || (j.seg_offset & 15) || end > arena_bytes) {
    set_error("dkv_pack: segment [%lld, %lld) outside the %lld-byte arena or misaligned",
              (long long)j.seg_offset, (long long)end, (long long)arena_bytes);
    return DKV_EINVAL;
  }
  if (j.n > 0) {
    if (!j.k || !j.v || !aligned16(j.k) || !aligned16(j.v) || (j.k_head_stride & 7) ||
        (j.k_tok_stride & 7) || (j.v_head_stride & 7) || (j.v_tok_stride & 7)) {
      set_error("dkv_pack: K/V must be 16-byte aligned with strides that are multiples of 8 elements");
      return DKV_EINVAL;
    }
  }
  return 0;
}

}  // namespace dkv

using namespace dkv;

extern "C" {

int dkv_version(void) { return DKV_ABI_VERSION; }

const char* dkv_last_error(void) { return dkv::g_err; }

int64_t dkv_subblock_bytes(int32_t rows, int32_t bits) { return subblock_bytes(rows, bits); }

int64_t dkv_slab_bytes(int32_t rows, int32_t bits, int32_t layers, int32_t heads) {
  return slab_bytes(rows, bits, layers, heads);
}

int dkv_pack(const dkv_pack_job* job, void* arena, int64_t arena_bytes, dkv_tile* tiles,
             int32_t layers, int32_t heads, void* stream) {
  clear_error();
  if (!job || !arena) {
    set_error("dkv_pack: null job or arena");
    return DKV_EINVAL;
  }
  if (int rc = check_job(*job, arena_bytes, layers, heads)) return rc;
  if (job->write_tiles && (!tiles || job->tile_index0 < 0)) {
    set_error("dkv_pack: write_tiles needs a tile table");
    return DKV_EINVAL;
  }
  const int rows = 2 * heads * job->n;
  const int blocks = (rows + PACK_ROWS_PER_BLOCK - 1) / PACK_ROWS_PER_BLOCK;
  const int grid = blocks > 0 ? blocks : (job->write_tiles ? 1 : 0);
  if (grid == 0) return 0;
  hipLaunchKernelGGL(pack_one_kernel, dim3(grid), dim3(PACK_THREADS), 0, (hipStream_t)stream, *job,
                     static_cast<uint8_t*>(arena), tiles, layers, heads);
  return (int)hipGetLastError();
}

int dkv_pack_batch(const dkv_pack_job* jobs, int32_t n_jobs, int32_t max_n, void* arena,
                   int64_t arena_bytes, dkv_tile* tiles, int32_t layers, int32_t heads, void* stream) {
  clear_error();
  (void)arena_bytes;  // jobs live in device memory; the host validated them when it built them
  if (!jobs || !arena || n_jobs < 0 || max_n < 0 || layers <= 0 || heads <= 0 || n_jobs > 65535) {
    set_error("dkv_pack_batch: bad arguments (jobs %p, n_jobs %d, max_n %d)", (const void*)jobs, n_jobs, max_n);
    return DKV_EINVAL;
  }
  if (n_jobs == 0) return 0;
  const int rows = 2 * heads * max_n;
  const int blocks = (rows + PACK_ROWS_PER_BLOCK - 1) / PACK_ROWS_PER_BLOCK;
  hipLaunchKernelGGL(pack_batch_kernel, dim3(blocks > 0 ? blocks : 1, n_jobs), dim3(PACK_THREADS), 0,
                     (hipStream_t)stream, jobs, static_cast<uint8_t*>(arena), tiles, layers, heads);
  return (int)hipGetLastError();
}

int dkv_reconstruct(const void* arena, const dkv_tile* tiles, int32_t n_tiles, int32_t n_tokens,
                    int32_t layer, int32_t layers, int32_t heads, void* out, int32_t out_dtype,
                    void* stream) {
  clear_error();
  if (!arena || (!tiles && n_tiles > 0) || !out || n_tiles < 0 || n_tokens < 0 || layer < 0 ||
      layer >= layers || heads <= 0 || (out_dtype != 0 && out_dtype != 1)) {
    set_error("dkv_reconstruct: bad arguments");
    return DKV_EINVAL;
  }
  if (n_tiles == 0 || n_tokens == 0) return 0;
  hipLaunchKernelGGL(reconstruct_kernel, dim3(n_tiles, 2 * heads), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint8_t*>(arena), tiles, n_tokens, layer, layers, heads, out,
                     out_dtype);
  return (int)hipGetLastError();
}

}  // extern "C"
