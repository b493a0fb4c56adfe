// Pack and reconstruct kernels of libdkv (gfx950).
//
// Pack: bf16 K/V rows of 64 elements -> 4-bit (two codes per byte, low nibble =
// even element), 8-bit or unchanged 16-bit rows, plus one fp32 (offset, scale)
// pair per 4/8-bit row. The arithmetic is the reference quantizer's, one group
// per (head, token) row because head_dim == group_size == 64
// (src/kv_quantization.py:57-71, src/gpu_kernels.py:19-46):
//   a = min(x); span = max(x) - a; s = span > 0 ? span / (2^b - 1) : 1
//   q = clamp(rint((x - a) / s), 0, 2^b - 1)
// with IEEE fp32 subtraction and division (the build passes -ffp-contract=off
// and -fhip-fp32-correctly-rounded-divide-sqrt).
//
// The per-element division is the expensive part (about ten VALU operations
// when correctly rounded), so the kernel first forms t = (x - a) * rcp(s). For
// 0 <= (x - a)/s <= 256, v_rcp_f32 (1 ulp) and the product put t within
// 2^-14.3 of the exact quotient and the correctly rounded quotient within
// 2^-16 of it, so both round to the same integer unless t is within 2^-13 of a
// half-integer. Those rows (and any row whose t is not finite, e.g. a
// subnormal scale) take the correctly rounded division instead; the result is
// bit-identical to rint((x - a) / s) in every case.
//
// Launch shape: one wave packs 64 consecutive tokens of one (K or V, head) of
// one job. Global loads and stores are 16 bytes per lane over contiguous
// rows; an LDS transpose hands each lane one whole row, so a row's min/max,
// scale and reciprocal are computed once.
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

constexpr int PACK_THREADS = 256;  // 4 waves
constexpr int WAVE_ROWS = 64;      // tokens of one (kv, head) per wave, one per lane
constexpr float TIE_GUARD = 0.5f - 0x1p-13f;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x8_t __attribute__((ext_vector_type(8)));

struct RowDst {
  uint8_t* payload;  // start of the row's payload
  float2* meta;      // the row's (offset, scale)
};

__device__ __forceinline__ RowDst row_dst(const dkv_pack_job& j, int kv, int head, int tok, uint8_t* arena,
                                          int layers, int heads) {
  const int r_seg = j.row0 + tok;
  const int ti = r_seg / TILE;
  const int rt = r_seg - ti * TILE;
  const int rows_i = min(TILE, j.seg_rows - ti * TILE);
  const int64_t sb = subblock_bytes(rows_i, j.bits);
  uint8_t* sub = arena + j.seg_offset + (int64_t)ti * slab_bytes(TILE, j.bits, layers, heads) +
                 ((int64_t)(j.layer * 2 + kv) * heads + head) * sb;
  RowDst d;
  d.payload = sub + (int64_t)rt * row_bytes(j.bits);
  d.meta = reinterpret_cast<float2*>(sub + (int64_t)rows_i * row_bytes(j.bits)) + rt;
  return d;
}

// The offset of a row whose minimum is zero: -0 when the row holds a -0, else
// +0, the sign IEEE 754-2019 minimum() gives. (v_min_f32 and torch's amin,
// src/kv_quantization.py:63, leave it to the order of the reduction; codes,
// scales and dequantized values do not depend on it.)
__device__ __forceinline__ float zero_min_sign(uint32_t has_neg_zero) { return has_neg_zero ? -0.0f : 0.0f; }

// Codes of 8 elements of a row whose (offset, scale) is (a, s), with r ~ 1/s,
// packed: BITS 4 -> out[0] (element e in bits 4e..4e+3), BITS 8 -> out[0..1]
// (element e in byte e). `fast` says r and every t below are finite.
//
// rint(t) comes from m = t + 2^23, which for 0 <= t < 2^22 rounds t to an
// integer (round to nearest even, as rintf) and leaves it in the low mantissa
// bits: byte 0 of m's bit pattern is the code. The group takes the exact
// division when any t is within 2^-13 of a half-integer.
template <int BITS>
__device__ __forceinline__ void quantize8(const float* x, float a, float s, float r, bool fast, uint32_t* out) {
  constexpr float LEVELS = BITS == 4 ? 15.0f : 255.0f;
  constexpr float MAGIC = 0x1p23f;
  uint32_t y[8];
  float dev = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float t = __fmul_rn(x[e] - a, r);
    const float m = __fadd_rn(t, MAGIC);
    dev = fmaxf(dev, fabsf(t - (m - MAGIC)));
    y[e] = __float_as_uint(m);
  }
  if (!(fast && dev < TIE_GUARD)) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      y[e] = (uint32_t)__builtin_amdgcn_fmed3f(rintf(__fdiv_rn(x[e] - a, s)), 0.0f, LEVELS);
  }
  if (BITS == 4) {
    uint32_t p[4];  // byte 0 of p[i] = element 2i + 1 in the high nibble, 2i in the low one
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = (y[2 * i + 1] << 4) | y[2 * i];
    const uint32_t lo = __builtin_amdgcn_perm(p[1], p[0], 0x07060400u);
    const uint32_t hi = __builtin_amdgcn_perm(p[3], p[2], 0x07060400u);
    out[0] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
  } else {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t lo = __builtin_amdgcn_perm(y[4 * w + 1], y[4 * w], 0x07060400u);
      const uint32_t hi = __builtin_amdgcn_perm(y[4 * w + 3], y[4 * w + 2], 0x07060400u);
      out[w] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    }
  }
}

// A wave packs 64 rows (one per lane) staged through LDS: lanes load and store
// global memory 16 bytes each, 8 lanes per row (every instruction covers 1 KB
// of contiguous rows), while the arithmetic runs one row per lane, so a row's
// min/max, scale and reciprocal are computed once. LDS rows are padded to
// 144 bytes, which makes both the 8-lanes-per-row and the lane-per-row
// accesses conflict-free.
constexpr int LROW = 144;                  // padded LDS row, bytes
constexpr int WAVE_LDS = WAVE_ROWS * LROW;  // 9216 bytes per wave

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Packs rows [tok0, tok0 + nrows) of the job's (kv, head) from registers: lane
// l holds columns [8c, 8c + 8) (c = l & 7) of rows 8i + (l >> 3) in w[i].
template <int BITS>
__device__ __forceinline__ void pack_loaded(const dkv_pack_job& j, int kv, int head, int tok0, int nrows,
                                            const u32x4* w, uint8_t* arena, int layers, int heads, uint8_t* lds) {
  const int lane = threadIdx.x & 63;
  const int c = lane & 7;
  // Destination: one wave-uniform sub-block base when the wave's rows sit in
  // one tile (every append that starts on a tile boundary).
  const int rfirst = j.row0 + tok0;
  const int rlast = rfirst + nrows - 1;
  const bool one_tile = rfirst / TILE == rlast / TILE;
  const RowDst d0 = row_dst(j, kv, head, tok0, arena, layers, heads);
  constexpr int RB = BITS == 4 ? 32 : (BITS == 8 ? 64 : 128);
  // Arena stores are nontemporal: lines written with plain stores stay dirty in
  // L2 and the end of the kernel writes all of them back before it completes.
  if (BITS == 16) {
    if (one_tile && nrows == WAVE_ROWS) {  // a full slice in one tile: no per-row tests
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = 8 * i + (lane >> 3);
        __builtin_nontemporal_store(w[i], reinterpret_cast<u32x4*>(d0.payload + r * 128 + 16 * c));
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 8 * i + (lane >> 3);
      if (r >= nrows) continue;
      uint8_t* dst = one_tile ? d0.payload + r * 128 : row_dst(j, kv, head, tok0 + r, arena, layers, heads).payload;
      __builtin_nontemporal_store(w[i], reinterpret_cast<u32x4*>(dst + 16 * c));
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
    *reinterpret_cast<u32x4*>(lds + (8 * i + (lane >> 3)) * LROW + 16 * c) = w[i];
  wave_sync_lds();
  float x[64];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(lds + lane * LROW + 16 * i);
    const f32x8_t f = __builtin_convertvector(__builtin_bit_cast(bf16x8_t, v), f32x8_t);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[8 * i + e] = f[e];
  }
  float lo = x[0], hi = x[0];
#pragma unroll
  for (int e = 1; e < 64; ++e) {
    lo = fminf(lo, x[e]);
    hi = fmaxf(hi, x[e]);
  }
  if (lo == 0.0f) {  // rare: the sign of a zero minimum (see zero_min_sign)
    uint32_t nz = 0;
#pragma unroll
    for (int e = 0; e < 64; ++e) nz |= __float_as_uint(x[e]) == 0x80000000u;
    lo = zero_min_sign(nz);
  }
  const float a = lo;
  const float span = hi - a;
  const float s = span > 0.0f ? __fdiv_rn(span, BITS == 4 ? 15.0f : 255.0f) : 1.0f;
  const float rs = __builtin_amdgcn_rcpf(s);
  const bool fast = s >= 0x1p-126f && s <= 0x1p125f;  // rs normal, every t finite and below 2^22
  uint32_t out[RB / 4];
#pragma unroll
  for (int i = 0; i < 8; ++i) quantize8<BITS>(x + 8 * i, a, s, rs, fast, out + (BITS == 4 ? i : 2 * i));
  const bool valid = lane < nrows;
  if (!one_tile) {  // rows straddle a tile boundary: each lane stores its own row
    if (valid) {
      const RowDst d = row_dst(j, kv, head, tok0 + lane, arena, layers, heads);
#pragma unroll
      for (int i = 0; i < RB / 16; ++i)
        *reinterpret_cast<u32x4*>(d.payload + 16 * i) = u32x4{out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]};
      *d.meta = make_float2(a, s);
    }
    return;
  }
  // (nrows == WAVE_ROWS: every lane's row is valid; the compiler cannot tell that from `valid`)
  if (valid || nrows == WAVE_ROWS) __builtin_nontemporal_store((f32x2_t{a, s}), reinterpret_cast<f32x2_t*>(d0.meta + lane));
  // Packed rows back through LDS (the wave's own region, already read), then
  // contiguous 16-byte stores: RB bytes per row, rows back to back.
  wave_sync_lds();
#pragma unroll
  for (int i = 0; i < RB / 16; ++i)
    *reinterpret_cast<u32x4*>(lds + lane * RB + 16 * i) = u32x4{out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]};
  wave_sync_lds();
  const int bytes = nrows * RB;
#pragma unroll
  for (int i = 0; i < RB / 16; ++i) {
    const int off = 16 * (lane + 64 * i);
    if (nrows == WAVE_ROWS || off < bytes)
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(lds + off), reinterpret_cast<u32x4*>(d0.payload + off));
  }
}

template <int BITS>
__device__ __forceinline__ void pack_wave(const dkv_pack_job& j, int kv, int head, int tok0, uint8_t* arena,
                                          int layers, int heads, uint8_t* lds) {
  const int lane = threadIdx.x & 63;
  const int c = lane & 7;
  const uint16_t* base = kv == 0 ? static_cast<const uint16_t*>(j.k) + head * j.k_head_stride
                                 : static_cast<const uint16_t*>(j.v) + head * j.v_head_stride;
  const int64_t ts = kv == 0 ? j.k_tok_stride : j.v_tok_stride;
  const int nrows = min(WAVE_ROWS, j.n - tok0);
  // The job's K/V pointers come from memory, so the compiler cannot tell they are global and
  // would emit flat loads; a full slice (every slice but a partial append's last) loads all
  // rows with no per-row test, so the eight loads go out back to back (72.9 -> 72.5 us for the
  // 32-layer, 96-frame volume).
  typedef const __attribute__((address_space(1))) u32x4 global_u32x4;
  u32x4 w[8];
  if (nrows == WAVE_ROWS) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 8 * i + (lane >> 3);
      w[i] = __builtin_nontemporal_load((global_u32x4*)(base + (tok0 + r) * ts + 8 * c));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 8 * i + (lane >> 3);
      w[i] = r < nrows ? __builtin_nontemporal_load((global_u32x4*)(base + (tok0 + r) * ts + 8 * c))
                       : u32x4{0, 0, 0, 0};
    }
  }
  pack_loaded<BITS>(j, kv, head, tok0, nrows, w, arena, layers, heads, lds);
}

__device__ __forceinline__ void write_segment_tiles(const dkv_pack_job& j, int layers, int heads,
                                                    dkv_tile* tiles) {
  write_tile_descriptors(j.seg_offset, j.seg_rows, j.seg_token_start, j.bits, j.tile_index0, layers, heads,
                         tiles);
}

// Wave index -> (kv, head, 64-token slice) of the job; the bit width is
// uniform per job, so the branch below is uniform per wave.
__device__ __forceinline__ void pack_job_wave(const dkv_pack_job& j, int wave, uint8_t* arena, int layers,
                                              int heads) {
  __shared__ __attribute__((aligned(16))) uint8_t stage[PACK_THREADS / 64][WAVE_LDS];
  uint8_t* lds = stage[(threadIdx.x >> 6)];
  const int slices = (j.n + WAVE_ROWS - 1) / WAVE_ROWS;
  const int per_kv = heads * slices;
  if (wave >= 2 * per_kv) return;
  const int kv = wave / per_kv;
  const int rem = wave - kv * per_kv;
  const int head = rem / slices;
  const int tok0 = (rem - head * slices) * WAVE_ROWS;
  if (j.bits == 4) pack_wave<4>(j, kv, head, tok0, arena, layers, heads, lds);
  else if (j.bits == 8) pack_wave<8>(j, kv, head, tok0, arena, layers, heads, lds);
  else pack_wave<16>(j, kv, head, tok0, arena, layers, heads, lds);
}

__global__ void __launch_bounds__(PACK_THREADS)
pack_one_kernel(dkv_pack_job j, uint8_t* arena, dkv_tile* tiles, int layers, int heads) {
  const int wave = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * (PACK_THREADS / 64) + (threadIdx.x >> 6)));
  if (j.write_tiles && wave == 0) write_segment_tiles(j, layers, heads, tiles);
  pack_job_wave(j, wave, arena, layers, heads);
}

// Waves are numbered across the whole batch (wpj waves per job, from the
// largest job), so no workgroup carries idle waves past the end of a job.
__global__ void __launch_bounds__(PACK_THREADS)
pack_batch_kernel(const dkv_pack_job* __restrict__ jobs, int n_jobs, int wpj, uint8_t* arena, dkv_tile* tiles,
                  int layers, int heads) {
  const int gw = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * (PACK_THREADS / 64) + (threadIdx.x >> 6)));
  const int ji = gw / wpj;
  if (ji >= n_jobs) return;
  const dkv_pack_job j = jobs[ji];
  const int wave = gw - ji * wpj;
  if (j.write_tiles && wave == 0) write_segment_tiles(j, layers, heads, tiles);
  pack_job_wave(j, wave, arena, layers, heads);
}

// Eight elements of one row after RoPE: y = bf16(bf16(x * cos) + bf16(sign *
// partner * sin)), where partner is the element 32 columns away (rotate_half)
// and sign is -1 on the first half of the row. Products of two bf16 values are
// exact in fp32, so this is transformers' apply_rotary_pos_emb in bf16
// operation by operation (q * cos + rotate_half(q) * sin, each op rounded).
__device__ __forceinline__ u32x4 rope8(const u32x4& x, const u32x4& partner, const u32x4& cs, const u32x4& sn,
                                       bool first_half) {
  const float sg = first_half ? -1.0f : 1.0f;
  u32x4 y;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float lo = round_bf16(round_bf16(bf16_lo(x[k]) * bf16_lo(cs[k])) +
                                round_bf16(sg * bf16_lo(partner[k]) * bf16_lo(sn[k])));
    const float hi = round_bf16(round_bf16(bf16_hi(x[k]) * bf16_hi(cs[k])) +
                                round_bf16(sg * bf16_hi(partner[k]) * bf16_hi(sn[k])));
    y[k] = pack_bf16(lo, hi);
  }
  return y;
}

// Packs one row held by 8 lanes (lane c of the row holds columns [8c, 8c + 8)
// in w): min/max over the row through the 8 lanes, then the arithmetic of
// pack_loaded (every lane of the row forms the same a, s and 1/s) and quantize8
// on the lane's 8 elements. Lanes of rows r >= nrows still take part in the
// exchanges but store nothing.
template <int BITS>
__device__ __forceinline__ void pack_row8(const dkv_pack_job& j, int kv, int head, int tok, bool valid, int c,
                                          const u32x4& w, uint8_t* arena, int layers, int heads) {
  float x[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[2 * e] = bf16_lo(w[e]);
    x[2 * e + 1] = bf16_hi(w[e]);
  }
  if (BITS == 16) {
    if (valid) *reinterpret_cast<u32x4*>(row_dst(j, kv, head, tok, arena, layers, heads).payload + 16 * c) = w;
    return;
  }
  float lo = x[0], hi = x[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) {
    lo = fminf(lo, x[e]);
    hi = fmaxf(hi, x[e]);
  }
  uint32_t nz = 0;  // the row holds a -0 (the sign of a zero minimum, see zero_min_sign)
#pragma unroll
  for (int e = 0; e < 8; ++e) nz |= __float_as_uint(x[e]) == 0x80000000u;
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) {
    lo = fminf(lo, __shfl_xor(lo, o));
    hi = fmaxf(hi, __shfl_xor(hi, o));
    nz |= __shfl_xor(nz, o);
  }
  const float a = lo == 0.0f ? zero_min_sign(nz) : lo;
  const float span = hi - a;
  const float s = span > 0.0f ? __fdiv_rn(span, BITS == 4 ? 15.0f : 255.0f) : 1.0f;
  const float rs = __builtin_amdgcn_rcpf(s);
  const bool fast = s >= 0x1p-126f && s <= 0x1p125f;
  uint32_t out[2];
  quantize8<BITS>(x, a, s, rs, fast, out);
  if (!valid) return;
  const RowDst d = row_dst(j, kv, head, tok, arena, layers, heads);
  if (BITS == 4) *reinterpret_cast<uint32_t*>(d.payload + 4 * c) = out[0];
  else *reinterpret_cast<uint2*>(d.payload + 8 * c) = make_uint2(out[0], out[1]);
  if (c == 0) *d.meta = make_float2(a, s);
}

// Joined Q/K/V projection rows -> RoPE -> q, k, v ([heads, n, 64] each) with K
// and V also packed into the job's segment: the projection split,
// apply_rotary_pos_emb and GPUCache.append of the patched attention forward
// (src/gpu_cache.py:164-172) in one launch. One wave per (projection head,
// 8-token slice), 8 lanes per token row (16 bytes each): heads [0, q_heads)
// are Q, then `heads` K heads (rotated, packed), then `heads` V heads
// (packed). A 64-token chunk is 25 x 8 waves at the 960-wide decoder's
// shapes, so the per-row work (one row's quantization spread over its 8
// lanes) runs on many CUs at once; the arithmetic is quantize8's, so the bytes
// equal dkv_pack's for the same bf16 rows. With DEVJOB the job is read from
// device memory when the kernel runs (HIP graph replays); the projection, not
// the job's k/v pointers, is the source.
constexpr int RP_ROWS = 8;  // token rows per wave

template <bool DEVJOB>
__global__ void __launch_bounds__(PACK_THREADS)
rope_pack_kernel(const uint16_t* __restrict__ qkv, int64_t qkv_stride, const uint16_t* __restrict__ cosv,
                 const uint16_t* __restrict__ sinv, int64_t cs_stride, int n, int q_heads,
                 uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out, uint16_t* __restrict__ v_out,
                 dkv_pack_job hjob, const dkv_pack_job* __restrict__ djob, uint8_t* arena, dkv_tile* tiles,
                 int layers, int heads) {
  const int gw = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * (PACK_THREADS / 64) + (threadIdx.x >> 6)));
  const int slices = (n + RP_ROWS - 1) / RP_ROWS;
  const int hh = gw / slices;
  if (hh >= q_heads + 2 * heads) return;
  const int lane = threadIdx.x & 63;
  const int c = lane & 7;
  const int tok = (gw - hh * slices) * RP_ROWS + (lane >> 3);
  const bool valid = tok < n;
  const int t = valid ? tok : n - 1;  // rows past the end read the last row and store nothing
  const bool is_v = hh >= q_heads + heads;

  // Every load first, so that they form one round trip: the row, its cos and sin, and the pack job
  // (scalar loads). Placed by their uses (the rotation of Q and K rows, the pack of K and V rows),
  // they went out after the row had arrived: two more round trips. V rows are rotated too and
  // keep their input (a select, not a branch the loads could be moved into).
  const dkv_pack_job j = DEVJOB ? *djob : hjob;
  const u32x4 x = *reinterpret_cast<const u32x4*>(qkv + (int64_t)t * qkv_stride + hh * D + 8 * c);
  const int64_t o = (int64_t)t * cs_stride + 8 * c;
  const u32x4 cs = *reinterpret_cast<const u32x4*>(cosv + o);
  const u32x4 sn = *reinterpret_cast<const u32x4*>(sinv + o);
  asm volatile("" ::: "memory");  // the job's loads stay above it
  // rotate_half pairs column d with d +- 32: lane c with lane c ^ 4 of the same row
  u32x4 p;
#pragma unroll
  for (int e = 0; e < 4; ++e) p[e] = __shfl_xor(x[e], 4);
  const u32x4 rot = rope8(x, p, cs, sn, c < 4);
  const u32x4 w = is_v ? x : rot;
  uint16_t* dst = hh < q_heads ? q_out + (int64_t)hh * n * D
                               : (is_v ? v_out + (int64_t)(hh - q_heads - heads) * n * D
                                       : k_out + (int64_t)(hh - q_heads) * n * D);
  if (valid) *reinterpret_cast<u32x4*>(dst + (int64_t)tok * D + 8 * c) = w;

  if (gw == 0 && j.write_tiles) write_segment_tiles(j, layers, heads, tiles);
  if (hh < q_heads) return;
  const bool packs = valid && tok < j.n;  // rows the job packs
  const int kv = is_v ? 1 : 0;
  const int head = hh - q_heads - kv * heads;
  const int bits = __builtin_amdgcn_readfirstlane(j.bits);
  if (bits == 4) pack_row8<4>(j, kv, head, tok, packs, c, w, arena, layers, heads);
  else if (bits == 8) pack_row8<8>(j, kv, head, tok, packs, c, w, arena, layers, heads);
  else pack_row8<16>(j, kv, head, tok, packs, c, w, arena, layers, heads);
}

static int pack_waves(int n, int heads) { return 2 * heads * ((n + WAVE_ROWS - 1) / WAVE_ROWS); }

static int pack_blocks(int n, int heads) {
  return (pack_waves(n, heads) + PACK_THREADS / 64 - 1) / (PACK_THREADS / 64);
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
  const int64_t end = segment_end(j.seg_offset, j.seg_rows, j.bits, layers, heads);
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
  const int blocks = pack_blocks(job->n, heads);
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
  if (!jobs || !arena || n_jobs < 0 || max_n < 0 || layers <= 0 || heads <= 0 ||
      (int64_t)n_jobs * pack_waves(max_n > 0 ? max_n : 1, heads) > INT32_MAX / 2) {
    set_error("dkv_pack_batch: bad arguments (jobs %p, n_jobs %d, max_n %d)", (const void*)jobs, n_jobs, max_n);
    return DKV_EINVAL;
  }
  if (n_jobs == 0) return 0;
  const int wpj = pack_waves(max_n > 0 ? max_n : 1, heads);
  const int64_t blocks = ((int64_t)n_jobs * wpj + PACK_THREADS / 64 - 1) / (PACK_THREADS / 64);
  hipLaunchKernelGGL(pack_batch_kernel, dim3((unsigned)blocks), dim3(PACK_THREADS), 0, (hipStream_t)stream, jobs,
                     n_jobs, wpj, static_cast<uint8_t*>(arena), tiles, layers, heads);
  return (int)hipGetLastError();
}

int dkv_rope_pack(const void* qkv, int64_t qkv_row_stride, const void* cos, const void* sin, int64_t cs_row_stride,
                  int32_t n, int32_t q_heads, void* q_out, void* k_out, void* v_out, const dkv_pack_job* job,
                  int32_t job_on_device, void* arena, int64_t arena_bytes, dkv_tile* tiles, int32_t layers,
                  int32_t heads, void* stream) {
  clear_error();
  if (!qkv || !cos || !sin || !q_out || !k_out || !v_out || !job || !arena || !tiles || n < 0 || q_heads <= 0 ||
      heads <= 0 || layers <= 0 || !aligned16(qkv) || !aligned16(cos) || !aligned16(sin) || !aligned16(q_out) ||
      !aligned16(k_out) || !aligned16(v_out) || (qkv_row_stride & 7) || (cs_row_stride & 7) ||
      qkv_row_stride < (int64_t)(q_heads + 2 * heads) * D || cs_row_stride < D) {
    set_error("dkv_rope_pack: bad arguments (16-byte aligned bf16 buffers, strides multiples of 8 elements)");
    return DKV_EINVAL;
  }
  if (job_on_device) {
    if (n < 1) {
      set_error("dkv_rope_pack: a device job needs a chunk of at least one token");
      return DKV_EINVAL;
    }
  } else {
    if (int rc = check_job(*job, arena_bytes, layers, heads)) return rc;
    if (job->n != n) {
      set_error("dkv_rope_pack: the job appends %d tokens, the projection holds %d", job->n, n);
      return DKV_EINVAL;
    }
    if (job->write_tiles && job->tile_index0 < 0) {
      set_error("dkv_rope_pack: write_tiles at a negative tile index");
      return DKV_EINVAL;
    }
  }
  if (n == 0) {  // nothing to rotate; the append may still open a segment
    if (!job->write_tiles) return 0;
    hipLaunchKernelGGL(pack_one_kernel, dim3(1), dim3(PACK_THREADS), 0, (hipStream_t)stream, *job,
                       static_cast<uint8_t*>(arena), tiles, layers, heads);
    return (int)hipGetLastError();
  }
  const int64_t waves = (int64_t)(q_heads + 2 * heads) * ((n + RP_ROWS - 1) / RP_ROWS);
  const unsigned blocks = (unsigned)((waves + PACK_THREADS / 64 - 1) / (PACK_THREADS / 64));
  const dkv_pack_job none = {};
  const auto* qp = static_cast<const uint16_t*>(qkv);
  const auto* cp = static_cast<const uint16_t*>(cos);
  const auto* sp = static_cast<const uint16_t*>(sin);
  auto* qo = static_cast<uint16_t*>(q_out);
  auto* ko = static_cast<uint16_t*>(k_out);
  auto* vo = static_cast<uint16_t*>(v_out);
  if (job_on_device)
    hipLaunchKernelGGL(rope_pack_kernel<true>, dim3(blocks), dim3(PACK_THREADS), 0, (hipStream_t)stream, qp,
                       qkv_row_stride, cp, sp, cs_row_stride, n, q_heads, qo, ko, vo, none, job,
                       static_cast<uint8_t*>(arena), tiles, layers, heads);
  else
    hipLaunchKernelGGL(rope_pack_kernel<false>, dim3(blocks), dim3(PACK_THREADS), 0, (hipStream_t)stream, qp,
                       qkv_row_stride, cp, sp, cs_row_stride, n, q_heads, qo, ko, vo, *job,
                       (const dkv_pack_job*)nullptr, static_cast<uint8_t*>(arena), tiles, layers, heads);
  return (int)hipGetLastError();
}

int dkv_pack_validate(const dkv_pack_job* jobs, int32_t n_jobs, int64_t arena_bytes, int32_t layers,
                      int32_t heads) {
  clear_error();
  if ((!jobs && n_jobs > 0) || n_jobs < 0) {
    set_error("dkv_pack_validate: bad job array");
    return DKV_EINVAL;
  }
  for (int i = 0; i < n_jobs; ++i) {
    if (int rc = check_job(jobs[i], arena_bytes, layers, heads)) return rc;
    if (jobs[i].write_tiles && jobs[i].tile_index0 < 0) {
      set_error("dkv_pack_validate: job %d writes tiles at a negative index", i);
      return DKV_EINVAL;
    }
  }
  return 0;
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
