// Split merges of the attention kernels: the arithmetic of one query row, run by one wave
// (merge_row_f32, merge_row_half) or by the waves of one workgroup (merge_row_*_wide, for launches
// with few query rows). The merge kernels (a second launch) and the frame-chunk kernel's in-kernel
// merge (the last workgroup of a KV head to finish) both call the one-wave form, so where the
// merge kernel takes it either path stores the same bits; the wide form sums the same terms in
// another order.
//
// A wave's lanes are (j, c): c picks a 16-byte chunk of the row, j a residue of the split index.
// Each lane loads the (max, sum) pair of every split it reads beside that split's O chunk, so the
// loads form one round trip and each lane computes its own splits' weights. The only exchanges
// are reductions over j, done on the VALU (DPP row_ror and the gfx950 permlane swaps) rather than
// through LDS: a chain of dependent ds_bpermute shuffles made most of the merge's latency.
#pragma once
#include "dkv_attn_common.h"

namespace dkv {

typedef float merge_f32x2 __attribute__((ext_vector_type(2)));

// Partials of launches with few query rows (one 16-row block per wave) are written with plain
// stores and read with plain loads: they are small, the end of the producing kernel writes them
// back from L2 at little cost, and the merge then reads them from the cache hierarchy. Larger
// partials use nontemporal stores and loads, which keep them from displacing the history.
template <bool PLAIN, typename T>
__device__ __forceinline__ T merge_load(const T* p) {
  if constexpr (PLAIN)
    return *p;
  else
    return __builtin_nontemporal_load(p);
}

// x combined with the value of lane l ^ 8 (DPP row_ror:8 inside each row of 16 lanes).
__device__ __forceinline__ float lane_xor8(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xf, 0xf, false));
}

// Reductions over lanes l ^ 16 and l ^ 32 (permlane32_swap, then permlane16_swap). Every lane
// ends with the same operands in the same order, so all lanes hold identical bits.
__device__ __forceinline__ float max_over_hi(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float sum_over_hi(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// Precision-1 merge state over splits [s_begin, s_end) (unnormalized fp32 O partials, 256 bytes
// per row), in one wave (lane = threadIdx.x % 64). Lane l = 16 j + c reads 16-byte chunk c
// (columns 4c + [0, 4)) and the (max, sum) of split s0 + 4 i + j for i = 0..PER-1, so each load
// instruction covers 4 splits, and accumulates them weighted by 2^(m_s - M). M and L end equal on
// every lane; acc is lane (j, c)'s share of chunk c, summed over j by the caller.
template <bool PLAIN, int PER>
__device__ __forceinline__ void merge_f32_range(int64_t base, int R, int s_begin, int s_end,
                                                const float* __restrict__ part_o,
                                                const float2* __restrict__ part_ml, float& M, float& L,
                                                float (&acc)[4]) {
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, c = lane & 15;
  const u32x4* rows = reinterpret_cast<const u32x4*>(part_o);  // 16 chunks of 16 bytes per row
  const merge_f32x2* mls = reinterpret_cast<const merge_f32x2*>(part_ml);
  for (int s0 = s_begin; s0 < s_end; s0 += 4 * PER) {
    const int cnt = min(4 * PER, s_end - s0);
    merge_f32x2 ml[PER];
    u32x4 raw[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i)  // splits past cnt load split cnt - 1 (no branches) and weigh 0
      ml[i] = merge_load<PLAIN>(mls + base + (int64_t)(s0 + min(4 * i + j, cnt - 1)) * R);
#pragma unroll
    for (int i = 0; i < PER; ++i)
      raw[i] = merge_load<PLAIN>(rows + (base + (int64_t)(s0 + min(4 * i + j, cnt - 1)) * R) * 16 + c);
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the first wait (one round trip)
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (4 * i + j >= cnt) ml[i].x = -INFINITY;
    float bm = ml[0].x;
#pragma unroll
    for (int i = 1; i < PER; ++i) bm = fmaxf(bm, ml[i].x);
    bm = fmaxf(max_over_hi(bm), M);
    // No branch on bm == -inf (no split so far saw a visible key): then every weight and f0 are 0
    // and the state stays (M, L, acc) = (-inf, 0, 0); a branch would sink the O loads below it.
    float w[PER], lsum = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      w[i] = ml[i].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml[i].x - bm);
      lsum = fmaf(ml[i].y, w[i], lsum);
    }
    lsum = sum_over_hi(lsum);
    const float f0 = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - bm);
    L = fmaf(L, f0, lsum);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] *= f0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float4 v = __builtin_bit_cast(float4, raw[i]);
      acc[0] = fmaf(v.x, w[i], acc[0]);
      acc[1] = fmaf(v.y, w[i], acc[1]);
      acc[2] = fmaf(v.z, w[i], acc[2]);
      acc[3] = fmaf(v.w, w[i], acc[3]);
    }
    M = bm;
  }
}

// Stores columns 4c + [0, 4) of merged row r (acc / L) in the output's dtype.
__device__ __forceinline__ void store_f32_row(const dkv_attn_args& a, int h, int r, int G, int c,
                                              const float (&acc)[4], float L) {
  const float inv = 1.f / L;
  const float v0 = acc[0] * inv, v1 = acc[1] * inv, v2 = acc[2] * inv, v3 = acc[3] * inv;
  const int gq = r / a.nq, m = r - gq * a.nq;
  const int64_t off = (int64_t)m * a.out_tok_stride + (int64_t)(h * G + gq) * a.out_head_stride + 4 * c;
  if (a.out_dtype == 1)
    *reinterpret_cast<float4*>(static_cast<float*>(a.out) + off) = make_float4(v0, v1, v2, v3);
  else
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + off) = make_uint2(
        f32_to_bf16_rne(v0) | (f32_to_bf16_rne(v1) << 16), f32_to_bf16_rne(v2) | (f32_to_bf16_rne(v3) << 16));
}

// Precision-1 merge of one query row by one wave: every split in passes of 64, then sums over j
// (lanes 16 and 32 apart), and lanes 0..15 store the row.
template <bool PLAIN = false>
__device__ __forceinline__ void merge_row_f32(const dkv_attn_args& a, int h, int r, int R, int G, int splits,
                                              int active, const float* __restrict__ part_o,
                                              const float2* __restrict__ part_ml) {
  const int lane = threadIdx.x & 63;
  float M = -INFINITY, L = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
  merge_f32_range<PLAIN, 16>((int64_t)h * splits * R + r, R, 0, active, part_o, part_ml, M, L, acc);
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = sum_over_hi(acc[e]);
  if (lane < 16)  // j == 0 (a guarded store, not an early return: callers loop over rows)
    store_f32_row(a, h, r, G, lane, acc, L);
}

// Precision-0 merge state over splits [s_begin, s_end) (fp16 O / sum partials, 128 bytes per row
// in half_slot() order), in one wave. Lane l = 8 j + c reads 16-byte chunk c and the (max, sum) of
// split s0 + 8 i + j for i = 0..PER-1, so each load instruction covers 8 splits, and accumulates 8
// columns weighted by that split's sum * 2^(m_s - M). M and L end equal on every lane; acc is lane
// (j, c)'s share of chunk c, summed over j by the caller. A pass reads 8 * PER splits with one
// round trip.
template <bool PLAIN, int PER>
__device__ __forceinline__ void merge_half_range(int64_t base, int R, int s_begin, int s_end,
                                                 const float* __restrict__ part_o,
                                                 const float2* __restrict__ part_ml, float& M, float& L,
                                                 float (&acc)[8]) {
  const int lane = threadIdx.x & 63;
  const int j = lane >> 3, c = lane & 7;
  const u32x4* rows = reinterpret_cast<const u32x4*>(part_o);  // 8 chunks of 16 bytes per row
  const merge_f32x2* mls = reinterpret_cast<const merge_f32x2*>(part_ml);
  for (int s0 = s_begin; s0 < s_end; s0 += 8 * PER) {
    const int cnt = min(8 * PER, s_end - s0);
    merge_f32x2 ml[PER];
    u32x4 raw[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i)  // splits past cnt load split cnt - 1 (no branches) and weigh 0
      ml[i] = merge_load<PLAIN>(mls + base + (int64_t)(s0 + min(8 * i + j, cnt - 1)) * R);
#pragma unroll
    for (int i = 0; i < PER; ++i)
      raw[i] = merge_load<PLAIN>(rows + (base + (int64_t)(s0 + min(8 * i + j, cnt - 1)) * R) * 8 + c);
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the first wait (one round trip)
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (8 * i + j >= cnt) ml[i].x = -INFINITY;
    float bm = ml[0].x;
#pragma unroll
    for (int i = 1; i < PER; ++i) bm = fmaxf(bm, ml[i].x);
    bm = fmaxf(bm, lane_xor8(bm));
    bm = fmaxf(max_over_hi(bm), M);
    // No branch on bm == -inf, as in merge_f32_range.
    float w[PER], lsum = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float f = ml[i].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml[i].x - bm);
      int ex;
      const float ls = half_partial_decode(ml[i].y, ex) * f;
      w[i] = ex ? __builtin_amdgcn_ldexpf(ls, ex) : ls;  // weight of the stored O / sum / 2^ex
      lsum += ls;
    }
    lsum += lane_xor8(lsum);
    lsum = sum_over_hi(lsum);
    const float f0 = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - bm);
    L = fmaf(L, f0, lsum);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= f0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint32_t q[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(q[e] & 0xffffu));
        const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(q[e] >> 16));
        acc[2 * e] = fmaf((float)lo, w[i], acc[2 * e]);
        acc[2 * e + 1] = fmaf((float)hi, w[i], acc[2 * e + 1]);
      }
    }
    M = bm;
  }
}

// Stores the 8 columns of slots 8c + [0, 8) of merged row r (acc / L) in the output's dtype.
__device__ __forceinline__ void store_half_row(const dkv_attn_args& a, int h, int r, int G, int c,
                                               const float (&acc)[8], float L) {
  const float inv = 1.f / L;
  const int gq = r / a.nq, m = r - gq * a.nq;
  const int64_t off = (int64_t)m * a.out_tok_stride + (int64_t)(h * G + gq) * a.out_head_stride;
#pragma unroll
  for (int half = 0; half < 2; ++half) {  // slots 8c + 4 half + [0, 4): 4 consecutive columns
    const int col = half_column(8 * c + 4 * half);
    const float v0 = acc[4 * half] * inv, v1 = acc[4 * half + 1] * inv;
    const float v2 = acc[4 * half + 2] * inv, v3 = acc[4 * half + 3] * inv;
    if (a.out_dtype == 1)
      *reinterpret_cast<float4*>(static_cast<float*>(a.out) + off + col) = make_float4(v0, v1, v2, v3);
    else
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + off + col) = make_uint2(
          f32_to_bf16_rne(v0) | (f32_to_bf16_rne(v1) << 16), f32_to_bf16_rne(v2) | (f32_to_bf16_rne(v3) << 16));
  }
}

// Precision-0 merge of one query row by one wave: every split in passes of 8 * PER (64 for
// nontemporal partials; 128 for the plainly stored partials of decode steps, which would
// otherwise take two dependent passes), then sums over j (lanes 8, 16 and 32 apart), and lanes
// 0..7 store the row.
template <bool PLAIN = false>
__device__ __forceinline__ void merge_row_half(const dkv_attn_args& a, int h, int r, int R, int G, int splits,
                                               int active, const float* __restrict__ part_o,
                                               const float2* __restrict__ part_ml) {
  const int lane = threadIdx.x & 63;
  float M = -INFINITY, L = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  merge_half_range<PLAIN, PLAIN ? 16 : 8>((int64_t)h * splits * R + r, R, 0, active, part_o, part_ml, M, L, acc);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    acc[e] += lane_xor8(acc[e]);
    acc[e] = sum_over_hi(acc[e]);
  }
  if (lane < 8)  // j == 0 (a guarded store, not an early return: callers loop over rows)
    store_half_row(a, h, r, G, lane, acc, L);
}

// One query row merged by the W waves of a workgroup (256 threads for W = 4): wave w takes splits
// [active w / W, active (w + 1) / W) in passes of 8 * PER (precision 0) or 4 * PER (precision 1),
// sums its lanes over j, and leaves its (M, L) and column sums in LDS; wave 0 then combines the W
// states in wave order (deterministic) and stores the row. Each wave waits on a quarter of the
// loads and does a quarter of the arithmetic of the one-wave merge, which runs with one wave per
// SIMD and so pays the full latency of every dependent instruction.
template <bool PLAIN, int W>
__device__ __forceinline__ void merge_row_half_wide(const dkv_attn_args& a, int h, int r, int R, int G, int splits,
                                                    int active, const float* __restrict__ part_o,
                                                    const float2* __restrict__ part_ml) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float M = -INFINITY, L = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  merge_half_range<PLAIN, 4>((int64_t)h * splits * R + r, R, active * wave / W, active * (wave + 1) / W, part_o,
                             part_ml, M, L, acc);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    acc[e] += lane_xor8(acc[e]);
    acc[e] = sum_over_hi(acc[e]);
  }
  __shared__ float wacc[W][8][8];
  __shared__ merge_f32x2 wml[W];
  if (lane < 8)
#pragma unroll
    for (int e = 0; e < 8; ++e) wacc[wave][lane][e] = acc[e];
  if (lane == 0) wml[wave] = merge_f32x2{M, L};
  __syncthreads();
  if (wave == 0 && lane < 8) {
    float mx = wml[0].x;
#pragma unroll
    for (int w = 1; w < W; ++w) mx = fmaxf(mx, wml[w].x);
    float lt = 0.f, o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const merge_f32x2 ml = wml[w];
      const float f = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml.x - mx);
      lt = fmaf(ml.y, f, lt);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = fmaf(wacc[w][lane][e], f, o[e]);
    }
    store_half_row(a, h, r, G, lane, o, lt);
  }
}

// merge_row_half_wide for precision 1 (16 chunks of 4 columns per row).
template <bool PLAIN, int W>
__device__ __forceinline__ void merge_row_f32_wide(const dkv_attn_args& a, int h, int r, int R, int G, int splits,
                                                   int active, const float* __restrict__ part_o,
                                                   const float2* __restrict__ part_ml) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float M = -INFINITY, L = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
  merge_f32_range<PLAIN, 4>((int64_t)h * splits * R + r, R, active * wave / W, active * (wave + 1) / W, part_o,
                            part_ml, M, L, acc);
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = sum_over_hi(acc[e]);
  __shared__ float wacc[W][16][4];
  __shared__ merge_f32x2 wml[W];
  if (lane < 16)
#pragma unroll
    for (int e = 0; e < 4; ++e) wacc[wave][lane][e] = acc[e];
  if (lane == 0) wml[wave] = merge_f32x2{M, L};
  __syncthreads();
  if (wave == 0 && lane < 16) {
    float mx = wml[0].x;
#pragma unroll
    for (int w = 1; w < W; ++w) mx = fmaxf(mx, wml[w].x);
    float lt = 0.f, o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const merge_f32x2 ml = wml[w];
      const float f = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml.x - mx);
      lt = fmaf(ml.y, f, lt);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = fmaf(wacc[w][lane][e], f, o[e]);
    }
    store_f32_row(a, h, r, G, lane, o, lt);
  }
}

}  // namespace dkv
