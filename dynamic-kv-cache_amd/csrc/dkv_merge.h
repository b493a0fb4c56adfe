// Split merges of the attention kernels: the arithmetic of one query row, run by one wave. The
// merge kernels (a second launch) and the frame-chunk kernel's in-kernel merge (the last workgroup
// of a KV head to finish) both call these, so either path stores the same bits.
#pragma once
#include "dkv_attn_common.h"

namespace dkv {

// Precision-1 merge (unnormalized fp32 O partials, 256 bytes per row): one wave per query row
// (lane = threadIdx.x % 64). Lane l = 16 j + c reads 16-byte chunk c (columns 4c + [0, 4)) of
// split s0 + 4 i + j for i = 0..15, so each load instruction covers 4 splits, and accumulates them
// weighted by 2^(m_s - M), computed once on lane s and fetched with a shuffle. The 4 lanes of one
// chunk are summed at the end, and lanes 0..15 store the row.
__device__ __forceinline__ void merge_row_f32(const dkv_attn_args& a, int h, int r, int R, int G, int splits,
                                              int active, const float* __restrict__ part_o,
                                              const float2* __restrict__ part_ml) {
  const int lane = threadIdx.x & 63;
  const int64_t base = (int64_t)h * splits * R + r;
  const int j = lane >> 4, c = lane & 15;
  const float4* rows = reinterpret_cast<const float4*>(part_o);  // 16 chunks of 16 bytes per row
  float M = -INFINITY, L = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < active; s0 += 64) {
    const int cnt = min(64, active - s0);
    const float2 ml = lane < cnt ? part_ml[base + (int64_t)(s0 + lane) * R] : make_float2(-INFINITY, 0.f);
    float4 raw[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int sp = 4 * i + j;
      const u32x4* src = reinterpret_cast<const u32x4*>(rows) + (base + (int64_t)(s0 + sp) * R) * 16 + c;
      raw[i] = sp < cnt ? __builtin_bit_cast(float4, __builtin_nontemporal_load(src)) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float bm = ml.x;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) bm = fmaxf(bm, __shfl_xor(bm, o));
    bm = fmaxf(bm, M);
    if (bm == -INFINITY) continue;  // wave-uniform: every split so far saw no visible key
    const float f = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml.x - bm);
    float lsum = ml.y * f;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) lsum += __shfl_xor(lsum, o);
    const float f0 = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - bm);
    L = fmaf(L, f0, lsum);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] *= f0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float w = __shfl(f, 4 * i + j);  // 0 for splits past cnt
      acc[0] = fmaf(raw[i].x, w, acc[0]);
      acc[1] = fmaf(raw[i].y, w, acc[1]);
      acc[2] = fmaf(raw[i].z, w, acc[2]);
      acc[3] = fmaf(raw[i].w, w, acc[3]);
    }
    M = bm;
  }
#pragma unroll
  for (int o = 16; o < 64; o <<= 1)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += __shfl_xor(acc[e], o);
  if (j == 0) {  // lanes 0..15 store the row (a guarded store, not an early return: callers loop over rows)
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
}

// Precision-0 merge (fp16 O / sum partials, 128 bytes per row in half_slot()
// order): one wave per query row. Lane l = 8 j + c reads 16-byte chunk c of
// split s0 + 8 i + j for i = 0..7, so each load instruction covers 8 splits,
// and accumulates 8 columns weighted by that split's sum * 2^(m_s - M)
// (fetched from lane s with a shuffle). The 8 lanes of one chunk are summed
// at the end, and lanes 0..7 store the row.
__device__ __forceinline__ void merge_row_half(const dkv_attn_args& a, int h, int r, int R, int G, int splits,
                                               int active, const float* __restrict__ part_o,
                                               const float2* __restrict__ part_ml) {
  const int lane = threadIdx.x & 63;
  const int64_t base = (int64_t)h * splits * R + r;
  const int j = lane >> 3, c = lane & 7;
  const uint4* rows = reinterpret_cast<const uint4*>(part_o);  // 8 chunks of 16 bytes per row
  float M = -INFINITY, L = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int s0 = 0; s0 < active; s0 += 64) {
    const int cnt = min(64, active - s0);
    const float2 ml = lane < cnt ? part_ml[base + (int64_t)(s0 + lane) * R] : make_float2(-INFINITY, 0.f);
    uint4 raw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int s = 8 * i + j;
      const u32x4* src = reinterpret_cast<const u32x4*>(rows) + (base + (int64_t)(s0 + s) * R) * 8 + c;
      raw[i] = s < cnt ? __builtin_bit_cast(uint4, __builtin_nontemporal_load(src)) : make_uint4(0, 0, 0, 0);
    }
    float bm = ml.x;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) bm = fmaxf(bm, __shfl_xor(bm, o));
    bm = fmaxf(bm, M);
    if (bm == -INFINITY) continue;  // wave-uniform: every split so far saw no visible key
    const float f = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml.x - bm);
    int ex;
    float lsum = half_partial_decode(ml.y, ex) * f;
    const float wsplit = ex ? __builtin_amdgcn_ldexpf(lsum, ex) : lsum;  // weight of the stored O / sum / 2^ex
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) lsum += __shfl_xor(lsum, o);
    const float f0 = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - bm);
    L = fmaf(L, f0, lsum);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= f0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float w = __shfl(wsplit, 8 * i + j);  // 0 for splits past cnt
      const uint32_t q[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(q[e] & 0xffffu));
        const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(q[e] >> 16));
        acc[2 * e] = fmaf((float)lo, w, acc[2 * e]);
        acc[2 * e + 1] = fmaf((float)hi, w, acc[2 * e + 1]);
      }
    }
    M = bm;
  }
#pragma unroll
  for (int o = 8; o < 64; o <<= 1)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], o);
  if (j == 0) {  // lanes 0..7 store the row (a guarded store, not an early return: callers loop over rows)
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
}

}  // namespace dkv
