// The decoder's pointwise operations around the packed-KV path, one launch
// each where the PyTorch compositions take two to ten:
//
//   rope_qkv_kernel   the joined Q/K/V projection row -> rotated q, k (RoPE) and
//                     v in [heads, n, 64] layout, bit-equal to transformers'
//                     apply_rotary_pos_emb in bf16 (q*cos + rotate_half(q)*sin,
//                     each product and the sum rounded to bf16), as the
//                     reference's patched attention forward calls it
//                     (src/gpu_cache.py:166-172);
//   rms_norm_kernel   rms_norm(x) * weight with torch's two bf16 roundings
//                     (src/gpu_ops.py:9-12);
//   silu_mul_kernel   silu(gate) * up over the joined gate/up projection, each
//                     op rounded to bf16 (src/gpu_ops.py:14-17).
//
// All three are bf16 in and out with fp32 arithmetic, memory-bound and tiny at
// decoder shapes (64-token chunks): what they save is launches.
#include "dkv_common.h"

namespace dkv {
namespace {

__device__ __forceinline__ void unpack8(const uint4& w, float* x) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = bf16_lo(ww[i]);
    x[2 * i + 1] = bf16_hi(ww[i]);
  }
}
__device__ __forceinline__ uint4 pack8(const float* x) {
  return make_uint4(pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3]), pack_bf16(x[4], x[5]), pack_bf16(x[6], x[7]));
}

// One thread = one token row of one head, eight elements of each half:
// columns [8c, 8c+8) and [32+8c, 32+8c+8), c = threadIdx.x & 3.
// Heads [0, q_heads) are Q, then kv_heads of K (both rotated), then V (copied).
__global__ void __launch_bounds__(256)
rope_qkv_kernel(const uint16_t* __restrict__ qkv, int64_t qkv_stride, const uint16_t* __restrict__ cosv,
                const uint16_t* __restrict__ sinv, int64_t cs_stride, int n, int q_heads, int kv_heads,
                uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out, uint16_t* __restrict__ v_out) {
  const int heads = q_heads + 2 * kv_heads;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  const int c = idx & 3;
  const int row = idx >> 2;  // (token, head)
  if (row >= n * heads) return;
  const int t = row / heads, h = row - t * heads;
  const uint16_t* src = qkv + (int64_t)t * qkv_stride + h * D;
  const uint4 w_lo = *reinterpret_cast<const uint4*>(src + 8 * c);
  const uint4 w_hi = *reinterpret_cast<const uint4*>(src + 32 + 8 * c);
  uint16_t* dst;
  if (h < q_heads) dst = q_out + ((int64_t)h * n + t) * D;
  else if (h < q_heads + kv_heads) dst = k_out + ((int64_t)(h - q_heads) * n + t) * D;
  else {
    dst = v_out + ((int64_t)(h - q_heads - kv_heads) * n + t) * D;
    *reinterpret_cast<uint4*>(dst + 8 * c) = w_lo;
    *reinterpret_cast<uint4*>(dst + 32 + 8 * c) = w_hi;
    return;
  }
  float x1[8], x2[8], c1[8], c2[8], s1[8], s2[8];
  unpack8(w_lo, x1);
  unpack8(w_hi, x2);
  const uint16_t* cp = cosv + (int64_t)t * cs_stride;
  const uint16_t* sp = sinv + (int64_t)t * cs_stride;
  unpack8(*reinterpret_cast<const uint4*>(cp + 8 * c), c1);
  unpack8(*reinterpret_cast<const uint4*>(cp + 32 + 8 * c), c2);
  unpack8(*reinterpret_cast<const uint4*>(sp + 8 * c), s1);
  unpack8(*reinterpret_cast<const uint4*>(sp + 32 + 8 * c), s2);
  float y1[8], y2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // rotate_half(x) = (-x2, x1); bf16 products of bf16 values are exact in fp32,
    // so rounding each product and the sum reproduces the three bf16 torch ops.
    y1[i] = round_bf16(round_bf16(x1[i] * c1[i]) + round_bf16(-x2[i] * s1[i]));
    y2[i] = round_bf16(round_bf16(x2[i] * c2[i]) + round_bf16(x1[i] * s2[i]));
  }
  *reinterpret_cast<uint4*>(dst + 8 * c) = pack8(y1);
  *reinterpret_cast<uint4*>(dst + 32 + 8 * c) = pack8(y2);
}

// One wave per row: sum of squares in fp32 over the row, then
// y = bf16(bf16(x * rsqrt(mean + eps)) * w).
__global__ void __launch_bounds__(256)
rms_norm_kernel(const uint16_t* __restrict__ x, int64_t x_stride, const uint16_t* __restrict__ wgt,
                uint16_t* __restrict__ out, int64_t out_stride, int rows, int dim, float eps) {
  const int row = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const uint16_t* xr = x + (int64_t)row * x_stride;
  float ss = 0.f;
  for (int c = lane; c < dim / 8; c += 64) {
    float v[8];
    unpack8(*reinterpret_cast<const uint4*>(xr + 8 * c), v);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __fmaf_rn(v[i], v[i], ss);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const float rstd = 1.f / sqrtf(ss / (float)dim + eps);
  uint16_t* orow = out + (int64_t)row * out_stride;
  for (int c = lane; c < dim / 8; c += 64) {
    float v[8], w[8];
    unpack8(*reinterpret_cast<const uint4*>(xr + 8 * c), v);
    unpack8(*reinterpret_cast<const uint4*>(wgt + 8 * c), w);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = round_bf16(v[i] * rstd) * w[i];
    *reinterpret_cast<uint4*>(orow + 8 * c) = pack8(v);
  }
}

// One thread = eight columns of one row: out = bf16(bf16(silu(g)) * u), with
// silu(g) = g / (1 + exp(-g)) in fp32.
__global__ void __launch_bounds__(256)
silu_mul_kernel(const uint16_t* __restrict__ gu, int64_t gu_stride, uint16_t* __restrict__ out,
                int64_t out_stride, int rows, int inter) {
  const int per_row = inter / 8;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * per_row) return;
  const int row = idx / per_row, c = idx - row * per_row;
  const uint16_t* src = gu + (int64_t)row * gu_stride + 8 * c;
  float g[8], u[8];
  unpack8(*reinterpret_cast<const uint4*>(src), g);
  unpack8(*reinterpret_cast<const uint4*>(src + inter), u);
#pragma unroll
  for (int i = 0; i < 8; ++i) g[i] = round_bf16(g[i] / (1.f + expf(-g[i]))) * u[i];
  *reinterpret_cast<uint4*>(out + (int64_t)row * out_stride + 8 * c) = pack8(g);
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace
}  // namespace dkv

using namespace dkv;

extern "C" {

int dkv_rope_qkv(const void* qkv, int64_t qkv_row_stride, const void* cos, const void* sin, int64_t cs_row_stride,
                 int32_t n, int32_t q_heads, int32_t kv_heads, void* q_out, void* k_out, void* v_out,
                 void* stream) {
  clear_error();
  if (!qkv || !cos || !sin || !q_out || !k_out || !v_out || n < 0 || q_heads <= 0 || kv_heads <= 0 ||
      !al16(qkv) || !al16(cos) || !al16(sin) || !al16(q_out) || !al16(k_out) || !al16(v_out) ||
      (qkv_row_stride & 7) || (cs_row_stride & 7) || qkv_row_stride < (int64_t)(q_heads + 2 * kv_heads) * D ||
      cs_row_stride < D) {
    set_error("dkv_rope_qkv: bad arguments (16-byte aligned bf16 buffers, strides multiples of 8 elements)");
    return DKV_EINVAL;
  }
  const int64_t threads = (int64_t)n * (q_heads + 2 * kv_heads) * 4;
  if (threads == 0) return 0;
  hipLaunchKernelGGL(rope_qkv_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint16_t*>(qkv), qkv_row_stride, static_cast<const uint16_t*>(cos),
                     static_cast<const uint16_t*>(sin), cs_row_stride, n, q_heads, kv_heads,
                     static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out), static_cast<uint16_t*>(v_out));
  return (int)hipGetLastError();
}

int dkv_rms_norm(const void* x, int64_t x_row_stride, const void* weight, void* out, int64_t out_row_stride,
                 int32_t rows, int32_t dim, float eps, void* stream) {
  clear_error();
  if (!x || !weight || !out || rows < 0 || dim <= 0 || (dim & 7) || !al16(x) || !al16(weight) || !al16(out) ||
      (x_row_stride & 7) || (out_row_stride & 7) || x_row_stride < dim || out_row_stride < dim) {
    set_error("dkv_rms_norm: bad arguments (16-byte aligned bf16 rows, dim a multiple of 8)");
    return DKV_EINVAL;
  }
  if (rows == 0) return 0;
  hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint16_t*>(x), x_row_stride, static_cast<const uint16_t*>(weight),
                     static_cast<uint16_t*>(out), out_row_stride, rows, dim, eps);
  return (int)hipGetLastError();
}

int dkv_silu_mul(const void* gate_up, int64_t row_stride, void* out, int64_t out_row_stride, int32_t rows,
                 int32_t inter, void* stream) {
  clear_error();
  if (!gate_up || !out || rows < 0 || inter <= 0 || (inter & 7) || !al16(gate_up) || !al16(out) ||
      (row_stride & 7) || (out_row_stride & 7) || row_stride < 2 * (int64_t)inter || out_row_stride < inter) {
    set_error("dkv_silu_mul: bad arguments (16-byte aligned bf16 rows, inter a multiple of 8)");
    return DKV_EINVAL;
  }
  const int64_t threads = (int64_t)rows * (inter / 8);
  if (threads == 0) return 0;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint16_t*>(gate_up), row_stride, static_cast<uint16_t*>(out), out_row_stride,
                     rows, inter);
  return (int)hipGetLastError();
}

}  // extern "C"
