// Short-chunk path of the fused packed-history attention (gfx950), path 3:
// decode steps and other chunks with at most 16 query rows per KV head
// (G * nq <= 16, e.g. one to five tokens of a 3-way GQA decoder), where the
// whole job is to stream the packed history once. The auto path takes the
// frame-chunk kernel for these too, which measured faster at every history
// length; this kernel stays as a second implementation.
//
// Work split: two waves own one 64-key unit (a history tile, or the chunk's
// own native rows), one 32-key half each; a workgroup of 8 waves owns a
// contiguous range of units of one KV head, four at a time, and the grid covers
// the history in ceil(units / 4) workgroups per head by default, so every
// tile's bytes are requested when the kernel starts. There is no barrier
// between the waves until the end:
//   - K goes from its loaded bytes straight into the MFMA A operand of
//     S^T = K Q^T (v_mfma_f32_16x16x32_bf16, keys on M, the <= 16 query rows on
//     N). The dot product runs over d in any order as long as K and Q agree, so
//     lane (i, g) holds d in [16g, 16g + 16) of its key: one contiguous slice of
//     the packed row (8, 16 or 32 bytes for 4, 8 or 16 bits);
//   - the keys of the A rows are permuted (key 8g' + 4j + i of a 32-key half
//     sits in row 4g' + i of S block j) so that the S^T accumulators are
//     exactly the P^T operand of O^T = V^T P^T: p never leaves registers;
//   - every register a unit's loads fill is loaded exactly once and
//     unconditionally (rows past the tile's end load row 0 and are zeroed
//     after), so all of a unit's loads are in flight together;
//   - V is dequantized from registers into the wave's own transposed bf16 tile
//     in LDS ([d][key] of its 32 keys), the A operand of O^T = V^T P^T;
//   - the online softmax over the unit's keys runs in base 2 per query column,
//     with the reference kernel's bf16 rounding of K, V and p at precision 0
//     (src/gpu_kernels.py:93-102) and hi/lo bf16 pairs at precision 1 (as the
//     frame-chunk kernel does).
// After its units the workgroup merges its 8 waves' (max, sum, O) in LDS and
// stores the output (one workgroup per head) or its partial, which
// combine_kernel merges. (Merging in the last-arriving workgroup of a head, with
// agent-scope stores, an arrival counter and agent-scope loads, measured no
// faster than the second launch: the write-through stores and the loads that
// bypass the XCD's L2 cost about as much as the launch they replace.)
#include "dkv_attn_common.h"

namespace dkv {
namespace shortpath {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int THREADS = 512;   // 8 waves
constexpr int WAVES = 8;
constexpr int UNIT_SLOTS = WAVES / 2;  // units a workgroup works on at once (two waves per unit)
constexpr int VT = 40;         // bf16 row stride of a wave's V^T tile [64 d][32 keys + 8 pad]
constexpr int VT_BYTES = D * VT * 2;

union Pack8 {
  bf16x8 v;
  uint4 u;
};

__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
}
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Max / sum over the four lanes col, col + 16, col + 32, col + 48 (one query column).
__device__ __forceinline__ float col_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = max_nn(__uint_as_float(r[0]), __uint_as_float(r[1]));
  auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_nn(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float col_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The bytes of 16 values [e0, e0 + 16) of row `row` of a unit's K (kv 0) or V
// (kv 1), and the row's (offset, scale), issued so that the compiler can keep
// every load of a unit in flight at once: each destination register is loaded
// exactly once, unconditionally, and only the second 16 bytes of a 16-bit row
// (w1) sit behind a (wave-uniform) branch, whose other path does not write
// them. A row at or past `valid` loads row 0 (every unit has one) and is zeroed
// after the load (dequant16). 4-bit values land in w0.xy or w0.zw, 8-bit in w0,
// 16-bit in w0 and w1.
__device__ __forceinline__ void load16(const dkv_attn_args& a, const Unit& un, int h, int kv, int row, int e0,
                                       uint4& w0, uint4& w1, float2& as) {
  const int rr = row < un.valid ? row : 0;
  const uint8_t* base;
  int64_t off;
  if (un.chunk) {
    const int64_t j = un.first + rr;
    base = kv == 0 ? static_cast<const uint8_t*>(a.k_new) + 2 * (h * a.kn_head_stride + j * a.kn_tok_stride)
                   : static_cast<const uint8_t*>(a.v_new) + 2 * (h * a.vn_head_stride + j * a.vn_tok_stride);
    off = 2 * e0;
  } else {
    base = (kv == 0 ? un.ksub : un.vsub) + (int64_t)rr * row_bytes(un.bits);
    off = un.bits == 4 ? (e0 >> 5) * 16 : (un.bits == 8 ? e0 : 2 * e0);  // 4-bit: the 16 bytes holding 32 values
  }
  const u32x4* src = reinterpret_cast<const u32x4*>(base + off);
  w0 = __builtin_bit_cast(uint4, __builtin_nontemporal_load(src));
  if (un.bits == 16) w1 = __builtin_bit_cast(uint4, __builtin_nontemporal_load(src + 1));
  // (offset, scale): the metadata row of 4/8-bit tiles; any readable 8 bytes otherwise (unused)
  const uint8_t* meta = un.chunk || un.bits == 16
                            ? base
                            : (kv == 0 ? un.ksub : un.vsub) + (int64_t)un.rows * row_bytes(un.bits) + 8 * rr;
  as = *reinterpret_cast<const float2*>(meta);
}

// 16 values of a loaded row slice as fp32, zeros when `ok` is false (a row
// past `valid`): codes * s + a (multiply and add rounded separately, as the
// reference's unpack and every other kernel here) for 4/8-bit, the bf16 values
// for 16-bit.
__device__ __forceinline__ void dequant16(const uint4& w0, const uint4& w1, float2 as, bool ok, int bits, int e0,
                                          float* x) {
  if (bits == 16) {
    const uint32_t u[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[2 * i] = ok ? bf_lo(u[i]) : 0.f;
      x[2 * i + 1] = ok ? bf_hi(u[i]) : 0.f;
    }
    return;
  }
  float q[16];
  if (bits == 4) {  // element 2t in the low nibble of byte t, 2t + 1 in the high one
    // the upper 8 bytes when (e0 / 16) is odd, as a mask blend: a select on a lane-varying
    // condition would be turned into a dynamically indexed vector element (scratch memory)
    const uint32_t m = 0u - (uint32_t)((e0 >> 4) & 1);
    const uint32_t u[2] = {w0.x ^ ((w0.x ^ w0.z) & m), w0.y ^ ((w0.y ^ w0.w) & m)};
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const uint32_t ev = u[b] & 0x0f0f0f0fu, od = (u[b] >> 4) & 0x0f0f0f0fu;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        q[8 * b + 2 * t] = (float)((ev >> (8 * t)) & 255u);
        q[8 * b + 2 * t + 1] = (float)((od >> (8 * t)) & 255u);
      }
    }
  } else {
    const uint32_t u[4] = {w0.x, w0.y, w0.z, w0.w};
#pragma unroll
    for (int t = 0; t < 16; ++t) q[t] = (float)((u[t >> 2] >> (8 * (t & 3))) & 255u);
  }
#pragma unroll
  for (int t = 0; t < 16; ++t) x[t] = ok ? __fadd_rn(__fmul_rn(q[t], as.y), as.x) : 0.f;
}

// Unit u of KV head h (as get_unit), with the history tile's 16-byte
// descriptor read as four dwords: u is wave-uniform, so that is one scalar load
// (the struct's 16- and 8-bit fields would otherwise be read by vector loads).
// This kernel keeps reading the device table: with the descriptors in its
// argument block instead (as the frame-chunk kernel takes them) a decode step at
// past 8128 ran 0.1-0.2 us slower.
__device__ __forceinline__ Unit unit_of(const dkv_attn_args& a, const Hist& hs, int u, int h) {
  if (u >= hs.n_tiles) return get_unit(a, hs, u, h);
  const uint4 d = *reinterpret_cast<const uint4*>(a.tiles + u);
  return history_unit(a, hs, d.x, d.y, d.z, d.w, h);
}

#ifdef DKV_TIMELINE
// events: 0 entry, 1 first tile descriptor, 2 first unit's K/V bytes, 3 units done,
// 4 workgroup merge, 5 arguments arrived
static __device__ uint64_t tl_short[TL_SLOTS * TL_EVENTS];
#endif

template <int PREC>
__global__ void __launch_bounds__(THREADS)
attn_short_kernel(dkv_attn_args a, int units, int nwg, float* __restrict__ part_o, float2* __restrict__ part_ml) {
  constexpr int NVT = PREC ? 2 : 1;  // V^T tiles per wave (hi, and lo at precision 1)
  constexpr int MRG_BYTES = WAVES * 16 * D * 4 + WAVES * 16 * 8;
  constexpr int SMEM = WAVES * NVT * VT_BYTES > MRG_BYTES ? WAVES * NVT * VT_BYTES : MRG_BYTES;
  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];

  DKV_TL(tl_short, 0);
  Hist hs;
  const int active = short_runtime_plan(a, hs, units, nwg);
  const int wg = blockIdx.x, h = blockIdx.y;
  if (wg >= active) return;  // graph replay over a shorter history than the launch bound
  DKV_TL(tl_short, 5);       // the argument block (and any step pair) has arrived
  const int G = a.q_heads / a.heads;
  const int R = G * a.nq;  // <= 16 (checked on the host)
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int slot = wave >> 1, kh = wave & 1;  // unit slot of the workgroup, key half of the unit
  const int col = lane & 15, g = lane >> 4;
  const int u0 = (int)((int64_t)units * wg / active);
  const int u1 = (int)((int64_t)units * (wg + 1) / active);
  const float xs = a.scale * LOG2E;
  uint16_t* vt_hi = reinterpret_cast<uint16_t*>(smem + wave * NVT * VT_BYTES);
  uint16_t* vt_lo = reinterpret_cast<uint16_t*>(smem + wave * NVT * VT_BYTES + (PREC ? VT_BYTES : 0));

  // Q^T operand (query row `col`, d in [16g + 8ks, 16g + 8ks + 8)) and this row's chunk window.
  Pack8 qb[2];
  qb[0].u = qb[1].u = make_uint4(0, 0, 0, 0);
  int qlo = 0, qhi = -1;
  if (col < R) {
    const int gq = col / a.nq, m = col - gq * a.nq;
    const uint16_t* src = static_cast<const uint16_t*>(a.q) + (int64_t)(h * G + gq) * a.q_head_stride +
                          (int64_t)m * a.q_tok_stride + 16 * g;
    qb[0].u = *reinterpret_cast<const uint4*>(src);
    qb[1].u = *reinterpret_cast<const uint4*>(src + 8);
    qlo = chunk_seg_start(a, m);
    qhi = m;
  }

  f32x4 acc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_part = 0.f;

  for (int u = u0 + slot; u < u1; u += UNIT_SLOTS) {
    const Unit un = unit_of(a, hs, u, h);
    if (u == u0) DKV_TL(tl_short, 1);
    // K rows of this key half for the A operand of S block j: lane (col, g)
    // holds key 32 kh + 8 (col / 4) + 4 j + col % 4, values [16g, 16g + 16).
    uint4 kw0[2], kw1[2];
    float2 kas[2];
    int kkey[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      kkey[j] = 32 * kh + 8 * (col >> 2) + 4 * j + (col & 3);
      load16(a, un, h, 0, kkey[j], 16 * g, kw0[j], kw1[j], kas[j]);
    }
    // V rows 32 kh + 2 kp and + 1, values [16 q, 16 q + 16).
    const int kp = lane & 15, q = lane >> 4;
    uint4 vw0[2], vw1[2];
    float2 vas[2];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) load16(a, un, h, 1, 32 * kh + 2 * kp + rr, 16 * q, vw0[rr], vw1[rr], vas[rr]);

    // V -> this wave's V^T tile of its 32 keys (bf16 key pairs, 4-byte stores along a d row).
    {
      float x0[16], x1[16];
      dequant16(vw0[0], vw1[0], vas[0], 32 * kh + 2 * kp < un.valid, un.bits, 16 * q, x0);
      dequant16(vw0[1], vw1[1], vas[1], 32 * kh + 2 * kp + 1 < un.valid, un.bits, 16 * q, x1);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int d = 16 * q + e;
        const uint32_t hv = pk_bf16(x0[e], x1[e]);
        *reinterpret_cast<uint32_t*>(vt_hi + d * VT + 2 * kp) = hv;
        if (PREC) *reinterpret_cast<uint32_t*>(vt_lo + d * VT + 2 * kp) = pk_bf16(x0[e] - bf_lo(hv), x1[e] - bf_hi(hv));
      }
    }
    if (u == u0) DKV_TL(tl_short, 2);

    // S^T = K Q^T over the 32 keys, one block of 16 keys at a time.
    f32x4 sc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float x[16];
      dequant16(kw0[j], kw1[j], kas[j], kkey[j] < un.valid, un.bits, 16 * g, x);
      Pack8 khi[2], klo[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        uint32_t wd[4], wl[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          wd[e] = pk_bf16(x[8 * ks + 2 * e], x[8 * ks + 2 * e + 1]);
          if (PREC) wl[e] = pk_bf16(x[8 * ks + 2 * e] - bf_lo(wd[e]), x[8 * ks + 2 * e + 1] - bf_hi(wd[e]));
        }
        khi[ks].u = make_uint4(wd[0], wd[1], wd[2], wd[3]);
        if (PREC) klo[ks].u = make_uint4(wl[0], wl[1], wl[2], wl[3]);
      }
      sc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khi[ks].v, qb[ks].v, sc[j], 0, 0, 0);
      if (PREC && un.bits != 16) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(klo[ks].v, qb[ks].v, sc[j], 0, 0, 0);
      }
    }

    // Online softmax of query column `col` over the half: lane (col, g) holds
    // keys 32 kh + 8 g + 4 j + e in sc[j][e].
    float s[8];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = 32 * kh + 8 * g + 4 * j + e;
        bool vis = key < un.valid;
        if (un.chunk) vis = vis && un.first + key >= qlo && un.first + key <= qhi;
        s[4 * j + e] = vis ? sc[j][e] : -INFINITY;
      }
    float mt = s[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mt = max_nn(mt, s[e]);
    const float mcand = col_max(mt) * xs;
    if (__builtin_amdgcn_ballot_w64(mcand > m_run + (PREC ? 8.f : 0.f))) {
      const float mnew = max_nn(m_run, mcand);
      const float alpha = mnew == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - mnew);
      m_run = mnew;
      l_part *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) acc[db] *= alpha;
    }
    const float mref = m_run == -INFINITY ? 0.f : m_run;
    float p[8], psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = __builtin_amdgcn_exp2f(__fmaf_rn(s[e], xs, -mref));
      psum += p[e];
    }
    l_part += psum;
    // P^T operand: keys 32 kh + 8 g + [0, 8) = p[0 .. 8).
    Pack8 phi, plo;
    {
      uint32_t wd[4], wl[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        wd[e] = pk_bf16(p[2 * e], p[2 * e + 1]);
        if (PREC) wl[e] = pk_bf16(p[2 * e] - bf_lo(wd[e]), p[2 * e + 1] - bf_hi(wd[e]));
      }
      phi.u = make_uint4(wd[0], wd[1], wd[2], wd[3]);
      if (PREC) plo.u = make_uint4(wl[0], wl[1], wl[2], wl[3]);
    }

    // O^T += V^T P^T: A operand row d = 16 db + col, keys 32 kh + 8 g + [0, 8).
    wave_lds_sync();
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      Pack8 va;
      va.u = *reinterpret_cast<const uint4*>(vt_hi + (16 * db + col) * VT + 8 * g);
      acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va.v, phi.v, acc[db], 0, 0, 0);
      if (PREC) {
        acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va.v, plo.v, acc[db], 0, 0, 0);
        if (un.bits != 16) {
          Pack8 vl;
          vl.u = *reinterpret_cast<const uint4*>(vt_lo + (16 * db + col) * VT + 8 * g);
          acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl.v, phi.v, acc[db], 0, 0, 0);
        }
      }
    }
    wave_lds_sync();  // the next unit overwrites the V^T tile
  }
  const float lsum = col_sum(l_part);
  DKV_TL(tl_short, 3);

  // Merge the 8 waves through LDS (over the V^T tiles): wave w's O^T rows
  // d = 16 db + 4 g + e of query column col, then (max, sum) per column.
  float* mrg_o = reinterpret_cast<float*>(smem);
  float2* mrg_ml = reinterpret_cast<float2*>(smem + WAVES * 16 * D * 4);
  __syncthreads();
#pragma unroll
  for (int db = 0; db < 4; ++db)
    *reinterpret_cast<f32x4*>(mrg_o + (wave * 16 + col) * D + 16 * db + 4 * g) = acc[db];
  if (g == 0) mrg_ml[wave * 16 + col] = make_float2(m_run, lsum);
  __syncthreads();

  // Threads 0..255: query row r = t / 16, columns [4c, 4c + 4).
  const int r = (t >> 4) & 15, c4 = 4 * (t & 15);
  const bool row_thread = t < 256 && r < R;
  float M = -INFINITY, L = 0.f;
  f32x4 O = f32x4{0.f, 0.f, 0.f, 0.f};
  if (row_thread) {
    float mw[WAVES];
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      mw[w] = mrg_ml[w * 16 + r].x;
      M = fmaxf(M, mw[w]);
    }
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float f = mw[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw[w] - M);
      L += mrg_ml[w * 16 + r].y * f;
      O += *reinterpret_cast<const f32x4*>(mrg_o + (w * 16 + r) * D + c4) * f;
    }
  }
  auto store_out = [&](int rr, int cc, f32x4 v) {
    const int gq = rr / a.nq, m = rr - gq * a.nq;
    const int64_t off = (int64_t)m * a.out_tok_stride + (int64_t)(h * G + gq) * a.out_head_stride + cc;
    if (a.out_dtype == 1)
      *reinterpret_cast<float4*>(static_cast<float*>(a.out) + off) = make_float4(v[0], v[1], v[2], v[3]);
    else
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + off) = make_uint2(pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3]));
  };
  DKV_TL(tl_short, 4);
  if (active == 1) {
    if (row_thread) store_out(r, c4, O * (1.f / L));
    return;
  }

  // This workgroup's partial, in the layout combine_kernel reads (fp32 O
  // relative to M, then (M, L); [head][split][R] rows).
  if (row_thread) {
    const int64_t pb = ((int64_t)h * nwg + wg) * R + r;
    *reinterpret_cast<f32x4*>(part_o + pb * D + c4) = O;
    if ((t & 15) == 0) part_ml[pb] = make_float2(M, L);
  }
}

}  // namespace shortpath

int launch_attn_short(const dkv_attn_args& a, const Plan& p, float* part_o, float2* part_ml, hipStream_t s) {
  const dim3 grid(p.splits, a.heads);
  const dim3 block(shortpath::THREADS);
  if (p.precision == 1)
    hipLaunchKernelGGL(shortpath::attn_short_kernel<1>, grid, block, 0, s, a, p.units, p.splits, part_o, part_ml);
  else
    hipLaunchKernelGGL(shortpath::attn_short_kernel<0>, grid, block, 0, s, a, p.units, p.splits, part_o, part_ml);
  return (int)hipGetLastError();
}

}  // namespace dkv

#ifdef DKV_TIMELINE
// Timeline build only: copies the short-chunk kernel's stamps of the last launch and clears them.
extern "C" int dkv_timeline_short(void* host, int64_t bytes) { return dkv::timeline_take(dkv::shortpath::tl_short, host, bytes); }
#endif
