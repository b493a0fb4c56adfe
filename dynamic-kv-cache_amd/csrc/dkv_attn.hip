// Fused causal GQA attention over the packed arena (gfx950).
//
// Semantics (src/gpu_kernels.py:71-105, src/cache_manager.py:43-63): query row
// m of Q head qh attends to every history token t < past of KV head
// qh / (q_heads / heads), dequantized as q*s + a, and to the chunk's own native
// K/V rows j <= m of its chunk segment. softmax(scale * q.k) weights V.
//
// Work split: a workgroup owns one KV head, one group of query rows (all GQA
// heads of that KV head share each K/V tile) and one contiguous range of
// "units" (history tiles, then 64-token pieces of the current chunk). With more
// than one range per head, each workgroup writes partial (O, max, sum) and a
// second kernel merges them with the usual log-sum-exp rescaling:
// combine_kernel for precision 1 (unnormalized O in fp32), combine_half_kernel
// for precision 0, the bf16 path (O / sum in fp16: 2^-11 of the normalized
// value, well under the bf16 output's rounding, at half the partial traffic).
// Softmax runs in base 2: x = score * scale * log2(e).
#include "dkv_attn_common.h"
#include "dkv_merge.h"
#include <mutex>

namespace dkv {

constexpr int ATT_THREADS = 256;

// Dequantizes 16 consecutive elements [c*16, c*16+16) of row r of a unit into
// fp32 (q*s + a with separately rounded multiply and add).
__device__ __forceinline__ void load_row16(const dkv_attn_args& a, const Unit& un, int kv, int r, int c,
                                           float* x) {
  if (un.chunk) {
    const int j = un.first + r;
    const uint16_t* src = kv == 0
        ? static_cast<const uint16_t*>(a.k_new) + blockIdx.y * a.kn_head_stride + (int64_t)j * a.kn_tok_stride
        : static_cast<const uint16_t*>(a.v_new) + blockIdx.y * a.vn_head_stride + (int64_t)j * a.vn_tok_stride;
    const uint4* p = reinterpret_cast<const uint4*>(src + c * 16);
    uint4 w0 = p[0], w1 = p[1];
    uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[2 * i] = bf16_lo(w[i]);
      x[2 * i + 1] = bf16_hi(w[i]);
    }
    return;
  }
  const uint8_t* sub = kv == 0 ? un.ksub : un.vsub;
  const uint8_t* prow = sub + (int64_t)r * row_bytes(un.bits);
  if (un.bits == 16) {
    const uint4* p = reinterpret_cast<const uint4*>(prow + c * 32);
    uint4 w0 = p[0], w1 = p[1];
    uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[2 * i] = bf16_lo(w[i]);
      x[2 * i + 1] = bf16_hi(w[i]);
    }
    return;
  }
  const float2 as = reinterpret_cast<const float2*>(sub + (int64_t)un.rows * row_bytes(un.bits))[r];
  uint32_t code[16];
  if (un.bits == 4) {
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

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// ---------------------------------------------------------------------------
// Vector path (path 1, on request): fp32 FMA instead of MFMA tiles, kept as a
// second implementation the MFMA kernel is checked against. A wave owns VEC_RPW query rows; lane n
// scores key n of the unit, lane d accumulates output column d. PREC 0 rounds
// the dequantized K/V and p to bf16 where the reference kernel does
// (src/gpu_kernels.py:93-94,102); PREC 1 stays in fp32 throughout.
constexpr int VEC_RPW = VEC_ROWS / 4;

template <int PREC>
__global__ void __launch_bounds__(ATT_THREADS)
attn_vec_kernel(dkv_attn_args a, int units, int splits, int cap, float* __restrict__ part_o,
                float2* __restrict__ part_ml) {
  __shared__ float Qs[VEC_ROWS][D];
  __shared__ float Kt[TILE][D + 1];
  __shared__ float Vt[TILE][D];
  __shared__ float Ps[4][TILE];

  Hist hs;
  const int active = runtime_plan(a, hs, units, splits, cap);
  const int split = blockIdx.x, h = blockIdx.y, rg = blockIdx.z;
  const int G = a.q_heads / a.heads;
  const int R = G * a.nq;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (split >= active) return;  // graph replay over a shorter history than the launch bound
  const int u0 = (int)((int64_t)units * split / active);
  const int u1 = (int)((int64_t)units * (split + 1) / active);
  const float xs = a.scale * LOG2E;

  // Stage this group's query rows in LDS as fp32.
  for (int idx = tid; idx < VEC_ROWS * (D / 8); idx += ATT_THREADS) {
    const int rl = idx / (D / 8), c8 = idx % (D / 8);
    const int r = rg * VEC_ROWS + rl;
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (r < R) {
      const int g = r / a.nq, m = r - g * a.nq;
      const uint16_t* src = static_cast<const uint16_t*>(a.q) + (int64_t)(h * G + g) * a.q_head_stride +
                            (int64_t)m * a.q_tok_stride + c8 * 8;
      uint4 wq = *reinterpret_cast<const uint4*>(src);
      uint32_t ww[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = bf16_lo(ww[i]);
        v[2 * i + 1] = bf16_hi(ww[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) Qs[rl][c8 * 8 + i] = v[i];
  }

  float acc[VEC_RPW], mx[VEC_RPW], sm[VEC_RPW];
#pragma unroll
  for (int i = 0; i < VEC_RPW; ++i) {
    acc[i] = 0.f;
    mx[i] = -INFINITY;
    sm[i] = 0.f;
  }

  for (int u = u0; u < u1; ++u) {
    const Unit un = get_unit(a, hs, u, h);
    __syncthreads();  // previous unit's readers are done; Qs is staged
    {
      const int r = tid >> 2, c = tid & 3;
      float xk[16], xv[16];
      if (r < un.valid) {
        load_row16(a, un, 0, r, c, xk);
        load_row16(a, un, 1, r, c, xv);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) xk[i] = xv[i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        Kt[r][c * 16 + i] = PREC ? xk[i] : round_bf16(xk[i]);
        Vt[r][c * 16 + i] = PREC ? xv[i] : round_bf16(xv[i]);
      }
    }
    __syncthreads();
    const int j = un.first + lane;  // chunk row of this lane's token (chunk units)
    const int jseg = un.chunk ? chunk_seg_start(a, j) : 0;
#pragma unroll
    for (int i = 0; i < VEC_RPW; ++i) {
      const int rl = w * VEC_RPW + i;
      const int r = rg * VEC_ROWS + rl;
      if (r >= R) break;  // wave-uniform
      const int m = r % a.nq;
      bool vis = lane < un.valid;
      if (un.chunk) vis = vis && j <= m && jseg == chunk_seg_start(a, m);
      float s = 0.f;
#pragma unroll 16
      for (int d = 0; d < D; ++d) s = fmaf(Qs[rl][d], Kt[lane][d], s);
      const float x = vis ? s * xs : -INFINITY;
      const float tmax = wave_max(x);
      if (tmax == -INFINITY) continue;  // wave-uniform: nothing visible here
      const float mnew = fmaxf(mx[i], tmax);
      const float alpha = exp2f(mx[i] - mnew);
      const float p = vis ? exp2f(x - mnew) : 0.f;
      sm[i] = sm[i] * alpha + wave_sum(p);
      mx[i] = mnew;
      Ps[w][lane] = PREC ? p : round_bf16(p);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      float o = acc[i] * alpha;
#pragma unroll 16
      for (int n = 0; n < TILE; ++n) o = fmaf(Ps[w][n], Vt[n][lane], o);
      acc[i] = o;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }

  // Epilogue: final output (one split running) or partials. The test is on the
  // splits that run, not the launch's: a graph replay over a short history can
  // run one split of a launch sized for more, and must then store exactly what
  // a direct one-split call stores (the merge kernels skip such launches).
#pragma unroll
  for (int i = 0; i < VEC_RPW; ++i) {
    const int r = rg * VEC_ROWS + w * VEC_RPW + i;
    if (r >= R) break;
    if (active == 1) {
      const int g = r / a.nq, m = r - g * a.nq;
      const float o = acc[i] / sm[i];
      const int64_t off = (int64_t)m * a.out_tok_stride + (int64_t)(h * G + g) * a.out_head_stride + lane;
      if (a.out_dtype == 1) static_cast<float*>(a.out)[off] = o;
      else static_cast<uint16_t*>(a.out)[off] = (uint16_t)f32_to_bf16_rne(o);
    } else {
      const int64_t base = ((int64_t)h * splits + split) * R + r;
      float l = sm[i];
      if (PREC) {
        __builtin_nontemporal_store(acc[i], part_o + base * D + lane);  // no dirty L2 lines at kernel end
      } else {  // O / l in fp16, half_slot() order
        const float y = l > 0.f ? acc[i] / l : 0.f;
        _Float16* dst = reinterpret_cast<_Float16*>(part_o) + base * D + half_slot(lane);
        __builtin_nontemporal_store((_Float16)y, dst);
        if (__builtin_amdgcn_ballot_w64(fabsf(y) >= 32768.f)) {  // rare: |V| near the fp16 range
          float amax = fabsf(y);
#pragma unroll
          for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
          const int ex = half_partial_exponent(amax);
          // stored again, scaled (the later store to the same address wins)
          __builtin_nontemporal_store((_Float16)__builtin_amdgcn_ldexpf(y, -ex), dst);
          l = half_partial_sum(l, ex);
        }
      }
      if (lane == 0) {
        __builtin_nontemporal_store(mx[i], reinterpret_cast<float*>(part_ml + base));
        __builtin_nontemporal_store(l, reinterpret_cast<float*>(part_ml + base) + 1);
      }
    }
  }
}

// Both merges read the partials once, with nontemporal loads (past 8128: 18.7 -> 18.5 us per
// layer; candidate batches 15.9 -> 15.7 us), or with plain loads where the producing launch stored
// them plainly (Plan::plain_parts).
//
#ifdef DKV_TIMELINE
// events (both merge kernels): 0 entry, 1 arguments arrived, 3 row stored
static __device__ uint64_t tl_comb[TL_SLOTS * TL_EVENTS];
#endif
//
// The arguments the merge kernels read before their first partial load, read together: placed by
// their uses, the compiler issued these scalar loads in four to six dependent rounds (each a
// round trip to the cache hierarchy); the empty asm needs them all at once.
__device__ __forceinline__ void merge_args_at_once(const dkv_attn_args& a, int splits, int cap, const void* part_o,
                                                   const void* part_ml) {
  asm volatile("" ::"s"(a.q_heads), "s"(a.heads), "s"(a.nq), "s"(a.n_tiles), "s"(a.past), "s"(a.step), "s"(splits),
               "s"(cap), "s"(part_o), "s"(part_ml), "s"(a.out), "s"(a.out_tok_stride), "s"(a.out_head_stride),
               "s"(a.out_dtype));
}

// The two merge kernels: one wave per query row of a KV head, the row's arithmetic in
// merge_row_f32 (precision 1) and merge_row_half (precision 0), dkv_merge.h.
template <bool PLAIN>
__global__ void __launch_bounds__(256)
combine_kernel(dkv_attn_args a, int splits, int cap, int short_plan, const float* __restrict__ part_o,
               const float2* __restrict__ part_ml) {
  DKV_TL(tl_comb, 0);
  merge_args_at_once(a, splits, cap, part_o, part_ml);
  const int h = blockIdx.y;
  const int G = a.q_heads / a.heads;
  const int R = G * a.nq;
  const int r = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (r >= R) return;
  int units = a.n_tiles + (a.nq + TILE - 1) / TILE;
  Hist hs;
  // partials written (graph replays: fewer), by the producing kernel's rule
  const int active = short_plan ? short_runtime_plan(a, hs, units, splits) : runtime_plan(a, hs, units, splits, cap);
  if (active <= 1) return;  // one split ran and stored the output itself
  DKV_TL(tl_comb, 1);
  merge_row_f32<PLAIN>(a, h, r, R, G, splits, active, part_o, part_ml);
  DKV_TL(tl_comb, 3);
}

template <bool PLAIN>
__global__ void __launch_bounds__(256)
combine_half_kernel(dkv_attn_args a, int splits, int cap, int short_plan, const float* __restrict__ part_o,
                    const float2* __restrict__ part_ml) {
  DKV_TL(tl_comb, 0);
  merge_args_at_once(a, splits, cap, part_o, part_ml);
  const int h = blockIdx.y;
  const int G = a.q_heads / a.heads;
  const int R = G * a.nq;
  const int r = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (r >= R) return;
  int units = a.n_tiles + (a.nq + TILE - 1) / TILE;
  Hist hs;
  // partials written (graph replays: fewer), by the producing kernel's rule
  const int active = short_plan ? short_runtime_plan(a, hs, units, splits) : runtime_plan(a, hs, units, splits, cap);
  if (active <= 1) return;  // one split ran and stored the output itself
  DKV_TL(tl_comb, 1);
  merge_row_half<PLAIN>(a, h, r, R, G, splits, active, part_o, part_ml);
  DKV_TL(tl_comb, 3);
}

// The same merges with MERGE_WAVES waves per query row (one row per workgroup, merge_row_*_wide):
// each wave merges a contiguous share of the splits and wave 0 combines the shares in wave order.
// A wave of the one-row-per-wave kernels above is alone on its SIMD, so every dependent load wait
// and instruction of its merge is on the critical path; a share of a quarter of the splits takes a
// quarter of that.
template <bool PLAIN>
__global__ void __launch_bounds__(64 * MERGE_WAVES)
combine_wide_kernel(dkv_attn_args a, int splits, int cap, const float* __restrict__ part_o,
                    const float2* __restrict__ part_ml) {
  DKV_TL(tl_comb, 0);
  merge_args_at_once(a, splits, cap, part_o, part_ml);
  const int h = blockIdx.y, r = blockIdx.x;
  const int G = a.q_heads / a.heads;
  const int R = G * a.nq;
  if (r >= R) return;  // uniform over the workgroup
  int units = a.n_tiles + (a.nq + TILE - 1) / TILE;
  Hist hs;
  const int active = runtime_plan(a, hs, units, splits, cap);
  if (active <= 1) return;
  DKV_TL(tl_comb, 1);
  merge_row_f32_wide<PLAIN, MERGE_WAVES>(a, h, r, R, G, splits, active, part_o, part_ml);
  DKV_TL(tl_comb, 3);
}

template <bool PLAIN>
__global__ void __launch_bounds__(64 * MERGE_WAVES)
combine_half_wide_kernel(dkv_attn_args a, int splits, int cap, const float* __restrict__ part_o,
                         const float2* __restrict__ part_ml) {
  DKV_TL(tl_comb, 0);
  merge_args_at_once(a, splits, cap, part_o, part_ml);
  const int h = blockIdx.y, r = blockIdx.x;
  const int G = a.q_heads / a.heads;
  const int R = G * a.nq;
  if (r >= R) return;  // uniform over the workgroup
  int units = a.n_tiles + (a.nq + TILE - 1) / TILE;
  Hist hs;
  const int active = runtime_plan(a, hs, units, splits, cap);
  if (active <= 1) return;
  DKV_TL(tl_comb, 1);
  merge_row_half_wide<PLAIN, MERGE_WAVES>(a, h, r, R, G, splits, active, part_o, part_ml);
  DKV_TL(tl_comb, 3);
}

// ---------------------------------------------------------------------------
// Host side.

static int num_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
  }
  return cus;
}

static int check_args(const dkv_attn_args& a) {
  if (!a.q || !a.k_new || !a.v_new || !a.out || (a.n_tiles > 0 && (!a.tiles || !a.arena))) {
    set_error("dkv_attend: null pointer argument");
    return DKV_EINVAL;
  }
  if (a.heads <= 0 || a.q_heads <= 0 || a.q_heads % a.heads || a.nq <= 0 || a.past < 0 ||
      a.n_tiles < 0 || a.layer < 0 || a.layer >= a.layers) {
    set_error("dkv_attend: bad shape (heads %d, q_heads %d, nq %d, past %d, layer %d/%d)", a.heads,
              a.q_heads, a.nq, a.past, a.layer, a.layers);
    return DKV_EINVAL;
  }
  if (a.n_segs < 0 || a.n_segs > DKV_MAX_CHUNK_SEGS) {
    set_error("dkv_attend: n_segs %d outside [0, %d]", a.n_segs, DKV_MAX_CHUNK_SEGS);
    return DKV_EINVAL;
  }
  if (a.n_segs > 1) {
    if (a.seg_bounds[0] != 0 || a.seg_bounds[a.n_segs] != a.nq) {
      set_error("dkv_attend: segment bounds must start at 0 and end at nq");
      return DKV_EINVAL;
    }
    for (int s = 0; s < a.n_segs; ++s)
      if (a.seg_bounds[s + 1] <= a.seg_bounds[s]) {
        set_error("dkv_attend: segment bounds must increase");
        return DKV_EINVAL;
      }
  }
  if (a.path < 0 || a.path > 3 || a.precision < 0 || a.precision > 1) {
    set_error("dkv_attend: path must be 0 (auto), 1 (vector), 2 (MFMA) or 3 (short chunk); precision 0 (bf16) or "
              "1 (fp32)");
    return DKV_EINVAL;
  }
  if (a.path == 3 && (a.q_heads / a.heads) * a.nq > SHORT_ROWS) {
    set_error("dkv_attend: the short-chunk path takes at most %d query rows per KV head (q_heads / heads * nq = %d)",
              SHORT_ROWS, (a.q_heads / a.heads) * a.nq);
    return DKV_EINVAL;
  }
  if (a.out_dtype != 0 && a.out_dtype != 1) {
    set_error("dkv_attend: out_dtype must be 0 (bf16) or 1 (fp32)");
    return DKV_EINVAL;
  }
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (!a16(a.q) || !a16(a.k_new) || !a16(a.v_new) || (a.q_head_stride & 7) || (a.q_tok_stride & 7) ||
      (a.kn_head_stride & 7) || (a.kn_tok_stride & 7) || (a.vn_head_stride & 7) || (a.vn_tok_stride & 7)) {
    set_error("dkv_attend: Q/K/V must be 16-byte aligned with strides that are multiples of 8 elements");
    return DKV_EINVAL;
  }
  if (!a16(a.out) || (a.out_tok_stride & 3) || (a.out_head_stride & 3)) {  // rows are stored 4 columns at a time
    set_error("dkv_attend: out must be 16-byte aligned with strides that are multiples of 4 elements");
    return DKV_EINVAL;
  }
  if (a.tiles_host && !a.step && a.n_tiles > 0 && a.n_tiles <= DKV_ARG_TILES) {
    // The host copy goes into the frame-chunk kernel's argument block as given: its tiles must be
    // well formed and cover [0, past) in token order, as the cache's table does.
    int next = 0;
    for (int i = 0; i < a.n_tiles; ++i) {
      const dkv_tile& t = a.tiles_host[i];
      if ((t.bits != 4 && t.bits != 8 && t.bits != 16) || t.rows < 1 || t.rows > TILE || t.offset < 0 ||
          t.token_start != next) {
        set_error("dkv_attend: tiles_host[%d] (token_start %d, rows %d, bits %d) is not the tile after "
                  "token %d", i, t.token_start, (int)t.rows, (int)t.bits, next);
        return DKV_EINVAL;
      }
      next += t.rows;
    }
    if (next < a.past || a.tiles_host[a.n_tiles - 1].token_start >= a.past) {
      set_error("dkv_attend: tiles_host's %d tiles do not end at past %d", a.n_tiles, a.past);
      return DKV_EINVAL;
    }
  }
  return 0;
}

static Plan make_plan(const dkv_attn_args& a) {
  Plan p;
  const int G = a.q_heads / a.heads;
  const int R = G * a.nq;
  p.path = a.path;
  // Auto: the frame-chunk MFMA kernel for every chunk, decode steps included. Measured on decode
  // steps (1 and 4 tokens over 256-8128 tokens, both precisions) it is faster than the
  // short-chunk kernel everywhere (8.6 vs 11.8 us at past 1024, 11.7 vs 12.5 us at 8128, bf16),
  // reading its descriptors from the argument block or from the device table; the short-chunk
  // kernel stays as path 3.
  if (p.path == 0) p.path = 2;
  p.precision = a.precision;
  p.rows_per_group = p.path == 3 ? SHORT_ROWS : (p.path == 2 ? MFMA_ROWS : VEC_ROWS);
  p.row_groups = (R + p.rows_per_group - 1) / p.rows_per_group;
  if (p.path == 2) {
    // The same number of groups, balanced: 16-row blocks spread evenly, so that no group (the
    // critical path of every unit) carries more blocks than it must. At most MFMA_ROWS rows.
    const int blocks = (R + 15) / 16;
    p.rows_per_group = 16 * ((blocks + p.row_groups - 1) / p.row_groups);
  }
  p.units = a.n_tiles + (a.nq + TILE - 1) / TILE;
  p.small = a.path == 0 && p.precision == 0 && R <= MFMA_SMALL_ROWS;
  int splits = a.splits;
  p.cap = 0;
  if (splits <= 0) {
    const int per = a.heads * p.row_groups;
    if (p.path == 3) {
      // two waves per unit, four units per workgroup: every tile of the history is requested
      // when the kernel starts (at most SHORT_MAX_SPLITS workgroups per KV head)
      splits = short_default_splits(p.units);
    } else {
      // MFMA: one 12-wave workgroup per CU, all resident at once (a grid one past the CU count
      // would take a second round for a single workgroup); balanced over the history. A launch
      // that reads its history from a device step pair (graph replays) is sized for the cap,
      // the most splits any history runs.
      p.cap = p.path == 2 ? (p.small ? MFMA_SMALL_PER_CU : 1) * num_cus() / per : (2 * num_cus() + per - 1) / per;
      if (p.cap < 1) p.cap = 1;
      splits = a.step ? p.cap : balanced_splits(p.units, p.cap);
    }
  }
  if (splits > p.units) splits = p.units;
  if (splits < 1) splits = 1;
  p.splits = splits;
  // At precision 1 a default plan that leaves half the CUs idle (short histories: 17 splits x 5
  // KV heads at past 1024) splits each KV head's rows over two workgroups instead (the same
  // units, half the query blocks each): 13.0 -> 12.2 us per layer at past 1024. Every row's
  // arithmetic is the same whichever workgroup computes it. At precision 0, whose units cost
  // half as much, it ran slower (11.07 -> 11.36 us).
  if (p.path == 2 && p.precision == 1 && a.splits <= 0 && !a.step && p.row_groups == 1) {
    const int blocks = (R + 15) / 16;
    if (blocks > MFMA_KG_WAVES && a.heads * splits * 2 <= num_cus()) {
      p.row_groups = 2;
      p.rows_per_group = 16 * ((blocks + 1) / 2);
    }
  }
  p.plain_parts = p.path == 2 && splits > 1 && mfma_blocks_per_wave(p.rows_per_group) == 1;
  // The merge with MERGE_WAVES waves per row where the one-wave merge would leave most SIMDs idle
  // (decode steps: 3-12 rows per KV head, 43-128 splits; 9.78 -> 9.11 us per layer at past 8128,
  // 4 tokens 10.52 -> 9.52). With more rows the one-wave merge already has a wave on most SIMDs,
  // and four times the workgroups ran slower (frame chunks at past 8128 15.80 -> 17.28 us).
  p.wide_merge = MERGE_WAVES > 1 && p.path != 3 && (int64_t)a.heads * R * MERGE_WAVES <= 4 * num_cus();
  p.fused = DKV_INKERNEL_MERGE && a.path == 0 && p.path == 2 && p.precision == 0 && splits > 1 &&
            a.heads * p.row_groups * 4 <= INKERNEL_COUNTER_BYTES;
  if (splits > 1) {
    if (p.path == 3) {  // unnormalized fp32 O and (max, sum), as combine_kernel reads them
      p.part_o_bytes = (int64_t)a.heads * splits * R * D * 4;
      p.part_ml_bytes = (int64_t)a.heads * splits * R * 8;
    } else {
      p.part_o_bytes = (int64_t)a.heads * splits * R * D * (p.precision ? 4 : 2);  // fp32 O or fp16 O / sum
      p.part_ml_bytes = (int64_t)a.heads * splits * R * 8;
    }
  } else {
    p.part_o_bytes = p.part_ml_bytes = 0;
  }
  return p;
}

// Workspace bytes of a plan: the split partials (none for one split), after the arrival counters in
// the in-kernel merge build.
static int64_t workspace_bytes(const Plan& p) {
  return p.splits > 1 ? INKERNEL_COUNTER_BYTES + p.part_o_bytes + p.part_ml_bytes : 0;
}

int launch_attn_vec(const dkv_attn_args& a, const Plan& p, float* part_o, float2* part_ml, hipStream_t s) {
  const dim3 grid(p.splits, a.heads, p.row_groups);
  if (p.precision == 1)
    hipLaunchKernelGGL(attn_vec_kernel<1>, grid, dim3(ATT_THREADS), 0, s, a, p.units, p.splits, p.cap, part_o,
                       part_ml);
  else
    hipLaunchKernelGGL(attn_vec_kernel<0>, grid, dim3(ATT_THREADS), 0, s, a, p.units, p.splits, p.cap, part_o,
                       part_ml);
  return (int)hipGetLastError();
}

// The launches of one attention call whose split partials go to `ws` (at least
// workspace_bytes(p) bytes, or unused for one split).
static int launch_attend(const dkv_attn_args& a, const Plan& p, void* ws, hipStream_t s) {
  uint32_t* counters = static_cast<uint32_t*>(ws);
  float* part_o = reinterpret_cast<float*>(static_cast<char*>(ws) + INKERNEL_COUNTER_BYTES);
  float2* part_ml = reinterpret_cast<float2*>(static_cast<char*>(ws) + INKERNEL_COUNTER_BYTES + p.part_o_bytes);
  const int rc = p.path == 3 ? launch_attn_short(a, p, part_o, part_ml, s)
                 : p.path == 2 ? launch_attn_mfma(a, p, part_o, part_ml, counters, s)
                               : launch_attn_vec(a, p, part_o, part_ml, s);
  if (rc) return rc;
  if (p.splits > 1 && !p.fused) {
    const int R = (a.q_heads / a.heads) * a.nq;
    const int short_plan = p.path == 3;
    const dim3 grid((R + 3) / 4, a.heads);
    if (p.wide_merge) {
      const dim3 wgrid(R, a.heads);
      if (p.precision == 1) {
        if (p.plain_parts)
          hipLaunchKernelGGL(combine_wide_kernel<true>, wgrid, dim3(64 * MERGE_WAVES), 0, s, a, p.splits, p.cap, part_o, part_ml);
        else
          hipLaunchKernelGGL(combine_wide_kernel<false>, wgrid, dim3(64 * MERGE_WAVES), 0, s, a, p.splits, p.cap, part_o, part_ml);
      } else if (p.plain_parts) {
        hipLaunchKernelGGL(combine_half_wide_kernel<true>, wgrid, dim3(64 * MERGE_WAVES), 0, s, a, p.splits, p.cap,
                           part_o, part_ml);
      } else {
        hipLaunchKernelGGL(combine_half_wide_kernel<false>, wgrid, dim3(64 * MERGE_WAVES), 0, s, a, p.splits, p.cap,
                           part_o, part_ml);
      }
    } else if (p.precision == 1 || short_plan) {  // the short-chunk kernel's partials are fp32 in both precisions
      if (p.plain_parts)
        hipLaunchKernelGGL(combine_kernel<true>, grid, dim3(256), 0, s, a, p.splits, p.cap, short_plan, part_o, part_ml);
      else
        hipLaunchKernelGGL(combine_kernel<false>, grid, dim3(256), 0, s, a, p.splits, p.cap, short_plan, part_o, part_ml);
    } else if (p.plain_parts) {
      hipLaunchKernelGGL(combine_half_kernel<true>, grid, dim3(256), 0, s, a, p.splits, p.cap, short_plan, part_o,
                         part_ml);
    } else {
      hipLaunchKernelGGL(combine_half_kernel<false>, grid, dim3(256), 0, s, a, p.splits, p.cap, short_plan, part_o,
                         part_ml);
    }
  }
  return (int)hipGetLastError();
}

// Scratch of dkv_attend_noalloc: the split partials of one call, in device
// memory that is part of the library's code object, so no call allocates. Each
// device holds its own copy at its own address until the process ends. Host
// code never passes this name to a kernel (on the host it is only a handle to
// the symbol): it looks the device address up with hipGetSymbolAddress, once
// per device, and uses that. Every call on a device shares the one copy; the
// kernels write every partial they later read, so nothing has to start at zero.
constexpr int SCRATCH_DEVICES = 64;
static __device__ __attribute__((aligned(256))) uint8_t scratch[DKV_NOALLOC_SCRATCH_BYTES];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[SCRATCH_DEVICES];  // device address of `scratch` per device index

static int scratch_address(void** ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= SCRATCH_DEVICES) {
    set_error("dkv_attend_noalloc: device index %d beyond %d", dev, SCRATCH_DEVICES);
    return DKV_EINVAL;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) {
      set_error("dkv_attend_noalloc: no device address for the scratch buffer");
      return DKV_EINVAL;
    }
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return 0;
}

}  // namespace dkv

using namespace dkv;

extern "C" {

int64_t dkv_attend_workspace_bytes(const dkv_attn_args* args) {
  if (!args || args->heads <= 0 || args->q_heads <= 0 || args->q_heads % args->heads || args->nq <= 0)
    return 0;
  return workspace_bytes(make_plan(*args));
}

int dkv_attend(const dkv_attn_args* args, void* stream) {
  clear_error();
  if (!args) {
    set_error("dkv_attend: null args");
    return DKV_EINVAL;
  }
  const dkv_attn_args& a = *args;
  if (int rc = check_args(a)) return rc;
  const Plan p = make_plan(a);
  const int64_t need = workspace_bytes(p);
  if (need > 0 && (!a.workspace || a.workspace_bytes < need)) {
    set_error("dkv_attend: workspace of %lld bytes needed, %lld given", (long long)need,
              (long long)a.workspace_bytes);
    return DKV_EINVAL;
  }
  return launch_attend(a, p, a.workspace, (hipStream_t)stream);
}

int dkv_attend_noalloc(const dkv_attn_args* args, void* stream) {
  clear_error();
  if (!args) {
    set_error("dkv_attend_noalloc: null args");
    return DKV_EINVAL;
  }
  const dkv_attn_args& a = *args;
  if (int rc = check_args(a)) return rc;
  const Plan p = make_plan(a);
  const int64_t need = workspace_bytes(p);
  if (need > DKV_NOALLOC_SCRATCH_BYTES) {
    set_error("dkv_attend_noalloc: this call's split partials need %lld bytes, more than the %d-byte "
              "scratch buffer (use dkv_attend with a workspace, or fewer splits)",
              (long long)need, DKV_NOALLOC_SCRATCH_BYTES);
    return DKV_EINVAL;
  }
  void* ws = nullptr;
  if (need > 0)
    if (int rc = scratch_address(&ws)) return rc;
  return launch_attend(a, p, ws, (hipStream_t)stream);
}

}  // extern "C"

#ifdef DKV_TIMELINE
// Timeline build only: copies the merge kernels' stamps of the last launch and clears them.
extern "C" int dkv_timeline_combine(void* host, int64_t bytes) { return dkv::timeline_take(dkv::tl_comb, host, bytes); }
#endif
