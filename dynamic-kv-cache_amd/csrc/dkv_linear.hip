// Decoder projections for short chunks: out = epilogue(prologue(x) w^T) with
// x [rows, k] and w [n, k] bf16 (both row-major, k contiguous), fp32
// accumulation on v_mfma_f32_16x16x32_bf16, bf16 out.
//
//   prologue  none, or RMSNorm of the x rows with the torch composition's two
//             bf16 roundings (bf16(bf16(x * rsqrt(mean(x^2) + eps)) * g),
//             src/gpu_ops.py:9-12) applied in registers;
//   epilogue  plain: bf16(acc);
//             residual: bf16(r + bf16(acc)), the decoder's residual add after
//             o_proj and down_proj;
//             silu_mul: w holds [gate | up] rows (2 * inter of them) and
//             out[:, c] = bf16(bf16(silu(bf16(g_c))) * bf16(u_c))
//             (src/gpu_ops.py:14-17, 23-25).
//
// The chunks are 1-100 rows, so the weights (1.8-9.8 MB per projection of the
// 960-wide decoder) dominate the traffic: the kernel is a weight stream. A
// workgroup owns NB column blocks of 16 weight rows and RB blocks of 16 x
// rows; its waves split k in 64-element pairs of MFMA steps (wave w takes
// pairs w, w + WAVES, ...), issue every load of their share before the first
// MFMA, and meet in LDS, where one wave per output tile sums the partials in
// wave order (deterministic). With Y^T = W X^T on the MFMA (weights on the M
// axis), lane (col, g) ends with 4 consecutive output columns of one row: 8
// byte stores. Consecutive workgroups go to different XCDs; the RB = 1 layout
// numbers its tiles so that the row blocks sharing a weight tile land on one
// XCD (one L2).
#include "dkv_common.h"

namespace dkv {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

union Op8 {
  bf16x8_t v;
  u32x4 u;
};

enum { EPI_PLAIN = 0, EPI_RESIDUAL = 1, EPI_SILU_MUL = 2 };

struct LinearArgs {  // passed by value and never written (a written copy would go to scratch)
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* w;
  int64_t ldw;
  const uint16_t* norm;  // RMSNorm weight [k] (prologue only)
  const uint16_t* res;   // residual [rows, n] (EPI_RESIDUAL only)
  int64_t ldr;
  uint16_t* out;
  int64_t ldo;
  float eps;
  int rows, k, kp;  // kp = k / 64
  int n_tiles;      // column tiles of 16 * NT output columns
  int row_groups;   // ceil(rows / (16 * RB))
  int up;           // n_out (EPI_SILU_MUL: the first weight row of the up half)
  int layout;       // LAYOUT_* bits: which of w, x and out are MFMA-tiled
};

// Operand layouts. Rows of k contiguous elements, or MFMA-tiled: the 16 rows x 64 k of one pair
// of MFMA steps are 2 KB in the order the lanes read them, one 1 KB half per step (element (r, c)
// at ((r / 16) * kp + c / 64) * 1024 + (c / 32 % 2) * 512 + ((c / 8 % 4) * 16 + r % 16) * 8 + c % 8),
// so that each 16-byte-per-lane load instruction reads 1 KB of consecutive bytes (8 full cache
// lines instead of 64-byte halves of 16). A tiled x or out has its rows rounded up to 16.
enum {
  LAYOUT_W_TILED = DKV_LINEAR_W_TILED,
  LAYOUT_X_TILED = DKV_LINEAR_X_TILED,
  LAYOUT_OUT_TILED = DKV_LINEAR_OUT_TILED,
  LAYOUT_RES_TILED = DKV_LINEAR_RES_TILED
};

// Offset of element (r, c) of a tiled matrix with kp pairs of 64 columns per row.
__device__ __forceinline__ int64_t tiled_offset(int r, int c, int kp) {
  return ((int64_t)(r >> 4) * kp + (c >> 6)) * 1024 + ((c >> 5) & 1) * 512 + (((c >> 3) & 3) * 16 + (r & 15)) * 8 + (c & 7);
}

__device__ __forceinline__ float lane_group_sum(float x) {
  // sum over lanes col, col + 16, col + 32, col + 48 (gfx950 lane swaps)
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

template <int CH, int NT, int WAVES, int RB, int EPI, bool NORM, int OPS>
__global__ void __launch_bounds__(64 * WAVES) linear_kernel(const LinearArgs a) {
  constexpr int NB = EPI == EPI_SILU_MUL ? 2 * NT : NT;  // column blocks multiplied
  // The arguments the first loads depend on, read together (placed by their uses, the compiler
  // read them in two dependent rounds of scalar loads, each a round trip to the cache hierarchy).
  asm volatile("" ::"s"(a.x), "s"(a.ldx), "s"(a.w), "s"(a.ldw), "s"(a.rows), "s"(a.kp), "s"(a.n_tiles),
               "s"(a.row_groups), "s"(a.up), "s"(a.layout));
  if constexpr (NORM) asm volatile("" ::"s"(a.norm));
  if constexpr (EPI == EPI_RESIDUAL) asm volatile("" ::"s"(a.res), "s"(a.ldr));
  const int b = blockIdx.x;
  const int xcd = b & 7, j = b >> 3;
  const int rg = j % a.row_groups;
  const int ct = (j / a.row_groups) * 8 + xcd;
  if (ct >= a.n_tiles) return;  // uniform over the workgroup
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, col = lane & 15, g = lane >> 4;
  const int n0 = ct * 16 * NT;

  // A lane's operand pointers for pair 0, half 0, and the element steps to pair p and half h
  // (k = 64 p + 32 h): rows of k elements, or the MFMA-tiled layout (OPS = the layout bits of w
  // and x, compile-time so that the steps are immediate offsets of the loads).
  constexpr bool w_tiled = OPS & LAYOUT_W_TILED, x_tiled = OPS & LAYOUT_X_TILED;
  constexpr int wsp = w_tiled ? 1024 : 64, wsh = w_tiled ? 512 : 32;
  constexpr int xsp = x_tiled ? 1024 : 64, xsh = x_tiled ? 512 : 32;
  const uint16_t* wrow[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int r = (EPI == EPI_SILU_MUL && nb >= NT) ? a.up + n0 + 16 * (nb - NT) : n0 + 16 * nb;
    wrow[nb] = w_tiled ? a.w + (int64_t)(r >> 4) * a.kp * 1024 + 8 * lane : a.w + (int64_t)(r + col) * a.ldw + 8 * g;
  }
  // Rows past the end read the last row (or a tiled x's padding rows): x row j only reaches
  // output row j, which is not stored.
  const uint16_t* xrow[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = min((rg * RB + rb) * 16 + col, a.rows - 1);
    xrow[rb] = x_tiled ? a.x + (int64_t)(rg * RB + rb) * a.kp * 1024 + 8 * lane : a.x + (int64_t)row * a.ldx + 8 * g;
  }

  constexpr int TILES = RB * NB, OUT = RB * NT;
  // The residual of the output tiles this wave finishes (tile o belongs to wave o % WAVES), loaded
  // first, so that it arrives with the operands: loaded in the epilogue it was one more memory
  // round trip after the reduction. Rows past the end read the last row (never stored).
  uint2 resv[EPI == EPI_RESIDUAL ? OUT : 1];
  if constexpr (EPI == EPI_RESIDUAL) {
#pragma unroll
    for (int o = 0; o < OUT; ++o) {
      if (o % WAVES != wave) continue;
      const int row = min((rg * RB + o / NT) * 16 + col, a.rows - 1), c = n0 + 16 * (o % NT) + 4 * g;
      // a tiled residual has its rows rounded up to 16: row (rg * RB + o / NT) * 16 + col is there
      resv[o] = *reinterpret_cast<const uint2*>(
          a.res + ((a.layout & LAYOUT_RES_TILED) ? tiled_offset((rg * RB + o / NT) * 16 + col, c, a.up >> 6)
                                                 : (int64_t)row * a.ldr + c));
    }
  }

  // Every load of this wave's pairs (the host guarantees CH * WAVES >= kp) is
  // issued before the first MFMA. With the RMSNorm prologue the x rows and
  // the norm weight go first, unconditionally (a pair past kp loads pair
  // kp - 1 and is skipped below, so the loads form one straight-line block
  // whose uses wait for exactly what they need), and the weight tiles, which
  // come from HBM, only once x has arrived (load_weights below): the prologue
  // normalizes while they are in flight. Without it the first MFMA needs both,
  // and pairs past kp (p < kp is uniform over the wave) load nothing.
  Op8 xa[CH][2][RB], wa[CH][2][NB], gn[NORM ? CH : 1][2];
  auto load_weights = [&]() {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int p = min(wave + WAVES * i, a.kp - 1);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = 64 * p + 32 * h;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) wa[i][h][nb].u = *reinterpret_cast<const u32x4*>(wrow[nb] + p * wsp + h * wsh);
      }
    }
  };
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int p = min(wave + WAVES * i, a.kp - 1);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = 64 * p + 32 * h;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) xa[i][h][rb].u = *reinterpret_cast<const u32x4*>(xrow[rb] + p * xsp + h * xsh);
        gn[i][h].u = *reinterpret_cast<const u32x4*>(a.norm + k + 8 * g);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int p = wave + WAVES * i;
      if (p < a.kp) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) wa[i][h][nb].u = *reinterpret_cast<const u32x4*>(wrow[nb] + p * wsp + h * wsh);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) xa[i][h][rb].u = *reinterpret_cast<const u32x4*>(xrow[rb] + p * xsp + h * xsh);
        }
      }
    }
  }
  if constexpr (NORM) {
    __shared__ float ssum[WAVES][RB][16];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        if (wave + WAVES * i < a.kp)
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float lo = bf16_lo(xa[i][h][rb].u[e]), hi = bf16_hi(xa[i][h][rb].u[e]);
              ss = __fmaf_rn(lo, lo, ss);
              ss = __fmaf_rn(hi, hi, ss);
            }
      }
      ss = lane_group_sum(ss);
      if (g == 0) ssum[wave][rb][col] = ss;
    }
    // The weight tiles go out once x is in: issued with x, the CU took the waves' loads in issue
    // order and the later waves' x rows queued behind the first waves' weight tiles, so the
    // normalization barrier waited 1-2 us longer for them. A wave issues its weights when its own
    // x has arrived, or, with 32 x rows per workgroup (the SiLU*up shape), when every wave's has
    // (after the barrier): in a chain of 32 dependent launches Q/K/V took 6.32 us per launch with
    // the weights issued with x, 5.24 with them after a barrier that waits for no memory, 5.13
    // after the wave's own x, 5.44 after every wave's; gate/up 10.66, 10.12, 9.85 and 9.70 us.
    constexpr bool AFTER_BARRIER = RB > 1;
    if constexpr (!AFTER_BARRIER) load_weights();
    __syncthreads();
    if constexpr (AFTER_BARRIER) load_weights();
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) tot += ssum[w][rb][col];
      const float rstd = 1.f / sqrtf(tot / (float)a.k + a.eps);
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        if (wave + WAVES * i < a.kp)
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t xv = xa[i][h][rb].u[e], gv = gn[i][h].u[e];
              xa[i][h][rb].u[e] = pack_bf16(round_bf16(bf16_lo(xv) * rstd) * bf16_lo(gv),
                                            round_bf16(bf16_hi(xv) * rstd) * bf16_hi(gv));
            }
      }
    }
  }
  f32x4_t acc[RB][NB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[rb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    if (wave + WAVES * i < a.kp)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            acc[rb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa[i][h][nb].v, xa[i][h][rb].v, acc[rb][nb], 0, 0, 0);
  }

  // The waves' partials are summed in wave order through LDS, TP tiles per
  // phase (at most 32 KB of partials). Output tile o = (rb, nt) belongs to
  // wave o % WAVES, which sums its gate (and up) partial tiles and runs the
  // epilogue.
  constexpr int TP = TILES < 32 / WAVES ? TILES : 32 / WAVES;
  __shared__ f32x4_t red[WAVES][TP][64];
  f32x4_t gsum[OUT], usum[OUT];
#pragma unroll
  for (int ph = 0; ph < (TILES + TP - 1) / TP; ++ph) {
    if (ph) __syncthreads();  // the previous phase's partials have been read
#pragma unroll
    for (int j = 0; j < TP; ++j) {
      const int t = ph * TP + j;
      if (t < TILES) red[wave][j][lane] = acc[t / NB][t % NB];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TP; ++j) {
      const int t = ph * TP + j;
      if (t >= TILES) continue;
      const int rb = t / NB, nb = t % NB;
      const int o = rb * NT + nb % NT;  // output tile of this partial tile
      if (o % WAVES != wave) continue;
      f32x4_t s = red[0][j][lane];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) {
        const f32x4_t v = red[w][j][lane];
        s[0] += v[0];
        s[1] += v[1];
        s[2] += v[2];
        s[3] += v[3];
      }
      if (nb < NT) gsum[o] = s;
      else usum[o] = s;
    }
  }
#pragma unroll
  for (int o = 0; o < OUT; ++o) {
    if (o % WAVES != wave) continue;
    const int rb = o / NT, nt = o % NT;
    const int row = (rg * RB + rb) * 16 + col;
    if (row >= a.rows) continue;
    const int c = n0 + 16 * nt + 4 * g;
    float y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = round_bf16(gsum[o][e]);
    if (EPI == EPI_RESIDUAL) {
      const uint2 r = resv[o];
      y[0] += bf16_lo(r.x);
      y[1] += bf16_hi(r.x);
      y[2] += bf16_lo(r.y);
      y[3] += bf16_hi(r.y);
    } else if (EPI == EPI_SILU_MUL) {
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = round_bf16(y[e] / (1.f + expf(-y[e]))) * round_bf16(usum[o][e]);
    }
    // a tiled out is the next projection's tiled x (k = n_out = a.up)
    uint16_t* dst = a.out + ((a.layout & LAYOUT_OUT_TILED) ? tiled_offset(row, c, a.up >> 6) : (int64_t)row * a.ldo + c);
    *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16(y[0], y[1]), pack_bf16(y[2], y[3]));
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Launch shapes, from graph-replay timings of the 960-wide decoder's projections at 64 rows
// (weights streamed from HBM): narrow outputs use one 16-row block per workgroup (more
// workgroups); the joined gate/up projection 32 x rows and 32 output columns per workgroup
// (160 workgroups at 64 rows, all resident at once). With the RMSNorm prologue every
// workgroup normalizes its own x rows, so fewer rows per workgroup cost less VALU time than
// the second read of each weight tile they bring (64 rows per workgroup: 13.3 us, 32: 11.4 us).
struct Shape {
  int ch, nt, waves, rb;
};

constexpr int MAX_CH = 5;       // pairs per wave: k <= 5 * 8 * 64 = 2560
constexpr int MAX_NORM_CH = 2;  // with the RMSNorm prologue (k <= 1024), which keeps those
                                // variants out of scratch

Shape pick(int n_out, int kp, int epilogue) {
  Shape s;
  s.waves = 8;
  if (epilogue == EPI_SILU_MUL) {  // 32 gate and 32 up weight rows, 32 x rows
    s.nt = 2;
    s.rb = 2;
  } else {
    s.nt = (n_out % 32 == 0 && n_out / 16 > 64) ? 2 : 1;
    s.rb = 1;
  }
  s.ch = (kp + s.waves - 1) / s.waves;  // every pair of a wave in registers at once
  return s;
}

template <int CH, int NT, int WAVES, int RB, int EPI, bool NORM, int OPS>
void launch_one(const LinearArgs& a, hipStream_t st) {
  const int groups = (a.n_tiles + 7) / 8;
  const unsigned blocks = (unsigned)groups * 8u * (unsigned)a.row_groups;
  hipLaunchKernelGGL((linear_kernel<CH, NT, WAVES, RB, EPI, NORM, OPS>), dim3(blocks), dim3(64 * WAVES), 0, st, a);
}

template <int NT, int WAVES, int RB, int EPI, bool NORM, int OPS>
void launch_ch(int ch, const LinearArgs& a, hipStream_t st) {
  if constexpr (NORM) {
    if (ch == 1) launch_one<1, NT, WAVES, RB, EPI, NORM, OPS>(a, st);
    else launch_one<MAX_NORM_CH, NT, WAVES, RB, EPI, NORM, OPS>(a, st);
  } else {
    switch (ch) {
      case 1: launch_one<1, NT, WAVES, RB, EPI, NORM, OPS>(a, st); break;
      case 2: launch_one<2, NT, WAVES, RB, EPI, NORM, OPS>(a, st); break;
      case 3: launch_one<3, NT, WAVES, RB, EPI, NORM, OPS>(a, st); break;
      case 4: launch_one<4, NT, WAVES, RB, EPI, NORM, OPS>(a, st); break;
      default:
        if constexpr (EPI != EPI_SILU_MUL) launch_one<MAX_CH, NT, WAVES, RB, EPI, NORM, OPS>(a, st);
        break;  // dkv_linear_supported rules out the rest
    }
  }
}

template <int EPI, bool NORM, int OPS>
void launch_ops(const Shape& s, const LinearArgs& a, hipStream_t st) {
  if constexpr (EPI == EPI_SILU_MUL) {
    launch_ch<2, 8, 2, EPI, NORM, OPS>(s.ch, a, st);
  } else {
    if (s.nt == 2) launch_ch<2, 8, 1, EPI, NORM, OPS>(s.ch, a, st);
    else launch_ch<1, 8, 1, EPI, NORM, OPS>(s.ch, a, st);
  }
}

template <int EPI, bool NORM>
void launch_epi(const Shape& s, const LinearArgs& a, hipStream_t st) {
  switch (a.layout & (LAYOUT_W_TILED | LAYOUT_X_TILED)) {
    case 0: launch_ops<EPI, NORM, 0>(s, a, st); break;
    case LAYOUT_W_TILED: launch_ops<EPI, NORM, LAYOUT_W_TILED>(s, a, st); break;
    case LAYOUT_X_TILED: launch_ops<EPI, NORM, LAYOUT_X_TILED>(s, a, st); break;
    default: launch_ops<EPI, NORM, LAYOUT_W_TILED | LAYOUT_X_TILED>(s, a, st); break;
  }
}

}  // namespace
}  // namespace dkv

using namespace dkv;

extern "C" {

int dkv_linear_supported(int32_t rows, int32_t n, int32_t k, int32_t has_norm, int32_t epilogue) {
  if (rows < 0 || n <= 0 || k <= 0 || (k & 63) || epilogue < 0 || epilogue > 2) return 0;
  const int n_out = epilogue == EPI_SILU_MUL ? n / 2 : n;
  if (epilogue == EPI_SILU_MUL && (n & 1)) return 0;
  if (n_out % 16) return 0;
  const Shape s = pick(n_out, k / 64, epilogue);
  const int max_ch = has_norm ? MAX_NORM_CH : (epilogue == EPI_SILU_MUL ? 4 : MAX_CH);  // register budget
  if (s.ch > max_ch) return 0;
  if (s.nt == 2 && n_out % 32) return 0;
  return 1;
}

int dkv_linear_tiled(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride, int32_t rows,
                     int32_t n, int32_t k, const void* norm_weight, float eps, int32_t epilogue, const void* residual,
                     int64_t residual_row_stride, void* out, int64_t out_row_stride, int32_t layout, void* stream) {
  clear_error();
  const bool norm = norm_weight != nullptr;
  const int n_out = epilogue == EPI_SILU_MUL ? n / 2 : n;
  // row strides of tiled operands are not used (their layout fixes every offset)
  const bool wt = layout & LAYOUT_W_TILED, xt = layout & LAYOUT_X_TILED, ot = layout & LAYOUT_OUT_TILED;
  const bool rt = layout & LAYOUT_RES_TILED;
  if (!x || !w || !out || !dkv_linear_supported(rows, n, k, norm, epilogue) || !al16(x) || !al16(w) ||
      !al16(out) || (norm && !al16(norm_weight)) || (layout & ~15) || ((ot || rt) && (n_out & 63)) ||
      (rt && epilogue != EPI_RESIDUAL) ||
      (!xt && ((x_row_stride & 7) || x_row_stride < k)) || (!wt && ((w_row_stride & 7) || w_row_stride < k)) ||
      (!ot && ((out_row_stride & 3) || out_row_stride < n_out)) ||
      (epilogue == EPI_RESIDUAL &&
       (!residual || ((uintptr_t)residual & 7) || (!rt && ((residual_row_stride & 3) || residual_row_stride < n_out))))) {
    set_error("dkv_linear: unsupported or bad arguments (rows %d, n %d, k %d, epilogue %d, layout %d; k a multiple "
              "of 64, 16-byte aligned bf16 rows, a tiled out or residual n_out a multiple of 64)", rows, n, k,
              epilogue, layout);
    return DKV_EINVAL;
  }
  if (rows == 0) return 0;
  const Shape s = pick(n_out, k / 64, epilogue);
  LinearArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = x_row_stride;
  a.w = static_cast<const uint16_t*>(w);
  a.ldw = w_row_stride;
  a.norm = static_cast<const uint16_t*>(norm_weight);
  a.res = static_cast<const uint16_t*>(residual);
  a.ldr = residual_row_stride;
  a.out = static_cast<uint16_t*>(out);
  a.ldo = out_row_stride;
  a.eps = eps;
  a.rows = rows;
  a.k = k;
  a.kp = k / 64;
  a.n_tiles = n_out / (16 * s.nt);
  a.row_groups = (rows + 16 * s.rb - 1) / (16 * s.rb);
  a.up = n_out;
  a.layout = layout;
  hipStream_t st = (hipStream_t)stream;
  if (epilogue == EPI_PLAIN) norm ? launch_epi<EPI_PLAIN, true>(s, a, st) : launch_epi<EPI_PLAIN, false>(s, a, st);
  else if (epilogue == EPI_RESIDUAL)
    norm ? launch_epi<EPI_RESIDUAL, true>(s, a, st) : launch_epi<EPI_RESIDUAL, false>(s, a, st);
  else norm ? launch_epi<EPI_SILU_MUL, true>(s, a, st) : launch_epi<EPI_SILU_MUL, false>(s, a, st);
  return (int)hipGetLastError();
}

int dkv_linear(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride, int32_t rows, int32_t n,
               int32_t k, const void* norm_weight, float eps, int32_t epilogue, const void* residual,
               int64_t residual_row_stride, void* out, int64_t out_row_stride, void* stream) {
  return dkv_linear_tiled(x, x_row_stride, w, w_row_stride, rows, n, k, norm_weight, eps, epilogue, residual,
                          residual_row_stride, out, out_row_stride, 0, stream);
}

}  // extern "C"
