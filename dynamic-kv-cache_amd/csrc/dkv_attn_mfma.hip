// MFMA path of the fused packed-history attention (gfx950,
// v_mfma_f32_16x16x32_bf16), used for every chunk length: a 64-token frame
// chunk times 3 GQA heads gives 192 query rows per KV head; a one-token decode
// step fills 3 of the 16 rows of one block.
//
// Workgroup = 12 waves = one KV head, up to 192 query rows (every GQA head of
// that KV head), one contiguous range of units (64-key history tiles, then
// 64-row pieces of the chunk). The waves form two key groups: group c
// (waves 6c..6c+5) handles keys [32c, 32c + 32) of every unit, so three waves
// share each SIMD and one's softmax overlaps another's MFMAs. Wave w of a
// group owns 16-row query blocks w and w+6 (at most 2 per wave, which keeps a
// wave within the 168 VGPRs of 3 waves per SIMD). The two groups keep
// separate online-softmax states and merge through LDS after the last unit.
// Threads 0..511 stage and dequantize the units; the others only compute.
//
// Decode steps at precision 0 (at most 32 query rows per KV head) take the SMALL variant instead:
// 4 waves (two key groups of 2), every thread loading and dequantizing two 16-byte pieces of K
// and of V per unit, one buffer of raw bytes and tiles (36 KB of LDS), four workgroups per CU, so
// the default plan gives each workgroup one 64-key unit: after the history's burst of loads each
// workgroup has one unit left to do rather than three.
//
// Per unit:
//   1. the raw K and V sub-blocks (codes + (offset, scale) pairs, or bf16 rows)
//      are copied to LDS with one 16-byte load per thread each;
//   2. the 512 threads dequantize (q*s + a with a separately rounded multiply
//      and add, the reference's unpack, src/kv_quantization.py:90-91, so K and
//      V equal what reconstruct() returns) into a bf16 K tile [key][d] and a
//      transposed bf16 V tile [d][key]. (A fused multiply-add, which a compiler
//      may make of the Triton expression at src/gpu_kernels.py:67-68, rounds
//      about 0.1% of the elements to another bf16 value; with logits near 65 one
//      such K element of a dominant key moves an output by ~0.1.)
//   3. each wave computes S^T = K Q^T for its blocks (keys on the MFMA M axis,
//      queries on N), runs the online softmax per query column in registers,
//      and accumulates O^T = V^T P^T with P^T taken straight from the S^T
//      accumulators: key k of the group's 32 keys sits in S^T block j at row
//      4g + i with k = 8g + 4j + i, so lane group g of blocks 0 and 1 holds
//      keys 8g .. 8g+7, the eight k-slots the PV MFMA wants from that group.
//
// Splitting the history: with several splits per KV head each workgroup
// writes partials to the workspace, (running max, sum) per row plus O: fp32
// and unnormalized at PREC 1 (combine_kernel merges them), fp16 O / sum at
// PREC 0 (combine_half_kernel; rows past the fp16 range are stored scaled,
// see half_partial_exponent). Frame chunks store the partials nontemporally:
// the end of a kernel writes every dirty L2 line back, and partials kept out
// of L2 leave nothing to write back (3 us less per launch at past 8128).
// Launches of one query block per wave (decode steps, short chunks) have
// small partials and store them plainly (part_store).
//
// The in-kernel merge build (DKV_INKERNEL_MERGE, a measurement build) merges
// the splits in this launch instead: each workgroup waits for its precision-0
// partial stores (vmcnt 0) and counts its arrival on its (KV head, row
// group)'s counter with an agent-scope release; the workgroup that arrives
// last acquires, resets the counter for the next launch and merges every split
// with the one-wave merge's row arithmetic (dkv_merge.h), so the output bits
// equal the two-launch path's wherever that merges one row per wave (launches
// of few rows use the wide merge, which sums in another order). No workgroup
// waits for another. Timed on this
// kernel, the arrival comes 2-3 us after a workgroup's stores, and one
// workgroup then reads all of its KV head's partials: decode steps at past
// 8128 ran 13.8 us against 11.7 with the second launch, and a 64-token frame
// chunk (192 rows x 43 splits, 1.1 MB of partials per KV head) 55.6 us
// against 16.1, so the library keeps the merge kernel.
//
// Precision (template PREC):
//   0  the reference kernel's rounding points (src/gpu_kernels.py:93-102):
//      dequantized K/V and p are rounded to bf16, fp32 accumulation;
//   1  fp32-accurate: K = K_hi + K_lo and V = V_hi + V_lo, p = p_hi + p_lo
//      (bf16 pairs, 2^-17 relative), S = Q K_hi + Q K_lo and
//      O = P_hi V_hi + P_hi V_lo + P_lo V_hi; the lo terms are skipped for
//      bf16 units, where they are exactly zero.
#include "dkv_attn_common.h"
#include "dkv_merge.h"
#include <type_traits>

namespace dkv {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int KG_WAVES = MFMA_KG_WAVES;    // waves per key group
constexpr int MF_THREADS = 2 * KG_WAVES * 64;  // 768
constexpr int MF_LOADERS = 512;            // threads that load, stage and dequantize a unit
constexpr int KS = 72;       // LDS row stride, in bf16 elements, of the K and V^T tiles
constexpr int RAWP = 9216;   // padded raw bytes of one sub-block (64 rows x 128 B + 16 B per 128 B)
constexpr int MRG_STRIDE = D + 4;  // fp32 row stride of the key-group merge: 16 query rows of one
                                   // store land on different banks

union Pack8 {
  bf16x8 v;
  uint4 u;
};

// Two fp32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
}
__device__ __forceinline__ float bf16_lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi_f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Max / sum over the four lane groups g = lane / 16 that hold one query
// column (lanes col, col + 16, col + 32, col + 48), with the gfx950 lane swaps
// (VALU, no LDS round trip): after permlane32_swap the pair is (x[l mod 32],
// x[l mod 32 + 32]), after permlane16_swap (x[row 2k], x[row 2k + 1]).
__device__ __forceinline__ float group_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = max_nn(__uint_as_float(r[0]), __uint_as_float(r[1]));
  auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_nn(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float group_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// The running max of a wave moves only when some column's max grows by more
// than this (log2 units); until then p = 2^(x - m) stays below 2^8 and the
// accumulators need no rescaling. Precision 0 keeps the reference's exact
// running max (p is rounded to bf16 relative to it, src/gpu_kernels.py:98-102),
// so it only skips the rescale when no column's max grew at all.
template <int PREC>
constexpr float rescale_log2() { return PREC ? 8.f : 0.f; }

// Split partials: plain stores in the one-block-per-wave variant (NBW 1, at most 96 query rows
// per group: decode steps and short chunks, whose partials are small, so the end of the kernel
// writes them back from L2 quickly and the merge finds them in the cache hierarchy); nontemporal
// stores otherwise, which keep the larger partials of frame chunks from being written back from
// L2 at the end of the kernel (+3 us at past 8128). A compile-time choice: a runtime branch
// between the two stores is merged by the compiler into one store without the nontemporal hint.
template <bool PLAIN, typename T>
__device__ __forceinline__ void part_store(const T& v, T* p) {
  if constexpr (PLAIN)
    *p = v;
  else
    __builtin_nontemporal_store(v, p);
}

// Raw sub-blocks sit in LDS with 16 bytes of padding after every 128 bytes,
// which spreads the rows a dequantizing wave reads over all banks.
__device__ __forceinline__ int padded(int off) { return off + ((off >> 7) << 4); }

// 8 fp32 values q*s + a of rows r0 and r0 + 1 (r0 even), columns [8*db, 8*db + 8), of a 4/8-bit
// raw sub-block in LDS (multiply and add rounded separately, as the reference's unpack). Every
// LDS read (the two rows' codes and their (offset, scale) pairs, which sit side by side) is
// issued before the first use, so a unit's dequantization waits on one LDS round trip (with one
// row per call and the width branch between the reads, the compiler waited on each row's reads
// in turn).
template <int BITS>
__device__ __forceinline__ void dequant_pair(const uint8_t* raw, int rows, int r0, int db, float* x0, float* x1) {
  constexpr int RB = BITS == 4 ? 32 : 64;
  const float4 as = *reinterpret_cast<const float4*>(raw + padded(rows * RB + 8 * r0));  // (a0, s0, a1, s1)
  float q0[8], q1[8];
  if (BITS == 4) {
    const uint32_t w0 = *reinterpret_cast<const uint32_t*>(raw + padded(r0 * 32 + db * 4));
    const uint32_t w1 = *reinterpret_cast<const uint32_t*>(raw + padded(r0 * 32 + 32 + db * 4));
    uint32_t ev0 = w0 & 0x0f0f0f0fu, od0 = (w0 >> 4) & 0x0f0f0f0fu;  // even / odd elements
    uint32_t ev1 = w1 & 0x0f0f0f0fu, od1 = (w1 >> 4) & 0x0f0f0f0fu;
    // Opaque to the optimizer (no instruction), which would otherwise fold each byte back into a
    // nibble extract of w (v_bfe, then a convert) instead of one v_cvt_f32_ubyteN per element.
    asm("" : "+v"(ev0), "+v"(od0), "+v"(ev1), "+v"(od1));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      q0[2 * i] = (float)((ev0 >> (8 * i)) & 255u);
      q0[2 * i + 1] = (float)((od0 >> (8 * i)) & 255u);
      q1[2 * i] = (float)((ev1 >> (8 * i)) & 255u);
      q1[2 * i + 1] = (float)((od1 >> (8 * i)) & 255u);
    }
  } else {
    const uint2 w0 = *reinterpret_cast<const uint2*>(raw + padded(r0 * 64 + db * 8));
    const uint2 w1 = *reinterpret_cast<const uint2*>(raw + padded(r0 * 64 + 64 + db * 8));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      q0[i] = (float)((w0.x >> (8 * i)) & 255u);
      q0[4 + i] = (float)((w0.y >> (8 * i)) & 255u);
      q1[i] = (float)((w1.x >> (8 * i)) & 255u);
      q1[4 + i] = (float)((w1.y >> (8 * i)) & 255u);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    x0[i] = __fadd_rn(__fmul_rn(q0[i], as.y), as.x);
    x1[i] = __fadd_rn(__fmul_rn(q1[i], as.w), as.z);
  }
}

// Row r, columns [8*db, 8*db + 8), of a bf16 raw sub-block (16-bit tiles and chunk pieces).
__device__ __forceinline__ uint4 bf16_row8(const uint8_t* raw, int r, int db) {
  return *reinterpret_cast<const uint4*>(raw + padded(r * 128 + db * 16));
}

// Loader index of a thread: which 512 threads load, stage and dequantize a unit. With two query
// blocks per wave (every wave computes) they are waves 0-7. With one (decode steps, short
// chunks: only query block 0 of each key group, waves 0 and 6, computes) they are waves 1-5, 7,
// 8 and 10, so the computing waves work on one unit while the others dequantize the next
// rather than after it (decode at past 8128: 10.9 -> 10.7 us; the frame chunk ran 0.3 us slower
// with this order). Wave w holds slot SLOTS >> 4w & 15 (15: no slot); waves 9 and 11 idle so
// that each SIMD keeps two loading waves (wave w runs on SIMD w mod 4).
template <int NBW>
__device__ __forceinline__ int loader_index(int wave, int lane) {
  constexpr uint64_t SLOTS = NBW == 1 ? 0xF7F65F43210FULL : 0xFFFF76543210ULL;
  const int slot = (int)((SLOTS >> (4 * wave)) & 15);
  return slot == 15 ? MF_LOADERS + lane : slot * 64 + lane;
}

// One 16-byte piece of K (loader index p = 0..511 -> pieces 0..511) and one of V;
// threads with p >= 512 load nothing (every sub-block is at most 512 pieces).
// Lanes whose piece is past the unit's bytes (or past the chunk's rows) load nothing and keep the
// registers' previous contents, which the staging copies to LDS bytes that dequantization never
// reads. Writing zeros into them here (the first version did) made the compiler wait for every
// load in flight before each unit's loads, since another branch's loads into the same registers
// could have been pending: units 1 and 2, prefetched at kernel start, went out only after unit
// 0's (and then unit 1's) bytes had arrived. The callers zero the registers once, before any load.
__device__ __forceinline__ void raw_load(const dkv_attn_args& a, const Unit& un, int h, int p, uint4& wk, uint4& wv) {
  // The kind of unit picks the addresses; one pair of loads after the choice (with a pair in each
  // branch, the registers' values had to be merged after the loads, and the copies waited for them).
  const uint8_t* kp;
  const uint8_t* vp;
  bool ok;
  if (un.chunk) {
    const int row = p >> 3, c = p & 7;
    ok = row < un.valid;
    const int64_t j = un.first + row;
    kp = static_cast<const uint8_t*>(a.k_new) + 2 * (h * a.kn_head_stride + j * a.kn_tok_stride + c * 8);
    vp = static_cast<const uint8_t*>(a.v_new) + 2 * (h * a.vn_head_stride + j * a.vn_tok_stride + c * 8);
  } else {
    ok = p < (int)(subblock_bytes(un.rows, un.bits) >> 4);
    kp = un.ksub + 16 * p;
    vp = un.vsub + 16 * p;
  }
  // history bytes are read once per launch: nontemporal loads (past 8128: 19.0 -> 18.6 us per
  // layer, a decode step 13.6 -> 13.0 us); the chunk's rows are read by one workgroup each too
  if (ok) {
    wk = __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp)));
    wv = __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vp)));
  }
}

// Unit u = u0 + rel of a workgroup's range. With `arg_tiles` the history
// descriptors come from the launch's argument block (one scalar load each).
// Otherwise the first 64 history tiles of the range come from `win`, the
// descriptors every wave loaded with one vector load at kernel start (lane i
// holds unit u0 + i), so the unit walk never waits on a scalar load; later
// tiles fall back to reading the table.
__device__ __forceinline__ Unit unit_at(const dkv_attn_args& a, const Hist& hs, int u, int rel, int h,
                                        const uint4& win, bool arg_tiles) {
  if (u >= hs.n_tiles) return get_unit(a, hs, u, h);
  if (arg_tiles) {
    const uint4 d = arg_tile(u);
    return history_unit(a, hs, d.x, d.y, d.z, d.w, h);
  }
  if (rel < 64)
    return history_unit(a, hs, (uint32_t)__builtin_amdgcn_readlane((int)win.x, rel),
                        (uint32_t)__builtin_amdgcn_readlane((int)win.y, rel),
                        (uint32_t)__builtin_amdgcn_readlane((int)win.z, rel),
                        (uint32_t)__builtin_amdgcn_readlane((int)win.w, rel), h);
  // past the window: the whole descriptor in one 16-byte load (not four narrow ones, whose
  // destination registers would make every iteration wait on the loads in flight)
  const uint4 d = *reinterpret_cast<const uint4*>(a.tiles + u);
  return history_unit(a, hs, __builtin_amdgcn_readfirstlane(d.x), __builtin_amdgcn_readfirstlane(d.y),
                      __builtin_amdgcn_readfirstlane(d.z), __builtin_amdgcn_readfirstlane(d.w), h);
}

// NBW = 16-row query blocks each wave computes (1..2). A wave whose first
// block is past the last row skips the MFMA work (a scalar branch); other
// waves compute all NBW blocks, those past the last row on zero queries, and
// store only real rows.
#ifdef DKV_TIMELINE
// events: 0 entry, 1 first unit staged in LDS, 2 first unit dequantized, 3 first unit computed,
// 4 last unit computed, 5 key groups merged, 6 stores issued, 7 arguments arrived; in the in-kernel
// merge build also 8 arrival counted, 9 splits merged and stored (by the last workgroup only)
static __device__ uint64_t tl_mfma[TL_SLOTS * TL_EVENTS];
#endif

// ARGT: the history's tile descriptors come in the argument block (first parameter ArgTiles)
// rather than from the device table (first parameter NoArgTiles).
// SMALL: the decode-step variant (precision 0, at most two query blocks per KV head): 4 waves in
// two key groups of 2, every thread loads and dequantizes two pieces of each unit, one buffer of
// raw bytes and tiles (36 KB of LDS), so four workgroups share a CU and the default plan gives
// each workgroup one unit of the history.
template <int PREC, int NBW, bool ARGT, bool SMALL>
__global__ void __launch_bounds__(SMALL ? 256 : MF_THREADS, SMALL ? MFMA_SMALL_PER_CU : 3)
attn_mfma_kernel(typename std::conditional<ARGT, ArgTiles, NoArgTiles>::type, dkv_attn_args a, int units,
                 int splits, int cap, int rpg, float* __restrict__ part_o, float2* __restrict__ part_ml
#if DKV_INKERNEL_MERGE
                 , int fused, uint32_t* __restrict__ counters
#endif
                 ) {
  // LDS: two raw stages of (K, V) sub-blocks and two sets of bf16 tiles
  // (K, V^T, and for PREC 1 their lo parts). After the last unit the same
  // bytes hold the key-group merge (O rows, then (max, sum) pairs).
  constexpr int KGW = SMALL ? 2 : KG_WAVES;  // waves per key group
  constexpr int NST = SMALL ? 1 : 2;          // raw stages and tile sets
  constexpr int PN = SMALL ? 2 : 1;           // 16-byte pieces of K and of V a loading thread takes
  constexpr int MROWS = KGW * 16 * NBW;       // query rows of one key group's blocks
  constexpr int NT = PREC ? 4 : 2;
  constexpr int RAW_BYTES = NST * 2 * RAWP;
  constexpr int TILE_BYTES = 64 * KS * 2;
  constexpr int SMEM = RAW_BYTES + NST * NT * TILE_BYTES;
  static_assert(SMEM >= MROWS * MRG_STRIDE * 4 + MROWS * 8, "merge buffer must fit");
  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];
  auto raw_buf = [&](int st, int kv) { return smem + ((NST > 1 ? st : 0) * 2 + kv) * RAWP; };
  auto tile = [&](int b, int which) {
    return reinterpret_cast<uint16_t*>(smem + RAW_BYTES + ((NST > 1 ? b : 0) * NT + which) * TILE_BYTES);
  };

  DKV_TL(tl_mfma, 0);
  // Every argument that the first history and query loads depend on, read together: placed by
  // their uses, the compiler issued these scalar loads in seven dependent rounds (each a round
  // trip to the cache hierarchy) before the first history load; the empty asm needs them all at
  // once, so they go out in one round.
  // A decode launch of the default plan has as many splits as units, so workgroup s walks unit s
  // alone: with the descriptors in the argument block, descriptor s is read in the same round and
  // used when u0 == s turns out to hold (a guess that costs one scalar load when it does not).
  uint4 spec = make_uint4(0, 0, 0, 0);
  if constexpr (ARGT && SMALL) spec = arg_tile(min((int)blockIdx.x, DKV_ARG_TILES - 1));
  if constexpr (ARGT)
    asm volatile("" ::"s"(units), "s"(splits), "s"(cap), "s"(rpg), "s"(a.past), "s"(a.n_tiles), "s"(a.step),
                 "s"(a.heads), "s"(a.q_heads), "s"(a.nq), "s"(a.q), "s"(a.q_head_stride), "s"(a.q_tok_stride),
                 "s"(a.arena), "s"(a.layer), "s"(a.n_segs), "s"(a.scale), "s"(spec.x), "s"(spec.y), "s"(spec.z),
                 "s"(spec.w));
  else
    asm volatile("" ::"s"(units), "s"(splits), "s"(cap), "s"(rpg), "s"(a.past), "s"(a.n_tiles), "s"(a.step),
                 "s"(a.heads), "s"(a.q_heads), "s"(a.nq), "s"(a.q), "s"(a.q_head_stride), "s"(a.q_tok_stride),
                 "s"(a.arena), "s"(a.layer), "s"(a.n_segs), "s"(a.scale), "s"(a.tiles));
  Hist hs;
  const int active = runtime_plan(a, hs, units, splits, cap);
  const int split = blockIdx.x, h = blockIdx.y, rg = blockIdx.z;
  const int G = a.q_heads / a.heads;
  const int R = G * a.nq;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lt = SMALL ? t : loader_index<NBW>(wave, lane);  // SMALL: pieces lt and lt + 256
  const int kg = wave / KGW, w = wave - kg * KGW;  // key group, wave within the group
  const int col = lane & 15, g = lane >> 4;
  if (split >= active) return;  // graph replay over a shorter history than the launch bound
  DKV_TL(tl_mfma, 7);           // the argument block (and any step pair) has arrived
  const int u0 = (int)((int64_t)units * split / active);
  const int u1 = (int)((int64_t)units * (split + 1) / active);
  const float xs = a.scale * LOG2E;
  // Row group rg holds rows [r0, r_end): rpg rows (a multiple of 16, at most MFMA_ROWS), the
  // last group fewer.
  const int r0 = rg * rpg, r_end = min(R, r0 + rpg);
  const bool wave_on = r0 + w * 16 < r_end;  // wave-uniform

  // Query operands and masking bounds of this lane's query column in each block.
  bf16x8 qop[NBW][2];
  int qlo[NBW], qhi[NBW];
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    const int r = r0 + (w + KGW * nb) * 16 + col;
    Pack8 q0, q1;
    q0.u = q1.u = make_uint4(0, 0, 0, 0);
    qlo[nb] = 0;
    qhi[nb] = -1;
    if (r < r_end) {
      const int gq = r / a.nq, m = r - gq * a.nq;
      const uint16_t* src = static_cast<const uint16_t*>(a.q) + (int64_t)(h * G + gq) * a.q_head_stride +
                            (int64_t)m * a.q_tok_stride + 8 * g;
      q0.u = *reinterpret_cast<const uint4*>(src);
      q1.u = *reinterpret_cast<const uint4*>(src + 32);
      qlo[nb] = chunk_seg_start(a, m);
      qhi[nb] = m;
    }
    qop[nb][0] = q0.v;
    qop[nb][1] = q1.v;
  }

  f32x4 acc_o[NBW][4];
  float m_run[NBW], l_part[NBW];
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
#pragma unroll
    for (int db = 0; db < 4; ++db) acc_o[nb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_run[nb] = -INFINITY;
    l_part[nb] = 0.f;
  }

  // Dequantize a staged unit into bf16 tiles. Threads 0..255 build K (thread =
  // key pair kp, column block db, db fastest: 16-byte row stores), threads
  // 256..511 build V^T (kp fastest, so the 4-byte stores of one instruction
  // cover 32 consecutive words of a V^T row). bf16 rows (16-bit tiles, chunk
  // pieces) are copied or byte-permuted without a float round trip.
  auto dequant_piece = [&](const Unit& un, int st, int b, int q) {
    if (q >= MF_LOADERS) return;
    const bool is_v = q >= 256;
    const int kp = is_v ? (q & 31) : ((q & 255) >> 3);
    const int db = is_v ? ((q & 255) >> 5) : (q & 7);
    const int r0 = 2 * kp, r1 = r0 + 1;
    const bool ok0 = r0 < un.valid, ok1 = r1 < un.valid;
    const uint8_t* raw = raw_buf(st, is_v ? 1 : 0);
    if (un.bits == 16) {
      const uint4 z = make_uint4(0, 0, 0, 0);
      const uint4 w0 = ok0 ? bf16_row8(raw, r0, db) : z;
      const uint4 w1 = ok1 ? bf16_row8(raw, r1, db) : z;
      if (!is_v) {
        uint16_t* k_hi = tile(b, 0);
        *reinterpret_cast<uint4*>(k_hi + r0 * KS + db * 8) = w0;
        *reinterpret_cast<uint4*>(k_hi + r1 * KS + db * 8) = w1;
      } else {
        uint16_t* v_hi = tile(b, 1);
        const uint32_t a0[4] = {w0.x, w0.y, w0.z, w0.w}, a1[4] = {w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          *reinterpret_cast<uint32_t*>(v_hi + (db * 8 + 2 * i) * KS + r0) = __builtin_amdgcn_perm(a1[i], a0[i], 0x05040100u);
          *reinterpret_cast<uint32_t*>(v_hi + (db * 8 + 2 * i + 1) * KS + r0) = __builtin_amdgcn_perm(a1[i], a0[i], 0x07060302u);
        }
      }
      return;
    }
    float x0[8], x1[8];
    if (un.bits == 4) dequant_pair<4>(raw, un.rows, r0, db, x0, x1);
    else dequant_pair<8>(raw, un.rows, r0, db, x0, x1);
    if (un.valid != TILE) {  // wave-uniform: every row of a full tile is valid
      // rows past `valid` hold stale staging bytes; they become zeros (P is 0 there, and a
      // stale NaN would still poison P.V)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        x0[i] = ok0 ? x0[i] : 0.f;
        x1[i] = ok1 ? x1[i] : 0.f;
      }
    }
    if (!is_v) {
      uint16_t* k_hi = tile(b, 0);
      uint16_t* k_lo = tile(b, PREC ? 2 : 0);
      uint4 h0, h1;
      h0 = make_uint4(pk_bf16(x0[0], x0[1]), pk_bf16(x0[2], x0[3]), pk_bf16(x0[4], x0[5]), pk_bf16(x0[6], x0[7]));
      h1 = make_uint4(pk_bf16(x1[0], x1[1]), pk_bf16(x1[2], x1[3]), pk_bf16(x1[4], x1[5]), pk_bf16(x1[6], x1[7]));
      *reinterpret_cast<uint4*>(k_hi + r0 * KS + db * 8) = h0;
      *reinterpret_cast<uint4*>(k_hi + r1 * KS + db * 8) = h1;
      if (PREC) {
        const uint32_t hw0[4] = {h0.x, h0.y, h0.z, h0.w}, hw1[4] = {h1.x, h1.y, h1.z, h1.w};
        uint32_t l0[4], l1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          l0[i] = pk_bf16(x0[2 * i] - bf16_lo_f(hw0[i]), x0[2 * i + 1] - bf16_hi_f(hw0[i]));
          l1[i] = pk_bf16(x1[2 * i] - bf16_lo_f(hw1[i]), x1[2 * i + 1] - bf16_hi_f(hw1[i]));
        }
        *reinterpret_cast<uint4*>(k_lo + r0 * KS + db * 8) = make_uint4(l0[0], l0[1], l0[2], l0[3]);
        *reinterpret_cast<uint4*>(k_lo + r1 * KS + db * 8) = make_uint4(l1[0], l1[1], l1[2], l1[3]);
      }
    } else {
      uint16_t* v_hi = tile(b, 1);
      uint16_t* v_lo = tile(b, PREC ? 3 : 1);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t hv = pk_bf16(x0[i], x1[i]);
        *reinterpret_cast<uint32_t*>(v_hi + (db * 8 + i) * KS + r0) = hv;
        if (PREC)
          *reinterpret_cast<uint32_t*>(v_lo + (db * 8 + i) * KS + r0) =
              pk_bf16(x0[i] - bf16_lo_f(hv), x1[i] - bf16_hi_f(hv));
      }
    }
  };
  // A loading thread's pieces of a unit: lt (and lt + 256 in SMALL, K then V^T).
  auto dequant = [&](const Unit& un, int st, int b) {
#pragma unroll
    for (int i = 0; i < PN; ++i) dequant_piece(un, st, b, lt + 256 * i);
  };

  // MFMA work of one dequantized unit held in tile set b; `first` marks the workgroup's first
  // unit, before which the running maxima are -inf and the accumulators zero.
  auto compute = [&](const Unit& un, int b, bool first) {
    if (!wave_on) return;
    const uint16_t* k_hi = tile(b, 0);
    const uint16_t* v_hi = tile(b, 1);
    const uint16_t* k_lo = tile(b, PREC ? 2 : 0);
    const uint16_t* v_lo = tile(b, PREC ? 3 : 1);
    const bool lo_on = PREC && un.bits != 16;
    // S^T = K Q^T over this group's 32 keys: block j holds keys 32 kg + 8 g' + 4 j + i
    // in its row 4 g' + i, so A-operand row `col` of block j is key
    // 32 kg + 8 (col / 4) + 4 j + col % 4.
    f32x4 sc[NBW][2];
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) sc[nb][0] = sc[nb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int pass = 0; pass < (PREC ? 2 : 1); ++pass) {
      if (pass == 1 && !lo_on) break;
      const uint16_t* kt = pass ? k_lo : k_hi;
      Pack8 ka[2][2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int key = 32 * kg + 8 * (col >> 2) + 4 * j + (col & 3);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          ka[j][ks].u = *reinterpret_cast<const uint4*>(kt + key * KS + 32 * ks + 8 * g);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int nb = 0; nb < NBW; ++nb)
            sc[nb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[j][ks].v, qop[nb][ks], sc[nb][j], 0, 0, 0);
    }
    // V^T operands: row d = 16 db + col, keys 32 kg + 8 g .. + 7.
    Pack8 va[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
      va[db].u = *reinterpret_cast<const uint4*>(v_hi + (16 * db + col) * KS + 32 * kg + 8 * g);

    // Online softmax per query column over the group's 32 keys (8 per lane).
    Pack8 p_hi[NBW], p_lo[NBW];
    const bool full = !un.chunk && un.valid == TILE;
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
      float s[8];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[4 * j + i] = sc[nb][j][i];
      if (!full) {
        // Visible keys of this column form one range [lo, hi) of the unit: keys
        // below `valid`, and for a chunk piece the causal / segment window
        // [qlo, qhi] of the query row. Lane group g holds keys base + e, e = 4 j + i.
        const int base = 32 * kg + 8 * g;
        const int lo = (un.chunk ? max(qlo[nb] - un.first, 0) : 0) - base;
        const int hi = (un.chunk ? min(qhi[nb] - un.first + 1, un.valid) : un.valid) - base;
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e] = (e >= lo && e < hi) ? s[e] : -INFINITY;
      }
      float mt = max_nn(max_nn(max_nn(s[0], s[1]), max_nn(s[2], s[3])), max_nn(max_nn(s[4], s[5]), max_nn(s[6], s[7])));
      const float mcand = group_max(mt) * xs;
      // Lazy rescaling: a wave moves its running maxima (and rescales its
      // accumulators) only when some column's max grew by more than
      // rescale_log2; otherwise p = 2^(x - m_run) <= 2^rescale_log2.
      if (PREC == 0 && first) {
        // nothing accumulated yet: the maxima move without rescaling zeros (the branch below
        // would multiply them by 0; at precision 0 and three units per workgroup it runs in most
        // units; at precision 1 it rarely runs past the first unit, and the separate first-unit
        // path made the kernel spill)
        m_run[nb] = max_nn(m_run[nb], mcand);
      } else if (__builtin_amdgcn_ballot_w64(mcand > m_run[nb] + rescale_log2<PREC>())) {
        const float mnew = max_nn(m_run[nb], mcand);
        const float alpha = mnew == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run[nb] - mnew);
        m_run[nb] = mnew;
        l_part[nb] *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db) acc_o[nb][db] *= alpha;
      }
      const float mref = m_run[nb] == -INFINITY ? 0.f : m_run[nb];
      float p[8], psum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[e] = __builtin_amdgcn_exp2f(__fmaf_rn(s[e], xs, -mref));
        psum += p[e];
      }
      l_part[nb] += psum;
      const uint32_t w0 = pk_bf16(p[0], p[1]), w1 = pk_bf16(p[2], p[3]);
      const uint32_t w2 = pk_bf16(p[4], p[5]), w3 = pk_bf16(p[6], p[7]);
      p_hi[nb].u = make_uint4(w0, w1, w2, w3);
      if (PREC)
        p_lo[nb].u = make_uint4(pk_bf16(p[0] - bf16_lo_f(w0), p[1] - bf16_hi_f(w0)),
                                pk_bf16(p[2] - bf16_lo_f(w1), p[3] - bf16_hi_f(w1)),
                                pk_bf16(p[4] - bf16_lo_f(w2), p[5] - bf16_hi_f(w2)),
                                pk_bf16(p[6] - bf16_lo_f(w3), p[7] - bf16_hi_f(w3)));
    }
    // O^T += V^T P^T.
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int nb = 0; nb < NBW; ++nb)
        acc_o[nb][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[db].v, p_hi[nb].v, acc_o[nb][db], 0, 0, 0);
    if (PREC) {
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb)
          acc_o[nb][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[db].v, p_lo[nb].v, acc_o[nb][db], 0, 0, 0);
      if (lo_on) {
#pragma unroll
        for (int db = 0; db < 4; ++db)
          va[db].u = *reinterpret_cast<const uint4*>(v_lo + (16 * db + col) * KS + 32 * kg + 8 * g);
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int nb = 0; nb < NBW; ++nb)
            acc_o[nb][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[db].v, p_hi[nb].v, acc_o[nb][db], 0, 0, 0);
      }
    }
  };

  // Software pipeline, one barrier per unit: iteration i dequantizes unit
  // i+1 into the other tile set, stages unit i+2's raw bytes (loaded during
  // iteration i-1; with two query blocks per wave unit 2's at kernel start) and
  // issues unit i+3's loads, then
  // runs unit i's MFMA work.
  // So one wave's dequantization overlaps another's MFMAs, and each unit's
  // HBM latency hides behind a full iteration.
  const int n = u1 - u0;
  constexpr bool in_args = ARGT;  // descriptors in the argument block
  uint4 win = make_uint4(0, 0, 0, 0);
  if (!in_args && u0 + lane < min(u1, hs.n_tiles)) win = *reinterpret_cast<const uint4*>(a.tiles + u0 + lane);
  // Wait for the window here, on every path (unit 0 reads it next anyway): a wait the compiler
  // cannot place before the loop lands inside it, where it also waits for the prefetches in flight.
  asm volatile("" ::"v"(win.x), "v"(win.y), "v"(win.z), "v"(win.w));
  auto unit = [&](int rel) {
    if (ARGT && SMALL && rel == 0 && u0 == split && u0 < hs.n_tiles)  // wave-uniform
      return history_unit(a, hs, spec.x, spec.y, spec.z, spec.w, h);
    return unit_at(a, hs, u0 + rel, rel, h, win, in_args);
  };
  // A thread's raw bytes of one unit: PN pieces of K and of V.
  struct Raw {
    uint4 k[PN], v[PN];
  };
  auto load = [&](int rel, Raw& r) {
#pragma unroll
    for (int i = 0; i < PN; ++i) raw_load(a, unit(rel), h, lt + 256 * i, r.k[i], r.v[i]);
  };
  // The zeros of a Raw, made opaque where they are written (the kernel's start): the compiler
  // would otherwise move them down to the loads, and each move brings back the wait described at
  // raw_load.
  auto opaque = [&](Raw& r) {
#pragma unroll
    for (int i = 0; i < PN; ++i)
      asm volatile("" : "+v"(r.k[i].x), "+v"(r.k[i].y), "+v"(r.k[i].z), "+v"(r.k[i].w), "+v"(r.v[i].x),
                   "+v"(r.v[i].y), "+v"(r.v[i].z), "+v"(r.v[i].w));
  };
  auto stage = [&](int st, const Raw& r) {
#pragma unroll
    for (int i = 0; i < PN; ++i) {
      const int q = lt + 256 * i;
      if (q >= MF_LOADERS) continue;  // a raw sub-block is at most MF_LOADERS pieces of 16 bytes
      *reinterpret_cast<uint4*>(raw_buf(st, 0) + padded(16 * q)) = r.k[i];
      *reinterpret_cast<uint4*>(raw_buf(st, 1) + padded(16 * q)) = r.v[i];
    }
  };
  if constexpr (SMALL) {
    // One buffer: per unit, load, stage, dequantize and compute, with a barrier after the
    // staging and one after the dequantization. The default plan gives each workgroup one unit;
    // graph replays over longer histories may give it more, whose loads then wait for the unit
    // before (no registers held across the MFMA work: four workgroups per CU need <= 128 VGPRs).
    Raw r = {};
    opaque(r);
    for (int i = 0; i < n; ++i) {
      load(i, r);
      if (i) __syncthreads();  // unit i - 1's MFMA work is done with the tiles
      stage(0, r);
      if (i == 0) DKV_TL(tl_mfma, 1);
      __syncthreads();
      dequant(unit(i), 0, 0);
      if (i == 0) DKV_TL(tl_mfma, 2);
      __syncthreads();
      compute(unit(i), 0, i == 0);
      if (i == 0) DKV_TL(tl_mfma, 3);
    }
  } else {
    Raw r = {}, r0 = {}, r2 = {};
    opaque(r);
    opaque(r0);
    opaque(r2);
    if (n > 0) load(0, r0);
    if (n > 1) load(1, r);  // in flight while unit 0 is staged
    // With two query blocks per wave (frame chunks, candidate batches) unit 2's loads go out at
    // once too, not after unit 0 is staged and dequantized (past 1024 11.60 -> 11.37 us, 4096
    // 13.98 -> 13.83). With one (decode steps), whose units compute little, the larger first
    // burst delayed unit 0 more than it saved (11.68 -> 11.83 us at past 8128).
    constexpr bool early2 = NBW == 2;
    if (early2 && n > 2) load(2, r2);
    if (n > 0) stage(0, r0);
    // unit 0's load registers are settled on every path before the loop (the compiler does not
    // tie the two n > 0 tests together and would otherwise wait on them inside the loop, where a
    // wait also drains the prefetches in flight)
    asm volatile("" ::"v"(r0.k[0].x), "v"(r0.k[0].y), "v"(r0.k[0].z), "v"(r0.k[0].w), "v"(r0.v[0].x),
                 "v"(r0.v[0].y), "v"(r0.v[0].z), "v"(r0.v[0].w));
    DKV_TL(tl_mfma, 1);
    __syncthreads();
    if (n > 0) dequant(unit(0), 0, 0);
    DKV_TL(tl_mfma, 2);
    if (n > 1) stage(1, r);
    if (!early2 && n > 2) load(2, r);
    for (int i = 0; i < n; ++i) {
      __syncthreads();
      if (i + 1 < n) dequant(unit(i + 1), (i + 1) & 1, (i + 1) & 1);
      if (i + 2 < n) {
        if (early2 && i == 0)
          stage(0, r2);
        else
          stage(i & 1, r);
        if (i + 3 < n) load(i + 3, r);
      }
      compute(unit(i), i & 1, i == 0);
      if (i == 0) DKV_TL(tl_mfma, 3);
    }
  }
  DKV_TL(tl_mfma, 4);

  // Merge the two key groups. Block nb of a wave is finalized by key group
  // owner(nb) (with two blocks per wave each group finalizes one, so both
  // groups fold and store at once); the other group parks its (max, sum, O)
  // for that block in LDS (over the staging buffers, once every wave is past
  // its last unit). Lane (g, col) of block nb holds O^T rows d = 16 db + 4 g + i
  // of local row (w + KGW nb) * 16 + col.
  auto owner = [](int nb) { return NBW == 2 ? nb : 0; };
  float lsum[NBW];
#pragma unroll
  for (int nb = 0; nb < NBW; ++nb) {
    lsum[nb] = group_sum(l_part[nb]);
  }
  float* mrg_o = reinterpret_cast<float*>(smem);
  float2* mrg_ml = reinterpret_cast<float2*>(smem + MROWS * MRG_STRIDE * 4);
  __syncthreads();
  if (wave_on) {
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
      if (owner(nb) == kg) continue;  // this group finalizes the block; the other parks it
      const int lr = (w + KGW * nb) * 16 + col;
#pragma unroll
      for (int db = 0; db < 4; ++db)
        *reinterpret_cast<f32x4*>(mrg_o + lr * MRG_STRIDE + 16 * db + 4 * g) = acc_o[nb][db];
      if (g == 0) mrg_ml[lr] = make_float2(m_run[nb], lsum[nb]);
    }
  }
  __syncthreads();
  DKV_TL(tl_mfma, 5);
  if (wave_on) {
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
      if (owner(nb) != kg) continue;
      const int lr = (w + KGW * nb) * 16 + col;
      const float2 o1 = mrg_ml[lr];
      const float mm = fmaxf(m_run[nb], o1.x);
      const float f0 = mm == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[nb] - mm);
      const float f1 = mm == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(o1.x - mm);
      float l = lsum[nb] * f0 + o1.y * f1;
      const int r = r0 + lr;
      f32x4 o[4];
#pragma unroll
      for (int db = 0; db < 4; ++db)
        o[db] = acc_o[nb][db] * f0 + *reinterpret_cast<const f32x4*>(mrg_o + lr * MRG_STRIDE + 16 * db + 4 * g) * f1;
      if (r >= r_end) continue;
      if (active == 1) {  // the splits that run (see attn_vec_kernel's epilogue)
        const int gq = r / a.nq, m = r - gq * a.nq;
        const float inv = 1.f / l;
        const int64_t off = (int64_t)m * a.out_tok_stride + (int64_t)(h * G + gq) * a.out_head_stride + 4 * g;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const f32x4 v = o[db] * inv;
          if (a.out_dtype == 1)
            *reinterpret_cast<float4*>(static_cast<float*>(a.out) + off + 16 * db) = make_float4(v[0], v[1], v[2], v[3]);
          else
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + off + 16 * db) =
                make_uint2(pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3]));
        }
      } else {
        const int64_t base = ((int64_t)h * splits + split) * R + r;
        if (PREC) {
#pragma unroll
          for (int db = 0; db < 4; ++db)
            part_store<NBW == 1>(o[db], reinterpret_cast<f32x4*>(part_o + base * D + 16 * db + 4 * g));
        } else {  // O / l in fp16, row order of half_slot(): chunks g and 4 + g of the row
          const float inv = l > 0.f ? 1.f / l : 0.f;
          _Float16* ph = reinterpret_cast<_Float16*>(part_o) + base * D + 8 * g;
          const f32x4 a0 = o[0] * inv, a1 = o[1] * inv, a2 = o[2] * inv, a3 = o[3] * inv;
          auto store_row = [&](const f32x4& b0, const f32x4& b1, const f32x4& b2, const f32x4& b3) {
            part_store<NBW == 1>(__builtin_convertvector(
                (f32x8{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]}), f16x8), reinterpret_cast<f16x8*>(ph));
            part_store<NBW == 1>(__builtin_convertvector(
                (f32x8{b2[0], b2[1], b2[2], b2[3], b3[0], b3[1], b3[2], b3[3]}), f16x8),
                reinterpret_cast<f16x8*>(ph + 32));
          };
          store_row(a0, a1, a2, a3);
          float amax = 0.f;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(a0[e]), fabsf(a1[e])), fmaxf(fabsf(a2[e]), fabsf(a3[e]))));
          // Rare (|V| near the fp16 range, where the stores above hold inf): the
          // row's maximum over its 4 lane groups (lanes col + 16 g, all active
          // since they share r) picks the exponent, and the lane stores the row
          // again, scaled (the later store to the same address wins).
          if (__builtin_amdgcn_ballot_w64(amax >= 32768.f)) {
            const int ex = half_partial_exponent(group_max(amax));
            if (ex) {
              const float sc = __builtin_amdgcn_ldexpf(1.f, -ex);
              store_row(a0 * sc, a1 * sc, a2 * sc, a3 * sc);
              l = half_partial_sum(l, ex);
            }
          }
        }
        if (g == 0) part_store<NBW == 1>((f32x2{mm, l}), reinterpret_cast<f32x2*>(part_ml + base));
      }
    }
  }
  DKV_TL(tl_mfma, 6);
#if DKV_INKERNEL_MERGE
  if constexpr (PREC == 0) {
    if (!fused || active <= 1) return;
    __shared__ int merge_here;
    __builtin_amdgcn_s_waitcnt(0);  // every wave's partial stores have completed
    __syncthreads();
    if (t == 0) {  // the release writes the XCD's L2 back, so all of the workgroup's partials
      uint32_t* ctr = counters + h * gridDim.z + rg;
      const uint32_t ticket = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      merge_here = ticket == (uint32_t)(active - 1);
      if (merge_here) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next launch
    }
    __syncthreads();
    DKV_TL(tl_mfma, 8);
    if (!merge_here) return;
    if (wave == 0) {  // acquire for the workgroup: invalidate the CU's L1 and the XCD's L2, and wait
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
#pragma unroll 1
    for (int r = r0 + wave; r < r_end; r += 2 * KGW)
      merge_row_half<NBW == 1>(a, h, r, R, G, splits, active, part_o, part_ml);
    DKV_TL(tl_mfma, 9);
  }
#endif
}

#if DKV_INKERNEL_MERGE
#define DKV_MERGE_ARGS , p.fused, counters
#else
#define DKV_MERGE_ARGS
#endif

template <int PREC>
static void launch_prec(const dkv_attn_args& a, const Plan& p, float* part_o, float2* part_ml, uint32_t* counters,
                        hipStream_t s) {
  const dim3 grid(p.splits, a.heads, p.row_groups);
  const int nbw = mfma_blocks_per_wave(p.rows_per_group);
  ArgTiles at;
  const NoArgTiles none = {0};
  const int rpg = p.rows_per_group;
  const bool argt = fill_arg_tiles(a, at);
  if constexpr (PREC == 0) {
    if (p.small) {  // decode steps: 4-wave workgroups, four per CU
      if (argt)
        hipLaunchKernelGGL((attn_mfma_kernel<PREC, 1, true, true>), grid, dim3(256), 0, s, at, a, p.units, p.splits,
                           p.cap, rpg, part_o, part_ml DKV_MERGE_ARGS);
      else
        hipLaunchKernelGGL((attn_mfma_kernel<PREC, 1, false, true>), grid, dim3(256), 0, s, none, a, p.units,
                           p.splits, p.cap, rpg, part_o, part_ml DKV_MERGE_ARGS);
      return;
    }
  }
  if (argt) {
    if (nbw >= 2)
      hipLaunchKernelGGL((attn_mfma_kernel<PREC, 2, true, false>), grid, dim3(MF_THREADS), 0, s, at, a, p.units,
                         p.splits, p.cap, rpg, part_o, part_ml DKV_MERGE_ARGS);
    else
      hipLaunchKernelGGL((attn_mfma_kernel<PREC, 1, true, false>), grid, dim3(MF_THREADS), 0, s, at, a, p.units,
                         p.splits, p.cap, rpg, part_o, part_ml DKV_MERGE_ARGS);
  } else if (nbw >= 2) {
    hipLaunchKernelGGL((attn_mfma_kernel<PREC, 2, false, false>), grid, dim3(MF_THREADS), 0, s, none, a, p.units,
                       p.splits, p.cap, rpg, part_o, part_ml DKV_MERGE_ARGS);
  } else {
    hipLaunchKernelGGL((attn_mfma_kernel<PREC, 1, false, false>), grid, dim3(MF_THREADS), 0, s, none, a, p.units,
                       p.splits, p.cap, rpg, part_o, part_ml DKV_MERGE_ARGS);
  }
}

int launch_attn_mfma(const dkv_attn_args& a, const Plan& p, float* part_o, float2* part_ml, uint32_t* counters,
                     hipStream_t s) {
  if (p.precision == 1) launch_prec<1>(a, p, part_o, part_ml, counters, s);
  else launch_prec<0>(a, p, part_o, part_ml, counters, s);
  return (int)hipGetLastError();
}

}  // namespace dkv

#ifdef DKV_TIMELINE
// Timeline build only: copies the frame-chunk kernel's stamps of the last launch and clears them.
extern "C" int dkv_timeline_mfma(void* host, int64_t bytes) { return dkv::timeline_take(dkv::tl_mfma, host, bytes); }
#endif
