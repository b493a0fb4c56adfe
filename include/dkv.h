/*
 * dkv.h - C ABI of the MI355X packed mixed-precision KV-cache library (libdkv.so).
 *
 * Plain pointers, sizes and a hipStream_t passed as void*. No torch types cross
 * this boundary. Every entry point returns 0 on success, DKV_EINVAL for a
 * contract violation (the message is available from dkv_last_error()) or a
 * positive hipError_t value for a runtime failure. No entry point synchronizes
 * the stream it is given.
 *
 * Storage format (shared by every entry point):
 *   - A cache owns one byte arena. A segment is one append at one bit width
 *     (4, 8 or 16). It is cut into tiles of up to 64 tokens.
 *   - Tile i of a segment starts at seg_offset + i * dkv_slab_bytes(64, bits).
 *     Inside a tile, the sub-block of (layer, kv, head), with kv 0 = K and 1 = V,
 *     starts at ((layer*2 + kv)*heads + head) * dkv_subblock_bytes(rows, bits).
 *   - A sub-block holds `rows` payload rows of 64 elements, then (for 4/8 bit)
 *     `rows` pairs of fp32 (offset a, scale s). 4-bit rows are 32 bytes, with the
 *     low nibble holding the even element. 8-bit rows are 64 bytes. 16-bit rows
 *     are the 128 input bytes unchanged. This is the byte format of the
 *     reference's quantizer and GPU pools (src/kv_quantization.py:57-73,
 *     src/gpu_kernels.py:24-46).
 */
#ifndef DKV_H
#define DKV_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DKV_ABI_VERSION 3
#define DKV_HEAD_DIM 64
#define DKV_TILE_TOKENS 64
#define DKV_MAX_CHUNK_SEGS 16
#define DKV_ARG_TILES 128 /* most tile descriptors a launch carries in its argument block */
#define DKV_EINVAL (-1)

/* One 64-token tile of the arena. The cache keeps these in token order in a
 * device array; the pack entry points write them, the attention and
 * reconstruct entry points read them. */
typedef struct dkv_tile {
  int64_t offset;      /* byte offset of the tile in the arena */
  int32_t token_start; /* logical index of the tile's first token */
  uint16_t rows;       /* rows the tile holds (1..64) */
  uint8_t bits;        /* 4, 8 or 16 */
  uint8_t reserved;
} dkv_tile;

/* One append of n tokens of one layer into a segment. k and v are bf16 views
 * [heads, n, 64] with element strides per head and per token and a contiguous
 * last dimension (V may be a transposed view, as in the reference tests). */
typedef struct dkv_pack_job {
  const void* k;
  const void* v;
  int64_t k_head_stride, k_tok_stride;
  int64_t v_head_stride, v_tok_stride;
  int64_t seg_offset;      /* byte offset of the segment in the arena */
  int32_t seg_rows;        /* tokens the segment can hold */
  int32_t seg_token_start; /* logical index of the segment's first token */
  int32_t row0;            /* first segment row written by this job */
  int32_t n;               /* tokens appended by this job */
  int32_t layer;
  int32_t bits;            /* 4, 8 or 16 */
  int32_t tile_index0;     /* table index of the segment's first tile */
  int32_t write_tiles;     /* nonzero: also write the segment's tile descriptors */
} dkv_pack_job;

/* Causal attention of a query chunk over the packed history plus the chunk's
 * own native K/V. Query row m of chunk segment c sees every history token
 * (token < past) and chunk tokens j with seg_bounds[c] <= j <= m. One segment
 * covering [0, nq) is the ordinary bottom-right causal mask. */
typedef struct dkv_attn_args {
  const void* q;     /* bf16 [q_heads, nq, 64] */
  int64_t q_head_stride, q_tok_stride;
  const void* k_new; /* bf16 [heads, nq, 64] */
  int64_t kn_head_stride, kn_tok_stride;
  const void* v_new; /* bf16 [heads, nq, 64] */
  int64_t vn_head_stride, vn_tok_stride;
  const void* arena;
  const dkv_tile* tiles; /* device array; tiles with token_start < past are read */
  int32_t n_tiles;       /* number of tiles covering [0, past) */
  int32_t past;          /* history tokens */
  int32_t layer, layers, heads, q_heads, nq;
  int32_t n_segs;        /* 0 or 1: one causal segment */
  int32_t seg_bounds[DKV_MAX_CHUNK_SEGS + 1];
  float scale;           /* softmax scale, 1/8 for head_dim 64 */
  void* out;             /* [nq, q_heads, 64] with the strides below */
  int64_t out_tok_stride, out_head_stride;
  int32_t out_dtype;     /* 0 = bf16, 1 = fp32 */
  int32_t path;          /* 0 = auto (the MFMA frame-chunk kernel, the fastest measured for every
                            chunk length, decode steps included),
                            1 = vector, 2 = MFMA (frame chunks), 3 = short chunk (decode steps) */
  int32_t splits;        /* 0 = auto; history split count per KV head */
  int32_t precision;     /* 0 = the reference kernel's bf16 rounding of K, V and p
                            (src/gpu_kernels.py:93-94,102); 1 = fp32-accurate */
  void* workspace;       /* device scratch of dkv_attend_workspace_bytes() (0 for one split): the
                            split partials; a workspace serves one call at a time */
  int64_t workspace_bytes;
  const int32_t* step;   /* NULL, or a DEVICE pair {past, n_tiles} read when the kernels run,
                            for launches recorded once in a HIP graph and replayed as the
                            history grows. `past` and `n_tiles` above then bound the launch
                            (grid, workspace) and the device pair must stay within them. */
  const dkv_tile* tiles_host; /* NULL, or a HOST copy of tiles[0, n_tiles), equal to the device
                            table. For a launch without `step` and n_tiles <= DKV_ARG_TILES the
                            frame-chunk kernel then takes the descriptors from its argument block
                            (read beside the arguments) instead of waiting on the device table
                            before its first history loads; otherwise it is ignored. A copy whose
                            tiles are not well formed or do not cover [0, past) in token order is
                            refused (DKV_EINVAL). The descriptors are copied into the launch when
                            dkv_attend is called, so a launch captured in a HIP graph keeps the
                            ones it was captured with: its replays read the tiles as they were then
                            (offsets, widths, rows), not the device table. Capture launches that
                            must follow a table that changes (a cache reset, appends at other
                            widths) with `step`, or with tiles_host = NULL. */
} dkv_attn_args;

/* One segment of the arena in the reference's CPU-cache layout: what
 * src/kv_quantization.py:41-77 (pack) produces for the [1, heads, rows, 64]
 * K or V tensor of one layer. For layer l = layer0 + i (i < n_layers) and
 * kv 0 = K, 1 = V:
 *   payload[kv] + ((i*heads + h)*rows + r)*row_bytes   row r of head h
 *       (row_bytes 32 / 64 / 128 for 4 / 8 / 16 bits: the PackedTensor payload)
 *   offsets[kv][(i*heads + h)*rows + r], scales[kv][...]   fp32 (4/8-bit only;
 *       the PackedTensor offsets and scales, one group per row)
 * Segment rows [row0, row0 + rows) move, as buffer rows [0, rows); the arena
 * geometry comes from seg_rows. The segment descriptor of src/cache_manager.py:9
 * ('<iiqqB7x': layer, frame, start, end, bits) stays on the host. */
typedef struct dkv_segment_io {
  void* payload[2];
  float* offsets[2];       /* NULL for 16-bit */
  float* scales[2];        /* NULL for 16-bit */
  int64_t seg_offset;      /* byte offset of the segment in the arena */
  int32_t seg_rows;        /* tokens the segment can hold */
  int32_t seg_token_start; /* logical index of the segment's first token */
  int32_t row0;            /* first segment row moved */
  int32_t rows;            /* rows moved */
  int32_t bits;            /* 4, 8 or 16 */
  int32_t layer0, n_layers;
  int32_t tile_index0;     /* import: table index of the segment's first tile */
  int32_t write_tiles;     /* import: nonzero also writes the segment's tile descriptors */
} dkv_segment_io;

/* Library version: DKV_ABI_VERSION. */
int dkv_version(void);

/* Message of the last DKV_EINVAL on the calling thread ("" if none). */
const char* dkv_last_error(void);

/* Bytes of one (layer, kv, head) sub-block of a tile of `rows` rows. */
int64_t dkv_subblock_bytes(int32_t rows, int32_t bits);

/* Bytes of a whole tile of `rows` rows: layers * 2 * heads sub-blocks. */
int64_t dkv_slab_bytes(int32_t rows, int32_t bits, int32_t layers, int32_t heads);

/* Pack one append into the arena. Replaces the reference's per-layer
 * pack_rows launch (src/gpu_cache.py:89-92, src/gpu_kernels.py:11-46). The
 * bytes, offsets and scales equal src/kv_quantization.py:41-77 bit for bit. */
int dkv_pack(const dkv_pack_job* job, void* arena, int64_t arena_bytes,
             dkv_tile* tiles, int32_t layers, int32_t heads, void* stream);

/* Pack n_jobs appends in one launch. `jobs` is a DEVICE array that the kernel
 * trusts: validate its host copy with dkv_pack_validate first. max_n bounds
 * every job's n. There is no reference counterpart for batching: it is the
 * whole-volume form of dkv_pack used when many (layer, frame) tiles are ready
 * at once, e.g. a prefill of several frames. */
int dkv_pack_batch(const dkv_pack_job* jobs, int32_t n_jobs, int32_t max_n,
                   void* arena, int64_t arena_bytes, dkv_tile* tiles,
                   int32_t layers, int32_t heads, void* stream);

/* Checks a HOST copy of a job table against the arena (what dkv_pack checks for
 * one job), so that a table can be validated before it is copied to the device
 * and launched with dkv_pack_batch. No reference counterpart (see dkv_pack_batch). */
int dkv_pack_validate(const dkv_pack_job* jobs, int32_t n_jobs, int64_t arena_bytes,
                      int32_t layers, int32_t heads);

/* Dequantize tokens [0, n_tokens) of one layer into out[2, heads, n_tokens, 64]
 * (bf16 or fp32 by out_dtype), as q*s + a in fp32 (src/kv_quantization.py:90-92).
 * Replaces GPUCache.materialize's reconstruct launch (src/gpu_cache.py:106-112,
 * src/gpu_kernels.py:107-119). */
int dkv_reconstruct(const void* arena, const dkv_tile* tiles, int32_t n_tiles,
                    int32_t n_tokens, int32_t layer, int32_t layers, int32_t heads,
                    void* out, int32_t out_dtype, void* stream);

/* Workspace bytes dkv_attend needs for these arguments. */
int64_t dkv_attend_workspace_bytes(const dkv_attn_args* args);

/* Fused packed-history causal GQA attention. Replaces GPUCache.attend's
 * packed_attention launch (src/gpu_cache.py:96-104, src/gpu_kernels.py:71-105).
 * Every chunk length runs a split-history MFMA kernel by default (path 0/2);
 * path 3 runs short chunks (at most 16 query rows per KV head, e.g. decode
 * steps) on a kernel with two waves per 64-key tile. A merge kernel combines
 * the history splits of either in a second launch.
 * Output rows are written to out + m*out_tok_stride + qh*out_head_stride
 * (elements), the reference's [1, nq, q_heads, 64] layout when contiguous.
 * Q, K and V must be 16-byte aligned with strides in multiples of 8 elements;
 * out 16-byte aligned with strides in multiples of 4 elements. */
int dkv_attend(const dkv_attn_args* args, void* stream);

/* dkv_attend without a workspace and without allocating: no counterpart in the
 * reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * split partials go to a scratch buffer of DKV_NOALLOC_SCRATCH_BYTES that the
 * library's code object holds on each device (resident until the process ends);
 * args->workspace and args->workspace_bytes are ignored. Results equal
 * dkv_attend's for the same arguments. A call whose partials need more than
 * DKV_NOALLOC_SCRATCH_BYTES (dkv_attend_workspace_bytes) returns DKV_EINVAL
 * without launching; the metric's shapes need at most 13 MB. The first call on
 * a device looks the buffer's address up (hipGetSymbolAddress): make that call
 * before capturing a graph. Calls share their device's buffer, so two calls on
 * one device that may overlap in time (different streams) race; serialize them
 * (one stream) or use dkv_attend with separate workspaces. */
#define DKV_NOALLOC_SCRATCH_BYTES (16 << 20)
int dkv_attend_noalloc(const dkv_attn_args* args, void* stream);

/* Copy one segment out of the arena into the reference's PackedTensor buffers
 * (src/kv_quantization.py:12-77). Together with the host-side 64-byte header
 * and the 32-byte segment descriptor (src/cache_manager.py:9,53-58), this
 * yields the segments src/cache_manager.py's MixedPrecisionCache.update
 * stores, byte for byte. A plain byte move: nothing is requantized. */
int dkv_export(const dkv_segment_io* io, const void* arena, int64_t arena_bytes,
               int32_t layers, int32_t heads, void* stream);

/* The inverse of dkv_export: writes PackedTensor payloads, offsets and scales
 * into a segment of the arena (and its tile descriptors when write_tiles), so
 * that segments packed elsewhere by src/kv_quantization.py:pack can be attended
 * without being requantized. */
int dkv_import(const dkv_segment_io* io, void* arena, int64_t arena_bytes, dkv_tile* tiles,
               int32_t layers, int32_t heads, void* stream);

/* Batched dkv_export / dkv_import over a DEVICE array of n_ios segments, one
 * launch (validate the host copy with dkv_segment_validate first). max_rows
 * bounds every segment's seg_rows and max_layers its n_layers. direction 0
 * exports, 1 imports. No reference counterpart: the whole-cache form of the
 * two calls above. */
int dkv_segment_batch(const dkv_segment_io* ios, int32_t n_ios, int32_t max_rows, int32_t max_layers,
                      int32_t direction, void* arena, int64_t arena_bytes, dkv_tile* tiles,
                      int32_t layers, int32_t heads, void* stream);

/* Checks a HOST copy of a dkv_segment_io table (what dkv_export and dkv_import
 * check for one segment). No reference counterpart (see dkv_segment_batch). */
int dkv_segment_validate(const dkv_segment_io* ios, int32_t n_ios, int32_t direction,
                         int64_t arena_bytes, int32_t layers, int32_t heads);

/* Decoder pointwise ops around the path (bf16 in and out, fp32 arithmetic,
 * 16-byte aligned buffers, row strides in elements and multiples of 8).
 *
 * dkv_rope_qkv: the joined Q/K/V projection [n, (q_heads + 2 kv_heads) * 64]
 * -> q_out [q_heads, n, 64], k_out and v_out [kv_heads, n, 64], with RoPE
 * applied to q and k exactly as transformers' apply_rotary_pos_emb computes it
 * in bf16 (q*cos + rotate_half(q)*sin, each product and the sum rounded), from
 * cos/sin rows [n, 64]. Replaces the split / view / apply_rotary_pos_emb steps
 * of the reference's patched attention forward (src/gpu_cache.py:166-172). */
int dkv_rope_qkv(const void* qkv, int64_t qkv_row_stride, const void* cos, const void* sin,
                 int64_t cs_row_stride, int32_t n, int32_t q_heads, int32_t kv_heads,
                 void* q_out, void* k_out, void* v_out, void* stream);

/* dkv_rope_qkv and dkv_pack in one launch: the projection split, RoPE and the
 * cache append of the reference's patched attention forward
 * (src/gpu_cache.py:164-172, the append at src/gpu_cache.py:68-94). Writes
 * q_out/k_out/v_out as dkv_rope_qkv does (kv_heads = heads) and packs k_out's
 * and v_out's rows into the job's segment, byte for byte what dkv_pack of the
 * same job over those outputs writes. The job's k/v pointers and strides are
 * not read: the projection is the source. job_on_device = 0: `job` is a host
 * struct, checked as dkv_pack checks it, and job->n must equal n.
 * job_on_device = 1: `job` is a DEVICE struct read when the kernel runs (HIP
 * graph replays; validate its host copy with dkv_pack_validate), n >= 1, and
 * the kernel packs min(job->n, n) rows. */
int dkv_rope_pack(const void* qkv, int64_t qkv_row_stride, const void* cos, const void* sin,
                  int64_t cs_row_stride, int32_t n, int32_t q_heads, void* q_out, void* k_out,
                  void* v_out, const dkv_pack_job* job, int32_t job_on_device, void* arena,
                  int64_t arena_bytes, dkv_tile* tiles, int32_t layers, int32_t heads, void* stream);

/* out = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * weight) per row of `dim`
 * elements: the reference's cuda_rms (src/gpu_ops.py:9-12) in one launch. */
int dkv_rms_norm(const void* x, int64_t x_row_stride, const void* weight, void* out,
                 int64_t out_row_stride, int32_t rows, int32_t dim, float eps, void* stream);

/* out[:, :inter] = bf16(bf16(silu(g)) * u) for rows [g | u] of 2 * inter
 * elements: the reference's activation_product over the joined gate/up
 * projection (src/gpu_ops.py:14-17, 23-25) in one launch. */
int dkv_silu_mul(const void* gate_up, int64_t row_stride, void* out, int64_t out_row_stride,
                 int32_t rows, int32_t inter, void* stream);

/* Decoder projections of short chunks (1-100 rows) on MFMA:
 *   out[rows, n_out] = epilogue(prologue(x) . w^T)
 * x [rows, k] and w [n, k] bf16 with contiguous rows (k a multiple of 64),
 * fp32 accumulation, bf16 out. These replace the library GEMMs and the
 * PyTorch ops around them in the decoder layer that calls the packed cache
 * (src/gpu_ops.py:19-48 joins the projections; src/gpu_cache.py:164-165, 183
 * and transformers' LlamaDecoderLayer run them):
 *   norm_weight != NULL: x rows pass through RMSNorm first, rounded as
 *     bf16(bf16(x * rsqrt(mean(x^2) + eps)) * norm_weight) (src/gpu_ops.py:9-12);
 *   DKV_LINEAR_PLAIN     out = bf16(acc), n_out = n;
 *   DKV_LINEAR_RESIDUAL  out = bf16(residual + bf16(acc)), residual [rows, n];
 *   DKV_LINEAR_SILU_MUL  w = [gate | up] (n = 2 n_out rows):
 *     out[:, c] = bf16(bf16(silu(bf16(gate_c))) * bf16(up_c)) (src/gpu_ops.py:14-17).
 * dkv_linear_supported says whether a shape has a launch (1) or not (0); an
 * unsupported call returns DKV_EINVAL without touching the device. */
#define DKV_LINEAR_PLAIN 0
#define DKV_LINEAR_RESIDUAL 1
#define DKV_LINEAR_SILU_MUL 2
int dkv_linear_supported(int32_t rows, int32_t n, int32_t k, int32_t has_norm, int32_t epilogue);
int dkv_linear(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
               int32_t rows, int32_t n, int32_t k, const void* norm_weight, float eps,
               int32_t epilogue, const void* residual, int64_t residual_row_stride,
               void* out, int64_t out_row_stride, void* stream);

/* dkv_linear with operands in the MFMA-tiled layout, which has no counterpart
 * in the reference (its projections are library GEMMs over row-major weights):
 * a layout for callers that keep a second copy of each weight (and of the
 * SiLU*up intermediate) so that every load instruction of the kernel reads
 * 1 KB of consecutive bytes. Element (r, c) of a tiled [R, K] matrix (R a
 * multiple of 16, rows past `rows` being padding) sits at
 *   ((r / 16) * (K / 64) + c / 64) * 1024 + (c / 32 % 2) * 512
 *     + ((c / 8 % 4) * 16 + r % 16) * 8 + c % 8.
 * layout bits: DKV_LINEAR_W_TILED (w, K = k), DKV_LINEAR_X_TILED (x, K = k,
 * rows rounded up to 16), DKV_LINEAR_OUT_TILED (out, K = n_out, a multiple of
 * 64; its padding rows are not written), DKV_LINEAR_RES_TILED (the residual of
 * DKV_LINEAR_RESIDUAL, K = n_out, a multiple of 64, rows rounded up to 16).
 * The row stride of a tiled operand is ignored. The results are bit-identical
 * to dkv_linear's; layout 0 is dkv_linear. */
#define DKV_LINEAR_W_TILED 1
#define DKV_LINEAR_X_TILED 2
#define DKV_LINEAR_OUT_TILED 4
#define DKV_LINEAR_RES_TILED 8
int dkv_linear_tiled(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
                     int32_t rows, int32_t n, int32_t k, const void* norm_weight, float eps,
                     int32_t epilogue, const void* residual, int64_t residual_row_stride,
                     void* out, int64_t out_row_stride, int32_t layout, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* DKV_H */
