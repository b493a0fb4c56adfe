"""Packed mixed-precision KV cache on one preallocated HBM arena.

Drop-in for the reference's GPUCache / install_packed_attention
(src/gpu_cache.py:10-183): same constructor, methods, return values, errors and
de-facto public attributes (seen, host_counts, backend, caps, codes, rows,
plan). The storage underneath is different: instead of three per-precision
pools with a per-token row map, every append at layer 0 opens a segment of
64-token tiles in one byte arena, and a device tile table records each tile's
offset, first token, rows and bit width. Pack, attention and reconstruct are
hand-written HIP kernels reached through libdkv's C ABI (include/dkv.h).
"""
import bisect
import ctypes
import types

import numpy as np
import torch
import torch.nn.functional as F

from . import _lib, formats

try:  # the reference subclasses transformers' DynamicCache; keep isinstance() working
    from transformers.cache_utils import DynamicCache as _CacheBase
except Exception:  # transformers absent: a plain object base keeps the kernels usable
    _CacheBase = object

TILE = 64
BITS = (4, 8, 16)
# 'bf16': dequantized K/V and p rounded to bf16 before the dot products, as the reference kernel
# does (src/gpu_kernels.py:93-94,102). 'fp32': fp32-accurate (split bf16 pairs on the MFMA path).
PRECISIONS = {'bf16': 0, 'fp32': 1}
PATHS = {'auto': 0, 'vector': 1, 'mfma': 2, 'short': 3}
SHORT_ROWS = 16  # query rows per KV head the short-chunk kernel takes (SHORT_ROWS of csrc/dkv_attn_common.h)


# The kernels store bf16 or fp32 (dkv_attn_args.out_dtype, dkv_reconstruct's out_dtype); any other
# dtype would receive bf16 bit patterns.
OUT_DTYPES = (torch.bfloat16, torch.float32)


def _check_dtype(dtype, what):
    if dtype not in OUT_DTYPES:
        raise ValueError(f'{what} must be torch.bfloat16 or torch.float32, got {dtype}')


def row_bytes(bits):
    return {4: 32, 8: 64, 16: 128}[bits]


def subblock_bytes(rows, bits):
    """Python mirror of dkv_subblock_bytes (include/dkv.h)."""
    b = rows * row_bytes(bits) + (rows * 8 if bits < 16 else 0)
    return (b + 15) & ~15


def slab_bytes(rows, bits, layers, heads):
    return subblock_bytes(rows, bits) * layers * 2 * heads


def segment_bytes(rows, bits, layers, heads):
    """Arena bytes of a segment of `rows` tokens: full tiles plus one partial."""
    full, rem = divmod(rows, TILE)
    return full * slab_bytes(TILE, bits, layers, heads) + (slab_bytes(rem, bits, layers, heads) if rem else 0)


# dkv_tile (include/dkv.h): 16 bytes per 64-token tile.
TILE_DTYPE = np.dtype([('offset', '<i8'), ('token_start', '<i4'), ('rows', '<u2'), ('bits', 'u1'),
                       ('reserved', 'u1')])
assert TILE_DTYPE.itemsize == 16


def worst_case_arena_bytes(tokens, layers, heads):
    """Bytes that hold `tokens` tokens at any mix of widths and segment cuts."""
    # 16-bit rows are the largest (128 B); each partial tile rounds up by < 16 B.
    return layers * 2 * heads * (tokens * row_bytes(16) + 16 * tokens)


class _Segment:
    __slots__ = ('start', 'rows', 'bits', 'offset', 'tile0', 'frame')

    def __init__(self, start, rows, bits, offset, tile0, frame=-1):
        self.start, self.rows, self.bits, self.offset, self.tile0 = start, rows, bits, offset, tile0
        self.frame = frame  # frame id of the select() that opened it (the segment descriptor's frame)

    @property
    def end(self):
        return self.start + self.rows

    @property
    def ntiles(self):
        return (self.rows + TILE - 1) // TILE


class GPUCache(_CacheBase):
    """Mixed 4/8/16-bit KV cache for batch one and head_dim 64 (src/gpu_cache.py:10-149)."""

    def __init__(self, plan=None, layers=30, heads=3, dim=64, device='cuda', dtype=torch.bfloat16,
                 backend='fused', block_m=16, block_n=64, max_tokens=8192, arena_bytes=None, precision='bf16'):
        if _CacheBase is not object:
            super().__init__()
        if dim != 64:
            raise ValueError('GPU kernel currently supports head_dim=64')
        if precision not in PRECISIONS:
            raise ValueError(f'precision must be one of {sorted(PRECISIONS)}')
        _check_dtype(dtype, 'dtype')
        self.precision = precision
        self.layers, self.heads, self.dim = layers, heads, dim
        self.dtype, self.device = dtype, torch.device(device)
        self.backend, self.block_m, self.block_n = backend, block_m, block_n
        self.seen = [0] * layers
        self.cursors = [0] * layers
        self.pending_bits = 16
        self.frame_id = -1
        self.chunk_segments = None  # default `segments` of attend() (batched continuations)
        # default `splits` of attend() for chunks of more than SHORT_ROWS query rows per KV head
        # (0: the library's plan, the shortest latency of a launch that has the GPU to itself)
        self.chunk_splits = 0
        self.online = plan is None
        self.plan = []  # (start, end, bits, row) per segment, as in the reference
        self.segments = []
        self.tile_starts = []  # first token of every tile, in token order
        self.host_counts = {4: 0, 8: 0, 16: 0}
        self.arena_used = 0
        planned = []
        for bits, n in (plan or []):
            if bits not in self.host_counts or n < 0:
                raise ValueError('Invalid GPU cache plan')
            planned.append((bits, n))
        if self.online:
            self.capacity = max_tokens
            need = worst_case_arena_bytes(max_tokens, layers, heads)
            max_tiles = max_tokens
        else:
            self.capacity = sum(n for _, n in planned)
            need = sum(segment_bytes(n, b, layers, heads) for b, n in planned if n)
            max_tiles = sum((n + TILE - 1) // TILE for _, n in planned)
        self.arena_bytes = int(arena_bytes) if arena_bytes is not None else max(need, 256)
        self.arena = torch.empty(self.arena_bytes, dtype=torch.uint8, device=self.device)
        self.tiles = torch.zeros((max(max_tiles, 1), 16), dtype=torch.uint8, device=self.device)
        # Host copy of the tile table, entry for entry what the pack launches write to the device
        # table (write_tile_descriptors): attention calls pass it in the launch's argument block.
        # Shared by forks, as the device table is.
        self.tiles_host = np.zeros(self.tiles.shape[0], dtype=TILE_DTYPE)
        self._tiles_host_ptr = self.tiles_host.ctypes.data  # fixed: the array is never replaced
        self._workspace = None
        self._graph = None  # GraphSteps while launches read their step parameters from the device
        self._fused_args, self._fused_key = None, None  # the argument block _fused_attention() reuses
        for bits, n in planned:
            if n:
                self._open_segment(self.segments[-1].end if self.segments else 0, n, bits)

    # -- bookkeeping -------------------------------------------------------
    def _open_segment(self, start, n, bits, frame=-1, grow=True):
        need = segment_bytes(n, bits, self.layers, self.heads)
        if self.arena_used + need > self.arena_bytes:
            if not grow:
                # a captured graph recorded the arena's address: a new arena would leave its
                # launches writing freed memory
                raise ValueError(f'graph steps cannot grow the arena: a {n}-token {bits}-bit segment needs '
                                 f'{self.arena_used + need} bytes, the arena holds {self.arena_bytes}')
            self._grow(self.arena_used + need)
        tile0 = len(self.tile_starts)
        if tile0 + (n + TILE - 1) // TILE > self.tiles.shape[0]:
            raise ValueError('GPU context limit exceeded')
        seg = _Segment(start, n, bits, self.arena_used, tile0, frame)
        self.segments.append(seg)
        self.tile_starts.extend(range(start, start + n, TILE))
        t = np.arange((n + TILE - 1) // TILE)
        entries = self.tiles_host[tile0:tile0 + len(t)]
        entries['offset'] = self.arena_used + t * slab_bytes(TILE, bits, self.layers, self.heads)
        entries['token_start'] = start + t * TILE
        entries['rows'] = np.minimum(n - t * TILE, TILE)
        entries['bits'] = bits
        entries['reserved'] = 0
        self.plan.append((start, start + n, bits, self.host_counts[bits]))
        self.host_counts[bits] += n
        self.arena_used += need
        return seg

    def _grow(self, needed):
        """Grows this cache's arena (forks keep theirs), like the reference's reserve()."""
        size = max(needed, ((int(self.arena_bytes * 1.5) + 255) // 256) * 256)
        target = torch.empty(size, dtype=torch.uint8, device=self.device)
        if self.arena_used:
            target[:self.arena_used].copy_(self.arena[:self.arena_used])
        self.arena, self.arena_bytes = target, size

    def reserve(self, bits, needed):
        """Makes room for `needed` rows of width `bits` in total (src/gpu_cache.py:44-59)."""
        more = needed - self.host_counts[bits]
        if more <= 0:
            return
        extra = segment_bytes(more, bits, self.layers, self.heads) + 16 * self.layers * 2 * self.heads
        if self.arena_used + extra > self.arena_bytes:
            self._grow(self.arena_used + extra)

    @property
    def caps(self):
        """Rows of each width the arena could hold (the reference's pool capacities)."""
        per = self.layers * 2 * self.heads
        return {b: self.arena_bytes // (per * (row_bytes(b) + (8 if b < 16 else 0))) for b in BITS}

    @property
    def codes(self):
        """Per-token bit width, uint8 on the device (the reference's precision map)."""
        out = torch.empty(self.capacity, dtype=torch.uint8)
        for start, end, bits, _ in self.plan:
            out[start:end] = bits
        return out.to(self.device)

    @property
    def rows(self):
        """Per-token row index within its width class (the reference's row map)."""
        out = torch.empty(self.capacity, dtype=torch.int32)
        for start, end, bits, row in self.plan:
            out[start:end] = torch.arange(row, row + end - start, dtype=torch.int32)
        return out.to(self.device)

    def select(self, bits, frame_id=-1):
        self.pending_bits, self.frame_id = bits, frame_id

    def get_seq_length(self, layer_idx=0):
        return self.seen[layer_idx]

    def get_max_cache_shape(self, layer_idx=0):
        return None

    def __len__(self):
        return self.layers

    # Mask-size queries of transformers 5.x (masking_utils._preprocess_mask_arguments). The fused
    # attention applies its own bottom-right causal mask and never reads the dense one.
    @property
    def is_sliding(self):
        return [False] * self.layers

    @property
    def is_compileable(self):
        return False

    def get_query_offset(self, layer_idx=0):
        return self.seen[layer_idx or 0]

    def get_mask_sizes(self, query_length, layer_idx=0):
        if isinstance(query_length, torch.Tensor):
            query_length = query_length.shape[0]
        return self.seen[layer_idx or 0] + query_length, 0

    def _tiles_before(self, past):
        return bisect.bisect_left(self.tile_starts, past)

    # -- hot path ----------------------------------------------------------
    @staticmethod
    def _kv_view(x):
        """[1, H, n, 64] view with contiguous rows, 16-byte aligned (copies otherwise)."""
        if (x.stride(-1) != 1 or x.stride(1) % 8 or x.stride(2) % 8 or x.data_ptr() % 16
                or x.dtype != torch.bfloat16):
            x = x.to(torch.bfloat16).contiguous()
        return x

    def append(self, k, v, layer):
        """Packs the new tokens of one layer; returns the history length (src/gpu_cache.py:68-94)."""
        if k.shape[0] != 1 or k.shape[-1] != self.dim or k.device.type != 'cuda':
            raise ValueError('GPU cache requires CUDA, batch one and the configured head dimension')
        if k.dim() != 4 or k.shape[1] != self.heads or v.shape != k.shape or v.device != k.device:
            raise ValueError(f'append expects k and v of shape [1, {self.heads}, n, {self.dim}]')
        if self._graph is not None:
            return self._graph.append(k, v, layer)
        n = k.shape[-2]
        past, seg, write_tiles = self._claim(layer, n)
        if n:
            k, v = self._kv_view(k), self._kv_view(v)
            job = self._job(k, v, layer, past, n, seg, write_tiles)
            lib = _lib.load()
            _lib.check(lib.dkv_pack(ctypes.byref(job), self.arena.data_ptr(), self.arena_bytes,
                                    self.tiles.data_ptr(), self.layers, self.heads,
                                    _lib.stream_handle(self.device)), 'dkv_pack')
        self.seen[layer] = past + n
        return past

    def _claim(self, layer, n):
        """Bookkeeping of an append of n tokens to `layer` (src/gpu_cache.py:70-88): the segment the
        tokens go to, opened on layer 0 in online mode. Returns (past, segment, write_tiles)."""
        past = self.seen[layer]
        if past + n > self.capacity:
            raise ValueError('GPU context limit exceeded')
        write_tiles = 0
        if self.online:
            if layer == 0:
                self._open_segment(past, n, self.pending_bits, self.frame_id)
                write_tiles = 1
            seg = self.segments[-1] if self.segments else None
        else:
            cursor = self.cursors[layer]
            while cursor < len(self.segments) and past >= self.segments[cursor].end:
                cursor += 1
            self.cursors[layer] = cursor
            seg = self.segments[cursor] if cursor < len(self.segments) else None
            if seg is not None and layer == 0 and past == seg.start:
                write_tiles = 1
                seg.frame = self.frame_id
        if seg is None or past + n > seg.end or seg.bits != self.pending_bits:
            raise ValueError(f'Cache append does not match plan at token {past}, length {n}, bits {self.pending_bits}')
        return past, seg, write_tiles

    @staticmethod
    def _job(k, v, layer, past, n, seg, write_tiles):
        return _lib.PackJob(k.data_ptr(), v.data_ptr(), k.stride(1), k.stride(2), v.stride(1), v.stride(2),
                            seg.offset, seg.rows, seg.start, past - seg.start, n, layer, seg.bits, seg.tile0,
                            write_tiles)

    def append_projection(self, qkv, cos, sin, q_heads, layer):
        """The joined Q/K/V projection of one layer -> (q, k, v, past), with RoPE on q and k and the
        new K/V packed, in one launch (dkv_rope_pack).

        Equivalent to splitting qkv [1, n, (q_heads + 2 heads) * 64], applying transformers'
        apply_rotary_pos_emb with cos/sin [1, n, 64] and calling append(k, v, layer), as the patched
        attention forward does (src/gpu_cache.py:164-172): q [1, q_heads, n, 64] and k, v
        [1, heads, n, 64] are bit-equal to that path and the packed bytes identical. Returns None
        when the inputs are outside what the kernel covers (the caller then takes that path).
        """
        n = qkv.shape[1] if qkv.dim() == 3 else -1
        if (n < 1 or qkv.shape[0] != 1 or qkv.shape[2] != (q_heads + 2 * self.heads) * self.dim
                or self.dim != 64 or cos.shape[-2:] != (n, 64) or sin.shape != cos.shape
                or not all(t.is_cuda and t.dtype == torch.bfloat16 for t in (qkv, cos, sin))):
            return None
        qkv2, cos2, sin2 = qkv.reshape(n, -1), cos.reshape(n, 64), sin.reshape(n, 64)
        if any(t.stride(-1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16 for t in (qkv2, cos2, sin2)):
            return None
        q = torch.empty((1, q_heads, n, 64), dtype=qkv.dtype, device=qkv.device)
        k = torch.empty((1, self.heads, n, 64), dtype=qkv.dtype, device=qkv.device)
        v = torch.empty_like(k)
        if self._graph is not None:
            past = self._graph.append_projection(qkv2, cos2, sin2, q_heads, layer, q, k, v)
            return q, k, v, past
        past, seg, write_tiles = self._claim(layer, n)
        job = self._job(k, v, layer, past, n, seg, write_tiles)
        _lib.check(_lib.load().dkv_rope_pack(
            qkv2.data_ptr(), qkv2.stride(0), cos2.data_ptr(), sin2.data_ptr(), cos2.stride(0), n, q_heads,
            q.data_ptr(), k.data_ptr(), v.data_ptr(), ctypes.byref(job), 0, self.arena.data_ptr(),
            self.arena_bytes, self.tiles.data_ptr(), self.layers, self.heads, _lib.stream_handle(self.device)),
            'dkv_rope_pack')
        self.seen[layer] = past + n
        return q, k, v, past

    def _fused_attention(self, n, q_heads, layer, qkv, qkv_stride, cos, sin, cs_stride, qkv_out, out, stream):
        """append_projection() then attend() for the fused decoder layer's eager launches: the same
        two launches with the same arguments (so the same bytes and outputs), without the per-call
        checks of the general entry points, which cost more host time than the GPU spends on a
        64-token chunk. Raw device addresses, which the caller guarantees to be what those checks
        establish: qkv [n, (q_heads + 2 heads) * 64] and cos / sin [n, 64] bf16 rows (element
        strides qkv_stride, cs_stride), qkv_out room for q | k | v as [heads, n, 64] blocks and out
        for the bf16 output [1, n, q_heads, 64], all 16-byte aligned; no graph steps (eager
        launches) and no chunk segments."""
        H, d = self.heads, self.dim
        past, seg, write_tiles = self._claim(layer, n)
        kp = qkv_out + q_heads * n * d * 2
        vp = kp + H * n * d * 2
        head = n * d  # element stride of the heads of q, k and v
        job = _lib.PackJob(kp, vp, head, d, head, d, seg.offset, seg.rows, seg.start, past - seg.start,
                           n, layer, seg.bits, seg.tile0, write_tiles)
        lib = _lib.load()
        _lib.check(lib.dkv_rope_pack(qkv, qkv_stride, cos, sin, cs_stride, n, q_heads, qkv_out, kp, vp,
                                     ctypes.byref(job), 0, self.arena.data_ptr(), self.arena_bytes,
                                     self.tiles.data_ptr(), self.layers, H, stream), 'dkv_rope_pack')
        self.seen[layer] = past + n
        a = self._fused_args
        if a is None or self._fused_key != (n, q_heads):
            # the fields that stay the same while the chunk shape does (attend_args() sets them alike)
            a = self._fused_args = _lib.AttnArgs()
            self._fused_key = (n, q_heads)
            a.q_head_stride = a.kn_head_stride = a.vn_head_stride = head
            a.q_tok_stride = a.kn_tok_stride = a.vn_tok_stride = d
            a.layers, a.heads, a.q_heads, a.nq = self.layers, H, q_heads, n
            a.scale = d ** -0.5
            a.out_tok_stride, a.out_head_stride = q_heads * d, d
        a.q, a.k_new, a.v_new, a.out = qkv_out, kp, vp, out
        a.arena, a.tiles, a.tiles_host = self.arena.data_ptr(), self.tiles.data_ptr(), self._tiles_host_ptr
        a.n_tiles, a.past, a.layer = self._tiles_before(past), past, layer
        a.precision = PRECISIONS[self.precision]
        if q_heads // H * n > SHORT_ROWS:
            a.splits = self.chunk_splits
        need = lib.dkv_attend_workspace_bytes(ctypes.byref(a))
        if need:
            ws = self._workspace_for(need)
            a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        else:
            a.workspace, a.workspace_bytes = None, 0
        _lib.check(lib.dkv_attend(ctypes.byref(a), stream), 'dkv_attend')

    def append_batch(self, k, v, bits, lengths):
        """Appends several segments for every layer in one pack launch.

        k, v: [layers, heads, sum(lengths), 64] bf16 device tensors (last dim contiguous).
        bits, lengths: width and token count of each segment, in order. Equivalent to calling
        select(bits[i]) and append() for every layer and segment; returns the history length
        before the batch. Returns a PackBatch that can re-run the same launch (benchmarks).
        """
        if k.shape[0] != self.layers or k.shape[1] != self.heads or k.shape[-1] != self.dim or k.device.type != 'cuda':
            raise ValueError('append_batch expects [layers, heads, tokens, 64] CUDA tensors')
        if sum(lengths) != k.shape[2] or len(bits) != len(lengths) or len(set(self.seen)) != 1:
            raise ValueError('append_batch: lengths must cover the tokens and every layer must be level')
        past = self.seen[0]
        if past + k.shape[2] > self.capacity:
            raise ValueError('GPU context limit exceeded')
        k, v = self._kv_view4(k), self._kv_view4(v)
        jobs = []
        start = past
        for b, n in zip(bits, lengths):
            if self.online:
                seg = self._open_segment(start, n, b, self.frame_id)
            else:
                seg = next((s for s in self.segments if s.start <= start < s.end), None)
                if seg is None or start + n > seg.end or seg.bits != b:
                    raise ValueError(f'Cache append does not match plan at token {start}, length {n}, bits {b}')
            for layer in range(self.layers):
                t0 = start - past
                jobs.append(_lib.PackJob(
                    k[layer, :, t0:].data_ptr(), v[layer, :, t0:].data_ptr(), k.stride(1), k.stride(2),
                    v.stride(1), v.stride(2), seg.offset, seg.rows, seg.start, start - seg.start, n, layer,
                    seg.bits, seg.tile0, int(layer == 0 and start == seg.start)))
            start += n
        batch = PackBatch(self, jobs, max(lengths), keep=(k, v))
        batch.run()
        self.seen = [start] * self.layers
        return batch

    @staticmethod
    def _kv_view4(x):
        if (x.stride(-1) != 1 or x.stride(1) % 8 or x.stride(2) % 8 or x.stride(0) % 8 or x.data_ptr() % 16
                or x.dtype != torch.bfloat16):
            x = x.to(torch.bfloat16).contiguous()
        return x

    def attend_args(self, q, k, v, layer, past, out, segments=None, path=0, splits=0, precision=None):
        """Fills the C argument block of one attention call."""
        nq = q.shape[-2]
        a = _lib.AttnArgs()
        a.q, a.q_head_stride, a.q_tok_stride = q.data_ptr(), q.stride(1), q.stride(2)
        a.k_new, a.kn_head_stride, a.kn_tok_stride = k.data_ptr(), k.stride(1), k.stride(2)
        a.v_new, a.vn_head_stride, a.vn_tok_stride = v.data_ptr(), v.stride(1), v.stride(2)
        a.arena, a.tiles = self.arena.data_ptr(), self.tiles.data_ptr()
        a.n_tiles, a.past = self._tiles_before(past), past
        a.tiles_host = self._tiles_host_ptr
        a.layer, a.layers, a.heads, a.q_heads, a.nq = layer, self.layers, self.heads, q.shape[1], nq
        if segments:
            if len(segments) - 1 > _lib.DKV_MAX_CHUNK_SEGS:  # bounds [0, b1, ..., nq]: one more than segments
                raise ValueError(f'at most {_lib.DKV_MAX_CHUNK_SEGS} chunk segments')
            a.n_segs = len(segments) - 1
            for i, b in enumerate(segments):
                a.seg_bounds[i] = b
        a.scale = self.dim ** -0.5
        a.out = out.data_ptr()
        a.out_tok_stride, a.out_head_stride = out.stride(1), out.stride(2)
        a.out_dtype = 1 if out.dtype == torch.float32 else 0
        a.path = PATHS[path] if isinstance(path, str) else int(path)
        a.splits = splits
        a.precision = PRECISIONS[precision or self.precision]
        return a

    def _workspace_for(self, nbytes):
        # Split partials of the attention kernels: every call writes what its merge reads.
        if self._workspace is None or self._workspace.numel() < nbytes or self._workspace.device != self.device:
            self._workspace = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=self.device)
        return self._workspace

    def attend(self, q, k, v, layer, past, out_dtype=None, segments=None, path=0, splits=0, precision=None):
        """Causal attention of q over history [0, past) plus the native chunk (src/gpu_cache.py:96-104).

        `segments` (optional) lists chunk boundaries [0, b1, ..., nq] for a block-diagonal batch of
        independent continuations that share the history, e.g. QA candidates. `path` is 'auto' (the
        frame-chunk MFMA kernel, the fastest for every chunk length, decode steps included),
        'mfma', 'short' (the short-chunk kernel, at most 16 query rows per KV head) or 'vector'; `precision` overrides the cache's 'bf16' / 'fp32'
        setting for this call.
        """
        if precision is not None and precision not in PRECISIONS:
            raise ValueError(f'precision must be one of {sorted(PRECISIONS)}')
        if isinstance(path, str) and path not in PATHS:
            raise ValueError(f'path must be one of {sorted(PATHS)}')
        n = q.shape[-2]
        if q.dim() != 4 or q.shape[0] != 1 or q.shape[-1] != self.dim or q.shape[1] % self.heads:
            raise ValueError('attend expects q [1, q_heads, n, 64] with q_heads a multiple of heads')
        if k.shape != (1, self.heads, n, self.dim) or v.shape != k.shape:
            raise ValueError(f'attend expects the chunk k, v of shape [1, {self.heads}, {n}, {self.dim}]')
        if past + n > self.capacity or past > self.seen[layer]:
            raise ValueError('attend: history longer than the cache holds')
        if q.device.type != 'cuda' or k.device != q.device or v.device != q.device:
            raise ValueError('attend requires CUDA tensors on one device')
        if segments is None:
            segments = self.chunk_segments
        if segments is not None and (segments[0] != 0 or segments[-1] != n):
            raise ValueError(f'chunk segments {segments} do not cover the {n}-token chunk')
        if splits == 0 and q.shape[1] // self.heads * n > SHORT_ROWS:
            splits = self.chunk_splits
        out_dtype = out_dtype or q.dtype
        _check_dtype(out_dtype, 'attend output dtype')
        q, k, v = self._kv_view(q), self._kv_view(k), self._kv_view(v)
        out = torch.empty((1, n, q.shape[1], self.dim), dtype=out_dtype, device=q.device)
        if self._graph is not None:
            a = self._graph.attend_args(q, k, v, layer, out, segments, path, splits, precision)
        else:
            a = self.attend_args(q, k, v, layer, past, out, segments, path, splits, precision)
        lib = _lib.load()
        need = lib.dkv_attend_workspace_bytes(ctypes.byref(a))
        if need:
            # A captured graph keeps the workspace it recorded: graph launches use their
            # GraphSteps' own buffer, so an ordinary call that grows the cache's buffer can never
            # free memory a graph still writes.
            ws = self._graph.workspace(need) if self._graph is not None else self._workspace_for(need)
            a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        _lib.check(lib.dkv_attend(ctypes.byref(a), _lib.stream_handle(self.device)), 'dkv_attend')
        return out

    def materialize(self, layer, out_dtype=None):
        """Dequantized history of one layer: (k, v), each [1, H, seen, 64] (src/gpu_cache.py:106-112)."""
        n = self.seen[layer]
        out_dtype = out_dtype or self.dtype
        _check_dtype(out_dtype, 'materialize output dtype')
        out = torch.empty((2, self.heads, n, self.dim), dtype=out_dtype, device=self.device)
        if n:
            lib = _lib.load()
            _lib.check(lib.dkv_reconstruct(self.arena.data_ptr(), self.tiles.data_ptr(), self._tiles_before(n), n,
                                           layer, self.layers, self.heads, out.data_ptr(),
                                           1 if out.dtype == torch.float32 else 0,
                                           _lib.stream_handle(self.device)), 'dkv_reconstruct')
        return out[0:1], out[1:2]

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        """HF Cache.update compatibility path (src/gpu_cache.py:114-119)."""
        self.append(key_states, value_states, layer_idx)
        k, v = self.materialize(layer_idx)
        k[:, :, -key_states.shape[-2]:].copy_(key_states)
        v[:, :, -value_states.shape[-2]:].copy_(value_states)
        return k, v

    def fork(self):
        """Branch that shares the arena and tile table (src/gpu_cache.py:121-132).

        Branches write only past the base's used bytes and tiles; branches of one base overwrite
        the same region, so they must run one after another on one stream.
        """
        other = object.__new__(GPUCache)
        other.__dict__ = self.__dict__.copy()
        other.seen = self.seen.copy()
        other.cursors = self.cursors.copy()
        other.plan = self.plan.copy()
        other.segments = self.segments.copy()
        other.tile_starts = self.tile_starts.copy()
        other.host_counts = self.host_counts.copy()
        other._workspace = None
        other._graph = None
        other._fused_args, other._fused_key = None, None
        other.pending_bits = 16
        return other

    def accounting(self):
        """Used vs. allocated bytes with the reference's keys and formulas (src/gpu_cache.py:134-149).

        token_mapping_bytes is the reference's 5 bytes per token (its int32 row index plus uint8
        width code, src/gpu_cache.py:143), so gpu_cache_used_bytes compares with the reference's
        figures; this cache maps tokens with one 16-byte descriptor per 64-token tile instead,
        reported as tile_table_bytes."""
        allocated = self.arena.numel() + self.tiles.numel()
        used = {4: 0, 8: 0, 16: 0}
        n = self.seen[0]
        for start, end, bits, _ in self.plan:
            used[bits] += max(0, min(n, end) - start)
        payload = self.layers * 2 * self.heads * self.dim * sum(used[b] * b / 8 for b in used)
        scales = self.layers * 2 * self.heads * 8 * (used[4] + used[8])
        mapping = 5 * n
        return dict(gpu_cache_used_bytes=int(payload + scales + mapping),
                    gpu_cache_allocated_bytes=allocated, cpu_cache_payload_bytes=0,
                    payload_bytes=int(payload), quantization_metadata_bytes=int(scales),
                    token_mapping_bytes=mapping, logical_index_capacity=self.capacity,
                    precision_pool_capacities=self.caps,
                    used_tokens=n, precision_token_counts=used,
                    arena_used_bytes=self.arena_used, tile_table_bytes=16 * self._tiles_before(n))


    # -- HIP graph replays (no reference counterpart) ---------------------------
    def begin_graph_steps(self, chunk, q_heads=None, steps=None):
        """Switches append()/attend() to launches that read their per-step parameters from device
        memory, so that a decoder forward over `chunk`-token chunks can be captured once in a HIP
        graph and replayed as the history grows. Before capturing, and before every replay, call
        graph_step(); in this mode append() and attend() only launch (no bookkeeping).

        `q_heads` pre-sizes the steps' attention workspace for the launch bounds (so nothing is
        allocated while capturing); graph launches use that buffer, never the one ordinary calls
        grow. `steps` re-attaches the GraphSteps of an earlier capture on this cache, or on any
        cache with the same arena and tile table (a fork of it, or a fork of the cache it forked
        from): the recorded launches address only those two buffers and the steps' own.
        """
        if len(set(self.seen)) != 1:
            raise ValueError('graph steps need every layer at the same length')
        if steps is not None and steps.cache is not self:
            if steps.arena is not self.arena or steps.tiles is not self.tiles:
                raise ValueError('these graph steps belong to a cache with another arena')
            steps.cache = self
        self._graph = steps or GraphSteps(self, chunk)
        if q_heads:
            self._graph.workspace(self._graph.workspace_bytes(q_heads))
        return self._graph

    def end_graph_steps(self):
        """Back to ordinary launches; returns the GraphSteps for a later begin_graph_steps()."""
        steps, self._graph = self._graph, None
        return steps

    def graph_step(self):
        """Bookkeeping of one chunk for every layer (at the pending width and frame, like a layer-0
        append) plus the upload of what the recorded launches read. Returns the history length
        before the chunk."""
        if self._graph is None:
            raise ValueError('graph_step() needs begin_graph_steps()')
        return self._graph.step()

    def reset(self):
        """Empties the cache in place, keeping its arena, tile table and device buffers (a new
        request on a reused cache keeps every pointer a captured graph recorded)."""
        self.seen = [0] * self.layers
        self.cursors = [0] * self.layers
        self.pending_bits, self.frame_id = 16, -1
        if self.online:
            self.segments, self.tile_starts, self.plan = [], [], []
            self.host_counts = {4: 0, 8: 0, 16: 0}
            self.arena_used = 0

    # -- the reference's serialized formats (src/kv_quantization.py:12-77, src/cache_manager.py:9-58) --
    def _layer_range(self, layers):
        layers = list(range(self.layers)) if layers is None else list(layers)
        if not layers or layers != list(range(layers[0], layers[0] + len(layers))) or layers[0] < 0 \
                or layers[-1] >= self.layers:
            raise ValueError(f'layers must be a nonempty ascending run of [0, {self.layers})')
        return layers

    def export_segments(self, layers=None, device=None):
        """The cache as src/cache_manager.py's MixedPrecisionCache would hold it: {layer: [Segment]}.

        Every segment's key and value become PackedTensors with the bytes
        src/kv_quantization.py:pack produces for that [1, heads, rows, 64] tensor (payload,
        fp32 scales and offsets, 64-byte header) and a 32-byte descriptor
        (layer, frame, start, end, bits). One byte-moving launch for all segments; nothing
        is requantized. `layers` (default all) must be consecutive and at the same length.
        The tensors stay on the cache's device unless `device` names another.
        """
        return SegmentExport(self, layers).run().segments(device)

    def import_segments(self, segments):
        """Appends {layer: [Segment]} (the MixedPrecisionCache layout) to every layer; returns the old length.

        Segment i of every layer must describe the same tokens, frame and width, starting at the
        cache's current length, and hold PackedTensors of [1, heads, rows, 64] tensors with group
        size 64 (16-bit ones in bf16). Their payload, offsets and scales are copied into the arena
        unchanged (one launch), so attending over them equals attending over the same tokens
        packed by append().
        """
        return self._import(segments)[0]

    def _import(self, segments):
        """import_segments(), also returning the SegmentBatch that ran (None if nothing moved)."""
        if sorted(segments) != list(range(self.layers)):
            raise ValueError('import_segments needs the segments of every layer')
        counts = {len(v) for v in segments.values()}
        if len(counts) != 1:
            raise ValueError('import_segments: layers hold different numbers of segments')
        if len(set(self.seen)) != 1:
            raise ValueError('import_segments: every layer must be at the same length')
        past = self.seen[0]
        entries, end = [], past
        for i in range(counts.pop()):
            fields = [formats.descriptor_fields(segments[l][i].descriptor) for l in range(self.layers)]
            layer0, frame, start, stop, bits = fields[0]
            for l, f in enumerate(fields):
                if f[0] != l:
                    raise ValueError(f'segment {i} of layer {l} is labelled layer {f[0]}')
                if f[1:] != (frame, start, stop, bits):
                    raise ValueError(f'layers disagree about segment {i}: {f[1:]} vs {(frame, start, stop, bits)}')
            if bits not in BITS or start != end or stop <= start:
                raise ValueError(f'segment {i} covers [{start}, {stop}) at {bits} bits; expected to start at {end}')
            for l in range(self.layers):
                formats.check_packed(segments[l][i].key, bits, self.heads, stop - start)
                formats.check_packed(segments[l][i].value, bits, self.heads, stop - start)
            entries.append((i, frame, start, stop - start, bits))
            end = stop
        if end > self.capacity:
            raise ValueError('GPU context limit exceeded')
        ios, keep, max_rows = [], [], 1
        for i, frame, start, rows, bits in entries:
            if self.online:
                seg = self._open_segment(start, rows, bits, frame)
            else:
                seg = next((s for s in self.segments if s.start <= start < s.end), None)
                if seg is None or start + rows > seg.end or seg.bits != bits:
                    raise ValueError(f'Cache append does not match plan at token {start}, length {rows}, bits {bits}')
            layer_segs = [segments[l][i] for l in range(self.layers)]
            pay = torch.stack([torch.stack([s.key.payload for s in layer_segs]),
                               torch.stack([s.value.payload for s in layer_segs])]).to(self.device)
            io = _lib.SegmentIO()
            if bits < 16:
                meta = torch.stack([torch.stack([torch.stack([getattr(s, kv).offsets for s in layer_segs]),
                                                 torch.stack([getattr(s, kv).scales for s in layer_segs])])
                                    for kv in ('key', 'value')]).to(self.device)
                keep.append(meta)
                for kv in range(2):
                    io.offsets[kv], io.scales[kv] = meta[kv, 0].data_ptr(), meta[kv, 1].data_ptr()
            keep.append(pay)
            for kv in range(2):
                io.payload[kv] = pay[kv].data_ptr()
            io.seg_offset, io.seg_rows, io.seg_token_start = seg.offset, seg.rows, seg.start
            io.row0, io.rows, io.bits, io.layer0, io.n_layers = start - seg.start, rows, bits, 0, self.layers
            io.tile_index0, io.write_tiles = seg.tile0, int(start == seg.start)
            if start == seg.start:
                seg.frame = frame
            ios.append(io)
        batch = SegmentBatch(self, ios, 1, keep=keep) if ios else None
        if batch is not None:
            batch.run()
        self.seen = [end] * self.layers
        return past, batch


def write_job_sources(jobs, kv):
    """The per-layer fields of a PackJob array (numpy view, GraphSteps.JOB dtype): the K/V views
    layer l's append recorded (pointer and head/token strides; zeros before the capture) and l."""
    for l, pair in enumerate(kv):
        kp, vp, ks, vs = (pair[0].data_ptr(), pair[1].data_ptr(), pair[0].stride(), pair[1].stride()) if pair \
            else (0, 0, (0, 0, 0, 0), (0, 0, 0, 0))
        jobs[l] = (kp, vp, ks[1], ks[2], vs[1], vs[2], 0, 0, 0, 0, 0, l, 0, 0, 0)


def write_step_jobs(jobs, seg, past, n, write):
    """The fields every layer's job of one step shares: the segment, the rows being appended and,
    on layer 0's job only, whether it writes the segment's tile descriptors."""
    jobs['seg_offset'] = seg.offset
    jobs['seg_rows'] = seg.rows
    jobs['seg_token_start'] = seg.start
    jobs['row0'] = past - seg.start
    jobs['n'] = n
    jobs['bits'] = seg.bits
    jobs['tile_index0'] = seg.tile0
    jobs['write_tiles'] = 0
    jobs['write_tiles'][0] = write


class GraphSteps:
    """Device-side step parameters of one GPUCache for HIP-graph replays.

    One device buffer holds a pack job per layer (dkv_pack_batch reads layer l's job) and the
    {past, n_tiles} pair every attention launch reads (dkv_attn_args.step). step() does the host
    bookkeeping of one chunk and uploads the buffer through a ring of pinned host copies, so the
    host can prepare step i+1 while the GPU still runs step i. The K/V pointers of the jobs are
    those append() saw while the graph was captured (they are fixed for a captured graph): a
    ring slot gets them once, and a step rewrites only the fields every layer's job shares.
    """
    RING = 4
    JOB = np.dtype(_lib.PackJob)

    def __init__(self, cache, chunk):
        self.cache, self.chunk = cache, chunk
        # the buffers the recorded launches address: step() refuses to run once the cache holds others
        self.arena, self.tiles = cache.arena, cache.tiles
        self.job_bytes = ctypes.sizeof(_lib.PackJob)
        self.nbytes = cache.layers * self.job_bytes + 8
        with torch.inference_mode(False):  # ordinary tensors: step() may run inside or outside inference mode
            self.dev = torch.zeros(self.nbytes, dtype=torch.uint8, device=cache.device)
        self.ring = None  # pinned host copies, allocated by the first upload()
        self.views = None
        self.slot = 0
        self.kv = [None] * cache.layers  # (k, v) views append() recorded, kept alive with the graph
        self.kv_version = 0  # bumped whenever append() records a view
        self.slot_kv = [-1] * self.RING  # kv_version each slot's pointer fields were written with
        self.state = None  # (past, segment, write_tiles) of the current step
        # Launch bounds: the largest history a chunk can attend to in this cache.
        self.past_bound = cache.capacity - chunk
        self.tiles_bound = cache.tiles.shape[0]
        self.ws = None  # attention workspace of the recorded launches (grow-only)
        self.retired = []  # smaller workspaces handed out before: graphs captured earlier still address them

    def workspace(self, nbytes):
        """The attention workspace graph launches use, at least `nbytes` bytes. A buffer once handed
        out is never freed while the steps live, even when a later call needs a larger one: a graph
        captured with it (on these steps, or re-attached ones) keeps writing its partials there."""
        if self.ws is None or self.ws.numel() < nbytes:
            if self.ws is not None:
                self.retired.append(self.ws)
            grow = 2 * self.ws.numel() if self.ws is not None else 0
            with torch.inference_mode(False):
                self.ws = torch.zeros(max(nbytes, grow, 1 << 20), dtype=torch.uint8, device=self.cache.device)
        return self.ws

    def _check_storage(self):
        c = self.cache
        if c.arena is not self.arena or c.tiles is not self.tiles:
            raise ValueError('the cache no longer holds the arena and tile table these graph steps recorded '
                             '(it grew or was rebuilt): capture again')

    def step(self):
        c, n = self.cache, self.chunk
        self._check_storage()
        past = c.seen[0]
        if len(set(c.seen)) != 1:
            raise ValueError('graph steps need every layer at the same length')
        if past + n > c.capacity:
            raise ValueError('GPU context limit exceeded')
        if c.online:
            seg = c._open_segment(past, n, c.pending_bits, c.frame_id, grow=False)
            write = 1
        else:
            seg = next((s for s in c.segments if s.start <= past < s.end), None)
            if seg is None or past + n > seg.end or seg.bits != c.pending_bits:
                raise ValueError(f'Cache append does not match plan at token {past}, length {n}, '
                                 f'bits {c.pending_bits}')
            write = int(past == seg.start)
            if write:
                seg.frame = c.frame_id
        self.state = (past, seg, write)
        c.seen = [past + n] * c.layers
        self.upload()
        return past

    def _view(self, host):
        """(jobs, tail) numpy views of a pinned ring buffer: the per-layer PackJob array, then the
        {past, n_tiles} int32 pair."""
        raw = host.numpy()
        split = self.cache.layers * self.job_bytes
        return raw[:split].view(self.JOB), raw[split:split + 8].view(np.int32)

    def upload(self):
        """Writes the current step's jobs and bounds to the device buffer (async, stream-ordered)."""
        c, n = self.cache, self.chunk
        self._check_storage()
        past, seg, write = self.state
        if self.ring is None:
            with torch.inference_mode(False):
                self.ring = [(torch.zeros(self.nbytes, dtype=torch.uint8, pin_memory=True), None)
                             for _ in range(self.RING)]
            self.views = [self._view(host) for host, _ in self.ring]
        host, event = self.ring[self.slot]
        if event is not None:
            event.synchronize()  # that slot's previous copy has been consumed
        jobs, tail = self.views[self.slot]
        if self.slot_kv[self.slot] != self.kv_version:
            write_job_sources(jobs, self.kv)
            self.slot_kv[self.slot] = self.kv_version
        write_step_jobs(jobs, seg, past, n, write)
        tail[0], tail[1] = past, c._tiles_before(past)
        if all(kv is not None for kv in self.kv):
            _lib.check(_lib.load().dkv_pack_validate(host.data_ptr(), c.layers, c.arena_bytes, c.layers, c.heads),
                       'dkv_pack_validate')
        self.dev.copy_(host, non_blocking=True)
        event = torch.cuda.Event()
        event.record()
        self.ring[self.slot] = (host, event)
        self.slot = (self.slot + 1) % self.RING

    def append(self, k, v, layer):
        c = self.cache
        if self.state is None:
            raise ValueError('graph_step() must run before the recorded append')
        if k.shape[-2] != self.chunk:
            raise ValueError(f'graph steps were set up for {self.chunk}-token chunks, got {k.shape[-2]}')
        k, v = c._kv_view(k), c._kv_view(v)
        self.kv[layer] = (k, v)
        self.kv_version += 1
        if not torch.cuda.is_current_stream_capturing():
            # an eager launch reads its job when it runs: upload the job again so that it carries
            # the K/V views just recorded (the last upload may predate them: null sources), ordered
            # on this stream before the launch
            self.upload()
        _lib.check(_lib.load().dkv_pack_batch(self.dev.data_ptr() + layer * self.job_bytes, 1, self.chunk,
                                              c.arena.data_ptr(), c.arena_bytes, c.tiles.data_ptr(), c.layers,
                                              c.heads, _lib.stream_handle(c.device)), 'dkv_pack_batch')
        return self.state[0]

    def append_projection(self, qkv, cos, sin, q_heads, layer, q, k, v):
        c = self.cache
        if self.state is None:
            raise ValueError('graph_step() must run before the recorded append')
        if qkv.shape[0] != self.chunk:
            raise ValueError(f'graph steps were set up for {self.chunk}-token chunks, got {qkv.shape[0]}')
        self.kv[layer] = (k, v)
        self.kv_version += 1
        _lib.check(_lib.load().dkv_rope_pack(
            qkv.data_ptr(), qkv.stride(0), cos.data_ptr(), sin.data_ptr(), cos.stride(0), self.chunk, q_heads,
            q.data_ptr(), k.data_ptr(), v.data_ptr(), self.dev.data_ptr() + layer * self.job_bytes, 1,
            c.arena.data_ptr(), c.arena_bytes, c.tiles.data_ptr(), c.layers, c.heads,
            _lib.stream_handle(c.device)), 'dkv_rope_pack')
        return self.state[0]

    def attend_args(self, q, k, v, layer, out, segments, path, splits, precision):
        c = self.cache
        a = c.attend_args(q, k, v, layer, self.past_bound, out, segments, path, splits, precision)
        a.n_tiles = self.tiles_bound
        a.step = self.dev.data_ptr() + c.layers * self.job_bytes
        return a

    def workspace_bytes(self, q_heads):
        a = _lib.AttnArgs()
        a.n_tiles, a.past = self.tiles_bound, self.past_bound
        a.layer, a.layers, a.heads, a.q_heads, a.nq = 0, self.cache.layers, self.cache.heads, q_heads, self.chunk
        a.precision = PRECISIONS[self.cache.precision]
        a.step = self.dev.data_ptr() + self.cache.layers * self.job_bytes  # launches sized for any history
        return _lib.load().dkv_attend_workspace_bytes(ctypes.byref(a))


class SegmentExport:
    """The export launch of a cache's filled segments and the buffers it fills; run() relaunches it."""

    def __init__(self, cache, layers=None):
        layers = cache._layer_range(layers)
        seen = {cache.seen[l] for l in layers}
        if len(seen) != 1:
            raise ValueError('export_segments: the exported layers differ in length')
        n, nl, heads = seen.pop(), len(layers), cache.heads
        self.cache, self.layers, self.parts, self.nbytes = cache, layers, [], 0
        ios = []
        for seg in cache.segments:
            rows = min(n, seg.end) - seg.start
            if rows <= 0:
                break
            rb = formats.row_bytes(seg.bits)
            pay = torch.empty((2, nl, heads, rows, rb), dtype=torch.uint8, device=cache.device)
            meta = (torch.empty((2, 2, nl, heads, rows), dtype=torch.float32, device=cache.device)
                    if seg.bits < 16 else None)
            io = _lib.SegmentIO()
            for kv in range(2):
                io.payload[kv] = pay[kv].data_ptr()
                if meta is not None:
                    io.offsets[kv], io.scales[kv] = meta[kv, 0].data_ptr(), meta[kv, 1].data_ptr()
            io.seg_offset, io.seg_rows, io.seg_token_start = seg.offset, seg.rows, seg.start
            io.row0, io.rows, io.bits, io.layer0, io.n_layers = 0, rows, seg.bits, layers[0], nl
            ios.append(io)
            self.parts.append((seg, rows, pay, meta))
            self.nbytes += pay.numel() + (meta.numel() * 4 if meta is not None else 0)
        self.batch = SegmentBatch(cache, ios, 0) if ios else None

    def run(self):
        if self.batch is not None:
            self.batch.run()
        return self

    def segments(self, device=None):
        """{layer: [Segment]} over the buffers (moved to `device` if given)."""
        c = self.cache
        out = {l: [] for l in self.layers}
        for seg, rows, pay, meta in self.parts:
            if device is not None:
                pay = pay.to(device)
                meta = meta.to(device) if meta is not None else None
            empty = torch.empty(0, dtype=torch.float32, device=pay.device)
            # 16-bit rows are stored as bf16; 4/8-bit headers carry the dtype the cache was given
            hdr_dtype = torch.bfloat16 if seg.bits == 16 else c.dtype
            for i, l in enumerate(self.layers):
                packed = []
                for kv in range(2):
                    hdr = formats.header(seg.bits, c.heads, rows, hdr_dtype)
                    if meta is None:
                        packed.append(formats.PackedTensor(pay[kv, i].flatten(), empty, empty, hdr))
                    else:
                        packed.append(formats.PackedTensor(pay[kv, i].flatten(), meta[kv, 1, i].flatten(),
                                                           meta[kv, 0, i].flatten(), hdr))
                desc = formats.descriptor(l, seg.frame, seg.start, seg.start + rows, seg.bits)
                out[l].append(formats.Segment(packed[0], packed[1], desc))
        return out


class SegmentBatch:
    """A device table for dkv_segment_batch (direction 0 exports, 1 imports); run() relaunches it."""

    def __init__(self, cache, ios, direction, keep=()):
        self.cache, self.direction, self.n, self._keep = cache, direction, len(ios), keep
        self.max_rows = max(io.seg_rows for io in ios)
        self.max_layers = max(io.n_layers for io in ios)
        table = (_lib.SegmentIO * len(ios))(*ios)
        # the kernel trusts the device table: check the host copy against the arena first
        _lib.check(_lib.load().dkv_segment_validate(ctypes.addressof(table), len(ios), direction, cache.arena_bytes,
                                                    cache.layers, cache.heads), 'dkv_segment_validate')
        self.table = torch.frombuffer(bytearray(bytes(table)), dtype=torch.uint8).to(cache.device)

    def run(self):
        c = self.cache
        _lib.check(_lib.load().dkv_segment_batch(self.table.data_ptr(), self.n, self.max_rows, self.max_layers,
                                                 self.direction, c.arena.data_ptr(), c.arena_bytes,
                                                 c.tiles.data_ptr(), c.layers, c.heads,
                                                 _lib.stream_handle(c.device)), 'dkv_segment_batch')


class PackBatch:
    """A device job table for dkv_pack_batch plus the cache it writes; run() relaunches it."""

    def __init__(self, cache, jobs, max_n, keep=()):
        self.cache, self.max_n, self.n_jobs, self._keep = cache, max_n, len(jobs), keep
        table = (_lib.PackJob * len(jobs))(*jobs)
        # the kernel trusts the device table: check the host copy against the arena first
        _lib.check(_lib.load().dkv_pack_validate(ctypes.addressof(table), len(jobs), cache.arena_bytes,
                                                 cache.layers, cache.heads), 'dkv_pack_validate')
        raw = torch.frombuffer(bytearray(bytes(table)), dtype=torch.uint8)
        self.table = raw.to(cache.device)
        self.arena, self.arena_bytes, self.tiles = cache.arena, cache.arena_bytes, cache.tiles

    def run(self):
        lib = _lib.load()
        _lib.check(lib.dkv_pack_batch(self.table.data_ptr(), self.n_jobs, self.max_n, self.arena.data_ptr(),
                                      self.arena_bytes, self.tiles.data_ptr(), self.cache.layers,
                                      self.cache.heads, _lib.stream_handle(self.cache.device)), 'dkv_pack_batch')


def attend_projection(module, cache, qkv, position_embeddings):
    """The packed-cache attention of one LlamaAttention from its joined projection qkv [1, n, (nq + 2 nkv) * d]:
    split + RoPE + append (one launch when dkv_rope_pack covers it), then attend. Returns the attention output
    [1, n, nq, d] (src/gpu_cache.py:164-174)."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    from .gpu_ops import rope_qkv
    hd, layer = module.head_dim, module.layer_idx
    nq, nkv = module._qkv_sizes[0] // hd, module._qkv_sizes[1] // hd
    packed = cache.append_projection(qkv, *position_embeddings, nq, layer) if nkv == cache.heads else None
    if packed is not None:
        q, k, v, past = packed
    else:
        roped = rope_qkv(qkv, *position_embeddings, nq, nkv, hd)  # split + RoPE in one launch
        if roped is not None:
            q, k, v = roped
        else:
            shape = qkv.shape[:-1]
            q, k, v = qkv.split(module._qkv_sizes, dim=-1)
            q = q.view(*shape, -1, hd).transpose(1, 2)
            k = k.view(*shape, -1, hd).transpose(1, 2)
            v = v.view(*shape, -1, hd).transpose(1, 2)
            q, k = apply_rotary_pos_emb(q, k, *position_embeddings)
        past = cache.append(k, v, layer)
    return cache.attend(q, k, v, layer, past)


def install_packed_attention(model):
    """Routes LlamaAttention through the packed cache when given a GPUCache (src/gpu_cache.py:151-183).

    All other caches keep the upstream forward. Accepts both the `past_key_value` keyword of
    transformers 4.x and the `past_key_values` keyword of 5.x.
    """
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    def forward(module, hidden_states, position_embeddings=None, attention_mask=None, past_key_value=None,
                cache_position=None, **kwargs):
        cache = past_key_value if past_key_value is not None else kwargs.get('past_key_values')
        fused = isinstance(cache, GPUCache) and cache.backend == 'fused'
        fast_gqa = getattr(cache, 'fast_gqa', False)
        if not fused and not fast_gqa:
            if past_key_value is not None:
                kwargs['past_key_value'] = past_key_value
            return module._original_forward(hidden_states=hidden_states, position_embeddings=position_embeddings,
                                            attention_mask=attention_mask, cache_position=cache_position, **kwargs)
        if kwargs.get('output_attentions', False):
            raise ValueError('Fused packed attention does not expose attention matrices')
        shape = hidden_states.shape[:-1]
        if fused and hasattr(module, '_qkv_weight'):
            qkv = F.linear(hidden_states, module._qkv_weight)
            output = attend_projection(module, cache, qkv, position_embeddings)
            return module.o_proj(output.reshape(*shape, -1).contiguous()), None
        q, k, v = module.q_proj(hidden_states), module.k_proj(hidden_states), module.v_proj(hidden_states)
        q = q.view(*shape, -1, module.head_dim).transpose(1, 2)
        k = k.view(*shape, -1, module.head_dim).transpose(1, 2)
        v = v.view(*shape, -1, module.head_dim).transpose(1, 2)
        q, k = apply_rotary_pos_emb(q, k, *position_embeddings)
        if fused:
            past = cache.append(k, v, module.layer_idx)
            output = cache.attend(q, k, v, module.layer_idx, past)
        else:
            k, v = cache.update(k, v, module.layer_idx, {'cache_position': cache_position})
            mask = None if attention_mask is None else attention_mask[:, :, :, :k.shape[-2]]
            output = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, dropout_p=0,
                                                    is_causal=mask is None and q.shape[-2] > 1,
                                                    scale=module.scaling, enable_gqa=True).transpose(1, 2)
        return module.o_proj(output.reshape(*shape, -1).contiguous()), None

    for module in model.modules():
        if module.__class__.__name__ == 'LlamaAttention' and not hasattr(module, '_original_forward'):
            module._original_forward = module.forward
            module.forward = types.MethodType(forward, module)
