"""Serialized formats on the GPU: export/import between the arena and the reference's
PackedTensor + segment-descriptor layout (src/kv_quantization.py:12-77,
src/cache_manager.py:9-58).

The expected bytes come from the oracle's restatement of the reference CPU cache
(oracle/cpu_path.py MixedPrecisionCache). Fed the same K/V, select() calls and
layer order as a GPUCache, its segments must equal GPUCache.export_segments()
byte for byte: payload, fp32 offsets and scales (compared as bit patterns),
64-byte headers and 32-byte descriptors. Import is checked the other way round:
the oracle's segments imported into a fresh cache give the same arena bytes,
reconstructions and attention outputs as appending the same tokens.
"""
import ctypes

import pytest
import torch

from conftest import announce
from dkv import _lib
from dkv.gpu_cache import GPUCache
from oracle.cpu_path import MixedPrecisionCache

pytestmark = pytest.mark.gpu

HEADS = 5
# (bits, frame, tokens): a 16-bit text prefix, frames at mixed widths, a ragged tail
SCHEDULE = [(16, -1, 16), (4, 0, 64), (8, 1, 64), (16, 2, 64), (4, 3, 64), (8, 4, 24), (4, 5, 2)]


def kv_chunks(layers, schedule, seed, device):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _, _, n in schedule:
        k = torch.randn((layers, 1, HEADS, n, 64), generator=g)
        v = torch.randn((layers, 1, n, HEADS, 64), generator=g).transpose(2, 3)  # strided V, as the model's views
        ch = torch.randperm(64, generator=g)[:4]
        k[..., ch] *= 8  # outlier channels
        out.append((k.to(torch.bfloat16).to(device), v.to(torch.bfloat16).to(device)))
    return out


def fill(cache, chunks, schedule):
    for (bits, frame, _), (k, v) in zip(schedule, chunks):
        cache.select(bits, frame)
        for l in range(k.shape[0]):
            if isinstance(cache, GPUCache):
                cache.append(k[l], v[l], l)
            else:
                cache.update(k[l].cpu(), v[l].cpu(), l)
    return cache


def bits_of(t):
    return t.view(torch.int32) if t.dtype == torch.float32 else t


def assert_packed_equal(got, ref):
    for name in ('payload', 'scales', 'offsets', 'header'):
        a, b = getattr(got, name).cpu(), getattr(ref, name).cpu()
        assert a.dtype == b.dtype and a.shape == b.shape, (name, a.shape, b.shape)
        assert torch.equal(bits_of(a), bits_of(b)), name
    assert got.fields() == ref.fields()


def assert_segments_equal(got, ref):
    assert sorted(got) == sorted(ref)
    for l in ref:
        assert len(got[l]) == len(ref[l])
        for g, r in zip(got[l], ref[l]):
            assert torch.equal(g.descriptor.cpu(), r.descriptor), (l, g.fields(), r.descriptor)
            assert_packed_equal(g.key, r.key)
            assert_packed_equal(g.value, r.value)


def test_export_equals_the_reference_cpu_cache_byte_for_byte(cuda):
    announce('segments: export vs oracle MixedPrecisionCache, 3 layers')
    layers = 3
    chunks = kv_chunks(layers, SCHEDULE, seed=11, device=cuda)
    gpu = fill(GPUCache(None, layers=layers, heads=HEADS, max_tokens=512), chunks, SCHEDULE)
    ref = fill(MixedPrecisionCache(), chunks, SCHEDULE)
    got = gpu.export_segments(device='cpu')
    assert_segments_equal(got, ref.segments)
    # the reference cache's byte accounting reads the exported segments the same way
    twin = MixedPrecisionCache()
    twin.segments = got
    assert twin.accounting() == ref.accounting()
    assert twin.accounting(frame_only=True) == ref.accounting(frame_only=True)


def test_import_of_reference_segments_reproduces_the_packed_cache(cuda):
    announce('segments: import oracle segments vs append')
    layers = 2
    chunks = kv_chunks(layers, SCHEDULE, seed=12, device=cuda)
    appended = fill(GPUCache(None, layers=layers, heads=HEADS, max_tokens=512), chunks, SCHEDULE)
    ref = fill(MixedPrecisionCache(), chunks, SCHEDULE)
    imported = GPUCache(None, layers=layers, heads=HEADS, max_tokens=512)
    assert imported.import_segments(ref.segments) == 0
    torch.cuda.synchronize()
    assert imported.seen == appended.seen
    assert imported.plan == appended.plan and imported.arena_used == appended.arena_used
    # every schedule length is even, so sub-blocks have no padding bytes and the arenas compare whole
    assert torch.equal(imported.arena[:imported.arena_used], appended.arena[:appended.arena_used])
    n_tiles = len(appended.tile_starts)
    assert torch.equal(imported.tiles[:n_tiles], appended.tiles[:n_tiles])
    assert [s.frame for s in imported.segments] == [f for _, f, _ in SCHEDULE]
    for l in range(layers):
        for a, b in zip(imported.materialize(l), appended.materialize(l)):
            assert torch.equal(a, b)
    g = torch.Generator().manual_seed(13)
    q = torch.randn((1, 3 * HEADS, 40, 64), generator=g).to(torch.bfloat16).to(cuda)
    k = torch.randn((1, HEADS, 40, 64), generator=g).to(torch.bfloat16).to(cuda)
    past = imported.seen[0]
    for path in ('vector', 'mfma'):
        a = imported.attend(q, k, k, 1, past, path=path)
        b = appended.attend(q, k, k, 1, past, path=path)
        assert torch.equal(a, b), path


def test_round_trip_planned_cache_partial_export_and_fork(cuda):
    announce('segments: planned cache, partial segment, layer subset, fork, round trip')
    layers = 3
    sched = [(8, 7, 40), (4, 8, 64), (16, 9, 30)]
    chunks = kv_chunks(layers, sched, seed=14, device=cuda)
    plan = [(8, 40), (4, 100), (16, 30)]  # the 4-bit plan segment is only partly filled
    c = fill(GPUCache(plan, layers=layers, heads=HEADS), chunks[:2], sched[:2])
    out = c.export_segments(layers=[1, 2])
    assert sorted(out) == [1, 2]
    assert [s.fields() for s in out[1]] == [(1, 7, 0, 40, 8), (1, 8, 40, 104, 4)]
    assert out[2][1].key.fields()[2] == (1, HEADS, 64, 64)
    full = c.export_segments()
    assert_segments_equal(out, {l: full[l] for l in (1, 2)})
    # a fork extends the history; exporting it leaves the base unchanged
    branch = c.fork()
    branch.select(4, 8)
    k, v = chunks[2]
    for l in range(layers):
        branch.append(k[l, :, :, :20], v[l, :, :, :20], l)
    assert [s.fields()[3] for s in branch.export_segments()[0]] == [40, 124]
    assert [s.fields()[3] for s in c.export_segments()[0]] == [40, 104]
    # round trip: import the export into an online cache and export again
    again = GPUCache(None, layers=layers, heads=HEADS, max_tokens=256)
    again.import_segments(full)
    assert_segments_equal(again.export_segments(device='cpu'), full)
    # importing into a matching plan continues a partly filled plan segment (row0 > 0)
    planned = GPUCache(plan, layers=layers, heads=HEADS)
    first = {l: [full[l][0]] for l in full}
    planned.import_segments(first)
    planned.select(4, 8)
    k4, v4 = chunks[1]
    for l in range(layers):
        planned.append(k4[l, :, :, :32], v4[l, :, :, :32], l)
    rest = {l: [without_first_rows(full[l][1], 32)] for l in full}
    planned.import_segments(rest)
    for l in range(layers):
        for a, b in zip(planned.materialize(l), c.materialize(l)):
            assert torch.equal(a, b)


def without_first_rows(seg, skip):
    """The segment minus its first `skip` rows, re-headed: what a later import of the rest holds."""
    from dkv import formats
    out = []
    for p in (seg.key, seg.value):
        bits, _, shape, _, _, _ = p.fields()
        heads, rows = shape[1], shape[2]
        pay = p.payload.view(heads, rows, formats.row_bytes(bits))[:, skip:].flatten()
        if bits < 16:
            sc = p.scales.view(heads, rows)[:, skip:].flatten()
            of = p.offsets.view(heads, rows)[:, skip:].flatten()
        else:
            sc = of = p.scales
        out.append(formats.PackedTensor(pay, sc, of, formats.header(bits, heads, rows - skip)))
    layer, frame, start, end, bits = seg.fields()
    return formats.Segment(out[0], out[1], formats.descriptor(layer, frame, start + skip, end, bits))


def test_single_segment_entry_points_match_the_batched_launch(cuda):
    announce('segments: dkv_export / dkv_import vs dkv_segment_batch')
    layers = 2
    chunks = kv_chunks(layers, SCHEDULE[:4], seed=15, device=cuda)
    c = fill(GPUCache(None, layers=layers, heads=HEADS, max_tokens=512), chunks, SCHEDULE[:4])
    batch = c.export_segments()
    lib = _lib.load()
    fresh = GPUCache(None, layers=layers, heads=HEADS, max_tokens=512)
    for i, seg in enumerate(c.segments):
        rb = {4: 32, 8: 64, 16: 128}[seg.bits]
        pay = torch.empty((2, 1, HEADS, seg.rows, rb), dtype=torch.uint8, device=cuda)
        meta = torch.empty((2, 2, 1, HEADS, seg.rows), dtype=torch.float32, device=cuda)
        io = _lib.SegmentIO()
        for kv in range(2):
            io.payload[kv] = pay[kv].data_ptr()
            if seg.bits < 16:
                io.offsets[kv], io.scales[kv] = meta[kv, 0].data_ptr(), meta[kv, 1].data_ptr()
        io.seg_offset, io.seg_rows, io.seg_token_start = seg.offset, seg.rows, seg.start
        io.row0, io.rows, io.bits, io.layer0, io.n_layers = 0, seg.rows, seg.bits, 1, 1
        _lib.check(lib.dkv_export(ctypes.byref(io), c.arena.data_ptr(), c.arena_bytes, layers, HEADS,
                                  _lib.stream_handle()), 'dkv_export')
        torch.cuda.synchronize()
        ref = batch[1][i]
        assert torch.equal(pay[0, 0].flatten(), ref.key.payload) and torch.equal(pay[1, 0].flatten(), ref.value.payload)
        if seg.bits < 16:
            assert torch.equal(bits_of(meta[1, 1, 0].flatten()), bits_of(ref.value.scales))
            assert torch.equal(bits_of(meta[0, 0, 0].flatten()), bits_of(ref.key.offsets))
        # the same bytes imported into layer 1 of a fresh cache's matching segment
        dst = fresh._open_segment(seg.start, seg.rows, seg.bits, seg.frame)
        io.seg_offset, io.tile_index0, io.write_tiles = dst.offset, dst.tile0, 1
        _lib.check(lib.dkv_import(ctypes.byref(io), fresh.arena.data_ptr(), fresh.arena_bytes,
                                  fresh.tiles.data_ptr(), layers, HEADS, _lib.stream_handle()), 'dkv_import')
    fresh.seen = list(c.seen)
    for a, b in zip(fresh.materialize(1), c.materialize(1)):
        assert torch.equal(a, b)
