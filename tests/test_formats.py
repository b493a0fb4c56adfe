"""The serialized formats' host side on the CPU: headers, descriptors and import checks.

Headers and descriptors are compared with the oracle's restatement of
src/kv_quantization.py:pack and src/cache_manager.py:53-58 on the same tensors;
literal bytes pin the struct layouts. Import validation runs on device='cpu'
caches and must reject every malformed segment before any kernel launch.
"""
import struct

import pytest
import torch

from dkv import formats
from dkv.gpu_cache import GPUCache
from oracle.cpu_path import MixedPrecisionCache
from oracle.kv_quantization import pack


@pytest.mark.parametrize('bits', [4, 8, 16])
@pytest.mark.parametrize('rows', [1, 24, 64])
def test_header_equals_the_quantizers(bits, rows):
    x = torch.randn(1, 5, rows, 64).to(torch.bfloat16)
    ref = pack(x, bits)
    assert torch.equal(formats.header(bits, 5, rows), ref.header)
    p = formats.PackedTensor(ref.payload, ref.scales, ref.offsets, formats.header(bits, 5, rows))
    assert p.fields() == ref.fields()
    assert (p.payload_bytes, p.metadata_bytes, p.storage_bytes) == (ref.payload_bytes, ref.metadata_bytes,
                                                                   ref.storage_bytes)
    formats.check_packed(p, bits, 5, rows)


def test_literal_header_and_descriptor_bytes():
    h = bytes(formats.header(4, 5, 64).tolist())
    assert len(h) == 64 and h[:8] == b'DKVC\x01\x04\x02\x04'
    assert struct.unpack('<4q', h[8:40]) == (1, 5, 64, 64)
    assert struct.unpack('<3Q', h[40:]) == (64, 5 * 64 * 64, 5 * 64)
    d = bytes(formats.descriptor(3, -1, 16, 80, 8).tolist())
    assert len(d) == 32 and d == struct.pack('<ii', 3, -1) + struct.pack('<qq', 16, 80) + b'\x08' + bytes(7)


def test_descriptor_equals_the_cpu_caches():
    c = MixedPrecisionCache()
    c.select(8, 4)
    x = torch.randn(1, 5, 12, 64).to(torch.bfloat16)
    c.update(x, x, 0)
    c.update(x, x, 0)
    assert torch.equal(formats.descriptor(0, 4, 12, 24, 8), c.segments[0][1].descriptor)
    assert formats.descriptor_fields(c.segments[0][1].descriptor) == (0, 4, 12, 24, 8)


def reference_segments(layers, schedule, heads=5):
    c = MixedPrecisionCache()
    g = torch.Generator().manual_seed(5)
    for bits, frame, n in schedule:
        c.select(bits, frame)
        for l in range(layers):
            x = torch.randn((1, heads, n, 64), generator=g).to(torch.bfloat16)
            c.update(x, x, l)
    return c.segments


def rejects(cache, segments, msg):
    before = (list(cache.seen), cache.arena_used, len(cache.segments))
    with pytest.raises(ValueError, match=msg):
        cache.import_segments(segments)
    assert (list(cache.seen), cache.arena_used, len(cache.segments)) == before


def test_import_rejects_malformed_segments_before_any_launch():
    segs = reference_segments(2, [(4, 0, 8), (16, 1, 6)])
    c = GPUCache(None, layers=2, heads=5, device='cpu')
    rejects(c, {0: segs[0]}, 'every layer')
    rejects(c, {0: segs[0], 1: segs[1][:1]}, 'different numbers')
    rejects(c, {0: segs[0], 1: [segs[0][0], segs[1][1]]}, 'labelled layer 0')
    rejects(c, {0: segs[0], 1: segs[1][::-1]}, 'disagree')
    wrong_heads = reference_segments(2, [(4, 0, 8)], heads=3)
    rejects(c, wrong_heads, 'does not fit')
    gap = reference_segments(2, [(4, 0, 8)])
    for l in gap:
        gap[l][0].descriptor = formats.descriptor(l, 0, 4, 12, 4)
    rejects(c, gap, 'expected to start at 0')
    relabel = reference_segments(2, [(8, 0, 8)])
    for l in relabel:
        relabel[l][0].descriptor = formats.descriptor(l, 0, 0, 8, 4)
    rejects(c, relabel, 'descriptor 4')
    fp16 = {}
    for l in range(2):
        x = torch.randn(1, 5, 8, 64).to(torch.float16)
        k = pack(x, 16)
        fp16[l] = [formats.Segment(k, k, formats.descriptor(l, 0, 0, 8, 16))]
    rejects(c, fp16, 'bf16')
    small = GPUCache(None, layers=2, heads=5, device='cpu', max_tokens=10)
    rejects(small, segs, 'context limit')


def test_export_needs_level_consecutive_layers():
    c = GPUCache(None, layers=3, heads=5, device='cpu')
    with pytest.raises(ValueError):
        c.export_segments(layers=[0, 2])
    with pytest.raises(ValueError):
        c.export_segments(layers=[3])
    c.seen = [4, 4, 0]
    with pytest.raises(ValueError, match='differ'):
        c.export_segments()
    assert c.export_segments(layers=[0, 1]) == {0: [], 1: []}
