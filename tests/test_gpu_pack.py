"""Pack kernel parity: arena bytes, offsets and scales bit-exact against the oracle quantizer."""
import numpy as np
import pytest
import torch

from arena_view import segment_rows
from conftest import announce
from dkv.gpu_cache import GPUCache
from dkv.workloads import bit_schedule, outlier_values, pack_volume
from oracle.attention import dequant_rows
from oracle.kv_quantization import pack_rows

pytestmark = pytest.mark.gpu


def assert_rows_match(arena, seg, layer, kv, head, layers, heads, x, upto=None):
    """x: [rows, 64] bf16 CPU source rows of this (layer, kv, head) in the segment."""
    payload, meta = segment_rows(arena, seg, layer, kv, head, layers, heads, upto)
    ref_p, ref_off, ref_sc = pack_rows(x, seg.bits)
    assert np.array_equal(payload, ref_p.numpy()), (layer, kv, head, seg.bits)
    if seg.bits < 16:
        assert np.array_equal(meta[:, 0].view(np.uint32), ref_off.numpy().view(np.uint32))
        assert np.array_equal(meta[:, 1].view(np.uint32), ref_sc.numpy().view(np.uint32))


@pytest.mark.parametrize('bits', [4, 8, 16])
def test_plan_segment_bitexact_with_strided_v(cuda, bits):
    announce(f'pack plan segment bits={bits} n=150 strided V')
    g = torch.Generator().manual_seed(100 + bits)
    layers, heads, n = 2, 5, 150
    c = GPUCache([(bits, n)], layers=layers, heads=heads)
    c.select(bits)
    src = []
    for layer in range(layers):
        k = outlier_values((heads, n, 64), g, 0)
        v = outlier_values((n, heads, 64), g, 1)  # stored token-major, viewed head-major
        c.append(k[None].to(cuda), v.to(cuda).transpose(0, 1)[None], layer)
        src.append((k, v.transpose(0, 1)))
    torch.cuda.synchronize()
    arena = c.arena.cpu().numpy()
    seg = c.segments[0]
    for layer in range(layers):
        for kv in range(2):
            for head in range(heads):
                assert_rows_match(arena, seg, layer, kv, head, layers, heads, src[layer][kv][head])


def test_ties_constants_and_extremes(cuda):
    announce('pack ties/constant rows')
    rows = torch.zeros(64, 64)
    rows[0, :16] = torch.tensor([0.0, 15.0] + [k + 0.5 for k in range(14)])
    rows[0, 16:] = 7.0
    rows[1, :] = -2.5  # constant row: scale 1, codes 0
    ties8 = [-3.0 + 2.0 * (k + 0.5) for k in range(60)]
    rows[2] = torch.tensor([-3.0, 507.0] + ties8 + [1.0, 1.0])
    rows[3] = torch.linspace(-3e4, 3e4, 64)
    rows[4] = torch.tensor([1e-30 * i for i in range(64)])  # tiny span
    rows[5] = torch.tensor([1e-39 * i for i in range(64)])  # fp32 subnormal values and scale
    rows[6] = torch.linspace(-1e38, 1e38, 64)  # span near the top of the fp32 range
    g = torch.Generator().manual_seed(4)
    rows[7:] = torch.randn(57, 64, generator=g) * torch.logspace(-3, 3, 57)[:, None]
    x = rows.to(torch.bfloat16)
    for bits in (4, 8):
        c = GPUCache([(bits, 64)], layers=1, heads=1)
        c.select(bits)
        c.append(x[None, None].to(cuda), x[None, None].to(cuda), 0)
        torch.cuda.synchronize()
        arena = c.arena.cpu().numpy()
        for kv in range(2):
            assert_rows_match(arena, c.segments[0], 0, kv, 0, 1, 1, x)


def test_online_mixed_appends_reconstruct_exactly(cuda):
    announce('pack online mixed appends + reconstruct fp32/bf16')
    g = torch.Generator().manual_seed(7)
    c = GPUCache(None, layers=1, heads=5, max_tokens=1024)
    ks, vs = [], []
    for bits, n in [(4, 79), (8, 93), (4, 88), (16, 71), (8, 1), (4, 64)]:
        k = outlier_values((5, n, 64), g, 0)
        v = outlier_values((5, n, 64), g, 0)
        c.select(bits)
        c.append(k[None].to(cuda), v[None].to(cuda), 0)
        for src, dst in ((k, ks), (v, vs)):
            p, off, sc = pack_rows(src, bits)
            dst.append(dequant_rows(p, off, sc, bits))
    rk, rv = c.materialize(0, out_dtype=torch.float32)
    assert torch.equal(rk[0].cpu(), torch.cat(ks, 1)) and torch.equal(rv[0].cpu(), torch.cat(vs, 1))
    bk, bv = c.materialize(0)
    assert torch.equal(bk[0].cpu(), torch.cat(ks, 1).to(torch.bfloat16))
    assert torch.equal(bv[0].cpu(), torch.cat(vs, 1).to(torch.bfloat16))


@pytest.mark.parametrize('layers,frames', [(4, 16), (32, 96)])
def test_batched_volume_bitexact(cuda, layers, frames):
    announce(f'pack batch volume layers={layers} frames={frames}')
    vol = pack_volume(seed=11, layers=layers, frames=frames)
    heads = 5
    c = GPUCache(None, layers=layers, heads=heads, max_tokens=frames * 64)
    c.append_batch(vol['k'].to(cuda), vol['v'].to(cuda), vol['bits'], [64] * frames)
    torch.cuda.synchronize()
    assert c.seen == [frames * 64] * layers
    arena = c.arena.cpu().numpy()
    # Oracle over the whole volume per width, then compare every row.
    for bits in (4, 8, 16):
        frames_b = [f for f in range(frames) if vol['bits'][f] == bits]
        if not frames_b:
            continue
        for kv, src in enumerate((vol['k'], vol['v'])):
            x = torch.stack([src[:, :, 64 * f:64 * f + 64] for f in frames_b])  # [F, L, H, 64, 64]
            ref_p, ref_off, ref_sc = pack_rows(x, bits)
            for i, f in enumerate(frames_b):
                seg = c.segments[f]
                assert seg.bits == bits
                for layer in range(layers):
                    for head in range(heads):
                        payload, meta = segment_rows(arena, seg, layer, kv, head, layers, heads)
                        assert np.array_equal(payload, ref_p[i, layer, head].numpy())
                        if bits < 16:
                            assert np.array_equal(meta[:, 0].view(np.uint32),
                                                  ref_off[i, layer, head].numpy().view(np.uint32))
                            assert np.array_equal(meta[:, 1].view(np.uint32),
                                                  ref_sc[i, layer, head].numpy().view(np.uint32))
    tiles = c.tiles.cpu().numpy()[:frames]
    starts = tiles[:, 8:12].copy().view(np.int32).ravel()
    assert starts.tolist() == [64 * f for f in range(frames)]
    assert tiles[:, 14].tolist() == vol['bits']
