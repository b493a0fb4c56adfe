"""libdkv against the committed golden fixtures (tests/golden/*.npz), without the oracle.

pack_rows.npz: the 64 rows appended as one K/V segment of one head must give the fixture's
payload, offsets and scales bit for bit at 4, 8 and 16 bits, and the segment's export must carry
the fixture's PackedTensor header and bytes. attention_chunk.npz: the history appended tile by
tile at the fixture's widths, then the 12-token chunk (and the same tokens as 3 candidates of 5, 3 and
4 tokens, a block-diagonal batch) attended with precision='fp32', must be
within 1e-3 (max-abs) of the stored fp64 oracle output; with precision='bf16' (the reference
kernel's bf16 rounding of K, V and p) within the reference's own scenario tolerance,
atol 0.035 + rtol 0.015 (tests/test_gpu_backend.py:82-101).
"""
import os

import numpy as np
import pytest
import torch

from arena_view import segment_rows
from conftest import announce
from dkv.gpu_cache import GPUCache

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')


def load(name):
    return np.load(os.path.join(GOLDEN, name))


def bf16_tensor(u16):
    return torch.from_numpy(u16.view(np.int16).copy()).view(torch.bfloat16)


@pytest.mark.parametrize('bits', [4, 8, 16])
def test_pack_matches_golden_bytes(cuda, bits):
    announce(f'golden pack rows bits={bits}')
    d = load('pack_rows.npz')
    x = bf16_tensor(d['x'])  # [64 tokens, 64]
    c = GPUCache(None, layers=1, heads=1, max_tokens=128)
    c.select(bits)
    c.append(x[None, None].to(cuda), x.flip(0)[None, None].to(cuda), 0)
    torch.cuda.synchronize()
    arena = c.arena.cpu().numpy()
    seg = c.segments[0]
    for kv, order in ((0, slice(None)), (1, slice(None, None, -1))):
        payload, meta = segment_rows(arena, seg, 0, kv, 0, 1, 1)
        assert np.array_equal(payload, d[f'payload{bits}'][order]), kv
        if bits < 16:
            assert np.array_equal(meta[:, 0].view(np.uint32), d[f'offset{bits}'][order]), kv
            assert np.array_equal(meta[:, 1].view(np.uint32), d[f'scale{bits}'][order]), kv
    seg_out = c.export_segments()[0][0]
    key = seg_out.key
    i = [j for j, (b, r) in enumerate(zip(d['header_bits'], d['header_rows'])) if b == bits and r == 64][0]
    assert np.array_equal(key.header.cpu().numpy(), d['header'][i])
    assert np.array_equal(key.payload.cpu().numpy().reshape(64, -1), d[f'payload{bits}'])
    if bits < 16:
        assert np.array_equal(key.offsets.cpu().numpy().view(np.uint32), d[f'offset{bits}'])
        assert np.array_equal(key.scales.cpu().numpy().view(np.uint32), d[f'scale{bits}'])


@pytest.mark.parametrize('candidates', [False, True])
@pytest.mark.parametrize('precision', ['fp32', 'bf16'])
def test_attention_matches_golden_output(cuda, precision, candidates):
    announce(f'golden attention chunk precision={precision} candidates={candidates}')
    d = load('attention_chunk.npz')
    k_hist, v_hist = bf16_tensor(d['k_hist']), bf16_tensor(d['v_hist'])
    H, past = k_hist.shape[:2]
    c = GPUCache(None, layers=1, heads=H, max_tokens=256)
    t0 = 0
    for b, n in zip(d['bits'].tolist(), d['tiles'].tolist()):
        c.select(b)
        c.append(k_hist[None, :, t0:t0 + n].to(cuda), v_hist[None, :, t0:t0 + n].to(cuda), 0)
        t0 += n
    assert t0 == past
    q, kn, vn = (bf16_tensor(d[x])[None].to(cuda) for x in ('q', 'k_new', 'v_new'))
    c.select(16)
    p = c.append(kn, vn, 0)
    assert p == past
    segments = d['cand_bounds'].tolist() if candidates else None
    out = c.attend(q, kn, vn, 0, p, out_dtype=torch.float32, segments=segments,
                   precision=precision)[0].cpu().double()
    ref = torch.from_numpy(d['out_cand' if candidates else 'out']).double()
    err = (out - ref).abs()
    if precision == 'fp32':
        assert err.max().item() <= 1e-3, err.max().item()
    else:
        assert bool((err <= 0.035 + 0.015 * ref.abs()).all()), err.max().item()
