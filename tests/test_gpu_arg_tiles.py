"""Tile descriptors carried in the launch's argument block (dkv_attn_args.tiles_host).

GPUCache keeps a host copy of its tile table and passes it with every attention call that has no
device step pair; the frame-chunk kernel then reads the history's descriptors beside its arguments
instead of waiting on the device table (for histories of at most DKV_ARG_TILES tiles; the
short-chunk kernel reads the device table either way). The copy must equal the
device table entry for entry whichever way a cache gets its segments (online appends of any length,
plans, forks, resets, imports), and a launch must give the same bits with or without it."""
import ctypes

import pytest
import torch

from conftest import announce
from dkv import _lib
from dkv.gpu_cache import TILE_DTYPE, GPUCache
from dkv.workloads import frame_chunk_case

pytestmark = pytest.mark.gpu


def assert_mirror(c):
    n = len(c.tile_starts)
    torch.cuda.synchronize()
    dev = c.tiles[:n].cpu().numpy().copy().view(TILE_DTYPE).reshape(-1)
    assert dev.tobytes() == c.tiles_host[:n].tobytes()


def append_all(c, bits, k, v):
    c.select(bits)
    for layer in range(c.layers):
        c.append(k, v, layer)


def test_host_tile_table_equals_the_device_table(cuda):
    announce('host tile table: online appends, fork, reset, plan, import')
    g = torch.Generator().manual_seed(3)

    def kv(n):
        return (torch.randn(1, 3, n, 64, generator=g).bfloat16().to(cuda) for _ in range(2))

    c = GPUCache(None, layers=2, heads=3, max_tokens=1024)
    for bits, n in ((4, 64), (8, 70), (16, 5), (4, 130), (8, 64)):
        append_all(c, bits, *kv(n))
    assert_mirror(c)
    exported = c.export_segments()
    f = c.fork()
    append_all(f, 8, *kv(20))
    assert_mirror(f)
    c.reset()
    append_all(c, 16, *kv(90))
    assert_mirror(c)
    p = GPUCache([(4, 100), (8, 64), (16, 30)], layers=2, heads=3)
    for bits, n in ((4, 100), (8, 64), (16, 30)):
        append_all(p, bits, *kv(n))
    assert_mirror(p)
    imported = GPUCache(None, layers=2, heads=3, max_tokens=1024)
    imported.import_segments(exported)
    assert_mirror(imported)


def run(c, q, kn, vn, past, path, precision, with_table, splits=0):
    lib = _lib.load()
    out = torch.full((1, q.shape[2], q.shape[1], 64), float('nan'), dtype=torch.float32, device=q.device)
    a = c.attend_args(q, kn, vn, 0, past, out, path=path, precision=precision, splits=splits)
    if not with_table:
        a.tiles_host = None
    need = lib.dkv_attend_workspace_bytes(ctypes.byref(a))
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=q.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(lib.dkv_attend(ctypes.byref(a), _lib.stream_handle(q.device)), 'dkv_attend')
    torch.cuda.synchronize()
    return out


SHAPES = [(2000, 64), (8128, 64), (8128, 1), (700, 4), (70, 37)]
# the short-chunk kernel takes at most 16 query rows per KV head (3 * nq <= 16 with 3-way GQA)
CASES = [(past, nq, path) for past, nq in SHAPES for path in ('auto', 'mfma', 'short')
         if path != 'short' or 3 * nq <= 16]


@pytest.mark.parametrize('past,nq,path', CASES)
@pytest.mark.parametrize('precision', ['bf16', 'fp32'])
def test_descriptors_in_the_argument_block_give_the_same_bits(cuda, past, nq, path, precision):
    """Histories of 2 to 127 tiles (mixed widths, a partial last tile at 2000 and 700), frame
    chunks and decode steps on the frame-chunk and short-chunk kernels, one split and the default
    plan: the same output bits with the host copy passed as without it."""
    announce(f'argument-block descriptors past={past} nq={nq} path={path} precision={precision}')
    case = frame_chunk_case(past, seed=past + nq, nq=nq)
    heads = case['k_hist'].shape[0]
    c = GPUCache(None, layers=1, heads=heads, max_tokens=past + nq + 64, precision=precision)
    for i, b in enumerate(case['bits']):
        n = min(64, past - 64 * i)
        c.select(b)
        c.append(case['k_hist'][None, :, 64 * i:64 * i + n].to(cuda),
                 case['v_hist'][None, :, 64 * i:64 * i + n].to(cuda), 0)
    q, kn, vn = (case[x][None].to(cuda) for x in ('q', 'k_new', 'v_new'))
    c.select(16)
    p0 = c.append(kn, vn, 0)
    assert 0 < c._tiles_before(p0) <= _lib.DKV_ARG_TILES
    assert_mirror(c)
    for splits in (0, 1):
        a = run(c, q, kn, vn, p0, path, precision, True, splits)
        b = run(c, q, kn, vn, p0, path, precision, False, splits)
        assert not torch.isnan(a).any()
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), splits


@pytest.mark.parametrize('nq,path', [(64, 'mfma'), (1, 'short')])
def test_histories_past_the_argument_block_use_the_device_table(cuda, nq, path):
    """A history of more than DKV_ARG_TILES tiles (here 200) runs from the device table even when
    the host copy is passed: the output equals the one without it, and the fp64 oracle."""
    from oracle.attention import attention, dequant_rows
    from oracle.kv_quantization import pack_rows
    announce(f'argument-block descriptors: 200-tile history nq={nq} path={path}')
    past = 200 * 64
    case = frame_chunk_case(past, seed=5, nq=nq, heads=1, q_heads=3)
    c = GPUCache(None, layers=1, heads=1, max_tokens=past + nq + 64, precision='fp32')
    dk, dv = [], []
    for i, b in enumerate(case['bits']):
        k = case['k_hist'][:, 64 * i:64 * i + 64]
        v = case['v_hist'][:, 64 * i:64 * i + 64]
        c.select(b)
        c.append(k[None].to(cuda), v[None].to(cuda), 0)
        dk.append(dequant_rows(*pack_rows(k, b), b))
        dv.append(dequant_rows(*pack_rows(v, b), b))
    q, kn, vn = (case[x][None].to(cuda) for x in ('q', 'k_new', 'v_new'))
    c.select(16)
    p0 = c.append(kn, vn, 0)
    assert c._tiles_before(p0) == 200 > _lib.DKV_ARG_TILES
    a = run(c, q, kn, vn, p0, path, 'fp32', True)
    b = run(c, q, kn, vn, p0, path, 'fp32', False)
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    ref = attention(case['q'], torch.cat(dk + [case['k_new'].float()], 1),
                    torch.cat(dv + [case['v_new'].float()], 1), past)
    assert (a[0].cpu().double() - ref).abs().max().item() <= 1e-3
