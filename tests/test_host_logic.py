"""GPUCache bookkeeping on the CPU (device='cpu' arenas; no kernel runs)."""
import os
import pytest
import torch

from dkv import _lib
from dkv.gpu_cache import GPUCache, GraphSteps, _Segment, segment_bytes, worst_case_arena_bytes, \
    write_job_sources, write_step_jobs


def test_rejects_bad_geometry_and_plans():
    with pytest.raises(ValueError):
        GPUCache(dim=128, device='cpu')
    with pytest.raises(ValueError):
        GPUCache([(5, 10)], device='cpu')
    with pytest.raises(ValueError):
        GPUCache([(4, -1)], device='cpu')


def test_plan_layout_matches_reference_plan_tuples():
    c = GPUCache([(16, 15), (4, 67), (8, 23), (4, 10)], layers=2, heads=3, device='cpu')
    # (start, end, bits, row within width class) as src/gpu_cache.py:25-29 builds them
    assert c.plan == [(0, 15, 16, 0), (15, 82, 4, 0), (82, 105, 8, 0), (105, 115, 4, 67)]
    assert c.host_counts == {4: 77, 8: 23, 16: 15}
    assert c.capacity == 115
    assert c.tile_starts == [0, 15, 79, 82, 105]
    offs = [s.offset for s in c.segments]
    sizes = [segment_bytes(s.rows, s.bits, 2, 3) for s in c.segments]
    assert offs == [sum(sizes[:i]) for i in range(4)]
    assert c.arena_used == sum(sizes) == c.arena_bytes
    assert c.codes.tolist() == [16] * 15 + [4] * 67 + [8] * 23 + [4] * 10
    assert c.rows.tolist()[:16] == list(range(15)) + [0]
    assert c.rows.tolist()[105:] == list(range(67, 77))


def test_append_requires_a_device_tensor():
    c = GPUCache(None, layers=1, device='cpu')
    with pytest.raises(ValueError):
        c.append(torch.zeros(1, 3, 4, 64), torch.zeros(1, 3, 4, 64), 0)
    with pytest.raises(ValueError):
        c.append(torch.zeros(2, 3, 4, 64), torch.zeros(2, 3, 4, 64), 0)


def test_online_arena_holds_any_mix():
    c = GPUCache(None, layers=4, heads=5, max_tokens=512, device='cpu')
    assert c.arena_bytes == worst_case_arena_bytes(512, 4, 5)
    # 512 one-token 16-bit segments, the costliest cut, still fit
    assert 512 * segment_bytes(1, 16, 4, 5) <= c.arena_bytes
    assert c.caps[16] >= 512 and c.caps[4] >= c.caps[8] >= c.caps[16]


def test_fork_copies_host_state_and_shares_storage():
    c = GPUCache([(4, 20), (16, 10)], layers=1, device='cpu')
    b = c.fork()
    assert b.arena is c.arena and b.tiles is c.tiles
    assert b.seen is not c.seen and b.plan is not c.plan and b.segments is not c.segments
    assert b.pending_bits == 16
    b.seen[0] = 5
    assert c.seen[0] == 0


def test_reserve_grows_only_the_caller():
    c = GPUCache(None, layers=1, heads=3, max_tokens=256, arena_bytes=4096, device='cpu')
    b = c.fork()
    old = c.arena
    b.reserve(16, 200)
    assert b.arena is not old and b.arena_bytes >= segment_bytes(200, 16, 1, 3)
    assert c.arena is old and c.arena_bytes == 4096


def test_accounting_reference_identities():
    c = GPUCache([(4, 64), (8, 64), (16, 64)], layers=2, heads=5, device='cpu')
    c.seen = [192, 192]
    a = c.accounting()
    assert a['payload_bytes'] == 2 * 2 * 5 * 64 * (64 * 4 // 8 + 64 * 8 // 8 + 64 * 16 // 8)
    assert a['quantization_metadata_bytes'] == 2 * 2 * 5 * 8 * 128
    assert a['gpu_cache_used_bytes'] == a['payload_bytes'] + a['quantization_metadata_bytes'] + a['token_mapping_bytes']
    assert a['precision_token_counts'] == {4: 64, 8: 64, 16: 64}
    assert a['gpu_cache_allocated_bytes'] >= a['arena_used_bytes']
    # the reference's 5 bytes per token (src/gpu_cache.py:143); the tile table is reported apart
    assert a['used_tokens'] == 192 and a['token_mapping_bytes'] == 5 * 192
    assert a['tile_table_bytes'] == 3 * 16


def test_graph_step_jobs_encode_like_ctypes_pack_jobs():
    """The numpy view a graph step writes into its pinned buffer holds the bytes of the ctypes
    PackJob array the C ABI reads (the layout, field order and per-layer values)."""
    import ctypes
    import numpy as np
    layers = 3
    assert GraphSteps.JOB.itemsize == ctypes.sizeof(_lib.PackJob)
    k = torch.zeros(1, 5, 64, 64, dtype=torch.bfloat16)
    v = torch.zeros(1, 64, 5, 64, dtype=torch.bfloat16).transpose(1, 2)  # strided V
    kv = [(k, v), None, (v, k)]
    buf = np.zeros(layers * GraphSteps.JOB.itemsize, dtype=np.uint8)
    jobs = buf.view(GraphSteps.JOB)
    write_job_sources(jobs, kv)
    for seg, past, n, write in ((_Segment(128, 64, 4, 4096, 2), 128, 64, 1),
                                (_Segment(100, 101, 8, 1 << 20, 3), 164, 37, 0)):
        write_step_jobs(jobs, seg, past, n, write)
        ref = (_lib.PackJob * layers)()
        for l, pair in enumerate(kv):
            kp, vp, ks, vs = (pair[0].data_ptr(), pair[1].data_ptr(), pair[0].stride(), pair[1].stride()) if pair \
                else (0, 0, (0, 0, 0, 0), (0, 0, 0, 0))
            ref[l] = _lib.PackJob(kp, vp, ks[1], ks[2], vs[1], vs[2], seg.offset, seg.rows, seg.start,
                                  past - seg.start, n, l, seg.bits, seg.tile0, write if l == 0 else 0)
        assert buf.tobytes() == bytes(ref)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus above 1 exits with status 2 and a JSON line that says so."""
    import json
    import subprocess
    import sys
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(repo, 'bench.py'), '--gpus', '2'], cwd=repo,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2, r.stderr
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert 'one GPU' in line['error']


def test_graph_steps_refuse_to_grow_the_arena():
    """A captured graph recorded the arena's address: a step whose segment does not fit the arena
    raises instead of growing it (a grown arena would leave the recorded launches on freed memory),
    and steps refuse to run once the cache holds another arena."""
    c = GPUCache(None, layers=2, heads=5, max_tokens=4096, arena_bytes=1 << 16, device='cpu')
    steps = c.begin_graph_steps(64)
    c.select(16)
    arena = c.arena
    with pytest.raises(ValueError, match='cannot grow the arena'):
        steps.step()
    assert c.arena is arena and c.arena_bytes == 1 << 16 and c.segments == []
    c.end_graph_steps()
    c.reserve(16, 2048)  # an ordinary reserve() may grow it
    assert c.arena is not arena
    with pytest.raises(ValueError, match='no longer holds'):
        c.begin_graph_steps(64, steps=steps)
        steps.step()


def test_unsupported_dtypes_are_rejected():
    """The kernels store bf16 or fp32 only: fp16 caches and outputs raise instead of receiving
    bf16 bit patterns."""
    with pytest.raises(ValueError, match='dtype'):
        GPUCache(None, layers=1, device='cpu', dtype=torch.float16)
    c = GPUCache(None, layers=1, heads=1, max_tokens=64, device='cpu', dtype=torch.float32)
    with pytest.raises(ValueError, match='dtype'):
        c.materialize(0, out_dtype=torch.float16)


@pytest.mark.parametrize('n_segs,ok', [(16, True), (17, False)])
def test_chunk_segment_limit(n_segs, ok):
    """attend_args accepts exactly DKV_MAX_CHUNK_SEGS segments (17 bounds) and rejects one more."""
    c = GPUCache(None, layers=1, heads=1, max_tokens=128, device='cpu')
    nq = 32
    q = torch.zeros(1, 3, nq, 64, dtype=torch.bfloat16)
    kv = torch.zeros(1, 1, nq, 64, dtype=torch.bfloat16)
    out = torch.zeros(1, nq, 3, 64, dtype=torch.bfloat16)
    bounds = list(range(0, 2 * n_segs, 2))[:n_segs] + [nq]
    assert len(bounds) == n_segs + 1
    if ok:
        a = c.attend_args(q, kv, kv, 0, 0, out, bounds)
        assert a.n_segs == n_segs and list(a.seg_bounds)[:n_segs + 1] == bounds
    else:
        with pytest.raises(ValueError, match='at most 16'):
            c.attend_args(q, kv, kv, 0, 0, out, bounds)


def test_pipelined_frames_take_a_quarter_of_the_split_cap(monkeypatch):
    """StreamingDecoder.group_split_count: a quarter of the library's default cap, CUs // (KV heads x
    192-row groups), at least 1; group_splits overrides it."""
    import types
    from dkv.streaming import StreamingDecoder
    monkeypatch.setattr(torch.cuda, 'get_device_properties', lambda dev: types.SimpleNamespace(multi_processor_count=256))

    def count(heads, kv_heads, chunk, group_splits=None):
        cfg = types.SimpleNamespace(num_attention_heads=heads, num_key_value_heads=kv_heads)
        fake = types.SimpleNamespace(config=cfg, group_splits=group_splits, device='cuda:0')
        return StreamingDecoder.group_split_count(fake, chunk)

    assert count(15, 5, 64) == 12  # 256 // 5 = 51 splits, a quarter of it
    assert count(15, 5, 16) == 12  # the 16-token prefix: still one 192-row group
    assert count(32, 4, 64) == 5   # 8 GQA heads x 64 tokens = 512 rows, 3 row groups: 256 // 12 // 4
    assert count(64, 64, 64) == 1  # never below one split
    assert count(15, 5, 64, group_splits=7) == 7


def test_mfma_tiled_layout_formula_and_inverse():
    """dkv_linear's tiled layout as include/dkv.h states it: element (r, c) of an [R, K] matrix at
    ((r / 16) * (K / 64) + c / 64) * 1024 + (c / 32 % 2) * 512 + ((c / 8 % 4) * 16 + r % 16) * 8
    + c % 8, rows rounded up to 16 with zeros; checked element by element on a 40 x 192 matrix of
    distinct values, and mfma_untiled inverts it."""
    from dkv import gpu_ops
    R, K = 40, 192
    t = torch.arange(R * K, dtype=torch.float32).view(R, K)
    tiled = gpu_ops.mfma_tiled(t)
    assert tiled.shape == (48, K) and tiled.is_contiguous()
    flat = tiled.view(-1)
    r = torch.arange(R).view(R, 1)
    c = torch.arange(K).view(1, K)
    off = ((r // 16) * (K // 64) + c // 64) * 1024 + (c // 32 % 2) * 512 + ((c // 8 % 4) * 16 + r % 16) * 8 + c % 8
    assert torch.equal(flat[off], t)
    assert int(off.max()) < 48 * K and len(set(off.view(-1).tolist())) == R * K
    pad = torch.ones(48 * K, dtype=torch.bool)
    pad[off.view(-1)] = False
    assert bool((flat[pad] == 0).all())  # the padding rows are zeros
    assert torch.equal(gpu_ops.mfma_untiled(tiled, R), t)
