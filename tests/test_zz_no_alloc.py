"""dkv_attend_noalloc, the attention entry point that allocates nothing, against dkv_attend through
the C ABI: the same arguments give bit-identical outputs on consecutive calls (the second one
smaller, so the shared scratch buffer still holds the first call's partials), and a call whose
split partials exceed DKV_NOALLOC_SCRATCH_BYTES is refused before any launch."""
import ctypes

import pytest
import torch

from conftest import announce
from dkv import _lib
from dkv.gpu_cache import GPUCache
from dkv.workloads import frame_chunk_case

pytestmark = pytest.mark.gpu


def cache_for(case, cuda, precision):
    heads, past = case['k_hist'].shape[:2]
    nq = case['q'].shape[1]
    c = GPUCache(None, layers=1, heads=heads, max_tokens=past + nq + 64, precision=precision)
    for i, b in enumerate(case['bits']):
        n = min(64, past - 64 * i)
        c.select(b)
        c.append(case['k_hist'][None, :, 64 * i:64 * i + n].to(cuda), case['v_hist'][None, :, 64 * i:64 * i + n].to(cuda), 0)
    q, kn, vn = (case[x][None].to(cuda) for x in ('q', 'k_new', 'v_new'))
    c.select(16)
    past = c.append(kn, vn, 0)
    return c, q, kn, vn, past


def both(c, q, kn, vn, past, out_dtype, splits=0):
    """(dkv_attend output, dkv_attend_noalloc output, workspace bytes dkv_attend needed)."""
    lib = _lib.load()
    nq, hq = q.shape[2], q.shape[1]
    outs = [torch.full((1, nq, hq, 64), float('nan'), dtype=out_dtype, device=q.device) for _ in range(2)]
    a = c.attend_args(q, kn, vn, 0, past, outs[0], splits=splits)
    need = lib.dkv_attend_workspace_bytes(ctypes.byref(a))
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=q.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(lib.dkv_attend(ctypes.byref(a), _lib.stream_handle(q.device)), 'dkv_attend')
    b = c.attend_args(q, kn, vn, 0, past, outs[1], splits=splits)
    assert not b.workspace and b.workspace_bytes == 0
    _lib.check(lib.dkv_attend_noalloc(ctypes.byref(b), _lib.stream_handle(q.device)), 'dkv_attend_noalloc')
    torch.cuda.synchronize()
    return outs[0], outs[1], need


def bits_equal(x, y):
    view = torch.int16 if x.dtype == torch.bfloat16 else torch.int32
    return torch.equal(x.view(view), y.view(view))


@pytest.mark.parametrize('precision', ['bf16', 'fp32'])
def test_noalloc_equals_attend_on_consecutive_calls(cuda, precision):
    # a 64-token frame over 8128 tokens (43 splits per KV head), then a 5-token chunk over 1000
    # tokens: the second call's partials are a fraction of the first's, over the same scratch
    for past, nq, seed, out_dtype in ((8128, 64, 1, torch.float32), (1000, 5, 2, torch.bfloat16),
                                      (8128, 64, 3, torch.bfloat16)):
        announce(f'noalloc precision={precision} past={past} nq={nq} out={out_dtype}')
        case = frame_chunk_case(past, seed=seed, nq=nq)
        c, q, kn, vn, p = cache_for(case, cuda, precision)
        ref, got, need = both(c, q, kn, vn, p, out_dtype)
        assert 0 < need <= _lib.DKV_NOALLOC_SCRATCH_BYTES
        assert not torch.isnan(ref.float()).any()
        assert bits_equal(ref, got), (ref.float() - got.float()).abs().max().item()


def test_noalloc_single_split_needs_no_scratch(cuda):
    announce('noalloc one split')
    case = frame_chunk_case(300, seed=4, nq=16)
    c, q, kn, vn, p = cache_for(case, cuda, 'bf16')
    ref, got, need = both(c, q, kn, vn, p, torch.float32, splits=1)
    assert need == 0 and bits_equal(ref, got)


def test_noalloc_refuses_partials_beyond_the_scratch(cuda):
    """fp32 precision, a 130-token chunk and 128 explicit splits: 5 x 128 x 390 rows of 264 bytes of
    partials, past the 16 MiB scratch. The call returns DKV_EINVAL before launching: the output
    keeps its NaN fill."""
    announce('noalloc oversize refusal')
    case = frame_chunk_case(8128, seed=5, nq=130)
    c, q, kn, vn, p = cache_for(case, cuda, 'fp32')
    lib = _lib.load()
    out = torch.full((1, 130, 15, 64), float('nan'), device=cuda)
    a = c.attend_args(q, kn, vn, 0, p, out, splits=128)
    assert lib.dkv_attend_workspace_bytes(ctypes.byref(a)) > _lib.DKV_NOALLOC_SCRATCH_BYTES
    rc = lib.dkv_attend_noalloc(ctypes.byref(a), _lib.stream_handle(cuda))
    assert rc == _lib.DKV_EINVAL
    assert b'scratch' in lib.dkv_last_error()
    torch.cuda.synchronize()
    assert torch.isnan(out).all()
