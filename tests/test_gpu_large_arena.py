"""Arenas past 4 GiB: tiles whose bytes sit beyond 2^32 pack, reconstruct and attend like any other.

The cache holds 64 layers x 8 KV heads, so a 16-bit tile's slab is 8 MiB: 506 such tiles end
48 MiB short of 4 GiB, and the 4/8/16-bit tiles after them (the last one ragged, 37 tokens) sit
past 2^32. Every offset in the pack, reconstruct and attention kernels is 64-bit; these tests show
it on the bytes: reconstruct is bit-exact against the oracle's pack + dequantize of the same rows
(src/kv_quantization.py:41-92), and fp32-precision attention over the whole 33,957-token history
(frame chunk on the MFMA and vector kernels, decode steps on the short-chunk kernel) is within
1e-3 of the fp64 oracle, as everywhere else. A causal chunk's first n query rows see exactly what
an n-token chunk's rows see, so one fp64 oracle run over the 64-token chunk serves every n.
"""
import pytest
import torch

from conftest import announce
from dkv.gpu_cache import GPUCache
from dkv.workloads import frame_chunk_case
from oracle.attention import attention, dequant_rows
from oracle.kv_quantization import pack_rows

pytestmark = pytest.mark.gpu

LAYERS, HEADS, Q_HEADS, NQ = 64, 8, 16, 64
BITS = [16] * 506 + [4, 8, 16] * 8 + [8]
LENGTHS = [64] * (len(BITS) - 1) + [37]
PAST = sum(LENGTHS)


@pytest.fixture(scope='module')
def big(cuda):
    announce(f'arena past 4 GiB: {LAYERS} layers x {HEADS} heads, {len(BITS)} tiles, {PAST} tokens')
    case = frame_chunk_case(PAST, seed=4242, heads=HEADS, q_heads=Q_HEADS, nq=NQ)
    c = GPUCache(None, layers=LAYERS, heads=HEADS, max_tokens=PAST + NQ)
    k = case['k_hist'].to(cuda)[None].expand(LAYERS, -1, -1, -1).contiguous()
    v = case['v_hist'].to(cuda)[None].expand(LAYERS, -1, -1, -1).contiguous()
    c.append_batch(k, v, BITS, LENGTHS)
    torch.cuda.synchronize()
    del k, v
    offsets = c.tiles[:len(BITS)].cpu().view(torch.int64)[:, 0]
    beyond = int((offsets >= 2 ** 32).sum())
    assert beyond >= 10, f'only {beyond} tiles start past 2^32'  # the test covers what it claims
    dk, dv = [], []
    t0 = 0
    for b, n in zip(BITS, LENGTHS):
        for src, dst in ((case['k_hist'][:, t0:t0 + n], dk), (case['v_hist'][:, t0:t0 + n], dv)):
            dst.append(dequant_rows(*pack_rows(src, b), b))
        t0 += n
    dk, dv = torch.cat(dk, 1), torch.cat(dv, 1)
    q, kn, vn = case['q'], case['k_new'], case['v_new']
    ref = attention(q, torch.cat((dk, kn.float()), 1), torch.cat((dv, vn.float()), 1), PAST)  # [NQ, Q_HEADS, 64]
    yield c, case, dk, dv, ref, beyond
    del c
    torch.cuda.empty_cache()


@pytest.mark.parametrize('layer', [0, LAYERS - 1])
def test_reconstruct_past_4gib_is_bit_exact(big, layer):
    c, case, dk, dv, _, beyond = big
    announce(f'arena past 4 GiB: reconstruct layer {layer} ({beyond} tiles past 2^32)')
    k, v = c.materialize(layer, torch.float32)
    assert torch.equal(k[0].cpu(), dk)
    assert torch.equal(v[0].cpu(), dv)


@pytest.mark.parametrize('path,nq', [('mfma', NQ), ('vector', NQ), ('short', 1), ('auto', 4)])
def test_attention_past_4gib_within_1e3_of_fp64_oracle(big, cuda, path, nq):
    c, case, _, _, ref, _ = big
    layer = LAYERS - 1
    announce(f'arena past 4 GiB: attention layer {layer} path={path} nq={nq} past={PAST}')
    q, kn, vn = (case[x][:, :nq] for x in ('q', 'k_new', 'v_new'))
    out = c.attend(q[None].to(cuda), kn[None].to(cuda), vn[None].to(cuda), layer, PAST,
                   out_dtype=torch.float32, path=path, precision='fp32')
    torch.cuda.synchronize()
    err = (out[0].cpu().double() - ref[:nq]).abs().max().item()
    print(f'[past-4GiB] path={path} nq={nq}: max-abs {err:.3e}', flush=True)
    assert err <= 1e-3, err
