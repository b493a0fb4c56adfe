"""GPUCache.append_projection (dkv_rope_pack: projection split + RoPE + pack in one launch)
against the two launches it replaces in the patched attention forward (src/gpu_cache.py:164-172):
rope_qkv, which is bit-equal to transformers' apply_rotary_pos_emb (test_gpu_ops), then append,
whose bytes equal the oracle quantizer's (test_gpu_pack). Everything must be identical: q, k, v,
the returned history length, every arena byte, the tile table and the cache's bookkeeping. The
first case also checks q, k, v against apply_rotary_pos_emb directly.

Chunks of 1, 10, 64, 100 and 130 tokens after a 10-token first append put rows across tile
boundaries (the per-row store path) as well as on them, for 4-, 8- and 16-bit segments, in
online and planned caches, with a projection whose rows are wider than the heads they hold.
"""
import pytest
import torch

from conftest import announce
from dkv import gpu_ops
from dkv.gpu_cache import GPUCache

pytestmark = pytest.mark.gpu

Q_HEADS, HEADS, LAYERS = 15, 5, 2


def rotary(cuda):
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    cfg = LlamaConfig(hidden_size=960, num_attention_heads=Q_HEADS, num_key_value_heads=HEADS, head_dim=64,
                      rope_theta=100000.0, max_position_embeddings=8192)
    return LlamaRotaryEmbedding(cfg, device=cuda)


def projection(n, past, seed, cuda, rot, pad=0):
    g = torch.Generator().manual_seed(seed)
    width = (Q_HEADS + 2 * HEADS) * 64
    wide = (torch.randn((1, n, width + pad), generator=g) * 3)
    wide[..., width - 2 * HEADS * 64 + 5] *= 8  # an outlier channel in every K head row
    wide = wide.to(torch.bfloat16).to(cuda)
    qkv = wide[..., :width]
    cos, sin = rot(qkv, torch.arange(past, past + n, device=cuda)[None])
    return qkv, cos, sin


def same_cache(a, b):
    torch.cuda.synchronize()
    assert torch.equal(a.arena, b.arena)
    assert torch.equal(a.tiles, b.tiles)
    assert a.seen == b.seen and a.host_counts == b.host_counts and a.tile_starts == b.tile_starts
    assert [(s.start, s.rows, s.bits, s.offset, s.tile0) for s in a.segments] == \
        [(s.start, s.rows, s.bits, s.offset, s.tile0) for s in b.segments]


def run_steps(a, b, steps, cuda, pad=0, direct_check=False):
    rot = rotary(cuda)
    for i, (bits, n) in enumerate(steps):
        a.select(bits, i)
        b.select(bits, i)
        for layer in range(LAYERS):
            announce(f'rope_pack: step {i} bits={bits} n={n} layer={layer} pad={pad}')
            qkv, cos, sin = projection(n, a.seen[layer], 100 * i + layer, cuda, rot, pad)
            q, k, v = gpu_ops.rope_qkv(qkv, cos, sin, Q_HEADS, HEADS)
            past_a = a.append(k, v, layer)
            got = b.append_projection(qkv, cos, sin, Q_HEADS, layer)
            assert got is not None
            q2, k2, v2, past_b = got
            torch.cuda.synchronize()
            assert past_a == past_b
            assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v, v2)
            if direct_check:
                from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
                rq, rk, rv = qkv.split([Q_HEADS * 64, HEADS * 64, HEADS * 64], dim=-1)
                rq = rq.view(1, n, Q_HEADS, 64).transpose(1, 2)
                rk = rk.view(1, n, HEADS, 64).transpose(1, 2)
                rv = rv.view(1, n, HEADS, 64).transpose(1, 2)
                rq, rk = apply_rotary_pos_emb(rq, rk, cos, sin)
                assert torch.equal(q2, rq) and torch.equal(k2, rk) and torch.equal(v2, rv)
    same_cache(a, b)


STEPS = [(16, 10), (4, 64), (8, 1), (4, 100), (16, 64), (8, 130), (4, 10)]


@pytest.mark.parametrize('pad', [0, 24])
def test_online_cache_matches_rope_then_append(cuda, pad):
    a = GPUCache(None, layers=LAYERS, heads=HEADS, max_tokens=1024)
    b = GPUCache(None, layers=LAYERS, heads=HEADS, max_tokens=1024)
    a.arena.fill_(0xA5)
    b.arena.fill_(0xA5)
    run_steps(a, b, STEPS, cuda, pad=pad, direct_check=pad == 0)


def test_planned_cache_matches_rope_then_append(cuda):
    plan = [(16, 10), (4, 64), (8, 101), (16, 64), (8, 130), (4, 10)]
    # several appends into one planned segment: (8, 1) then (8, 100) share the 101-token segment
    steps = [(16, 10), (4, 64), (8, 1), (8, 100), (16, 64), (8, 130), (4, 10)]
    a = GPUCache(plan, layers=LAYERS, heads=HEADS)
    b = GPUCache(plan, layers=LAYERS, heads=HEADS)
    a.arena.fill_(0x5A)
    b.arena.fill_(0x5A)
    run_steps(a, b, steps, cuda)


def test_attention_after_fused_append_matches(cuda):
    """The attention output over a cache filled by append_projection equals the two-launch path's."""
    a = GPUCache(None, layers=LAYERS, heads=HEADS, max_tokens=1024)
    b = GPUCache(None, layers=LAYERS, heads=HEADS, max_tokens=1024)
    rot = rotary(cuda)
    for i, (bits, n) in enumerate([(4, 64), (8, 64), (16, 64), (4, 64)]):
        a.select(bits, i)
        b.select(bits, i)
        announce(f'rope_pack: attend step {i}')
        qkv, cos, sin = projection(n, a.seen[0], i, cuda, rot)
        q, k, v = gpu_ops.rope_qkv(qkv, cos, sin, Q_HEADS, HEADS)
        out_a = a.attend(q, k, v, 0, a.append(k, v, 0))
        q2, k2, v2, past = b.append_projection(qkv, cos, sin, Q_HEADS, 0)
        out_b = b.attend(q2, k2, v2, 0, past)
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b)


def test_uncovered_inputs_return_none(cuda):
    c = GPUCache(None, layers=1, heads=HEADS, max_tokens=256)
    rot = rotary(cuda)
    qkv, cos, sin = projection(8, 0, 0, cuda, rot)
    assert c.append_projection(qkv.float(), cos, sin, Q_HEADS, 0) is None  # not bf16
    assert c.append_projection(qkv[..., :-64], cos, sin, Q_HEADS, 0) is None  # head count mismatch
    assert c.append_projection(qkv, cos[:, :4], sin[:, :4], Q_HEADS, 0) is None  # rows mismatch
    assert c.seen == [0]  # nothing was claimed
