"""The decoder's fused pointwise kernels against the torch compositions they replace.

- rope_qkv vs transformers' apply_rotary_pos_emb on the split Q/K/V views (the reference's
  patched attention forward, src/gpu_cache.py:166-172): bit-equal. Every product of two bf16
  values is exact in fp32, so rounding each product and the sum to bf16 reproduces torch's three
  bf16 ops exactly.
- cuda_rms vs torch.nn.functional.rms_norm(x) * w (src/gpu_ops.py:9-12) and activation_product vs
  silu(g) * u (src/gpu_ops.py:14-17): the kernels round at the same two points, but rsqrt / exp in
  fp32 may differ from torch's by an ulp, which can move a bf16 rounding. Tolerance: at most
  1 bf16 ulp (2^-7 relative, plus 2^-126 absolute) from the torch result everywhere, and within
  2^-8 relative + 1e-6 of a float64 evaluation of the same two-rounding formula.
"""
import pytest
import torch

from conftest import announce
from dkv import gpu_ops

pytestmark = pytest.mark.gpu


def within_one_ulp(got, ref):
    g, r = got.float(), ref.float()
    return bool(((g - r).abs() <= r.abs() * 2.0 ** -7 + 2.0 ** -126).all())


@pytest.mark.parametrize('n', [1, 17, 64])
def test_rope_qkv_equals_apply_rotary_pos_emb(cuda, n):
    announce(f'ops: rope_qkv n={n}')
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding, apply_rotary_pos_emb
    cfg = LlamaConfig(hidden_size=960, num_attention_heads=15, num_key_value_heads=5, head_dim=64,
                      rope_theta=100000.0, max_position_embeddings=8192)
    rot = LlamaRotaryEmbedding(cfg, device=cuda)
    g = torch.Generator().manual_seed(n)
    qkv = (torch.randn((1, n, 25 * 64), generator=g) * 3).to(torch.bfloat16).to(cuda)
    pos = torch.arange(1000, 1000 + n, device=cuda)[None]
    cos, sin = rot(qkv, pos)
    q, k, v = gpu_ops.rope_qkv(qkv, cos, sin, 15, 5)
    rq, rk, rv = qkv.split([960, 320, 320], dim=-1)
    rq = rq.view(1, n, 15, 64).transpose(1, 2)
    rk = rk.view(1, n, 5, 64).transpose(1, 2)
    rv = rv.view(1, n, 5, 64).transpose(1, 2)
    rq, rk = apply_rotary_pos_emb(rq, rk, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(q, rq) and torch.equal(k, rk) and torch.equal(v, rv)


@pytest.mark.parametrize('rows,dim', [(1, 960), (64, 960), (77, 64)])
def test_rms_norm_matches_torch(cuda, rows, dim):
    announce(f'ops: rms_norm {rows}x{dim}')
    g = torch.Generator().manual_seed(rows)
    x = (torch.randn((1, rows, dim), generator=g) * 4).to(torch.bfloat16).to(cuda)
    w = (torch.rand((dim,), generator=g) + 0.5).to(torch.bfloat16).to(cuda)
    got = gpu_ops.cuda_rms(x, w, 1e-5)
    ref = torch.nn.functional.rms_norm(x, (dim,), None, 1e-5) * w
    assert within_one_ulp(got, ref)
    xd = x.double()
    y = (xd * torch.rsqrt((xd * xd).mean(-1, keepdim=True) + 1e-5)).to(torch.bfloat16).double() * w.double()
    assert bool(((got.double() - y).abs() <= y.abs() * 2.0 ** -8 + 1e-6).all())


@pytest.mark.parametrize('rows,inter', [(1, 2560), (64, 2560), (5, 8)])
def test_silu_mul_matches_torch(cuda, rows, inter):
    announce(f'ops: silu_mul {rows}x{inter}')
    g = torch.Generator().manual_seed(inter + rows)
    gu = (torch.randn((1, rows, 2 * inter), generator=g) * 3).to(torch.bfloat16).to(cuda)
    gate, up = gu.chunk(2, dim=-1)
    ref = torch.nn.functional.silu(gate) * up
    joined = gpu_ops.silu_mul(gu)
    chunks = gpu_ops.activation_product(gate, up)
    separate = gpu_ops.activation_product(gate.clone(), up.clone())
    torch.cuda.synchronize()
    assert torch.equal(joined, chunks) and torch.equal(joined, separate)
    assert within_one_ulp(joined, ref)
    gd = gate.double()
    y = (gd / (1 + torch.exp(-gd))).to(torch.bfloat16).double() * up.double()
    assert bool(((joined.double() - y).abs() <= y.abs() * 2.0 ** -8 + 1e-6).all())


def test_uncovered_inputs_take_the_reference_composition(cuda):
    announce('ops: fp32 inputs')
    x = torch.randn((3, 40), device=cuda)
    w = torch.rand((40,), device=cuda)
    assert torch.equal(gpu_ops.cuda_rms(x, w, 1e-6), torch.nn.functional.rms_norm(x, (40,), None, 1e-6) * w)
    assert gpu_ops.rope_qkv(x[None], x[None, :, :64 - 24], x[None, :, :40], 1, 1) is None


@pytest.mark.parametrize('dim', [576, 960])
def test_cuda_rms_matches_upstream_reference_bounds(cuda, dim):
    """Port of tests/test_gpu_backend.py:103-109 with its own bounds (max .063, mean .001)."""
    announce(f'ops: reference rms bounds dim={dim}')
    torch.manual_seed(dim)
    x = torch.randn(1, 19, dim, device=cuda, dtype=torch.bfloat16)
    weight = torch.randn(dim, device=cuda, dtype=torch.bfloat16)
    reference = weight * (x.float() * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + 1e-5)).bfloat16()
    actual = gpu_ops.cuda_rms(x, weight, 1e-5)
    diff = (reference.float() - actual.float()).abs()
    assert diff.max() < .063 and diff.mean() < .001


def test_fused_activation_matches_upstream_reference_bounds(cuda):
    """Port of tests/test_gpu_backend.py:111-122 with its own bounds."""
    announce('ops: reference activation bounds')
    torch.manual_seed(23)
    gate = torch.randn(1, 23, 2560, device=cuda, dtype=torch.bfloat16)
    up = torch.randn_like(gate)
    expected = torch.nn.functional.silu(gate) * up
    diff = (expected.float() - gpu_ops.activation_product(gate, up).float()).abs()
    assert diff.max() < .063 and diff.mean() < .001
    joined = torch.randn(1, 23, 5120, device=cuda, dtype=torch.bfloat16)
    gate, up = joined.chunk(2, -1)
    expected = torch.nn.functional.silu(gate) * up
    assert torch.allclose(gpu_ops.activation_product(gate, up), expected, atol=.063, rtol=.01)
