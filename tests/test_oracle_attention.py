"""Pins oracle/attention.py on the CPU."""
import math

import pytest
import torch

from oracle.attention import attention, dequant_rows, reference_semantics, visible_mask
from oracle.kv_quantization import pack, pack_rows, unpack


def loop_attention(q, k, v, past, scale):
    """Pure-Python triple loop: softmax(scale q.k) v, causal chunk, kv head = qh // G."""
    hq, nq, d = q.shape
    g = hq // k.shape[0]
    out = [[[0.0] * d for _ in range(hq)] for _ in range(nq)]
    for qh in range(hq):
        kh = qh // g
        for m in range(nq):
            keys = range(past + m + 1)
            s = [scale * sum(q[qh, m, i].item() * k[kh, t, i].item() for i in range(d)) for t in keys]
            mx = max(s)
            e = [math.exp(x - mx) for x in s]
            z = sum(e)
            for i in range(d):
                out[m][qh][i] = sum(e[t] * v[kh, t, i].item() for t in keys) / z
    return torch.tensor(out, dtype=torch.float64)


def test_matches_python_loop():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(4, 3, 8, generator=g)
    k = torch.randn(2, 7, 8, generator=g)
    v = torch.randn(2, 7, 8, generator=g)
    got = attention(q, k, v, past=4, scale=0.3)
    assert torch.allclose(got, loop_attention(q, k, v, 4, 0.3), atol=1e-12)


def test_identical_keys_give_mean_of_visible_values():
    g = torch.Generator().manual_seed(6)
    q = torch.randn(3, 5, 64, generator=g)
    k = torch.randn(1, 1, 64, generator=g).expand(1, 12, 64)
    v = torch.randn(1, 12, 64, generator=g)
    out = attention(q, k, v, past=7)
    for m in range(5):
        expect = v[0, :8 + m].double().mean(0)
        assert torch.allclose(out[m], expect.expand(3, 64), atol=1e-12)


def test_gqa_head_map_uses_qh_div_group():
    q = torch.randn(15, 4, 64)
    k = torch.randn(5, 10, 64)
    v = torch.arange(5, dtype=torch.float32)[:, None, None].expand(5, 10, 64)
    out = attention(q, k, v, past=6)
    for qh in range(15):
        assert torch.allclose(out[:, qh], torch.full((4, 64), float(qh // 3), dtype=torch.float64))


def test_segments_equal_separate_calls():
    g = torch.Generator().manual_seed(8)
    past, lens = 20, [3, 5, 2]
    nq = sum(lens)
    q = torch.randn(6, nq, 64, generator=g)
    k = torch.randn(2, past + nq, 64, generator=g)
    v = torch.randn(2, past + nq, 64, generator=g)
    bounds = [0, 3, 8, 10]
    got = attention(q, k, v, past, segments=bounds)
    for c in range(3):
        lo, hi = bounds[c], bounds[c + 1]
        kc = torch.cat((k[:, :past], k[:, past + lo:past + hi]), 1)
        vc = torch.cat((v[:, :past], v[:, past + lo:past + hi]), 1)
        alone = attention(q[:, lo:hi], kc, vc, past)
        assert torch.allclose(got[lo:hi], alone, atol=1e-12)


def test_visible_mask_shape_and_causality():
    m = visible_mask(3, 4)
    assert m.shape == (4, 7) and m[:, :3].all()
    assert m[0, 3] and not m[0, 4] and m[3, 6]


def test_dequant_rows_equals_unpack():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(3, 10, 64, generator=g)
    for bits in (4, 8):
        payload, off, sc = pack_rows(x, bits)
        ref = unpack(pack(x.view(1, 3, 10, 64), bits), torch.float32).view(3, 10, 64)
        assert torch.equal(dequant_rows(payload, off, sc, bits), ref)


@pytest.mark.parametrize('query_length', [1, 77])
def test_reference_scenario_semantics_within_reference_tolerance(query_length):
    # tests/test_gpu_backend.py:157-176: 4-bit 501 + 8-bit 498 history, 5 KV / 15 Q heads.
    torch.manual_seed(97)
    hist = []
    for bits, n in [(4, 501), (8, 498)]:
        x = torch.randn(2, 5, n, 64).bfloat16()
        hist.append(torch.stack([unpack(pack(x[i:i + 1], bits), torch.float32)[0] for i in range(2)]))
    hk = torch.cat([h[0] for h in hist], 1)
    hv = torch.cat([h[1] for h in hist], 1)
    n = query_length
    q = torch.randn(15, n, 64).bfloat16()
    kn, vn = torch.randn(5, n, 64).bfloat16(), torch.randn(5, n, 64).bfloat16()
    k = torch.cat((hk, kn.float()), 1)
    v = torch.cat((hv, vn.float()), 1)
    exact = attention(q, k, v, past=hk.shape[1])
    emulated = reference_semantics(q, k, v, past=hk.shape[1])
    assert torch.allclose(emulated.double(), exact, atol=.035, rtol=.015)


def _closed_form(q, k, v, past):
    """bf16(exp(s - max)) @ bf16(V) / sum(exp(s - max)), one pass over all keys."""
    g = q.shape[0] // k.shape[0]
    kb = k.bfloat16().float().repeat_interleave(g, 0)
    vb = v.bfloat16().float().repeat_interleave(g, 0)
    s = (q.float() @ kb.transpose(1, 2)) * 0.125
    s = s.masked_fill(~visible_mask(past, q.shape[1]), float('-inf'))
    p = torch.exp(s - s.amax(-1, keepdim=True))
    return ((p.bfloat16().float() @ vb) / p.sum(-1, keepdim=True)).transpose(0, 1), s


def test_reference_semantics_one_block_closed_form():
    # One block over every key: the emulation is exactly the closed form, and the rounding
    # points are really there (it differs from the unrounded fp32 result).
    g = torch.Generator().manual_seed(31)
    q = torch.randn(6, 5, 64, generator=g).bfloat16()
    k = torch.randn(2, 155, 64, generator=g)
    v = torch.randn(2, 155, 64, generator=g)
    got = reference_semantics(q, k, v, 150, block=256, out_dtype=torch.float32)
    expect, _ = _closed_form(q, k, v, 150)
    assert torch.allclose(got, expect, rtol=1e-6, atol=1e-6)
    assert (got - attention(q, k, v, 150, dtype=torch.float32)).abs().max() > 1e-4


def test_reference_semantics_blocks_without_rescaling():
    # When the first 64-key block holds every row's maximum, the online loop never rescales and
    # must equal the closed form even with 64-key blocks.
    g = torch.Generator().manual_seed(33)
    q = (torch.randn(6, 5, 64, generator=g) + 2).bfloat16()
    k = torch.randn(2, 155, 64, generator=g)
    k[:, 0] = 0.5
    k[:, 64:] *= 0.1
    v = torch.randn(2, 155, 64, generator=g)
    got = reference_semantics(q, k, v, 150, out_dtype=torch.float32)
    expect, s = _closed_form(q, k, v, 150)
    assert torch.equal(s.argmax(-1), torch.zeros(6, 5, dtype=torch.long))
    assert torch.allclose(got, expect, rtol=1e-6, atol=1e-6)


def test_reference_semantics_rounds_p_against_the_running_max():
    """The reference rounds p to bf16 against the maximum known when a block is processed and
    rescales the accumulated P.V by alpha in fp32 afterwards (src/gpu_kernels.py:97-102). A case
    whose every score is exact: block 0 holds 32 keys of score 1 (V = 1) and 32 of score 0 (V = 2),
    block 1 raises the maximum to 3 (64 keys, V = -1), the chunk's own key scores 3 (V = -1).
    Block 0's p are 1 and bf16(e^-1), scaled by e^-2 when block 1 arrives, so the output is
    ((32 + 64 bf16(e^-1)) e^-2 - 65) / ((32 + 32 e^-1) e^-2 + 65). Rounding p against the final
    maximum instead, or not rounding it, gives values 2.8e-4 and 8.5e-5 away."""
    past = 128
    q = torch.zeros(1, 1, 64)
    q[0, 0, 0] = 8.0  # score = 8 * k[0] * 0.125 = k[0]
    k = torch.zeros(1, past + 1, 64)
    v = torch.zeros(1, past + 1, 64)
    k[0, 0:64:2, 0], v[0, 0:64:2] = 1.0, 1.0
    k[0, 1:64:2, 0], v[0, 1:64:2] = 0.0, 2.0
    k[0, 64:, 0], v[0, 64:] = 3.0, -1.0
    got = reference_semantics(q.bfloat16(), k, v, past, out_dtype=torch.float32)[0, 0].double()

    def bf16(x):
        return float(torch.tensor(x).bfloat16())

    e1, e2 = math.exp(-1), math.exp(-2)
    den = (32 + 32 * e1) * e2 + 65
    expect = ((32 + 64 * bf16(e1)) * e2 - 65) / den
    late = (32 * bf16(e2) + 64 * bf16(math.exp(-3)) - 65) / den
    unrounded = ((32 + 64 * e1) * e2 - 65) / den
    assert torch.allclose(got, torch.full((64,), expect, dtype=torch.float64), rtol=1e-6, atol=0)
    for wrong in (late, unrounded):
        assert (got - wrong).abs().min().item() > 5e-5


def test_reference_semantics_segments_equal_separate_calls():
    g = torch.Generator().manual_seed(32)
    past, bounds = 70, [0, 4, 9]
    q = torch.randn(3, 9, 64, generator=g).bfloat16()
    k = torch.randn(1, past + 9, 64, generator=g)
    v = torch.randn(1, past + 9, 64, generator=g)
    got = reference_semantics(q, k, v, past, segments=bounds, out_dtype=torch.float32)
    for lo, hi in ((0, 4), (4, 9)):
        kc = torch.cat((k[:, :past], k[:, past + lo:past + hi]), 1)
        vc = torch.cat((v[:, :past], v[:, past + lo:past + hi]), 1)
        alone = reference_semantics(q[:, lo:hi], kc, vc, past, out_dtype=torch.float32)
        assert torch.allclose(got[lo:hi], alone, atol=1e-6)


def test_reference_semantics_skips_blocks_a_segment_cannot_see():
    """With chunk segments a row's first key blocks can be fully masked (never so in the reference,
    whose chunk is one causal segment): the emulation must keep the empty state there (no nan) and
    stay within bf16 rounding of the exact oracle."""
    g = torch.Generator().manual_seed(5)
    q = torch.randn((2, 65, 64), generator=g).to(torch.bfloat16)
    k = torch.randn((1, 65, 64), generator=g)
    v = torch.randn((1, 65, 64), generator=g)
    exact = attention(q, k, v, 0, segments=[0, 60, 65])
    for block in (16, 32, 64):
        got = reference_semantics(q, k, v, 0, block=block, segments=[0, 60, 65], out_dtype=torch.float32)
        assert not torch.isnan(got).any()
        assert (got.double() - exact).abs().max().item() <= 2e-2
