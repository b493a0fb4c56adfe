"""dkv_linear (the decoder's short-chunk projections on MFMA) against the torch compositions it
replaces, and the fused decoder layer against the upstream layer forward.

Reference for a projection: the torch ops of the reference's decoder in bf16 (src/gpu_ops.py:9-48:
rms_norm(x) * weight, F.linear over the joined weights, silu(gate) * up, residual + y), with the
GEMM itself evaluated in float64 so that only the rounding points remain. The kernel accumulates in
fp32 in another order and may compute rsqrt an ulp apart, which can move a bf16 rounding; one such
move changes an output by one bf16 ulp, or, through a flipped normalized input, by far less. Bound:
every output within 2 bf16 ulps of its reference value, plus one ulp of the GEMM result before the
residual add (under cancellation that ulp is larger than the sum's) or the SiLU*up product's
sensitivity to one ulp of gate or up, plus 2^-12 of the output's RMS. With the RMSNorm prologue,
rsqrt an ulp apart (torch's kernels and this one sum the squares in other orders) flips some
normalized inputs by one ulp; allowance: 3 sigma of independent one-ulp flips of every input,
3 * 2^-7 * sqrt(sum_k (xn_k w_nk)^2). And the mean deviation below
2^-9 of the mean magnitude (a dropped term, a wrong row or column fails both by orders of
magnitude). Against torch's own bf16 GEMM (another accumulation order) the allowance doubles.

Shapes: the 960-wide decoder (Q/K/V 1600, o_proj 960, gate/up 2 x 2560, down_proj from 2560) and
the 384-wide test decoder, at 1, 17, 64 and 100 rows.
"""
import pytest
import torch

from conftest import announce
from dkv import gpu_ops

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def bf(x):
    return x.to(BF).double()


def reference(x, w, norm=None, eps=1e-5, residual=None, silu_mul=False):
    """(reference output, per-element allowance for one flipped rounding of the GEMM result before
    the epilogue: one ulp of y for the residual add, the SiLU*up product's sensitivity for gate/up)."""
    xd = x.double()
    flips = 0.0
    if norm is not None:
        xd = bf(torch.nn.functional.rms_norm(x.float(), (x.shape[-1],), None, eps)).double() * norm.double()
        xd = bf(xd)
        # rsqrt an ulp apart flips some normalized inputs by one bf16 ulp: 3 sigma of independent flips
        flips = 3 * 2.0 ** -7 * ((xd ** 2) @ (w.double() ** 2).t()).sqrt()
    y = xd @ w.double().t()
    if silu_mul:
        n = w.shape[0] // 2
        g, u = bf(y[:, :n]), bf(y[:, n:])
        fl = flips[:, :n] * u.abs() * 1.1 + flips[:, n:] * g.abs() if norm is not None else 0.0
        return bf(bf(g.float() / (1 + torch.exp(-g.float()))) * u), (g * u).abs() * 2.0 ** -6 + fl
    y = bf(y)
    if residual is not None:
        return bf(y + residual.double()), y.abs() * 2.0 ** -7 + flips
    return y, torch.zeros_like(y) + flips


def check(got, ref, extra):
    g, r = got.double(), ref.double()
    ulp = r.abs() * 2.0 ** -7
    rms = r.pow(2).mean().sqrt().item()
    err = (g - r).abs()
    assert bool((err <= 2 * ulp + extra + rms * 2.0 ** -12).all()), (err - 2 * ulp - extra).max().item()
    assert err.mean().item() <= r.abs().mean().item() * 2.0 ** -9


SHAPES = [  # (k, n, norm, epilogue)
    (960, 1600, True, 'plain'), (960, 960, False, 'residual'), (960, 5120, True, 'silu'),
    (2560, 960, False, 'residual'), (384, 640, True, 'plain'), (384, 1536, True, 'silu'),
    (768, 384, False, 'residual'), (960, 960, False, 'plain'), (2560, 960, False, 'plain'),
]


@pytest.mark.parametrize('rows', [1, 17, 64, 100])
@pytest.mark.parametrize('k,n,norm,epi', SHAPES)
def test_linear_matches_torch_composition(cuda, rows, k, n, norm, epi):
    announce(f'linear: rows={rows} k={k} n={n} norm={norm} epi={epi}')
    g = torch.Generator().manual_seed(rows * 7 + k + n)
    x = (torch.randn(rows, k, generator=g) * 2).to(BF).to(cuda)
    w = (torch.randn(n, k, generator=g) / k ** 0.5).to(BF).to(cuda)
    nw = (torch.rand(k, generator=g) + 0.5).to(BF).to(cuda) if norm else None
    n_out = n // 2 if epi == 'silu' else n
    res = (torch.randn(rows, n_out, generator=g)).to(BF).to(cuda) if epi == 'residual' else None
    got = gpu_ops.linear(x, w, norm=nw, eps=1e-5, residual=res, silu_mul=epi == 'silu')
    assert got is not None and got.shape == (rows, n_out)
    torch.cuda.synchronize()
    ref, extra = reference(x.cpu(), w.cpu(), None if nw is None else nw.cpu(), 1e-5,
                           None if res is None else res.cpu(), epi == 'silu')
    check(got.cpu(), ref, extra)
    # and against torch's own bf16 ops on the GPU (library GEMM)
    xt = x if nw is None else torch.nn.functional.rms_norm(x, (k,), None, 1e-5) * nw
    yt = torch.nn.functional.linear(xt, w)
    if epi == 'silu':
        yt = torch.nn.functional.silu(yt[:, :n_out]) * yt[:, n_out:]
    elif epi == 'residual':
        yt = res + yt
    check(got.cpu(), yt.cpu(), 2 * extra)


@pytest.mark.parametrize('rows', [1, 17, 64, 100])
@pytest.mark.parametrize('k,n,norm,epi', SHAPES)
def test_tiled_layouts_equal_row_major(cuda, rows, k, n, norm, epi):
    """dkv_linear_tiled reads the MFMA-tiled copies of w (and of x) and writes a tiled out: every lane
    loads the same values as from the row-major operands, so every output bit is the same."""
    announce(f'linear tiled: rows={rows} k={k} n={n} norm={norm} epi={epi}')
    g = torch.Generator().manual_seed(rows * 5 + k + n)
    x = (torch.randn(rows, k, generator=g) * 2).to(BF).to(cuda)
    w = (torch.randn(n, k, generator=g) / k ** 0.5).to(BF).to(cuda)
    nw = (torch.rand(k, generator=g) + 0.5).to(BF).to(cuda) if norm else None
    n_out = n // 2 if epi == 'silu' else n
    res = (torch.randn(rows, n_out, generator=g)).to(BF).to(cuda) if epi == 'residual' else None
    kw = dict(norm=nw, eps=1e-5, residual=res, silu_mul=epi == 'silu')
    want = gpu_ops.linear(x, w, **kw)
    wt = gpu_ops.mfma_tiled(w)
    xt = gpu_ops.mfma_tiled(x)
    assert torch.equal(gpu_ops.linear(x, w, weight_tiled=wt, **kw), want)
    assert torch.equal(gpu_ops.linear(xt, w, x_tiled=True, rows=rows, **kw), want)
    assert torch.equal(gpu_ops.linear(xt, w, weight_tiled=wt, x_tiled=True, rows=rows, **kw), want)
    if n_out % 64 == 0:
        got = gpu_ops.linear(x, w, weight_tiled=wt, out_tiled=True, **kw)
        assert got.shape == ((rows + 15) // 16 * 16, n_out)
        assert torch.equal(gpu_ops.mfma_untiled(got, rows), want)
        if res is not None:  # a tiled residual too
            kw['residual'] = gpu_ops.mfma_tiled(res)
            got = gpu_ops.linear(xt, w, weight_tiled=wt, x_tiled=True, rows=rows, residual_tiled=True, **kw)
            assert torch.equal(got, want)
    torch.cuda.synchronize()


def test_linear_strided_rows_and_uncovered_inputs(cuda):
    announce('linear: strided x, uncovered inputs')
    g = torch.Generator().manual_seed(5)
    wide = torch.randn(40, 1024 + 64, generator=g).to(BF).to(cuda)
    x = wide[:, :960]  # row stride 1088 elements
    w = (torch.randn(960, 960, generator=g) / 31).to(BF).to(cuda)
    got = gpu_ops.linear(x, w)
    check(got.cpu(), *reference(x.cpu(), w.cpu()))
    assert gpu_ops.linear(x.float(), w) is None  # fp32 input
    assert gpu_ops.linear(x[:, :900], w[:, :900].contiguous()) is None  # k not a multiple of 64
    w2 = (torch.randn(1000, 960, generator=g)).to(BF).to(cuda)
    assert gpu_ops.linear(x, w2) is None  # 1000 output columns: not a multiple of 16
    big = (torch.randn(4, 2048, generator=g)).to(BF).to(cuda)
    wb = (torch.randn(64, 2048, generator=g)).to(BF).to(cuda)
    assert gpu_ops.linear(big, wb, norm=torch.ones(2048, dtype=BF, device=cuda)) is None  # norm needs k <= 1024


def test_fused_layers_match_upstream_layers(cuda):
    """The decoder with fused layers (dkv_linear + fused attention launches) against the same packed
    cache driven through the upstream layer forwards with the fused ops (library GEMMs, the
    reference's composition): logits within 0.05 (scale ~1) after a prefix, two frames and a question."""
    announce('linear: fused decoder layers vs upstream layers')
    from dkv.streaming import StreamingDecoder, build_decoder
    model = build_decoder(layers=2, hidden=384, heads=6, kv_heads=2, intermediate=768, vocab=512, seed=21)
    dec = StreamingDecoder(model, precision='fp32')
    g = torch.Generator().manual_seed(22)
    prefix = torch.randint(0, 512, (1, 16), generator=g)
    question = torch.randint(0, 512, (1, 24), generator=g)
    ids = torch.randint(0, 512, (2, 64), generator=g).to(cuda)
    with torch.inference_mode():
        emb = model.model.get_input_embeddings()(ids)
    frames = [emb[i:i + 1] for i in range(2)]
    out = {}
    for layers in (True, False):
        dec.ops_state['layers'] = layers
        cache = dec.ingest(prefix, frames, [4, 8])
        out[layers] = dec.forward(cache, ids=question, logits=question.shape[1])
    dec.ops_state['layers'] = True
    torch.cuda.synchronize()
    diff = (out[True] - out[False]).abs().max().item()
    assert diff <= 0.05, diff


def test_eager_fused_layers_follow_weight_changes(cuda):
    """The eager fused layers check a layer once per chunk length and keep its weight objects, reading
    their data pointers at every call: a weight whose storage moves (param.data replaced, as
    Module.to() does), a weight replaced by a new Parameter and a weight changed in place are all
    used by the next forward (the layer's MFMA-tiled weight copies are made again). Logits change
    and stay within 0.05 of the upstream layers with the new weights."""
    announce('linear: eager fused layers follow weight changes')
    from dkv.streaming import StreamingDecoder, build_decoder
    model = build_decoder(layers=2, hidden=384, heads=6, kv_heads=2, intermediate=768, vocab=512, seed=23)
    dec = StreamingDecoder(model, precision='fp32')
    g = torch.Generator().manual_seed(24)
    prefix = torch.randint(0, 512, (1, 16), generator=g)
    question = torch.randint(0, 512, (1, 24), generator=g)
    ids = torch.randint(0, 512, (1, 64), generator=g).to(cuda)
    with torch.inference_mode():
        emb = model.model.get_input_embeddings()(ids)
    cache = dec.ingest(prefix, [emb], [8])

    def logits(layers):
        dec.ops_state['layers'] = layers
        try:
            out = dec.forward(cache.fork(), ids=question, logits=question.shape[1])
        finally:
            dec.ops_state['layers'] = True
        torch.cuda.synchronize()
        return out

    before = logits(True)
    layer = model.model.layers[1]
    with torch.no_grad():
        layer.mlp.down_proj.weight.data = layer.mlp.down_proj.weight.data * 2  # same Parameter, new storage
        layer.self_attn.o_proj.weight = torch.nn.Parameter(layer.self_attn.o_proj.weight.detach() * 0.5,
                                                           requires_grad=False)
    fused, upstream = logits(True), logits(False)
    # plans of the other chunk lengths (the prefix's, the frames') held the old tensors: dropped
    plans = layer.__dict__.get('_dkv_plans', {})
    assert plans and all(p is None or p.holds(layer) for p in plans.values())
    changed = (fused - before).abs().max().item()
    diff = (fused - upstream).abs().max().item()
    print(f'[fused-weights] change {changed:.3e}, fused vs upstream {diff:.3e}', flush=True)
    assert changed > 1e-2, changed
    assert diff <= 0.05, diff
    # an in-place change of a joined weight (through its q_proj view: one version counter) makes the
    # next forward tile the layer's weight copies again
    with torch.no_grad():
        layer.self_attn.q_proj.weight.mul_(1.5)
    fused2, upstream2 = logits(True), logits(False)
    changed2 = (fused2 - fused).abs().max().item()
    diff2 = (fused2 - upstream2).abs().max().item()
    print(f'[fused-weights] in place: change {changed2:.3e}, fused vs upstream {diff2:.3e}', flush=True)
    assert changed2 > 1e-2, changed2
    assert diff2 <= 0.05, diff2
