"""Joined decoder projections and fused pointwise ops (src/gpu_ops.py:1-48).

Same surface as the reference: cuda_rms, activation_product and
install_fused_ops. The reference keeps RMSNorm and SiLU*up as PyTorch library
ops; here bf16 CUDA tensors go through one HIP launch each (libdkv's
dkv_rms_norm and dkv_silu_mul), with the same bf16 rounding points as the
torch compositions. rope_qkv() is the joined Q/K/V split plus RoPE of the
patched attention forward in one launch (dkv_rope_qkv).

linear() is libdkv's short-chunk projection (dkv_linear): the joined GEMMs on
MFMA with the RMSNorm before them and the residual add or SiLU*up after them
folded in. install_fused_ops also patches LlamaDecoderLayer so that, on a
packed GPUCache, a layer runs as five launches plus the attention: Q/K/V
(with input_layernorm), split + RoPE + pack, attention, o_proj + residual,
gate/up (with post_attention_layernorm) + SiLU*up, down_proj + residual.

Tensors the kernels do not cover (other dtypes, CPU tensors, other shapes)
take the reference's own torch composition.
"""
import functools
import types

import torch

from . import _lib


def _rows(x):
    """2-D view [rows, dim] with unit column stride and 16-byte aligned rows (copies otherwise)."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2


def _fused(*ts):
    return all(t.is_cuda and t.dtype == torch.bfloat16 for t in ts) and ts[0].shape[-1] % 8 == 0


def cuda_rms(x, weight, eps):
    """RMSNorm rounded to x.dtype before the weight multiply (src/gpu_ops.py:9-12); one HIP launch for bf16."""
    if not _fused(x, weight) or weight.dim() != 1 or weight.stride(0) != 1 or weight.data_ptr() % 16:
        return torch.nn.functional.rms_norm(x, (x.shape[-1],), None, eps) * weight
    x2 = _rows(x)
    out = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    _lib.check(_lib.load().dkv_rms_norm(x2.data_ptr(), x2.stride(0), weight.data_ptr(), out.data_ptr(), out.stride(0),
                                        x2.shape[0], x2.shape[1], float(eps), _lib.stream_handle(x.device)),
               'dkv_rms_norm')
    return out.view(x.shape)


def silu_mul(gate_up):
    """silu(gate) * up over a joined [..., 2 * inter] projection (gate first), one HIP launch."""
    inter = gate_up.shape[-1] // 2
    g2 = _rows(gate_up)
    out = torch.empty((g2.shape[0], inter), dtype=gate_up.dtype, device=gate_up.device)
    _lib.check(_lib.load().dkv_silu_mul(g2.data_ptr(), g2.stride(0), out.data_ptr(), out.stride(0), g2.shape[0],
                                        inter, _lib.stream_handle(gate_up.device)), 'dkv_silu_mul')
    return out.view(*gate_up.shape[:-1], inter)


def activation_product(gate, up):
    """silu(gate) * up (src/gpu_ops.py:14-17); one HIP launch for bf16."""
    if not _fused(gate, up) or gate.shape != up.shape:
        return torch.nn.functional.silu(gate) * up
    inter = gate.shape[-1]
    joined = (gate.untyped_storage().data_ptr() == up.untyped_storage().data_ptr()
              and up.storage_offset() == gate.storage_offset() + inter and gate.stride() == up.stride()
              and gate.stride(-1) == 1)
    if joined:  # the two chunks of one joined projection: read them in place
        full = gate.as_strided(gate.shape[:-1] + (2 * inter,), gate.stride())
        return silu_mul(full)
    return silu_mul(torch.cat((gate, up), dim=-1))


def rope_qkv(qkv, cos, sin, q_heads, kv_heads, head_dim=64):
    """Joined projection [1, n, (q_heads + 2 kv_heads) * 64] -> q [1, q_heads, n, 64], k, v [1, kv_heads, n, 64]
    with RoPE on q and k as transformers' apply_rotary_pos_emb computes it in bf16 (one HIP launch).
    Returns None when the kernel does not cover the inputs."""
    if (head_dim != 64 or qkv.dim() != 3 or qkv.shape[0] != 1 or not _fused(qkv, cos, sin)
            or cos.shape[-1] != 64 or cos.shape[-2] != qkv.shape[1] or sin.shape != cos.shape):
        return None
    n = qkv.shape[1]
    q2, c2, s2 = _rows(qkv), _rows(cos), _rows(sin)
    q = torch.empty((1, q_heads, n, 64), dtype=qkv.dtype, device=qkv.device)
    k = torch.empty((1, kv_heads, n, 64), dtype=qkv.dtype, device=qkv.device)
    v = torch.empty((1, kv_heads, n, 64), dtype=qkv.dtype, device=qkv.device)
    _lib.check(_lib.load().dkv_rope_qkv(q2.data_ptr(), q2.stride(0), c2.data_ptr(), s2.data_ptr(), c2.stride(0), n,
                                        q_heads, kv_heads, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                        _lib.stream_handle(qkv.device)), 'dkv_rope_qkv')
    return q, k, v


LINEAR_PLAIN, LINEAR_RESIDUAL, LINEAR_SILU_MUL = 0, 1, 2


def _weight_rows(w):
    return (w.dim() == 2 and w.is_cuda and w.dtype == torch.bfloat16 and w.stride(1) == 1
            and w.stride(0) % 8 == 0 and w.data_ptr() % 16 == 0)


@functools.lru_cache(maxsize=None)
def _linear_supported(rows, n, k, norm, epilogue):
    return bool(_lib.load().dkv_linear_supported(rows, n, k, norm, epilogue))


def linear_covered(rows, weight, norm=False, epilogue=LINEAR_PLAIN):
    """Whether dkv_linear has a launch for x [rows, weight.shape[1]] . weight^T with this prologue/epilogue."""
    return _weight_rows(weight) and _linear_supported(rows, weight.shape[0], weight.shape[1], int(norm), epilogue)


LINEAR_W_TILED, LINEAR_X_TILED, LINEAR_OUT_TILED, LINEAR_RES_TILED = 1, 2, 4, 8


def mfma_tiled(t):
    """A copy of the bf16 matrix t [R, k] (k a multiple of 64) in dkv_linear's MFMA-tiled layout,
    rows rounded up to 16 with zeros: element (r, c) at ((r // 16) * (k // 64) + c // 64) * 1024
    + (c // 32 % 2) * 512 + ((c // 8 % 4) * 16 + r % 16) * 8 + c % 8, the order in which the
    kernel's lanes read a 16-row x 64-column block, so that each of its load instructions reads
    1 KB of consecutive bytes. Returned as a contiguous [R16, k] tensor."""
    R, k = t.shape
    R16 = (R + 15) // 16 * 16
    if R16 != R:
        t = torch.cat((t, t.new_zeros(R16 - R, k)))
    return t.reshape(R16 // 16, 16, k // 64, 2, 4, 8).permute(0, 2, 3, 4, 1, 5).contiguous().view(R16, k)


def mfma_untiled(t, rows):
    """The first `rows` rows of a matrix held in the MFMA-tiled layout (mfma_tiled's inverse)."""
    R16, k = t.shape
    return t.view(R16 // 16, k // 64, 2, 4, 16, 8).permute(0, 4, 1, 2, 3, 5).reshape(R16, k)[:rows]


def linear(x, weight, norm=None, eps=1e-6, residual=None, silu_mul=False, weight_tiled=None, x_tiled=False,
           out_tiled=False, rows=None, residual_tiled=False):
    """x [..., k] . weight[n, k]^T in one launch, optionally with RMSNorm(x) * norm first and the
    residual add (out = residual + y) or SiLU*up over [gate | up] weight rows after; the rounding
    points are the torch compositions'. Returns None when the kernel does not cover the inputs.

    weight_tiled: mfma_tiled(weight), read instead of weight (same results). x_tiled: x is a
    [rows rounded up to 16, k] matrix in the tiled layout, `rows` its row count. out_tiled: the
    output is returned in the tiled layout ([rows rounded up to 16, n_out], padding rows not
    written), as the x of a following x_tiled call. residual_tiled: the residual is such a tiled
    [rows rounded up to 16, n_out] matrix."""
    epi = LINEAR_SILU_MUL if silu_mul else (LINEAR_RESIDUAL if residual is not None else LINEAR_PLAIN)
    if not _fused(x) or not _weight_rows(weight) or x.shape[-1] != weight.shape[1]:
        return None
    layout = 0
    if weight_tiled is not None:
        if not (_fused(weight_tiled) and weight_tiled.is_contiguous() and weight_tiled.shape == weight.shape
                and weight_tiled.data_ptr() % 16 == 0):
            return None
        layout |= LINEAR_W_TILED
    if x_tiled:
        if rows is None or x.dim() != 2 or not x.is_contiguous() or x.shape[0] != (rows + 15) // 16 * 16 \
                or x.data_ptr() % 16:
            return None
        x2 = x
        layout |= LINEAR_X_TILED
    else:
        x2 = _rows(x)
        rows = x2.shape[0]
    k = x2.shape[1]
    n_out = weight.shape[0] // 2 if silu_mul else weight.shape[0]
    if out_tiled:
        if n_out % 64:
            return None
        layout |= LINEAR_OUT_TILED
    if norm is not None and (not _fused(norm) or norm.dim() != 1 or norm.shape[0] != k or norm.stride(0) != 1
                             or norm.data_ptr() % 16):
        return None
    r2 = None
    if residual is not None:
        if not _fused(residual) or residual.shape[-1] != n_out:
            return None
        if residual_tiled:
            if n_out % 64 or residual.shape != ((rows + 15) // 16 * 16, n_out) or not residual.is_contiguous() \
                    or residual.data_ptr() % 16:
                return None
            r2 = residual
            layout |= LINEAR_RES_TILED
        else:
            r2 = residual.reshape(-1, n_out)
            if r2.shape[0] != rows or r2.stride(-1) != 1 or r2.stride(0) % 4 or r2.data_ptr() % 8:
                return None
    if not _linear_supported(rows, weight.shape[0], k, int(norm is not None), epi):
        return None
    out = torch.empty(((rows + 15) // 16 * 16 if out_tiled else rows, n_out), dtype=x.dtype, device=x.device)
    w = weight if weight_tiled is None else weight_tiled
    _lib.check(_lib.load().dkv_linear_tiled(
        x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0), rows, weight.shape[0], k,
        None if norm is None else norm.data_ptr(), float(eps), epi, None if r2 is None else r2.data_ptr(),
        0 if r2 is None else r2.stride(0), out.data_ptr(), out.stride(0), layout, _lib.stream_handle(x.device)),
        'dkv_linear')
    if out_tiled:
        return out
    return out.view(*(x.shape[:-1] if not x_tiled else (rows,)), n_out)


class _LayerPlan:
    """What fused_decoder_layer checked once for one decoder layer and chunk length, and the
    constant arguments of its launches: the weight and norm tensors it checked (a layer that holds
    other objects gets a new plan; their data pointers are read at every launch, since moving a
    module swaps a parameter's storage in place), their row strides and row counts, the norm
    epsilons and the head counts."""
    __slots__ = ('qkv_w', 'o_w', 'gu_w', 'd_w', 'ln1_w', 'ln2_w', 'qkv_args', 'o_args', 'gu_args', 'd_args',
                 'eps1', 'eps2', 'q_heads', 'kv_heads', 'eager_ok', 'layer_idx', 'width', 'inter')

    def holds(self, layer):
        # the modules' own dicts: nn.Module attribute lookups cost more than the rest of this check
        m = layer._modules
        attn, mlp = m['self_attn'], m['mlp']
        return (self.qkv_w is attn._qkv_weight and self.gu_w is mlp._gate_up_weight
                and self.o_w is attn._modules['o_proj']._parameters['weight']
                and self.d_w is mlp._modules['down_proj']._parameters['weight']
                and self.ln1_w is m['input_layernorm']._parameters['weight']
                and self.ln2_w is m['post_attention_layernorm']._parameters['weight'])


def _layer_tiles(layer, p):
    """mfma_tiled copies of the layer's four projection weights (Q/K/V, o_proj, gate/up,
    down_proj), which its dkv_linear launches read instead of the row-major weights (the same
    results; each load instruction then reads 1 KB of consecutive bytes). One set per layer, shared
    by its plans, made again (into the same memory, so that graphs captured earlier read the new
    values on their next replay) when a weight's storage or version counter has changed. None when
    a graph is being captured and no current copies exist: allocating them inside the capture would
    tie them to it, and the launches then read the row-major weights."""
    ws = (p.qkv_w, p.o_w, p.gu_w, p.d_w)
    key = tuple((w.data_ptr(), w._version) for w in ws)
    cur = layer.__dict__.get('_dkv_tiles')
    if cur is not None and all(a is b for a, b in zip(cur[0], ws)):
        if cur[1] == key:
            return cur[2]
        if torch.cuda.is_current_stream_capturing():
            return None
        with torch.no_grad():
            for t, w in zip(cur[2], ws):
                t.copy_(mfma_tiled(w))
        layer.__dict__['_dkv_tiles'] = (ws, key, cur[2])
        return cur[2]
    if torch.cuda.is_current_stream_capturing():
        return None
    with torch.no_grad():
        tiles = tuple(mfma_tiled(w) for w in ws)
    layer.__dict__['_dkv_tiles'] = (ws, key, tiles)
    return tiles


def _layer_plan(layer, n, width):
    """The _LayerPlan of (layer, n) (built on first use), or None when dkv_linear does not cover the
    layer's projections at n rows."""
    plans = layer.__dict__.setdefault('_dkv_plans', {})
    attn, mlp = layer.self_attn, layer.mlp
    p = plans.get((n, width))
    if p is not None:
        if p.holds(layer):
            return p
        # the layer holds other weights now: every plan of it (other chunk lengths too) still refers
        # to the old tensors, which would stay alive with them
        plans.clear()
    ln1, ln2 = layer.input_layernorm, layer.post_attention_layernorm
    o_w, d_w = attn.o_proj.weight, mlp.down_proj.weight
    if not (attn.o_proj.bias is None and mlp.down_proj.bias is None
            and getattr(ln1, 'weight', None) is not None and getattr(ln2, 'weight', None) is not None
            and linear_covered(n, attn._qkv_weight, True, LINEAR_PLAIN)
            and linear_covered(n, o_w, False, LINEAR_RESIDUAL) and o_w.shape[0] == width
            and linear_covered(n, mlp._gate_up_weight, True, LINEAR_SILU_MUL)
            and linear_covered(n, d_w, False, LINEAR_RESIDUAL) and d_w.shape[0] == width
            and all(_fused(w) and w.dim() == 1 and w.stride(0) == 1 and w.data_ptr() % 16 == 0
                    for w in (ln1.weight, ln2.weight))):
        plans[(n, width)] = None
        return None
    p = _LayerPlan()
    p.qkv_w, p.o_w, p.gu_w, p.d_w = attn._qkv_weight, o_w, mlp._gate_up_weight, d_w
    p.ln1_w, p.ln2_w = ln1.weight, ln2.weight
    p.eps1, p.eps2 = float(ln1.variance_epsilon), float(ln2.variance_epsilon)
    # (weight, row stride, weight rows, k) of each dkv_linear launch
    p.qkv_args = (p.qkv_w, p.qkv_w.stride(0), p.qkv_w.shape[0], p.qkv_w.shape[1])
    p.o_args = (o_w, o_w.stride(0), o_w.shape[0], o_w.shape[1])
    p.gu_args = (p.gu_w, p.gu_w.stride(0), p.gu_w.shape[0], p.gu_w.shape[1])
    p.d_args = (d_w, d_w.stride(0), d_w.shape[0], d_w.shape[1])
    sizes, hd = attn._qkv_sizes, attn.head_dim
    p.q_heads, p.kv_heads = sizes[0] // hd, sizes[1] // hd
    # the eager launches split q | k | v as dkv_rope_pack does: 64-wide heads, K and V alike
    p.eager_ok = hd == 64 and sizes[1] == sizes[2] and p.qkv_w.shape[0] == sum(sizes) and sizes[0] % hd == 0
    p.layer_idx, p.width, p.inter = attn.layer_idx, width, p.gu_w.shape[0] // 2
    plans[(n, width)] = p
    return p


def _fused_layer_eager(p, tiles, h, n, cache, cos, sin):
    """The fused layer's eager launches for a checked plan: the launches and arguments linear() and
    attend_projection() would make, without their per-call checks (which cost more host time than
    the GPU spends on a 64-token chunk). The intermediates (the joined projection, q | k | v, the
    attention output, the post-attention residual, SiLU*up) share one allocation; the kernels read
    and write it in stream order, and the allocator hands it out again only to later work on the
    same stream."""
    lib = _lib.load()
    stream = _lib.stream_handle(h.device)
    width, inter = p.width, p.inter
    qw, qld, qrows, qk = p.qkv_args
    ow, old, orows, ok = p.o_args
    gw, gld, grows, gk = p.gu_args
    dw, dld, drows, dk = p.d_args
    ql = ol = gl = dl = 0  # dkv_linear_tiled layouts of Q/K/V, o_proj, gate/up, down_proj
    if tiles is not None:
        (qw, ow, gw, dw), qld, old, gld, dld = tiles, qk, ok, gk, dk
        ql = ol = gl = dl = LINEAR_W_TILED
        if inter % 64 == 0:  # SiLU*up goes to down_proj in the tiled layout
            gl |= LINEAR_OUT_TILED
            dl |= LINEAR_X_TILED
        if orows % 64 == 0:  # and the post-attention residual h2 to gate/up and down_proj
            ol |= LINEAR_OUT_TILED
            gl |= LINEAR_X_TILED
            dl |= LINEAR_RES_TILED
    # element offsets of [qkv | q,k,v | attention out | h2 | act], each n rows (multiples of 64
    # columns; act in rows rounded up to 16 when tiled)
    o_qkvo = n * qrows
    o_att = o_qkvo + n * qrows
    o_h2 = o_att + n * ok
    n16 = (n + 15) // 16 * 16
    o_act = o_h2 + n16 * orows
    scratch = torch.empty(o_act + n16 * inter, dtype=torch.bfloat16, device=h.device)
    out = torch.empty((1, n, drows), dtype=torch.bfloat16, device=h.device)
    base = scratch.data_ptr()
    xp, qkv, att, h2, act = h.data_ptr(), base, base + 2 * o_att, base + 2 * o_h2, base + 2 * o_act
    _lib.check(lib.dkv_linear_tiled(xp, width, qw.data_ptr(), qld, n, qrows, qk, p.ln1_w.data_ptr(), p.eps1,
                                    LINEAR_PLAIN, None, 0, qkv, qrows, ql, stream), 'dkv_linear')
    cache._fused_attention(n, p.q_heads, p.layer_idx, qkv, qrows, cos.data_ptr(), sin.data_ptr(), cos.stride(0),
                           base + 2 * o_qkvo, att, stream)
    _lib.check(lib.dkv_linear_tiled(att, ok, ow.data_ptr(), old, n, orows, ok, None, 1e-6, LINEAR_RESIDUAL, xp,
                                    width, h2, orows, ol, stream), 'dkv_linear')
    _lib.check(lib.dkv_linear_tiled(h2, width, gw.data_ptr(), gld, n, grows, gk, p.ln2_w.data_ptr(), p.eps2,
                                    LINEAR_SILU_MUL, None, 0, act, inter, gl, stream), 'dkv_linear')
    _lib.check(lib.dkv_linear_tiled(act, inter, dw.data_ptr(), dld, n, drows, dk, None, 1e-6, LINEAR_RESIDUAL, h2,
                                    width, out.data_ptr(), drows, dl, stream), 'dkv_linear')
    return out


def fused_decoder_layer(layer, hidden_states, cache, position_embeddings):
    """One LlamaDecoderLayer forward on a packed GPUCache as six launches plus the attention's
    two; None when the layer, the inputs or the cache are outside what they cover. What depends
    only on the layer and the chunk length is checked once (_layer_plan); eager launches on
    contiguous inputs then take _fused_layer_eager, and graph captures the general path below."""
    from .gpu_cache import GPUCache, attend_projection
    attn, mlp = layer._modules['self_attn'], layer._modules['mlp']
    h = hidden_states
    if not (isinstance(cache, GPUCache) and cache.backend == 'fused' and position_embeddings is not None
            and hasattr(attn, '_qkv_weight') and hasattr(mlp, '_gate_up_weight') and h.dim() == 3
            and h.shape[0] == 1 and _fused(h)):
        return None
    n, width = h.shape[1], h.shape[2]
    p = _layer_plan(layer, n, width)
    if p is None:
        return None
    tiles = _layer_tiles(layer, p)
    if p.eager_ok and p.kv_heads == cache.heads and cache._graph is None and cache.chunk_segments is None:
        cos, sin = position_embeddings
        if (h.is_contiguous() and h.data_ptr() % 16 == 0 and cos.shape == (1, n, 64) and sin.shape == cos.shape
                and cos.dtype == torch.bfloat16 and sin.dtype == torch.bfloat16 and cos.is_contiguous()
                and sin.is_contiguous() and cos.data_ptr() % 16 == 0 and sin.data_ptr() % 16 == 0):
            return _fused_layer_eager(p, tiles, h, n, cache, cos.view(n, 64), sin.view(n, 64))
    ln1, ln2 = layer.input_layernorm, layer.post_attention_layernorm
    o_w, d_w = attn.o_proj.weight, mlp.down_proj.weight
    x = h.reshape(n, width)
    qt, ot, gt, dt = tiles if tiles is not None else (None,) * 4
    qkv = linear(x, attn._qkv_weight, norm=ln1.weight, eps=ln1.variance_epsilon, weight_tiled=qt)
    o = attend_projection(attn, cache, qkv.view(1, n, -1), position_embeddings)
    # SiLU*up to down_proj, and h2 to gate/up and down_proj, in the tiled layout
    act_tiled = tiles is not None and p.inter % 64 == 0
    h2_tiled = tiles is not None and width % 64 == 0
    h2 = linear(o.view(n, -1), o_w, residual=x, weight_tiled=ot, out_tiled=h2_tiled)
    act = linear(h2, mlp._gate_up_weight, norm=ln2.weight, eps=ln2.variance_epsilon, silu_mul=True,
                 weight_tiled=gt, x_tiled=h2_tiled, out_tiled=act_tiled, rows=n)
    return linear(act, d_w, residual=h2, weight_tiled=dt, x_tiled=act_tiled, rows=n,
                  residual_tiled=h2_tiled).view(1, n, width)


def install_fused_ops(text, state):
    """Joins Q/K/V and gate/up weights and patches RMSNorm/MLP (src/gpu_ops.py:19-48), and the
    decoder layers (fused_decoder_layer, transformers 5.x layer signature).

    `state['enabled']` switches between the joined path and the untouched upstream forwards;
    `state['layers']` (default True) enables the fused decoder layers on a packed cache.
    """
    def rms_forward(module, x):
        return cuda_rms(x, module.weight, module.variance_epsilon) if state['enabled'] else module._original_rms(x)

    def mlp_forward(module, x):
        if not state['enabled']:
            return module._original_mlp(x)
        gu = torch.nn.functional.linear(x, module._gate_up_weight)
        if _fused(gu):
            return module.down_proj(silu_mul(gu))
        gate, up = gu.chunk(2, dim=-1)
        return module.down_proj(activation_product(gate, up))

    def join(modules):
        # One storage for the joined weight; each original Parameter becomes a view of it, so the
        # upstream path keeps bit-identical weights and no extra copy stays resident.
        with torch.no_grad():
            joined = torch.cat([m.weight for m in modules], dim=0)
            offset = 0
            for m in modules:
                n = m.weight.shape[0]
                view = joined[offset:offset + n]
                if not torch.equal(view, m.weight):
                    raise RuntimeError('Projection values changed during joining')
                m.weight = torch.nn.Parameter(view, requires_grad=False)
                offset += n
        return joined

    def layer_forward(module, hidden_states, *args, **kwargs):
        if state['enabled'] and state.get('layers', True) and not args and not kwargs.get('output_attentions'):
            cache = kwargs.get('past_key_values', kwargs.get('past_key_value'))
            out = fused_decoder_layer(module, hidden_states, cache, kwargs.get('position_embeddings'))
            if out is not None:
                return out
        return module._original_layer(hidden_states, *args, **kwargs)

    import transformers
    layers_return_tensors = int(transformers.__version__.split('.')[0]) >= 5
    for module in text.modules():
        name = module.__class__.__name__
        if name == 'LlamaDecoderLayer' and layers_return_tensors and not hasattr(module, '_original_layer'):
            module._original_layer = module.forward
            module.forward = types.MethodType(layer_forward, module)
        if name == 'LlamaAttention' and all(m.bias is None for m in (module.q_proj, module.k_proj, module.v_proj)):
            module._qkv_weight = join([module.q_proj, module.k_proj, module.v_proj])
            module._qkv_sizes = [module.q_proj.out_features, module.k_proj.out_features, module.v_proj.out_features]
        elif name == 'LlamaRMSNorm':
            module._original_rms = module.forward
            module.forward = types.MethodType(rms_forward, module)
        elif name == 'LlamaMLP' and text.config.hidden_act == 'silu':
            module._gate_up_weight = join([module.gate_proj, module.up_proj])
            module._original_mlp = module.forward
            module.forward = types.MethodType(mlp_forward, module)
