"""Attention oracles for the packed-history path. TEST INFRASTRUCTURE ONLY.

attention(): dequantize-then-SDPA, the fp32/fp64 oracle. Query row m of Q head
qh attends to KV head qh // (Hq // H) (src/gpu_kernels.py:77;
repeat_interleave in tests/test_gpu_backend.py:97-98), to every history token
t < past and to chunk tokens j <= m of its chunk segment (the bottom-right
causal mask of src/gpu_kernels.py:96 and scripts/test_gpu_backend.py:8-10).
Pinned by tests/test_oracle_attention.py against a pure-Python loop on tiny
inputs, torch SDPA on the reference's own test scenario, and closed forms
(identical keys -> mean of visible V; constant V -> that constant).

reference_semantics(): the reference Triton kernel's rounding points
(src/gpu_kernels.py:84-105): dequantized K/V and the current chunk are cast to
bf16, scores are fp32 dot products times D^-0.5, the online softmax runs over
64-token blocks with exp, p is cast to bf16 before P.V, the fp32 accumulator
is divided by the running sum and stored in bf16.
"""
import torch


def dequant_rows(payload, offsets, scales, bits):
    """fp32 rows from per-row packed data: q * s + a with separate rounding (src/kv_quantization.py:90-91)."""
    if bits == 16:
        return payload.contiguous().view(torch.bfloat16).float()
    if bits == 4:
        q = torch.stack((payload & 15, payload >> 4), dim=-1).flatten(-2)
    else:
        q = payload
    return q.float() * scales[..., None] + offsets[..., None]


def visible_mask(past, nq, segments=None):
    """[nq, past + nq] bool: history fully visible, chunk causal within its segment."""
    bounds = list(segments) if segments else [0, nq]
    seg = torch.zeros(nq, dtype=torch.long)
    for i in range(1, len(bounds) - 1):
        seg[bounds[i]:] = i
    m = torch.arange(nq)[:, None]
    j = torch.arange(nq)[None, :]
    chunk = (j <= m) & (seg[None, :] == seg[:, None])
    return torch.cat((torch.ones(nq, past, dtype=torch.bool), chunk), dim=1)


def attention(q, k, v, past, scale=0.125, segments=None, dtype=torch.float64):
    """q [Hq, nq, 64]; k, v [H, past + nq, 64] (dequantized history then native chunk).

    Returns [nq, Hq, 64] in `dtype`.
    """
    hq, nq, _ = q.shape
    g = hq // k.shape[0]
    kx = k.to(dtype).repeat_interleave(g, 0)
    vx = v.to(dtype).repeat_interleave(g, 0)
    s = (q.to(dtype) @ kx.transpose(1, 2)) * scale
    s = s.masked_fill(~visible_mask(past, nq, segments), float('-inf'))
    return (torch.softmax(s, dim=-1) @ vx).transpose(0, 1).contiguous()


def reference_semantics(q, k, v, past, scale=0.125, block=64, segments=None, out_dtype=torch.bfloat16):
    """Emulation of the reference kernel's bf16 rounding (src/gpu_kernels.py:84-105).

    q [Hq, nq, 64] bf16; k, v [H, past + nq, 64] fp32 (dequantized history, native chunk).
    Returns [nq, Hq, 64] in out_dtype (the reference stores bf16; fp32 keeps acc / den unrounded).
    """
    hq, nq, _ = q.shape
    g = hq // k.shape[0]
    qf = q.float()
    kb = k.to(torch.bfloat16).float().repeat_interleave(g, 0)
    vb = v.to(torch.bfloat16).float().repeat_interleave(g, 0)
    total = past + nq
    mask = visible_mask(past, nq, segments)
    mx = torch.full((hq, nq), float('-inf'))
    den = torch.zeros(hq, nq)
    acc = torch.zeros(hq, nq, 64)
    for b0 in range(0, total, block):
        b1 = min(b0 + block, total)
        s = (qf @ kb[:, b0:b1].transpose(1, 2)) * scale
        s = s.masked_fill(~mask[None, :, b0:b1], float('-inf'))
        new = torch.maximum(mx, s.amax(-1))
        # A row with no visible key yet (only possible with chunk segments, which the reference
        # does not have) keeps its empty state instead of exp(-inf - -inf) = nan.
        ref = torch.where(new == float('-inf'), torch.zeros_like(new), new)
        alpha = torch.exp(mx - ref)
        p = torch.exp(s - ref[..., None])
        den = den * alpha + p.sum(-1)
        acc = acc * alpha[..., None] + p.to(torch.bfloat16).float() @ vb[:, b0:b1]
        mx = new
    return (acc / den[..., None]).to(out_dtype).transpose(0, 1).contiguous()
