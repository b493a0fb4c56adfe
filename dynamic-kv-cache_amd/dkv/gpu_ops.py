"""Joined decoder projections and fused pointwise ops (src/gpu_ops.py:1-48).

Same surface as the reference: cuda_rms, activation_product and
install_fused_ops. The reference keeps RMSNorm and SiLU*up as PyTorch library
ops; here bf16 CUDA tensors go through one HIP launch each (libdkv's
dkv_rms_norm and dkv_silu_mul), with the same bf16 rounding points as the
torch compositions. rope_qkv() is the joined Q/K/V split plus RoPE of the
patched attention forward in one launch (dkv_rope_qkv). The projections stay
library GEMMs (one joined GEMM for Q/K/V and one for gate/up).

Tensors the kernels do not cover (other dtypes, CPU tensors) take the
reference's own torch composition.
"""
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


def install_fused_ops(text, state):
    """Joins Q/K/V and gate/up weights and patches RMSNorm/MLP (src/gpu_ops.py:19-48).

    `state['enabled']` switches between the joined path and the untouched upstream forwards.
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

    for module in text.modules():
        name = module.__class__.__name__
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
