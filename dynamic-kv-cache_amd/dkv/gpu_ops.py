"""Joined decoder projections and library normalization (src/gpu_ops.py:1-48).

Same surface as the reference: cuda_rms, activation_product and
install_fused_ops. These stay PyTorch-library ops (rms_norm, silu, one joined
GEMM for Q/K/V and for gate/up); they are not part of the packed-KV kernels.
"""
import types

import torch


def cuda_rms(x, weight, eps):
    """RMSNorm via torch's fused op, rounding to x.dtype before the weight multiply (src/gpu_ops.py:9-12)."""
    return torch.nn.functional.rms_norm(x, (x.shape[-1],), None, eps) * weight


def activation_product(gate, up):
    """silu(gate) * up (src/gpu_ops.py:14-17)."""
    return torch.nn.functional.silu(gate) * up


def install_fused_ops(text, state):
    """Joins Q/K/V and gate/up weights and patches RMSNorm/MLP (src/gpu_ops.py:19-48).

    `state['enabled']` switches between the joined path and the untouched upstream forwards.
    """
    def rms_forward(module, x):
        return cuda_rms(x, module.weight, module.variance_epsilon) if state['enabled'] else module._original_rms(x)

    def mlp_forward(module, x):
        if not state['enabled']:
            return module._original_mlp(x)
        gate, up = torch.nn.functional.linear(x, module._gate_up_weight).chunk(2, dim=-1)
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
