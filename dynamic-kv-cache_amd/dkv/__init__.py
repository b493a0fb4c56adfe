"""dkv: MI355X-native packed mixed-precision KV cache (pack + fused packed-history attention).

Public surface mirrors the reference's src/gpu_cache.py and src/gpu_ops.py:
GPUCache, install_packed_attention, cuda_rms, activation_product, install_fused_ops.
The kernels live in libdkv.so (HIP, gfx950), reached through ctypes (dkv._lib).
"""
from .gpu_cache import GPUCache, install_packed_attention
from .gpu_ops import activation_product, cuda_rms, install_fused_ops

__all__ = ['GPUCache', 'install_packed_attention', 'cuda_rms', 'activation_product', 'install_fused_ops']
