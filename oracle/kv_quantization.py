"""Restatement of the reference quantizer (src/kv_quantization.py:12-92). TEST INFRASTRUCTURE ONLY.

pack(tensor, bits, group_size=64) follows src/kv_quantization.py:41-77:
  - validation: bits in {4, 8, 16}, positive group size, 4-D nonempty float,
    finite values (:42-48), else ValueError;
  - 16-bit: fp16/bf16 bytes kept verbatim, other floats cast to fp16 (:49-55);
  - 4/8-bit: flatten, groups of `group_size` padded by repeating the last value
    (:57-62); offset = group min (:63; a zero minimum carries the IEEE 754-2019
    minimum()'s sign, see canonical_zero_min); span = max - offset (:64);
    scale = span / (2^b - 1) if span > 0 else 1 (:65);
    q = round_half_even((x - offset) / scale) clamped to [0, 2^b - 1] (:66-67);
    4-bit payload byte i = q[2i] | q[2i+1] << 4 (:68-71);
  - 64-byte header '<4sBBBB4qQQQ' = magic b'DKVC', version 1, bits, dtype code
    (fp16 1, bf16 2, fp32 3), ndim, shape, group size, numel, groups (:12-13, :74-76).
unpack follows :79-92: q * scale + offset in fp32 (separate multiply and add),
then cast to the requested dtype.

Pinned by tests/test_oracle_pack.py: the reference's own assertions
(tests/test_quantization.py:6-36), an independent numpy float32 implementation,
exact half-way ties, min -> 0 / max -> 2^b-1, nibble order on hand-built rows,
and literal header bytes.
"""
import math
import struct
from dataclasses import dataclass

import torch

HEADER = struct.Struct('<4sBBBB4qQQQ')
DTYPE_CODES = {torch.float16: 1, torch.bfloat16: 2, torch.float32: 3}


@dataclass
class PackedTensor:
    payload: torch.Tensor
    scales: torch.Tensor
    offsets: torch.Tensor
    header: torch.Tensor

    def fields(self):
        magic, version, bits, dtype, ndim, *rest = HEADER.unpack(bytes(self.header.tolist()))
        if magic != b'DKVC' or version != 1:
            raise ValueError('Invalid packed tensor header')
        return bits, dtype, tuple(rest[:ndim]), rest[4], rest[5], rest[6]

    @property
    def payload_bytes(self):
        return self.payload.numel() * self.payload.element_size()

    @property
    def metadata_bytes(self):
        return sum(t.numel() * t.element_size() for t in (self.scales, self.offsets, self.header))

    @property
    def storage_bytes(self):
        return self.payload_bytes + self.metadata_bytes


def canonical_zero_min(groups, offsets):
    """The sign of a zero group minimum, fixed as IEEE 754-2019 minimum() fixes it: -0 when the
    group holds a -0 (and no negative value), else +0.

    The reference's offset is torch's amin (src/kv_quantization.py:63), whose sign for a minimum
    that is a zero present with both signs depends on the reduction order of the build and CPU it
    runs on. Codes, scales and dequantized values do not depend on that sign; this pins the one
    bit left open so that packed bytes compare bit for bit.
    """
    neg_zero = (groups.view(torch.int32) == -0x80000000).any(dim=1)
    zero = offsets == 0
    return torch.where(zero, torch.where(neg_zero, -0.0, 0.0), offsets)


def quantize_groups(groups, bits):
    """Per-group affine codes of a float32 [n_groups, group_size] tensor.

    Returns (codes uint8, offsets fp32, scales fp32) with the reference's op order.
    """
    levels = (1 << bits) - 1
    offsets = canonical_zero_min(groups, groups.amin(dim=1))
    spans = groups.amax(dim=1) - offsets
    scales = torch.where(spans > 0, spans / levels, torch.ones_like(spans))
    q = ((groups - offsets[:, None]) / scales[:, None]).round().clamp(0, levels)
    return q.to(torch.uint8), offsets, scales


def nibble_pack(codes):
    """Two 4-bit codes per byte, the even-indexed code in the low nibble."""
    if codes.numel() % 2:
        codes = torch.cat((codes, codes.new_zeros(1)))
    return (codes[0::2] | (codes[1::2] << 4)).contiguous()


def pack(tensor, bits, group_size=64):
    if bits not in (4, 8, 16) or group_size <= 0:
        raise ValueError('Supported bit widths: 4, 8, 16; positive group size required')
    if tensor.ndim != 4 or not tensor.is_floating_point() or tensor.numel() == 0:
        raise ValueError('Expected nonempty [batch, heads, tokens, head_dim] float tensor')
    x = tensor.detach().to('cpu').contiguous()
    if not torch.isfinite(x).all():
        raise ValueError('Nonfinite KV tensor')
    if bits == 16:
        if x.dtype not in (torch.float16, torch.bfloat16):
            x = x.to(torch.float16)
        payload = x.view(torch.uint8).flatten().clone()
        scales = offsets = torch.empty(0, dtype=torch.float32)
        n_groups = 0
    else:
        flat = x.float().flatten()
        n_groups = math.ceil(flat.numel() / group_size)
        pad = n_groups * group_size - flat.numel()
        if pad:
            flat = torch.cat((flat, flat[-1:].expand(pad)))
        codes, offsets, scales = quantize_groups(flat.view(n_groups, group_size), bits)
        codes = codes.flatten()[:x.numel()]
        payload = nibble_pack(codes) if bits == 4 else codes.contiguous()
    raw = HEADER.pack(b'DKVC', 1, bits, DTYPE_CODES[x.dtype], x.ndim, *x.shape, group_size, x.numel(), n_groups)
    return PackedTensor(payload, scales, offsets, torch.tensor(list(raw), dtype=torch.uint8))


def unpack(packed, dtype=None, device='cpu'):
    bits, dtype_code, shape, group_size, numel, n_groups = packed.fields()
    source = next(k for k, v in DTYPE_CODES.items() if v == dtype_code)
    dtype = source if dtype is None else dtype
    if bits == 16:
        return packed.payload.view(source).reshape(shape).to(dtype=dtype, device=device)
    if bits == 4:
        q = torch.stack((packed.payload & 15, packed.payload >> 4), dim=-1).flatten()[:numel]
    else:
        q = packed.payload
    q = torch.cat((q, q.new_zeros(n_groups * group_size - numel))).float().view(n_groups, group_size)
    x = q * packed.scales[:, None] + packed.offsets[:, None]
    return x.flatten()[:numel].reshape(shape).to(dtype=dtype, device=device)


def pack_rows(x, bits):
    """Per-row view of pack() for [..., 64] inputs: (payload [..., row_bytes] uint8, offsets, scales).

    With head_dim == group_size == 64 every (head, token) row is one group, which is the
    layout libdkv stores; this reshapes pack()'s flat outputs accordingly.
    """
    lead = x.shape[:-1]
    p = pack(x.reshape(1, 1, -1, 64), bits, 64)
    rb = {4: 32, 8: 64, 16: 128}[bits]
    payload = p.payload.view(*lead, rb)
    if bits == 16:
        return payload, None, None
    return payload, p.offsets.view(lead), p.scales.view(lead)
