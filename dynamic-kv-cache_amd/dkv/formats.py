"""The reference's serialized KV formats, produced from and loaded into the arena.

- PackedTensor (src/kv_quantization.py:12-39): payload, fp32 scales and offsets
  with one group per 64-element row, and a 64-byte header
  '<4sBBBB4qQQQ' = magic b'DKVC', version 1, bits, dtype code, ndim, shape,
  group size, numel, groups (src/kv_quantization.py:74-76).
- Segment (src/cache_manager.py:9-15): the key and value PackedTensors of one
  update of one layer, with a 32-byte descriptor '<iiqqB7x' = layer, frame,
  absolute start, absolute end, bits.

GPUCache.export_segments() returns {layer: [Segment]}, the structure
src/cache_manager.py's MixedPrecisionCache keeps in `segments`, and
GPUCache.import_segments() appends such a structure to a cache. Both move bytes
only (dkv_export / dkv_import / dkv_segment_batch in libdkv): the arena already
holds the quantizer's payload, offsets and scales.
"""
import struct
from dataclasses import dataclass

import torch

HEADER = struct.Struct('<4sBBBB4qQQQ')
SEGMENT = struct.Struct('<iiqqB7x')
MAGIC, VERSION = b'DKVC', 1
DTYPE_CODES = {torch.float16: 1, torch.bfloat16: 2, torch.float32: 3}
GROUP = 64


@dataclass
class PackedTensor:
    """Same fields, header checks and byte counts as src/kv_quantization.py:15-39."""
    payload: torch.Tensor
    scales: torch.Tensor
    offsets: torch.Tensor
    header: torch.Tensor

    def fields(self):
        """(bits, dtype code, shape, group size, numel, groups); ValueError on a foreign header."""
        if self.header.numel() != HEADER.size:
            raise ValueError('Invalid packed tensor header')
        magic, version, bits, dtype, ndim, *rest = HEADER.unpack(bytes(self.header.cpu().tolist()))
        if magic != MAGIC or version != VERSION or not 0 < ndim <= 4:
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


@dataclass
class Segment:
    """One layer's key/value PackedTensors and 32-byte descriptor (src/cache_manager.py:11-15)."""
    key: PackedTensor
    value: PackedTensor
    descriptor: torch.Tensor

    def fields(self):
        """(layer, frame, start, end, bits)."""
        return descriptor_fields(self.descriptor)


def descriptor_fields(t):
    """(layer, frame, start, end, bits) of a 32-byte descriptor tensor (src/cache_manager.py:35,80)."""
    if t.numel() != SEGMENT.size or t.dtype != torch.uint8:
        raise ValueError('Invalid segment descriptor')
    return SEGMENT.unpack(bytes(t.cpu().tolist()))


def header(bits, heads, rows, dtype=torch.bfloat16):
    """The 64-byte header pack() writes for a [1, heads, rows, 64] tensor (src/kv_quantization.py:74-76)."""
    numel = heads * rows * GROUP
    groups = 0 if bits == 16 else heads * rows
    raw = HEADER.pack(MAGIC, VERSION, bits, DTYPE_CODES[dtype], 4, 1, heads, rows, GROUP, GROUP, numel, groups)
    return torch.tensor(list(raw), dtype=torch.uint8)


def descriptor(layer, frame, start, end, bits):
    """The 32-byte segment descriptor (src/cache_manager.py:9,56)."""
    return torch.tensor(list(SEGMENT.pack(layer, frame, start, end, bits)), dtype=torch.uint8)


def row_bytes(bits):
    return {4: 32, 8: 64, 16: 128}[bits]


def check_packed(p, bits, heads, rows):
    """Validates one PackedTensor of a segment being imported; returns it unchanged.

    The arena stores 16-bit rows as bf16 and every group as one 64-element row, so
    only tensors of shape [1, heads, rows, 64] with group size 64 (and bf16 at 16
    bits) can be imported without changing their bytes.
    """
    got_bits, dtype, shape, group, numel, groups = p.fields()
    if got_bits != bits:
        raise ValueError(f'Packed tensor has {got_bits} bits, its segment descriptor {bits}')
    if shape != (1, heads, rows, GROUP) or group != GROUP or numel != heads * rows * GROUP:
        raise ValueError(f'Packed tensor of shape {shape}, group {group} does not fit [1, {heads}, {rows}, 64] rows')
    if bits == 16 and dtype != DTYPE_CODES[torch.bfloat16]:
        raise ValueError('16-bit segments must hold bf16 values to be imported')
    if p.payload.dtype != torch.uint8 or p.payload.numel() != heads * rows * row_bytes(bits):
        raise ValueError('Packed tensor payload size does not match its header')
    if bits < 16:
        if groups != heads * rows:
            raise ValueError('Packed tensor group count does not match its header')
        for t in (p.scales, p.offsets):
            if t.dtype != torch.float32 or t.numel() != heads * rows:
                raise ValueError('Packed tensor scales/offsets must be fp32 with one entry per row')
    return p
