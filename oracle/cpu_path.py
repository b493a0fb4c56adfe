"""The reference's CPU cache path, restated. TEST INFRASTRUCTURE / CPU BASELINE ONLY.

MixedPrecisionCache follows src/cache_manager.py:17-90: select() sets the
pending width (:28-31); update() unpacks every historical segment of the layer,
packs the new K/V with the pending width, records a 32-byte descriptor
'<iiqqB7x' = (layer, frame, start, end, bits) and returns history (dequantized)
concatenated with the native new K/V (:43-63); accounting() sums payload and
metadata bytes (:76-90).

cpu_attention_step() is the flow bench.py times as the CPU baseline: the update
above for one layer, then causal GQA scaled_dot_product_attention over the
returned K/V, as the upstream attention does with the cache's output.

Pinned by tests/test_oracle_cpu_path.py with the reference's own assertions
(tests/test_cache.py:7-27).
"""
import struct
import time
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .kv_quantization import pack, unpack

SEGMENT = struct.Struct('<iiqqB7x')


@dataclass
class Segment:
    key: object
    value: object
    descriptor: torch.Tensor


class MixedPrecisionCache:
    def __init__(self, group_size=64):
        self.segments = {}
        self.group_size = group_size
        self.pending_bits = 16
        self.frame_id = -1
        self.pack_seconds = 0.0
        self.unpack_seconds = 0.0
        self.retrievals = 0

    def select(self, bits, frame_id=-1):
        if bits not in (4, 8, 16):
            raise ValueError('Invalid precision')
        self.pending_bits, self.frame_id = bits, frame_id

    def get_seq_length(self, layer_idx=0):
        segs = self.segments.get(layer_idx, [])
        return SEGMENT.unpack(bytes(segs[-1].descriptor.tolist()))[3] if segs else 0

    def __len__(self):
        return len(self.segments)

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        history = self.segments.setdefault(layer_idx, [])
        start = self.get_seq_length(layer_idx)
        t = time.perf_counter()
        keys = [unpack(s.key, key_states.dtype, key_states.device) for s in history]
        values = [unpack(s.value, value_states.dtype, value_states.device) for s in history]
        self.unpack_seconds += time.perf_counter() - t
        self.retrievals += len(history)
        t = time.perf_counter()
        k = pack(key_states, self.pending_bits, self.group_size)
        v = pack(value_states, self.pending_bits, self.group_size)
        end = start + key_states.shape[-2]
        raw = SEGMENT.pack(layer_idx, self.frame_id, start, end, self.pending_bits)
        history.append(Segment(k, v, torch.tensor(list(raw), dtype=torch.uint8)))
        self.pack_seconds += time.perf_counter() - t
        return torch.cat([*keys, key_states], dim=-2), torch.cat([*values, value_states], dim=-2)

    def __getitem__(self, layer_idx):
        segs = self.segments[layer_idx]
        return (torch.cat([unpack(s.key) for s in segs], dim=-2), torch.cat([unpack(s.value) for s in segs], dim=-2))

    def accounting(self, frame_only=False):
        payload = metadata = 0
        by_bits = {4: 0, 8: 0, 16: 0}
        for segs in self.segments.values():
            for s in segs:
                _, frame, _, _, bits = SEGMENT.unpack(bytes(s.descriptor.tolist()))
                if frame_only and frame < 0:
                    continue
                payload += s.key.payload_bytes + s.value.payload_bytes
                meta = s.key.metadata_bytes + s.value.metadata_bytes + s.descriptor.numel()
                metadata += meta
                by_bits[bits] += s.key.payload_bytes + s.value.payload_bytes + meta
        return dict(cpu_payload_bytes=payload, cpu_metadata_bytes=metadata, cpu_cache_bytes=payload + metadata,
                    gpu_cache_bytes=0, disk_cache_bytes=0, bytes_by_precision=by_bits)


def cpu_attention_step(cache, q, k_new, v_new, layer=0, scale=0.125):
    """One layer of the CPU path: cache.update then causal GQA SDPA. q [1, Hq, n, 64]."""
    k, v = cache.update(k_new, v_new, layer)
    n, total = q.shape[-2], k.shape[-2]
    mask = torch.arange(total)[None, :] <= (total - n) + torch.arange(n)[:, None]
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scale, enable_gqa=True).transpose(1, 2)
