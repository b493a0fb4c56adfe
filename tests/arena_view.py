"""Reads rows of one (layer, kv, head) back out of a copied arena (test helper)."""
import numpy as np

from dkv.gpu_cache import TILE, row_bytes, slab_bytes, subblock_bytes


def segment_rows(arena, seg, layer, kv, head, layers, heads, upto=None):
    """Payload [rows, row_bytes] uint8 and (offset, scale) [rows, 2] float32 (None for 16-bit)."""
    rows = seg.rows if upto is None else upto
    rb = row_bytes(seg.bits)
    payload, meta = [], []
    for ti in range((rows + TILE - 1) // TILE):
        cap = min(TILE, seg.rows - TILE * ti)
        take = min(TILE, rows - TILE * ti)
        base = seg.offset + ti * slab_bytes(TILE, seg.bits, layers, heads) + \
            ((layer * 2 + kv) * heads + head) * subblock_bytes(cap, seg.bits)
        payload.append(arena[base:base + take * rb].reshape(take, rb))
        if seg.bits < 16:
            m = arena[base + cap * rb:base + cap * rb + take * 8]
            meta.append(np.frombuffer(m.tobytes(), dtype=np.float32).reshape(take, 2))
    return np.concatenate(payload), (np.concatenate(meta) if meta else None)
