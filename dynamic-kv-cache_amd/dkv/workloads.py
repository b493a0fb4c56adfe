"""Seeded synthetic inputs for the packed-KV workloads (CPU tensors, bf16).

Values are N(0, 1) with 4 outlier channels per head scaled by 8, the same
channels for every token of that head. Per-tile bit widths are drawn like the
reference's seeded random policy (benchmarks/gpu_evaluate.py:27-29):
random.Random(seed).choices([4, 8, 16], weights=[.4, .4, .2]).
"""
import random

import torch

TILE = 64
OUTLIERS = 4
OUTLIER_GAIN = 8.0


def bit_schedule(seed, tiles, weights=(0.4, 0.4, 0.2)):
    return random.Random(seed).choices([4, 8, 16], weights=list(weights), k=tiles)


def outlier_values(shape, gen, head_axis):
    """N(0,1) fp32 tensor with OUTLIERS channels per head (last axis) scaled by OUTLIER_GAIN, as bf16."""
    x = torch.randn(shape, generator=gen)
    heads = shape[head_axis]
    for h in range(heads):
        ch = torch.randperm(shape[-1], generator=gen)[:OUTLIERS]
        index = [slice(None)] * len(shape)
        index[head_axis] = h
        sub = x[tuple(index)]
        sub[..., ch] *= OUTLIER_GAIN
    return x.to(torch.bfloat16)


def frame_chunk_case(past, seed=0, heads=5, q_heads=15, nq=64):
    """Frame-append attention: history K/V [heads, past, 64], chunk q/k/v, per-tile bits."""
    g = torch.Generator().manual_seed(seed)
    k_hist = outlier_values((heads, past, 64), g, 0)
    v_hist = outlier_values((heads, past, 64), g, 0)
    q = outlier_values((q_heads, nq, 64), g, 0)
    k_new = outlier_values((heads, nq, 64), g, 0)
    v_new = outlier_values((heads, nq, 64), g, 0)
    bits = bit_schedule(seed, (past + TILE - 1) // TILE)
    return dict(k_hist=k_hist, v_hist=v_hist, q=q, k_new=k_new, v_new=v_new, bits=bits)


def candidate_lengths(seed, count=4, low=8, high=24):
    rng = random.Random(seed * 7919 + 1)
    return [rng.randint(low, high) for _ in range(count)]


def candidate_case(bits, seed=0, past=6144, heads=5, q_heads=15, count=4):
    """Candidate scoring: one shared history of uniform width, `count` continuations of 8-24 tokens."""
    lengths = candidate_lengths(seed, count)
    nq = sum(lengths)
    g = torch.Generator().manual_seed(seed)
    k_hist = outlier_values((heads, past, 64), g, 0)
    v_hist = outlier_values((heads, past, 64), g, 0)
    q = outlier_values((q_heads, nq, 64), g, 0)
    k_new = outlier_values((heads, nq, 64), g, 0)
    v_new = outlier_values((heads, nq, 64), g, 0)
    bounds = [0]
    for n in lengths:
        bounds.append(bounds[-1] + n)
    return dict(k_hist=k_hist, v_hist=v_hist, q=q, k_new=k_new, v_new=v_new,
                bits=[bits] * ((past + TILE - 1) // TILE), segments=bounds, lengths=lengths)


def pack_volume(seed=0, layers=32, heads=5, frames=96):
    """Whole-volume pack input: K, V [layers, heads, frames*64, 64] bf16 and per-frame bits."""
    g = torch.Generator().manual_seed(seed)
    tokens = frames * TILE
    k = outlier_values((layers * heads, tokens, 64), g, 0).view(layers, heads, tokens, 64)
    v = outlier_values((layers * heads, tokens, 64), g, 0).view(layers, heads, tokens, 64)
    return dict(k=k, v=v, bits=bit_schedule(seed, frames))
