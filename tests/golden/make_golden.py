"""Writes the committed golden fixtures of this directory (run from the repository root:
`python tests/golden/make_golden.py`). TEST INFRASTRUCTURE ONLY.

The reference keeps no stored golden vectors for the packed-KV path: its tests assert
properties (tests/test_quantization.py:6-36, tests/test_gpu_backend.py:13-54,82-101). These
fixtures freeze the outputs of the oracle, which tests/test_oracle_pack.py and
tests/test_oracle_attention.py pin against those assertions, closed forms and independent
implementations, and tests/test_golden.py checks the fixtures once more against closed forms and
a numpy restatement. The GPU tests compare libdkv with the stored bytes and values directly.

pack_rows.npz
  x            [64, 64] uint16   bf16 bits of the source rows: half-way ties at 4 and 8 bits,
                                 a constant row, wide / tiny / subnormal / near-fp32-max spans,
                                 one-sided rows, zero minima with both signs (offset -0) and
                                 with +0 only, then seeded N(0, 1) rows with 4 outlier
                                 channels x 8 (the metric's value generator)
  payload{b}   [64, row bytes]   uint8 codes of src/kv_quantization.py:pack at b = 4, 8, 16
  offset{b}, scale{b} [64]       uint32 fp32 bits (b = 4, 8)
  header_bits, header_rows, header [n, 64] uint8: the 64-byte PackedTensor header of a
                                 [1, 1, rows, 64] bf16 tensor packed at that width
attention_chunk.npz
  q [6, 12, 64], k_hist / v_hist [2, 144, 64], k_new / v_new [2, 12, 64]: uint16 bf16 bits
  bits [3]      widths of the history tiles (64, 64, 16 tokens)
  out [12, 6, 64] float32: fp64 dequantize-then-SDPA oracle (2 KV heads, 6 Q heads, a 12-token
                causal chunk after 144 packed history tokens, scale 1/8), rounded to fp32
  cand_bounds [4], out_cand [12, 6, 64] float32: the same 12 tokens as 3 candidate continuations
                of 5, 3 and 4 tokens (bounds 0, 5, 8, 12), each causal within itself and blind to
                the others, all over the full history (the block-diagonal batch of
                src/streaming.py's candidate scoring)
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle.attention import attention, dequant_rows  # noqa: E402
from oracle.kv_quantization import pack, pack_rows  # noqa: E402


def bits_u16(t):
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def outlier_rows(shape, g):
    x = torch.randn(*shape, generator=g)
    x[..., torch.randperm(64, generator=g)[:4]] *= 8
    return x.to(torch.bfloat16)


def pack_rows_case():
    rows = torch.zeros(64, 64)
    rows[0, :16] = torch.tensor([0.0, 15.0] + [k + 0.5 for k in range(14)])  # 4-bit ties, scale 1
    rows[0, 16:] = 7.0
    rows[1] = -2.5  # constant row: scale 1, offset -2.5, codes 0
    rows[2] = torch.tensor([0.0, 255.0] + [k + 0.5 for k in range(0, 120, 2)] + [1.0, 1.0])  # 8-bit ties, scale 1
    rows[3] = torch.linspace(-3e4, 3e4, 64)
    rows[4] = torch.tensor([1e-30 * i for i in range(64)])  # tiny span
    rows[5] = torch.tensor([1e-39 * i for i in range(64)])  # fp32-subnormal values and scale
    rows[6] = torch.linspace(-1e38, 1e38, 64)  # span near the top of the fp32 range
    rows[7] = -torch.arange(1, 65, dtype=torch.float32) / 7  # all negative
    rows[8] = 0.25
    rows[8, 17] = 96.0  # one outlier above a constant floor
    rows[9] = torch.arange(64, dtype=torch.float32) % 3 - 1  # three levels
    rows[10] = torch.arange(64, dtype=torch.float32) / 8
    rows[10, 0], rows[10, 37] = 0.0, -0.0  # zero minimum with both signs: offset -0
    rows[11] = torch.arange(64, dtype=torch.float32) % 5
    rows[11, 50] = 0.0  # zero minimum, only +0: offset +0
    g = torch.Generator().manual_seed(20240611)
    rows[12:] = outlier_rows((52, 64), g).float()
    x = rows.to(torch.bfloat16)
    out = {'x': bits_u16(x)}
    for b in (4, 8, 16):
        payload, off, sc = pack_rows(x, b)
        out[f'payload{b}'] = payload.numpy().copy()
        if b < 16:
            out[f'offset{b}'] = off.numpy().view(np.uint32).copy()
            out[f'scale{b}'] = sc.numpy().view(np.uint32).copy()
    hb, hr, hd = [], [], []
    for b in (4, 8, 16):
        for n in (64, 16):
            hb.append(b)
            hr.append(n)
            hd.append(pack(torch.zeros(1, 1, n, 64, dtype=torch.bfloat16), b, 64).header.numpy())
    out.update(header_bits=np.array(hb, np.int32), header_rows=np.array(hr, np.int32),
               header=np.stack(hd).astype(np.uint8))
    return out


def attention_case():
    g = torch.Generator().manual_seed(77)
    H, G, nq, bits, tiles = 2, 3, 12, [4, 8, 16], [64, 64, 16]
    past = sum(tiles)
    q = (torch.randn(H * G, nq, 64, generator=g)).to(torch.bfloat16)
    k_hist, v_hist = outlier_rows((H, past, 64), g), outlier_rows((H, past, 64), g)
    k_new, v_new = outlier_rows((H, nq, 64), g), outlier_rows((H, nq, 64), g)
    dk, dv, t0 = [], [], 0
    for b, n in zip(bits, tiles):
        dk.append(dequant_rows(*pack_rows(k_hist[:, t0:t0 + n], b), b))
        dv.append(dequant_rows(*pack_rows(v_hist[:, t0:t0 + n], b), b))
        t0 += n
    k = torch.cat(dk + [k_new.float()], 1)
    v = torch.cat(dv + [v_new.float()], 1)
    out = attention(q, k, v, past).float()
    bounds = [0, 5, 8, 12]
    out_cand = attention(q, k, v, past, segments=bounds).float()
    return dict(q=bits_u16(q), k_hist=bits_u16(k_hist), v_hist=bits_u16(v_hist), k_new=bits_u16(k_new),
                v_new=bits_u16(v_new), bits=np.array(bits, np.int32), tiles=np.array(tiles, np.int32),
                out=out.numpy(), cand_bounds=np.array(bounds, np.int32), out_cand=out_cand.numpy())


if __name__ == '__main__':
    np.savez_compressed(os.path.join(HERE, 'pack_rows.npz'), **pack_rows_case())
    np.savez_compressed(os.path.join(HERE, 'attention_chunk.npz'), **attention_case())
    for f in ('pack_rows.npz', 'attention_chunk.npz'):
        print(f, os.path.getsize(os.path.join(HERE, f)), 'bytes')
