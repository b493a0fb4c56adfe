"""Pins oracle/kv_quantization.py (the restated reference quantizer) on the CPU."""
import math

import numpy as np
import pytest
import torch

from oracle.kv_quantization import HEADER, pack, pack_rows, unpack
from dkv.workloads import outlier_values


# -- the reference's own assertions (tests/test_quantization.py:6-36) ------------------------
@pytest.mark.parametrize('bits', [4, 8, 16])
def test_payload_bytes_and_roundtrip(bits):
    torch.manual_seed(10)
    x = torch.randn(1, 3, 7, 65)
    p = pack(x, bits, 64)
    assert p.payload_bytes == math.ceil(x.numel() * bits / 8)
    assert p.payload.dtype == torch.uint8 and p.payload.is_contiguous()
    assert p.metadata_bytes == HEADER.size + (0 if bits == 16 else 8 * math.ceil(x.numel() / 64))
    out = unpack(p, torch.float32)
    assert out.shape == x.shape
    if bits == 16:
        assert torch.equal(out, x.half().float())
    else:
        err = (out - x).abs().flatten()
        scale = p.scales.repeat_interleave(64)[:x.numel()]
        assert torch.all(err <= scale / 2 + 1e-5)


@pytest.mark.parametrize('bits', [4, 8, 16])
def test_constant_group_exact(bits):
    x = torch.full((1, 1, 3, 17), -2.5)
    assert torch.equal(unpack(pack(x, bits), torch.float32), x)


def test_bfloat16_preserved_exactly():
    x = torch.randn(1, 3, 5, 64).bfloat16()
    assert torch.equal(unpack(pack(x, 16)), x)


@pytest.mark.parametrize('bad', [float('nan'), float('inf'), float('-inf')])
def test_reject_nonfinite(bad):
    with pytest.raises(ValueError):
        pack(torch.full((1, 1, 1, 1), bad), 4)


def test_reject_bad_arguments():
    with pytest.raises(ValueError):
        pack(torch.zeros(1, 1, 1, 64), 5)
    with pytest.raises(ValueError):
        pack(torch.zeros(1, 1, 64), 4)
    with pytest.raises(ValueError):
        pack(torch.zeros(1, 1, 1, 64), 4, group_size=0)
    with pytest.raises(ValueError):
        pack(torch.zeros(1, 1, 0, 64), 8)


def ieee_min(x):
    """Row minima of float32 rows as IEEE 754-2019 minimum() defines them: a zero minimum is -0 when
    the row holds a -0 (numpy's min leaves that sign to the order of the reduction)."""
    a = x.min(1)
    neg_zero = (x.view(np.uint32) == 0x80000000).any(1)
    return np.where(a == 0, np.where(neg_zero, np.float32(-0.0), np.float32(0.0)), a).astype(np.float32)


# -- independent restatement: numpy float32 ----------------------------------------------------
def numpy_pack_rows(x, bits):
    """Row-wise affine codes computed with numpy's IEEE float32 ops (not torch)."""
    x = np.asarray(x, dtype=np.float32)
    levels = np.float32((1 << bits) - 1)
    a = ieee_min(x)
    span = (x.max(axis=1) - a).astype(np.float32)
    s = np.where(span > 0, span / levels, np.float32(1)).astype(np.float32)
    q = np.clip(np.rint((x - a[:, None]) / s[:, None]), 0, levels).astype(np.uint8)
    return q, a, s


@pytest.mark.parametrize('bits', [4, 8])
@pytest.mark.parametrize('seed', [0, 1, 2])
def test_matches_numpy_float32(bits, seed):
    g = torch.Generator().manual_seed(seed)
    x = outlier_values((5, 257, 64), g, 0)
    payload, off, sc = pack_rows(x, bits)
    q, a, s = numpy_pack_rows(x.float().reshape(-1, 64).numpy(), bits)
    assert np.array_equal(off.reshape(-1).numpy().view(np.uint32), a.view(np.uint32))
    assert np.array_equal(sc.reshape(-1).numpy().view(np.uint32), s.view(np.uint32))
    if bits == 8:
        assert np.array_equal(payload.reshape(-1, 64).numpy(), q)
    else:
        p = payload.reshape(-1, 32).numpy()
        assert np.array_equal(p & 15, q[:, 0::2]) and np.array_equal(p >> 4, q[:, 1::2])


# -- closed forms -------------------------------------------------------------------------------
def test_half_way_ties_round_to_even_4bit():
    # min 0, max 15 -> scale exactly 1; k + 0.5 is an exact tie and must round to even.
    row = [0.0, 15.0] + [k + 0.5 for k in range(14)] + [7.0] * 48
    payload, off, sc = pack_rows(torch.tensor(row).view(1, 64), 4)
    codes = torch.stack((payload & 15, payload >> 4), -1).flatten().tolist()
    assert codes[:16] == [0, 15, 0, 2, 2, 4, 4, 6, 6, 8, 8, 10, 10, 12, 12, 14]
    assert off.item() == 0.0 and sc.item() == 1.0


def test_half_way_ties_round_to_even_8bit_scaled():
    # min -3, max 507 -> span 510, scale exactly 2; x = -3 + 2(k + 0.5) is a tie at k + 0.5.
    ties = [-3.0 + 2.0 * (k + 0.5) for k in range(60)]
    row = [-3.0, 507.0] + ties + [1.0, 1.0]
    payload, off, sc = pack_rows(torch.tensor(row).view(1, 64), 8)
    codes = payload.flatten().tolist()
    assert codes[:2] == [0, 255] and sc.item() == 2.0
    assert codes[2:62] == [k if k % 2 == 0 else k + 1 for k in range(60)]


def test_nibble_order_low_is_even_element():
    row = torch.arange(16, dtype=torch.float32).repeat(4).view(1, 64)
    payload, _, _ = pack_rows(row, 4)
    assert payload.flatten()[:8].tolist() == [0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE]


@pytest.mark.parametrize('bits', [4, 8])
def test_min_and_max_map_to_code_ends(bits):
    g = torch.Generator().manual_seed(3)
    x = outlier_values((4, 100, 64), g, 0).float().view(-1, 64)
    payload, off, sc = pack_rows(x, bits)
    q = torch.stack((payload & 15, payload >> 4), -1).flatten(-2) if bits == 4 else payload
    lo, hi = x.argmin(1), x.argmax(1)
    rows = torch.arange(x.shape[0])
    assert torch.all(q[rows, lo] == 0)
    assert torch.all(q[rows, hi] == (1 << bits) - 1)
    assert torch.equal(off, x.amin(1))


def test_header_bytes_literal():
    p = pack(torch.zeros(1, 3, 7, 65), 4)
    fields = [1, 3, 7, 65, 64, 1365, 22]
    expect = b'DKVC' + bytes([1, 4, 3, 4]) + b''.join(v.to_bytes(8, 'little') for v in fields)
    assert bytes(p.header.tolist()) == expect and len(expect) == 64
    p16 = pack(torch.zeros(1, 2, 3, 64, dtype=torch.bfloat16), 16)
    assert bytes(p16.header.tolist())[:8] == b'DKVC' + bytes([1, 16, 2, 4])
    assert p16.fields() == (16, 2, (1, 2, 3, 64), 64, 384, 0)


@pytest.mark.parametrize('bits', [4, 8])
def test_zero_minimum_takes_the_ieee_minimum_sign(bits):
    """A row whose minimum is zero gets offset -0 when it holds a -0 and +0 otherwise, wherever
    the zeros sit (torch's amin leaves that sign to its reduction order); codes and scales do not
    depend on it."""
    g = torch.Generator().manual_seed(7)
    base = torch.rand(6, 64, generator=g) + 0.5
    rows = base.clone()
    rows[0, 3], rows[0, 40] = 0.0, -0.0  # both signs, +0 first
    rows[1, 3], rows[1, 40] = -0.0, 0.0  # both signs, -0 first
    rows[2, 63] = -0.0                   # only -0
    rows[3, 0] = 0.0                     # only +0
    rows[4, :] = -0.0                    # constant -0: scale 1
    rows[5, 10], rows[5, 11] = -0.0, -1.0  # negative minimum: the zero's sign is irrelevant
    x = rows.bfloat16()
    payload, off, sc = pack_rows(x, bits)
    bits_of = off.view(torch.int32).tolist()
    assert bits_of[:5] == [-0x80000000, -0x80000000, -0x80000000, 0, -0x80000000]
    assert off[5].item() == -1.0
    plus = x.float().abs().where(x.float() == 0, x.float()).bfloat16()  # every -0 made +0
    p2, o2, s2 = pack_rows(plus, bits)
    assert torch.equal(payload, p2) and torch.equal(sc, s2)
    assert o2.view(torch.int32)[:5].tolist() == [0, 0, 0, 0, 0]
