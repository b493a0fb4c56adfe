"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

Each fixture is checked two ways on the CPU:
  - the oracle reproduces it (pack bytes and header bit for bit, attention within 1e-6), so a
    change to the oracle cannot drift away from the data the GPU tests compare against;
  - independently of the oracle: the pack bytes against a numpy float32 statement of
    src/kv_quantization.py:57-71 (offset = min, scale = span / (2^b - 1) or 1, codes = clamped
    round-half-even of (x - offset) / scale, low nibble = even element), the closed forms
    (min -> 0, max -> 2^b - 1, constant rows, exact half-way ties to even, 16-bit = the bf16 bits),
    the header fields of src/kv_quantization.py:12-13,74-76, and the attention output against a
    numpy float64 dequantize-then-softmax with the GQA head map qh // (Hq / H) and the
    bottom-right causal mask (src/gpu_kernels.py:77-105).
"""
import os
import struct

import numpy as np
import pytest
import torch

from oracle.attention import attention, dequant_rows
from oracle.kv_quantization import pack, pack_rows

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden')


def load(name):
    return np.load(os.path.join(GOLDEN, name))  # allow_pickle stays False


def bf16_tensor(u16):
    return torch.from_numpy(u16.view(np.int16).copy()).view(torch.bfloat16)


def bf16_values(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


def codes_of(payload, bits):
    if bits == 4:
        return np.stack((payload & 15, payload >> 4), -1).reshape(payload.shape[0], -1).astype(np.int64)
    return payload.astype(np.int64)


def ieee_min(x):
    """Row minima of float32 rows as IEEE 754-2019 minimum() defines them: a zero minimum is -0 when
    the row holds a -0 (numpy's min leaves that sign to the order of the reduction)."""
    a = x.min(1)
    neg_zero = (x.view(np.uint32) == 0x80000000).any(1)
    return np.where(a == 0, np.where(neg_zero, np.float32(-0.0), np.float32(0.0)), a).astype(np.float32)


def numpy_pack(x, bits):
    """(codes, offset, scale) of float32 rows [n, 64] in float32 arithmetic."""
    a = ieee_min(x)
    span = x.max(1) - a
    levels = np.float32(2 ** bits - 1)
    s = np.where(span > 0, span / levels, np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint((x - a[:, None]) / s[:, None]), 0, 2 ** bits - 1).astype(np.int64)
    return q, a, s


@pytest.mark.parametrize('bits', [4, 8, 16])
def test_oracle_reproduces_pack_fixture(bits):
    d = load('pack_rows.npz')
    payload, off, sc = pack_rows(bf16_tensor(d['x']), bits)
    assert np.array_equal(payload.numpy(), d[f'payload{bits}'])
    if bits < 16:
        assert np.array_equal(off.numpy().view(np.uint32), d[f'offset{bits}'])
        assert np.array_equal(sc.numpy().view(np.uint32), d[f'scale{bits}'])


@pytest.mark.parametrize('bits', [4, 8])
def test_pack_fixture_against_numpy_and_closed_forms(bits):
    d = load('pack_rows.npz')
    x = bf16_values(d['x'])
    codes = codes_of(d[f'payload{bits}'], bits)
    off, sc = d[f'offset{bits}'].view(np.float32), d[f'scale{bits}'].view(np.float32)
    q, a, s = numpy_pack(x, bits)
    assert np.array_equal(off.view(np.uint32), a.view(np.uint32))
    assert np.array_equal(sc.view(np.uint32), s.view(np.uint32))
    assert np.array_equal(codes, q)
    top = 2 ** bits - 1
    rows = np.arange(x.shape[0])
    varying = x.max(1) > x.min(1)
    assert (codes[rows, x.argmin(1)] == 0).all()
    assert (codes[rows[varying], x[varying].argmax(1)] == top).all()
    # constant rows: scale 1, offset = the value, every code 0
    assert not varying[1] and sc[1] == 1.0 and off[1] == -2.5 and (codes[1] == 0).all()
    # error bound of a code: half a step, plus the two fp32 roundings of the affine map q*s + a
    # (each at most half an ulp of its result, so 2^-23 (|q s| + |a|) together)
    qs = codes.astype(np.float32) * sc[:, None]
    deq = qs + off[:, None]
    ok = np.isfinite(x).all(1) & (np.abs(x).max(1) < 1e37)
    err = np.abs(deq - x)[ok]
    slop = (np.abs(qs) + np.abs(off)[:, None])[ok] * 2 ** -23
    assert (err <= (sc[ok, None] * 0.5) * (1 + 2 ** -20) + slop).all()


def test_pack_fixture_ties_round_to_even():
    d = load('pack_rows.npz')
    x = bf16_values(d['x'])
    for row, bits in ((0, 4), (2, 8)):  # offset 0 and scale 1 by construction
        codes = codes_of(d[f'payload{bits}'], bits)[row]
        assert d[f'scale{bits}'][row].view(np.float32) == 1.0 and d[f'offset{bits}'][row] == 0
        ties = np.nonzero(x[row] != np.floor(x[row]))[0]
        assert len(ties) >= 14
        for i in ties:
            lo = int(np.floor(x[row, i]))
            assert codes[i] == (lo if lo % 2 == 0 else lo + 1), (row, i, x[row, i], codes[i])


def test_pack_fixture_16bit_is_the_bf16_bits():
    d = load('pack_rows.npz')
    assert np.array_equal(d['payload16'], d['x'].astype('<u2').view(np.uint8).reshape(64, 128))


def test_header_fixture_fields_and_oracle():
    d = load('pack_rows.npz')
    for bits, rows, raw in zip(d['header_bits'], d['header_rows'], d['header']):
        magic, version, b, dtype, ndim, *rest = struct.unpack('<4sBBBB4qQQQ', raw.tobytes())
        assert (magic, version, b, dtype, ndim) == (b'DKVC', 1, bits, 2, 4)
        shape, group, numel, groups = rest[:4], rest[4], rest[5], rest[6]
        assert shape == [1, 1, rows, 64] and group == 64 and numel == rows * 64
        assert groups == (rows if bits < 16 else 0)  # 16-bit keeps no groups (src/kv_quantization.py:55)
        oracle = pack(torch.zeros(1, 1, int(rows), 64, dtype=torch.bfloat16), int(bits), 64).header.numpy()
        assert np.array_equal(oracle, raw)


def numpy_attention(d, bounds=None):
    """float64 softmax(q k^T / 8 + bottom-right causal mask) v over the dequantized history; with
    candidate bounds, chunk token i sees the chunk tokens of its own candidate up to itself."""
    kh, vh = bf16_values(d['k_hist']), bf16_values(d['v_hist'])
    parts_k, parts_v, t0 = [], [], 0
    for b, n in zip(d['bits'], d['tiles']):
        for src, dst in ((kh, parts_k), (vh, parts_v)):
            rows = src[:, t0:t0 + n].reshape(-1, 64)
            if b == 16:
                deq = rows
            else:
                q, a, s = numpy_pack(rows, int(b))
                deq = q.astype(np.float32) * s[:, None] + a[:, None]
            dst.append(deq.reshape(src.shape[0], n, 64))
        t0 += n
    past = t0
    k = np.concatenate(parts_k + [bf16_values(d['k_new'])], 1).astype(np.float64)
    v = np.concatenate(parts_v + [bf16_values(d['v_new'])], 1).astype(np.float64)
    q = bf16_values(d['q']).astype(np.float64)
    hq, nq, _ = q.shape
    group = hq // k.shape[0]
    out = np.zeros((nq, hq, 64))
    starts = np.zeros(nq, np.int64)
    if bounds is not None:
        for lo, hi in zip(bounds[:-1], bounds[1:]):
            starts[lo:hi] = lo
    for h in range(hq):
        s = q[h] @ k[h // group].T / 8
        for i in range(nq):
            s[i, past + i + 1:] = -np.inf
            s[i, past:past + starts[i]] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        out[:, h] = (p / p.sum(1, keepdims=True)) @ v[h // group]
    return out


def test_attention_fixture_against_numpy():
    d = load('attention_chunk.npz')
    ref = numpy_attention(d)
    assert np.abs(ref - d['out']).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    cand = numpy_attention(d, d['cand_bounds'].tolist())
    assert np.abs(cand - d['out_cand']).max() <= 1e-5 * max(1.0, np.abs(cand).max())
    # the first candidate's rows see exactly what the plain chunk's first rows see
    assert np.array_equal(d['out_cand'][:5], d['out'][:5])


def test_oracle_reproduces_attention_fixture():
    d = load('attention_chunk.npz')
    k_hist, v_hist = bf16_tensor(d['k_hist']), bf16_tensor(d['v_hist'])
    dk, dv, t0 = [], [], 0
    for b, n in zip(d['bits'].tolist(), d['tiles'].tolist()):
        dk.append(dequant_rows(*pack_rows(k_hist[:, t0:t0 + n], b), b))
        dv.append(dequant_rows(*pack_rows(v_hist[:, t0:t0 + n], b), b))
        t0 += n
    k = torch.cat(dk + [bf16_tensor(d['k_new']).float()], 1)
    v = torch.cat(dv + [bf16_tensor(d['v_new']).float()], 1)
    out = attention(bf16_tensor(d['q']), k, v, t0).float().numpy()
    assert np.abs(out - d['out']).max() <= 1e-6
    cand = attention(bf16_tensor(d['q']), k, v, t0, segments=d['cand_bounds'].tolist()).float().numpy()
    assert np.abs(cand - d['out_cand']).max() <= 1e-6


def test_committed_script_regenerates_the_fixtures():
    """tests/golden/make_golden.py, run again, gives the committed arrays (pack bit for bit; the
    fp64 attention outputs, stored as fp32, within 1e-6 across BLAS builds)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location('make_golden', os.path.join(GOLDEN, 'make_golden.py'))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    for name, fresh in (('pack_rows.npz', mod.pack_rows_case()), ('attention_chunk.npz', mod.attention_case())):
        stored = load(name)
        assert sorted(stored.files) == sorted(fresh), name
        for key, value in fresh.items():
            if value.dtype.kind == 'f':
                assert np.abs(value - stored[key]).max() <= 1e-6, (name, key)
            else:
                assert np.array_equal(value, stored[key]), (name, key)
