"""Pins oracle/cpu_path.py with the reference's own assertions (tests/test_cache.py:7-27)."""
import torch

from oracle.cpu_path import SEGMENT, MixedPrecisionCache, cpu_attention_step
from oracle.attention import attention
from oracle.kv_quantization import unpack


def test_mixed_retrieval_shapes_positions_and_reuse():
    torch.manual_seed(7)
    c = MixedPrecisionCache()
    expected_k = []
    for frame, bits in enumerate([4, 8, 16]):
        c.select(bits, frame)
        k, v = torch.randn(1, 3, 7, 64).bfloat16(), torch.randn(1, 3, 7, 64).bfloat16()
        out_k, out_v = c.update(k, v, 0)
        assert out_k.shape == out_v.shape == (1, 3, (frame + 1) * 7, 64)
        assert torch.equal(out_k[..., -7:, :], k)
        if frame:
            assert torch.equal(out_k[..., :-7, :], torch.cat(expected_k, dim=-2))
        expected_k.append(unpack(c.segments[0][-1].key))
        record = SEGMENT.unpack(bytes(c.segments[0][-1].descriptor.tolist()))
        assert record == (0, frame, frame * 7, (frame + 1) * 7, bits)
    assert c.get_seq_length() == 21 and c.retrievals == 3
    assert torch.equal(c[0][0], torch.cat(expected_k, dim=-2))
    a = c.accounting()
    assert a['cpu_cache_bytes'] == a['cpu_payload_bytes'] + a['cpu_metadata_bytes']
    assert all(a['bytes_by_precision'][b] > 0 for b in [4, 8, 16])
    assert SEGMENT.size == 32


def test_cpu_step_matches_oracle_attention():
    torch.manual_seed(3)
    c = MixedPrecisionCache()
    hk, hv = [], []
    for bits in (4, 8, 16):
        c.select(bits)
        k, v = torch.randn(1, 5, 64, 64), torch.randn(1, 5, 64, 64)
        c.update(k, v, 0)
        hk.append(unpack(c.segments[0][-1].key, torch.float32))
        hv.append(unpack(c.segments[0][-1].value, torch.float32))
    q, kn, vn = torch.randn(1, 15, 64, 64), torch.randn(1, 5, 64, 64), torch.randn(1, 5, 64, 64)
    c.select(16)
    got = cpu_attention_step(c, q, kn, vn)
    k = torch.cat(hk + [kn], 2)[0]
    v = torch.cat(hv + [vn], 2)[0]
    exact = attention(q[0], k, v, past=192)
    assert torch.allclose(got[0].double(), exact, atol=1e-5)
