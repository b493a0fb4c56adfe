"""Ports of the reference's GPU cache tests (tests/test_gpu_backend.py:13-54) plus fork/growth."""
import pytest
import torch

from conftest import announce
from dkv.gpu_cache import GPUCache

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('bits', [4, 8, 16])
def test_gpu_pack_independent_error_bound(cuda, bits):
    announce(f'error bound bits={bits}')
    torch.manual_seed(71)
    k = torch.randn((1, 3, 19, 64), device=cuda, dtype=torch.bfloat16)
    v = torch.randn((1, 19, 3, 64), device=cuda, dtype=torch.bfloat16).transpose(1, 2)
    c = GPUCache([(bits, 19)], layers=1)
    c.select(bits)
    c.append(k, v, 0)
    rk, rv = c.materialize(0)
    for x, y in [(k, rk), (v, rv)]:
        if bits == 16:
            assert torch.equal(x, y)
        else:
            xf = x.float()
            scale = (xf.amax(-1, keepdim=True) - xf.amin(-1, keepdim=True)) / ((1 << bits) - 1)
            assert torch.all((xf - y.float()).abs() <= scale * .501 + .032)


def test_gpu_branch_does_not_advance_video_cache(cuda):
    announce('fork does not advance base')
    c = GPUCache([(4, 20), (16, 10)], layers=1)
    k = torch.randn(1, 3, 20, 64, device=cuda, dtype=torch.bfloat16)
    c.select(4)
    c.append(k, k, 0)
    before = c.materialize(0)[0].clone()
    branch = c.fork()
    q = torch.randn(1, 3, 5, 64, device=cuda, dtype=torch.bfloat16)
    branch.append(q, q, 0)
    assert c.get_seq_length() == 20 and branch.get_seq_length() == 25
    assert torch.equal(c.materialize(0)[0], before)


def test_online_growth_and_mapping(cuda):
    announce('online growth and mapping')
    c = GPUCache(None, layers=1, max_tokens=512)
    expected = []
    for i, (bits, n) in enumerate([(4, 79), (8, 93), (4, 88), (16, 71)]):
        x = torch.randn(1, 3, n, 64, device=cuda, dtype=torch.bfloat16)
        c.select(bits, i)
        c.append(x, x, 0)
        expected.extend([bits] * n)
    assert c.codes[:len(expected)].tolist() == expected
    assert c.caps[4] >= 167 and c.caps[8] >= 93 and c.caps[16] >= 71
    assert c.get_seq_length() == len(expected)
    before = c.materialize(0)[0].clone()
    branch = c.fork()
    branch.select(16)
    z = torch.randn(1, 3, 90, 64, device=cuda, dtype=torch.bfloat16)
    old_caps = c.caps.copy()
    branch.append(z, z, 0)
    assert c.caps == old_caps
    assert torch.equal(c.materialize(0)[0], before)


def test_growth_keeps_history_and_forks_keep_old_arena(cuda):
    announce('arena growth')
    c = GPUCache(None, layers=2, heads=5, max_tokens=1024, arena_bytes=1 << 16)
    xs = []
    for i in range(6):
        x = torch.randn(1, 5, 64, 64, device=cuda, dtype=torch.bfloat16)
        c.select(16)
        for layer in range(2):
            c.append(x, x, layer)
        xs.append(x)
    assert c.arena_bytes > 1 << 16
    k, _ = c.materialize(1)
    assert torch.equal(k, torch.cat(xs, 2))


def test_candidate_forks_sequentially_reuse_the_qa_region(cuda):
    announce('sequential candidate forks')
    torch.manual_seed(5)
    c = GPUCache(None, layers=1, heads=5, max_tokens=1024)
    h = torch.randn(1, 5, 256, 64, device=cuda, dtype=torch.bfloat16)
    c.select(4)
    c.append(h, h, 0)
    outs = []
    for _ in range(2):
        for n in (9, 17):
            b = c.fork()
            q = torch.randn(1, 15, n, 64, device=cuda, dtype=torch.bfloat16)
            k = torch.randn(1, 5, n, 64, device=cuda, dtype=torch.bfloat16)
            past = b.append(k, k, 0)
            outs.append((past, b.attend(q, k, k, 0, past).clone()))
    assert all(p == 256 for p, _ in outs)
    assert c.get_seq_length() == 256 and len(c.segments) == 1


def test_graph_steps_created_in_inference_mode_step_outside_it(cuda):
    """GraphSteps' device and pinned buffers are ordinary tensors, so graph_step() works whether or
    not the caller is in inference mode (no launch here: nothing was recorded)."""
    announce('cache: graph steps across inference mode')
    c = GPUCache(None, layers=2, heads=5, max_tokens=512)
    with torch.inference_mode():
        c.begin_graph_steps(64, q_heads=15)
        c.select(4, 0)
        assert c.graph_step() == 0
    c.select(8, 1)
    assert c.graph_step() == 64
    with torch.inference_mode():
        c.select(16, 2)
        assert c.graph_step() == 128
    c.end_graph_steps()
    torch.cuda.synchronize()
    assert c.seen == [192, 192] and [s.bits for s in c.segments] == [4, 8, 16]


def test_graph_launches_keep_their_workspace(cuda):
    """A captured attention launch keeps the workspace it recorded: an ordinary call on the same
    cache that needs a larger workspace afterwards (a 300-token chunk) must not move it, so the
    next replay still equals an ordinary call of the same step, bit for bit."""
    announce('cache: graph workspace survives a larger ordinary call')
    g = torch.Generator().manual_seed(41)
    hist = [torch.randn(1, 5, 128, 64, generator=g).to(torch.bfloat16).to(cuda) for _ in range(2)]
    q = torch.randn(1, 15, 64, 64, generator=g).to(torch.bfloat16).to(cuda)
    k = torch.randn(1, 5, 64, 64, generator=g).to(torch.bfloat16).to(cuda)
    v = torch.randn(1, 5, 64, 64, generator=g).to(torch.bfloat16).to(cuda)

    def filled():
        c = GPUCache(None, layers=1, heads=5, max_tokens=1024)
        c.select(4, 0)
        c.append(*hist, 0)
        c.select(8, 1)
        return c

    ref_cache = filled()
    ref = ref_cache.attend(q, k, v, 0, ref_cache.append(k, v, 0))
    c = filled()
    steps = c.begin_graph_steps(64, q_heads=15)
    past = c.graph_step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        c.append(k, v, 0)
        out = c.attend(q, k, v, 0, past)
    steps.upload()
    c.end_graph_steps()
    qb = torch.randn(1, 15, 300, 64, generator=g).to(torch.bfloat16).to(cuda)
    kb = torch.randn(1, 5, 300, 64, generator=g).to(torch.bfloat16).to(cuda)
    c.attend(qb, kb, kb, 0, 128)  # grows the cache's own workspace
    graph.replay()
    torch.cuda.synchronize()
    assert past == 128 and torch.equal(out, ref)


def test_graph_captured_first_survives_a_larger_capture_on_the_same_steps(cuda):
    """Two graphs of 5-token steps captured on one GraphSteps: first on the 12-wave frame-chunk
    kernel (path 'mfma', 51 splits' partials: 0.5 MB), then on the short-chunk kernel, whose fp32
    partials (15 query rows per KV head, 64 workgroups per head for a launch sized by the cache's
    whole tile table: 1.27 MB) need a larger workspace than the first capture's (1 MiB, the least
    the steps allocate; begin_graph_steps() without q_heads reserves nothing ahead). The steps hand
    the second capture a new buffer but keep the first one, so replaying the first graph
    afterwards must still equal a direct call on the same history, bit for bit."""
    announce('cache: first graph survives a second capture that grows the steps workspace')
    g = torch.Generator().manual_seed(43)
    heads, q_heads = 5, 15
    c = GPUCache(None, layers=1, heads=heads, max_tokens=2048)
    q = torch.randn(1, q_heads, 5, 64, generator=g).to(torch.bfloat16).to(cuda)
    kn = torch.randn(1, heads, 5, 64, generator=g).to(torch.bfloat16).to(cuda)
    vn = torch.randn(1, heads, 5, 64, generator=g).to(torch.bfloat16).to(cuda)
    steps = c.begin_graph_steps(5)
    graphs, outs, sizes = [], [], []
    for path in ('mfma', 'short'):
        c.reset()
        c.begin_graph_steps(5, steps=steps)
        c.select(16)
        c.graph_step()
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            c.append(kn, vn, 0)
            c.attend(q, kn, vn, 0, 0, path=path)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            c.append(kn, vn, 0)
            outs.append(c.attend(q, kn, vn, 0, 0, path=path))
        graphs.append(graph)
        sizes.append(steps.ws.numel())
        c.end_graph_steps()
    assert sizes[1] > sizes[0] and steps.retired  # the second capture did need more
    c.reset()
    for bits in (4, 8, 16, 4, 8, 4, 16, 8, 4, 8):  # 10 tiles: several splits either way
        c.select(bits)
        c.append(torch.randn(1, heads, 64, 64, generator=g).to(torch.bfloat16).to(cuda),
                 torch.randn(1, heads, 64, 64, generator=g).to(torch.bfloat16).to(cuda), 0)
    past = c.seen[0]
    for path, graph, out in zip(('mfma', 'short'), graphs, outs):
        f = c.fork()  # same arena and tile table: the steps re-attach to it
        f.begin_graph_steps(5, steps=steps)
        f.select(16)
        f.graph_step()
        graph.replay()
        f.end_graph_steps()
        got = out.clone()
        ref = c.fork().attend(q, kn, vn, 0, past, path=path)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (path, (got.float() - ref.float()).abs().max().item())
