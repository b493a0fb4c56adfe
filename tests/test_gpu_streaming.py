"""The decoder side of the path: a random-init Llama running on the packed cache.

Mirrors the reference's integration checks: the packed fused path against the
upstream DynamicCache + SDPA forward (scripts/gpu_model_smoke.py:23-24 compares
fused and native label scores with a 0.3 bound), and candidate scoring
(src/streaming.py:209-225).

Tolerances:
  all-16-bit packed cache (precision='fp32') vs native DynamicCache: logits max-abs <= 0.05.
    Both run the same bf16 GEMMs; only attention differs (fp32-accurate packed kernel vs
    torch SDPA in bf16), so the logits agree to a few bf16 ulps of their ~N(0, 1) scale.
  batched candidate scoring vs one fork per candidate: mean log-likelihoods within 2e-2. The
    chunk's GEMMs run at different M, which can change bf16 rounding; the scores are means
    over 8-24 tokens of log-softmax over a 512-word vocabulary (|score| ~ 6).
"""
import pytest
import torch

from conftest import announce
from dkv.gpu_cache import GPUCache
from dkv.streaming import StreamingDecoder, build_decoder

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, hidden=384, heads=6, kv_heads=2, intermediate=768, vocab=512, max_positions=4096)


def frames_for(model, n_frames, seed, tokens=64):
    """Frame embeddings: embeddings of random token ids (the model's own input scale)."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, model.config.vocab_size, (n_frames, tokens), generator=g)
    emb = model.model.get_input_embeddings()(ids.to(model.lm_head.weight.device))
    return [emb[i:i + 1] for i in range(n_frames)]


def native_logits(model, prefix, frames, question):
    from transformers import DynamicCache
    cache = DynamicCache()
    with torch.inference_mode():
        model.model(input_ids=prefix.cuda(), past_key_values=cache, use_cache=True)
        for emb in frames:
            model.model(inputs_embeds=emb, past_key_values=cache, use_cache=True)
        out = model.model(input_ids=question.cuda(), past_key_values=cache, use_cache=True)
        return model.lm_head(out.last_hidden_state).float()


def test_packed_16bit_matches_native_decoder(cuda):
    announce('streaming: 16-bit packed vs native DynamicCache, 2-layer decoder')
    model = build_decoder(**SMALL, seed=3)
    g = torch.Generator().manual_seed(4)
    prefix = torch.randint(0, 512, (1, 16), generator=g)
    question = torch.randint(0, 512, (1, 24), generator=g)
    frames = frames_for(model, 5, seed=5)
    ref = native_logits(model, prefix, frames, question)
    dec = StreamingDecoder(model, precision='fp32')
    cache = dec.ingest(prefix, frames, [16] * len(frames))
    got = dec.forward(cache, ids=question, logits=question.shape[1])
    torch.cuda.synchronize()
    assert cache.get_seq_length() == 16 + 5 * 64 + 24
    err = (got - ref).abs().max().item()
    assert err <= 0.05, err


def test_batched_candidates_match_sequential_forks(cuda):
    announce('streaming: batched candidate scoring vs sequential forks')
    model = build_decoder(**SMALL, seed=6)
    dec = StreamingDecoder(model, precision='fp32')
    g = torch.Generator().manual_seed(7)
    prefix = torch.randint(0, 512, (1, 16), generator=g)
    frames = frames_for(model, 4, seed=8)
    cache = dec.ingest(prefix, frames, [4, 8, 16, 4])
    question = torch.randint(0, 512, (1, 20), generator=g)
    cands = [torch.randint(0, 512, (1, n), generator=g) for n in (9, 17, 12, 24)]
    seen = cache.get_seq_length()
    seq = dec.answer(cache, question, cands)
    bat = dec.answer_batched(cache, question, cands)
    torch.cuda.synchronize()
    assert cache.get_seq_length() == seen  # forks never advance the base cache
    assert torch.isfinite(seq).all() and torch.isfinite(bat).all()
    assert (seq - bat).abs().max().item() <= 2e-2, (seq, bat)


def test_mixed_width_ingest_tracks_the_schedule(cuda):
    announce('streaming: mixed-width ingest accounting')
    model = build_decoder(**SMALL, seed=9)
    dec = StreamingDecoder(model)
    prefix = torch.randint(0, 512, (1, 16))
    bits = [4, 8, 16, 4, 8, 4]
    cache = dec.ingest(prefix, frames_for(model, len(bits), seed=10), bits)
    acct = cache.accounting()
    assert acct['precision_token_counts'] == {4: 3 * 64, 8: 2 * 64, 16: 64 + 16}
    assert [s.bits for s in cache.segments] == [16] + bits
    logits = dec.forward(cache, ids=torch.randint(0, 512, (1, 8)), logits=8)
    assert torch.isfinite(logits).all()


@pytest.mark.parametrize('precision', ['fp32', 'bf16'])
@pytest.mark.parametrize('pipeline', [1, 2, 3, 8])
def test_graph_replayed_ingest_matches_eager(cuda, pipeline, precision):
    """Frames 2..n replay captured HIP graphs of the decoder forward (launches read their step
    parameters from the device, and the attention runs the splits the host plan would choose for
    the current history); with pipeline=k, k consecutive frames replay one graph of their
    forwards, each a layer behind the one before on its own stream. The cache bookkeeping, the
    packed bytes and the logits must equal the eager ingest's exactly, and a second request that
    reuses the captured graphs on the reset cache must reproduce the first bit for bit. (At bf16
    precision a replayed chunk whose history runs one split of a launch sized for more must store
    its output like a direct one-split call: the 16-token prefix over an empty history.)"""
    announce(f'streaming: graph-replayed ingest vs eager, two requests, pipeline={pipeline}, precision={precision}')
    model = build_decoder(**SMALL, seed=12)
    dec = StreamingDecoder(model, precision=precision, pipeline=pipeline)
    g = torch.Generator().manual_seed(13)
    prefix = torch.randint(0, 512, (1, 16), generator=g)
    question = torch.randint(0, 512, (1, 24), generator=g)
    bits = [4, 8, 16, 4, 8, 4]
    frames = frames_for(model, len(bits), seed=14)

    def run():
        cache = dec.ingest(prefix, frames, bits)
        logits = dec.forward(cache.fork(), ids=question, logits=question.shape[1])
        torch.cuda.synchronize()
        return cache, logits

    eager_cache, eager = run()
    dec.graphs = True
    graph_cache, first = run()
    assert graph_cache is dec._cache
    # frames 1-5: alone; as pairs 1-2, 3-4 and frame 5 alone; as groups 1-3 and 4-5; as one group
    # of 5 (the default depth, 8: more streams than the process's 4 hardware queues)
    expect = {1: ({64}, set()), 2: ({64}, {(64, 2)}), 3: (set(), {(64, 3), (64, 2)}),
              8: (set(), {(64, 5)})}[pipeline]
    assert (set(dec._graphs), set(dec._group_graphs)) == expect
    assert graph_cache.plan == eager_cache.plan and graph_cache.seen == eager_cache.seen
    assert [s.frame for s in graph_cache.segments] == [s.frame for s in eager_cache.segments]
    assert graph_cache.accounting()['precision_token_counts'] == eager_cache.accounting()['precision_token_counts']
    for layer in (0, SMALL['layers'] - 1):
        for a, b in zip(graph_cache.materialize(layer), eager_cache.materialize(layer)):
            assert torch.equal(a, b)
    assert torch.equal(first, eager), (first - eager).abs().max().item()
    _, second = run()  # the prefix now replays a captured 16-token forward as well
    assert 16 in dec._graphs
    assert torch.equal(first, second)
    dec.graphs = False


def test_pipelined_ingest_with_mixed_frame_lengths(cuda):
    """Groups form only from consecutive frames of one length: with frames of 64, 64, 40, 64, 64,
    64, 64, 64, 24 tokens and pipeline=3, frames 1-2 and 3-5 replay as groups, 6-7 as a pair,
    40- and 24-token frames alone. Cache bytes and logits equal the eager ingest's."""
    announce('streaming: pipelined ingest, mixed frame lengths')
    model = build_decoder(**SMALL, seed=41)
    dec = StreamingDecoder(model, precision='fp32', pipeline=3)
    g = torch.Generator().manual_seed(42)
    prefix = torch.randint(0, 512, (1, 16), generator=g)
    question = torch.randint(0, 512, (1, 12), generator=g)
    lengths = [64, 64, 40, 64, 64, 64, 64, 64, 24]
    bits = [4, 8, 16, 8, 4, 4, 16, 8, 4]
    frames = [f[:, :n] for f, n in zip(frames_for(model, len(lengths), seed=43), lengths)]

    def run():
        cache = dec.ingest(prefix, frames, bits)
        logits = dec.forward(cache.fork(), ids=question, logits=question.shape[1])
        torch.cuda.synchronize()
        return cache, logits

    eager_cache, eager = run()
    dec.graphs = True
    for request in range(2):
        cache, got = run()
        assert [(s.start, s.rows, s.bits) for s in cache.segments] == \
            [(s.start, s.rows, s.bits) for s in eager_cache.segments]
        for layer in (0, SMALL['layers'] - 1):
            for a, b in zip(cache.materialize(layer), eager_cache.materialize(layer)):
                assert torch.equal(a, b)
        assert torch.equal(got, eager), (request, (got - eager).abs().max().item())
    assert {(64, 3), (64, 2)} <= set(dec._group_graphs)
    dec.graphs = False


def test_graph_replayed_answers_match_eager(cuda):
    """With graphs=True the question and candidate forwards on forks of the reused cache replay
    captured graphs (forward + lm_head) from the third time a shape is seen; every protocol's
    scores must equal the eager ones bit for bit on each of three requests."""
    announce('streaming: graph-replayed answers vs eager, three requests')
    model = build_decoder(**SMALL, seed=31)
    dec = StreamingDecoder(model, precision='fp32')
    g = torch.Generator().manual_seed(32)
    prefix = torch.randint(0, 512, (1, 16), generator=g)
    question = torch.randint(0, 512, (1, 12), generator=g)
    cands = [torch.randint(0, 512, (1, n), generator=g) for n in (5, 9, 7)]
    bits = [4, 8, 16, 4]
    frames = frames_for(model, len(bits), seed=33)

    def request():
        cache = dec.ingest(prefix, frames, bits)
        out = (dec.answer_batched(cache, question, cands), dec.answer(cache, question, cands),
               dec.answer_labels(cache, question, [3, 5, 7]))
        torch.cuda.synchronize()
        return out

    eager = request()
    dec.graphs = True
    for i in range(3):
        got = request()
        for a, b in zip(got, eager):
            assert torch.equal(a, b), (i, a, b)
    # question (shared by the batched and label protocols), candidates batch, three question+candidate
    assert len(dec._qa_graphs) == 5
    dec.graphs = False


def test_label_protocol_and_calibration_prior(cuda):
    """The 'label' protocol reads the last position's logits at the label ids on a fork (the base
    cache keeps its length), and the calibration prior is the candidate scoring on a prefix-only
    cache: it must equal answer() on such a cache built by hand."""
    announce('streaming: label protocol and calibration prior')
    model = build_decoder(**SMALL, seed=15)
    dec = StreamingDecoder(model, precision='fp32')
    g = torch.Generator().manual_seed(16)
    prefix = torch.randint(0, 512, (1, 16), generator=g)
    question = torch.randint(0, 512, (1, 20), generator=g)
    labels = [3, 77, 101, 250]
    cache = dec.ingest(prefix, frames_for(model, 3, seed=17), [4, 8, 16])
    seen = cache.get_seq_length()
    got = dec.answer_labels(cache, question, labels)
    full = dec.forward(cache.fork(), ids=question, logits=1)[0, -1]
    torch.cuda.synchronize()
    assert cache.get_seq_length() == seen
    assert torch.equal(got, full[torch.tensor(labels, device=full.device)])
    cands = [torch.randint(0, 512, (1, n), generator=g) for n in (9, 13)]
    prior = dec.prior_scores(prefix, question, cands)
    bare = dec.create_cache(128)
    bare.select(16, -1)
    dec.forward(bare, ids=prefix)
    torch.cuda.synchronize()
    assert torch.equal(prior, dec.answer(bare, question, cands))


def test_compat_update_returns_dequantized_history_and_the_native_chunk(cuda):
    """GPUCache.update (the HF Cache.update compat path, src/gpu_cache.py:114-119): append, then
    return (k, v) [1, H, seen, 64] whose earlier rows are the dequantized history materialize()
    returns and whose last n rows are the native chunk, bit for bit, at every width."""
    announce('compat: GPUCache.update rows')
    torch.manual_seed(51)
    c = GPUCache(None, layers=2, heads=5, max_tokens=1024, backend='sdpa')
    seen = 0
    for bits, n in [(4, 64), (8, 37), (16, 64), (4, 1), (8, 90)]:
        k = torch.randn(1, 5, n, 64, device=cuda, dtype=torch.bfloat16)
        v = torch.randn(1, n, 5, 64, device=cuda, dtype=torch.bfloat16).transpose(1, 2)  # strided V
        c.select(bits)
        for layer in range(2):
            rk, rv = c.update(k, v, layer)
            assert rk.shape == rv.shape == (1, 5, seen + n, 64) and rk.dtype == torch.bfloat16
            hk, hv = c.materialize(layer)
            assert torch.equal(rk[:, :, :seen], hk[:, :, :seen]) and torch.equal(rv[:, :, :seen], hv[:, :, :seen])
            assert torch.equal(rk[:, :, seen:], k) and torch.equal(rv[:, :, seen:], v)
            if bits < 16:  # the cache itself holds the quantized rows; update() hands back the native ones
                assert not torch.equal(hk[:, :, seen:], k)
        seen += n
    assert c.get_seq_length() == seen


def test_sdpa_backend_decoder_matches_native_and_fused(cuda):
    """The decoder on GPUCache(backend='sdpa'): install_packed_attention falls through to the
    upstream attention forward, which calls GPUCache.update and runs SDPA on the returned K/V
    (src/gpu_cache.py:174-178, the reference's 'reconstruct' mode, src/streaming.py:165).
    All-16-bit: the K/V are the native ones bit for bit, so logits equal native DynamicCache's
    within 0.05 (the 16-bit case of test_packed_16bit_matches_native_decoder). Mixed widths: within
    0.3 of the fused packed backend on the same schedule (the reference's fused-vs-native score
    bound, scripts/gpu_model_smoke.py:23-24)."""
    announce('compat: backend=sdpa decoder vs native and fused')
    model = build_decoder(**SMALL, seed=52)
    g = torch.Generator().manual_seed(53)
    prefix = torch.randint(0, 512, (1, 16), generator=g)
    question = torch.randint(0, 512, (1, 24), generator=g)
    frames = frames_for(model, 4, seed=54)
    dec = StreamingDecoder(model)
    ref = native_logits(model, prefix, frames, question)
    total = 16 + 4 * 64 + 24 + 64
    sdpa = dec.ingest(prefix, frames, [16] * 4, cache=dec.create_cache(total, backend='sdpa'))
    got = dec.forward(sdpa, ids=question, logits=question.shape[1])
    torch.cuda.synchronize()
    assert sdpa.get_seq_length() == 16 + 4 * 64 + 24
    err = (got - ref).abs().max().item()
    print(f'[compat] sdpa backend 16-bit vs native: max-abs {err:.4e}', flush=True)
    assert err <= 0.05, err
    bits = [4, 8, 16, 4]
    mixed = dec.ingest(prefix, frames, bits, cache=dec.create_cache(total, backend='sdpa'))
    got = dec.forward(mixed, ids=question, logits=question.shape[1])
    fused = dec.ingest(prefix, frames, bits)
    want = dec.forward(fused, ids=question, logits=question.shape[1])
    torch.cuda.synchronize()
    err = (got - want).abs().max().item()
    print(f'[compat] sdpa backend mixed widths vs fused: max-abs {err:.4e}', flush=True)
    assert torch.isfinite(got).all() and err <= 0.3, err


@pytest.mark.parametrize('n_frames', [16, 64, 96])
def test_full_size_decoder_configuration(cuda, n_frames):
    """The metric's end-to-end decoder at its configured size (build_decoder() defaults: 32 layers,
    hidden 960, 15 / 5 heads, SwiGLU 2560, vocab 49280) over 16, 64 and 96 mixed-width frames, the
    frame counts bench.py times (src/streaming.py:168-237; 96 frames reach 6,184 cache tokens, 97
    tiles, and the pipelined replays run 12 history splits):
      - pipelined graph replays (8 frames per group) ingest the cache bit for bit like eager
        launches (arena bytes, bookkeeping, question logits);
      - an all-16-bit packed cache at precision='fp32' gives question logits within 0.25 of native
        DynamicCache + SDPA (32 layers of bf16 GEMMs and bf16 SDPA against the fp32-accurate packed
        kernel; the 2-layer decoder holds 0.05);
      - batched candidate scores equal one fork per candidate within 2e-2."""
    announce(f'streaming: full-size decoder, {n_frames} frames')
    from dkv.workloads import bit_schedule, candidate_lengths
    model = build_decoder(seed=0)
    vocab = model.config.vocab_size
    g = torch.Generator().manual_seed(61)
    prefix = torch.randint(0, vocab, (1, 16), generator=g)
    question = torch.randint(0, vocab, (1, 24), generator=g)
    cands = [torch.randint(0, vocab, (1, n), generator=g) for n in candidate_lengths(0, 4)]
    frames = frames_for(model, n_frames, seed=62)
    bits = bit_schedule(n_frames, n_frames)
    assert set(bits) == {4, 8, 16}

    dec = StreamingDecoder(model, pipeline=8)

    def request():
        cache = dec.ingest(prefix, frames, bits)
        logits = dec.forward(cache.fork(), ids=question, logits=question.shape[1])
        torch.cuda.synchronize()
        return cache, logits

    eager_cache, eager = request()
    eager_arena = eager_cache.arena[:eager_cache.arena_used].clone()
    eager_plan, eager_tiles = list(eager_cache.plan), eager_cache.tiles.clone()
    dec.graphs = True
    request()  # captures
    graph_cache, replayed = request()
    assert (64, 8) in dec._group_graphs
    assert graph_cache.plan == eager_plan and graph_cache.seen == eager_cache.seen
    assert torch.equal(graph_cache.arena[:graph_cache.arena_used], eager_arena)
    assert torch.equal(graph_cache.tiles[:len(graph_cache.tile_starts)], eager_tiles[:len(graph_cache.tile_starts)])
    assert torch.equal(replayed, eager), (replayed - eager).abs().max().item()

    seq = dec.answer(graph_cache, question, cands)
    bat = dec.answer_batched(graph_cache, question, cands)
    torch.cuda.synchronize()
    print(f'[full-size {n_frames}] batched vs per-fork candidate scores: {seq.tolist()} / {bat.tolist()}', flush=True)
    assert (seq - bat).abs().max().item() <= 2e-2, (seq, bat)
    dec.graphs = False

    ref = native_logits(model, prefix, frames, question)
    exact = StreamingDecoder(model, precision='fp32')
    cache16 = exact.ingest(prefix, frames, [16] * n_frames)
    got = exact.forward(cache16, ids=question, logits=question.shape[1])
    torch.cuda.synchronize()
    err = (got - ref).abs().max().item()
    print(f'[full-size {n_frames}] 16-bit packed (fp32) vs native logits: max-abs {err:.4e}, '
          f'logit scale {ref.abs().max().item():.3f}', flush=True)
    assert err <= 0.25, err
