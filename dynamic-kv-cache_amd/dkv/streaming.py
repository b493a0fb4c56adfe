"""Streaming decoder over the packed cache: frame ingestion and candidate scoring.

The caller side of the packed-KV path, following the reference's StreamingModel
(src/streaming.py:89-237) on a text decoder with synthetic frame embeddings in
place of the vision encoder:

- ingest(): one decoder forward for a text prefix, then one per 64-token frame.
  The cache's width is selected per frame (cache.select(bits, i),
  src/streaming.py:178), and every LlamaAttention packs its K/V and attends
  over the packed history (install_packed_attention).
- answer(): the reference's 'candidate' protocol (src/streaming.py:209-225).
  For each candidate, a fork of the cache runs question + candidate tokens, and
  the score is the mean log-likelihood of the candidate tokens. answer_labels()
  is the 'label' protocol and prior_scores() the prior of 'candidate_calibrated'.
- answer_batched(): the same scores from one forward of the question on a fork,
  then one forward of all candidates together. The candidates sit back to back
  in one chunk with per-candidate positions and a block-diagonal chunk mask
  (GPUCache.chunk_segments), so the shared history is read once per batch
  instead of once per candidate.

The model is a random-init LlamaForCausalLM. There is no checkpoint, and the
workloads are synthetic; see dkv.workloads.decoder_config.
"""
import torch

from .gpu_cache import GPUCache, install_packed_attention
from .gpu_ops import install_fused_ops

MFMA_ROWS = 192  # query rows per frame-chunk attention workgroup (MFMA_ROWS of csrc/dkv_attn_common.h)


def build_decoder(layers=32, hidden=960, heads=15, kv_heads=5, intermediate=2560, vocab=49280,
                  rope_theta=100000.0, max_positions=8192, seed=0, device='cuda', dtype=torch.bfloat16):
    """A random-init Llama text decoder of the given shape, on `device`, in eval mode."""
    from transformers import LlamaConfig, LlamaForCausalLM
    config = LlamaConfig(vocab_size=vocab, hidden_size=hidden, intermediate_size=intermediate,
                         num_hidden_layers=layers, num_attention_heads=heads, num_key_value_heads=kv_heads,
                         head_dim=hidden // heads, hidden_act='silu', rms_norm_eps=1e-5,
                         max_position_embeddings=max_positions, rope_theta=rope_theta,
                         tie_word_embeddings=True, attn_implementation='sdpa')
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        model = LlamaForCausalLM(config)
    return model.to(device=device, dtype=dtype).eval()


class StreamingDecoder:
    """Frame-by-frame ingestion into a GPUCache and candidate scoring (src/streaming.py:89-237)."""

    def __init__(self, model, fused_ops=True, precision='bf16', graphs=False, pipeline=8, group_splits=None):
        self.model = model
        self.text = model.model
        self.config = model.config
        self.precision = precision
        self.graphs = graphs
        self.pipeline = pipeline
        # History splits of the frame-chunk attention in pipelined groups (None: group_split_count())
        self.group_splits = group_splits
        self.ops_state = {'enabled': fused_ops}
        install_fused_ops(self.text, self.ops_state)
        install_packed_attention(model)
        self._cache = None  # reused across requests when graphs=True (a captured graph records its buffers)
        self._graphs = {}  # chunk length -> captured forward of that length on self._cache
        self._group_graphs = {}  # (chunk length, k) -> captured forwards of k consecutive chunks (pipelined)
        self._qa_graphs = {}  # (chunk length, logits, segments) -> captured forward + lm_head on a fork
        self._qa_seen = set()  # QA shapes already run once eagerly (warms the library paths a capture records)

    @property
    def device(self):
        return self.model.lm_head.weight.device

    def group_split_count(self, chunk):
        """History splits per KV head of the frame-chunk attention while frames are pipelined
        (pipeline > 1). The library's default plan gives one launch the whole GPU (one workgroup
        per CU per split), the shortest latency when it runs alone. In a pipelined group several
        frames' launches run at once and the GPU is throughput-bound, so each takes a quarter of
        that: fewer workgroups, each over more units, pay the per-workgroup prologue, merge and
        partial stores fewer times. 96 frames + 4 candidates (5 KV heads, 256 CUs): 1079 frames/s
        at the default 51-split cap, 1134-1139 at 12 splits, 1132-1134 at 16, 1111-1121 at 24,
        1106-1108 at 8; frames one at a time are fastest at the default (586 vs 528 at 12).
        With the later, faster attention kernel 8 to 24 splits all gave 1122-1141 frames/s."""
        if self.group_splits is not None:
            return self.group_splits
        c = self.config
        rows = c.num_attention_heads // c.num_key_value_heads * chunk
        row_groups = -(-rows // MFMA_ROWS)
        cus = torch.cuda.get_device_properties(self.device).multi_processor_count
        return max(1, cus // (c.num_key_value_heads * row_groups) // 4)

    def create_cache(self, max_tokens, **kw):
        c = self.config
        return GPUCache(None, layers=c.num_hidden_layers, heads=c.num_key_value_heads, dim=c.head_dim,
                        dtype=self.model.dtype, max_tokens=max_tokens, precision=self.precision,
                        device=self.device, **kw)

    @torch.inference_mode()
    def forward(self, cache, ids=None, embeddings=None, positions=None, logits=0):
        """One decoder forward of a chunk. Returns fp32 logits of the last `logits` positions."""
        if embeddings is None:
            embeddings = self.text.get_input_embeddings()(ids.to(self.device))
        past = cache.get_seq_length()
        n = embeddings.shape[1]
        if positions is None:
            positions = torch.arange(past, past + n, device=self.device)
        out = self.text(inputs_embeds=embeddings, past_key_values=cache, use_cache=True,
                        position_ids=positions[None], attention_mask=None, return_dict=True)
        if not logits:
            return None
        return self.model.lm_head(out.last_hidden_state[:, -int(logits):]).float()

    @torch.inference_mode()
    def ingest(self, prefix_ids, frames, bits, cache=None, qa_reserve=256):
        """Prefix at 16 bits, then each frame embedding [1, T, hidden] at its width (src/streaming.py:168-187).

        With graphs=True the frames after the first run as replays of one captured HIP graph of the
        whole decoder forward (the cache's launches read their step parameters from the device), on
        a cache the decoder keeps and resets between requests. With pipeline=k > 1 as well, k
        consecutive frames replay one graph of their k forwards in which frame i + 1's layer l
        waits only for frame i's layer l (the K/V it attends to) and its own layer l - 1: each
        forward runs one layer behind the one before it, on its own stream. The launches and the
        data are those of one frame after the other; the GPU overlaps them. With pipeline > 1 every
        chunk's attention (eager or replayed) runs group_split_count() history splits, so replays
        still equal eager ingestion bit for bit; question and candidate forwards keep the default.
        """
        if len(frames) != len(bits):
            raise ValueError('one bit width per frame')
        total = prefix_ids.shape[1] + sum(f.shape[1] for f in frames) + qa_reserve
        if cache is None:
            cache = self._reused_cache(total) if self.graphs else self.create_cache(total)
        # pipelined frames share the GPU: their frame-chunk attention takes fewer history splits
        cache.chunk_splits = (self.group_split_count(max(f.shape[1] for f in frames))
                              if self.pipeline > 1 and frames else 0)
        try:
            self._ingest_chunks(cache, prefix_ids, frames, bits)
        finally:
            cache.chunk_splits = 0
        return cache

    def _ingest_chunks(self, cache, prefix_ids, frames, bits):
        cache.select(16, -1)
        graphed = self.graphs and cache is self._cache
        # The first request's prefix and first frame run eagerly (they warm up the library paths
        # a capture records); after that every chunk replays the captured forward of its length
        # (captured on first use).
        warm = bool(self._graphs or self._group_graphs)
        if graphed and warm:
            self._graph_chunk(cache, self.text.get_input_embeddings()(prefix_ids.to(self.device)))
        else:
            self.forward(cache, ids=prefix_ids)
        i = 0
        while i < len(frames):
            emb, b = frames[i], bits[i]
            replay = graphed and (i > 0 or warm)
            k = 1
            while k < self.pipeline and i + k < len(frames) and frames[i + k].shape[1] == emb.shape[1]:
                k += 1
            if replay and k > 1:
                self._graph_group(cache, frames[i:i + k], bits[i:i + k], i)
                i += k
                continue
            cache.select(b, i)
            if replay:
                self._graph_chunk(cache, emb)
            else:
                self.forward(cache, embeddings=emb)
            i += 1
        cache.select(16, -1)
        if len(set(cache.seen)) != 1:
            raise RuntimeError('Decoder layers disagree about the cache length')

    def _reused_cache(self, total):
        if self._cache is None or self._cache.capacity < total:
            self._cache = self.create_cache(max(total, 8192))
            # a captured graph records the old cache's buffers
            self._graphs, self._group_graphs, self._qa_graphs, self._qa_seen = {}, {}, {}, set()
        else:
            self._cache.reset()
        return self._cache

    def _graph_chunk(self, cache, emb):
        """One chunk as a replay of the captured forward of its length (captured on first use)."""
        fg = self._graphs.get(emb.shape[1])
        if fg is None:
            self._capture_chunk(cache, emb)
            return
        cache.begin_graph_steps(fg['chunk'], steps=fg['steps'])
        try:
            past = cache.graph_step()
            fg['emb'].copy_(emb)
            torch.add(fg['arange'], past, out=fg['pos'][0])
            fg['graph'].replay()
        finally:
            cache.end_graph_steps()

    def _capture_chunk(self, cache, emb):
        chunk = emb.shape[1]
        static_emb = emb.clone()
        arange = torch.arange(chunk, device=self.device)
        pos = torch.empty((1, chunk), dtype=torch.long, device=self.device)
        steps = cache.begin_graph_steps(chunk, q_heads=self.config.num_attention_heads)
        try:
            past = cache.graph_step()
            torch.add(arange, past, out=pos[0])
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self.text(inputs_embeds=static_emb, past_key_values=cache, use_cache=True, position_ids=pos,
                          attention_mask=None, return_dict=True)
            steps.upload()  # the jobs now carry the K/V addresses recorded in the graph
            graph.replay()
        finally:
            cache.end_graph_steps()
        self._graphs[chunk] = dict(chunk=chunk, graph=graph, steps=steps, emb=static_emb, pos=pos, arange=arange)

    def _group_steps(self, cache, chunk, bits, frame, steps):
        """Host bookkeeping of frames frame .. frame + k - 1 (one GraphSteps each, since their
        forwards run at once); returns their history lengths and the GraphSteps."""
        past, out = [], []
        for j, st in enumerate(steps):
            cache.select(bits[j], frame + j)
            cache.begin_graph_steps(chunk, q_heads=None if st else self.config.num_attention_heads, steps=st)
            try:
                past.append(cache.graph_step())
            finally:
                out.append(cache.end_graph_steps())
        return past, out

    def _graph_group(self, cache, embs, bits, frame):
        """k consecutive frames as one replay of their pipelined forwards (captured on first use)."""
        chunk, k = embs[0].shape[1], len(embs)
        fg = self._group_graphs.get((chunk, k))
        if fg is None:
            self._capture_group(cache, embs, bits, frame)
            return
        past, _ = self._group_steps(cache, chunk, bits, frame, fg['steps'])
        for j in range(k):
            fg['emb'][j].copy_(embs[j])
            torch.add(fg['arange'], past[j], out=fg['pos'][j][0])
        fg['graph'].replay()

    def _capture_group(self, cache, embs, bits, frame):
        chunk, k = embs[0].shape[1], len(embs)
        static_emb = [e.clone() for e in embs]
        arange = torch.arange(chunk, device=self.device)
        pos = [torch.empty((1, chunk), dtype=torch.long, device=self.device) for _ in range(k)]
        past, steps = self._group_steps(cache, chunk, bits, frame, [None] * k)
        for j in range(k):
            torch.add(arange, past[j], out=pos[j][0])
        layers = self.text.layers
        done = [[torch.cuda.Event() for _ in layers] for _ in range(k - 1)]  # frame j's layer l has finished
        streams = [torch.cuda.Stream(device=self.device) for _ in range(k - 1)]
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        hooks = []
        try:
            with torch.cuda.graph(graph):
                first = torch.cuda.current_stream()
                for st in streams:
                    st.wait_stream(first)  # the fork: the other forwards join the capture here
                for j in range(k):
                    stream = first if j == 0 else streams[j - 1]
                    if j > 0:  # layer l after the previous frame's layer l
                        hooks += [m.register_forward_pre_hook(
                            lambda mod, inp, l=l, ev=done[j - 1], st=stream: st.wait_event(ev[l]))
                            for l, m in enumerate(layers)]
                    if j < k - 1:
                        hooks += [m.register_forward_hook(lambda mod, inp, out, l=l, ev=done[j]: ev[l].record())
                                  for l, m in enumerate(layers)]
                    cache.begin_graph_steps(chunk, steps=steps[j])
                    with torch.cuda.stream(stream):
                        self.text(inputs_embeds=static_emb[j], past_key_values=cache, use_cache=True,
                                  position_ids=pos[j], attention_mask=None, return_dict=True)
                    cache.end_graph_steps()
                    for h in hooks:
                        h.remove()
                    hooks = []
                for st in streams:
                    first.wait_stream(st)
        finally:
            for h in hooks:
                h.remove()
            cache.end_graph_steps()
        for st in steps:
            st.upload()  # the jobs now carry the K/V addresses recorded in the graph
        graph.replay()
        self._group_graphs[(chunk, k)] = dict(graph=graph, steps=steps, emb=static_emb, pos=pos, arange=arange,
                                              events=done, streams=streams)

    def _fork_forward(self, branch, ids, logits, lengths=None):
        """fp32 logits of the last `logits` positions of one forward on a fork of the decoder's
        reused cache. `lengths` splits the chunk into continuations of the fork's history, each
        with its own positions and attending to itself only (a block-diagonal chunk mask). With
        graphs=True a shape seen before replays a captured forward + lm_head (captured the second
        time it is seen; the first run is eager and warms the library paths)."""
        emb = self.text.get_input_embeddings()(ids.to(self.device))
        chunk = emb.shape[1]
        lengths = list(lengths) if lengths else None
        segments, rel = None, None
        if lengths:
            segments = [0]
            for n in lengths:
                segments.append(segments[-1] + n)
            rel = torch.cat([torch.arange(n, device=self.device) for n in lengths])
        else:
            rel = torch.arange(chunk, device=self.device)
        key = (chunk, int(logits), tuple(lengths) if lengths else None)
        graphed = self.graphs and self._cache is not None and branch.arena is self._cache.arena
        if not graphed or key not in self._qa_seen:
            if graphed:
                self._qa_seen.add(key)
            past = branch.get_seq_length()
            branch.chunk_segments = segments
            try:
                return self.forward(branch, embeddings=emb, positions=rel + past, logits=logits)
            finally:
                branch.chunk_segments = None
        fg = self._qa_graphs.get(key)
        steps = fg['steps'] if fg else None
        branch.begin_graph_steps(chunk, q_heads=None if fg else self.config.num_attention_heads, steps=steps)
        try:
            past = branch.graph_step()
            if fg is None:
                static_emb, pos = emb.clone(), torch.empty((1, chunk), dtype=torch.long, device=self.device)
                torch.add(rel, past, out=pos[0])
                branch.chunk_segments = segments
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    out = self.text(inputs_embeds=static_emb, past_key_values=branch, use_cache=True,
                                    position_ids=pos, attention_mask=None, return_dict=True)
                    lg = self.model.lm_head(out.last_hidden_state[:, -int(logits):]).float()
                fg = self._qa_graphs[key] = dict(graph=graph, steps=branch._graph, emb=static_emb, pos=pos,
                                                 rel=rel.clone(), logits=lg)
                fg['steps'].upload()  # the jobs now carry the K/V addresses recorded in the graph
            else:
                fg['emb'].copy_(emb)
                torch.add(fg['rel'], past, out=fg['pos'][0])
            fg['graph'].replay()
            return fg['logits'].clone()
        finally:
            branch.chunk_segments = None
            branch.end_graph_steps()

    @staticmethod
    def _mean_loglik(logits, targets):
        return logits.log_softmax(-1).gather(1, targets[:, None]).mean()

    @torch.inference_mode()
    def answer(self, cache, question_ids, candidates):
        """Mean token log-likelihood of each candidate on its own fork (src/streaming.py:209-225)."""
        scores = []
        for cand in candidates:
            ids = torch.cat((question_ids, cand), dim=1).to(self.device)
            branch = cache.fork()
            lg = self._fork_forward(branch, ids, cand.shape[1] + 1)
            scores.append(self._mean_loglik(lg[0, :-1], cand[0].to(self.device)))
        return torch.stack(scores)

    @torch.inference_mode()
    def answer_labels(self, cache, question_ids, label_ids):
        """The reference's 'label' protocol (src/streaming.py:202-208): one forward of the question
        on a fork; the scores are the last position's logits at the option-label token ids."""
        branch = cache.fork()
        logits = self._fork_forward(branch, question_ids, 1)[0, -1]
        return logits[torch.as_tensor(label_ids, device=self.device)]

    @torch.inference_mode()
    def prior_scores(self, prefix_ids, question_ids, candidates):
        """Candidate scores without the video, for the 'candidate_calibrated' protocol
        (src/streaming.py:124-127, 226-233): the same scoring on a cache holding only the prefix.
        Calibrated scores are answer(...) - prior_scores(...)."""
        total = prefix_ids.shape[1] + question_ids.shape[1] + max(c.shape[1] for c in candidates) + 64
        cache = self.create_cache(total)
        cache.select(16, -1)
        self.forward(cache, ids=prefix_ids)
        return self.answer(cache, question_ids, candidates)

    @torch.inference_mode()
    def answer_batched(self, cache, question_ids, candidates):
        """The same scores with the question once and all candidates in one block-diagonal chunk."""
        branch = cache.fork()
        q_logits = self._fork_forward(branch, question_ids, 1)[0]  # predicts each candidate's first token
        ids = torch.cat(candidates, dim=1)
        bounds = [0]
        for cand in candidates:
            bounds.append(bounds[-1] + cand.shape[1])
        # every candidate continues the question: positions restart at the fork's length for each
        lg = self._fork_forward(branch, ids, ids.shape[1], lengths=[c.shape[1] for c in candidates])[0]
        scores = []
        for i, cand in enumerate(candidates):
            pred = torch.cat((q_logits, lg[bounds[i]:bounds[i + 1] - 1]), 0)
            scores.append(self._mean_loglik(pred, cand[0].to(self.device)))
        return torch.stack(scores)
