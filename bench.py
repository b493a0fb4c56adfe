"""Benchmark of the packed-KV hot path on one MI355X.

Headline (`value`): pack throughput on the whole-volume pack workload
(32 layers x 5 KV heads x 6144 tokens of bf16 K and V, 96 frame tiles of 64 tokens with
seeded 4/8/16-bit widths), in algorithmic GB/s = (bytes read + bytes written) / time.
Also reported on the same line: frame-chunk attention (15 Q / 5 KV heads, 64-token
causal chunk over 1024/4096/8128-token mixed histories) in us/layer, GB/s and TFLOP/s;
candidate scoring (4 continuations of 8-24 tokens over a 6144-token 4-bit / 8-bit
history); and the reference CPU path timed on this host (the oracle restatement).

Attention timings rotate over distinct per-layer histories whose total exceeds the
256 MB Infinity Cache, so the history is read from HBM.
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, 'dynamic-kv-cache_amd'))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
LAYERS, HEADS, Q_HEADS, TILE = 32, 5, 15, 64
PIPELINE = int(os.environ.get('DKV_PIPELINE', '8'))  # frames per pipelined graph replay in the e2e run


def parse():
    p = argparse.ArgumentParser()
    p.add_argument('--gpus', type=int, default=1)
    p.add_argument('--steps', type=int, default=200)
    p.add_argument('--warmup', type=int, default=20)
    p.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline')
    p.add_argument('--only', choices=['pack', 'seg', 'attn', 'cand', 'e2e', 'all'], default='all')
    p.add_argument('--rotate', type=int, default=48, help='distinct layers attention rotates over')
    return p.parse_args()


WARM_S = 0.03  # minimum warm-up: after idle the first ~15 ms of launches run ~7% slower (clock ramp)


def time_launches(fn, steps, warmup):
    """ms per fn() over `steps` calls, after `warmup` untimed calls and at least WARM_S seconds of
    untimed calls (so the timed calls run at the steady-state clock)."""
    import torch
    t0 = time.perf_counter()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < WARM_S:
        fn()
        torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    end.synchronize()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per launch


def pack_traffic():
    """HBM bytes per pack launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes, each
    scaled by what the counter reads for a 256 MiB copy (profiles/pack_batch_kernel_pack_volume.md)."""
    path = os.path.join(REPO, 'profiles', 'pack_batch_kernel_traffic.json')
    if not os.path.exists(path):
        return None
    t = json.load(open(path))
    fetch = t['fetch_kib'] * t['copy_bytes'] / t['copy_fetch_kib']
    write = t['write_kib'] * t['copy_bytes'] / t['copy_write_kib']
    return int(fetch + write)


def pack_bytes(bits, layers=LAYERS, heads=HEADS, tile=TILE):
    rows_per_frame = layers * 2 * heads * tile
    read = rows_per_frame * 128 * len(bits)
    write = sum(rows_per_frame * {4: 40, 8: 72, 16: 128}[b] for b in bits)
    return read, write


def graph_of(fn, reps):
    """A HIP graph that runs fn() `reps` times back to back (captured on torch's stream)."""
    import torch
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    torch.cuda.synchronize()
    return graph


def bench_pack(steps, warmup, reps=10):
    """One step = one launch packing the whole volume; timed as graph replays of `reps` launches."""
    import torch
    from dkv.gpu_cache import GPUCache
    from dkv.workloads import pack_volume
    vol = pack_volume(seed=0, layers=LAYERS, frames=96)
    dev = torch.device('cuda:0')
    k, v = vol['k'].to(dev), vol['v'].to(dev)
    cache = GPUCache(None, layers=LAYERS, heads=HEADS, max_tokens=96 * TILE)
    batch = cache.append_batch(k, v, vol['bits'], [TILE] * 96)
    graph = graph_of(batch.run, reps)
    rounds = max(1, steps // reps)
    ms = time_launches(graph.replay, rounds, max(1, warmup // reps)) / reps
    read, write = pack_bytes(vol['bits'])
    gbs = (read + write) / (ms * 1e-3) / 1e9
    return dict(ms=ms, gbs=gbs, read_bytes=read, write_bytes=write, bits=vol['bits'], steps=rounds * reps)


def bench_segments(steps, warmup, reps=10):
    """Export of the whole pack volume into the reference's PackedTensor layout (one launch over all
    96 segments x 32 layers), and import of those segments into a second cache. Both are byte moves:
    algorithmic bytes = payload + fp32 offsets/scales read once and written once."""
    import torch
    from dkv.gpu_cache import GPUCache, SegmentExport
    from dkv.workloads import pack_volume
    vol = pack_volume(seed=0, layers=LAYERS, frames=96)
    dev = torch.device('cuda:0')
    src = GPUCache(None, layers=LAYERS, heads=HEADS, max_tokens=96 * TILE)
    src.append_batch(vol['k'].to(dev), vol['v'].to(dev), vol['bits'], [TILE] * 96)
    exp = SegmentExport(src).run()
    rounds = max(1, steps // reps)
    ms_export = time_launches(graph_of(exp.run, reps).replay, rounds, max(1, warmup // reps)) / reps
    dst = GPUCache(None, layers=LAYERS, heads=HEADS, max_tokens=96 * TILE)
    _, batch = dst._import(exp.segments())
    ms_import = time_launches(graph_of(batch.run, reps).replay, rounds, max(1, warmup // reps)) / reps
    torch.cuda.synchronize()
    same = bool(torch.equal(dst.arena[:dst.arena_used], src.arena[:src.arena_used]))
    moved = 2 * exp.nbytes
    return dict(export_us=ms_export * 1e3, export_gbs=moved / (ms_export * 1e-3) / 1e9,
                import_us=ms_import * 1e3, import_gbs=moved / (ms_import * 1e-3) / 1e9,
                algorithmic_bytes=moved, segments=len(exp.parts), arena_round_trip_equal=same)


def bench_copy(steps, nbytes=256 << 20, reps=10):
    """Device-to-device copy of nbytes (torch copy_): the attainable streaming rate, read + write."""
    import torch
    dev = torch.device('cuda:0')
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    graph = graph_of(lambda: dst.copy_(src), reps)
    ms = time_launches(graph.replay, max(1, steps // reps), 1) / reps
    return dict(ms=ms, gbs=2 * nbytes / (ms * 1e-3) / 1e9, bytes=nbytes)


def attention_setup(past, rotate, bits, nq=64, segments=None, seed=0, precision='bf16', path='auto', splits=0):
    """`rotate` layers, each with its own copy of one seeded history, and one graph that runs
    the attention of every layer once (distinct histories, so the reads come from HBM)."""
    import ctypes
    import torch
    from dkv import _lib
    from dkv.gpu_cache import GPUCache
    from dkv.workloads import outlier_values
    dev = torch.device('cuda:0')
    g = torch.Generator().manual_seed(seed)
    hk = outlier_values((HEADS, past, 64), g, 0).to(dev)
    hv = outlier_values((HEADS, past, 64), g, 0).to(dev)
    q = outlier_values((Q_HEADS, nq, 64), g, 0).to(dev)[None]
    kn = outlier_values((HEADS, nq, 64), g, 0).to(dev)[None]
    vn = outlier_values((HEADS, nq, 64), g, 0).to(dev)[None]
    cache = GPUCache(None, layers=rotate, heads=HEADS, max_tokens=past + nq, precision=precision)
    tiles = (past + TILE - 1) // TILE
    lengths = [min(TILE, past - TILE * i) for i in range(tiles)]
    cache.append_batch(hk[None].expand(rotate, -1, -1, -1).contiguous(),
                       hv[None].expand(rotate, -1, -1, -1).contiguous(), bits, lengths)
    cache.select(16)
    for layer in range(rotate):
        cache.append(kn, vn, layer)
    out = torch.empty((1, nq, Q_HEADS, 64), dtype=torch.bfloat16, device=dev)
    lib = _lib.load()
    args = [cache.attend_args(q, kn, vn, layer, past, out, segments, path=path, splits=splits)
            for layer in range(rotate)]
    need = lib.dkv_attend_workspace_bytes(ctypes.byref(args[0]))
    ws = torch.zeros(max(need, 16), dtype=torch.uint8, device=dev)
    for a in args:
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    refs = [ctypes.byref(a) for a in args]

    def launch_all():
        stream = _lib.stream_handle(dev)
        for r in refs:
            rc = lib.dkv_attend(r, stream)
            if rc:
                _lib.check(rc, 'dkv_attend')
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        launch_all()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch_all()
    torch.cuda.synchronize()
    hist_bytes = sum(HEADS * 2 * n * {4: 40, 8: 72, 16: 128}[b] for b, n in zip(bits, lengths))
    chunk_bytes = (Q_HEADS * nq * 64 * 2) * 2 + HEADS * nq * 64 * 2 * 2  # q + out, k_new + v_new
    keep = dict(cache=cache, keep=(hk, hv, q, kn, vn, out, ws, args), graph=graph)
    return graph.replay, hist_bytes + chunk_bytes, keep


def attention_flops(past, lengths):
    # 2 matmuls (QK^T and PV) of 2*64 flops per (q row, visible key), per Q head
    visible = sum(n * past + n * (n + 1) // 2 for n in lengths)
    return 4 * 64 * Q_HEADS * visible


def bench_attention(past, steps, warmup, rotate, precision='bf16'):
    from dkv.workloads import bit_schedule
    bits = bit_schedule(past, (past + TILE - 1) // TILE)
    replay, nbytes, keep = attention_setup(past, rotate, bits, seed=past, precision=precision)
    ms = time_launches(replay, max(1, steps // 10), max(1, warmup // 10)) / rotate
    flops = attention_flops(past, [64])
    del keep
    return dict(us_per_layer=ms * 1e3, gbs=nbytes / (ms * 1e-3) / 1e9, tflops=flops / (ms * 1e-3) / 1e12,
                bytes=nbytes, flops=flops, mfma_frac=flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                hbm_frac=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, **attainable(nbytes, flops, ms))


def attainable(nbytes, flops, ms):
    """The roofline time min over (HBM, bf16 MFMA) bounds, max(bytes/8 TB/s, flops/2.5 PFLOP/s), and the
    measured time's fraction of it (the attainable roofline of a mixed-intensity workload)."""
    t = max(nbytes / (HBM_PEAK_GBS * 1e9), flops / (BF16_PEAK_TFLOPS * 1e12))
    return dict(roofline_us=t * 1e6, attainable_frac=t / (ms * 1e-3))


def bench_decode(past, nq, steps, warmup, rotate, precision='bf16'):
    """A short chunk (nq = 1: one decode token) over a mixed history; us per layer."""
    from dkv.workloads import bit_schedule
    bits = bit_schedule(past, (past + TILE - 1) // TILE)
    replay, nbytes, keep = attention_setup(past, rotate, bits, nq=nq, seed=past + nq, precision=precision)
    ms = time_launches(replay, max(1, steps // 10), max(1, warmup // 10)) / rotate
    flops = attention_flops(past, [nq])
    del keep
    return dict(us_per_layer=ms * 1e3, gbs=nbytes / (ms * 1e-3) / 1e9, bytes=nbytes,
                hbm_frac=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, **attainable(nbytes, flops, ms))


def bench_candidates(bits, steps, warmup, rotate, precision='bf16'):
    from dkv.workloads import candidate_lengths
    lengths = candidate_lengths(0, 4)
    bounds = [0]
    for n in lengths:
        bounds.append(bounds[-1] + n)
    past = 6144
    replay, nbytes, keep = attention_setup(past, rotate, [bits] * (past // TILE), nq=bounds[-1], segments=bounds,
                                           seed=bits, precision=precision)
    ms = time_launches(replay, max(1, steps // 10), max(1, warmup // 10)) / rotate
    flops = attention_flops(past, lengths)
    del keep
    return dict(us_per_batch=ms * 1e3, gbs=nbytes / (ms * 1e-3) / 1e9, tflops=flops / (ms * 1e-3) / 1e12,
                bytes=nbytes, flops=flops, lengths=lengths, hbm_frac=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                mfma_frac=flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, **attainable(nbytes, flops, ms))


def bench_e2e(frame_counts=(16, 64, 96), reps=2):
    """Streaming request: random-init 32-layer decoder, 64-token synthetic frames, 4 candidates.

    frames/s = frames / (ingest + candidate scoring) seconds, the reference's request definition
    (benchmarks/gpu_evaluate.py:105) without video decode and the vision encoder.
    """
    import torch
    from dkv.streaming import StreamingDecoder, build_decoder
    from dkv.workloads import bit_schedule, candidate_lengths
    dev = torch.device('cuda:0')
    model = build_decoder(seed=0, device=dev)
    dec = StreamingDecoder(model, graphs=True)
    g = torch.Generator().manual_seed(0)
    vocab = model.config.vocab_size
    prefix = torch.randint(0, vocab, (1, 16), generator=g)
    question = torch.randint(0, vocab, (1, 24), generator=g)
    cands = [torch.randint(0, vocab, (1, n), generator=g) for n in candidate_lengths(0, 4)]
    out = {}
    for nf in frame_counts:
        ids = torch.randint(0, vocab, (nf, 64), generator=g).to(dev)
        with torch.inference_mode():
            emb = model.model.get_input_embeddings()(ids)
        frames = [emb[i:i + 1] for i in range(nf)]
        bits = bit_schedule(nf, nf)
        best = {}
        # eager launches; graph replays of consecutive frames pipelined in groups (the default);
        # graph replays one frame at a time
        for mode, graphs, pipeline in (('eager', False, 1), ('graph', True, PIPELINE), ('graph1', True, 1)):
            dec.graphs, dec.pipeline = graphs, pipeline
            for proto in ('forks', 'batched'):
                times = []
                for _ in range(reps + 1):  # the first request warms up kernels, GEMM selection, the capture
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    cache = dec.ingest(prefix, frames, bits)
                    if proto == 'forks':
                        scores = dec.answer(cache, question, cands)
                    else:
                        scores = dec.answer_batched(cache, question, cands)
                    scores.cpu()
                    torch.cuda.synchronize()
                    times.append(time.perf_counter() - t0)
                    del cache
                best[(mode, proto)] = min(times[1:])
        r = out[f'frames_{nf}'] = dict(tokens=16 + 64 * nf + 24 + sum(c.shape[1] for c in cands))
        for (mode, proto), t in best.items():
            r[f'frames_per_s_{mode}_{proto}'] = round(nf / t, 2)
            r[f'request_s_{mode}_{proto}'] = round(t, 4)
        print(f"# e2e {nf} frames: eager {r['frames_per_s_eager_forks']} / {r['frames_per_s_eager_batched']}, "
              f"graph {r['frames_per_s_graph_forks']} / {r['frames_per_s_graph_batched']}, "
              f"graph frame by frame {r['frames_per_s_graph1_forks']} / {r['frames_per_s_graph1_batched']} "
              f"frames/s (forks / batched)", flush=True)
    dec.graphs, dec.pipeline = False, PIPELINE
    return out


def cpu_baselines(target_s=8.0):
    """The reference CPU path restated in torch on this host's cores (oracle; timed, not checked)."""
    import torch
    from dkv.workloads import frame_chunk_case, pack_volume
    from oracle.cpu_path import MixedPrecisionCache, cpu_attention_step
    from oracle.kv_quantization import pack
    cores = torch.get_num_threads()
    # Pack: 2 layers of the pack workload (1/16 of the volume), every tile packed as the CPU path does.
    vol = pack_volume(seed=0, layers=2, frames=96)
    t0 = time.perf_counter()
    reps = 0
    while True:
        for f, b in enumerate(vol['bits']):
            for layer in range(2):
                pack(vol['k'][layer:layer + 1, :, 64 * f:64 * f + 64], b)
                pack(vol['v'][layer:layer + 1, :, 64 * f:64 * f + 64], b)
        reps += 1
        if time.perf_counter() - t0 > target_s / 2:
            break
    dt = (time.perf_counter() - t0) / reps
    read, write = pack_bytes(vol['bits'], layers=2)
    pack_gbs = (read + write) / dt / 1e9
    # Attention: the CPU path's per-layer update + SDPA for one 64-token frame over 8128 history tokens.
    case = frame_chunk_case(8128, seed=8128)
    c = MixedPrecisionCache()
    for i, b in enumerate(case['bits']):
        c.select(b)
        c.update(case['k_hist'][None, :, 64 * i:64 * i + 64], case['v_hist'][None, :, 64 * i:64 * i + 64], 0)
    t0 = time.perf_counter()
    reps = 0
    while True:
        c2 = MixedPrecisionCache()
        c2.segments = {0: list(c.segments[0])}
        c2.select(16)
        cpu_attention_step(c2, case['q'][None], case['k_new'][None], case['v_new'][None])
        reps += 1
        if time.perf_counter() - t0 > target_s / 2:
            break
    attn_ms = (time.perf_counter() - t0) / reps * 1e3
    return dict(pack_gbs=pack_gbs, attn_ms_per_layer_8128=attn_ms, cores=cores,
                pack_sample='2 of 32 layers of the pack workload (96 tiles, K and V)',
                attn_sample='one layer, 64-token frame over 8128 mixed history tokens (127 tiles)')


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps(dict(error='bench.py measures one GPU; --gpus must be 1',
                              detail='the kernels run one GPU\'s share (a whole layer, or a history '
                                     'slice via splits); sharding across GPUs is not built')), flush=True)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps(dict(error='no HIP device visible')), flush=True)
        sys.exit(2)
    from dkv import _lib
    _lib.load()
    res = {}
    if args.only in ('pack', 'all'):
        res['pack'] = bench_pack(args.steps, args.warmup)
        print(f"# pack: {res['pack']['ms'] * 1e3:.1f} us/launch, {res['pack']['gbs']:.0f} GB/s", flush=True)
        res['copy'] = bench_copy(args.steps)
        print(f"# copy 256 MiB: {res['copy']['ms'] * 1e3:.1f} us, {res['copy']['gbs']:.0f} GB/s", flush=True)
    if args.only in ('seg', 'all'):
        r = res['segments'] = bench_segments(args.steps, args.warmup)
        print(f"# segments: export {r['export_us']:.1f} us ({r['export_gbs']:.0f} GB/s), import {r['import_us']:.1f} "
              f"us ({r['import_gbs']:.0f} GB/s), round trip equal {r['arena_round_trip_equal']}", flush=True)
    if args.only in ('attn', 'all'):
        res['attention'] = {}
        for prec in ('bf16', 'fp32'):
            for past in (1024, 4096, 8128):
                r = bench_attention(past, args.steps, args.warmup, args.rotate, prec)
                res['attention'][f'{prec}_past_{past}'] = r
                print(f"# attn {prec} past={past}: {r['us_per_layer']:.2f} us/layer, {r['gbs']:.0f} GB/s, "
                      f"{r['tflops']:.1f} TFLOP/s", flush=True)
    if args.only in ('attn', 'all'):
        res['decode'] = {}
        for prec in ('bf16', 'fp32'):
            for nq in (1, 4):
                r = bench_decode(8128, nq, args.steps, args.warmup, args.rotate, prec)
                res['decode'][f'{prec}_past_8128_nq_{nq}'] = r
                print(f"# decode {prec} past=8128 nq={nq}: {r['us_per_layer']:.2f} us/layer, {r['gbs']:.0f} GB/s",
                      flush=True)
    if args.only in ('cand', 'all'):
        res['candidates'] = {}
        for prec in ('bf16', 'fp32'):
            for bits in (4, 8):
                r = bench_candidates(bits, args.steps, args.warmup, args.rotate, prec)
                res['candidates'][f'{prec}_{bits}bit'] = r
                print(f"# candidates {prec} {bits}-bit: {r['us_per_batch']:.2f} us, {r['gbs']:.0f} GB/s, "
                      f"{r['tflops']:.1f} TFLOP/s", flush=True)
    if args.only in ('e2e', 'all'):
        res['e2e'] = bench_e2e()
    cpu = None if args.no_cpu else cpu_baselines()
    p = res.get('pack')
    line = dict(
        metric='packed-KV attn us/layer + HBM GB/s @8k mixed history; pack GB/s; frames/s e2e',
        value=round(p['gbs'], 2) if p else None, unit='GB/s', n_gpus=1, steps=p['steps'] if p else args.steps,
        warmup=args.warmup,
        ms_per_step=round(p['ms'], 5) if p else None, higher_is_better=True, scaling='weak', vs_baseline=None,
        dtype='bf16->u4/u8/bf16', data='synthetic',
        config=dict(workload='pack: 32 layers x 5 KV heads x 6144 tokens (96 tiles of 64) bf16 K+V, '
                             'seeded 40/40/20 4/8/16-bit tiles, one launch', parallelism='none (1 GPU)'),
    )
    if p:
        line['roofline'] = dict(bound='hbm', achieved=round(p['gbs'], 1), peak=HBM_PEAK_GBS,
                                unit='GB/s', frac=round(p['gbs'] / HBM_PEAK_GBS, 4), traffic=pack_traffic(),
                                algorithmic_bytes=p['read_bytes'] + p['write_bytes'])
        line['copy_reference_gbs'] = round(res['copy']['gbs'], 1)
    if 'attention' in res:
        line['attention'] = {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in r.items()}
                             for k, r in res['attention'].items()}
    if 'decode' in res:
        line['decode'] = {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in r.items()}
                          for k, r in res['decode'].items()}
    if 'candidates' in res:
        line['candidates'] = {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in r.items()}
                              for k, r in res['candidates'].items()}
    if 'segments' in res:
        line['segments'] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in res['segments'].items()}
    if 'e2e' in res:
        line['e2e'] = res['e2e']
    if cpu:
        line['cpu_baseline'] = dict(value=round(cpu['pack_gbs'], 4), unit='GB/s', cores=cpu['cores'], kind='port',
                                    sample=cpu['pack_sample'],
                                    attn_ms_per_layer_8128=round(cpu['attn_ms_per_layer_8128'], 3),
                                    attn_sample=cpu['attn_sample'])
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
