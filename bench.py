"""Benchmark of the full-attention path on one MI355X.

A step is one token's attention over all 16 full-attention layers of the
model (24 query heads, 4 KV heads, head_dim 256), each layer with its own
fp16 KV cache of 139,264 tokens in HBM (64 keys per layer scaled x8): the
decode at maximum context.  `value` is the achieved HBM bandwidth over the
algorithmic K+V bytes (each key read once), whole step including the
split-K combine; `roofline` is the split-K kernel alone, timed with HIP events
on the stream it runs on.  Secondary workloads (speculative verify-8 on a
16K prefix, decode at 4K) are reported under `extra`.

The CPU baseline is the numpy fp32 restatement of the reference's CPU
attention (oracle/attention_ref.py), run on this host on one layer's decode.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = 'µs/layer + achieved HBM GB/s, GQA decode/verify-8 @16K and 139,264 ctx'
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK = 2.5e15   # dense bf16 FLOP/s
LAYERS = 16


def log(msg):
    print(f'[bench] {msg}', file=sys.stderr, flush=True)


def make_layers(torch, A, w, layers, seed):
    """One PagedKV per layer with N(0, kv_std) fp16 keys/values (outlier keys
    scaled by outlier_gain) and one query per layer, generated on the GPU."""
    gen = torch.Generator(device='cuda')
    gen.manual_seed(seed)
    caches, queries = [], []
    capacity = A.round_capacity(w.keys)
    dtype = torch.bfloat16 if w.dtype == 'bf16' else torch.float16
    for _ in range(layers):
        k = torch.randn((w.keys, w.kv_heads, w.head_dim), generator=gen, device='cuda',
                        dtype=torch.float32) * w.kv_std
        v = torch.randn((w.keys, w.kv_heads, w.head_dim), generator=gen, device='cuda',
                        dtype=torch.float32) * w.kv_std
        if w.outliers:
            idx = torch.randperm(w.keys, generator=gen, device='cuda')[:w.outliers]
            k[idx] *= w.outlier_gain
        cache = A.PagedKV(w.kv_heads, w.head_dim, capacity, dtype)
        cache.pack(k.to(dtype), v.to(dtype))
        del k, v
        q = (torch.randn((w.tokens, w.q_heads, w.head_dim), generator=gen, device='cuda') * w.q_std).to(dtype)
        caches.append(cache)
        queries.append(q)
    torch.cuda.synchronize()
    return caches, queries


def time_workload(torch, A, w, layers, steps, warmup, seed):
    """Times `steps` steps of `layers` attention calls.

    Returns dict(ms_per_step: one step replayed as a captured HIP graph,
    eager_ms_per_step: the same launches issued one by one, split_us: average
    duration of the split-K kernel from events recorded around each of its
    launches in the eager loop, on the stream it runs on)."""
    caches, queries = make_layers(torch, A, w, layers, seed)
    ws = A.workspace(A.attention_workspace_bytes(w.q_heads, w.kv_heads, w.head_dim, w.tokens, w.position))
    outs = [torch.empty_like(q) for q in queries]
    one_chunk = w.tokens * w.group <= A.MAX_CHUNK_ROWS

    def step(events=None):
        for i in range(layers):
            if events is not None:
                events[i][0].record()
            if one_chunk:
                A.attention_split(queries[i], caches[i], w.position, w.scale, ws)
            else:
                A.attention(queries[i], caches[i], w.position, w.scale, out=outs[i], ws=ws)
            if events is not None:
                events[i][1].record()
            if one_chunk:
                A.attention_combine(outs[i], caches[i], w.position, ws)

    def timed(fn, n):
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for s in range(n):
            fn(s)
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / n

    for _ in range(warmup):
        step()
    ev = [[[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(layers)]
          for _ in range(steps)]
    eager_ms = timed(lambda s: step(ev[s]), steps)
    split_ms = [e[0].elapsed_time(e[1]) for st in ev for e in st]

    # The same step captured once and replayed (no per-launch host overhead).
    graph = torch.cuda.CUDAGraph()
    capture_stream = torch.cuda.Stream()
    capture_stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(capture_stream):
        step()                      # plans resolved before capture
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=capture_stream):
            step()
    torch.cuda.current_stream().wait_stream(capture_stream)
    for _ in range(warmup):
        graph.replay()
    graph_ms = timed(lambda s: graph.replay(), steps)
    del graph, caches
    torch.cuda.empty_cache()
    return dict(ms_per_step=graph_ms, eager_ms_per_step=eager_ms,
                split_us=1000.0 * sum(split_ms) / len(split_ms))


def cpu_baseline(w, target_s=10.0):
    """Single-thread numpy fp32 restatement (oracle) on one layer's decode."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle.attention_ref import gqa_attention_fp32
    from redshift_amd.workloads import make_inputs

    q, k, v, _ = make_inputs(w)
    with threadpool_limits(limits=1):
        gqa_attention_fp32(q, k, v, w.position, w.scale)  # warm-up
        times = []
        t_end = time.perf_counter() + target_s
        while len(times) < 3 or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            gqa_attention_fp32(q, k, v, w.position, w.scale)
            times.append(time.perf_counter() - t0)
    sec = float(np.median(times))
    return {
        'value': round(w.kv_bytes() / sec / 1e9, 3), 'unit': 'GB/s', 'cores': 1, 'kind': 'port',
        'us_per_layer': round(sec * 1e6, 1),
        'sample': f'{len(times)} single-layer {w.name} calls ({w.keys} keys, 24/4/256, fp16 cache '
                  f'widened to fp32, fp32 BLAS, 1 thread), median; host affinity '
                  f'{len(os.sched_getaffinity(0))} cores',
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=50)
    ap.add_argument('--warmup', type=int, default=5)
    ap.add_argument('--layers', type=int, default=LAYERS)
    ap.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline')
    ap.add_argument('--no-extra', action='store_true', help='skip the secondary workloads')
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one GPU only: the attention path runs on a single MI355X; '
              'multi-GPU sharding is a design note, not a measured configuration.', file=sys.stderr)
        sys.exit(2)

    import torch

    from redshift_amd import attention as A
    from redshift_amd.runtime import load_library
    from redshift_amd.workloads import WORKLOADS

    load_library()
    assert torch.cuda.is_available(), 'bench.py needs a GPU'
    torch.cuda.set_device(0)

    w = WORKLOADS['decode_139k']
    log(f'decode_139k: {args.layers} layers x {w.keys} keys, steps={args.steps} warmup={args.warmup}')
    r = time_workload(torch, A, w, args.layers, args.steps, args.warmup, seed=3)
    step_bytes = args.layers * w.kv_bytes()
    gbs = step_bytes / (r['ms_per_step'] * 1e-3) / 1e9
    split_gbs = w.kv_bytes() / (r['split_us'] * 1e-6) / 1e9
    result = {
        'metric': METRIC, 'value': round(gbs, 1), 'unit': 'GB/s', 'n_gpus': 1,
        'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': round(r['ms_per_step'], 4),
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f16',
        'data': 'synthetic',
        'config': {'workload': 'decode_139k', 'q_heads': w.q_heads, 'kv_heads': w.kv_heads,
                   'head_dim': w.head_dim, 'keys': w.keys, 'tokens': w.tokens,
                   'layers': args.layers, 'kv_dtype': 'f16', 'outlier_keys': w.outliers},
        'us_per_layer': round(1000 * r['ms_per_step'] / args.layers, 2),
        'eager_us_per_layer': round(1000 * r['eager_ms_per_step'] / args.layers, 2),
        'timing': 'step = 16 layers x (split-K kernel + combine) replayed as one HIP graph; '
                  'roofline kernel_us = split-K kernel alone, HIP events in an eager loop',
        'roofline': {'bound': 'hbm', 'kernel': 'attention_split (decode)',
                     'achieved': round(split_gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': round(split_gbs / HBM_PEAK_GBS, 4), 'traffic': None,
                     'kernel_us': round(r['split_us'], 2), 'bytes_per_launch': w.kv_bytes()},
    }
    if not args.no_extra:
        extra = {}
        for name, steps in (('verify8_16k', args.steps), ('decode_4k', args.steps)):
            wx = WORKLOADS[name]
            log(f'{name}: {args.layers} layers')
            rx = time_workload(torch, A, wx, args.layers, steps, args.warmup, seed=1)
            us = 1000 * rx['ms_per_step'] / args.layers
            extra[name] = {'us_per_layer': round(us, 2),
                           'GB/s': round(wx.kv_bytes() / (us * 1e-6) / 1e9, 1),
                           'eager_us_per_layer': round(1000 * rx['eager_ms_per_step'] / args.layers, 2),
                           'split_kernel_us': round(rx['split_us'], 2),
                           'split_kernel_GB/s': round(wx.kv_bytes() / (rx['split_us'] * 1e-6) / 1e9, 1),
                           'frac_hbm': round(wx.kv_bytes() / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        wp = WORKLOADS['prefill_2k']
        log(f'prefill_2k: 4 layers')
        rp = time_workload(torch, A, wp, 4, max(3, args.steps // 4), 2, seed=2)
        kernel_s = rp['split_us'] * 1e-6
        extra['prefill_2k'] = {'us_per_layer': round(1000 * rp['ms_per_step'] / 4, 1),
                               'kernel_us': round(rp['split_us'], 1),
                               'TFLOP/s': round(wp.flops() / kernel_s / 1e12, 1),
                               'frac_mfma_peak': round(wp.flops() / kernel_s / MFMA_BF16_PEAK, 4),
                               'flops_per_layer': wp.flops()}
        result['extra'] = extra
    if not args.no_cpu:
        log('cpu baseline (numpy fp32, 1 thread, one layer)')
        result['cpu_baseline'] = cpu_baseline(w)
    print(json.dumps(result), flush=True)


if __name__ == '__main__':
    main()
