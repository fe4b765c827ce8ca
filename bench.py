"""Benchmark of the full-attention path on one MI355X.

A step is one token's attention over all 16 full-attention layers of the
model (24 query heads, 4 KV heads, head_dim 256), each layer with its own
fp16 KV cache of 139,264 tokens in HBM (64 keys per layer scaled x8): the
decode at maximum context.  Each layer is two kernels: split-K over the
pages, then the log-sum-exp combine.  `value` is the achieved HBM bandwidth
over the algorithmic K+V bytes (each key read once) of the whole step
replayed as a HIP graph; `roofline` is the split-K kernel alone, timed with
HIP events on the stream it runs on.  Secondary workloads (speculative
verify-8 on a 16K prefix, decode at 4K, chunked prefill, and the device
drop-in of the reference's fused k_attention at verify-8/16K and decode/139K)
are under `extra`.

The CPU baseline is the numpy fp32 restatement of the reference's CPU
attention (oracle/attention_ref.py), run on this host on one layer's decode.
"""
import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = 'µs/layer + achieved HBM GB/s, GQA decode/verify-8 @16K and 139,264 ctx'
# HBM bytes per launch of the decode kernel, from rocprofv3 FETCH_SIZE and
# WRITE_SIZE passes scaled by a plain-copy calibration (see the file).
TRAFFIC_FILE = ROOT / 'profiles' / 'attention_stream_decode_139k_traffic.txt'
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK = 2.5e15   # dense bf16 FLOP/s
LAYERS = 16
# Seconds of full load before every timed region (see settle).
SETTLE_S = 0.25


def log(msg):
    print(f'[bench] {msg}', file=sys.stderr, flush=True)


def settle(torch, run, minimum, seconds=SETTLE_S):
    """Runs `run` (one step) at least `minimum` times and until `seconds` of
    wall time have passed, synchronising every 8 runs; returns the count.

    The GPU's clock and board power ramp up over tens of milliseconds of full
    load.  Measured on decode_139k graph replays after the eager loop: the
    first ~15 replays (30 ms) took 90.3-91.2 us per layer while sclk rose
    from 2121 to 2176 MHz and power from 556 to 630 W; from about 650 W and
    2190 MHz on, every replay took 85.6-86.3 us.  A timed region that starts
    inside the ramp measures the ramp, so every one starts after this."""
    torch.cuda.synchronize()
    t_end = time.perf_counter() + seconds
    n = 0
    while n < minimum or time.perf_counter() < t_end:
        for _ in range(8):
            run()
            n += 1
        torch.cuda.synchronize()
    return n


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


def time_workload(torch, A, w, layers, steps, warmup, seed, sample=None):
    """Times `steps` steps of `layers` attention calls.

    Returns dict(ms_per_step: one step replayed as a captured HIP graph,
    eager_ms_per_step: the same launches issued one by one, replay_ms: each
    timed replay, split_us: median duration of the split-K (or prefill)
    kernel from events recorded around each of its launches in the eager
    loop, on the stream it runs on, and split_us_mean: their mean).  With
    `sample`, also its results right before and right after the timed
    replays (device_before, device_after)."""
    caches, queries = make_layers(torch, A, w, layers, seed)
    ws = A.workspace(A.attention_workspace_bytes(w.q_heads, w.kv_heads, w.head_dim, w.tokens, w.position))
    outs = [torch.empty_like(q) for q in queries]
    one_chunk = w.tokens * w.group <= A.MAX_CHUNK_ROWS

    # One layer: the split-K kernel then the combine kernel (the two launches
    # qv_attention makes, issued through its two phases so that events can
    # bracket the split kernel alone), or the prefill kernel.
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

    settled = settle(torch, step, warmup)
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
    settled_graph = settle(torch, graph.replay, warmup)
    # One event pair per replay as well (recorded between replays, outside
    # the graph): the spread of the step time over the timed steps.
    replay_ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]

    def replay(s):
        replay_ev[s][0].record()
        graph.replay()
        replay_ev[s][1].record()

    device_before = sample() if sample else None
    graph_ms = timed(replay, steps)
    device_after = sample() if sample else None
    replay_ms = [e[0].elapsed_time(e[1]) for e in replay_ev]
    del graph
    split_graph_us = None
    if one_chunk:
        # The split kernels alone, replayed as one graph: the kernel's time
        # without the host launch overhead that eager events include.
        def splits_only():
            for i in range(layers):
                A.attention_split(queries[i], caches[i], w.position, w.scale, ws)
        sgraph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(capture_stream):
            splits_only()
            torch.cuda.synchronize()
            with torch.cuda.graph(sgraph, stream=capture_stream):
                splits_only()
        torch.cuda.current_stream().wait_stream(capture_stream)
        settle(torch, sgraph.replay, warmup)
        split_graph_us = 1000.0 * timed(lambda s: sgraph.replay(), steps) / layers
        del sgraph
    del caches
    torch.cuda.empty_cache()
    return dict(ms_per_step=graph_ms, eager_ms_per_step=eager_ms, replay_ms=replay_ms,
                device_before=device_before, device_after=device_after,
                settle_steps=settled, settle_replays=settled_graph,
                split_us=1000.0 * statistics.median(split_ms), split_us_mean=1000.0 * sum(split_ms) / len(split_ms),
                split_graph_us=split_graph_us)


def sha256_of(paths):
    """SHA-256 over the given files' bytes, in order, or None if one is missing."""
    import hashlib
    h = hashlib.sha256()
    try:
        for path in paths:
            h.update(path.read_bytes())
    except OSError:
        return None
    return h.hexdigest()


def commit_of(lib_sha256):
    """The commit the line was measured at and where that is known from:
    the checkout's .git, else the commit recorded when the library was built
    (redshift_amd/lib/build_info.json), if it describes the loaded library."""
    from redshift_amd.build import BUILD_INFO, git_head
    head = git_head(ROOT)
    if head is not None:
        return head, 'checkout'
    try:
        info = json.loads(BUILD_INFO.read_text())
    except (OSError, ValueError):
        return None, None
    if info.get('library_sha256') == lib_sha256 and info.get('git_head'):
        return info['git_head'], 'build'
    return None, None


def gpu_card(torch):
    """The DRM card of cuda:0, matched by PCI domain and bus, or None."""
    props = torch.cuda.get_device_properties(0)
    want = (getattr(props, 'pci_domain_id', None), getattr(props, 'pci_bus_id', None))
    for card in sorted(Path('/sys/class/drm').glob('card[0-9]*')):
        if '-' in card.name:
            continue
        try:
            pci = os.path.basename(os.path.realpath(card / 'device'))   # dddd:bb:dd.f
            domain, bus = (int(x, 16) for x in pci.split(':')[:2])
        except (OSError, ValueError):
            continue
        if (domain, bus) == want:
            return card
    return None


def gpu_clocks(card):
    """The state of cuda:0, read as plain files (no subprocess): the current
    DPM level of pp_dpm_sclk, pp_dpm_mclk and pp_dpm_fclk (the starred line),
    and the hwmon readings (temperatures in C, clocks in MHz, power in W)."""
    clocks = {}
    if card is None:
        return clocks
    for name in ('sclk', 'mclk', 'fclk'):
        try:
            lines = (card / 'device' / f'pp_dpm_{name}').read_text().splitlines()
        except OSError:
            continue
        current = [line.split(':', 1)[1].replace('*', '').strip() for line in lines if line.rstrip().endswith('*')]
        clocks[name] = current[0] if current else None
    for hwmon in sorted((card / 'device' / 'hwmon').glob('hwmon*')):
        for path in sorted(hwmon.glob('*_input')) + sorted(hwmon.glob('power*_average')):
            kind = path.name.split('_')[0]
            try:
                label = (hwmon / f'{kind}_label').read_text().strip()
            except OSError:
                label = kind
            try:
                raw = int(path.read_text().strip())
            except (OSError, ValueError):
                continue
            scale = 1e-3 if kind.startswith('temp') else 1e-6
            clocks[f'{label}_{path.name.split("_", 1)[1]}'] = round(raw * scale, 1)
    return clocks


def provenance(torch, lib_path):
    """What the line was measured with: the library's and the sources'
    SHA-256, the commit where known, the device and its clock levels."""
    sources = sorted((ROOT / 'redshift_amd' / 'csrc').glob('*')) + sorted((ROOT / 'include').glob('*.h')) + \
        sorted((ROOT / 'redshift_amd').glob('*.py')) + [ROOT / 'bench.py']
    props = torch.cuda.get_device_properties(0)
    card = gpu_card(torch)
    lib_sha = sha256_of([Path(lib_path)])
    head, head_from = commit_of(lib_sha)
    return {'library_sha256': lib_sha, 'sources_sha256': sha256_of(sources),
            'sources': 'redshift_amd/csrc/*, include/*.h, redshift_amd/*.py, bench.py',
            'git_head': head, 'git_head_from': head_from, 'device': props.name, 'arch': props.gcnArchName,
            'cus': props.multi_processor_count, 'torch': torch.__version__,
            'hip': getattr(torch.version, 'hip', None),
            'drm_card': card.name if card is not None else None}


def spread(values_ms, layers):
    """min / median / max of per-replay step times, in us per layer."""
    us = sorted(1000.0 * v / layers for v in values_ms)
    return {'min': round(us[0], 2), 'median': round(statistics.median(us), 2), 'max': round(us[-1], 2),
            'replays': len(us)}


def measured_traffic():
    """traffic_bytes_per_launch from the committed counter summary, or None."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith('traffic_bytes_per_launch'):
                return int(line.split('=')[1])
    except (OSError, ValueError, IndexError):
        pass
    return None


def trace_summary(db_path, gap=1.6):
    """Median kernel durations of a rocprofv3 kernel trace (the rocpd SQLite
    database `-o run` writes as run_results.db), per kernel name, grid and
    work-group size, each such group split into duration clusters where
    consecutive sorted durations jump by more than `gap` times (the same
    kernel and grid serving workloads of different sizes, e.g. decode at
    139,264 and at 16,392 keys).  Prints one line per cluster."""
    import sqlite3
    con = sqlite3.connect(f'file:{db_path}?mode=ro', uri=True)
    groups = {}
    for name, grid, wg, duration in con.execute(
            'select name, grid_x, workgroup_x, duration from kernels order by start'):
        groups.setdefault((name, grid, wg), []).append(duration)
    con.close()
    for (name, grid, wg), durations in groups.items():
        durations.sort()
        clusters, cur = [], [durations[0]]
        for d in durations[1:]:
            if d > gap * cur[-1] and len(cur) > 2:
                clusters.append(cur)
                cur = [d]
            else:
                cur.append(d)
        clusters.append(cur)
        for c in clusters:
            print(f'{name[:110]}  grid_x={grid} wg={wg} calls={len(c)} '
                  f'median_ns={statistics.median(c):.0f} mean_ns={statistics.mean(c):.0f}')


def copy_probe(mib, repeats=5):
    """A plain device copy of `mib` MiB, `repeats` times: the calibration
    kernel for the FETCH_SIZE / WRITE_SIZE counters (bytes known exactly)."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device='cuda')
    dst = torch.empty_like(src)
    for _ in range(repeats):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f'copy probe: {repeats} x {mib} MiB device-to-device copies')


def read_probe(torch, A, w, sets=16, rounds=20, ahead=3, splits=None, merge=True):
    """The plain read of one split-K launch's KV pages (rsp_read_pages in
    libredshift_probe.so): the grid, runs and page addresses of
    attention_ring for workload `w` (57 splits x 4 KV heads for verify8_16k),
    non-temporal 16-byte loads, no arithmetic.  `sets` caches of the
    workload's size rotate, so that the 256 MB Infinity Cache holds none of
    the pages a launch reads (16 x 67 MB).  Each launch is timed by an event
    pair, in graphs of `sets` launches replayed `rounds` times; returns the
    median and mean us per launch and the read rate of the algorithmic bytes.
    `splits` replaces the launch's own key splits (the same pages over
    another grid); the merge reads are then not measured, nor with
    merge=False."""
    import ctypes as ct

    from redshift_amd.build import PROBE_LIBRARY
    from redshift_amd.runtime import library
    probe = ct.CDLL(str(PROBE_LIBRARY))
    probe.rsp_read_pages.argtypes = [ct.c_void_p, ct.c_void_p] + [ct.c_int] * 6 + [ct.c_void_p, ct.c_void_p]
    probe.rsp_read_pages.restype = ct.c_int
    lib = library()
    capacity = A.round_capacity(w.keys)
    caches = [A.PagedKV(w.kv_heads, w.head_dim, capacity, torch.float16) for _ in range(sets)]
    for c in caches:
        c.k.normal_()
        c.v.normal_()
    # The split plan of the workload's own launch: its workspace is
    # kv_heads x splits x rows x (head_dim + 2) floats of partials.
    rows = w.group * w.tokens
    per_split = w.kv_heads * rows * (w.head_dim + 2) * 4
    ws = A.attention_workspace_bytes(w.q_heads, w.kv_heads, w.head_dim, w.tokens, w.position)
    assert rows <= A.MAX_CHUNK_ROWS and ws % per_split == 0, 'not a one-launch split-K workload'
    own = splits is None
    n_pages, splits = -(-w.keys // 32), ws // per_split if own else splits
    sink = torch.zeros(splits * w.kv_heads * 512, dtype=torch.int32, device='cuda')
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(sets * rounds)]

    def launch(c):
        stream = torch.cuda.current_stream().cuda_stream
        rc = probe.rsp_read_pages(c.k.data_ptr(), c.v.data_ptr(), w.kv_heads, w.head_dim, capacity, n_pages,
                                  splits, ahead, sink.data_ptr(), stream)
        assert rc == 0, 'rsp_read_pages refused its arguments'

    for c in caches:
        launch(c)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    capture_stream = torch.cuda.Stream()
    capture_stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(capture_stream):
        with torch.cuda.graph(graph, stream=capture_stream):
            for c in caches:
                launch(c)
    torch.cuda.current_stream().wait_stream(capture_stream)
    settle(torch, graph.replay, 1)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(rounds):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    us_graph = 1000 * start.elapsed_time(end) / (rounds * sets)
    # The same launches one by one, an event pair around each.
    for i in range(sets * rounds):
        ev[i][0].record()
        launch(caches[i % sets])
        ev[i][1].record()
    torch.cuda.synchronize()
    us = sorted(1000 * e[0].elapsed_time(e[1]) for e in ev)
    del graph, caches, lib
    torch.cuda.empty_cache()
    merge_reads = merge_read_probe(torch, probe) if own and merge else None
    page_bytes = 2 * w.kv_heads * n_pages * 32 * w.head_dim * 2
    med = statistics.median(us)
    return {'workload': w.name, 'grid': f'{splits} splits x {w.kv_heads} KV heads, 512 threads',
            'pages_per_head': n_pages, 'pages_in_flight': ahead, 'buffer_sets': sets,
            'us_per_launch_in_graph': round(us_graph, 2), 'us_per_launch_median': round(med, 2),
            'us_per_launch_min': round(us[0], 2),
            'GB/s': round(w.kv_bytes() / (us_graph * 1e-6) / 1e9, 1),
            'frac_hbm': round(w.kv_bytes() / (us_graph * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            'algorithmic_bytes': w.kv_bytes(), 'page_bytes': page_bytes,
            'merge_reads': merge_reads,
            'what': 'plain non-temporal read of the pages one split-K launch of the workload streams; '
                    'GB/s and frac_hbm over the algorithmic K+V bytes and the in-graph time per launch'}


def merge_read_probe(torch, probe, launches=16, rounds=20):
    """rsp_read_rows: one workgroup per KV head reading that head's split-K
    partials, the reads a merge by the last-arriving workgroup of each head
    would make (4 heads; verify-8 at 16K: 57 splits x 48 fp16 O/l rows of
    256 dims plus m and l; decode: 48 splits x 6 fp32 rows plus m and l),
    with default loads and with device-coherent (sc1) loads.  Per launch in
    a graph of `launches`, the buffers read again and again (so from the
    Infinity Cache, as partials just written would be)."""
    import ctypes as ct
    probe.rsp_read_rows.argtypes = [ct.c_void_p, ct.c_int, ct.c_longlong, ct.c_int, ct.c_void_p, ct.c_void_p]
    probe.rsp_read_rows.restype = ct.c_int
    heads = 4
    shapes = {'verify8_16k': 57 * (48 * 256 * 2 + 2 * 48 * 4), 'decode': 48 * (6 * 256 * 4 + 2 * 6 * 4)}
    out = {}
    sink = torch.zeros(heads * 512, dtype=torch.int32, device='cuda')
    for name, per_head in shapes.items():
        per_head = (per_head + 15) // 16 * 16
        buf = torch.randint(0, 1 << 30, (heads * per_head // 4,), dtype=torch.int32, device='cuda')
        for coherent in (0, 1):
            def launch():
                rc = probe.rsp_read_rows(buf.data_ptr(), heads, per_head, coherent, sink.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream)
                assert rc == 0, 'rsp_read_rows refused its arguments'
            launch()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                with torch.cuda.graph(graph, stream=side):
                    for _ in range(launches):
                        launch()
            torch.cuda.current_stream().wait_stream(side)
            settle(torch, graph.replay, 1)
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(rounds):
                graph.replay()
            end.record()
            torch.cuda.synchronize()
            us = 1000 * start.elapsed_time(end) / (rounds * launches)
            out[f'{name}_{"coherent" if coherent else "default"}'] = {
                'bytes_per_head': per_head, 'us_per_launch_in_graph': round(us, 2)}
            del graph
        del buf
    return out


def drop_in_rate(lib, cases=((1, 139263), (8, 16384), (1, 4095)), repeats=5):
    """Times the host-buffer drop-in qv_test_attention (allocation, cache
    upload and download, synchronisation included): the PCIe-inclusive rate,
    reported beside the device-resident figures and never as `value`."""
    import ctypes as ct

    import numpy as np
    H, HKV, D = 24, 4, 256
    rows = []
    for batch, position in cases:
        rng = np.random.default_rng(0)
        n = position + batch
        kc = (rng.standard_normal((n, HKV, D)) * .5).astype(np.float16)
        vc = (rng.standard_normal((n, HKV, D)) * .5).astype(np.float16)
        qg = rng.standard_normal((batch, H, 2 * D)).astype(np.float32)
        k = rng.standard_normal((batch, HKV, D)).astype(np.float32)
        v = rng.standard_normal((batch, HKV, D)).astype(np.float32)
        gamma = np.ones(D, np.float32)
        out = np.empty((batch, H, D), np.float32)
        ptrs = [a.ctypes.data_as(ct.c_void_p) for a in (out, kc, vc, qg, k, v, gamma, gamma)]
        times = []
        for i in range(repeats + 1):
            t0 = time.perf_counter()
            if lib.qv_test_attention(*ptrs, batch, position, ct.c_float(1e-6)) != 0:
                raise RuntimeError(lib.qv_error().decode())
            if i:
                times.append(time.perf_counter() - t0)
        sec = float(np.median(times))
        cache = 2 * position * HKV * D * 2
        rows.append({'batch': batch, 'position': position, 'ms': round(sec * 1e3, 2),
                     'cache_GB/s': round(cache / sec / 1e9, 2)})
    return rows


def time_fused(torch, A, w, layers, steps, warmup, seed):
    """Times the device drop-in of the reference's k_attention
    (qv_attention_fused: prepare + append + attention + gate, fp32 q_gate /
    key / value of the 24/4/256 model) on `layers` caches of workload `w`,
    one call per layer, replayed as a HIP graph.  Returns ms per step."""
    caches, _ = make_layers(torch, A, w, layers, seed)
    gen = torch.Generator(device='cuda')
    gen.manual_seed(seed + 1)
    batch = w.tokens
    q_gate = [torch.randn((batch, 24, 512), generator=gen, device='cuda') for _ in range(layers)]
    key = [torch.randn((batch, 4, 256), generator=gen, device='cuda') for _ in range(layers)]
    value = [torch.randn((batch, 4, 256), generator=gen, device='cuda') for _ in range(layers)]
    norm = torch.ones(256, device='cuda')
    out = torch.empty((batch, 24, 256), device='cuda')
    ws = A.workspace(A.fused_workspace_bytes(batch, w.position))

    def step():
        for i in range(layers):
            A.attention_fused(q_gate[i], key[i], value[i], norm, norm, caches[i], w.position, 1e-6,
                              out=out, ws=ws)

    for _ in range(warmup):
        step()
    graph = torch.cuda.CUDAGraph()
    capture_stream = torch.cuda.Stream()
    capture_stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(capture_stream):
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=capture_stream):
            step()
    torch.cuda.current_stream().wait_stream(capture_stream)
    settle(torch, graph.replay, warmup)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    del graph, caches
    torch.cuda.empty_cache()
    return start.elapsed_time(end) / steps


def time_kv_copy(torch, A, w, layers, steps, warmup, seed):
    """The KV-cache manager's checkpoint copy (qv_kv_copy, the reference's
    copy_state prefix copy, src/runtime.cu:455-485) of a full `w.keys`-token
    prefix, every page of K and V, from each of `layers` caches to a snapshot
    cache.  Returns microseconds per layer (one copy: one kernel, K and V)."""
    from redshift_amd.kvcache import copy_prefix
    caches, _ = make_layers(torch, A, w, layers, seed)
    dtype = caches[0].dtype
    snaps = [A.PagedKV(w.kv_heads, w.head_dim, caches[0].capacity, dtype) for _ in range(layers)]

    def step():
        for i in range(layers):
            copy_prefix(snaps[i], caches[i], w.keys)

    settle(torch, step, warmup)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ok = all(torch.equal(snaps[i].k[:caches[i].k.numel()], caches[i].k) for i in (0, layers - 1))
    del caches, snaps
    torch.cuda.empty_cache()
    assert ok, 'checkpoint copy differs from its source'
    return 1000 * start.elapsed_time(end) / (steps * layers)


def cpu_baseline(torch, A, w, target_s=8.0):
    """The numpy fp32 restatement of the reference's CPU attention (oracle),
    one layer's decode, timed single-threaded and on all host cores (capped
    at 16 threads): median of at least 5 calls, about target_s each.

    The same layer also runs once through the HIP path, and its output is
    checked against the oracle's within max-abs 2e-3 and relative L2 1e-3
    (`check`); a result outside them ends the bench with an error."""
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits

    from oracle.attention_ref import gqa_attention_fp32
    from redshift_amd.workloads import make_inputs

    q, k, v, _ = make_inputs(w)
    k32, v32 = k.astype(np.float32), v.astype(np.float32)
    expected = None

    def run(threads):
        nonlocal expected
        with threadpool_limits(limits=threads):
            expected = gqa_attention_fp32(q, k32, v32, w.position, w.scale)   # warm-up
            times = []
            t_end = time.perf_counter() + target_s
            while len(times) < 5 or time.perf_counter() < t_end:
                t0 = time.perf_counter()
                gqa_attention_fp32(q, k32, v32, w.position, w.scale)
                times.append(time.perf_counter() - t0)
        return float(np.median(times)), len(times)

    host = len(os.sched_getaffinity(0))
    threads = max(1, min(host, 16))
    one, n_one = run(1)
    many, n_many = run(threads)
    model = 'unknown'
    try:
        model = next(line.split(':', 1)[1].strip() for line in open('/proc/cpuinfo')
                     if line.startswith('model name'))
    except (OSError, StopIteration):
        pass
    blas = next((f"{i['internal_api']} {i['version']}" for i in threadpool_info()
                 if i.get('user_api') == 'blas'), 'unknown')
    gbs = lambda sec: round(w.kv_bytes() / sec / 1e9, 3)
    check = gpu_check(torch, A, w, q, k, v, expected)
    return {
        'value': gbs(many), 'unit': 'GB/s', 'cores': threads, 'kind': 'port',
        'us_per_layer': round(many * 1e6, 1),
        'single_thread': {'value': gbs(one), 'unit': 'GB/s', 'cores': 1, 'us_per_layer': round(one * 1e6, 1)},
        'sample': f'median of {n_many} ({threads} threads) and {n_one} (1 thread) single-layer {w.name} '
                  f'calls: {w.keys} keys, 24/4/256, fp16 cache widened to fp32 before timing, fp32 BLAS '
                  f'({blas}) per KV group; host {model}, {host} cores in affinity',
        'check': check,
    }


def gpu_check(torch, A, w, q, k, v, expected):
    """The HIP path on the baseline's inputs (one layer, its own cache),
    compared with the oracle's fp32 output."""
    import numpy as np

    dtype = torch.bfloat16 if w.dtype == 'bf16' else torch.float16
    to_dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to('cuda')
    cache = A.PagedKV(w.kv_heads, w.head_dim, A.round_capacity(w.keys), dtype)
    cache.pack(to_dev(k).to(dtype), to_dev(v).to(dtype))
    got = A.attention(to_dev(q).to(dtype), cache, w.position, w.scale).float().cpu().numpy()
    del cache
    torch.cuda.empty_cache()
    diff = got.astype(np.float64) - expected.astype(np.float64)
    max_abs = float(np.abs(diff).max())
    rel_l2 = float(np.linalg.norm(diff) / np.linalg.norm(expected.astype(np.float64)))
    ok = bool(np.isfinite(got).all() and max_abs <= 2e-3 and rel_l2 <= 1e-3)
    return {'against': 'oracle fp32 output on the same inputs', 'max_abs': max_abs, 'rel_l2': rel_l2,
            'tol_max_abs': 2e-3, 'tol_rel_l2': 1e-3, 'ok': ok}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=50)
    ap.add_argument('--warmup', type=int, default=5)
    ap.add_argument('--layers', type=int, default=LAYERS)
    ap.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline')
    ap.add_argument('--no-extra', action='store_true', help='skip the secondary workloads')
    ap.add_argument('--extras', default='verify8_16k,decode_16k,decode_4k,prefill_2k,prefill512_6k,fused_verify8_16k,'
                                        'fused_decode_139k,'
                                        'fused_prefill_2k,fused_prefill64_16k,fused_verify8_prefix16,'
                                        'fused_verify8_prefix128,kv_checkpoint_139k',
                    help='comma-separated secondary workloads to run')
    ap.add_argument('--drop-in', action='store_true',
                    help='only time the host-buffer qv_test_attention (PCIe-inclusive) and exit')
    ap.add_argument('--copy-probe', type=int, metavar='MIB',
                    help='only run a plain MIB-MiB device copy (counter calibration) and exit')
    ap.add_argument('--read-probe', nargs='?', const='verify8_16k', metavar='WORKLOAD',
                    help='only time the plain read of the KV pages one split-K launch of WORKLOAD '
                         '(default verify8_16k) streams, and exit')
    ap.add_argument('--ahead', type=int, default=3, help='--read-probe: pages of loads in flight per wave (1-4)')
    ap.add_argument('--trace-summary', metavar='DB',
                    help='only print the median kernel durations of a rocprofv3 kernel trace database, and exit')
    ap.add_argument('--probe-splits', metavar='S[,S...]',
                    help='--read-probe: read the same pages over these key splits per KV head instead of '
                         'the launch\'s own (one line each)')
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one GPU only: the attention path runs on a single MI355X; '
              'multi-GPU sharding is a design note, not a measured configuration.', file=sys.stderr)
        sys.exit(2)

    import torch

    from redshift_amd import attention as A
    from redshift_amd.runtime import load_library
    from redshift_amd.workloads import WORKLOADS, Workload

    assert torch.cuda.is_available(), 'bench.py needs a GPU'
    torch.cuda.set_device(0)
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    lib = load_library()
    if args.read_probe:
        grids = [int(x) for x in args.probe_splits.split(',')] if args.probe_splits else [None]
        for splits in grids:
            r = read_probe(torch, A, WORKLOADS[args.read_probe], ahead=args.ahead, splits=splits)
            print(json.dumps({'read_probe': r}), flush=True)
        return
    if args.drop_in:
        print(json.dumps({'drop_in': 'qv_test_attention, host buffers, median of 5 after 1 warm-up',
                          'cases': drop_in_rate(lib)}), flush=True)
        return

    w = WORKLOADS['decode_139k']
    log(f'decode_139k: {args.layers} layers x {w.keys} keys, steps={args.steps} warmup={args.warmup}')
    prov = provenance(torch, lib._name)
    card = gpu_card(torch)
    r = time_workload(torch, A, w, args.layers, args.steps, args.warmup, seed=3, sample=lambda: gpu_clocks(card))
    prov['device_before'], prov['device_after'] = r['device_before'], r['device_after']
    prov['device_is'] = ('sysfs DPM levels and hwmon readings of the GPU right before and right after '
                         'the timed graph replays of decode_139k')
    step_bytes = args.layers * w.kv_bytes()
    gbs = step_bytes / (r['ms_per_step'] * 1e-3) / 1e9
    split_gbs = w.kv_bytes() / (r['split_graph_us'] * 1e-6) / 1e9
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
        'timing': 'step = 16 layers x (split-K kernel + combine kernel) replayed as one HIP graph; '
                  'roofline kernel_us = the split-K kernel alone: a graph of its 16 launches (one per '
                  'layer, back to back) timed by HIP events around each replay, per launch '
                  '(kernel_us_eager_median: the median of event pairs around single eager launches, which '
                  'include the dispatch gap); every timed region starts after the warmup '
                  f'steps and at least {SETTLE_S} s of full load (settle_steps eager steps, '
                  'settle_replays graph replays), past the clock and power ramp',
        'settle_steps': r['settle_steps'], 'settle_replays': r['settle_replays'],
        'roofline': {'bound': 'hbm', 'kernel': 'attention_stream (decode split-K)',
                     'achieved': round(split_gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': round(split_gbs / HBM_PEAK_GBS, 4), 'traffic': measured_traffic(),
                     'kernel_us': round(r['split_graph_us'], 2),
                     'kernel_us_eager_median': round(r['split_us'], 2),
                     'kernel_us_eager_mean': round(r['split_us_mean'], 2),
                     'bytes_per_launch': w.kv_bytes(),
                     'frac_step': round(gbs / HBM_PEAK_GBS, 4),
                     'frac_is': 'frac: the split-K kernel alone (kernel_us, in its graph); frac_step: the '
                                'whole layer, split-K + combine kernels in the graph step (us_per_layer)'},
        'step_spread': {**spread(r['replay_ms'], args.layers),
                        'what': 'us per layer of each timed graph replay (an event pair around each)'},
        'provenance': prov,
    }
    # A plain read of the same pages with the same grid, timed the same way
    # (a graph of launches): what reading those bytes alone costs.
    log('decode_139k: plain read of its pages')
    try:
        plain = read_probe(torch, A, w, sets=16, rounds=10, ahead=2, merge=False)
        result['roofline']['plain_read'] = {
            'us': plain['us_per_launch_in_graph'], 'frac_hbm': plain['frac_hbm'], 'grid': plain['grid'],
            'kernel_over_plain_read': round(r['split_graph_us'] / plain['us_per_launch_in_graph'], 4),
            'what': 'rsp_read_pages (libredshift_probe.so): non-temporal 16-byte loads of the same K and V '
                    'pages with the same runs and grid, 512 threads per workgroup, 2 pages in flight per wave, '
                    'no arithmetic, 16 rotating cache sets; us per launch in a graph. A reference point, not '
                    'a bound: the split kernel pipelines its own loads and can read them as fast or faster'}
    except Exception as e:   # a measurement aid: its absence does not void the line
        log(f'plain read not measured: {e}')
    chosen = [] if args.no_extra else [x for x in args.extras.split(',') if x]
    if chosen:
        extra = {}
        for name in ('verify8_16k', 'decode_16k', 'decode_4k'):
            if name not in chosen:
                continue
            wx = WORKLOADS[name]
            log(f'{name}: {args.layers} layers')
            rx = time_workload(torch, A, wx, args.layers, args.steps, args.warmup, seed=1)
            us = 1000 * rx['ms_per_step'] / args.layers
            extra[name] = {'us_per_layer': round(us, 2),
                           'step_spread': spread(rx['replay_ms'], args.layers),
                           'GB/s': round(wx.kv_bytes() / (us * 1e-6) / 1e9, 1),
                           'eager_us_per_layer': round(1000 * rx['eager_ms_per_step'] / args.layers, 2),
                           'split_kernel_us': round(rx['split_us'], 2),
                           'split_kernel_GB/s': round(wx.kv_bytes() / (rx['split_us'] * 1e-6) / 1e9, 1),
                           'split_graph_us': round(rx['split_graph_us'], 2),
                           'split_graph_frac_hbm': round(wx.kv_bytes() / (rx['split_graph_us'] * 1e-6) / 1e9
                                                         / HBM_PEAK_GBS, 4),
                           'frac_hbm': round(wx.kv_bytes() / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        if 'prefill_2k' in chosen:
            wp = WORKLOADS['prefill_2k']
            log('prefill_2k: 4 layers')
            # At least 52 timed calls at the default 50 steps (13 steps of 4 layers).
            rp = time_workload(torch, A, wp, 4, max(3, (args.steps + 3) // 4), 2, seed=2)
            kernel_s = rp['split_us'] * 1e-6
            layer_s = rp['ms_per_step'] * 1e-3 / 4
            extra['prefill_2k'] = {'us_per_layer': round(1000 * rp['ms_per_step'] / 4, 1),
                                   'kernel_us': round(rp['split_us'], 1),
                                   'kernel_us_mean': round(rp['split_us_mean'], 1),
                                   'kernel_is': 'conversion pass + prefill kernel of one eager call, median '
                                                'of the HIP-event-timed calls',
                                   'TFLOP/s': round(wp.flops() / layer_s / 1e12, 1),
                                   'frac_mfma_peak': round(wp.flops() / layer_s / MFMA_BF16_PEAK, 4),
                                   'kernel_TFLOP/s': round(wp.flops() / kernel_s / 1e12, 1),
                                   'frac_mfma_peak_kernel': round(wp.flops() / kernel_s / MFMA_BF16_PEAK, 4),
                                   'frac_is': 'frac_mfma_peak: the layer (conversion pass + prefill kernel) '
                                              'replayed in a HIP graph, us_per_layer; frac_mfma_peak_kernel: '
                                              'the eager HIP-event median, kernel_us, whose calls run the same '
                                              'kernels between host launch gaps',
                                   'flops_per_layer': wp.flops()}
        if 'prefill512_6k' in chosen:
            # A 512-token bf16 chunk after 6144 cached tokens: 16 row workgroups
            # per KV head, 64 in all, so the call splits every workgroup's pages
            # into 4 runs and combines the partial rows (combine_prefill).
            w5 = Workload('prefill512_6k', 24, 4, 256, 512, 6144, 1 / 16, 'bf16', 2)
            log('prefill512_6k: 4 layers')
            r5 = time_workload(torch, A, w5, 4, max(3, (args.steps + 3) // 4), 2, seed=11)
            layer_s = r5['ms_per_step'] * 1e-3 / 4
            extra['prefill512_6k'] = {'us_per_layer': round(1e6 * layer_s, 1),
                                      'eager_call_us': round(r5['split_us'], 1),
                                      'TFLOP/s': round(w5.flops() / layer_s / 1e12, 1),
                                      'frac_mfma_peak': round(w5.flops() / layer_s / MFMA_BF16_PEAK, 4),
                                      'what': 'qv_attention, 512 bf16 tokens at 6144, graph step: V conversion '
                                              '+ prefill with its keys split in 4 + combine_prefill'}
        for name in ('fused_verify8_16k', 'fused_decode_139k'):
            if name not in chosen:
                continue
            wf = WORKLOADS[name[len('fused_'):]]
            log(f'{name}: {args.layers} layers')
            us = 1000 * time_fused(torch, A, wf, args.layers, args.steps, args.warmup, seed=4) / args.layers
            extra[name] = {'us_per_layer': round(us, 2),
                           'GB/s': round(wf.kv_bytes() / (us * 1e-6) / 1e9, 1),
                           'frac_hbm': round(wf.kv_bytes() / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                           'what': 'qv_attention_fused per layer: prepare + append + attention + gate'
                                   + (' (one token: query prepared and key and value appended in the '
                                      'split kernel, the new key added in the combine; two launches)'
                                      if wf.tokens == 1 else
                                      ' (query prepared in the ring kernel while its first pages load, '
                                      'new keys attended to and appended by its first split; gated '
                                      'combine; two launches)')}
        if 'fused_prefill_2k' in chosen:
            # The fused drop-in on a 2048-token prefill chunk at position 6144
            # (fp16 pages, the model's fp32 q_gate/key/value), one call per layer.
            wq = Workload('fused_prefill_2k', 24, 4, 256, 2048, 6144, 1 / 16, 'f16', 2, kv_std=0.5)
            log('fused_prefill_2k: 4 layers')
            ms = time_fused(torch, A, wq, 4, max(3, args.steps // 4), 2, seed=6)
            us = 1000 * ms / 4
            extra['fused_prefill_2k'] = {'us_per_layer': round(us, 1),
                                         'TFLOP/s': round(wq.flops() / (us * 1e-6) / 1e12, 1),
                                         'frac_mfma_peak': round(wq.flops() / (us * 1e-6) / MFMA_BF16_PEAK, 4),
                                         'what': 'qv_attention_fused on a 2048-token chunk at 6144: prepare + '
                                                 'append + precise prefill (fp32 q as fp16 hi + lo, hi + lo P) + gate'}
        if 'fused_prefill64_16k' in chosen:
            # A short prefill chunk on a long prefix (64 tokens at 16,384): six
            # query heads per KV head make 384 rows, three workgroups of 128
            # per KV head, so the call splits its keys over the device's CUs
            # and combines the partial rows (with the gate).
            wc = Workload('fused_prefill64_16k', 24, 4, 256, 64, 16384, 1 / 16, 'f16', 9, kv_std=0.5)
            log(f'fused_prefill64_16k: {args.layers} layers')
            us = 1000 * time_fused(torch, A, wc, args.layers, args.steps, args.warmup, seed=10) / args.layers
            extra['fused_prefill64_16k'] = {
                'us_per_layer': round(us, 2),
                'TFLOP/s': round(wc.flops() / (us * 1e-6) / 1e12, 1),
                'frac_mfma_peak': round(wc.flops() / (us * 1e-6) / MFMA_BF16_PEAK, 4),
                'GB/s': round(wc.kv_bytes() / (us * 1e-6) / 1e9, 1),
                'frac_hbm': round(wc.kv_bytes() / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                'what': 'qv_attention_fused on a 64-token chunk at 16,384: prepare + append + precise prefill '
                        'with its keys split over the CUs + gated combine, graph step'}
        for prefix in (16, 128):
            name = f'fused_verify8_prefix{prefix}'
            if name not in chosen:
                continue
            # The reference's only published timing of this path: T=8
            # candidates on a short prefix, qv::attention 8,642.7 ns plus
            # qv::attn_prepare 4,088.0 ns per layer on a V100
            # (reports/llama-v100-profile-redshift-b8.txt:14-15).
            ws_ = Workload(name, 24, 4, 256, 8, prefix, 1 / 16, 'f16', 7, kv_std=0.5)
            log(f'{name}: {args.layers} layers')
            us = 1000 * time_fused(torch, A, ws_, args.layers, args.steps, args.warmup, seed=8) / args.layers
            extra[name] = {'us_per_layer': round(us, 2),
                           'reference_v100_us': 12.73,
                           'what': f'qv_attention_fused per layer, 8 tokens after a {prefix}-token prefix '
                                   '(prepare + append + attention + gate), graph step; reference: '
                                   'V100 qv::attention 8.64 us + qv::attn_prepare 4.09 us'}
        if 'kv_checkpoint_139k' in chosen:
            log('kv_checkpoint_139k: 4 layers')
            us = time_kv_copy(torch, A, w, 4, max(5, args.steps // 2), 2, seed=5)
            moved = 2 * w.kv_bytes()   # every byte of K and V read once and written once
            extra['kv_checkpoint_139k'] = {
                'us_per_layer': round(us, 1), 'GB/s': round(moved / (us * 1e-6) / 1e9, 1),
                'frac_hbm': round(moved / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                'what': 'qv_kv_copy of a 139,264-token prefix (K and V pages, read + write bytes)'}
        result['extra'] = extra
    if not args.no_cpu:
        log('cpu baseline (numpy fp32, 1 thread, one layer)')
        result['cpu_baseline'] = cpu_baseline(torch, A, w)
    print(json.dumps(result), flush=True)
    if 'cpu_baseline' in result and not result['cpu_baseline']['check']['ok']:
        sys.exit('bench: the HIP output differs from the oracle beyond tolerance: '
                 + json.dumps(result['cpu_baseline']['check']))


if __name__ == '__main__':
    main()
