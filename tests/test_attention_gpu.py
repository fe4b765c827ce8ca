"""GPU parity tests of libredshift_hip against the CPU oracle.

Ports of the reference's attention tests (tests/test_cuda.py:72-87,201-273)
through the drop-in host-pointer entry qv_test_attention, with the same
tolerances, and raw-core parity on the seeded workloads through the device
ABI: max-abs <= 2e-3 and relative-L2 <= 1e-3 against the float64 oracle.
"""
import ctypes as ct

import numpy as np
import pytest

from oracle import attention_ref as ref
from oracle import kat
from redshift_amd import attention as A
from redshift_amd import layout
from redshift_amd.workloads import WORKLOADS, Workload, make_inputs, to_float

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2 = 2e-3, 1e-3


def ptr(a):
    return a.ctypes.data_as(ct.c_void_p)


def f32(a):
    return np.ascontiguousarray(a, np.float32)


def assert_close(actual, expected, tolerance):
    """tests/test_cuda.py:65-70: |a - e| <= tol * (1 + |e|) and finite."""
    actual = np.asarray(actual, np.float64).reshape(-1)
    expected = np.asarray(expected, np.float64).reshape(-1)
    assert actual.shape == expected.shape
    assert np.all(np.isfinite(actual))
    bad = np.abs(actual - expected) > tolerance * (1 + np.abs(expected))
    assert not bad.any(), f'{bad.sum()} mismatches, first at {np.argmax(bad)}: ' \
                          f'{actual[np.argmax(bad)]} vs {expected[np.argmax(bad)]}'


def assert_parity(actual, expected, max_abs=MAX_ABS, rel_l2=REL_L2):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    assert np.all(np.isfinite(actual))
    err = np.abs(actual - expected).max()
    rel = np.linalg.norm(actual - expected) / np.linalg.norm(expected)
    assert err <= max_abs and rel <= rel_l2, (err, rel)


def run_test_attention(lib, prefix_k, prefix_v, q_gate, key, value, q_norm, k_norm, batch, position, eps):
    """Call qv_test_attention with host buffers; returns (out, kc, vc)."""
    n = position + batch
    kc = np.zeros(n * 1024, np.float16)
    vc = np.zeros(n * 1024, np.float16)
    kc[:position * 1024] = np.asarray(prefix_k, np.float16).reshape(-1)
    vc[:position * 1024] = np.asarray(prefix_v, np.float16).reshape(-1)
    out = np.zeros(batch * 6144, np.float32)
    args = [f32(q_gate), f32(key), f32(value), f32(q_norm), f32(k_norm)]
    rc = lib.qv_test_attention(ptr(out), ptr(kc), ptr(vc), *[ptr(a) for a in args], batch, position, eps)
    assert rc == 0, lib.qv_error()
    return out, kc, vc


def test_attention_cpu_prefix_causality_and_chunking(lib, gpu):
    """tests/test_cuda.py:201-235."""
    c = kat.sine_wave_case()
    batch, position = c['batch'], c['position']
    expected = ref.fused_attention(c['key_cache'], c['value_cache'], c['q_gate'], c['key'], c['value'],
                                   c['q_norm'], c['k_norm'], batch, position, c['epsilon'])
    out, kc, vc = run_test_attention(lib, c['key_cache'], c['value_cache'], c['q_gate'], c['key'],
                                     c['value'], c['q_norm'], c['k_norm'], batch, position, c['epsilon'])
    assert_close(out, expected[0], 3e-4)
    assert_close(kc, expected[1], 2e-3)
    assert_close(vc, expected[2], 0)
    np.testing.assert_array_equal(kc[:position * 1024].view(np.uint16),
                                  c['key_cache'].reshape(-1).view(np.uint16))
    # Sequential evaluation cannot see the later tokens in the chunk.
    seq_k, seq_v = c['key_cache'], c['value_cache']
    sequential = []
    for t in range(batch):
        row, seq_k, seq_v = run_test_attention(
            lib, seq_k, seq_v, c['q_gate'][t], c['key'][t], c['value'][t], c['q_norm'], c['k_norm'],
            1, position + t, c['epsilon'])
        sequential.append(row)
    assert_close(out, np.concatenate(sequential), 3e-5)
    np.testing.assert_array_equal(kc.view(np.uint16), seq_k.view(np.uint16))
    np.testing.assert_array_equal(vc.view(np.uint16), seq_v.view(np.uint16))


@pytest.mark.parametrize('position,batch', [(2047, 3), (32767, 1), (139263, 1), (139262, 2), (139256, 8),
                                            (16384, 8)])
def test_attention_long_context_against_closed_form(lib, gpu, position, batch):
    """tests/test_cuda.py:237-273 (position 139,263 + 1 = the 139,264 capacity),
    also with verification batches that end at the capacity: two tokens (the
    stream kernel preparing its query) and eight (the ring kernel, whose
    first split attends to the new keys)."""
    c = kat.long_context_case(position, batch)
    out, kc, vc = run_test_attention(lib, c['key_cache'], c['value_cache'], c['q_gate'], c['key'],
                                     c['value'], c['q_norm'], c['k_norm'], batch, position, c['epsilon'])
    assert_close(out, c['expected'], 3e-5)
    n = position * 1024
    np.testing.assert_array_equal(kc[:n].view(np.uint16), c['key_cache'].reshape(-1).view(np.uint16))
    np.testing.assert_array_equal(vc[:n].view(np.uint16), c['value_cache'].reshape(-1).view(np.uint16))


@pytest.mark.parametrize('position', [0, 1, 31, 32, 33, 1000])
def test_fused_decode_matches_oracle(gpu, position):
    """One token through the device fused entry: from position 1 on, the
    split kernel prepares the query itself and the combine adds, and
    appends, the new key (no prepare launch); position 0 has no cached key
    and takes the prepared path.  Against the oracle on the reference's
    sine-wave fixture and tolerances; the appended rows must equal the
    prepare kernel's bit for bit (same functions), checked through a batch
    of two that ends at the same token."""
    torch = gpu
    c = kat.sine_wave_case(batch=2, position=position)
    one = {k: (c[k][:1] if k in ('q_gate', 'key', 'value') else c[k]) for k in c}
    expected = ref.fused_attention(one['key_cache'], one['value_cache'], one['q_gate'], one['key'], one['value'],
                                   one['q_norm'], one['k_norm'], 1, position, c['epsilon'])
    capacity = A.round_capacity(position + 2)
    cache = A.PagedKV(4, 256, capacity, torch.float16)
    # Slots past the prefix hold NaN: the split kernel reads the new token's
    # slot (masked) while the first split writes it.
    cache.k.fill_(float('nan'))
    cache.v.fill_(float('nan'))
    if position:
        cache.pack(torch.from_numpy(c['key_cache']).cuda(), torch.from_numpy(c['value_cache']).cuda())
    dev = [torch.from_numpy(f32(one[name])).cuda() for name in ('q_gate', 'key', 'value', 'q_norm', 'k_norm')]
    out = A.attention_fused(*dev, cache, position, c['epsilon'])
    kc, vc = cache.unpack(0, position + 1)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), expected[0], 3e-4)
    assert_close(kc.float().cpu().numpy(), expected[1], 2e-3)
    assert_close(vc.float().cpu().numpy(), expected[2], 0)
    # The prepared path (a batch of two) appends the same bits for token 0.
    cache2 = A.PagedKV(4, 256, capacity, torch.float16)
    cache2.k.fill_(float('nan'))
    cache2.v.fill_(float('nan'))
    if position:
        cache2.pack(torch.from_numpy(c['key_cache']).cuda(), torch.from_numpy(c['value_cache']).cuda())
    dev2 = [torch.from_numpy(f32(c[name])).cuda() for name in ('q_gate', 'key', 'value', 'q_norm', 'k_norm')]
    out2 = A.attention_fused(*dev2, cache2, position, c['epsilon'])
    kc2, vc2 = cache2.unpack(0, position + 1)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(kc.cpu().numpy().view(np.uint16), kc2.cpu().numpy().view(np.uint16))
    np.testing.assert_array_equal(vc.cpu().numpy().view(np.uint16), vc2.cpu().numpy().view(np.uint16))
    assert_close(out.cpu().numpy(), out2[:1].cpu().numpy(), 3e-5)


@pytest.mark.parametrize('batch,position', [(3, 5), (8, 40)])
def test_drop_in_matches_reference_vectors(lib, gpu, batch, position):
    """qv_test_attention against the output of the reference's own CPU
    attention (tests/cpu_reference.py) on its sine-wave fixture, committed
    in tests/golden/fused_attention.npz, with the reference test's
    tolerances (tests/test_cuda.py:218-221)."""
    from pathlib import Path
    z = np.load(Path(__file__).resolve().parent / 'golden' / 'fused_attention.npz')
    g = {k[len(f'b{batch}_p{position}_'):]: z[k] for k in z.files if k.startswith(f'b{batch}_p{position}_')}
    out, kc, vc = run_test_attention(lib, g['kc'][:position], g['vc'][:position], g['q_gate'], g['key'],
                                     g['value'], g['q_norm'], g['k_norm'], batch, position, 1e-6)
    assert_close(out, g['out'], 3e-4)
    assert_close(kc.astype(np.float64), g['kc'].astype(np.float64), 2e-3)
    np.testing.assert_array_equal(vc, g['vc'].reshape(-1))
    np.testing.assert_array_equal(kc[:position * 1024], g['kc'][:position].reshape(-1))


def test_error_is_cleared_after_a_successful_call(lib, gpu):
    """tests/test_cuda.py:85-87."""
    one = np.ones(1, np.float32)
    assert lib.qv_test_attention(*([ptr(one)] * 8), 8, 139257, 1e-6) == -1
    assert lib.qv_error()
    c = kat.sine_wave_case(batch=1, position=0)
    run_test_attention(lib, c['key_cache'], c['value_cache'], c['q_gate'], c['key'], c['value'],
                       c['q_norm'], c['k_norm'], 1, 0, 1e-6)
    assert lib.qv_error() == b''


# ---- raw core on the paged cache ------------------------------------------

def to_torch(x, dtype, torch):
    if dtype == 'bf16':
        return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(torch.bfloat16).cuda()
    return torch.from_numpy(np.ascontiguousarray(x, np.float16)).cuda()


def make_cache(k, v, w, torch, capacity=None, fill_nan=False):
    dtype = torch.bfloat16 if w.dtype == 'bf16' else torch.float16
    cache = A.PagedKV(w.kv_heads, w.head_dim, capacity or A.round_capacity(w.keys), dtype)
    if fill_nan:
        cache.k.fill_(float('nan'))
        cache.v.fill_(float('nan'))
    cache.pack(to_torch(k, w.dtype, torch), to_torch(v, w.dtype, torch))
    return cache


def gpu_attention(w, q, k, v, torch, out_dtype=None, **kw):
    cache = make_cache(k, v, w, torch, **kw)
    out = A.attention(to_torch(q, w.dtype, torch), cache, w.position, w.scale, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return out.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize('name', ['decode_4k', 'decode_16k', 'verify8_16k', 'decode_139k'])
def test_raw_attention_workloads(gpu, name):
    w = WORKLOADS[name]
    q, k, v, _ = make_inputs(w)
    got = gpu_attention(w, q, k, v, gpu)
    want = ref.gqa_attention(q, k, v, w.position, w.scale)
    assert_parity(got, want)


def test_raw_attention_cpu_plumbing_shape(gpu):
    """8/2/128 on fp16-rounded inputs (the cache stores 16-bit values); the
    oracle runs on exactly those rounded values."""
    w = WORKLOADS['cpu_plumbing']
    q, k, v, _ = make_inputs(w)
    w16 = Workload(**{**w.__dict__, 'dtype': 'f16'})
    q, k, v = (x.astype(np.float16) for x in (q, k, v))
    assert_parity(gpu_attention(w16, q, k, v, gpu), ref.gqa_attention(q, k, v, w.position, w.scale))


def test_raw_attention_prefill_shape_sampled_rows(gpu):
    """2048 bf16 queries on 8192 keys; the oracle checks 24 sampled rows.
    bf16 output rounding alone is ~1.6e-3 relative RMS, so the relative-L2
    bound applies to the oracle rounded to bf16; max-abs uses the unrounded
    oracle."""
    w = WORKLOADS['prefill_2k']
    q, k, v, _ = make_inputs(w)
    got = gpu_attention(w, q, k, v, gpu)
    rows = np.unique(np.concatenate([[0, 1, 2047], np.linspace(3, 2046, 21).astype(int)]))
    want = ref.gqa_attention(to_float(q, 'bf16'), to_float(k, 'bf16'), to_float(v, 'bf16'),
                             w.position, w.scale, rows=rows)
    from redshift_amd.workloads import f32_to_bf16_bits
    want_bf16 = to_float(f32_to_bf16_bits(want.astype(np.float32)), 'bf16')
    assert np.abs(got[rows] - want).max() <= MAX_ABS
    assert_parity(got[rows], want_bf16)


@pytest.mark.parametrize('T,position', [(1, 0), (1, 31), (1, 32), (2, 30), (3, 5), (5, 1000),
                                        (8, 0), (8, 28), (8, 31), (8, 4089), (7, 139257)])
def test_raw_attention_edges_and_stale_pages(gpu, T, position):
    """Ragged last page, first page, capacity boundary; pages past the last
    key hold NaN, which must never reach the result."""
    w = Workload('edge', 24, 4, 256, T, position, 1 / 16, 'f16', 100 + T, 1.0, 0.5)
    q, k, v, _ = make_inputs(w)
    got = gpu_attention(w, q, k, v, gpu, fill_nan=True)
    assert_parity(got, ref.gqa_attention(q, k, v, w.position, w.scale))


@pytest.mark.parametrize('T,position,dtype', [(1, 20000, 'f16'), (1, 20000, 'bf16'), (3, 3000, 'f16')])
def test_single_kv_head_many_splits(gpu, T, position, dtype):
    """One KV head spreads a row's keys over many splits (157 at 20,000
    keys, more than one combine round of 64), fp32 partials of the decode
    kernel and fp16 ones of the verify kernel."""
    w = Workload('one_head', 24, 1, 256, T, position, 1 / 16, dtype, 600 + T, 1.0, 0.5)
    q, k, v, _ = make_inputs(w)
    want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), position, w.scale)
    assert_parity(gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32), want)


def test_verify_peaked_softmax(gpu):
    """Verify-8 whose softmax is dominated by a few keys scaled x8: the
    output is then close to single V rows, the largest values the fp16
    partial rows of the verify kernel (O / l) and the fp16 output can hold;
    both roundings stay inside the bounds."""
    w = Workload('peaked', 24, 4, 256, 8, 5000, 1 / 16, 'f16', 41, q_std=1.0, kv_std=0.5, outliers=16)
    q, k, v, _ = make_inputs(w)
    want = ref.gqa_attention(q, k, v, w.position, w.scale)
    assert np.abs(want).max() > 0.5   # some rows follow single keys
    assert_parity(gpu_attention(w, q, k, v, gpu, fill_nan=True), want)


def test_raw_attention_grouped_equals_sequential(gpu):
    w = Workload('group', 24, 4, 256, 8, 777, 1 / 16, 'f16', 9, 1.0, 0.5)
    q, k, v, _ = make_inputs(w)
    torch = gpu
    cache = make_cache(k, v, w, torch)
    qt = to_torch(q, 'f16', torch)
    grouped = A.attention(qt, cache, w.position, w.scale).float()
    sequential = torch.cat([A.attention(qt[t:t + 1], cache, w.position + t, w.scale).float()
                            for t in range(w.tokens)])
    torch.cuda.synchronize()
    assert torch.allclose(grouped, sequential, atol=2e-3, rtol=0)
    assert_parity(grouped.cpu().numpy(), ref.gqa_attention(q, k, v, w.position, w.scale))


@pytest.mark.parametrize('head_dim', [128, 256])
def test_pages_round_trip_bitwise(gpu, head_dim):
    torch = gpu
    rng = np.random.default_rng(head_dim)
    n, capacity, heads = 77, 96, 3
    bits = rng.integers(0, 1 << 16, size=(2, n, heads, head_dim), dtype=np.uint16)
    k_rows = torch.from_numpy(bits[0].view(np.int16)).cuda().view(torch.float16)
    v_rows = torch.from_numpy(bits[1].view(np.int16)).cuda().view(torch.float16)
    cache = A.PagedKV(heads, head_dim, capacity, torch.float16)
    cache.pack(k_rows[:40], v_rows[:40], first=0).pack(k_rows[40:], v_rows[40:], first=40)
    k2, v2 = cache.unpack(0, n)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(k2.view(torch.int16).cpu().numpy().view(np.uint16), bits[0])
    np.testing.assert_array_equal(v2.view(torch.int16).cpu().numpy().view(np.uint16), bits[1])
    # The pack kernel agrees with the host description of the layout.
    pk = cache.k.view(torch.int16).cpu().numpy().view(np.uint16)
    pv = cache.v.view(torch.int16).cpu().numpy().view(np.uint16)
    off_k = layout.k_offsets(n, head_dim)
    off_v = layout.v_offsets(n, head_dim)
    for h in range(heads):
        np.testing.assert_array_equal(pk[h * capacity * head_dim + off_k], bits[0][:, h, :])
        np.testing.assert_array_equal(pv[h * capacity * head_dim + off_v], bits[1][:, h, :])


def test_fused_device_path_matches_oracle(gpu):
    torch = gpu
    c = kat.sine_wave_case(batch=8, position=300)
    position, batch = c['position'], c['batch']
    expected = ref.fused_attention(c['key_cache'], c['value_cache'], c['q_gate'], c['key'], c['value'],
                                   c['q_norm'], c['k_norm'], batch, position, c['epsilon'])
    cache = A.PagedKV(4, 256, A.round_capacity(position + batch), torch.float16)
    cache.pack(torch.from_numpy(c['key_cache']).cuda(), torch.from_numpy(c['value_cache']).cuda())
    dev = [torch.from_numpy(f32(c[name])).cuda() for name in ('q_gate', 'key', 'value', 'q_norm', 'k_norm')]
    out = A.attention_fused(*dev, cache, position, c['epsilon'])
    kc, vc = cache.unpack(0, position + batch)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), expected[0], 3e-4)
    assert_close(kc.float().cpu().numpy(), expected[1], 2e-3)
    assert_close(vc.float().cpu().numpy(), expected[2], 0)


@pytest.mark.parametrize('batch,position', [(5, 5000), (8, 20000), (3, 40), (2, 100), (4, 31), (6, 33),
                                            (7, 1), (2, 257), (2, 3000), (3, 300), (4, 1000), (6, 4097),
                                            (7, 9000), (8, 249), (3, 254), (2, 255)])
def test_fused_verify_matches_oracle(gpu, batch, position):
    """Fused verification batches of 2-8 tokens on the reference's sine-wave
    fixture and tolerances, with the appended cache rows: on short contexts
    the one-launch kernel (a first cached page that is full, 31 + 1, or
    holds one key); past 256 keys the split kernels preparing the fp32 query
    in their prologue (two tokens: the stream kernel; 3-8: the ring kernel,
    whose first split attends to the new keys), at split lengths of 1 to
    ~11 pages."""
    torch = gpu
    c = kat.sine_wave_case(batch=batch, position=position)
    expected = ref.fused_attention(c['key_cache'], c['value_cache'], c['q_gate'], c['key'], c['value'],
                                   c['q_norm'], c['k_norm'], batch, position, c['epsilon'])
    cache = A.PagedKV(4, 256, A.round_capacity(position + batch), torch.float16)
    cache.pack(torch.from_numpy(c['key_cache']).cuda(), torch.from_numpy(c['value_cache']).cuda())
    dev = [torch.from_numpy(f32(c[name])).cuda() for name in ('q_gate', 'key', 'value', 'q_norm', 'k_norm')]
    out = A.attention_fused(*dev, cache, position, c['epsilon'])
    kc, vc = cache.unpack(0, position + batch)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), expected[0], 3e-4)
    assert_close(kc.float().cpu().numpy(), expected[1], 2e-3)
    assert_close(vc.float().cpu().numpy(), expected[2], 0)


@pytest.mark.parametrize('position', [0, 100, 247])
def test_short_fused_appends_the_prepare_kernels_bits(gpu, position):
    """A short context (8 tokens, position + 8 <= 256) runs in one launch
    that prepares and appends the new keys itself; the same tokens as the
    start of a 9-token prefill chunk go through the prepare kernel.  Both
    append the same bits, and both outputs match the oracle."""
    torch = gpu
    c = kat.sine_wave_case(batch=9, position=position)
    dev = {name: torch.from_numpy(f32(c[name])).cuda() for name in ('q_gate', 'key', 'value', 'q_norm', 'k_norm')}
    caches = []
    for _ in range(2):
        cache = A.PagedKV(4, 256, A.round_capacity(position + 9), torch.float16)
        cache.k.fill_(float('nan'))
        cache.v.fill_(float('nan'))
        if position:
            cache.pack(torch.from_numpy(c['key_cache']).cuda(), torch.from_numpy(c['value_cache']).cuda())
        caches.append(cache)
    short = A.attention_fused(dev['q_gate'][:8], dev['key'][:8], dev['value'][:8], dev['q_norm'], dev['k_norm'],
                              caches[0], position, c['epsilon'])
    chunk = A.attention_fused(dev['q_gate'], dev['key'], dev['value'], dev['q_norm'], dev['k_norm'],
                              caches[1], position, c['epsilon'])
    kc = [cache.unpack(0, position + 8) for cache in caches]
    torch.cuda.synchronize()
    for a, b in zip(kc[0], kc[1]):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    expected = ref.fused_attention(c['key_cache'], c['value_cache'], c['q_gate'], c['key'], c['value'],
                                   c['q_norm'], c['k_norm'], 9, position, c['epsilon'])
    assert_close(short.cpu().numpy().reshape(-1), expected[0][:8 * 6144], 3e-4)
    assert_close(chunk.cpu().numpy().reshape(-1), expected[0], 3e-4)
    assert_close(short.cpu().numpy(), chunk[:8].cpu().numpy(), 3e-5)


@pytest.mark.parametrize('batch,position', [
    (9, 0), (120, 8),          # prepared prefill, one run (no or few cached keys): the gated rows directly
    (100, 300), (57, 1),       # prepared prefill: one run of the cached keys, then the chunk's
    (64, 6000),                # prepared prefill: the cached keys in many runs, combine_prefill
    (16, 16000),               # prepared prefill: 62 runs, merged by attention_combine
    (121, 8), (2048, 40),      # the chunk's keys past four pages: prepare launch, then the prefill
])
def test_fused_prefill_chunk_matches_oracle(gpu, batch, position):
    """A prefill chunk through the fused entry (more than 8 tokens) on the
    reference's sine-wave fixture (tests/test_cuda.py:201-216), with that
    test's tolerances: output 3e-4, appended K 2e-3, V exact.  A chunk whose
    keys fit four pages from the one holding key `position` runs the
    prepared prefill (query and keys prepared in the kernel, no prepare
    launch) and combines its splits (gated) when there are cached keys;
    longer chunks take the prepare launch, and 2048 tokens run two passes of
    192 rows per workgroup (one round of workgroups on 256 CUs)."""
    torch = gpu
    c = kat.sine_wave_case(batch=batch, position=position)
    expected = ref.fused_attention(c['key_cache'], c['value_cache'], c['q_gate'], c['key'], c['value'],
                                   c['q_norm'], c['k_norm'], batch, position, c['epsilon'])
    cache = A.PagedKV(4, 256, A.round_capacity(position + batch), torch.float16)
    cache.k.fill_(float('nan'))
    cache.v.fill_(float('nan'))
    if position:
        cache.pack(torch.from_numpy(c['key_cache']).cuda(), torch.from_numpy(c['value_cache']).cuda())
    dev = [torch.from_numpy(f32(c[name])).cuda() for name in ('q_gate', 'key', 'value', 'q_norm', 'k_norm')]
    q_parts = batch * 24 * 256 * 4
    if position < 1000:
        assert A.fused_workspace_bytes(batch, position) == q_parts   # no key splits: q parts only
    else:
        assert A.fused_workspace_bytes(batch, position) > q_parts    # and the split partials
    out = A.attention_fused(*dev, cache, position, c['epsilon'])
    kc, vc = cache.unpack(0, position + batch)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), expected[0], 3e-4)
    assert_close(kc.float().cpu().numpy(), expected[1], 2e-3)
    assert_close(vc.float().cpu().numpy(), expected[2], 0)


@pytest.mark.parametrize('batch,position', [(8192, 0), (2048, 139264 - 2048)])
def test_fused_chunk_at_its_limits(gpu, batch, position):
    """The fused entry at its documented limits: the largest chunk (8,192
    tokens, the prepare launch then the precise prefill) and a 2048-token
    chunk that fills the 139,264-token capacity to its last slot.  Random
    inputs as in test_fused_random_shapes_against_oracle, except that the
    cached keys have standard deviation 3 (so that a few of the 137,216 keys
    dominate each row, rather than a near-uniform softmax averaging V to
    almost zero); 16 token rows (the first and last, page edges, the middle
    and random ones) against the oracle's selected-rows form with the
    reference test's tolerance (output 3e-4) and relative L2 1e-3, every
    appended K row within 2e-3 and V row exact, and the prefix unchanged bit
    for bit."""
    torch = gpu
    rng = np.random.default_rng(batch + position)
    kc = (rng.standard_normal((position, 4, 256), dtype=np.float32) * 3).astype(np.float16)
    vc = (rng.standard_normal((position, 4, 256), dtype=np.float32) * .5).astype(np.float16)
    q_gate = rng.standard_normal((batch, 24, 512), dtype=np.float32)
    key = rng.standard_normal((batch, 4, 256), dtype=np.float32)
    value = rng.standard_normal((batch, 4, 256), dtype=np.float32)
    q_norm = (1 + .25 * rng.uniform(-1, 1, 256)).astype(np.float32)
    k_norm = (1 + .25 * rng.uniform(-1, 1, 256)).astype(np.float32)
    eps = 1e-6
    rows = sorted({0, 1, 31, 32, batch // 2, batch - 2, batch - 1, *rng.choice(batch, 9, replace=False).tolist()})
    print(f'fused limits: batch={batch} position={position} rows={rows}', flush=True)
    want, k_all, v_all = ref.fused_attention_rows(kc, vc, q_gate, key, value, q_norm, k_norm, batch, position,
                                                  eps, rows)
    cache = A.PagedKV(4, 256, A.round_capacity(position + batch), torch.float16)
    cache.k.fill_(float('nan'))
    cache.v.fill_(float('nan'))
    if position:
        cache.pack(torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda())
    dev = [torch.from_numpy(x).cuda() for x in (q_gate, key, value, q_norm, k_norm)]
    out = A.attention_fused(*dev, cache, position, eps)
    new_k, new_v = cache.unpack(position, batch)
    torch.cuda.synchronize()
    got = out.cpu().numpy()[rows].astype(np.float64)
    assert_close(got, want, 3e-4)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) <= 1e-3
    assert_close(new_k.float().cpu().numpy(), k_all[position:], 2e-3)
    assert_close(new_v.float().cpu().numpy(), v_all[position:], 0)
    if position:
        old_k, old_v = cache.unpack(0, position)
        np.testing.assert_array_equal(old_k.cpu().numpy().view(np.uint16), kc.view(np.uint16))
        np.testing.assert_array_equal(old_v.cpu().numpy().view(np.uint16), vc.view(np.uint16))


@pytest.mark.parametrize('position', [200, 3000])
def test_fused_prefill_chunk_equals_eight_token_steps(gpu, position):
    """One 64-token chunk (prefill kernel; after 3,000 tokens with its keys
    split) against the same tokens in eight 8-token calls (split kernels),
    as the reference's grouped-vs-sequential check (tests/test_cuda.py:
    222-235): outputs within 3e-5, caches bitwise."""
    torch = gpu
    batch = 64
    c = kat.sine_wave_case(batch=batch, position=position)
    caches = []
    for _ in range(2):
        cache = A.PagedKV(4, 256, A.round_capacity(position + batch), torch.float16)
        cache.pack(torch.from_numpy(c['key_cache']).cuda(), torch.from_numpy(c['value_cache']).cuda())
        caches.append(cache)
    dev = [torch.from_numpy(f32(c[name])).cuda() for name in ('q_gate', 'key', 'value', 'q_norm', 'k_norm')]
    whole = A.attention_fused(*dev, caches[0], position, c['epsilon'])
    steps = torch.cat([A.attention_fused(dev[0][t:t + 8], dev[1][t:t + 8], dev[2][t:t + 8], dev[3], dev[4],
                                         caches[1], position + t, c['epsilon']) for t in range(0, batch, 8)])
    torch.cuda.synchronize()
    assert_close(whole.cpu().numpy(), steps.cpu().numpy(), 3e-5)
    for a, b in zip(caches[0].unpack(0, position + batch), caches[1].unpack(0, position + batch)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize('q_heads,kv_heads,head_dim,T,position,dtype', [
    (24, 4, 256, 1, 0, 'f16'), (24, 4, 256, 1, 255, 'bf16'),       # stream kernel, 1 and 8 pages
    (24, 4, 256, 8, 16, 'f16'), (24, 4, 256, 8, 248, 'bf16'),      # ring kernel, 1 and 8 pages
    (16, 2, 128, 3, 100, 'f16'), (8, 8, 128, 1, 200, 'bf16'),
])
def test_short_context_direct_output_equals_combined(gpu, q_heads, kv_heads, head_dim, T, position, dtype):
    """Up to 8 pages per KV head, qv_attention runs one split per KV head
    that writes the rows itself; the two-phase entry points store partials
    and combine them.  Both against the oracle, and against each other."""
    torch = gpu
    w = Workload('short', q_heads, kv_heads, head_dim, T, position, 1 / head_dim ** .5, dtype, 40 + T, 1.0, 0.5)
    q, k, v, _ = make_inputs(w)
    want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), position, w.scale)
    cache = make_cache(k, v, w, torch, fill_nan=True)
    qt = to_torch(q, dtype, torch)
    ws = A.workspace(A.attention_workspace_bytes(q_heads, kv_heads, head_dim, T, position))
    direct = A.attention(qt, cache, position, w.scale, ws=ws, out_dtype=torch.float32)
    combined = torch.empty_like(direct)
    A.attention_split(qt, cache, position, w.scale, ws)
    A.attention_combine(combined, cache, position, ws)
    torch.cuda.synchronize()
    direct, combined = direct.cpu().numpy().astype(np.float64), combined.cpu().numpy().astype(np.float64)
    assert_parity(direct, want)
    assert_parity(combined, want)
    # The fp16 ring kernel's partial rows are fp16 O / l (2^-11 relative);
    # every other pair differs by fp32 reassociation only.
    half_parts = dtype == 'f16' and T * (q_heads // kv_heads) > 16
    tolerance = 2.0 ** -10 * np.abs(want).max() if half_parts else 1e-5
    assert np.abs(direct - combined).max() <= tolerance


@pytest.mark.parametrize('T,position,dtype', [(1, 50000, 'f16'), (8, 2000, 'f16'), (8, 100, 'f16'),
                                              (16, 16000, 'f16'),    # prefill, keys split + combine
                                              (64, 9000, 'bf16')])   # V conversion, split prefill, combine
def test_graph_replay_matches_eager(gpu, T, position, dtype):
    """The device entry points enqueue kernels only (no allocation, no
    synchronisation, no memset), so they can be captured in a HIP graph; every
    replay, with eager work and synchronisations in between, reproduces the
    eager result bit for bit."""
    torch = gpu
    w = Workload('graph', 24, 4, 256, T, position, 1 / 16, dtype, 21, 1.0, 0.5)
    q, k, v, _ = make_inputs(w)
    cache = make_cache(k, v, w, torch)
    qt = to_torch(q, dtype, torch)
    ws = A.workspace(A.attention_workspace_bytes(24, 4, 256, T, position))
    eager = A.attention(qt, cache, position, w.scale, ws=ws).clone()
    out = torch.empty_like(qt)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        A.attention(qt, cache, position, w.scale, out=out, ws=ws)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            A.attention(qt, cache, position, w.scale, out=out, ws=ws)
    torch.cuda.current_stream().wait_stream(side)
    for _ in range(3):
        out.zero_()
        A.attention(qt[:1], cache, position, w.scale, ws=ws)   # eager work reusing the workspace
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize('q_heads,kv_heads,head_dim,T,position,dtype', [
    (24, 4, 256, 9, 0, 'f16'),      # 54 rows: just past the split-K path
    (24, 4, 256, 100, 37, 'bf16'),
    (24, 4, 256, 300, 1000, 'f16'),
    (8, 2, 128, 13, 5, 'bf16'),     # 52 rows, head_dim 128
    (8, 2, 128, 200, 64, 'f16'),
])
def test_prefill_kernel_all_rows(gpu, q_heads, kv_heads, head_dim, T, position, dtype):
    """Long token runs go through the prefill kernel; every row against the
    oracle, pages past the last key filled with NaN.  The float32 output
    (the reference's output type) is held to both bounds; the 16-bit output
    must equal that value up to its own rounding (half an ulp)."""
    w = Workload('prefill', q_heads, kv_heads, head_dim, T, position, 1 / head_dim ** .5, dtype, 300 + T, 1.0, 1.0)
    q, k, v, _ = make_inputs(w)
    want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), position, w.scale)
    got32 = gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32)
    assert_parity(got32, want)
    got16 = gpu_attention(w, q, k, v, gpu, fill_nan=True)
    half_ulp = np.abs(want) * (2.0 ** -8 if dtype == 'bf16' else 2.0 ** -11)
    assert np.all(np.abs(got16 - want) <= MAX_ABS + half_ulp)


@pytest.mark.parametrize('dtype', ['f16', 'bf16'])
def test_split_path_float32_output(gpu, dtype):
    """Verify-shaped call (8 tokens, split-K + combine) with float32 output,
    both input types, against the oracle to the full bounds."""
    w = Workload('verify', 24, 4, 256, 8, 3000, 1 / 16, dtype, 77, 1.0, 0.5)
    q, k, v, _ = make_inputs(w)
    want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), w.position, w.scale)
    assert_parity(gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32), want)


@pytest.mark.parametrize('q_heads,kv_heads,head_dim,T,position,dtype', [
    (24, 4, 256, 8, 0, 'f16'),       # one page, one split
    (24, 4, 256, 3, 40, 'bf16'),     # 18 rows, two pages
    (24, 4, 256, 8, 70, 'f16'),      # three pages
    (24, 4, 256, 8, 16384, 'bf16'),  # the verify shape in bf16
    (16, 4, 128, 8, 1000, 'f16'),    # head_dim 128, 32 rows
    (16, 2, 128, 6, 777, 'bf16'),    # head_dim 128, 48 rows
    (24, 1, 256, 1, 5000, 'f16'),    # 24 rows of one token
])
def test_multi_tile_split_kernel(gpu, q_heads, kv_heads, head_dim, T, position, dtype):
    """17..48 query rows per KV head (several 16-row tiles) go through the
    paged split kernel and the combine; pages past the last key hold NaN."""
    w = Workload('tiles', q_heads, kv_heads, head_dim, T, position, 1 / head_dim ** .5, dtype, 500 + T, 1.0, 0.5)
    q, k, v, _ = make_inputs(w)
    want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), position, w.scale)
    assert_parity(gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32), want)


def test_one_workspace_across_shapes_and_phases(gpu):
    """One workspace serves calls of different shapes in a row (different
    split counts, KV-head counts and head dims), repeatedly; the two-phase
    entry points (split, then combine) give exactly qv_attention's result."""
    cases = [Workload('a', 24, 4, 256, 1, 9000, 1 / 16, 'f16', 11, 1.0, 0.5),
             Workload('b', 24, 4, 256, 8, 3000, 1 / 16, 'f16', 12, 1.0, 0.5),
             Workload('c', 16, 2, 128, 3, 700, 1 / 128 ** .5, 'bf16', 13, 1.0, 0.5)]
    ws = A.workspace(max(A.attention_workspace_bytes(w.q_heads, w.kv_heads, w.head_dim, w.tokens, w.position)
                         for w in cases))
    prepared = []
    for w in cases:
        q, k, v, _ = make_inputs(w)
        want = ref.gqa_attention(to_float(q, w.dtype), to_float(k, w.dtype), to_float(v, w.dtype), w.position, w.scale)
        prepared.append((w, to_torch(q, w.dtype, gpu), make_cache(k, v, w, gpu, fill_nan=True), want))
    for _ in range(3):
        for w, qt, cache, want in prepared:
            out = A.attention(qt, cache, w.position, w.scale, ws=ws, out_dtype=gpu.float32)
            gpu.cuda.synchronize()
            assert_parity(out.cpu().numpy().astype(np.float64), want)
    for w, qt, cache, want in prepared[:2]:
        out = gpu.empty((w.tokens, w.q_heads, w.head_dim), dtype=gpu.float16, device='cuda')
        A.attention_split(qt, cache, w.position, w.scale, ws)
        A.attention_combine(out, cache, w.position, ws)
        fused = A.attention(qt, cache, w.position, w.scale, ws=ws)
        gpu.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), fused.cpu().numpy())


# ---- KV-cache manager (checkpoint / restore / commit) ----------------------

@pytest.mark.parametrize('head_dim,kv_heads,tokens', [(256, 4, 1000), (128, 2, 1000),
                                                     (128, 2, 970),    # 31 pages: the half-size blocks
                                                     (256, 4, 970)])
def test_kv_copy_prefix_bitwise(gpu, head_dim, kv_heads, tokens):
    """qv_kv_copy moves the pages of a prefix between caches of different
    capacities, every value bit for bit; a snapshot of 1000 tokens needs 1024
    (970 tokens: 992)."""
    from redshift_amd.kvcache import copy_prefix
    rng = np.random.default_rng(7)
    rows = gpu.from_numpy(rng.standard_normal((3000, kv_heads, head_dim)).astype(np.float16)).cuda()
    big = A.PagedKV(kv_heads, head_dim, 4096, gpu.float16).pack(rows, -rows)
    snap = A.PagedKV(kv_heads, head_dim, A.round_capacity(tokens), gpu.float16)
    copy_prefix(snap, big, tokens)
    other = A.PagedKV(kv_heads, head_dim, 2048, gpu.float16)
    other.k.fill_(float('nan'))
    other.v.fill_(float('nan'))
    copy_prefix(other, snap, tokens)
    for cache in (snap, other):
        k, v = cache.unpack(0, tokens)
        np.testing.assert_array_equal(k.cpu().numpy().view(np.uint16), rows[:tokens].cpu().numpy().view(np.uint16))
        np.testing.assert_array_equal(v.cpu().numpy().view(np.uint16), (-rows[:tokens]).cpu().numpy().view(np.uint16))


def random_shapes(n, seed=2024):
    """Seeded shapes across both kernels' ranges: KV heads 1-8, groups 1-8,
    head_dim 128/256, fp16/bf16, 1-24 tokens (split-K up to 48 rows per KV
    head, the prefill kernel beyond), positions 0-3000, with and without
    outlier keys."""
    rng = np.random.default_rng(seed)
    shapes = []
    for i in range(n):
        kv = int(rng.choice([1, 2, 4, 8]))
        group = int(rng.integers(1, 9))
        tokens = int(rng.choice([1, 2, 3, 5, 8, 9, 13, 24]))
        shapes.append((kv * group, kv, int(rng.choice([128, 256])), tokens, int(rng.integers(0, 3001)),
                       str(rng.choice(['f16', 'bf16'])), int(rng.choice([0, 16])), 900 + i))
    return shapes


@pytest.mark.parametrize('q_heads,kv_heads,head_dim,T,position,dtype,outliers,seed', random_shapes(24))
def test_random_shapes_against_oracle(gpu, q_heads, kv_heads, head_dim, T, position, dtype, outliers, seed):
    """qv_attention with float32 output on seeded random shapes, pages past
    the last key filled with NaN, against the oracle to the full bounds."""
    outliers = min(outliers, position + T)
    w = Workload('random', q_heads, kv_heads, head_dim, T, position, 1 / head_dim ** .5, dtype, seed, 1.0, 0.5,
                 outliers, 8.0)
    q, k, v, _ = make_inputs(w)
    want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), position, w.scale)
    assert_parity(gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32), want)


@pytest.mark.parametrize('q_heads,kv_heads,head_dim,T,position,dtype', [
    (48, 1, 128, 1, 1000, 'f16'),     # 48 rows, the group limit: the ring kernel's three tiles
    (16, 1, 256, 3, 500, 'bf16'),     # 48 rows from three tokens
    (24, 1, 256, 1, 3000, 'f16'),     # 24 rows: two tiles, one token
    (12, 1, 128, 4, 100, 'bf16'),     # a direct (one-split) plan
    (32, 1, 128, 2, 2000, 'f16'),     # 64 rows: the prefill kernel, a group spanning its tiles
    (48, 2, 256, 5, 300, 'f16'),      # 240 rows per KV head
    (96, 2, 256, 1, 6000, 'bf16'),    # 48 rows per KV head, two KV heads
])
def test_large_groups_against_oracle(gpu, q_heads, kv_heads, head_dim, T, position, dtype):
    """Query groups of 12-48 heads per KV head (up to the documented limit of
    48), on both sides of the 48-row split between the split-K kernels and the
    prefill kernel, float32 output, pages past the last key filled with NaN,
    against the oracle to the full bounds."""
    w = Workload('groups', q_heads, kv_heads, head_dim, T, position, 1 / head_dim ** .5, dtype, 31, 1.0, 0.5)
    q, k, v, _ = make_inputs(w)
    want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), position, w.scale)
    assert_parity(gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32), want)


def random_fused_shapes(n, seed=77):
    """Seeded (batch, position) pairs over every route of the fused entry:
    one launch on short contexts, decode, verification batches, prefill
    chunks whole or with their keys split (longer batches on shorter
    prefixes, to keep the oracle quick)."""
    rng = np.random.default_rng(seed)
    shapes = []
    for i in range(n):
        batch = int(rng.choice([1, 2, 3, 5, 8, 9, 16, 33, 64, 100]))
        limit = 20000 if batch <= 64 else 4000
        position = int(rng.choice([int(rng.integers(0, 256)), int(rng.integers(256, limit + 1))]))
        shapes.append((batch, min(position, 139264 - batch), 3000 + i))
    return shapes


@pytest.mark.parametrize('batch,position,seed', random_fused_shapes(14))
def test_fused_random_shapes_against_oracle(gpu, batch, position, seed):
    """qv_attention_fused on seeded random inputs (fp16 prefix caches of
    N(0,1)/2 values, q_gate, key and value N(0,1), norms 1 +- 1/4) against the
    oracle's fused attention, with the reference test's tolerances: output
    3e-4, appended K 2e-3, V exact; the prefix unchanged."""
    torch = gpu
    rng = np.random.default_rng(seed)
    kc = (rng.standard_normal((position, 4, 256)) * .5).astype(np.float16)
    vc = (rng.standard_normal((position, 4, 256)) * .5).astype(np.float16)
    q_gate = rng.standard_normal((batch, 24, 512)).astype(np.float32)
    key = rng.standard_normal((batch, 4, 256)).astype(np.float32)
    value = rng.standard_normal((batch, 4, 256)).astype(np.float32)
    q_norm = (1 + .25 * rng.uniform(-1, 1, 256)).astype(np.float32)
    k_norm = (1 + .25 * rng.uniform(-1, 1, 256)).astype(np.float32)
    eps = 1e-6
    print(f'fused random: batch={batch} position={position} seed={seed}', flush=True)
    expected = ref.fused_attention(kc, vc, q_gate, key, value, q_norm, k_norm, batch, position, eps)
    cache = A.PagedKV(4, 256, A.round_capacity(position + batch), torch.float16)
    cache.k.fill_(float('nan'))
    cache.v.fill_(float('nan'))
    if position:
        cache.pack(torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda())
    dev = [torch.from_numpy(x).cuda() for x in (q_gate, key, value, q_norm, k_norm)]
    out = A.attention_fused(*dev, cache, position, eps)
    kcache, vcache = cache.unpack(0, position + batch)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), expected[0], 3e-4)
    assert_close(kcache.float().cpu().numpy(), expected[1], 2e-3)
    assert_close(vcache.float().cpu().numpy(), expected[2], 0)


@pytest.mark.parametrize('batch,position', [(1, 16000), (2, 3000), (5, 300), (8, 16000), (1400, 100), (64, 16000),
                                            (40, 0), (16, 16000)])
def test_fused_graph_replay_matches_eager(gpu, batch, position):
    """The fused entry (prepare in the split kernels' prologue, the new keys
    appended by the kernels; for a prefill chunk the prepare launch, the
    precise prefill in two passes (1400 tokens) or with its keys split (64
    tokens at 16,000) and the gated combine) enqueues kernels only, so it
    can be captured in a HIP graph: every replay, with eager calls reusing
    the workspace and synchronisations in between, reproduces the eager
    output and caches bit for bit."""
    torch = gpu
    rng = np.random.default_rng(position + batch)
    kc = (rng.standard_normal((position, 4, 256)) * .5).astype(np.float16)
    vc = (rng.standard_normal((position, 4, 256)) * .5).astype(np.float16)
    cache = A.PagedKV(4, 256, A.round_capacity(position + batch), torch.float16)
    cache.k.fill_(float('nan'))
    cache.v.fill_(float('nan'))
    if position:
        cache.pack(torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda())
    dev = [torch.from_numpy(x).cuda() for x in (
        rng.standard_normal((batch, 24, 512)).astype(np.float32),
        rng.standard_normal((batch, 4, 256)).astype(np.float32),
        rng.standard_normal((batch, 4, 256)).astype(np.float32),
        (1 + .25 * rng.uniform(-1, 1, 256)).astype(np.float32),
        (1 + .25 * rng.uniform(-1, 1, 256)).astype(np.float32))]
    ws = A.workspace(A.fused_workspace_bytes(batch, position))
    eager = A.attention_fused(*dev, cache, position, 1e-6, ws=ws).clone()
    k0, v0 = cache.k.clone(), cache.v.clone()
    out = torch.empty_like(eager)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        A.attention_fused(*dev, cache, position, 1e-6, out=out, ws=ws)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            A.attention_fused(*dev, cache, position, 1e-6, out=out, ws=ws)
    torch.cuda.current_stream().wait_stream(side)
    for _ in range(3):
        out.zero_()
        A.attention_fused(*dev, cache, position, 1e-6, ws=ws)   # eager work reusing the workspace
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(cache.k.view(torch.int16), k0.view(torch.int16))   # bits: unused slots hold NaN
        assert torch.equal(cache.v.view(torch.int16), v0.view(torch.int16))


def test_fused_front_end_realigns_input_views(gpu):
    """The device ABI takes 16-byte aligned buffers; the torch front end
    passes an input view that starts elsewhere (here the norm weights and the
    key at a 4-byte offset into their storage) as an aligned copy, with the
    same result bit for bit."""
    torch = gpu
    rng = np.random.default_rng(5)
    batch, position = 8, 3000
    kc = torch.from_numpy((rng.standard_normal((position, 4, 256)) * .5).astype(np.float16)).cuda()
    vc = torch.from_numpy((rng.standard_normal((position, 4, 256)) * .5).astype(np.float16)).cuda()
    q_gate = torch.from_numpy(rng.standard_normal((batch, 24, 512)).astype(np.float32)).cuda()
    key = torch.from_numpy(rng.standard_normal((batch, 4, 256)).astype(np.float32)).cuda()
    value = torch.from_numpy(rng.standard_normal((batch, 4, 256)).astype(np.float32)).cuda()
    norms = torch.from_numpy((1 + .25 * rng.uniform(-1, 1, 512)).astype(np.float32)).cuda()
    q_norm, k_norm = norms[:256].clone(), norms[256:].clone()
    outs = []
    for offset in (False, True):
        cache = A.PagedKV(4, 256, A.round_capacity(position + batch), torch.float16)
        cache.pack(kc, vc)
        args = [q_gate, key, value, q_norm, k_norm]
        if offset:
            views = []
            for t in (key, q_norm, k_norm):
                buf = torch.empty(t.numel() + 1, dtype=torch.float32, device=t.device)
                v = buf[1:].view(t.shape)
                v.copy_(t)
                assert v.data_ptr() % 16 != 0
                views.append(v)
            args = [q_gate, views[0], value, views[1], views[2]]
        outs.append((A.attention_fused(*args, cache, position, 1e-6).clone(), cache.k.clone()))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1].view(torch.int16), outs[1][1].view(torch.int16))
