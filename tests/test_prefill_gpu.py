"""GPU parity of the chunked prefill on bf16 caches, whose V pages a
streaming pass converts to fp16 in the workspace (exact for bf16 values in
[2^-14, 65280]) before the prefill kernel multiplies them by an fp16 P.

The pass flags a KV head with a V value outside that range, and the exact
instance (bf16 V, P as bf16 hi + lo parts) computes that head's rows
instead.  These tests put such values in the cache (far above the fp16
range, a whole KV head below it, one dead head dimension) and hold the
fp32 output to the oracle's bounds, and check on ordinary data that the
pass flags nothing (the converted products are the ones that ran).
"""
import numpy as np
import pytest

from oracle import attention_ref as ref
from redshift_amd import attention as A
from redshift_amd.workloads import Workload, f32_to_bf16_bits, make_inputs, to_float

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2 = 2e-3, 1e-3


def bf16_bits(x):
    return f32_to_bf16_bits(np.ascontiguousarray(x, np.float32))


def run(w, q, k, v, torch, ws=None):
    """fp32 output of qv_attention on a bf16 cache whose slots past the last
    key hold NaN; q, k, v are bf16 bits."""
    def t(x):
        return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(torch.bfloat16).cuda()
    cache = A.PagedKV(w.kv_heads, w.head_dim, A.round_capacity(w.keys), torch.bfloat16)
    cache.k.fill_(float('nan'))
    cache.v.fill_(float('nan'))
    cache.pack(t(k), t(v))
    if ws is None:
        ws = A.workspace(A.attention_workspace_bytes(w.q_heads, w.kv_heads, w.head_dim, w.tokens, w.position))
    out = A.attention(t(q), cache, w.position, w.scale, ws=ws, out_dtype=torch.float32)
    torch.cuda.synchronize()
    return out.cpu().numpy().astype(np.float64)


def check(got, want, scale=1.0):
    """Both bounds, relative to the output's own magnitude `scale`."""
    assert np.all(np.isfinite(got))
    err = np.abs(got - want).max()
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert err <= MAX_ABS * scale and rel <= REL_L2, (err, rel)


def inputs(T, position, q_heads=24, kv_heads=4, head_dim=256, seed=0):
    w = Workload('prefill_bf16', q_heads, kv_heads, head_dim, T, position, 1 / 16, 'bf16', seed, 1.0, 1.0)
    q, k, v, _ = make_inputs(w)
    return w, to_float(q, 'bf16'), to_float(k, 'bf16'), to_float(v, 'bf16')


def test_ordinary_values_take_the_converted_products(gpu):
    """N(0,1) bf16 values all lie in the fp16 range: every word of the
    conversion pass stays 0 (no head takes the exact instance), and the
    result meets both bounds."""
    w, q, k, v = inputs(600, 900, seed=11)
    ws = A.workspace(A.attention_workspace_bytes(w.q_heads, w.kv_heads, w.head_dim, w.tokens, w.position))
    ws.fill_(0xAB)
    got = run(w, bf16_bits(q), bf16_bits(k), bf16_bits(v), gpu, ws=ws)
    check(got, ref.gqa_attention(q, k, v, w.position, w.scale))
    # The workspace holds the fp16 copy of the V pages, then (256-byte
    # aligned) one word per page, per KV head.
    pages = -(-w.keys // 32)
    offset = -(-(w.kv_heads * pages * 32 * w.head_dim * 2) // 256) * 256
    blocks = w.kv_heads * pages
    words = ws[offset:offset + 4 * blocks].cpu().numpy().view(np.uint32)
    assert np.all(words == 0), words


@pytest.mark.parametrize('case', ['huge_page', 'tiny_head', 'dead_dim', 'huge_page_d128', 'huge_page_split21'])
def test_values_outside_the_fp16_range(gpu, case):
    """V values the fp16 conversion cannot hold: the KV heads that have
    them take the exact bf16 products.  (400 tokens at 700 split their keys
    in 4 runs; huge_page_split21, 70 tokens at 9,000, in 21, whose partial
    rows the combine requests in one round: flagged heads' rows as fp32
    halves in two planes, the others as fp16.)"""
    if case == 'huge_page_d128':
        w, q, k, v = inputs(300, 500, q_heads=16, kv_heads=2, head_dim=128, seed=12)
    elif case == 'huge_page_split21':
        w, q, k, v = inputs(70, 9000, seed=14)
    else:
        w, q, k, v = inputs(400, 700, seed=13)
    scale = 1.0
    if case.startswith('huge_page'):
        # Keys 640..671 (one page) of KV head 1 far above 65504, and one
        # key of head 0 just above it.
        v[640:672, 1 % w.kv_heads] *= 2.0 ** 20
        v[100, 0, 7] = 70000.0
        scale = 2.0 ** 20
    elif case == 'tiny_head':
        # Every value of KV head 2 below 2^-14 (an fp16 subnormal would keep
        # a few bits of each); head 3 normal.
        v[:, 2] *= 2.0 ** -20
    else:
        # One head dimension of every key close to zero (2^-30 scale), the
        # others normal: every page has a lane below 2^-14.
        v[:, :, 37] *= 2.0 ** -30
    q16, k16, v16 = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    q, k, v = to_float(q16, 'bf16'), to_float(k16, 'bf16'), to_float(v16, 'bf16')
    want = ref.gqa_attention(q, k, v, w.position, w.scale)
    got = run(w, q16, k16, v16, gpu)
    check(got, want, scale)
    if case == 'tiny_head':
        # The tiny head's rows on their own scale, too.
        heads = slice(2 * w.q_heads // w.kv_heads, 3 * w.q_heads // w.kv_heads)
        check(got[:, heads], want[:, heads], 2.0 ** -20)


def random_prefill_shapes(n, seed=4096, max_rows=1400, max_position=4000, first_seed=1700):
    """Seeded prefill shapes: KV heads 1-8, groups 1-8, head_dim 128/256,
    fp16/bf16, more than 48 query rows per KV head (the prefill kernel),
    up to max_rows of them (several workgroups per KV head), positions up to
    max_position (tail pages of every fill; most calls split their keys),
    with and without outlier keys."""
    rng = np.random.default_rng(seed)
    shapes = []
    for i in range(n):
        kv = int(rng.choice([1, 2, 4, 8]))
        group = int(rng.integers(1, 9))
        tokens = int(rng.integers(49 // group + 1, max_rows // group + 1))
        shapes.append((kv * group, kv, int(rng.choice([128, 256])), tokens, int(rng.integers(0, max_position + 1)),
                       str(rng.choice(['f16', 'bf16'])), int(rng.choice([0, 16])), first_seed + i))
    return shapes


@pytest.mark.parametrize('q_heads,kv_heads,head_dim,T,position,dtype,outliers,seed',
                         random_prefill_shapes(12) + random_prefill_shapes(8, seed=9000, max_rows=400,
                                                                            max_position=20000, first_seed=2300))
def test_random_prefill_shapes(gpu, q_heads, kv_heads, head_dim, T, position, dtype, outliers, seed):
    """The prefill path on seeded random shapes, cache slots past the last
    key NaN: the float32 output to both bounds, the 16-bit output within
    the max-abs bound plus its own rounding (half an ulp)."""
    from tests.test_attention_gpu import gpu_attention
    outliers = min(outliers, position + T)
    w = Workload('random_prefill', q_heads, kv_heads, head_dim, T, position, 1 / head_dim ** .5, dtype, seed,
                 1.0, 0.5, outliers, 8.0)
    assert T * (q_heads // kv_heads) > 48
    q, k, v, _ = make_inputs(w)
    want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), position, w.scale)
    got32 = gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32)
    check(got32, want)
    got16 = gpu_attention(w, q, k, v, gpu, fill_nan=True)
    half_ulp = np.abs(want) * (2.0 ** -8 if dtype == 'bf16' else 2.0 ** -11)
    assert np.all(np.abs(got16 - want) <= MAX_ABS + half_ulp)


@pytest.mark.parametrize('q_heads,kv_heads,head_dim,T,position,dtype', [
    (24, 4, 256, 16, 16000, 'f16'),    # 4 row workgroups: 62 key splits of about 8 pages
    (24, 4, 256, 64, 16000, 'bf16'),   # 8 row workgroups: 32 splits, V through the fp16 copy
    (16, 2, 128, 40, 9000, 'bf16'),
    (1, 1, 128, 2400, 0, 'f16'),       # 9 splits; a workgroup's early rows see no key of its last run
    (8, 1, 256, 1100, 0, 'bf16'),      # 4 splits; the early workgroups' later runs are empty
    (24, 4, 256, 300, 300, 'f16'),     # 19 pages: not split
    (24, 4, 256, 96, 16000, 'f16'),    # 12 row workgroups: 21 splits, one combine round of 24
    (24, 4, 256, 70, 9000, 'bf16'),    # 12 row workgroups: 21 splits, V through the fp16 copy
    (24, 4, 256, 800, 2000, 'bf16'),   # 25 row workgroups: 2 splits (the combine's 4-split batch)
    (24, 4, 256, 600, 1000, 'f16'),    # 19 row workgroups: 3 splits
])
def test_split_prefill_against_oracle(gpu, q_heads, kv_heads, head_dim, T, position, dtype):
    """Calls with too few row workgroups to fill the device split their keys
    over more workgroups and combine the partial rows: every row against the
    oracle, cache slots past the last key NaN; the float32 output to both
    bounds, the 16-bit output within the max-abs bound plus half an ulp."""
    from tests.test_attention_gpu import gpu_attention
    w = Workload('split_prefill', q_heads, kv_heads, head_dim, T, position, 1 / head_dim ** .5, dtype, 40 + T,
                 1.0, 0.5, min(16, position + T), 8.0)
    q, k, v, _ = make_inputs(w)
    want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), position, w.scale)
    got32 = gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32)
    check(got32, want)
    got16 = gpu_attention(w, q, k, v, gpu, fill_nan=True)
    half_ulp = np.abs(want) * (2.0 ** -8 if dtype == 'bf16' else 2.0 ** -11)
    assert np.all(np.abs(got16 - want) <= MAX_ABS + half_ulp)



@pytest.mark.parametrize('scale,dtype', [(0.0, 'f16'), (-1 / 16, 'bf16')])
def test_split_prefill_any_scale(gpu, scale, dtype):
    """A split call (100 tokens after 2,000: 8 runs of pages per row
    workgroup) under a zero scale (the mean of the visible values) and a
    negative one, cache slots past the last key NaN, float32 output against
    the oracle to both bounds."""
    from tests.test_attention_gpu import gpu_attention
    w = Workload('split_scale', 24, 4, 256, 100, 2000, scale, dtype, 61, 1.0, 0.5)
    q, k, v, _ = make_inputs(w)
    want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), w.position, scale)
    check(gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32), want)
