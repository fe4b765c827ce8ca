"""The workload shapes at full size and at their stated precision, the
precise (fp32-query) entry, and scores under any finite scale.

Every check holds the float32 output to max-abs 2e-3 and relative-L2 1e-3
against the float64 oracle (oracle/attention_ref.py, the restatement of the
reference's tests/cpu_reference.py:55-89) on the same seeded inputs.
"""
import numpy as np
import pytest

from oracle import attention_ref as ref
from redshift_amd import attention as A
from redshift_amd.workloads import WORKLOADS, Workload, f32_to_bf16_bits, make_inputs, to_float
from tests.test_attention_gpu import MAX_ABS, assert_parity, gpu_attention, make_cache

pytestmark = pytest.mark.gpu

# The fp32 query travels as fp16 hi + lo parts (about 22 significant bits)
# and P as hi + lo parts: far inside the parity bounds.
PRECISE_REL_L2 = 5e-5


def rel_l2(got, want):
    return float(np.linalg.norm(got - want) / np.linalg.norm(want))


def precise_attention(w, q32, k16, v16, torch, fill_nan=True):
    """qv_attention_precise of an fp32 query on an fp16 cache."""
    wf16 = Workload(**{**w.__dict__, 'dtype': 'f16'})
    cache = make_cache(k16, v16, wf16, torch, fill_nan=fill_nan)
    out = A.attention_precise(torch.from_numpy(np.ascontiguousarray(q32, np.float32)).cuda(), cache,
                              w.position, w.scale)
    torch.cuda.synchronize()
    return out.cpu().numpy().astype(np.float64)


def test_cpu_plumbing_at_its_stated_precision(gpu):
    """8/2/128, one query on 128 keys, fp32 Q/K/V from N(0,1) with seed 0,
    scale 1/sqrt(128): the fp32 query through qv_attention_precise; K and V
    are the fp16 cache entries (the reference's caches are fp16 and its CPU
    oracle rounds them with half(), tests/cpu_reference.py:57,75-76).  The
    oracle runs on exactly the fp32 query and those fp16 keys and values."""
    w = WORKLOADS['cpu_plumbing']
    q, k, v, _ = make_inputs(w)
    assert q.dtype == np.float32
    k16, v16 = k.astype(np.float16), v.astype(np.float16)
    got = precise_attention(w, q, k16, v16, gpu)
    want = ref.gqa_attention(q, k16, v16, w.position, w.scale)
    assert_parity(got, want)
    assert rel_l2(got, want) <= PRECISE_REL_L2
    # The same keys with the query rounded to fp16 (the raw 16-bit entry)
    # carry the query's own rounding: the precise entry is the closer one.
    q16 = q.astype(np.float16)
    got16 = gpu_attention(Workload(**{**w.__dict__, 'dtype': 'f16'}), q16, k16, v16, gpu, out_dtype=gpu.float32)
    assert rel_l2(got, want) < rel_l2(got16, want)


@pytest.mark.parametrize('kv_dtype', ['bf16', 'f16'])
def test_prefill_chunk_full_size_float32_output(gpu, kv_dtype):
    """2048 query tokens appended to a 6144-token cache (8192 keys), causal,
    24/4/256, inputs N(0,1) from seed 2, float32 output: every element of
    all 2048 token rows x 24 heads to both bounds (bf16 caches as stated,
    and fp16 caches of the same shape), as the reference's own test compares
    every output element (tests/test_cuda.py:218).  The 16-bit output of the
    same call must equal that float32 value up to its own rounding (half an
    ulp) on every element."""
    w = Workload(**{**WORKLOADS['prefill_2k'].__dict__, 'dtype': kv_dtype})
    q, k, v, _ = make_inputs(w)
    print(f'prefill 2048 at 6144, {kv_dtype}', flush=True)
    got32 = gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32)
    got16 = gpu_attention(w, q, k, v, gpu, fill_nan=True)
    want = ref.gqa_attention(to_float(q, kv_dtype), to_float(k, kv_dtype), to_float(v, kv_dtype),
                             w.position, w.scale)
    assert want.shape == got32.shape == (2048, 24, 256)
    assert_parity(got32, want)
    half_ulp = np.abs(want) * (2.0 ** -8 if kv_dtype == 'bf16' else 2.0 ** -11)
    assert np.all(np.abs(got16 - want) <= MAX_ABS + half_ulp)
    if kv_dtype == 'bf16':
        want16 = to_float(f32_to_bf16_bits(want.astype(np.float32)), 'bf16')
        assert rel_l2(got16, want16) <= 1e-3


def test_prefill_chunk_full_size_precise(gpu):
    """The same chunk with an fp32 query on fp16 caches through the precise
    entry (the reference's precision: fp32 q, fp16 cache), every element."""
    w = WORKLOADS['prefill_2k']
    rng = np.random.default_rng(w.seed)
    q = rng.standard_normal((w.tokens, w.q_heads, w.head_dim), dtype=np.float32)
    k = rng.standard_normal((w.keys, w.kv_heads, w.head_dim), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((w.keys, w.kv_heads, w.head_dim), dtype=np.float32).astype(np.float16)
    got = precise_attention(w, q, k, v, gpu)
    want = ref.gqa_attention(q, k, v, w.position, w.scale)
    assert want.shape == got.shape == (2048, 24, 256)
    assert_parity(got, want)
    assert rel_l2(got, want) <= PRECISE_REL_L2


@pytest.mark.parametrize('q_heads,kv_heads,head_dim,T,position', [
    (24, 4, 256, 1, 5000),      # decode: stream kernel
    (24, 4, 256, 2, 31),
    (16, 2, 128, 1, 5000),      # stream kernel at head_dim 128, split + combine (fp32 query split in-kernel)
    (8, 2, 128, 2, 3000),       # the same, two tokens of 4 query heads per KV head
    (24, 4, 256, 8, 16384),     # verify-8 at 16K: ring kernel
    (8, 2, 128, 8, 300),        # 32 rows, head_dim 128
    (16, 2, 128, 6, 777),       # 48 rows, head_dim 128
    (24, 1, 256, 1, 20000),     # one KV head, many splits
    (24, 4, 256, 100, 37),      # prefill kernel
    (8, 2, 128, 200, 64),       # prefill kernel, head_dim 128
    (24, 4, 256, 64, 16000),    # prefill kernel, keys split over 21 workgroups per row workgroup
    (24, 4, 256, 200, 3000),    # prefill kernel, 6 key splits
    (16, 2, 128, 40, 9000),     # prefill kernel at head_dim 128, 35 key splits
    (24, 4, 256, 1400, 100),    # two passes of 192 rows (on 256 CUs; three padding tiles)
])
def test_precise_entry_against_oracle(gpu, q_heads, kv_heads, head_dim, T, position):
    """qv_attention_precise across its kernels (fp32 query, fp16 pages,
    pages past the last key filled with NaN)."""
    w = Workload('precise', q_heads, kv_heads, head_dim, T, position, 1 / head_dim ** .5, 'f32', 700 + T,
                 1.0, 0.5, min(16, position + T), 8.0)
    q, k, v, _ = make_inputs(w)
    k16, v16 = k.astype(np.float16), v.astype(np.float16)
    got = precise_attention(w, q, k16, v16, gpu)
    want = ref.gqa_attention(q, k16, v16, position, w.scale)
    assert_parity(got, want)
    assert rel_l2(got, want) <= PRECISE_REL_L2


@pytest.mark.parametrize('T,dtype', [(1, 'bf16'), (8, 'bf16'), (1, 'f32'), (4, 'f32')])
def test_full_context_other_precisions(gpu, T, dtype):
    """The 139,264-token capacity filled to its last slot on the routes the
    fp16 workloads leave out: bf16 pages (P as hi + lo parts) and the fp32
    query of qv_attention_precise, for decode (the stream kernel, 48 splits
    per head) and verification (the ring kernel), 64 outlier keys."""
    position = 139264 - T
    w = Workload('full', 24, 4, 256, T, position, 1 / 16, dtype, 900 + T, 0.5, 0.5, 64, 8.0)
    q, k, v, _ = make_inputs(w)
    if dtype == 'f32':
        k16, v16 = k.astype(np.float16), v.astype(np.float16)
        got = precise_attention(w, q, k16, v16, gpu)
        want = ref.gqa_attention(q, k16, v16, position, w.scale)
        assert rel_l2(got, want) <= PRECISE_REL_L2
    else:
        got = gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32)
        want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), position, w.scale)
    assert_parity(got, want)


@pytest.mark.parametrize('T,position', [(2048, 139264 - 2048), (8192, 0)])
@pytest.mark.parametrize('dtype', ['f16', 'bf16'])
def test_prefill_chunk_fills_the_capacity(gpu, dtype, T, position):
    """A 2048-token raw chunk whose last key is the 139,264-token capacity's
    last slot (the prefill kernel; bf16 through the V conversion pass over
    all 4,352 pages), and 8,192 tokens on an empty cache (1,024 row
    workgroups: four rounds over 256 CUs), 64 outlier keys, slots past the
    last key NaN: 24 token rows (the first and last, page edges, the middle
    and random ones) against the oracle to both bounds, float32 output."""
    w = Workload('full_prefill', 24, 4, 256, T, position, 1 / 16, dtype, 950, 1.0, 0.5, 64, 8.0)
    q, k, v, _ = make_inputs(w)
    rng = np.random.default_rng(951)
    rows = sorted({0, 1, 31, 32, 1023, 1024, T - 2, T - 1, *rng.choice(T, 16, replace=False).tolist()})
    print(f'prefill limits: {dtype} T={T} position={position} rows={rows}', flush=True)
    got = gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32)[rows]
    want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), position, w.scale,
                             rows=rows)
    assert_parity(got, want)


@pytest.mark.parametrize('T,scale,dtype', [
    (100, 0.0, 'f16'), (100, -1 / 16, 'f16'), (100, -1 / 16, 'bf16'),   # prefill kernel
    (3, 0.0, 'f16'), (8, -0.2, 'bf16'),                                 # ring kernel
    (1, 0.0, 'bf16'), (1, -1 / 16, 'f16'),                              # stream kernel
])
def test_any_finite_scale(gpu, T, scale, dtype):
    """Scores are scaled before they are masked and their maximum taken, so
    a zero scale gives the mean of the visible values and a negative one
    the softmax of the negated scores; NaN in the pages past the last key
    never reaches the result."""
    w = Workload('scale', 24, 4, 256, T, 500, scale, dtype, 800 + T, 1.0, 0.5)
    q, k, v, _ = make_inputs(w)
    want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), w.position, scale)
    got = gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32)
    assert_parity(got, want)
    if scale == 0.0:
        vf = to_float(v, dtype)
        t = T - 1     # the last row sees keys 0..position+T-1: their plain mean
        mean = vf[:w.position + T].mean(axis=0)                    # [kv_heads, D]
        np.testing.assert_allclose(got[t], np.repeat(mean, w.group, axis=0), atol=2e-3)
