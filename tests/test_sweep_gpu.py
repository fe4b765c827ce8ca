"""A seeded sweep over wider shape ranges than the other parity tests draw
from: raw calls (fp16 and bf16 pages, 1-8 KV heads, groups up to 12, 1-40
tokens, positions up to 40,000 on the split-K kernels), precise calls (fp32
query) and fused calls (batches of 1-200 tokens on the 24/4/256 model),
each against the oracle with the bounds of the test it extends:

* raw: test_attention_gpu.test_random_shapes_against_oracle (max-abs 2e-3,
  relative L2 1e-3, float32 output, slots past the last key NaN);
* precise: test_configs_gpu.test_precise_entry_against_oracle (the same,
  plus relative L2 5e-5);
* fused: test_attention_gpu.test_fused_random_shapes_against_oracle (the
  reference test's output 3e-4, appended K 2e-3, appended V exact).
"""
import numpy as np
import pytest

from oracle import attention_ref as ref
from redshift_amd import attention as A
from redshift_amd.workloads import Workload, make_inputs, to_float
from tests.test_attention_gpu import assert_close, assert_parity, gpu_attention
from tests.test_configs_gpu import PRECISE_REL_L2, precise_attention

pytestmark = pytest.mark.gpu


def raw_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        kv = int(rng.choice([1, 2, 4, 8]))
        group = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 12]))
        tokens = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 9, 13, 16, 24, 40]))
        head_dim = int(rng.choice([128, 256]))
        dtype = str(rng.choice(['f16', 'bf16']))
        position = int(rng.choice([rng.integers(0, 300), rng.integers(300, 6000), rng.integers(6000, 40000)]))
        if tokens * group > 48 and position > 6000:      # the prefill kernel: keep the oracle quick
            position = int(rng.integers(0, 6000))
        cases.append((kv, group, tokens, head_dim, dtype, position, int(rng.choice([0, 16])), seed + i))
    return cases


def precise_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        tokens = int(rng.choice([1, 2, 3, 8, 16, 40, 100]))
        cases.append((int(rng.choice([1, 2, 4])), int(rng.choice([1, 2, 4, 6, 8])), tokens,
                      int(rng.choice([128, 256])), int(rng.integers(1, 20000 if tokens <= 16 else 3000)), seed + i))
    return cases


def fused_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        batch = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16, 33, 64, 65, 100, 128, 200]))
        limit = 40000 if batch <= 8 else (16000 if batch <= 128 else 3000)
        position = int(rng.choice([rng.integers(0, 300), rng.integers(300, limit + 1)]))
        cases.append((batch, min(position, 139264 - batch), seed + i))
    return cases


@pytest.mark.parametrize('kv,group,tokens,head_dim,dtype,position,outliers,seed', raw_cases(80, 5000))
def test_raw_sweep(gpu, kv, group, tokens, head_dim, dtype, position, outliers, seed):
    w = Workload('sweep', kv * group, kv, head_dim, tokens, position, 1 / head_dim ** .5, dtype, seed, 1.0, 0.5,
                 min(outliers, position + tokens), 8.0)
    q, k, v, _ = make_inputs(w)
    want = ref.gqa_attention(to_float(q, dtype), to_float(k, dtype), to_float(v, dtype), position, w.scale)
    assert_parity(gpu_attention(w, q, k, v, gpu, fill_nan=True, out_dtype=gpu.float32), want)


@pytest.mark.parametrize('kv,group,tokens,head_dim,position,seed', precise_cases(40, 6000))
def test_precise_sweep(gpu, kv, group, tokens, head_dim, position, seed):
    w = Workload('sweep_precise', kv * group, kv, head_dim, tokens, position, 1 / head_dim ** .5, 'f32', seed,
                 1.0, 0.5, min(16, position + tokens), 8.0)
    q, k, v, _ = make_inputs(w)
    k16, v16 = k.astype(np.float16), v.astype(np.float16)
    got = precise_attention(w, q, k16, v16, gpu)
    want = ref.gqa_attention(q, k16, v16, position, w.scale)
    assert_parity(got, want)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) <= PRECISE_REL_L2


@pytest.mark.parametrize('batch,position,seed', fused_cases(40, 7000))
def test_fused_sweep(gpu, batch, position, seed):
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
    print(f'fused sweep: batch={batch} position={position} seed={seed}', flush=True)
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
