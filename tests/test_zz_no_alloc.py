"""qv_attention_noalloc (no workspace argument, its workspace in the
library's static device array) against qv_attention with its own
workspace: the same kernels and plan, so the same bits.  Two calls in a row
share the array, the second with a smaller input; a call with more rows
than the split kernels take (the prefill kernel, no workspace), a bf16 one,
and a bf16 prefill (its fp16 copy of the V pages in the array) follow."""
import numpy as np
import pytest

from redshift_amd import attention as A
from redshift_amd.workloads import Workload, make_inputs
from tests.test_attention_gpu import make_cache, to_torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('order', ['large_then_small', 'small_then_large'])
def test_noalloc_equals_workspace_entry(gpu, order):
    torch = gpu
    shapes = [Workload('verify', 24, 4, 256, 8, 16384, 1 / 16, 'f16', 31, 1.0, 0.5),   # 11.3 MB of partials
              Workload('decode', 24, 4, 256, 1, 3000, 1 / 16, 'f16', 32, 1.0, 0.5)]
    if order == 'small_then_large':
        shapes = shapes[::-1]
    shapes += [Workload('prefill', 24, 4, 256, 50, 700, 1 / 16, 'f16', 33, 1.0, 0.5),
               Workload('bf16', 16, 2, 128, 3, 5000, 1 / 128 ** .5, 'bf16', 34, 1.0, 0.5),
               Workload('bf16_prefill', 24, 4, 256, 100, 2000, 1 / 16, 'bf16', 35, 1.0, 0.5)]
    prepared = []
    for w in shapes:
        q, k, v, _ = make_inputs(w)
        prepared.append((w, to_torch(q, w.dtype, torch), make_cache(k, v, w, torch, fill_nan=True)))
    for w, qt, cache in prepared:
        print(f'noalloc: {w.name} {w.q_heads}/{w.kv_heads}/{w.head_dim} tokens={w.tokens} '
              f'position={w.position} {w.dtype}', flush=True)
        for out_dtype in (None, torch.float32):
            ws = A.workspace(A.attention_workspace_bytes(w.q_heads, w.kv_heads, w.head_dim, w.tokens, w.position))
            want = A.attention(qt, cache, w.position, w.scale, ws=ws, out_dtype=out_dtype)
            got = A.attention_noalloc(qt, cache, w.position, w.scale, out_dtype=out_dtype)
            torch.cuda.synchronize()
            assert torch.isfinite(got.float()).all()
            assert torch.equal(got, want), float((got.float() - want.float()).abs().max())
