"""The reference session's attention side through the fused device path.

AttentionKV drives every full-attention layer with the reference's
k_attention semantics (src/runtime.cu:398-407): fp32 q_gate, key and value,
the layer's q_norm / k_norm, prepare + fp16 append + causal attention +
sigmoid gate at the session position, on the layer's paged caches.  Each
step is checked against the oracle's restatement of tests/cpu_reference.py
on the logical token-major caches that the same session operations produce,
with the reference test's tolerances (tests/test_cuda.py:218-220): output
3e-4, K cache 2e-3, V cache exact.
"""
import numpy as np
import pytest

from oracle import attention_ref as ref
from tests.test_attention_gpu import assert_close

pytestmark = pytest.mark.gpu

EPS = 1e-6


@pytest.mark.parametrize('first', [40, 300])
def test_session_fused_prefill_verify_commit_checkpoint_restore(gpu, first):
    """The sequence after a first prefill chunk of `first` tokens: at 40 the
    later steps run the one-launch kernel of short contexts; at 300 they run
    the split kernels that prepare their own query (the stream kernel for one
    or two tokens, the ring kernel for 5 and 8)."""
    torch = gpu
    from redshift_amd.kvcache import AttentionKV, SessionError
    layers = 2
    rng = np.random.default_rng(11)
    kv = AttentionKV(layers, context=1024, epsilon=EPS)
    norms = [[(1 + .1 * rng.standard_normal(256)).astype(np.float32) for _ in range(2)] for _ in range(layers)]
    logical = [[np.zeros((0, 4, 256), np.float16)] * 2 for _ in range(layers)]

    def dev(x):
        return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()

    def run(T, recording=False):
        if T > 8:
            kv.begin_prefill(T)
        else:
            kv.begin(T, recording)
        pos = kv.position
        steps = []
        for layer in range(layers):
            q_gate = rng.standard_normal((T, 24, 512)).astype(np.float32)
            key = rng.standard_normal((T, 4, 256)).astype(np.float32)
            value = rng.standard_normal((T, 4, 256)).astype(np.float32)
            qn, kn = norms[layer]
            lk, lv = logical[layer]
            want = ref.fused_attention(lk[:pos], lv[:pos], q_gate, key, value, qn, kn, T, pos, EPS)
            got = kv.attend(layer, dev(q_gate), dev(key), dev(value), dev(qn), dev(kn))
            steps.append((got, want))
        kv.end()
        print(f'session step: {T} tokens at {pos}, recording={recording}', flush=True)
        for layer, (got, (out, kc, vc)) in enumerate(steps):
            assert_close(got.cpu().numpy(), out, 3e-4)
            k_dev, v_dev = kv.caches[layer].unpack(0, pos + T)
            torch.cuda.synchronize()
            assert_close(k_dev.float().cpu().numpy(), kc, 2e-3)
            assert_close(v_dev.float().cpu().numpy(), vc, 0)
            logical[layer] = [k_dev.cpu().numpy(), v_dev.cpu().numpy()]

    run(first)                       # a prefill chunk (prefill kernel)
    run(8)                           # the server's 8-token prefill step (split kernels)
    run(1)                           # decode (fused split: query prepared, key appended in-kernel)
    assert kv.position == first + 9
    run(8, recording=True)           # verification
    assert (kv.position, kv.pending) == (first + 17, 8)
    with pytest.raises(SessionError, match='commit or abort'):
        kv.begin(1)
    with pytest.raises(SessionError, match='commit or abort'):
        kv.checkpoint()
    with pytest.raises(SessionError, match='acceptance outside'):
        kv.commit(9)
    kv.commit(1)
    assert (kv.position, kv.pending) == (first + 10, 0)
    with pytest.raises(SessionError, match='between 1 and 8$'):
        kv.begin(9, recording=True)
    run(1)                           # overwrites the first rejected row (first + 10)
    kv.checkpoint()
    saved = [[a.copy() for a in pair] for pair in logical]
    run(5, recording=True)
    kv.commit(5)
    run(1)
    assert kv.position == first + 17
    kv.restore()
    assert (kv.position, kv.pending) == (first + 11, 0)
    logical = saved
    run(2)                           # from the restored prefix
    kv.reset()
    assert kv.position == 0
    with pytest.raises(SessionError, match='no valid checkpoint'):
        kv.restore()


def test_session_poisoned_after_a_failure_until_restore(gpu):
    """A failure inside a step poisons the session (src/runtime.cu:297-300,
    374-375): every step, commit and checkpoint is refused until restore()
    or reset(); restore() returns to the checkpoint, whose prefix attends
    as before."""
    torch = gpu
    from redshift_amd.kvcache import AttentionKV, SessionError
    rng = np.random.default_rng(12)
    kv = AttentionKV(1, context=256, epsilon=EPS)
    ones = torch.ones(256, device='cuda')

    def inputs(T):
        return [torch.from_numpy(rng.standard_normal(s).astype(np.float32)).cuda()
                for s in ((T, 24, 512), (T, 4, 256), (T, 4, 256))]

    kv.begin(3)
    first = kv.attend(0, *inputs(3), ones, ones).clone()
    kv.end()
    kv.checkpoint()
    probe = inputs(1)
    kv.begin(1)
    before = kv.attend(0, *probe, ones, ones).clone()
    kv.end()
    kv.begin(2)
    bad = inputs(2)
    with pytest.raises(ValueError):
        kv.attend(0, bad[0].double(), *bad[1:], ones, ones)     # refused by the front end
    assert kv.poisoned
    for refused in (lambda: kv.begin(1), lambda: kv.checkpoint()):
        with pytest.raises(SessionError, match='invalid after a CUDA failure'):
            refused()
    kv.restore()
    assert (kv.position, kv.poisoned) == (3, False)
    kv.begin(1)
    after = kv.attend(0, *probe, ones, ones)
    kv.end()
    torch.cuda.synchronize()
    assert torch.equal(before, after)
    assert torch.isfinite(first).all()
