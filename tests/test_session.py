"""The session's refusals and poisoned state without a GPU: the checks run
before any library call (src/runtime.cu:297-300,356-375,432-485)."""
import pytest
import torch

from redshift_amd.kvcache import AttentionKV, SessionError


def session():
    return AttentionKV(2, context=64, epsilon=1e-6, device='cpu')


def test_preflight_refusals_leave_the_state_clean():
    kv = session()
    # begin() keeps evaluate()'s rule and message (src/runtime.cu:65-67).
    for batch, recording in ((0, False), (9, False), (9, True), (0, True)):
        with pytest.raises(SessionError, match='^batch must be between 1 and 8$'):
            kv.begin(batch, recording)
    with pytest.raises(SessionError, match='prefill chunk must be between 1 and 8192 tokens'):
        kv.begin_prefill(0)
    with pytest.raises(SessionError, match='prefill chunk must be between 1 and 8192 tokens'):
        kv.begin_prefill(8193)
    with pytest.raises(SessionError, match='exceeds context capacity'):
        kv.begin_prefill(65)
    with pytest.raises(SessionError, match='no pending verification'):
        kv.commit(0)
    with pytest.raises(SessionError, match='no valid checkpoint'):
        kv.restore()
    with pytest.raises(SessionError, match='no batch in progress'):
        kv.end()
    assert not kv.poisoned and kv.position == 0
    with pytest.raises(SessionError, match='context must be'):
        AttentionKV(1, context=139265, device='cpu')
    with pytest.raises(SessionError, match='epsilon'):
        AttentionKV(1, context=64, epsilon=0.0, device='cpu')


def test_a_failure_inside_a_step_poisons_until_reset():
    kv = session()
    kv.begin(2)
    assert kv.poisoned                         # past the preflight checks
    bad = [torch.zeros((2, 24, 512), dtype=torch.float64), torch.zeros((2, 4, 256)),
           torch.zeros((2, 4, 256)), torch.ones(256), torch.ones(256)]
    with pytest.raises(ValueError, match='q_gate must be float32'):
        kv.attend(0, *bad)
    for refused in (lambda: kv.begin(1), lambda: kv.checkpoint(), lambda: kv.commit(0)):
        with pytest.raises(SessionError, match='model state is invalid after a CUDA failure; reset or restore'):
            refused()
    kv.reset()
    assert (kv.poisoned, kv.position, kv.pending) == (False, 0, 0)
    kv.begin(1, recording=True)
    kv.end()                                   # no layer attended: the bookkeeping alone
    assert (kv.position, kv.pending, kv.verify_position) == (1, 1, 0)
    kv.commit(0)
    assert (kv.position, kv.pending) == (0, 0)


def test_prefill_chunk_bookkeeping():
    kv = session()
    kv.begin_prefill(40)
    assert kv.poisoned
    kv.end()
    assert (kv.position, kv.pending, kv.poisoned) == (40, 0, False)
    kv.begin(8, recording=True)
    kv.end()
    assert (kv.position, kv.pending) == (48, 8)
    with pytest.raises(SessionError, match='commit or abort'):
        kv.begin_prefill(1)
