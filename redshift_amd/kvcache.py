"""KV caches of the model's full-attention layers on the paged layout, with
the reference model session's bookkeeping for them.

The reference keeps, per full-attention layer, token-major fp16 K and V
caches of `context` rows (src/runtime.cu:291-296) inside `Model`
(src/runtime.cu:255-266).  Its evaluate() runs, for every full-attention
layer, k_attention on the layer's caches at `position` with the projected
fp32 q_gate, key and value and the layer's q_norm / k_norm weights
(src/runtime.cu:398-407): prepare, fp16 append at position.., causal
attention, sigmoid gate.  Around that:

* evaluate(batch, recording) needs a ready model (not poisoned,
  src/runtime.cu:297-300), refuses to run while a verification is pending,
  requires position + batch <= context, records verify_position when
  recording, marks the state poisoned once the preflight checks have
  passed, and on success advances position by batch and clears the poison
  (src/runtime.cu:356-375,427-430);
* commit(accepted) needs a ready model and a pending verification with
  0 <= accepted <= batch; position becomes verify_position + accepted.
  Rejected rows need no work: they are unreachable and overwritten by later
  appends (src/runtime.cu:432-454);
* checkpoint / restore copy the valid prefix of each cache to a snapshot
  sized for that prefix and back (copy_state, src/runtime.cu:455-485);
  restore needs a valid checkpoint only, and clears the poison;
* reset() returns to position 0 and clears the poison (src/runtime.cu:301-311).

Here the caches are `PagedKV` pages, k_attention is qv_attention_fused, and
the copies are qv_kv_copy; the refusals carry the reference's messages.  A
step is begin(), one attend() per full-attention layer, end(): any failure
between begin() and the end of end() (a library error, a device fault that
the synchronisation in end() reports) leaves the session poisoned until
reset() or restore(), as a failure inside the reference's evaluate() does.

One addition has no counterpart in the reference: begin_prefill(batch) opens
a non-recording step of up to 8192 tokens (a whole prompt chunk through the
prefill kernel, where the reference's server feeds 8 tokens per evaluate(),
qvelox/server.py:177-192).  begin() itself keeps evaluate()'s 1..8 rule and
message.
"""
import torch

from .attention import (PAGE_TOKENS, PagedKV, _ptr, _stream, attention_fused, check_fused_inputs,
                        fused_workspace_bytes, round_capacity, workspace)
from .runtime import check, library

# The reference's fixed attention geometry (src/runtime.h:38-41).
Q_HEADS, KV_HEADS, HEAD_DIM = 24, 4, 256
# evaluate() takes 1..8 tokens (src/runtime.cu:65-67,358); begin_prefill's
# chunks (no recording) take up to the fused entry's 8192 tokens.
MAX_BATCH, MAX_CHUNK = 8, 8192


class SessionError(RuntimeError):
    """A call that the reference's model session refuses."""


def _require(condition, message):
    if not condition:
        raise SessionError(message)


def copy_prefix(dst, src, tokens):
    """Pages holding tokens 0..tokens-1 of every KV head, K and V, src -> dst."""
    lib = library()
    check(lib, lib.qv_kv_copy(_ptr(dst.k), _ptr(dst.v), _ptr(src.k), _ptr(src.v), src.kv_heads,
                              src.head_dim, dst.capacity, src.capacity, tokens, _stream()))


class AttentionKV:
    """The full-attention layers' caches of one session (fp16 pages of the
    24/4/256 model, `context` tokens each)."""

    def __init__(self, layers, context=139264, epsilon=1e-6, device='cuda'):
        _require(type(context) is int and 1 <= context <= 139264, 'context must be in 1..139264')
        _require(epsilon > 0 and epsilon == epsilon and epsilon != float('inf'),
                 'epsilon must be finite and positive')
        self.context, self.epsilon, self.device = context, float(epsilon), device
        self.caches = [PagedKV(KV_HEADS, HEAD_DIM, round_capacity(context), torch.float16, device)
                       for _ in range(layers)]
        self.position = 0
        self.pending = 0          # batch of the verification awaiting commit
        self.verify_position = 0
        self.saved = False
        self.saved_position = 0
        self.poisoned = False
        self._snapshots = [None] * layers
        self._batch = None
        self._recording = False
        self._ws = None

    def _ready(self):
        _require(not self.poisoned, 'model state is invalid after a CUDA failure; reset or restore')

    def _workspace(self, batch):
        need = fused_workspace_bytes(batch, self.position)
        if self._ws is None or self._ws.numel() < need:
            self._ws = workspace(need, self.device)
        return self._ws

    # -- one evaluated batch ----------------------------------------------
    def begin(self, batch, recording=False):
        """Preflight of evaluate() (src/runtime.cu:356-375), with its batch
        rule (1..8, src/runtime.cu:65-67); afterwards the state counts as
        poisoned until end() returns."""
        self._begin(batch, recording, MAX_BATCH, 'batch must be between 1 and 8')

    def begin_prefill(self, batch):
        """begin() for a prompt chunk of 1..8192 tokens that does not record
        (no counterpart in the reference, whose server prefills 8 tokens per
        evaluate()); the same preflight otherwise."""
        self._begin(batch, False, MAX_CHUNK, 'prefill chunk must be between 1 and 8192 tokens')

    def _begin(self, batch, recording, limit, message):
        self._ready()
        _require(not self.pending, 'commit or abort the pending verification first')
        _require(type(batch) is int and 1 <= batch <= limit, message)
        _require(self.position <= self.context - batch, 'evaluation exceeds context capacity')
        if recording:
            self.verify_position = self.position
        self.poisoned = True
        self._batch, self._recording = batch, recording

    def attend(self, layer, q_gate, key, value, q_norm, k_norm, out=None):
        """k_attention for one full-attention layer (src/runtime.cu:398-407):
        q_gate [batch][24][512], key and value [batch][4][256], q_norm and
        k_norm [256], all float32 on the session's device.  Prepares q and k,
        appends k and v to the layer's pages at the current position,
        attends over keys 0..position+t and applies the sigmoid gate;
        returns float32 [batch][24][256] (stream-ordered)."""
        _require(self._batch is not None, 'no batch in progress')
        _require(q_gate.shape[0] == self._batch, f'q_gate holds {q_gate.shape[0]} tokens, the batch {self._batch}')
        check_fused_inputs(q_gate, key, value, q_norm, k_norm, self.caches[layer])
        return attention_fused(q_gate, key, value, q_norm, k_norm, self.caches[layer], self.position,
                               self.epsilon, out=out, ws=self._workspace(self._batch))

    def end(self):
        """Finish the batch: the stream is synchronised (the reference's
        finish(), which reports device failures), position advances and the
        poison clears; a recording batch waits for commit
        (src/runtime.cu:425-430)."""
        _require(self._batch is not None, 'no batch in progress')
        if str(self.device).startswith('cuda'):
            torch.cuda.current_stream().synchronize()
        self.position += self._batch
        self.poisoned = False
        if self._recording:
            self.pending = self._batch
        self._batch = None

    # -- verification, checkpoints ------------------------------------------
    def commit(self, accepted):
        """src/runtime.cu:432-454: keep `accepted` of the verified rows."""
        self._ready()
        _require(self.pending > 0, 'no pending verification')
        _require(type(accepted) is int and 0 <= accepted <= self.pending, 'acceptance outside verified batch')
        self.position = self.verify_position + accepted
        self.pending = 0
        self.poisoned = False

    def checkpoint(self):
        """copy_state(false), src/runtime.cu:455-485: snapshot the prefix."""
        self._ready()
        _require(not self.pending, 'commit or abort the pending verification first')
        self.saved = False
        need = max(PAGE_TOKENS, -(-self.position // PAGE_TOKENS) * PAGE_TOKENS)
        for i, cache in enumerate(self.caches):
            snap = self._snapshots[i]
            if snap is None or snap.capacity < need:
                snap = self._snapshots[i] = PagedKV(cache.kv_heads, cache.head_dim, need, cache.dtype, self.device)
            copy_prefix(snap, cache, self.position)
        torch.cuda.current_stream().synchronize()
        self.saved_position = self.position
        self.saved = True

    def restore(self):
        """copy_state(true): the snapshot's prefix back; position as saved,
        no pending verification, the poison cleared."""
        _require(self.saved, 'no valid checkpoint')
        self.poisoned = True
        for cache, snap in zip(self.caches, self._snapshots):
            copy_prefix(cache, snap, self.saved_position)
        torch.cuda.current_stream().synchronize()
        self.position = self.saved_position
        self.poisoned = False
        self.pending = 0
        self._batch = None

    def reset(self):
        """src/runtime.cu:301-311 (the attention caches need no clearing)."""
        self.saved = False
        self.pending = 0
        self.position = 0
        self.poisoned = False
        self._batch = None
