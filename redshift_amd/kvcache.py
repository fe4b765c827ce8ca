"""KV caches of the model's full-attention layers on the paged layout, with
the reference model session's position bookkeeping for them.

The reference keeps, per full-attention layer, token-major fp16 K and V
caches of `context` rows (src/runtime.cu:291-296), appends the new rows of
every evaluated batch at `position` (src/kernels.cu:416-434), and manages
them in `Model` (src/runtime.cu:256-266):

* evaluate(batch, recording) refuses to run while a verification is pending,
  requires position + batch <= context, records verify_position when
  recording, and advances position by batch (src/runtime.cu:356-375,430);
* commit(accepted) needs a pending verification and 0 <= accepted <= batch;
  position becomes verify_position + accepted.  Rejected rows need no work:
  they are unreachable and overwritten by later appends
  (src/runtime.cu:432-454);
* checkpoint / restore copy the valid prefix of each cache to a snapshot
  sized for that prefix and back (copy_state, src/runtime.cu:455-485);
* reset() returns to position 0 (src/runtime.cu:301-311).

Here the caches are `PagedKV` pages and the copies are qv_kv_copy; the
messages of the refusals are the reference's.
"""
import torch

from .attention import PAGE_TOKENS, PagedKV, _ptr, _stream, attention, round_capacity
from .runtime import check, library


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
    """The full-attention layers' caches of one session."""

    def __init__(self, layers, kv_heads=4, head_dim=256, context=139264, dtype=torch.float16):
        _require(type(context) is int and 1 <= context, 'context must be a positive integer')
        self.context = context
        self.caches = [PagedKV(kv_heads, head_dim, round_capacity(context), dtype) for _ in range(layers)]
        self.position = 0
        self.pending = 0          # batch of the verification awaiting commit
        self.verify_position = 0
        self.saved = False
        self.saved_position = 0
        self._snapshots = [None] * layers
        self._batch = None
        self._recording = False

    # -- one evaluated batch ----------------------------------------------
    def begin(self, batch, recording=False):
        """Start a batch of `batch` tokens (src/runtime.cu:356-375)."""
        _require(not self.pending, 'commit or abort the pending verification first')
        _require(1 <= batch <= 8, 'batch must be between 1 and 8')
        _require(self.position <= self.context - batch, 'evaluation exceeds context capacity')
        if recording:
            self.verify_position = self.position
        self._batch, self._recording = batch, recording

    def attend(self, layer, q, k_rows, v_rows, scale):
        """Append the batch's K/V rows to `layer` at the current position and
        attend its queries over keys 0 .. position + t."""
        _require(self._batch is not None and k_rows.shape[0] == self._batch, 'no batch in progress')
        cache = self.caches[layer]
        cache.pack(k_rows, v_rows, first=self.position)
        return attention(q, cache, self.position, scale, out_dtype=torch.float32)

    def end(self):
        """Finish the batch: position advances; a recording batch waits for
        commit (src/runtime.cu:427-430)."""
        _require(self._batch is not None, 'no batch in progress')
        self.position += self._batch
        if self._recording:
            self.pending = self._batch
        self._batch = None

    # -- verification, checkpoints ------------------------------------------
    def commit(self, accepted):
        """src/runtime.cu:432-454: keep `accepted` of the verified rows."""
        _require(self.pending > 0, 'no pending verification')
        _require(0 <= accepted <= self.pending, 'acceptance outside verified batch')
        self.position = self.verify_position + accepted
        self.pending = 0

    def checkpoint(self):
        """copy_state(false), src/runtime.cu:455-485: snapshot the prefix."""
        _require(not self.pending, 'commit or abort the pending verification first')
        self.saved = False
        need = max(PAGE_TOKENS, -(-self.position // PAGE_TOKENS) * PAGE_TOKENS)
        for i, cache in enumerate(self.caches):
            snap = self._snapshots[i]
            if snap is None or snap.capacity < need:
                snap = self._snapshots[i] = PagedKV(cache.kv_heads, cache.head_dim, need, cache.dtype)
            copy_prefix(snap, cache, self.position)
        self.saved_position = self.position
        self.saved = True

    def restore(self):
        """copy_state(true): the snapshot's prefix back; position as saved."""
        _require(self.saved, 'no valid checkpoint')
        for cache, snap in zip(self.caches, self._snapshots):
            copy_prefix(cache, snap, self.saved_position)
        self.position = self.saved_position
        self.pending = 0

    def reset(self):
        """src/runtime.cu:301-311 (the attention caches need no clearing)."""
        self.saved = False
        self.pending = 0
        self.position = 0
