"""numpy restatement of the reference's CPU attention oracle (test infrastructure).

Follows ``tests/cpu_reference.py`` of the reference:
  * ``sigmoid``          <- tests/cpu_reference.py:6-7
  * ``half``             <- tests/cpu_reference.py:14-15 (``struct '<e'`` = IEEE
                            binary16, round to nearest even; numpy's float64 ->
                            float16 cast rounds the same way, in one step)
  * ``rmsnorm``/``rope`` <- tests/cpu_reference.py:62-70 (the ``prepare`` closure:
                            RMS over 256 dims, times gamma, then rotate pairs
                            (i, i+32) for i < 32 by pos * 1e7 ** (-i/32))
  * ``fused_attention``  <- tests/cpu_reference.py:55-89 (fp16 K/V append, causal
                            GQA softmax with kv head h // 6, scale 1/16, times
                            sigmoid(gate)); the order of operations follows
                            src/kernels.cu:416-434 (prepare) and 466-503.
  * ``fused_attention_rows`` <- the same function on selected tokens of a
                            long chunk: its prepare and fp16 append steps,
                            then ``gqa_attention`` on the selected rows, times
                            sigmoid(gate) (checked against ``fused_attention``
                            in tests/test_oracle.py)
  * ``gqa_attention``    <- the raw core inside the same function
                            (tests/cpu_reference.py:79-87 without prepare and
                            gate), parametric in heads, head_dim and scale, as
                            the raw-core workloads need.  Row t of a chunk that
                            starts at ``position`` sees keys 0..position+t.

Everything accumulates in float64 unless the name says fp32.  The fp32 variant
(``gqa_attention_fp32``) is the CPU path that the benchmark times beside the
GPU: BLAS-batched Q.K^T and P.V per KV-head group, fp32 softmax.
"""
import numpy as np

# Model constants of the reference's fixed attention shape
# (src/runtime.h:38-41, qvelox/model.py:11-13, src/kernels.cu:419-455).
Q_HEADS, KV_HEADS, HEAD_DIM = 24, 4, 256
ROPE_PAIRS, ROPE_BASE = 32, 10000000.0
CAPACITY = 139264
FUSED_SCALE = 1.0 / 16.0


def sigmoid(x):
    """Logistic function (tests/cpu_reference.py:6-7)."""
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


def half(x):
    """Round to IEEE binary16 with round-to-nearest-even, returned as float64
    (tests/cpu_reference.py:14-15)."""
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def rmsnorm(row, weight, epsilon):
    """row * rsqrt(mean(row^2) + eps) * weight over the last axis
    (tests/cpu_reference.py:62-64)."""
    row = np.asarray(row, np.float64)
    inv = 1.0 / np.sqrt(np.sum(row * row, axis=-1, keepdims=True) / row.shape[-1] + epsilon)
    return row * inv * np.asarray(weight, np.float64)


def rope(row, pos):
    """Rotate pairs (i, i+32), i < 32, by angle pos * 1e7 ** (-i/32)
    (tests/cpu_reference.py:65-69).  ``pos`` is a scalar or broadcasts against
    the leading axes of ``row``."""
    row = np.array(row, np.float64, copy=True)
    i = np.arange(ROPE_PAIRS, dtype=np.float64)
    angle = np.asarray(pos, np.float64)[..., None] * ROPE_BASE ** (-i / ROPE_PAIRS)
    c, s = np.cos(angle), np.sin(angle)
    x = row[..., :ROPE_PAIRS].copy()
    y = row[..., ROPE_PAIRS:2 * ROPE_PAIRS].copy()
    row[..., :ROPE_PAIRS] = x * c - y * s
    row[..., ROPE_PAIRS:2 * ROPE_PAIRS] = x * s + y * c
    return row


def prepare(row, weight, pos, epsilon):
    """The reference's ``prepare`` closure: RMSNorm, gamma, then RoPE
    (tests/cpu_reference.py:61-70; src/kernels.cu:421-430)."""
    return rope(rmsnorm(row, weight, epsilon), pos)


def fused_attention(key_cache, value_cache, q_gate, key, value, q_norm, k_norm,
                    batch, position, epsilon):
    """Restatement of ``attention`` (tests/cpu_reference.py:55-89).

    Shapes follow the reference's flat buffers (src/runtime.h:38-42):
    key_cache/value_cache hold at least ``position*1024`` values (token-major
    [pos, 4, 256]); q_gate is [batch, 24, 512]; key/value are [batch, 4, 256];
    q_norm/k_norm are [256].  Returns ``(out, kc, vc)``: out is flat
    [batch*24*256] float64, kc/vc are flat [(position+batch)*1024] float64
    holding the prefix unchanged and the appended fp16-rounded rows.
    """
    H, HKV, D = Q_HEADS, KV_HEADS, HEAD_DIM
    G = H // HKV
    kc = np.asarray(key_cache, np.float64).reshape(-1)[:position * HKV * D]
    vc = np.asarray(value_cache, np.float64).reshape(-1)[:position * HKV * D]
    kc = kc.reshape(position, HKV, D)
    vc = vc.reshape(position, HKV, D)
    qg = np.asarray(q_gate, np.float64).reshape(batch, H, 2 * D)
    key = np.asarray(key, np.float64).reshape(batch, HKV, D)
    value = np.asarray(value, np.float64).reshape(batch, HKV, D)
    pos = position + np.arange(batch)
    new_k = half(prepare(key, k_norm, pos[:, None], epsilon))        # [batch, 4, 256]
    new_v = half(value)
    kc = np.concatenate([kc, new_k], axis=0)
    vc = np.concatenate([vc, new_v], axis=0)
    query = prepare(qg[:, :, :D], q_norm, pos[:, None], epsilon)     # [batch, 24, 256]
    gate = qg[:, :, D:]
    out = np.empty((batch, H, D), np.float64)
    for t in range(batch):
        n = position + t + 1
        for g in range(HKV):
            k_g = np.ascontiguousarray(kc[:n, g, :])
            v_g = np.ascontiguousarray(vc[:n, g, :])
            q_g = query[t, g * G:(g + 1) * G, :]                     # heads h with h // 6 == g
            scores = (q_g @ k_g.T) * FUSED_SCALE
            scores = np.exp(scores - scores.max(axis=1, keepdims=True))
            out[t, g * G:(g + 1) * G, :] = (scores @ v_g) / scores.sum(axis=1, keepdims=True)
    out *= sigmoid(gate)
    return out.reshape(-1), kc.reshape(-1), vc.reshape(-1)


def fused_attention_rows(key_cache, value_cache, q_gate, key, value, q_norm, k_norm,
                         batch, position, epsilon, rows):
    """``fused_attention`` on the tokens ``rows`` of the chunk only, for
    chunks too long for its per-token loop: the same prepare and fp16 append
    steps (tests/cpu_reference.py:61-76) for every new token, the causal GQA
    softmax (``gqa_attention``, scale 1/16, kv head h // 6) for the selected
    rows, times sigmoid(gate) (tests/cpu_reference.py:79-88).  Returns
    ``(out, kc, vc)``: out is float64 [len(rows), 24, 256], kc/vc token-major
    [position+batch, 4, 256] float64 caches with the appended rows.
    """
    H, HKV, D = Q_HEADS, KV_HEADS, HEAD_DIM
    kc = np.asarray(key_cache, np.float64).reshape(-1)[:position * HKV * D].reshape(position, HKV, D)
    vc = np.asarray(value_cache, np.float64).reshape(-1)[:position * HKV * D].reshape(position, HKV, D)
    qg = np.asarray(q_gate, np.float64).reshape(batch, H, 2 * D)
    key = np.asarray(key, np.float64).reshape(batch, HKV, D)
    value = np.asarray(value, np.float64).reshape(batch, HKV, D)
    pos = position + np.arange(batch)
    kc = np.concatenate([kc, half(prepare(key, k_norm, pos[:, None], epsilon))], axis=0)
    vc = np.concatenate([vc, half(value)], axis=0)
    rows = np.asarray(rows).reshape(-1)
    query = prepare(qg[rows, :, :D], q_norm, pos[rows][:, None], epsilon)
    full = np.zeros((batch, H, D), np.float64)
    full[rows] = query
    out = gqa_attention(full, kc, vc, position, FUSED_SCALE, rows=rows)
    return out * sigmoid(qg[rows, :, D:]), kc, vc


def gqa_attention(q, k, v, position, scale, rows=None):
    """Raw causal GQA core in float64.

    q: [T, Hq, D]; k, v: [n >= position+T, Hkv, D] token-major; query head h
    reads kv head h // (Hq // Hkv); row t sees keys 0..position+t.  ``rows``
    optionally selects a subset of the T query tokens (the result then has
    len(rows) rows).  Returns float64 [T or len(rows), Hq, D].

    The tokens go through BLAS in blocks of about 768 query rows.  Within a
    block the scores of keys past a row's last key are set to -inf (a
    select, so stale NaN or huge keys there change nothing), and P.V runs in
    two parts: one product over the keys every row of the block sees, then
    each row's remaining visible keys alone, so a value past a row's last
    key is never multiplied, not even by a zero weight.
    """
    q = np.asarray(q)
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    tokens = np.arange(T) if rows is None else np.asarray(rows).reshape(-1)
    out = np.empty((len(tokens), Hq, D), np.float64)
    n_max = position + int(tokens.max()) + 1
    block = max(1, 768 // G)
    for g in range(Hkv):
        k_g = np.asarray(k[:n_max, g, :], np.float64)
        v_g = np.asarray(v[:n_max, g, :], np.float64)
        for b0 in range(0, len(tokens), block):
            tb = tokens[b0:b0 + block]
            last = position + tb + 1                            # keys per row
            n_b, n_common = int(last.max()), int(last.min())
            q_b = np.asarray(q[tb, g * G:(g + 1) * G, :], np.float64)     # [B, G, D]
            s = (q_b @ k_g[:n_b].T) * scale                     # [B, G, n_b]
            visible = np.arange(n_b)[None, :] < last[:, None]   # [B, n_b]
            s = np.where(visible[:, None, :], s, -np.inf)
            s = np.exp(s - s.max(axis=2, keepdims=True))
            o = s[:, :, :n_common] @ v_g[:n_common]             # [B, G, D]
            for i in np.flatnonzero(last > n_common):
                o[i] += s[i, :, n_common:last[i]] @ v_g[n_common:last[i]]
            out[b0:b0 + len(tb), g * G:(g + 1) * G, :] = o / s.sum(axis=2, keepdims=True)
    return out


def gqa_attention_fp32(q, k, v, position, scale):
    """The CPU path timed beside the GPU: same contract as ``gqa_attention``,
    fp32 throughout, BLAS-batched Q.K^T and P.V per KV-head group.  K/V may be
    stored as float16 (the cache format); each group is widened to fp32 inside
    the call, as a CPU implementation of the fp16 cache must."""
    q = np.asarray(q, np.float32)
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    n = position + T
    out = np.empty((T, Hq, D), np.float32)
    limit = position + np.arange(T)
    mask = np.arange(n)[None, :] > limit[:, None]                   # [T, n]
    for g in range(Hkv):
        k_g = np.asarray(k[:n, g, :], np.float32)
        v_g = np.asarray(v[:n, g, :], np.float32)
        q_g = q[:, g * G:(g + 1) * G, :].reshape(T * G, D)
        s = (q_g @ k_g.T) * np.float32(scale)                       # [T*G, n]
        s = s.reshape(T, G, n)
        if T > 1:
            s[np.broadcast_to(mask[:, None, :], s.shape)] = -np.inf
        s -= s.max(axis=2, keepdims=True)
        np.exp(s, out=s)
        denom = s.sum(axis=2, keepdims=True)
        o = (s.reshape(T * G, n) @ v_g).reshape(T, G, D) / denom
        out[:, g * G:(g + 1) * G, :] = o
    return out
