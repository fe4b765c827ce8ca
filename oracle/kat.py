"""Known-answer tests that pin the oracle (test infrastructure only).

``long_context_case`` restates the reference's closed-form attention test
(tests/test_cuda.py:237-273): K rows cycle with period 7 (dims 0..63 zero, so
RoPE is inert), V rows cycle with period 11, the new keys are zero and the
gate is zero, so the expected output is analytic.  The other helpers give
textbook closed forms for the pieces that KAT leaves open: RoPE on a one-hot
row (rotate-half pairs), RMSNorm of a constant row, binary16 bit patterns.
"""
import math

import numpy as np

D = 256
ROPE_BASE = 10000000.0


def _key_row(level):
    # tests/test_cuda.py:241: [0]*64 + [level]*192 for each of the 4 kv heads.
    return np.tile(np.concatenate([np.zeros(64), np.full(192, level)]), 4)


def _value_row(p):
    # tests/test_cuda.py:243-245
    h = np.repeat(np.arange(4), 256)
    d = np.tile(np.arange(256), 4)
    return (p - 5) * .125 + h * .03125 + (d % 4) * .0625


def long_context_case(position, batch):
    """Inputs and the analytic output of tests/test_cuda.py:246-270.

    Returns a dict with token-major fp16 prefix caches ``key_cache`` and
    ``value_cache`` (numpy float16, [position, 4, 256]), ``q_gate``
    [batch, 24, 512], ``key``/``value`` [batch, 4, 256], ``q_norm``/``k_norm``
    [256], ``epsilon`` and ``expected`` (float64, [batch, 24, 256]).
    """
    key_rows = np.stack([_key_row((i - 3) * .25) for i in range(7)]).astype(np.float16)
    value_rows = np.stack([_value_row(p) for p in range(11)]).astype(np.float16)
    p = np.arange(position)
    key_cache = key_rows[p % 7].reshape(position, 4, 256)
    value_cache = value_rows[p % 11].reshape(position, 4, 256)
    query = np.concatenate([np.zeros(64), (np.arange(192) % 4 + 1) * .03125])
    q_gate = np.tile(np.concatenate([query, np.zeros(256)]), (batch, 24, 1))
    key = np.zeros((batch, 4, 256))
    t = np.arange(batch)[:, None, None]
    h = np.arange(4)[None, :, None]
    d = np.arange(256)[None, None, :]
    value = (t + 1) * .125 + h * .03125 + (d % 4) * .0625
    norm = np.ones(256)
    eps = 1e-6
    # Closed form (tests/test_cuda.py:251-270).
    scale = 1 / math.sqrt(float(np.sum(query * query)) / 256 + eps)
    qsum = float(np.sum(query)) * scale
    weights = np.exp(qsum * ((p % 7 - 3) * .25) / 16)
    total = float(np.sum(weights))
    numerator = float(np.sum(weights * (p % 11 - 5) * .125))
    expected = np.empty((batch, 24, 256))
    hh = np.arange(24)[:, None]
    dd = np.arange(256)[None, :]
    for tt in range(batch):
        total += 1
        numerator += (tt + 1) * .125
        expected[tt] = .5 * (numerator / total + (hh // 6) * .03125 + (dd % 4) * .0625)
    return dict(key_cache=key_cache, value_cache=value_cache, q_gate=q_gate,
                key=key, value=value, q_norm=norm, k_norm=norm, epsilon=eps,
                expected=expected)


def sine_wave_case(batch=3, position=5):
    """Inputs of the reference's CPU-prefix fixture (tests/test_cuda.py:201-216):
    ``scale * sin(i * .051 + phase)`` waves, fp16 prefix caches,
    q_norm = 1 + i/512, k_norm = 1 - i/512, epsilon 1e-6.  Computed in float32
    like the ctypes ``c_float`` buffers the reference test builds."""
    def wave(n, phase, scale=.3):
        i = np.arange(n, dtype=np.float64)
        return (scale * np.sin(i * .051 + phase)).astype(np.float32)
    prefix_k = wave(position * 1024, .5).astype(np.float16)
    prefix_v = wave(position * 1024, .9).astype(np.float16)
    return dict(
        key_cache=prefix_k.reshape(position, 4, 256),
        value_cache=prefix_v.reshape(position, 4, 256),
        q_gate=wave(batch * 12288, 1.5).reshape(batch, 24, 512),
        key=wave(batch * 1024, .1).reshape(batch, 4, 256),
        value=wave(batch * 1024, .7).reshape(batch, 4, 256),
        q_norm=(1 + np.arange(256) / 512).astype(np.float32),
        k_norm=(1 - np.arange(256) / 512).astype(np.float32),
        epsilon=1e-6, batch=batch, position=position)


def rope_one_hot(i, pos, gamma, epsilon, amplitude=1.0):
    """Closed form of prepare() on the row amplitude*e_i (i < 32 or 32 <= i < 64).

    RMSNorm of a one-hot row is amplitude/sqrt(amplitude^2/256 + eps) at dim i,
    times gamma[i]; the rotate-half RoPE then moves it into the pair (j, j+32)
    with j = i mod 32 and angle pos * 1e7 ** (-j/32):
      i <  32: out[j] =  v cos(a), out[j+32] = v sin(a)
      i >= 32: out[j] = -v sin(a), out[j+32] = v cos(a)
    Returns the full expected row (float64, [256])."""
    v = amplitude / math.sqrt(amplitude * amplitude / 256 + epsilon) * float(gamma[i])
    j = i % 32
    a = pos * ROPE_BASE ** (-j / 32)
    out = np.zeros(256)
    if i < 32:
        out[j], out[j + 32] = v * math.cos(a), v * math.sin(a)
    else:
        out[j], out[j + 32] = -v * math.sin(a), v * math.cos(a)
    return out


# IEEE binary16 known answers: (value, expected bit pattern).  Ties go to even.
HALF_BITS = [
    (0.0, 0x0000), (-0.0, 0x8000), (1.0, 0x3C00), (-2.0, 0xC000),
    (65504.0, 0x7BFF), (65520.0, 0x7C00),                  # max finite; rounds to inf
    (1.0 / 3.0, 0x3555), (0.1, 0x2E66),
    (1.0 + 2.0 ** -11, 0x3C00),                            # tie -> even (down)
    (1.0 + 3 * 2.0 ** -11, 0x3C02),                        # tie -> even (up)
    (2.0 ** -24, 0x0001), (2.0 ** -25, 0x0000),            # smallest subnormal; tie -> 0
    (6.103515625e-05, 0x0400),                             # smallest normal
]
