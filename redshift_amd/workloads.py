"""Seeded synthetic inputs of the attention workloads (numpy, host memory).

The five shapes are the path's parity and benchmark cases:
  cpu_plumbing  8/2/128 GQA decode, 128 keys, fp32 N(0,1), seed 0, scale 1/sqrt(128)
  decode_4k     24/4/256 decode, 4,096 keys, KV N(0,1)*0.5 fp16, Q N(0,1) fp16, scale 1/16
  verify8_16k   8 candidates on a 16,384-token prefix (+ their own 8 K/V rows),
                causal in the candidate block, all values N(0,1)*0.5 fp16, seed 1
  decode_139k   1 query on 139,264 keys, N(0,1)*0.5 fp16, 64 keys scaled x8 at
                seeded random positions (softmax stability)
  prefill_2k    2,048 new tokens on a 6,144-token cache (8,192 keys), causal,
                bf16 N(0,1), seed 2
Shapes: q [tokens][q_heads][head_dim]; k, v token-major [keys][kv_heads][head_dim];
row t of q sees keys 0..position+t.
"""
import math
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Workload:
    name: str
    q_heads: int
    kv_heads: int
    head_dim: int
    tokens: int
    position: int
    scale: float
    dtype: str          # 'f32', 'f16' or 'bf16' storage of q/k/v
    seed: int
    q_std: float = 1.0
    kv_std: float = 1.0
    outliers: int = 0   # keys scaled by `outlier_gain` at random positions
    outlier_gain: float = 8.0

    @property
    def keys(self):
        return self.position + self.tokens

    @property
    def group(self):
        return self.q_heads // self.kv_heads

    def kv_bytes(self):
        """Algorithmic K+V bytes one call reads (each key once)."""
        elem = 4 if self.dtype == 'f32' else 2
        return 2 * self.keys * self.kv_heads * self.head_dim * elem

    def flops(self):
        """2 FLOP per multiply-add of Q.K^T and P.V over the causal (row, key) pairs."""
        pairs = self.tokens * self.position + self.tokens * (self.tokens + 1) // 2
        return 4 * self.head_dim * self.q_heads * pairs


WORKLOADS = {
    w.name: w for w in [
        Workload('cpu_plumbing', 8, 2, 128, 1, 127, 1 / math.sqrt(128), 'f32', 0),
        Workload('decode_4k', 24, 4, 256, 1, 4095, 1 / 16, 'f16', 0, q_std=1.0, kv_std=0.5),
        Workload('verify8_16k', 24, 4, 256, 8, 16384, 1 / 16, 'f16', 1, q_std=0.5, kv_std=0.5),
        # One token over the verify-8 workload's 16,392 keys: the same K/V
        # bytes streamed with one query row per query head.
        Workload('decode_16k', 24, 4, 256, 1, 16391, 1 / 16, 'f16', 1, q_std=0.5, kv_std=0.5),
        Workload('decode_139k', 24, 4, 256, 1, 139263, 1 / 16, 'f16', 3, q_std=0.5, kv_std=0.5,
                 outliers=64),
        Workload('prefill_2k', 24, 4, 256, 2048, 6144, 1 / 16, 'bf16', 2),
    ]
}


def _cast(x, dtype):
    """float32 numpy -> storage dtype; bf16 is returned as uint16 bit patterns
    (round to nearest even), fp16 as numpy float16."""
    if dtype == 'f32':
        return x.astype(np.float32)
    if dtype == 'f16':
        return x.astype(np.float16)
    if dtype == 'bf16':
        return f32_to_bf16_bits(x)
    raise ValueError(dtype)


def f32_to_bf16_bits(x):
    """IEEE float32 -> bfloat16 bits, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, (u >> 16) | 0x40, rounded).astype(np.uint16)


def bf16_bits_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_float(x, dtype):
    """Storage array -> float64 values."""
    if dtype == 'bf16':
        return bf16_bits_to_f32(x).astype(np.float64)
    return np.asarray(x, np.float64)


def make_inputs(w: Workload):
    """Seeded q, k, v (storage dtype) and the outlier positions (may be empty)."""
    rng = np.random.default_rng(w.seed)
    n = w.keys
    q = rng.standard_normal((w.tokens, w.q_heads, w.head_dim), dtype=np.float32) * np.float32(w.q_std)
    k = rng.standard_normal((n, w.kv_heads, w.head_dim), dtype=np.float32) * np.float32(w.kv_std)
    v = rng.standard_normal((n, w.kv_heads, w.head_dim), dtype=np.float32) * np.float32(w.kv_std)
    outliers = np.sort(rng.choice(n, size=w.outliers, replace=False)) if w.outliers else np.zeros(0, np.int64)
    if w.outliers:
        k[outliers] *= np.float32(w.outlier_gain)
    return _cast(q, w.dtype), _cast(k, w.dtype), _cast(v, w.dtype), outliers
