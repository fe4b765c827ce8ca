"""Host-side description of the KV page layout (mirror of the offset functions
in csrc/common.hpp), for building or reading pages in numpy.

Per KV head, tokens live in 32-token pages of 32*D 16-bit elements.
  K element (token p, dim d), page offset:
      (p%32 // 16) * 16*D + (d // 8) * 128 + (p % 16) * 8 + d % 8
  V element (token p, dim d), page offset:
      (d // 16) * 512 + ((p // 4) % 4) * 128 + (d % 16) * 8 + (p%32 // 16) * 4 + p % 4
"""
import numpy as np

PAGE_TOKENS = 32


def k_offsets(tokens, head_dim):
    """Offsets within one head's run for K elements [tokens, head_dim]."""
    p = np.arange(tokens)[:, None]
    d = np.arange(head_dim)[None, :]
    q = p % PAGE_TOKENS
    return ((p // PAGE_TOKENS) * PAGE_TOKENS * head_dim + (q // 16) * 16 * head_dim
            + (d // 8) * 128 + (q % 16) * 8 + d % 8)


def v_offsets(tokens, head_dim):
    """Offsets within one head's run for V elements [tokens, head_dim]."""
    p = np.arange(tokens)[:, None]
    d = np.arange(head_dim)[None, :]
    q = p % PAGE_TOKENS
    return ((p // PAGE_TOKENS) * PAGE_TOKENS * head_dim + (d // 16) * 512
            + ((q // 4) % 4) * 128 + (d % 16) * 8 + (q // 16) * 4 + q % 4)


def to_pages(rows, capacity, value=False, fill=0):
    """Token-major [n, kv_heads, D] array -> flat page array [kv_heads*capacity*D]."""
    n, kv_heads, head_dim = rows.shape
    pages = np.full(kv_heads * capacity * head_dim, fill, dtype=rows.dtype)
    off = (v_offsets if value else k_offsets)(n, head_dim)
    for h in range(kv_heads):
        pages[h * capacity * head_dim + off] = rows[:, h, :]
    return pages


def from_pages(pages, n, kv_heads, head_dim, capacity, value=False):
    """Flat page array -> token-major [n, kv_heads, D]."""
    off = (v_offsets if value else k_offsets)(n, head_dim)
    rows = np.empty((n, kv_heads, head_dim), dtype=pages.dtype)
    for h in range(kv_heads):
        rows[:, h, :] = pages[h * capacity * head_dim + off]
    return rows
