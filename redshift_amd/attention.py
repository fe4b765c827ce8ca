"""Torch-tensor front end for the device ABI of libredshift_hip.

torch only supplies device memory and the stream; every computation runs in
the HIP library.  All calls are stream-ordered on torch's current stream.
"""
import ctypes as ct

import torch

from .runtime import QV_BF16, QV_F16, QV_F32, check, library

PAGE_TOKENS = 32
# Query rows (group * tokens) per KV head that one split/combine pair serves.
MAX_CHUNK_ROWS = 48


def dtype_code(dtype):
    if dtype == torch.float16:
        return QV_F16
    if dtype == torch.bfloat16:
        return QV_BF16
    raise ValueError(f'unsupported KV dtype {dtype}: use float16 or bfloat16')


def out_code(dtype):
    """Output type code: the input's 16-bit type or float32."""
    return QV_F32 if dtype == torch.float32 else dtype_code(dtype)


def round_capacity(tokens):
    """Smallest page-aligned capacity holding `tokens` tokens."""
    return -(-tokens // PAGE_TOKENS) * PAGE_TOKENS


def _stream():
    return ct.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ct.c_void_p(t.data_ptr())


def _require(condition, message):
    if not condition:
        raise ValueError(message)


def _same_device(tensors, device):
    for name, t in tensors:
        _require(t.device == device, f'{name} is on {t.device}, the cache on {device}')


def _nbytes(t):
    return t.numel() * t.element_size()


class PagedKV:
    """K and V caches of one attention layer in the library's page layout:
    per KV head, `capacity` tokens in 32-token pages (include/runtime.h)."""

    def __init__(self, kv_heads, head_dim, capacity, dtype=torch.float16, device='cuda'):
        lib = library()
        size = ct.c_uint64()
        check(lib, lib.qv_kv_bytes(ct.byref(size), kv_heads, head_dim, capacity))
        self.kv_heads, self.head_dim, self.capacity, self.dtype = kv_heads, head_dim, capacity, dtype
        self.k = torch.empty(size.value // 2, dtype=dtype, device=device)
        self.v = torch.empty(size.value // 2, dtype=dtype, device=device)

    def pack(self, k_rows, v_rows, first=0):
        """Write token-major rows [count][kv_heads][head_dim] at tokens first..."""
        lib = library()
        shape = (self.kv_heads, self.head_dim)
        _require(k_rows.dim() == 3 and k_rows.shape == v_rows.shape and tuple(k_rows.shape[1:]) == shape,
                 f'K and V rows must both be [count, {shape[0]}, {shape[1]}]')
        _same_device([('k_rows', k_rows), ('v_rows', v_rows)], self.k.device)
        k_rows = k_rows.to(self.dtype).contiguous()
        v_rows = v_rows.to(self.dtype).contiguous()
        check(lib, lib.qv_kv_pack(_ptr(self.k), _ptr(self.v), _ptr(k_rows), _ptr(v_rows),
                                  self.kv_heads, self.head_dim, self.capacity, first,
                                  k_rows.shape[0], _stream()))
        return self

    def unpack(self, first, count):
        """Token-major copies [count][kv_heads][head_dim] of tokens first..."""
        lib = library()
        k_rows = torch.empty((count, self.kv_heads, self.head_dim), dtype=self.dtype, device=self.k.device)
        v_rows = torch.empty_like(k_rows)
        check(lib, lib.qv_kv_unpack(_ptr(k_rows), _ptr(v_rows), _ptr(self.k), _ptr(self.v),
                                    self.kv_heads, self.head_dim, self.capacity, first, count,
                                    _stream()))
        return k_rows, v_rows


def attention_workspace_bytes(q_heads, kv_heads, head_dim, tokens, position):
    lib = library()
    size = ct.c_uint64()
    check(lib, lib.qv_attention_workspace(ct.byref(size), q_heads, kv_heads, head_dim, tokens, position))
    return size.value


def workspace(nbytes, device='cuda'):
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def attention(q, cache, position, scale, out=None, ws=None, out_dtype=None):
    """Raw causal GQA attention: q [tokens][q_heads][head_dim] (cache dtype),
    row t sees keys 0..position+t of `cache` (a PagedKV).  The output has
    q's dtype, or float32 when out_dtype (or out's dtype) says so."""
    lib = library()
    _check_query(q, cache)
    q = q.contiguous()
    tokens, q_heads, head_dim = q.shape
    if out is None:
        out = torch.empty(q.shape, dtype=out_dtype or q.dtype, device=q.device)
    _check_output(out, q)
    if ws is None:
        ws = workspace(attention_workspace_bytes(q_heads, cache.kv_heads, head_dim, tokens, position), q.device)
    _same_device([('workspace', ws)], cache.k.device)
    check(lib, lib.qv_attention(_ptr(out), _ptr(q), _ptr(cache.k), _ptr(cache.v), dtype_code(q.dtype),
                                out_code(out.dtype), q_heads, cache.kv_heads, head_dim, tokens,
                                position, cache.capacity, float(scale), _ptr(ws), _nbytes(ws),
                                _stream()))
    return out


def precise_workspace_bytes(q_heads, kv_heads, head_dim, tokens, position):
    lib = library()
    size = ct.c_uint64()
    check(lib, lib.qv_attention_precise_workspace(ct.byref(size), q_heads, kv_heads, head_dim, tokens, position))
    return size.value


def attention_precise(q, cache, position, scale, out=None, ws=None):
    """Raw causal GQA attention at the reference's precision: a float32
    query [tokens][q_heads][head_dim] on an fp16 cache, float32 output
    (qv_attention_precise; the library splits q into fp16 hi + lo parts)."""
    lib = library()
    _require(q.dim() == 3, 'q must be [tokens, q_heads, head_dim]')
    _require(q.dtype == torch.float32, f'q must be float32, not {q.dtype}')
    _require(cache.dtype == torch.float16, 'the precise path runs on an fp16 cache')
    _require(q.shape[2] == cache.head_dim, f'q has head_dim {q.shape[2]}, the cache {cache.head_dim}')
    _same_device([('q', q)], cache.k.device)
    q = q.contiguous()
    tokens, q_heads, head_dim = q.shape
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    _require(tuple(out.shape) == tuple(q.shape) and out.dtype == torch.float32 and out.is_contiguous(),
             f'out must be a contiguous float32 tensor of shape {tuple(q.shape)}')
    _same_device([('out', out)], q.device)
    if ws is None:
        ws = workspace(precise_workspace_bytes(q_heads, cache.kv_heads, head_dim, tokens, position), q.device)
    _same_device([('workspace', ws)], cache.k.device)
    check(lib, lib.qv_attention_precise(_ptr(out), _ptr(q), _ptr(cache.k), _ptr(cache.v), q_heads,
                                        cache.kv_heads, head_dim, tokens, position, cache.capacity,
                                        float(scale), _ptr(ws), _nbytes(ws), _stream()))
    return out


def attention_noalloc(q, cache, position, scale, out=None, out_dtype=None):
    """`attention` without a workspace: qv_attention_noalloc keeps the
    split-K partials in the library's static device array (serialise calls
    on one GPU)."""
    lib = library()
    _check_query(q, cache)
    q = q.contiguous()
    tokens, q_heads, head_dim = q.shape
    if out is None:
        out = torch.empty(q.shape, dtype=out_dtype or q.dtype, device=q.device)
    _check_output(out, q)
    check(lib, lib.qv_attention_noalloc(_ptr(out), _ptr(q), _ptr(cache.k), _ptr(cache.v), dtype_code(q.dtype),
                                        out_code(out.dtype), q_heads, cache.kv_heads, head_dim, tokens,
                                        position, cache.capacity, float(scale), _stream()))
    return out


def _check_query(q, cache):
    """The query must be [tokens, q_heads, head_dim] of the cache's 16-bit
    type on the cache's device (the library sees untyped pointers)."""
    _require(q.dim() == 3, 'q must be [tokens, q_heads, head_dim]')
    _require(q.dtype == cache.dtype, f'q is {q.dtype}, the cache holds {cache.dtype}')
    _require(q.shape[2] == cache.head_dim, f'q has head_dim {q.shape[2]}, the cache {cache.head_dim}')
    _same_device([('q', q)], cache.k.device)


def _check_output(out, q):
    _require(tuple(out.shape) == tuple(q.shape), f'out must have the shape of q, {tuple(q.shape)}')
    _require(out.dtype in (q.dtype, torch.float32), f'out must be {q.dtype} or float32, not {out.dtype}')
    _require(out.is_contiguous(), 'out must be contiguous')
    _same_device([('out', out)], q.device)


def attention_split(q, cache, position, scale, ws):
    """Phase 1 of `attention` for one chunk (split-K partials into ws)."""
    lib = library()
    _check_query(q, cache)
    q = q.contiguous()
    tokens, q_heads, head_dim = q.shape
    _same_device([('workspace', ws)], cache.k.device)
    check(lib, lib.qv_attention_split(_ptr(q), _ptr(cache.k), _ptr(cache.v), dtype_code(q.dtype),
                                      q_heads, cache.kv_heads, head_dim, tokens, position,
                                      cache.capacity, float(scale), _ptr(ws), _nbytes(ws), _stream()))


def attention_combine(out, cache, position, ws):
    """Phase 2 of `attention` for one chunk (log-sum-exp combine into out)."""
    lib = library()
    _require(out.dim() == 3 and out.shape[2] == cache.head_dim, 'out must be [tokens, q_heads, head_dim]')
    _require(out.dtype in (cache.dtype, torch.float32), f'out must be {cache.dtype} or float32')
    _require(out.is_contiguous(), 'out must be contiguous')
    _same_device([('out', out), ('workspace', ws)], cache.k.device)
    tokens, q_heads, head_dim = out.shape
    check(lib, lib.qv_attention_combine(_ptr(out), dtype_code(cache.dtype), out_code(out.dtype), q_heads,
                                        cache.kv_heads, head_dim, tokens, position, _ptr(ws),
                                        _nbytes(ws), _stream()))


def fused_workspace_bytes(batch, position):
    lib = library()
    size = ct.c_uint64()
    check(lib, lib.qv_attention_fused_workspace(ct.byref(size), batch, position))
    return size.value


def check_fused_inputs(q_gate, key, value, q_norm, k_norm, cache):
    """The fused entry's tensors: float32 q_gate [batch][24][512], key and
    value [batch][4][256], q_norm and k_norm [256] on the device of `cache`,
    an fp16 PagedKV(4, 256, ...).  Returns the named tensors."""
    _require((cache.dtype, cache.kv_heads, cache.head_dim) == (torch.float16, 4, 256),
             'the fused path runs on an fp16 PagedKV(4, 256, ...)')
    batch = q_gate.shape[0]
    shapes = {'q_gate': (batch, 24, 512), 'key': (batch, 4, 256), 'value': (batch, 4, 256),
              'q_norm': (256,), 'k_norm': (256,)}
    named = list(zip(shapes, (q_gate, key, value, q_norm, k_norm)))
    for name, t in named:
        _require(t.dtype == torch.float32, f'{name} must be float32, not {t.dtype}')
        _require(t.numel() == torch.Size(shapes[name]).numel(),
                 f'{name} must hold {shapes[name]} values, not {tuple(t.shape)}')
    _same_device(named, cache.k.device)
    return named


def _aligned16(t):
    """t as a contiguous tensor whose data starts on a 16-byte boundary (the
    device ABI's requirement): t itself when it already is one, else a copy."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def attention_fused(q_gate, key, value, q_norm, k_norm, cache, position, epsilon, out=None, ws=None):
    """Device-side fused attention of the fixed 24/4/256 model (the reference's
    k_attention): prepares q/k, appends k/v at position.., attends and gates.
    All inputs float32 device tensors; `cache` is an fp16 PagedKV(4, 256, ...)."""
    lib = library()
    named = check_fused_inputs(q_gate, key, value, q_norm, k_norm, cache)
    batch = q_gate.shape[0]
    if out is None:
        out = torch.empty((batch, 24, 256), dtype=torch.float32, device=q_gate.device)
    _require(out.dtype == torch.float32 and out.numel() == batch * 24 * 256 and out.is_contiguous(),
             'out must be a contiguous float32 [batch, 24, 256]')
    if ws is None:
        ws = workspace(fused_workspace_bytes(batch, position), q_gate.device)
    _same_device([('out', out), ('workspace', ws)], cache.k.device)
    tensors = [_aligned16(t) for _, t in named]
    check(lib, lib.qv_attention_fused(_ptr(out), _ptr(cache.k), _ptr(cache.v),
                                      *[_ptr(t) for t in tensors], batch, position, cache.capacity,
                                      float(epsilon), _ptr(ws), _nbytes(ws), _stream()))
    return out
