"""C-ABI checks that need no GPU: the header compiles as C11 with -Werror and
keeps the reference's prototypes (tests/test_native_abi.py:11-29 of the
reference), the library exports every declared symbol, and argument
validation rejects bad calls before any buffer is read or any HIP call is made
(tests/test_cuda.py:72-87)."""
import ctypes as ct
import math
import re
import shutil
import subprocess

import pytest

from redshift_amd.runtime import DEFAULT_LIBRARY, QV_BF16, QV_F16, QV_F32

from conftest import ROOT

HEADER = ROOT / 'include' / 'runtime.h'


def declared_functions():
    text = re.sub(r'/\*.*?\*/', '', HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r'\b(qv_\w+)\s*\(', text)))


@pytest.mark.skipif(not shutil.which('cc'), reason='a C compiler is required')
def test_public_header_is_usable_from_c(tmp_path):
    source = '''
#include "runtime.h"
int main(void) {
    const char *(*error)(void) = qv_error;
    int (*mm)(float *, const void *, const float *, int, int, int, int) = qv_test_mm;
    int (*norm)(float *, const float *, const float *, int, int, float) = qv_test_norm;
    int (*verify)(void *, const int *, int, float *) = qv_verify;
    int (*commit)(void *, int) = qv_commit;
    int (*attention)(float *, void *, void *, const float *, const float *, const float *,
                     const float *, const float *, int, int, float) = qv_test_attention;
    int (*raw)(void *, const void *, const void *, const void *, int, int, int, int, int, int,
               int, int, float, void *, uint64_t, void *) = qv_attention;
    int out_types = QV_F16 + QV_BF16 + QV_F32;
    return error == 0 || mm == 0 || norm == 0 || verify == 0 || commit == 0 ||
           attention == 0 || raw == 0 || out_types != 6;
}
'''
    path = tmp_path / 'abi.c'
    path.write_text(source)
    result = subprocess.run(['cc', '-std=c11', '-Wall', '-Wextra', '-Werror', '-fsyntax-only',
                             f'-I{HEADER.parent}', str(path)], capture_output=True, text=True)
    assert result.returncode == 0, result.stderr


def test_library_exports_every_declared_function(lib):
    names = declared_functions()
    assert 'qv_test_attention' in names and 'qv_attention' in names
    for name in names:
        assert hasattr(lib, name), name
    # the reference loader's required set (qvelox/runtime.py:18-21)
    for name in ('qv_error', 'qv_test_mm', 'qv_test_mm_fast', 'qv_test_norm', 'qv_test_delta',
                 'qv_test_attention'):
        assert hasattr(lib, name)


def test_library_is_built_for_gfx950_only():
    text = subprocess.run(['strings', str(DEFAULT_LIBRARY)], capture_output=True, text=True).stdout
    targets = set(re.findall(r'amdgcn-amd-amdhsa--(gfx\w+)', text))
    assert targets == {'gfx950'}, targets


def floats(values):
    return (ct.c_float * len(values))(*values)


def test_rejects_invalid_attention_arguments_before_accessing_buffers(lib):
    value = floats([1.])
    # tests/test_cuda.py:85 of the reference: batch 8 at position 139257 overflows.
    assert lib.qv_test_attention(*([value] * 8), 8, 139257, 1e-6) == -1
    assert lib.qv_error() == b'attention context exceeds 139264'
    for batch in (0, 9, -1):
        assert lib.qv_test_attention(*([value] * 8), batch, 0, 1e-6) == -1
        assert lib.qv_error() == b'batch must be between 1 and 8'
    for epsilon in (0., -1., math.nan, math.inf):
        assert lib.qv_test_attention(*([value] * 8), 1, 0, epsilon) == -1
        assert lib.qv_error() == b'epsilon must be finite and positive'
    assert lib.qv_test_attention(*([value] * 8), 1, -1, 1e-6) == -1
    assert lib.qv_error() == b'attention context exceeds 139264'
    for i in range(8):
        args = [value] * 8
        args[i] = None
        assert lib.qv_test_attention(*args, 1, 0, 1e-6) == -1
        assert lib.qv_error() == b'null attention buffer'
    # batch is checked before epsilon, epsilon before position (src/runtime.cu:172-174)
    assert lib.qv_test_attention(*([value] * 8), 9, 139264, math.nan) == -1
    assert lib.qv_error() == b'batch must be between 1 and 8'
    assert lib.qv_test_attention(*([value] * 8), 1, 139264, math.nan) == -1
    assert lib.qv_error() == b'epsilon must be finite and positive'


def test_out_of_path_entry_points_fail_with_a_message(lib):
    value = floats([1.])
    assert lib.qv_test_mm(value, value, value, 8, 1, 32, 1) == -1
    assert b'not part of libredshift_hip' in lib.qv_error()
    assert lib.qv_test_mm_fast(value, value, value, 8, 1, 32, 1) == -1
    assert lib.qv_test_norm(value, value, value, 1, 1, 1e-6) == -1
    assert lib.qv_test_delta(*([value] * 11), 1, 1, 1, 32, 1e-6) == -1
    handle = ct.c_void_p(1234)
    assert lib.qv_create(ct.byref(handle), b'model.gguf', 2048, 1e-6) == -1
    assert handle.value is None
    assert lib.qv_commit(None, 0) == -1 and lib.qv_error()
    lib.qv_destroy(None)


def test_kv_bytes_and_geometry_validation(lib):
    size = ct.c_uint64()
    assert lib.qv_kv_bytes(ct.byref(size), 4, 256, 139264) == 0
    assert size.value == 4 * 139264 * 256 * 2
    assert lib.qv_error() == b''
    assert lib.qv_kv_bytes(ct.byref(size), 4, 256, 100) == -1
    assert b'multiple of 32' in lib.qv_error()
    assert lib.qv_kv_bytes(ct.byref(size), 4, 192, 128) == -1
    assert b'head_dim' in lib.qv_error()
    assert lib.qv_kv_bytes(None, 4, 256, 128) == -1


def test_device_entry_points_validate_before_touching_the_device(lib):
    p = ct.c_void_p(4096)   # never dereferenced: every call below fails validation
    ws = ct.c_uint64(1 << 20)
    args = dict(q_heads=24, kv_heads=4, head_dim=256, tokens=1, position=4095, capacity=4096)

    def call(dtype=QV_F16, out_dtype=None, scale=0.0625, out=p, **kw):
        a = {**args, **kw}
        return lib.qv_attention(out, p, p, p, dtype, dtype if out_dtype is None else out_dtype,
                                a['q_heads'], a['kv_heads'], a['head_dim'], a['tokens'],
                                a['position'], a['capacity'], scale, p, ws, None)

    assert call(dtype=7) == -1 and b'dtype' in lib.qv_error()
    assert call(dtype=QV_F32) == -1 and b'dtype must be QV_F16 or QV_BF16' in lib.qv_error()
    assert call(dtype=QV_F16, out_dtype=QV_BF16) == -1 and b'out_dtype' in lib.qv_error()
    assert call(q_heads=25) == -1 and b'multiple of kv_heads' in lib.qv_error()
    assert call(head_dim=64) == -1 and b'head_dim' in lib.qv_error()
    assert call(tokens=0) == -1 and b'tokens' in lib.qv_error()
    assert call(position=4096) == -1 and b'capacity' in lib.qv_error()
    assert call(capacity=4100) == -1 and b'multiple of 32' in lib.qv_error()
    assert call(scale=math.inf) == -1 and b'scale' in lib.qv_error()
    assert call(out=None) == -1 and lib.qv_error() == b'null attention buffer'
    assert call(out=ct.c_void_p(4098)) == -1 and b'aligned' in lib.qv_error()
    assert call(dtype=QV_BF16, q_heads=24 * 17, kv_heads=1) == -1 and b'48 query heads' in lib.qv_error()
    rows = 2 ** 28 // 48 + 1      # q_heads*tokens past 2^28 (32-bit row and launch arithmetic)
    assert call(q_heads=48, kv_heads=1, tokens=rows, position=0, capacity=-(-rows // 32) * 32) == -1
    assert b'2^28' in lib.qv_error()
    assert lib.qv_kv_pack(p, p, p, p, 4, 256, 128, 100, 29, None) == -1
    assert b'capacity' in lib.qv_error()
    assert lib.qv_kv_pack(p, None, None, p, 4, 256, 128, 0, 1, None) == -1
    assert lib.qv_kv_copy(p, p, p, p, 4, 256, 64, 4096, 65, None) == -1
    assert b'capacity' in lib.qv_error()
    assert lib.qv_kv_copy(p, p, p, p, 4, 256, 100, 4096, 10, None) == -1
    assert b'multiple of 32' in lib.qv_error()
    assert lib.qv_kv_copy(p, None, p, p, 4, 256, 64, 4096, 10, None) == -1
    assert lib.qv_error() == b'null KV cache'
    assert lib.qv_kv_copy(p, p, p, p, 4, 256, 64, 4096, -1, None) == -1
    assert b'non-negative' in lib.qv_error()
    # The device fused entry also takes prefill chunks, up to 8192 tokens.
    assert lib.qv_attention_fused(*([p] * 8), 8193, 0, 16384, 1e-6, p, ws, None) == -1
    assert lib.qv_error() == b'batch must be between 1 and 8192'
    assert lib.qv_attention_fused(*([p] * 8), 0, 0, 128, 1e-6, p, ws, None) == -1
    assert lib.qv_error() == b'batch must be between 1 and 8192'
    assert lib.qv_attention_fused(*([p] * 8), 100, 0, 64, 1e-6, p, ws, None) == -1
    assert b'capacity' in lib.qv_error()
    assert lib.qv_attention_fused(*([p] * 8), 100, 139200, 139264, 1e-6, p, ws, None) == -1
    assert b'139264' in lib.qv_error()
    # Every device buffer of the fused entry is 16-byte aligned (the prefill
    # chunk stores 16-byte vectors to out; the verification kernels read the
    # query, the norm weights and the new keys and values 16 bytes at a time).
    assert lib.qv_attention_fused(ct.c_void_p(4100), *([p] * 7), 100, 0, 128, 1e-6, p, ws, None) == -1
    assert b'aligned' in lib.qv_error()
    for i in range(3, 8):   # q_gate, key, value, q_norm, k_norm
        args = [p] * 8
        args[i] = ct.c_void_p(4100)
        assert lib.qv_attention_fused(*args, 8, 1000, 1024, 1e-6, p, ws, None) == -1
        assert b'aligned' in lib.qv_error()


def test_front_end_rejects_mismatched_tensors(lib):
    """The torch front end checks what the untyped C ABI cannot see (dtype,
    shape and device of every tensor) before any library call."""
    import torch
    import redshift_amd.attention as A
    cache = A.PagedKV(4, 256, 64, torch.float16, device='cpu')
    q = torch.zeros((1, 24, 256), dtype=torch.float16)
    with pytest.raises(ValueError, match='the cache holds'):
        A.attention(q.to(torch.bfloat16), cache, 0, 1 / 16)
    with pytest.raises(ValueError, match='head_dim'):
        A.attention(torch.zeros((1, 24, 128), dtype=torch.float16), cache, 0, 1 / 16)
    with pytest.raises(ValueError, match=r'\[tokens, q_heads, head_dim\]'):
        A.attention(torch.zeros((24, 256), dtype=torch.float16), cache, 0, 1 / 16)
    with pytest.raises(ValueError, match='shape of q'):
        A.attention(q, cache, 0, 1 / 16, out=torch.zeros((2, 24, 256), dtype=torch.float16))
    with pytest.raises(ValueError, match='or float32'):
        A.attention(q, cache, 0, 1 / 16, out=torch.zeros((1, 24, 256), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match='K and V rows'):
        cache.pack(torch.zeros((2, 4, 256)), torch.zeros((3, 4, 256)))
    with pytest.raises(ValueError, match='fp16 PagedKV'):
        A.attention_fused(*([None] * 5), A.PagedKV(4, 256, 64, torch.bfloat16, device='cpu'), 0, 1e-6)
    inputs = [torch.zeros(s) for s in ((1, 24, 512), (1, 4, 256), (1, 4, 256), (256,), (256,))]
    with pytest.raises(ValueError, match='q_gate must be float32'):
        A.attention_fused(inputs[0].half(), *inputs[1:], cache, 0, 1e-6)
    with pytest.raises(ValueError, match='value must hold'):
        A.attention_fused(*inputs[:2], torch.zeros((2, 4, 256)), *inputs[3:], cache, 0, 1e-6)


def test_build_refuses_scratch_in_kernels_with_untracked_loads():
    """redshift_amd.build reads the compiler's resource remarks of ring.hip
    and prefill.hip and fails on scratch or VGPR spills in the kernels whose
    operands arrive through untracked asm loads; a compile without remarks
    fails too, so the check cannot pass by not running."""
    from redshift_amd.build import RESOURCE_REMARKS, check_no_scratch

    def remarks(name, scratch, spills):
        tag = f' [{RESOURCE_REMARKS}]'
        return '\n'.join(f'prefill.hip:1:1: remark: {line}{tag}' for line in (
            f'Function Name: {name}', '    VGPRs: 168', f'    ScratchSize [bytes/lane]: {scratch}',
            f'    VGPRs Spill: {spills}'))

    kernel = '_ZN2rs12_GLOBAL__N_122attention_prefill_bf16ILi256ELi0ELi192EEEvNS0_11PrefillArgsE'
    other = '_ZN2rs12_GLOBAL__N_115combine_prefillILi256EfLi2ELi8EEEvNS0_18CombinePrefillArgsE'
    assert check_no_scratch('prefill.hip', 'a warning\n' + remarks(kernel, 0, 0)) == 'a warning'
    assert check_no_scratch('prefill.hip', remarks(kernel, 0, 0) + '\n' + remarks(other, 16, 4)) == ''
    with pytest.raises(RuntimeError, match='ScratchSize'):
        check_no_scratch('prefill.hip', remarks(kernel, 28, 0))
    with pytest.raises(RuntimeError, match='VGPRs Spill 6'):
        check_no_scratch('ring.hip', remarks(kernel.replace('prefill_bf16', 'ring'), 0, 6))
    with pytest.raises(RuntimeError, match='did not run'):
        check_no_scratch('ring.hip', 'no remarks at all')
