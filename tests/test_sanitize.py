"""The host-sanitizer gate: tests/native/abi_sanitize, the library's sources
built with AddressSanitizer and UndefinedBehaviorSanitizer on the host side
(redshift_amd.build.build_sanitizer), driving every entry point of
include/runtime.h.  The reference gates its kernel tests with
compute-sanitizer memcheck and racecheck (Makefile:23-26); device code has no
sanitizer here, so the gate covers the host half: validation and its
messages, size and split-plan arithmetic over int32 extremes, and host
buffers of exactly the documented sizes for qv_test_attention.
"""
import subprocess

import pytest

from redshift_amd.build import SANITIZE_BINARY


def run_driver(args, timeout):
    assert SANITIZE_BINARY.exists(), f'{SANITIZE_BINARY} is missing: run redshift_amd.build.build_sanitizer()'
    print(f'running {SANITIZE_BINARY.name} {" ".join(args)}', flush=True)
    result = subprocess.run([str(SANITIZE_BINARY), *args], capture_output=True, text=True, timeout=timeout)
    print(result.stdout[-2000:], result.stderr[-4000:], flush=True)
    return result


def test_host_half_under_sanitizers():
    """Validation, stubs, qv_kv_bytes and the split planner: no device."""
    result = run_driver(['--host-only'], timeout=240)
    assert result.returncode == 0, result.stderr[-4000:]
    assert ' 0 failed' in result.stdout


@pytest.mark.gpu
def test_device_calls_under_sanitizers(gpu):
    """Every entry point called for real on the GPU (null and created
    streams) with the host code under the sanitizers."""
    result = run_driver([], timeout=240)
    assert result.returncode == 0, result.stderr[-4000:]
    assert 'running device checks' in result.stdout and ' 0 failed' in result.stdout
