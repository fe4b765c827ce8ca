"""Build libredshift_hip.so in-tree with hipcc for gfx950 only.

Usage: ``python -m redshift_amd.build`` (or ``__graft_entry__.build()``).
Objects go to ``redshift_amd/_build/``, the library to
``redshift_amd/lib/libredshift_hip.so``.  Every call recompiles.
"""
import hashlib
import json
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
SOURCES = ['abi.cpp', 'attention.hip', 'kv.hip', 'prefill.hip', 'ring.hip', 'short.hip']
LIBRARY = PACKAGE / 'lib' / 'libredshift_hip.so'
# Measurement probes for bench.py (a plain read of a launch's KV pages), kept
# out of the attention library.
PROBE_SOURCES = ['probe.hip']
PROBE_LIBRARY = PACKAGE / 'lib' / 'libredshift_probe.so'
# The commit the library was built from and the library's SHA-256, written
# beside it by build(), for trees copied without their .git (bench.py's
# provenance).
BUILD_INFO = PACKAGE / 'lib' / 'build_info.json'
ARCH = 'gfx950'
# The host-sanitizer gate: the library's sources and a driver over its C ABI,
# with AddressSanitizer and UndefinedBehaviorSanitizer on the host code only
# (every -fsanitize flag goes to the host pass; the device code is the
# ordinary gfx950 build).
SANITIZE_DRIVER = ROOT / 'tests' / 'native' / 'abi_sanitize.cpp'
SANITIZE_BINARY = ROOT / 'tests' / 'native' / 'abi_sanitize'
SANITIZE_FLAGS = [
    '-Xarch_host', '-fsanitize=address', '-Xarch_host', '-fsanitize=undefined',
    '-Xarch_host', '-fno-sanitize-recover=undefined', '-Xarch_host', '-fno-omit-frame-pointer',
    '-Xarch_host', '-g',
]

# Packed-FP32 instructions are kept out of every code object: hipcc would
# otherwise form v_pk_{add,mul,fma}_f32 from ordinary float code.
COMMON_FLAGS = [
    '-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}',
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Wall', '-Wno-unused-result',
    f'-I{ROOT / "include"}', f'-I{PACKAGE / "csrc"}',
]


# Per-source flags.  ring.hip and prefill.hip keep MFMA accumulators in
# architectural VGPRs: with AGPR accumulators the compiler copies them out
# and back on every page (for the rarely taken softmax rescale).
SOURCE_FLAGS = {name: ['-mllvm', '-amdgpu-mfma-vgpr-form'] for name in ('ring.hip', 'prefill.hip')}
# No operation in prefill.hip makes a NaN from its valid inputs: keys are
# masked to -inf and stale V slots zeroed explicitly, and every exponent is
# taken against a finite reference point (0 while a row has seen no key), so
# -inf - (-inf) never occurs.  Its maxima then need no NaN quieting.
SOURCE_FLAGS['prefill.hip'] = SOURCE_FLAGS['prefill.hip'] + ['-fno-honor-nans']


# Kernels whose MFMA operand registers are filled by asm loads that the
# compiler does not track (lds.hpp: global_load16 and lds_read; ring.hip:
# global_load4), each followed later by an explicit wait.  A spill or copy
# of such a register between the load and its wait would hand stale values
# to the matrix cores, so the build fails if any of them uses scratch: the
# compiler's resource remarks give every kernel's scratch bytes and spills.
UNTRACKED_LOAD_SOURCES = ('ring.hip', 'prefill.hip')
UNTRACKED_LOAD_KERNELS = ('attention_ring', 'attention_prefill')
RESOURCE_REMARKS = '-Rpass-analysis=kernel-resource-usage'


def check_no_scratch(name, stderr):
    """Parses the resource remarks of one source's compile; raises if a
    kernel that uses untracked loads has scratch or VGPR spills.  Returns the
    messages without the remarks."""
    kernel, checked, bad, rest = None, 0, [], []
    for line in stderr.splitlines():
        if 'remark:' not in line or RESOURCE_REMARKS not in line:
            rest.append(line)
            continue
        text = line.split('remark:', 1)[1].split('[-Rpass', 1)[0].strip()
        key, _, value = text.partition(':')
        key, value = key.strip(), value.strip()
        if key == 'Function Name':
            kernel = value if any(k in value for k in UNTRACKED_LOAD_KERNELS) else None
            checked += kernel is not None
        elif kernel and key in ('ScratchSize [bytes/lane]', 'VGPRs Spill') and value != '0':
            bad.append(f'{kernel}: {key} {value}')
    if bad:
        raise RuntimeError(f'{name}: kernels with untracked loads use scratch:\n' + '\n'.join(bad))
    if not checked:
        raise RuntimeError(f'{name}: no resource remarks for its kernels; the scratch check did not run')
    return '\n'.join(rest)


def hipcc():
    path = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not Path(path).exists():
        raise RuntimeError('hipcc not found: the HIP toolchain is required to build libredshift_hip')
    return path


def _run(cmd):
    result = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 target feature; that
    # warning is expected and dropped.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    stderr = '\n'.join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f'command failed ({result.returncode}): {" ".join(cmd)}\n{stderr}')
    return stderr


def _compile_all(objdir, sources, extra, jobs):
    """Compile (name, path) sources into objdir in parallel; returns the
    objects and the compilers' messages."""
    compiler = hipcc()
    objdir.mkdir(parents=True, exist_ok=True)

    def compile_one(item):
        name, src = item
        obj = objdir / (name + '.o')
        checked = name in UNTRACKED_LOAD_SOURCES
        cmd = [compiler, '-x', 'hip', *COMMON_FLAGS, *SOURCE_FLAGS.get(name, []), *extra,
               *([RESOURCE_REMARKS] if checked else []), '-c', str(src), '-o', str(obj)]
        stderr = _run(cmd)
        return obj, check_no_scratch(name, stderr) if checked else stderr

    jobs = jobs or min(len(sources), os.cpu_count() or 1)
    with ThreadPoolExecutor(jobs) as pool:
        return list(pool.map(compile_one, sources))


def _link(objects, library):
    library.parent.mkdir(exist_ok=True)
    tmp = library.with_suffix('.so.tmp')
    _run([hipcc(), '-shared', '-fPIC', f'--offload-arch={ARCH}', *[str(o) for o in objects], '-o', str(tmp)])
    os.replace(tmp, library)


def build(verbose=False, jobs=None):
    """Compile every source and link the shared library (and the probe
    library beside it); returns the attention library's path."""
    names = SOURCES + PROBE_SOURCES
    results = _compile_all(PACKAGE / '_build', [(name, PACKAGE / 'csrc' / name) for name in names], [], jobs)
    for _, stderr in results:
        if verbose and stderr:
            print(stderr, file=sys.stderr)
    objects = dict(zip(names, (o for o, _ in results)))
    _link([objects[name] for name in SOURCES], LIBRARY)
    _link([objects[name] for name in PROBE_SOURCES], PROBE_LIBRARY)
    BUILD_INFO.write_text(json.dumps({'git_head': git_head(),
                                      'library_sha256': hashlib.sha256(LIBRARY.read_bytes()).hexdigest()}) + '\n')
    return LIBRARY


def git_head(root=ROOT):
    """The checked-out commit, read from .git as plain files (None where the
    tree was copied without it)."""
    try:
        head = (root / '.git' / 'HEAD').read_text().strip()
        if head.startswith('ref: '):
            ref = head[5:]
            path = root / '.git' / ref
            if path.exists():
                return path.read_text().strip()
            for line in (root / '.git' / 'packed-refs').read_text().splitlines():
                if line.endswith(' ' + ref):
                    return line.split()[0]
            return None
        return head
    except OSError:
        return None


def build_sanitizer(verbose=False, jobs=None):
    """Link the host-sanitizer driver with a sanitized build of every source;
    returns the executable's path."""
    sources = [(name, PACKAGE / 'csrc' / name) for name in SOURCES]
    sources.append((SANITIZE_DRIVER.name, SANITIZE_DRIVER))
    results = _compile_all(PACKAGE / '_build' / 'sanitize', sources, SANITIZE_FLAGS, jobs)
    for _, stderr in results:
        if verbose and stderr:
            print(stderr, file=sys.stderr)
    tmp = SANITIZE_BINARY.with_name(SANITIZE_BINARY.name + '.tmp')
    _run([hipcc(), f'--offload-arch={ARCH}', *SANITIZE_FLAGS[:4], *[str(o) for o, _ in results],
          '-o', str(tmp)])
    os.replace(tmp, SANITIZE_BINARY)
    return SANITIZE_BINARY


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv))
    print(build_sanitizer(verbose='-v' in sys.argv))
