"""redshift_amd: the full-attention path of the qvelox/Redshift runtime for
AMD Instinct MI355X (gfx950).

The product is ``lib/libredshift_hip.so`` (HIP kernels + C ABI, built by
``redshift_amd.build``).  ``runtime.load_library`` is the ctypes loader with the
reference's signatures; ``attention`` wraps the device ABI for torch tensors;
``workloads`` generates the seeded synthetic inputs; ``layout`` describes the
KV page layout on the host.
"""
from .runtime import DEFAULT_LIBRARY, load_library  # noqa: F401

__all__ = ['DEFAULT_LIBRARY', 'load_library']
