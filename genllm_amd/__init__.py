"""genllm_amd -- MI355X (gfx950) paged KV-cache attention for Genllm.

The product is libgenllm_hip.so (HIP kernels + the C ABI of
include/genllm_paged.h); this package builds and binds it.  ``genllm_amd.paged``
holds the Python face of the operator interface.
"""
from .build import build_library  # noqa: F401

__version__ = "0.1.0"
