"""MI355X-native (gfx950) paged-decode attention for xLLM.

libxllm_hip_backend.so (built from xllms_amd/csrc) is the product: hand-written
HIP kernels behind the reference's operator C-ABI (nxt_paged_attention*) and
its dlopen plugin ABI (nxt_backend_init/run/fini).  This package is the thin
Python host mirror used by the tests and the benchmark.
"""
from . import _lib  # noqa: F401

__version__ = "0.1.0"
