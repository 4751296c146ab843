"""MI355X paged attention for vllm-lite: HIP kernels behind a C ABI.

The product is ``libpa.so`` (built from ``csrc/`` by ``build_lib.build``).
This package is the thin Python face of it: ctypes bindings (``_lib``),
torch-tensor wrappers of the stateless entry points (``ops``) and the
``PagedKvCache`` mirror of the reference's cache object (``kv_cache``).
There is no fallback path: importing the wrappers without a built library
raises.
"""
from . import _lib
from .ops import (
    BLOCK_SIZE,
    PaError,
    argmax,
    block_hash,
    decode,
    decode_workspace_size,
    prefill,
    read_kv,
    reshape_and_cache,
    reshape_and_cache_fp8,
    rope_inv_freq,
    layer_norm,
    linear,
    rms_norm,
    rope_reshape_and_cache,
    silu_mul,
    slot_mapping,
)
from .kv_cache import PagedKvCache, StepBatch

__all__ = [
    "BLOCK_SIZE",
    "PaError",
    "PagedKvCache",
    "StepBatch",
    "argmax",
    "block_hash",
    "decode",
    "decode_workspace_size",
    "prefill",
    "read_kv",
    "reshape_and_cache",
    "reshape_and_cache_fp8",
    "rope_inv_freq",
    "layer_norm",
    "linear",
    "rms_norm",
    "rope_reshape_and_cache",
    "silu_mul",
    "slot_mapping",
]
