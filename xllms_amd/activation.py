"""Python host mirror of the activation operators (torch tensors in).

Thin ctypes layer over libxllm_hip_backend.so that mirrors the reference's
activation API (include/operator_api.h:122-150): same entry-point names, same
argument order and meaning; tensors are torch tensors on the GPU instead of
`void*`.  Every call goes to the gfx950 kernels; there is no CPU path here.

Layouts: input [num_tokens, 2*d] for the gated ops (row = gate | up) and
[num_tokens, d] for the element-wise ones; out [num_tokens, d].
"""
from __future__ import annotations

from . import _lib
from .paged_attention import (NXT_ATTN_OK, PagedAttentionError, _ptr, _stream_handle,
                              kv_dtype_of)

NXT_ACT_SILU_AND_MUL = 1
NXT_ACT_MUL_AND_SILU = 2
NXT_ACT_GELU_AND_MUL = 3
NXT_ACT_GELU_TANH_AND_MUL = 4
NXT_ACT_GELU = 5
NXT_ACT_SILU = 6

# reference entry point -> op code
ENTRY_POINTS = {
    "nxt_silu_and_mul": NXT_ACT_SILU_AND_MUL,
    "nxt_mul_and_silu": NXT_ACT_MUL_AND_SILU,
    "nxt_gelu_and_mul": NXT_ACT_GELU_AND_MUL,
    "nxt_gelu_tanh_and_mul": NXT_ACT_GELU_TANH_AND_MUL,
    "nxt_gelu_elementwise": NXT_ACT_GELU,
    "nxt_silu_elementwise": NXT_ACT_SILU,
}
OP_NAMES = {v: k[len("nxt_"):] for k, v in ENTRY_POINTS.items()}


def is_gated(op: int) -> bool:
    return NXT_ACT_SILU_AND_MUL <= op <= NXT_ACT_GELU_TANH_AND_MUL


def activation(op: int, out, input, *, num_tokens: int | None = None, d: int | None = None,
               dtype: int | None = None, entry: str | None = None, stream=None,
               check: bool = True) -> int:
    """Launch one activation on the current (or given) stream.

    entry=None uses nxt_activation_ex (fp16, bf16 or fp32; 64-bit token
    count); entry names one of the reference's void entry points
    (dtype_size 2 = fp16, 4 = fp32), after which the thread's last status is
    read.  num_tokens / d default to out's shape.  Returns the status; raises
    PagedAttentionError (the library's shared status type) when check.
    """
    lib = _lib.backend()
    if num_tokens is None:
        num_tokens = out.shape[0]
    if d is None:
        d = out.shape[-1]
    if entry is None:
        if dtype is None:
            dtype = kv_dtype_of(out)
        status = lib.nxt_activation_ex(op, _ptr(out), _ptr(input), num_tokens, d, dtype,
                                       _stream_handle(stream))
    else:
        if ENTRY_POINTS.get(entry) != op:
            raise ValueError(f"entry point {entry} does not compute op {op}")
        getattr(lib, entry)(_ptr(out), _ptr(input), num_tokens, d, out.element_size(),
                            _stream_handle(stream))
        status = lib.nxt_attn_last_status()
    if check and status != NXT_ATTN_OK:
        raise PagedAttentionError(status, lib.nxt_attn_last_error().decode())
    return status


def silu_and_mul(out, input, **kw) -> int:
    return activation(NXT_ACT_SILU_AND_MUL, out, input, **kw)


def mul_and_silu(out, input, **kw) -> int:
    return activation(NXT_ACT_MUL_AND_SILU, out, input, **kw)


def gelu_and_mul(out, input, **kw) -> int:
    return activation(NXT_ACT_GELU_AND_MUL, out, input, **kw)


def gelu_tanh_and_mul(out, input, **kw) -> int:
    return activation(NXT_ACT_GELU_TANH_AND_MUL, out, input, **kw)


def gelu_elementwise(out, input, **kw) -> int:
    return activation(NXT_ACT_GELU, out, input, **kw)


def silu_elementwise(out, input, **kw) -> int:
    return activation(NXT_ACT_SILU, out, input, **kw)
