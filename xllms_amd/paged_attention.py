"""Python host mirror of the paged-attention operator C-ABI (torch tensors in).

Thin ctypes layer over libxllm_hip_backend.so for tests, the benchmark and
Python callers.  It mirrors the reference's operator API
(include/operator_api.h:63-115): same entry-point names, same argument order
and meaning; tensors are torch tensors on the GPU instead of `void*`.  Every
call goes to the gfx950 kernels; there is no CPU path here.

Layouts (the reference's operator-API layout, tests/test_attention.c:141-143):
  query / out   [num_seqs, num_heads, head_size]
  key/value     [num_blocks, num_kv_heads, block_size, head_size]
                (kv_block_stride = num_kv_heads*block_size*head_size,
                 kv_head_stride = block_size*head_size, in elements)
  block_tables  int32 [num_seqs, max_num_blocks_per_seq]
  seq_lens      int32 [num_seqs]
"""
from __future__ import annotations

import ctypes

from . import _lib

NXT_KV_FP16 = 1
NXT_KV_BF16 = 2
NXT_KV_FP32 = 3

NXT_ATTN_OK = 0
NXT_ATTN_E_INVALID = -1
NXT_ATTN_E_UNSUPPORTED = -2
NXT_ATTN_E_HIP = -3
NXT_ATTN_E_NOMEM = -4

ENTRY_POINTS = ("nxt_paged_attention", "nxt_paged_attention_v2", "nxt_paged_attention_flash")

_DTYPE_NAMES = {NXT_KV_FP16: "float16", NXT_KV_BF16: "bfloat16", NXT_KV_FP32: "float32"}


class PagedAttentionError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"paged attention failed ({status}): {message}")
        self.status = status


def kv_dtype_of(tensor) -> int:
    import torch
    return {torch.float16: NXT_KV_FP16, torch.bfloat16: NXT_KV_BF16,
            torch.float32: NXT_KV_FP32}[tensor.dtype]


def last_status() -> tuple[int, str]:
    lib = _lib.backend()
    return lib.nxt_attn_last_status(), lib.nxt_attn_last_error().decode()


def version() -> str:
    return _lib.backend().nxt_attn_version().decode()


def _ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def _stream_handle(stream) -> int:
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def paged_attention(out, query, key_cache, value_cache, block_tables, seq_lens, *,
                    num_kv_heads: int, scale: float, block_size: int | None = None,
                    max_num_blocks_per_seq: int | None = None, kv_block_stride: int | None = None,
                    kv_head_stride: int | None = None, partition_tokens: int = 0,
                    kv_dtype: int | None = None, entry: str | None = None, stream=None,
                    check: bool = True) -> int:
    """Launch the decode attention on the current (or given) stream.

    entry=None uses nxt_paged_attention_ex (any dtype, explicit partition
    length); entry in ENTRY_POINTS calls that reference-named void entry point
    (dtype_size 2 = fp16, 4 = fp32) and then reads the thread's last status.
    Returns the status; raises PagedAttentionError on failure when check.
    """
    lib = _lib.backend()
    num_seqs, num_heads, head_size = query.shape
    if block_size is None:
        block_size = key_cache.shape[2]
    if max_num_blocks_per_seq is None:
        max_num_blocks_per_seq = block_tables.shape[1]
    if kv_head_stride is None:
        kv_head_stride = key_cache.stride(1)
    if kv_block_stride is None:
        kv_block_stride = key_cache.stride(0)
    if kv_dtype is None:
        kv_dtype = kv_dtype_of(key_cache)
    dtype_size = key_cache.element_size()
    args = (_ptr(out), _ptr(query), _ptr(key_cache), _ptr(value_cache), _ptr(block_tables),
            _ptr(seq_lens), num_seqs, num_heads, head_size, num_kv_heads, ctypes.c_float(scale),
            max_num_blocks_per_seq, block_size, dtype_size, kv_block_stride, kv_head_stride,
            _stream_handle(stream))
    if entry is None:
        status = lib.nxt_paged_attention_ex(*args, kv_dtype, partition_tokens)
    else:
        if entry not in ENTRY_POINTS:
            raise ValueError(f"unknown entry point {entry}")
        getattr(lib, entry)(*args)
        status = lib.nxt_attn_last_status()
    if check and status != NXT_ATTN_OK:
        raise PagedAttentionError(status, lib.nxt_attn_last_error().decode())
    return status


def auto_waves(num_seqs: int, num_heads: int, head_size: int, num_kv_heads: int,
               max_num_blocks_per_seq: int, block_size: int, kv_dtype: int) -> int:
    """Wavefronts the automatic stream-K plan launches for this shape."""
    return _lib.backend().nxt_paged_attention_auto_waves(
        num_seqs, num_heads, head_size, num_kv_heads, max_num_blocks_per_seq, block_size, kv_dtype)


def release_workspaces() -> int:
    return _lib.backend().nxt_attn_release_workspaces()


def paged_kv_append(key_cache, value_cache, key, value, *, block_tables=None, positions=None,
                    slot_mapping=None, num_kv_heads: int | None = None,
                    block_size: int | None = None, kv_block_stride: int | None = None,
                    kv_head_stride: int | None = None, kv_dtype: int | None = None, stream=None,
                    check: bool = True) -> int:
    """Store new K/V rows (key / value [num_tokens, num_kv_heads, head_size])
    in the paged caches: with block_tables + positions (decode: row s is
    sequence s's token at positions[s]) through nxt_paged_kv_append, or with
    slot_mapping (flat slot per row) through nxt_paged_kv_write_slots."""
    lib = _lib.backend()
    num_tokens, kvh, head_size = key.shape
    if num_kv_heads is None:
        num_kv_heads = kvh
    if block_size is None:
        block_size = key_cache.shape[2]
    if kv_block_stride is None:
        kv_block_stride = key_cache.stride(0)
    if kv_head_stride is None:
        kv_head_stride = key_cache.stride(1)
    if kv_dtype is None:
        kv_dtype = kv_dtype_of(key_cache)
    st = _stream_handle(stream)
    if slot_mapping is not None:
        status = lib.nxt_paged_kv_write_slots(
            _ptr(key_cache), _ptr(value_cache), _ptr(key), _ptr(value), _ptr(slot_mapping),
            num_tokens, num_kv_heads, head_size, block_size, kv_block_stride, kv_head_stride,
            kv_dtype, st)
    else:
        if block_tables is None or positions is None:
            raise ValueError("need block_tables and positions, or slot_mapping")
        status = lib.nxt_paged_kv_append(
            _ptr(key_cache), _ptr(value_cache), _ptr(key), _ptr(value), _ptr(block_tables),
            _ptr(positions), num_tokens, num_kv_heads, head_size, block_tables.shape[1],
            block_size, kv_block_stride, kv_head_stride, kv_dtype, st)
    if check and status != NXT_ATTN_OK:
        raise PagedAttentionError(status, lib.nxt_attn_last_error().decode())
    return status


def paged_kv_copy_slots(key_cache, value_cache, src_slots, dst_slots, *,
                        num_kv_heads: int | None = None, block_size: int | None = None,
                        kv_block_stride: int | None = None, kv_head_stride: int | None = None,
                        kv_dtype: int | None = None, stream=None, check: bool = True) -> int:
    """Copy the K/V rows of page slots src_slots[i] to dst_slots[i] (int32
    device tensors) inside the caches (nxt_paged_kv_copy_slots): the
    copy-on-write of a partly shared page at admission."""
    lib = _lib.backend()
    _, kvh, bs, head_size = key_cache.shape
    num_kv_heads = kvh if num_kv_heads is None else num_kv_heads
    block_size = bs if block_size is None else block_size
    kv_block_stride = key_cache.stride(0) if kv_block_stride is None else kv_block_stride
    kv_head_stride = key_cache.stride(1) if kv_head_stride is None else kv_head_stride
    kv_dtype = kv_dtype_of(key_cache) if kv_dtype is None else kv_dtype
    status = lib.nxt_paged_kv_copy_slots(
        _ptr(key_cache), _ptr(value_cache), _ptr(src_slots), _ptr(dst_slots),
        src_slots.shape[0], num_kv_heads, head_size, block_size, kv_block_stride,
        kv_head_stride, kv_dtype, _stream_handle(stream))
    if check and status != NXT_ATTN_OK:
        raise PagedAttentionError(status, lib.nxt_attn_last_error().decode())
    return status


def paged_attention_cascade(out, query, key_cache, value_cache, block_tables, seq_lens,
                            prefix_group, prefix_blocks, *, num_kv_heads: int, scale: float,
                            max_groups: int | None = None, block_size: int | None = None,
                            kv_block_stride: int | None = None, kv_head_stride: int | None = None,
                            kv_dtype: int | None = None, stream=None, check: bool = True) -> int:
    """Prefix-aware decode (nxt_paged_attention_cascade): same result as
    paged_attention, reading each shared prefix page once per 32 query rows
    (16 for fp32 or head_size > 128) of the sequences that share it.  prefix_group: int32 [num_seqs] (-1 = none),
    prefix_blocks: int32 [max_groups] shared leading pages per group."""
    lib = _lib.backend()
    num_seqs, num_heads, head_size = query.shape
    if max_groups is None:
        max_groups = prefix_blocks.shape[0]
    if block_size is None:
        block_size = key_cache.shape[2]
    if kv_head_stride is None:
        kv_head_stride = key_cache.stride(1)
    if kv_block_stride is None:
        kv_block_stride = key_cache.stride(0)
    if kv_dtype is None:
        kv_dtype = kv_dtype_of(key_cache)
    status = lib.nxt_paged_attention_cascade(
        _ptr(out), _ptr(query), _ptr(key_cache), _ptr(value_cache), _ptr(block_tables),
        _ptr(seq_lens), _ptr(prefix_group), _ptr(prefix_blocks), max_groups, num_seqs, num_heads,
        head_size, num_kv_heads, ctypes.c_float(scale), block_tables.shape[1], block_size,
        kv_block_stride, kv_head_stride, kv_dtype, _stream_handle(stream))
    if check and status != NXT_ATTN_OK:
        raise PagedAttentionError(status, lib.nxt_attn_last_error().decode())
    return status


def prefix_groups(block_tables, seq_lens, *, block_size: int, stream=None):
    """Shared-prefix groups of a batch found from its block tables
    (nxt_paged_prefix_groups).  Returns device tensors (prefix_group [B],
    prefix_blocks [B // 2 + 1]) and the device int32 count [1]."""
    import torch
    lib = _lib.backend()
    B = seq_lens.shape[0]
    dev = seq_lens.device
    group = torch.empty(B, dtype=torch.int32, device=dev)
    blocks = torch.zeros(B // 2 + 1, dtype=torch.int32, device=dev)
    count = torch.zeros(1, dtype=torch.int32, device=dev)
    status = lib.nxt_paged_prefix_groups(_ptr(block_tables), _ptr(seq_lens), B,
                                         block_tables.shape[1], block_size, _ptr(group),
                                         _ptr(blocks), _ptr(count), _stream_handle(stream))
    if status != NXT_ATTN_OK:
        raise PagedAttentionError(status, lib.nxt_attn_last_error().decode())
    return group, blocks, count
