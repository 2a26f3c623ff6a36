"""Python mirror of the reference backend manager's plugin handling.

Loads libxllm_hip_backend.so the way src/core/backend_manager.c:264-317 loads a
backend plugin (dlopen RTLD_NOW|RTLD_LOCAL, dlsym of nxt_backend_init / run /
fini, state UNINITIALIZED -> INITIALIZING -> READY, or ERROR when init
fails), runs it like :339-344 (refuses a backend that is not READY) and
unloads it like :319-337.  The ctypes structures are layout mirrors of
include/backend.h:128-151 and backends/cuda_backend.h:29-46; the tests check
their offsets against the values the reference documents.
"""
from __future__ import annotations

import ctypes
import os

from . import _lib

STATE_UNINITIALIZED = 0
STATE_INITIALIZING = 1
STATE_READY = 2
STATE_ERROR = 3
STATE_UNLOADING = 4


class NxtBackendAPI(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in (
        "backend_init", "backend_run", "backend_fini", "model_init", "model_fini",
        "instance_init", "instance_fini", "instance_exec")]


class NxtBackend(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("so_path", ctypes.c_char_p),
        ("dl_handle", ctypes.c_void_p),
        ("api", NxtBackendAPI),
        ("state", ctypes.c_int),
        ("priority", ctypes.c_int32),
        ("model_count", ctypes.c_uint32),
        ("models", ctypes.c_void_p),
        ("backend_state", ctypes.c_void_p),
    ]


class NxtPagedAttentionInput(ctypes.Structure):
    _fields_ = [
        ("query", ctypes.c_void_p),
        ("key_cache", ctypes.c_void_p),
        ("value_cache", ctypes.c_void_p),
        ("block_tables", ctypes.c_void_p),
        ("seq_lens", ctypes.c_void_p),
        ("num_seqs", ctypes.c_int),
        ("num_heads", ctypes.c_int),
        ("head_size", ctypes.c_int),
        ("num_kv_heads", ctypes.c_int),
        ("scale", ctypes.c_float),
        ("max_num_blocks_per_seq", ctypes.c_int),
        ("block_size", ctypes.c_int),
        ("dtype_size", ctypes.c_int),
        ("kv_block_stride", ctypes.c_int),
        ("kv_head_stride", ctypes.c_int),
        ("stream", ctypes.c_void_p),
    ]


class NxtPagedAttentionInputEx(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("base", NxtPagedAttentionInput),
        ("kv_dtype", ctypes.c_int),
        ("partition_tokens", ctypes.c_int),
    ]


_InitFn = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.POINTER(NxtBackend))
_RunFn = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.POINTER(NxtBackend), ctypes.c_void_p,
                          ctypes.c_void_p)
_FiniFn = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.POINTER(NxtBackend))


class LoadedBackend:
    """One plugin loaded and initialised like nxt_backend_load does."""

    def __init__(self, so_path: str | None = None, name: str = "hip", priority: int = 0):
        so_path = so_path or _lib.BACKEND_SO
        if not os.path.exists(so_path):
            raise _lib.NativeLibraryMissing(f"{so_path} is not built")
        self.so_path = so_path
        self.dl = ctypes.CDLL(so_path, mode=os.RTLD_NOW | os.RTLD_LOCAL)
        self._name = name.encode()
        self._path = so_path.encode()
        self.handle = NxtBackend()
        self.handle.name = self._name
        self.handle.so_path = self._path
        self.handle.priority = priority
        self.handle.state = STATE_UNINITIALIZED
        self.init_fn = _InitFn(("nxt_backend_init", self.dl))
        self.run_fn = _RunFn(("nxt_backend_run", self.dl))
        self.fini_fn = _FiniFn(("nxt_backend_fini", self.dl))
        self.run_ex_fn = _RunFn(("nxt_backend_run_ex", self.dl))
        self.handle.api.backend_init = ctypes.cast(self.init_fn, ctypes.c_void_p)
        self.handle.api.backend_run = ctypes.cast(self.run_fn, ctypes.c_void_p)
        self.handle.api.backend_fini = ctypes.cast(self.fini_fn, ctypes.c_void_p)

    def init(self) -> int:
        self.handle.state = STATE_INITIALIZING
        rc = self.init_fn(ctypes.byref(self.handle))
        if rc != 0:
            self.handle.state = STATE_ERROR
            return rc
        self.handle.state = STATE_READY
        return 0

    @property
    def state(self) -> int:
        return self.handle.state

    def run(self, desc: NxtPagedAttentionInput | None, output: int) -> int:
        if self.handle.state != STATE_READY:
            return -1
        return self.run_fn(ctypes.byref(self.handle),
                           ctypes.cast(ctypes.byref(desc), ctypes.c_void_p) if desc is not None
                           else None, output or None)

    def run_ex(self, desc: NxtPagedAttentionInputEx, output: int) -> int:
        if self.handle.state != STATE_READY:
            return -1
        return self.run_ex_fn(ctypes.byref(self.handle),
                              ctypes.cast(ctypes.byref(desc), ctypes.c_void_p), output or None)

    def fini(self) -> int:
        self.handle.state = STATE_UNLOADING
        return self.fini_fn(ctypes.byref(self.handle))


def make_input(query, key_cache, value_cache, block_tables, seq_lens, *, num_kv_heads: int,
               scale: float, stream: int = 0) -> NxtPagedAttentionInput:
    """Descriptor for torch tensors in the operator-API layout."""
    num_seqs, num_heads, head_size = query.shape
    d = NxtPagedAttentionInput()
    d.query = query.data_ptr()
    d.key_cache = key_cache.data_ptr()
    d.value_cache = value_cache.data_ptr()
    d.block_tables = block_tables.data_ptr()
    d.seq_lens = seq_lens.data_ptr()
    d.num_seqs = num_seqs
    d.num_heads = num_heads
    d.head_size = head_size
    d.num_kv_heads = num_kv_heads
    d.scale = scale
    d.max_num_blocks_per_seq = block_tables.shape[1]
    d.block_size = key_cache.shape[2]
    d.dtype_size = key_cache.element_size()
    d.kv_block_stride = key_cache.stride(0)
    d.kv_head_stride = key_cache.stride(1)
    d.stream = stream or None
    return d
