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


# ---------------------------------------------------------------- models
# Layout mirrors of include/backend.h:54-189 (sizes 48 / 120 / 168 / 48 / 56
# bytes, as the reference header compiles on LP64) and of NxtDecodeIo.
NXT_TYPE_INT32, NXT_TYPE_FP16, NXT_TYPE_FP32, NXT_TYPE_BF16_HIP = 8, 10, 11, 256


class NxtTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int),
                ("shape", ctypes.POINTER(ctypes.c_int64)), ("dims_count", ctypes.c_uint32),
                ("byte_size", ctypes.c_uint64), ("memory_type", ctypes.c_int),
                ("memory_type_id", ctypes.c_int32)]


class _VersionConfig(ctypes.Structure):
    _fields_ = [("policy", ctypes.c_int), ("num_versions", ctypes.c_uint32),
                ("versions", ctypes.c_void_p), ("versions_count", ctypes.c_uint32)]


class _BatchingConfig(ctypes.Structure):
    _fields_ = [("preferred_batch_size_ratio", ctypes.c_float),
                ("max_queue_delay_ms", ctypes.c_double), ("preserve_ordering", ctypes.c_bool),
                ("priority_levels", ctypes.c_int32)]


class NxtModelConfig(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("backend_name", ctypes.c_char_p),
                ("model_path", ctypes.c_char_p), ("max_batch_size", ctypes.c_int32),
                ("input_count", ctypes.c_uint32), ("inputs", ctypes.POINTER(ctypes.POINTER(NxtTensor))),
                ("output_count", ctypes.c_uint32), ("outputs", ctypes.c_void_p),
                ("instance_group_count", ctypes.c_uint32), ("instance_groups", ctypes.c_void_p),
                ("version_config", _VersionConfig), ("dynamic_batching", _BatchingConfig)]


class NxtModelInstance(ctypes.Structure):
    _fields_ = [("model", ctypes.c_void_p), ("name", ctypes.c_char_p), ("kind", ctypes.c_int),
                ("device_id", ctypes.c_int32), ("instance_state", ctypes.c_void_p),
                ("exec_count", ctypes.c_uint64), ("total_exec_ms", ctypes.c_double)]


class NxtModel(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("version", ctypes.c_int32),
                ("config", NxtModelConfig), ("backend", ctypes.c_void_p),
                ("instances", ctypes.POINTER(NxtModelInstance)), ("instance_count", ctypes.c_uint32),
                ("state", ctypes.c_int), ("backend_state", ctypes.c_void_p)]


class NxtInferRequest(ctypes.Structure):
    _fields_ = [("request_id", ctypes.c_char_p), ("batch_size", ctypes.c_uint32),
                ("input_count", ctypes.c_uint32), ("inputs", ctypes.c_void_p),
                ("requested_output_count", ctypes.c_uint32),
                ("requested_output_names", ctypes.c_void_p),
                ("enqueue_time_ns", ctypes.c_uint64), ("priority", ctypes.c_int32)]


class NxtDecodeIo(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("num_tokens", ctypes.c_int32),
                ("token_ids", ctypes.c_void_p), ("key", ctypes.c_void_p),
                ("value", ctypes.c_void_p), ("query", ctypes.c_void_p),
                ("output", ctypes.c_void_p), ("release", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


class DecodeModel:
    """A decode model on the plugin, created the way nxt_model_create does
    (src/core/backend_manager.c:373-402: the config copied into an NxtModel,
    then the plugin's nxt_model_init), and executed the way the scheduler's
    poll does (src/core/scheduler.c:482-486:
    instance_exec(model->instances, requests, count))."""

    def __init__(self, *, num_blocks: int, num_kv_heads: int, block_size: int, head_size: int,
                 num_heads: int, dtype: int = NXT_TYPE_FP16, max_batch_size: int = 256,
                 max_blocks_per_seq: int | None = None, name: str = "default"):
        self.dl = ctypes.CDLL(_lib.BACKEND_SO, mode=os.RTLD_NOW | os.RTLD_LOCAL)
        vp = ctypes.c_void_p
        for fn in ("nxt_model_init", "nxt_model_fini"):
            getattr(self.dl, fn).argtypes = [ctypes.POINTER(NxtModel)]
            getattr(self.dl, fn).restype = ctypes.c_int
        self.dl.nxt_model_instance_exec.argtypes = [ctypes.POINTER(NxtModelInstance), vp,
                                                    ctypes.c_uint32]
        self.dl.nxt_model_instance_exec.restype = ctypes.c_int
        self.dl.nxt_model_instance_bind.argtypes = [ctypes.POINTER(NxtModelInstance),
                                                    ctypes.c_char_p, ctypes.POINTER(NxtDecodeIo)]
        self.dl.nxt_model_instance_bind.restype = ctypes.c_int
        self.dl.nxt_model_instance_set_deferred.argtypes = [ctypes.POINTER(NxtModelInstance),
                                                            ctypes.c_int]
        self.dl.nxt_model_instance_set_deferred.restype = ctypes.c_int
        self.dl.nxt_model_instance_flush.argtypes = [ctypes.POINTER(NxtModelInstance)]
        self.dl.nxt_model_instance_flush.restype = ctypes.c_int
        self._keep = []      # config structures, alive as long as the model

        def tensor(tname, dtype_code, shape):
            sh = (ctypes.c_int64 * len(shape))(*shape)
            t = NxtTensor(name=tname.encode(), dtype=dtype_code, shape=sh, dims_count=len(shape))
            self._keep += [sh, t]
            return ctypes.pointer(t)

        ins = [tensor("key_cache", dtype, [num_blocks, num_kv_heads, block_size, head_size]),
               tensor("query", dtype, [num_heads, head_size])]
        if max_blocks_per_seq:
            ins.append(tensor("block_tables", NXT_TYPE_INT32, [max_batch_size, max_blocks_per_seq]))
        arr = (ctypes.POINTER(NxtTensor) * len(ins))(*ins)
        self._keep.append(arr)
        self._name = name.encode()
        self.model = NxtModel()
        self.model.name = self._name
        self.model.version = 1
        self.model.config.name = self._name
        self.model.config.backend_name = b"hip"
        self.model.config.max_batch_size = max_batch_size
        self.model.config.input_count = len(ins)
        self.model.config.inputs = arr
        self.status = self.dl.nxt_model_init(ctypes.byref(self.model))
        self.model.state = STATE_READY if self.status == 0 else STATE_ERROR

    @property
    def instance(self):
        return self.model.instances

    def bind(self, request_id: str, *, tokens=None, key=None, value=None, query=None,
             output=None, release: bool = False) -> int:
        import numpy as np
        io = NxtDecodeIo(struct_size=ctypes.sizeof(NxtDecodeIo))
        if tokens is not None and len(tokens):
            t = np.ascontiguousarray(tokens, dtype=np.int32)  # copied by the bind
            io.num_tokens = len(t)
            io.token_ids = t.ctypes.data
        ptr = lambda x: None if x is None else x.data_ptr()
        io.key, io.value, io.query, io.output = ptr(key), ptr(value), ptr(query), ptr(output)
        io.release = int(release)
        return self.dl.nxt_model_instance_bind(self.instance, request_id.encode(),
                                               ctypes.byref(io))

    def requests(self, request_ids):
        """The NxtInferRequest* array of a batch, built once and reusable
        (exec_requests) while the ids stay the same."""
        ids = [r.encode() for r in request_ids]
        reqs = (NxtInferRequest * max(1, len(ids)))()
        ptrs = (ctypes.POINTER(NxtInferRequest) * max(1, len(ids)))()
        for i, rid in enumerate(ids):
            reqs[i].request_id = rid
            reqs[i].batch_size = 1
            ptrs[i] = ctypes.pointer(reqs[i])
        return (ids, reqs, ptrs, len(ids), ctypes.cast(ptrs, ctypes.c_void_p))

    def exec_requests(self, prepared) -> int:
        return self.dl.nxt_model_instance_exec(self.instance, prepared[4], prepared[3])

    def exec(self, request_ids) -> int:
        return self.exec_requests(self.requests(request_ids))

    def set_deferred(self, on: bool) -> int:
        """Deferred mode: exec queues requests; a flush runs them as one batch."""
        return self.dl.nxt_model_instance_set_deferred(self.instance, int(on))

    def flush(self) -> int:
        return self.dl.nxt_model_instance_flush(self.instance)

    def close(self) -> int:
        rc = self.dl.nxt_model_fini(ctypes.byref(self.model))
        return rc
