"""Locate and load the native libraries of this package (ctypes).

The product path is libxllm_hip_backend.so: the gfx950 kernels plus the
reference-compatible C-ABI.  There is no fallback: if the library is missing
every entry point raises, so nothing can silently compute on the CPU.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "lib")
BACKEND_SO = os.path.join(LIB_DIR, "libxllm_hip_backend.so")
WORKLOAD_SO = os.path.join(LIB_DIR, "libxllm_workload.so")
STREAM_PROBE_SO = os.path.join(LIB_DIR, "libxllm_stream_probe.so")
# The same library with per-workgroup timestamps (measurement tool of
# bench.py --wg-trace; never the product path).
BACKEND_TRACE_SO = os.path.join(LIB_DIR, "libxllm_hip_backend_trace.so")

_lock = threading.Lock()
_cache: dict[str, ctypes.CDLL] = {}

c_int = ctypes.c_int
c_void_p = ctypes.c_void_p
c_float = ctypes.c_float


class NativeLibraryMissing(RuntimeError):
    pass


def _load(path: str) -> ctypes.CDLL:
    with _lock:
        lib = _cache.get(path)
        if lib is not None:
            return lib
        if not os.path.exists(path):
            raise NativeLibraryMissing(
                f"{path} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `make -C xllms_amd/csrc`")
        lib = ctypes.CDLL(path, mode=os.RTLD_NOW | os.RTLD_LOCAL)
        _cache[path] = lib
        return lib


# Exported symbols of libxllm_hip_backend.so, exactly the declarations of
# include/xllm_hip_operator_api.h and include/xllm_hip_backend.h.
OPERATOR_SYMBOLS = (
    "nxt_paged_attention",
    "nxt_paged_attention_v2",
    "nxt_paged_attention_flash",
    "nxt_paged_attention_ex",
    "nxt_paged_attention_noalloc",
    "nxt_paged_attention_auto_waves",
    "nxt_attn_last_status",
    "nxt_attn_last_error",
    "nxt_attn_set_trace_events",
    "nxt_attn_release_workspaces",
    "nxt_attn_version",
    "nxt_paged_kv_append",
    "nxt_paged_kv_write_slots",
    "nxt_paged_attention_cascade",
    "nxt_paged_prefix_groups",
    "nxt_paged_kv_copy_slots",
    "nxt_silu_and_mul",
    "nxt_mul_and_silu",
    "nxt_gelu_and_mul",
    "nxt_gelu_tanh_and_mul",
    "nxt_gelu_elementwise",
    "nxt_silu_elementwise",
    "nxt_activation_ex",
)
# The reference-named activation entry points (include/operator_api.h:122-150).
ACTIVATION_ENTRY_POINTS = OPERATOR_SYMBOLS[-7:-1]
# include/xllm_hip_kv_index.h (host code in the same library)
KV_INDEX_SYMBOLS = (
    "nxt_kv_index_create", "nxt_kv_index_destroy",
    "nxt_kv_block_alloc", "nxt_kv_block_ref_inc", "nxt_kv_block_ref_dec", "nxt_kv_block_refs",
    "nxt_kv_blocks_free",
    "nxt_kv_prefix_match", "nxt_kv_prefix_insert", "nxt_kv_prefix_evict", "nxt_kv_prefix_lock",
    "nxt_kv_prefix_unlock", "nxt_kv_prefix_stats",
    "nxt_kv_seq_admit", "nxt_kv_seq_append", "nxt_kv_batch_append", "nxt_kv_seq_cache",
    "nxt_kv_seq_release", "nxt_kv_seq_len", "nxt_kv_batch_tables", "nxt_kv_batch_prefix_groups",
)
PLUGIN_SYMBOLS = ("nxt_backend_init", "nxt_backend_run", "nxt_backend_fini", "nxt_backend_run_ex",
                  "nxt_model_init", "nxt_model_fini", "nxt_model_instance_init",
                  "nxt_model_instance_fini", "nxt_model_instance_exec", "nxt_model_instance_bind",
                  "nxt_model_instance_set_deferred", "nxt_model_instance_flush")

_LEGACY_ARGS = [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                c_int, c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_int, c_int, c_void_p]


def backend(trace: bool = False) -> ctypes.CDLL:
    """The product library, or with trace=True its instrumented build (the
    same entry points plus xhip_set_wg_trace / xhip_wg_trace_words)."""
    lib = _load(BACKEND_TRACE_SO if trace else BACKEND_SO)
    if trace and not getattr(lib, "_xllm_trace_typed", False):
        lib.xhip_set_wg_trace.argtypes = [c_void_p]
        lib.xhip_set_wg_trace.restype = None
        lib.xhip_wg_trace_words.argtypes = []
        lib.xhip_wg_trace_words.restype = ctypes.c_ulonglong
        lib._xllm_trace_typed = True
    if not getattr(lib, "_xllm_typed", False):
        for name in ("nxt_paged_attention", "nxt_paged_attention_v2", "nxt_paged_attention_flash"):
            fn = getattr(lib, name)
            fn.argtypes = _LEGACY_ARGS
            fn.restype = None
        lib.nxt_paged_attention_ex.argtypes = _LEGACY_ARGS + [c_int, c_int]
        lib.nxt_paged_attention_ex.restype = c_int
        lib.nxt_paged_attention_noalloc.argtypes = _LEGACY_ARGS + [c_int, c_int]
        lib.nxt_paged_attention_noalloc.restype = c_int
        lib.nxt_paged_attention_auto_waves.argtypes = [c_int] * 7
        lib.nxt_paged_attention_auto_waves.restype = c_int
        lib.nxt_attn_last_status.argtypes = []
        lib.nxt_attn_last_status.restype = c_int
        lib.nxt_attn_last_error.argtypes = []
        lib.nxt_attn_last_error.restype = ctypes.c_char_p
        lib.nxt_attn_release_workspaces.argtypes = []
        lib.nxt_attn_release_workspaces.restype = c_int
        lib.nxt_attn_set_trace_events.argtypes = [c_void_p, c_void_p]
        lib.nxt_attn_set_trace_events.restype = None
        lib.nxt_attn_version.argtypes = []
        lib.nxt_attn_version.restype = ctypes.c_char_p
        lib.nxt_paged_kv_append.argtypes = [c_void_p] * 6 + [c_int] * 8 + [c_void_p]
        lib.nxt_paged_kv_append.restype = c_int
        lib.nxt_paged_kv_write_slots.argtypes = [c_void_p] * 5 + [c_int] * 7 + [c_void_p]
        lib.nxt_paged_kv_write_slots.restype = c_int
        lib.nxt_paged_attention_cascade.argtypes = ([c_void_p] * 8 + [c_int] * 5 + [c_float] +
                                                    [c_int] * 5 + [c_void_p])
        lib.nxt_paged_attention_cascade.restype = c_int
        lib.nxt_paged_prefix_groups.argtypes = [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p,
                                                c_void_p, c_void_p, c_void_p]
        lib.nxt_paged_prefix_groups.restype = c_int
        lib.nxt_paged_kv_copy_slots.argtypes = [c_void_p] * 4 + [c_int] * 7 + [c_void_p]
        lib.nxt_paged_kv_copy_slots.restype = c_int
        for name in ACTIVATION_ENTRY_POINTS:
            fn = getattr(lib, name)
            fn.argtypes = [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]
            fn.restype = None
        lib.nxt_activation_ex.argtypes = [c_int, c_void_p, c_void_p, ctypes.c_int64, c_int, c_int,
                                          c_void_p]
        lib.nxt_activation_ex.restype = c_int
        _type_kv_index(lib)
        lib._xllm_typed = True
    return lib


def _type_kv_index(lib: ctypes.CDLL) -> None:
    vp, i32, u64 = c_void_p, ctypes.c_int32, ctypes.c_uint64
    sig = {
        "nxt_kv_index_create": ([c_int, c_int, c_int], vp),
        "nxt_kv_index_destroy": ([vp], None),
        "nxt_kv_block_alloc": ([vp], c_int),
        "nxt_kv_block_ref_inc": ([vp, c_int], c_int),
        "nxt_kv_block_ref_dec": ([vp, c_int], c_int),
        "nxt_kv_block_refs": ([vp, c_int], c_int),
        "nxt_kv_blocks_free": ([vp], c_int),
        "nxt_kv_prefix_match": ([vp, vp, i32, vp, vp], c_int),
        "nxt_kv_prefix_insert": ([vp, vp, i32, vp, i32], i32),
        "nxt_kv_prefix_evict": ([vp, i32], i32),
        "nxt_kv_prefix_lock": ([vp, u64], c_int),
        "nxt_kv_prefix_unlock": ([vp, u64], c_int),
        "nxt_kv_prefix_stats": ([vp, vp], c_int),
        "nxt_kv_seq_admit": ([vp, vp, i32, vp, vp, vp, vp], c_int),
        "nxt_kv_seq_append": ([vp, i32, vp, i32, vp], c_int),
        "nxt_kv_batch_append": ([vp, vp, i32, vp, vp], c_int),
        "nxt_kv_seq_cache": ([vp, i32], i32),
        "nxt_kv_seq_release": ([vp, i32, c_int], c_int),
        "nxt_kv_seq_len": ([vp, i32], i32),
        "nxt_kv_batch_tables": ([vp, vp, i32, i32, vp, vp], c_int),
        "nxt_kv_batch_prefix_groups": ([vp, vp, i32, vp, vp, vp], c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res


def workload() -> ctypes.CDLL:
    lib = _load(WORKLOAD_SO)
    if not getattr(lib, "_xllm_typed", False):
        u64 = ctypes.c_uint64
        lib.xw_fill_normal.argtypes = [c_void_p, ctypes.c_size_t, c_int, u64, u64, c_float, c_int]
        lib.xw_fill_normal.restype = None
        lib.xw_scale_rows.argtypes = [c_void_p, c_void_p, ctypes.c_size_t, ctypes.c_size_t, c_int,
                                      u64, u64, c_float, c_int]
        lib.xw_scale_rows.restype = None
        lib.xw_normal.argtypes = [u64, u64]
        lib.xw_normal.restype = c_float
        lib.xw_uniform_u64.argtypes = [u64, u64]
        lib.xw_uniform_u64.restype = u64
        lib.xw_float_to_half.argtypes = [c_float]
        lib.xw_float_to_half.restype = ctypes.c_uint16
        lib.xw_float_to_bf16.argtypes = [c_float]
        lib.xw_float_to_bf16.restype = ctypes.c_uint16
        lib.xw_num_threads.argtypes = []
        lib.xw_num_threads.restype = c_int
        lib._xllm_typed = True
    return lib


def stream_probe() -> ctypes.CDLL:
    """The read-only K/V access-pattern probe (measurement tool of bench.py)."""
    lib = _load(STREAM_PROBE_SO)
    if not getattr(lib, "_xllm_typed", False):
        lib.xllm_stream_probe.argtypes = [c_void_p, c_void_p, c_void_p, ctypes.c_longlong, c_int,
                                          c_int, c_void_p, c_void_p]
        lib.xllm_stream_probe.restype = c_int
        lib._xllm_typed = True
    return lib
