"""ctypes wrapper of the C oracle (oracle/paged_attention_oracle.c) and of the
reference's own compiled CPU attention (oracle/_ref, built from
examples/run_gpt2.c by `make -C oracle ref`).  TEST INFRASTRUCTURE ONLY.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref_gpt2_attn.so")
REFERENCE_ROOT = os.environ.get("XLLM_REFERENCE_ROOT", "/root/reference")

_lib = None
_ref = None

FP16, BF16, FP32 = 1, 2, 3


def build(ref: bool = True) -> None:
    """Compile the oracle (and oracle/_ref when the reference tree exists)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if ref and os.path.isdir(os.path.join(REFERENCE_ROOT, "examples")):
        subprocess.run(["make", "-s", "-C", HERE, "ref", f"REF={REFERENCE_ROOT}"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            build(ref=False)
        L = ctypes.CDLL(ORACLE_SO)
        vp, ci, cf, ll = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_longlong
        common = [vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, cf, ci, ci, ci, ll, ll]
        L.oracle_paged_attention_f32.argtypes = common
        L.oracle_paged_attention_f32.restype = ci
        L.oracle_paged_attention_f64.argtypes = common
        L.oracle_paged_attention_f64.restype = ci
        L.oracle_paged_attention_f32_mt.argtypes = common + [ci]
        L.oracle_paged_attention_f32_mt.restype = ci
        L.oracle_num_threads.argtypes = []
        L.oracle_num_threads.restype = ci
        L.oracle_gpt2_paged_attention.argtypes = [vp, vp, vp, vp, ci, ci, ci, ci, vp]
        L.oracle_gpt2_paged_attention.restype = None
        L.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        L.oracle_half_to_float.restype = cf
        L.oracle_bf16_to_float.argtypes = [ctypes.c_uint16]
        L.oracle_bf16_to_float.restype = cf
        L.oracle_paged_kv_append.argtypes = [vp, vp, vp, vp, vp, vp, vp, ci, ci, ci, ci, ci, ll,
                                             ll, ci]
        L.oracle_paged_kv_append.restype = ci
        _lib = L
    return _lib


def ref_lib():
    """The reference's compiled run_gpt2.c paged_attention, or None."""
    global _ref
    if _ref is None and os.path.exists(REF_SO):
        R = ctypes.CDLL(REF_SO)
        vp, ci = ctypes.c_void_p, ctypes.c_int
        R.ref_gpt2_paged_attention.argtypes = [vp, vp, vp, vp, ci, ci, ci, ci, vp]
        R.ref_gpt2_paged_attention.restype = None
        _ref = R
    return _ref


def _c(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a)


def _args(q, k, v, bt, sl, num_kv_heads, scale, block_size, dtype, kv_block_stride,
          kv_head_stride):
    q, k, v, bt, sl = _c(q), _c(k), _c(v), _c(bt.astype(np.int32)), _c(sl.astype(np.int32))
    B, H, D = q.shape
    keep = (q, k, v, bt, sl)
    args = [q.ctypes.data, k.ctypes.data, v.ctypes.data, bt.ctypes.data, sl.ctypes.data,
            B, H, D, num_kv_heads, ctypes.c_float(scale), bt.shape[1], block_size, dtype,
            kv_block_stride, kv_head_stride]
    return keep, args, (B, H, D)


def paged_attention(q, k, v, block_tables, seq_lens, *, num_kv_heads, scale, block_size,
                    dtype, kv_block_stride=None, kv_head_stride=None, precision="f32",
                    threads=0) -> np.ndarray:
    """Reference CPU decode attention over operator-API buffers.  q/k/v are
    numpy arrays holding the element bits (uint16 for fp16/bf16).  Returns fp32
    (or fp64 for precision='f64') [B][H][D]."""
    D = q.shape[2]
    if kv_head_stride is None:
        kv_head_stride = block_size * D
    if kv_block_stride is None:
        kv_block_stride = num_kv_heads * block_size * D
    keep, args, shape = _args(q, k, v, block_tables, seq_lens, num_kv_heads, scale, block_size,
                              dtype, kv_block_stride, kv_head_stride)
    L = lib()
    if precision == "f64":
        out = np.empty(shape, dtype=np.float64)
        rc = L.oracle_paged_attention_f64(out.ctypes.data, *args)
    elif precision == "mt":
        out = np.empty(shape, dtype=np.float32)
        rc = L.oracle_paged_attention_f32_mt(out.ctypes.data, *args, threads)
    else:
        out = np.empty(shape, dtype=np.float32)
        rc = L.oracle_paged_attention_f32(out.ctypes.data, *args)
    del keep
    if rc != 0:
        raise ValueError("oracle rejected the arguments")
    return out


def run_workload(wl, precision="f32", threads=0, seqs=None) -> np.ndarray:
    """Oracle output for a xllms_amd.workloads.Workload (optionally only the
    sequences in `seqs`, a slice or index array)."""
    q, bt, sl = wl.query, wl.block_tables, wl.seq_lens
    if seqs is not None:
        q, bt, sl = q[seqs], bt[seqs], sl[seqs]
    return paged_attention(q, wl.key_cache, wl.value_cache, bt, sl,
                           num_kv_heads=wl.num_kv_heads, scale=wl.scale,
                           block_size=wl.block_size, dtype=wl.kv_dtype,
                           kv_block_stride=wl.kv_block_stride,
                           kv_head_stride=wl.kv_head_stride, precision=precision,
                           threads=threads)


def gpt2_paged_attention(query, key_cache, value_cache, page_table, seq_len, num_heads,
                         head_dim, page_size, use_reference=False) -> np.ndarray:
    """examples/run_gpt2.c:46-83 semantics (MHA, per-token page table, KV
    layout [page][slot][head][d]).  use_reference=True calls the reference's
    own compiled function from oracle/_ref instead of the restatement."""
    q = _c(query.astype(np.float32))
    k = _c(key_cache.astype(np.float32))
    v = _c(value_cache.astype(np.float32))
    pt = _c(np.asarray(page_table, dtype=np.int32))
    out = np.empty((num_heads, head_dim), dtype=np.float32)
    if use_reference:
        R = ref_lib()
        if R is None:
            raise FileNotFoundError(REF_SO)
        fn = R.ref_gpt2_paged_attention
    else:
        fn = lib().oracle_gpt2_paged_attention
    fn(q.ctypes.data, k.ctypes.data, v.ctypes.data, pt.ctypes.data, seq_len, num_heads,
       head_dim, page_size, out.ctypes.data)
    return out


def widen(bits: np.ndarray, dtype: int) -> np.ndarray:
    """Element bits -> float32 (exact), matching the oracle's widening."""
    if dtype == FP32:
        return bits.astype(np.float32)
    if dtype == FP16:
        return bits.view(np.float16).astype(np.float32)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def paged_kv_append(key_cache: np.ndarray, value_cache: np.ndarray, key: np.ndarray,
                    value: np.ndarray, *, block_size: int, kv_block_stride: int,
                    kv_head_stride: int, slots=None, block_tables=None, positions=None):
    """KV-cache write of text_gen.c:1274-1278 over the paged layout (see
    oracle_paged_kv_append): returns updated copies of the two caches.
    key / value: [num_tokens, num_kv_heads, head_size] in the cache dtype
    (any 2- or 4-byte numpy dtype; bytes are copied unchanged)."""
    kc = np.array(key_cache, copy=True, order="C")
    vc = np.array(value_cache, copy=True, order="C")
    k = _c(key)
    v = _c(value)
    n, kvh, d = k.shape
    if slots is not None:
        sl = _c(np.asarray(slots, dtype=np.int32))
        bt = pos = None
        max_blocks = 0
    else:
        sl = None
        bt = _c(np.asarray(block_tables, dtype=np.int32))
        pos = _c(np.asarray(positions, dtype=np.int32))
        max_blocks = bt.shape[1]
    ptr = lambda a: None if a is None else a.ctypes.data
    rc = lib().oracle_paged_kv_append(kc.ctypes.data, vc.ctypes.data, k.ctypes.data,
                                      v.ctypes.data, ptr(sl), ptr(bt), ptr(pos), n, kvh, d,
                                      max_blocks, block_size, kv_block_stride, kv_head_stride,
                                      k.dtype.itemsize)
    if rc != 0:
        raise ValueError("oracle_paged_kv_append rejected its arguments")
    return kc, vc


def paged_kv_copy_slots(key_cache: np.ndarray, value_cache: np.ndarray, src, dst, *,
                        num_kv_heads: int, head_size: int, block_size: int,
                        kv_block_stride: int, kv_head_stride: int):
    """Copy-on-write of page slots (nxt_paged_kv_copy_slots): the rows of
    slot src[i] (every kv head) are gathered from the caches and stored at
    slot dst[i] through oracle_paged_kv_append; a negative source or
    destination skips the pair.  Returns updated copies of the two caches."""
    src = np.asarray(src, dtype=np.int64)
    dst = np.asarray(dst, dtype=np.int32).copy()
    keep = src >= 0
    dst[~keep] = -1
    s = np.where(keep, src, 0)
    base = ((s // block_size) * kv_block_stride + (s % block_size) * head_size)[:, None, None]
    idx = base + (np.arange(num_kv_heads) * kv_head_stride)[None, :, None] + \
        np.arange(head_size)[None, None, :]
    k = key_cache.reshape(-1)[idx]
    v = value_cache.reshape(-1)[idx]
    return paged_kv_append(key_cache, value_cache, k, v, block_size=block_size,
                           kv_block_stride=kv_block_stride, kv_head_stride=kv_head_stride,
                           slots=dst)


ACT_SILU_AND_MUL, ACT_MUL_AND_SILU, ACT_GELU_AND_MUL, ACT_GELU_TANH_AND_MUL, ACT_GELU, ACT_SILU = \
    range(1, 7)


def _act_lib():
    L = lib()
    if not getattr(L, "_act_typed", False):
        vp, ci, ll = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong
        L.oracle_activation.argtypes = [ci, vp, vp, ll, ci, ci]
        L.oracle_activation.restype = ci
        L.oracle_activation_mt.argtypes = [ci, vp, vp, ll, ci, ci, ci]
        L.oracle_activation_mt.restype = ci
        L.oracle_float_to_half.argtypes = [ctypes.c_float]
        L.oracle_float_to_half.restype = ctypes.c_uint16
        L.oracle_float_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_float_to_bf16.restype = ctypes.c_uint16
        L._act_typed = True
    return L


def activation(op: int, x: np.ndarray, dtype: int, threads: int = 0) -> np.ndarray:
    """operators/activation_kernels.cu semantics (see oracle_activation):
    x holds the element bits (uint16 for fp16/bf16, float32 for fp32), shape
    [num_tokens, 2d] for the gated ops and [num_tokens, d] otherwise.
    Returns the output bits [num_tokens, d] in the same numpy dtype."""
    x = _c(x)
    n = x.shape[0]
    d = x.shape[1] // 2 if op <= ACT_GELU_TANH_AND_MUL else x.shape[1]
    out = np.empty((n, d), dtype=x.dtype)
    L = _act_lib()
    if threads > 0:
        rc = L.oracle_activation_mt(op, out.ctypes.data, x.ctypes.data, n, d, dtype, threads)
    else:
        rc = L.oracle_activation(op, out.ctypes.data, x.ctypes.data, n, d, dtype)
    if rc != 0:
        raise ValueError("oracle_activation rejected its arguments")
    return out


def float_to_half_bits(x: float) -> int:
    return int(_act_lib().oracle_float_to_half(x))


def float_to_bf16_bits(x: float) -> int:
    return int(_act_lib().oracle_float_to_bf16(x))
