"""Python binding of the paged KV-cache index (include/xllm_hip_kv_index.h):
block pool, radix tree of token ids with flat slot ids, and the sequence
table that yields block tables, new-token slots and shared-prefix groups
for the decode kernels.  Host code of libxllm_hip_backend.so; no GPU needed.

Method names follow the reference interfaces they replace:
nxt_page_alloc / nxt_page_ref_inc / nxt_page_ref_dec
(src/core/memory_manager.c:207-272) and nxt_prefix_match / insert / evict /
lock / unlock (include/prefix_sharing.h:86-155).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

OK, E_INVALID, E_NO_BLOCKS, E_CAPACITY = 0, -1, -2, -3
MAX_MATCH = 2048  # NXT_PREFIX_MAX_MATCH_PAGES


class KvIndexError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: status {status}")
        self.status = status


class _Match(ctypes.Structure):
    _fields_ = [("matched_tokens", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("last_node", ctypes.c_uint64)]


class _Stats(ctypes.Structure):
    _fields_ = [("total_tokens", ctypes.c_int32), ("node_count", ctypes.c_int32),
                ("evictable_size", ctypes.c_int32), ("protected_size", ctypes.c_int32)]


class _Admit(ctypes.Structure):
    _fields_ = [("seq", ctypes.c_int32), ("cached_tokens", ctypes.c_int32),
                ("shared_blocks", ctypes.c_int32), ("copy_count", ctypes.c_int32),
                ("write_count", ctypes.c_int32)]


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class KvIndex:
    def __init__(self, num_blocks: int, block_size: int, max_blocks_per_seq: int):
        self._lib = _lib.backend()
        self._h = self._lib.nxt_kv_index_create(num_blocks, block_size, max_blocks_per_seq)
        if not self._h:
            raise KvIndexError(E_INVALID, "nxt_kv_index_create")
        self.num_blocks, self.block_size = num_blocks, block_size
        self.max_blocks = max_blocks_per_seq

    def close(self) -> None:
        if self._h:
            self._lib.nxt_kv_index_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- block pool
    def block_alloc(self) -> int:
        return self._lib.nxt_kv_block_alloc(self._h)

    def block_ref_inc(self, b: int) -> int:
        return self._lib.nxt_kv_block_ref_inc(self._h, b)

    def block_ref_dec(self, b: int) -> int:
        return self._lib.nxt_kv_block_ref_dec(self._h, b)

    def block_refs(self, b: int) -> int:
        return self._lib.nxt_kv_block_refs(self._h, b)

    def blocks_free(self) -> int:
        return self._lib.nxt_kv_blocks_free(self._h)

    # ---- radix tree
    def prefix_match(self, tokens):
        """-> (matched tokens, slots [matched], last node id)."""
        t = _i32(tokens)
        slots = np.zeros(max(1, min(len(t), MAX_MATCH)), dtype=np.int32)
        m = _Match()
        st = self._lib.nxt_kv_prefix_match(self._h, _p(t), len(t), _p(slots), ctypes.byref(m))
        if st != OK:
            raise KvIndexError(st, "nxt_kv_prefix_match")
        return m.matched_tokens, slots[:m.matched_tokens].copy(), m.last_node

    def prefix_insert(self, tokens, slots, priority: int = 0) -> int:
        t, s = _i32(tokens), _i32(slots)
        if len(t) != len(s):
            raise ValueError("one slot per token")
        return self._lib.nxt_kv_prefix_insert(self._h, _p(t), len(t), _p(s), priority)

    def prefix_evict(self, num_tokens: int) -> int:
        return self._lib.nxt_kv_prefix_evict(self._h, num_tokens)

    def prefix_lock(self, node: int) -> int:
        return self._lib.nxt_kv_prefix_lock(self._h, node)

    def prefix_unlock(self, node: int) -> int:
        return self._lib.nxt_kv_prefix_unlock(self._h, node)

    def prefix_stats(self):
        """-> (total tokens, node count, evictable size, protected size)."""
        s = _Stats()
        self._lib.nxt_kv_prefix_stats(self._h, ctypes.byref(s))
        return s.total_tokens, s.node_count, s.evictable_size, s.protected_size

    # ---- sequences
    def seq_admit(self, tokens):
        """-> (info dict, slot_mapping [len], copy_src, copy_dst)."""
        t = _i32(tokens)
        n = max(1, len(t))
        mapping = np.zeros(n, np.int32)
        src = np.zeros(n, np.int32)
        dst = np.zeros(n, np.int32)
        a = _Admit()
        st = self._lib.nxt_kv_seq_admit(self._h, _p(t), len(t), _p(mapping), _p(src), _p(dst),
                                         ctypes.byref(a))
        if st != OK:
            raise KvIndexError(st, "nxt_kv_seq_admit")
        info = {k: getattr(a, k) for k, _ in _Admit._fields_}
        c = a.copy_count
        return info, mapping[:len(t)], src[:c].copy(), dst[:c].copy()

    def seq_append(self, seq: int, tokens) -> np.ndarray:
        t = _i32(tokens)
        slots = np.zeros(max(1, len(t)), np.int32)
        st = self._lib.nxt_kv_seq_append(self._h, seq, _p(t), len(t), _p(slots))
        if st != OK:
            raise KvIndexError(st, "nxt_kv_seq_append")
        return slots[:len(t)]

    def batch_append(self, seqs, tokens) -> np.ndarray:
        s, t = _i32(seqs), _i32(tokens)
        slots = np.zeros(max(1, len(s)), np.int32)
        st = self._lib.nxt_kv_batch_append(self._h, _p(s), len(s), _p(t), _p(slots))
        if st != OK:
            raise KvIndexError(st, "nxt_kv_batch_append")
        return slots[:len(s)]

    def seq_cache(self, seq: int) -> int:
        return self._lib.nxt_kv_seq_cache(self._h, seq)

    def seq_release(self, seq: int, cache: bool = False) -> int:
        return self._lib.nxt_kv_seq_release(self._h, seq, int(cache))

    def seq_len(self, seq: int) -> int:
        return self._lib.nxt_kv_seq_len(self._h, seq)

    def batch_tables(self, seqs, max_blocks: int | None = None):
        """-> (block_tables [n][max_blocks] int32, seq_lens [n] int32)."""
        s = _i32(seqs)
        mb = max_blocks or self.max_blocks
        bt = np.zeros((max(1, len(s)), mb), np.int32)
        lens = np.zeros(max(1, len(s)), np.int32)
        st = self._lib.nxt_kv_batch_tables(self._h, _p(s), len(s), mb, _p(bt), _p(lens))
        if st != OK:
            raise KvIndexError(st, "nxt_kv_batch_tables")
        return bt[:len(s)], lens[:len(s)]

    def batch_prefix_groups(self, seqs):
        """-> (prefix_group [n], prefix_blocks [num_groups])."""
        s = _i32(seqs)
        group = np.zeros(max(1, len(s)), np.int32)
        blocks = np.zeros(len(s) // 2 + 1, np.int32)
        ng = ctypes.c_int32(0)
        st = self._lib.nxt_kv_batch_prefix_groups(self._h, _p(s), len(s), _p(group), _p(blocks),
                                                  ctypes.byref(ng))
        if st != OK:
            raise KvIndexError(st, "nxt_kv_batch_prefix_groups")
        return group[:len(s)], blocks[:ng.value].copy()
