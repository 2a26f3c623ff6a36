"""CPU restatement of the host structures that feed the paged decode: the
page pool, the radix tree and the sequence table of the KV-cache index
(the product is xllms_amd/csrc/kv_index.cpp behind include/xllm_hip_kv_index.h).
TEST INFRASTRUCTURE ONLY: tests/ use it as the checker.

- Pool: src/core/memory_manager.c:207-272 for one tier and one page type.
  Allocation takes the head of a FIFO free list; a page whose count drops to
  zero is appended at the tail.
- PrefixTree: src/core/prefix_sharing.c:26-449 with one page id per token
  (:306), here a flat slot id.  Where the build departs from the reference on
  purpose (logical clock, match cap, page references held by the tree, counts
  that never go negative), this restatement follows the build; the departures
  are listed in include/xllm_hip_kv_index.h.  Pinned against the reference's
  own compiled tree and pool (oracle/_ref) and against brute force in
  tests/test_kv_index_oracle.py.
- KvIndex: the sequence rules of the build, which have no reference
  counterpart (the reference never turns tree pages into block tables).
  Pinned by data-integrity and reference-count properties in
  tests/test_kv_index_oracle.py.
"""
from __future__ import annotations

import collections
from dataclasses import dataclass, field

MAX_MATCH = 2048  # NXT_PREFIX_MAX_MATCH_PAGES, include/prefix_sharing.h:61


class Pool:
    """memory_manager.c:207-272 (nxt_page_alloc / nxt_page_free /
    nxt_page_ref_inc / nxt_page_ref_dec), one tier, one type."""

    def __init__(self, n: int):
        self.refs = [0] * n
        self.free = collections.deque(range(n))

    def alloc(self) -> int:
        if not self.free:
            return -2
        b = self.free.popleft()
        self.refs[b] = 1
        return b

    def inc(self, b: int) -> int:
        if not 0 <= b < len(self.refs) or self.refs[b] <= 0:
            return -1
        self.refs[b] += 1
        return self.refs[b]

    def dec(self, b: int) -> int:
        if not 0 <= b < len(self.refs) or self.refs[b] <= 0:
            return -1
        self.refs[b] -= 1
        if self.refs[b] == 0:
            self.free.append(b)
        return self.refs[b]


@dataclass(eq=False)
class Node:
    tokens: list
    slots: list
    parent: "Node | None" = None
    children: list = field(default_factory=list)
    nid: int = 0
    last: int = 0
    created: int = 0
    lock: int = 0
    hits: int = 0
    prio: int = 0


class PrefixTree:
    """prefix_sharing.c with slots for page ids.  `pool` None: no page
    references (the reference's tests run without a pool)."""

    def __init__(self, pool: Pool | None = None, block_size: int = 16):
        self.pool, self.bs = pool, block_size
        self.clock = 0
        self.ids = 0
        self.nodes: dict[int, Node] = {}
        self.evictable = 0
        self.protected = 0
        self.root = self._node([], [], 0)  # prefix_sharing.c:194-204
        self.root.lock = 1

    def _tick(self) -> int:
        self.clock += 1
        return self.clock

    def _pages(self, slots) -> list:
        """Distinct pages of a run of slots, ascending: references are taken
        and given back in this order, which fixes the free list's order."""
        return sorted({s // self.bs for s in slots})

    def _node(self, tokens, slots, prio) -> Node:  # node_create, :26-60
        self.ids += 1
        n = Node(list(tokens), list(slots), nid=self.ids, prio=prio)
        n.created = n.last = self._tick()
        if self.pool is not None:
            for p in self._pages(slots):
                self.pool.inc(p)
        self.nodes[n.nid] = n
        return n

    def _destroy(self, n: Node) -> None:  # node_destroy, :63-72
        for c in n.children:
            self._destroy(c)
        if self.pool is not None:
            for p in self._pages(n.slots):
                self.pool.dec(p)
        del self.nodes[n.nid]

    @staticmethod
    def _child(n: Node, tok: int):  # find_child, :75-82
        for c in n.children:
            if c.tokens and c.tokens[0] == tok:
                return c
        return None

    @staticmethod
    def _cpl(a, b) -> int:  # common_prefix_len, :114-120
        i = 0
        while i < min(len(a), len(b)) and a[i] == b[i]:
            i += 1
        return i

    def _split(self, child: Node, k: int) -> Node:  # split_node, :123-188
        head = self._node(child.tokens[:k], child.slots[:k], child.prio)
        head.hits, head.lock, head.parent = child.hits, child.lock, child.parent
        sib = child.parent.children
        sib[sib.index(child)] = head
        before = self._pages(child.slots)
        child.tokens, child.slots = child.tokens[k:], child.slots[k:]
        if self.pool is not None:
            after = set(self._pages(child.slots))
            for p in (p for p in before if p not in after):
                self.pool.dec(p)
        child.parent = head
        head.children.append(child)
        return head

    def match(self, tokens, cap: int = MAX_MATCH):
        """nxt_prefix_match, :211-265 -> (matched tokens, slots, last node)."""
        slots, last = [], self.root
        if not len(tokens):
            return 0, slots, last
        now = self._tick()
        self.root.last = now
        node, off = self.root, 0
        while off < len(tokens):
            c = self._child(node, tokens[off])
            if c is None:
                break
            c.last = now
            c.hits += 1
            m = self._cpl(c.tokens, tokens[off:])
            if len(slots) + m > cap:
                break
            if m < len(c.tokens):
                head = self._split(c, m)
                slots += head.slots
                last = head
                break
            slots += c.slots
            last, off, node = c, off + m, c
        return len(slots), slots, last

    def insert(self, tokens, slots, prio: int = 0) -> int:
        """nxt_prefix_insert, :267-325 (one slot per token)."""
        if not len(tokens):
            return 0
        now = self._tick()
        self.root.last = now
        node, off = self.root, 0
        while off < len(tokens):
            c = self._child(node, tokens[off])
            if c is None:
                break
            c.last = now
            c.prio = max(c.prio, prio)
            m = self._cpl(c.tokens, tokens[off:])
            if m < len(c.tokens):
                node = self._split(c, m)
                node.prio = max(node.prio, prio)
                off += m
                break
            off += m
            node = c
        if off < len(tokens):
            leaf = self._node(tokens[off:], slots[off:], prio)
            leaf.parent = node
            node.children.append(leaf)
            self.evictable += len(tokens) - off
        return off

    def _leaf(self, n: Node) -> bool:  # :359-362
        return n is not self.root and not n.children and n.lock == 0 and len(n.tokens) > 0

    def evict(self, num_tokens: int, until_free: int | None = None) -> int:
        """nxt_prefix_evict, :327-399: the least recently used unlocked leaf,
        again and again (rescanned each time, as the reference does)."""
        evicted = 0
        while True:
            if until_free is not None:
                if len(self.pool.free) >= until_free:
                    break
            elif evicted >= num_tokens:
                break
            leaves = [n for n in self.nodes.values() if self._leaf(n)]
            if not leaves:
                break
            v = min(leaves, key=lambda n: (n.last, n.created))
            evicted += len(v.tokens)
            self.evictable -= len(v.tokens)
            v.parent.children.remove(v)
            self._destroy(v)
        return evicted

    def lock(self, nid: int) -> int:  # nxt_prefix_lock, :401-412
        n = self.nodes.get(nid)
        if n is None:
            return -1
        while n is not None and n is not self.root:
            if n.lock == 0:
                self.evictable -= len(n.tokens)
                self.protected += len(n.tokens)
            n.lock += 1
            n = n.parent
        return 0

    def unlock(self, nid: int) -> int:  # nxt_prefix_unlock, :414-425
        n = self.nodes.get(nid)
        if n is None:
            return -1
        path = []
        while n is not None and n is not self.root:
            path.append(n)
            n = n.parent
        if any(x.lock <= 0 for x in path):
            return -1
        for x in path:
            x.lock -= 1
            if x.lock == 0:
                self.evictable += len(x.tokens)
                self.protected -= len(x.tokens)
        return 0

    def stats(self):
        """(total tokens, node count, evictable, protected): :427-449."""
        return (sum(len(n.tokens) for n in self.nodes.values()), len(self.nodes),
                self.evictable, self.protected)


@dataclass
class Seq:
    tokens: list
    blocks: list
    locked: int = 0
    shared: int = 0


class KvIndex:
    """The sequence rules of the build (admission with copy-on-write of a
    partly matched page, append, release, batch tables and groups)."""

    def __init__(self, num_blocks: int, block_size: int, max_blocks: int):
        self.bs, self.max_blocks = block_size, max_blocks
        self.pool = Pool(num_blocks)
        self.tree = PrefixTree(self.pool, block_size)
        self.seqs: list[Seq | None] = []
        self.free_handles: list[int] = []

    def slot(self, s: Seq, t: int) -> int:
        return s.blocks[t // self.bs] * self.bs + t % self.bs

    def _ensure(self, need: int) -> bool:
        if len(self.pool.free) < need:
            self.tree.evict(0, until_free=need)
        return len(self.pool.free) >= need

    def _handle(self) -> int:
        if self.free_handles:
            return self.free_handles.pop()
        self.seqs.append(None)
        return len(self.seqs) - 1

    def admit(self, tokens):
        """-> (status, info dict, slot_mapping, copy_src, copy_dst)."""
        bs, L = self.bs, len(tokens)
        if L <= 0:
            return -1, None, None, None, None
        if L > self.max_blocks * bs:
            return -3, None, None, None, None
        M, mslots, last = self.tree.match(list(tokens))
        P = 0
        while (P + 1) * bs <= M:
            first = mslots[P * bs]
            if first % bs or mslots[P * bs:(P + 1) * bs] != list(range(first, first + bs)):
                break
            P += 1
        nblocks = -(-L // bs)
        lock = last.nid if M > 0 else 0
        if lock:
            self.tree.lock(lock)
        if not self._ensure(nblocks - P):
            if lock:
                self.tree.unlock(lock)
            return -2, None, None, None, None
        s = Seq(list(tokens), [], lock, P)
        for j in range(P):
            b = mslots[j * bs] // bs
            self.pool.inc(b)
            s.blocks.append(b)
        s.blocks += [self.pool.alloc() for _ in range(P, nblocks)]
        mapping, src, dst = [], [], []
        for t in range(L):
            if t < P * bs:
                mapping.append(-1)
            elif t < M:
                mapping.append(-1)
                src.append(mslots[t])
                dst.append(self.slot(s, t))
            else:
                mapping.append(self.slot(s, t))
        h = self._handle()
        self.seqs[h] = s
        info = dict(seq=h, cached_tokens=M, shared_blocks=P, copy_count=len(src),
                    write_count=L - M)
        return 0, info, mapping, src, dst

    def append(self, h: int, tokens):
        s = self.seqs[h] if 0 <= h < len(self.seqs) else None
        if s is None:
            return -1, None
        L, n = len(s.tokens), len(tokens)
        if L + n > self.max_blocks * self.bs:
            return -3, None
        need = -(-(L + n) // self.bs) - len(s.blocks)
        if need > 0 and not self._ensure(need):
            return -2, None
        s.blocks += [self.pool.alloc() for _ in range(max(need, 0))]
        s.tokens += list(tokens)
        return 0, [self.slot(s, L + i) for i in range(n)]

    def batch_append(self, hs, tokens):
        if len(set(hs)) != len(hs) or any(not 0 <= h < len(self.seqs) or self.seqs[h] is None
                                          for h in hs):
            return -1, None
        if any(len(self.seqs[h].tokens) + 1 > self.max_blocks * self.bs for h in hs):
            return -3, None
        need = sum(len(self.seqs[h].tokens) % self.bs == 0 for h in hs)
        if need > 0 and not self._ensure(need):
            return -2, None
        out = []
        for h, tok in zip(hs, tokens):
            s = self.seqs[h]
            if len(s.tokens) % self.bs == 0:
                s.blocks.append(self.pool.alloc())
            s.tokens.append(tok)
            out.append(self.slot(s, len(s.tokens) - 1))
        return 0, out

    def cache(self, h: int) -> int:
        s = self.seqs[h]
        return self.tree.insert(s.tokens, [self.slot(s, t) for t in range(len(s.tokens))], 0)

    def release(self, h: int, cache: bool) -> int:
        s = self.seqs[h] if 0 <= h < len(self.seqs) else None
        if s is None:
            return -1
        if cache:
            self.cache(h)
        if s.locked:
            self.tree.unlock(s.locked)
        for b in s.blocks:
            self.pool.dec(b)
        self.seqs[h] = None
        self.free_handles.append(h)
        return 0

    def tables(self, hs, max_blocks: int):
        import numpy as np
        bt = np.full((len(hs), max_blocks), -1, dtype=np.int32)
        lens = np.zeros(len(hs), dtype=np.int32)
        for i, h in enumerate(hs):
            s = self.seqs[h]
            bt[i, :len(s.blocks)] = s.blocks
            lens[i] = len(s.tokens)
        return bt, lens


# ---- the reference's own tree and pool, compiled into oracle/_ref (make -C oracle ref)
_REF_DIR = __import__("os").path.join(__import__("os").path.dirname(__file__), "_ref")
REF_PREFIX_SO = _REF_DIR + "/libref_prefix_sharing.so"
REF_POOL_SO = _REF_DIR + "/libref_page_pool.so"


def _ref_lib(path: str):
    import ctypes
    import os
    if not os.path.exists(path):
        return None
    return ctypes.CDLL(path)


class RefPrefixTree:
    """src/core/prefix_sharing.c itself, without a pool.  Nodes are the
    reference's pointers (opaque ints here)."""

    def __init__(self):
        import ctypes
        L = _ref_lib(REF_PREFIX_SO)
        if L is None:
            raise FileNotFoundError(REF_PREFIX_SO)
        vp, i32 = ctypes.c_void_p, ctypes.c_int32
        L.refps_new.restype = vp
        L.refps_free.argtypes = [vp]
        L.refps_match.argtypes = [vp, vp, i32, vp, vp, ctypes.POINTER(vp)]
        L.refps_match.restype = ctypes.c_int
        L.refps_insert.argtypes = [vp, vp, i32, vp, i32, i32]
        L.refps_insert.restype = ctypes.c_int
        L.refps_evict.argtypes = [vp, i32]
        L.refps_evict.restype = ctypes.c_int
        L.refps_lock.argtypes = [vp, vp]
        L.refps_unlock.argtypes = [vp, vp]
        L.refps_stats.argtypes = [vp, vp]
        self.L, self.ct = L, ctypes
        self.t = L.refps_new()

    def close(self):
        if self.t:
            self.L.refps_free(self.t)
            self.t = None

    def match(self, tokens):
        import numpy as np
        ct = self.ct
        tok = np.ascontiguousarray(tokens, dtype=np.int32)
        pages = np.zeros(MAX_MATCH, dtype=np.uint32)
        count = ct.c_int32(0)
        last = ct.c_void_p()
        m = self.L.refps_match(self.t, tok.ctypes.data if len(tok) else None, len(tok),
                               pages.ctypes.data, ct.byref(count), ct.byref(last))
        return m, [int(x) for x in pages[:count.value]], last.value or 0

    def insert(self, tokens, slots, prio=0):
        import numpy as np
        tok = np.ascontiguousarray(tokens, dtype=np.int32)
        sl = np.ascontiguousarray(slots, dtype=np.uint32)
        return self.L.refps_insert(self.t, tok.ctypes.data if len(tok) else None, len(tok),
                                   sl.ctypes.data if len(sl) else None, len(sl), prio)

    def evict(self, n):
        return self.L.refps_evict(self.t, n)

    def lock(self, node):
        self.L.refps_lock(self.t, node)

    def unlock(self, node):
        self.L.refps_unlock(self.t, node)

    def stats(self):
        import numpy as np
        out = np.zeros(4, dtype=np.int32)
        self.L.refps_stats(self.t, out.ctypes.data)
        return tuple(int(x) for x in out)


class RefPool:
    """src/core/memory_manager.c itself: HBM pages of type DATA, ids 0..n-1."""

    def __init__(self, n: int):
        import ctypes
        L = _ref_lib(REF_POOL_SO)
        if L is None:
            raise FileNotFoundError(REF_POOL_SO)
        vp, ci = ctypes.c_void_p, ctypes.c_int
        L.refpool_new.argtypes = [ci]
        L.refpool_new.restype = vp
        L.refpool_free.argtypes = [vp]
        for name in ("refpool_alloc", "refpool_free_count"):
            getattr(L, name).argtypes = [vp]
            getattr(L, name).restype = ci
        for name in ("refpool_ref_inc", "refpool_ref_dec"):
            getattr(L, name).argtypes = [vp, ci]
        L.refpool_refs.argtypes = [vp, ci]
        L.refpool_refs.restype = ci
        self.L, self.p = L, L.refpool_new(n)

    def close(self):
        if self.p:
            self.L.refpool_free(self.p)
            self.p = None

    def alloc(self):
        return self.L.refpool_alloc(self.p)

    def inc(self, b):
        self.L.refpool_ref_inc(self.p, b)

    def dec(self, b):
        self.L.refpool_ref_dec(self.p, b)

    def refs(self, b):
        return self.L.refpool_refs(self.p, b)

    def free_count(self):
        return self.L.refpool_free_count(self.p)
