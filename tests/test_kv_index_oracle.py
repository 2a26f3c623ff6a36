"""Pins the restatement of the KV-cache index (oracle/kv_index_oracle.py),
CPU only:

- the reference's own tests of the radix tree (tests/test_prefix_sharing.c)
  and page pool (tests/test_page_pool.c), their asserted values restated;
- the reference's compiled tree and pool (oracle/_ref, built by
  `make -C oracle ref` from src/core/prefix_sharing.c and
  src/core/memory_manager.c + lru_k.c) on seeded random operation sequences;
- brute force: a match equals the longest common prefix with any cached
  sequence, and its slots are those of the earliest sequence that cached
  each position;
- data integrity of the sequence rules: a simulated cache written through
  slot mappings, copy lists and appends holds, at every block-table position
  of every live sequence, the value of exactly that token's prefix;
- reference counts: every page's count equals its holders (sequences and
  tree nodes), and the free list is exactly the pages with none.
"""
from __future__ import annotations

import os
import random

import numpy as np
import pytest

from oracle import kv_index_oracle as K
from tests.cascade_cases import detect_prefix_groups

needs_ref_tree = pytest.mark.skipif(not os.path.exists(K.REF_PREFIX_SO),
                                    reason="oracle/_ref not built (needs the reference tree)")
needs_ref_pool = pytest.mark.skipif(not os.path.exists(K.REF_POOL_SO),
                                    reason="oracle/_ref not built (needs the reference tree)")


# ------------------------------------------------ the reference's own tests, restated
def test_reference_prefix_sharing_suite():
    """tests/test_prefix_sharing.c:26-271, the asserted values."""
    t = K.PrefixTree()                                    # tree_init_destroy :26-41
    assert t.root.lock == 1 and t.stats()[:2] == (0, 1)

    t = K.PrefixTree()                                    # insert_single :44-58
    assert t.insert([1, 2, 3, 4, 5], [100, 101, 102, 103, 104]) == 0
    assert t.stats()[1] >= 2 and t.stats()[0] == 5

    t = K.PrefixTree()                                    # match_full :61-78
    t.insert([10, 20, 30, 40, 50], [200, 201, 202, 203, 204])
    m, slots, _ = t.match([10, 20, 30, 40, 50])
    assert m == 5 and len(slots) == 5 and slots[0] == 200 and slots[4] == 204

    t = K.PrefixTree()                                    # match_partial :81-99
    t.insert([1, 2, 3], [10, 20, 30])
    m, slots, _ = t.match([1, 2, 3, 4, 5])
    assert m == 3 and len(slots) == 3 and slots[0] == 10

    t = K.PrefixTree()                                    # shared_prefix :102-127
    assert t.insert([1, 2, 3, 4, 5], [100, 101, 102, 103, 104]) == 0
    assert t.insert([1, 2, 3, 6, 7], [300, 301, 302, 303, 304]) == 3
    m, slots, _ = t.match([1, 2, 3, 4, 5])
    assert m == 5 and len(slots) == 5

    t = K.PrefixTree()                                    # empty_query :130-145
    t.insert([1, 2, 3], [10, 20, 30])
    m, _, last = t.match([])
    assert m == 0 and last is t.root

    t = K.PrefixTree()                                    # lock_unlock :148-182
    t.insert([7, 8, 9], [70, 80, 90])
    m, _, last = t.match([7, 8, 9])
    assert m == 3
    before = t.stats()[2]
    assert before > 0
    t.lock(last.nid)
    assert t.stats()[2] < before
    t.evict(100)
    assert t.stats()[0] > 0
    t.unlock(last.nid)
    t.evict(100)
    assert t.stats()[0] == 0

    t = K.PrefixTree()                                    # eviction :185-213
    t.insert([1, 2, 3], [10, 20, 30])
    t.insert([4, 5, 6, 7], [40, 50, 60, 70])
    t.insert([8, 9], [80, 90])
    assert t.stats()[0] == 9
    assert t.evict(3) >= 3
    assert t.stats()[0] < 9

    t = K.PrefixTree()                                    # divergent_branches :216-251
    t.insert([1, 2, 3, 4], [100, 101, 102, 103])
    assert t.insert([1, 2, 5, 6], [200, 201, 202, 203]) == 2
    assert t.insert([1, 2, 3, 7, 8], [300, 301, 302, 303, 304]) == 3
    assert t.match([1, 2, 3, 4])[0] == 4
    assert t.match([1, 2, 5, 6])[0] == 4
    assert t.match([1, 2, 3, 7, 8])[0] == 5
    assert t.match([1, 2, 3, 4, 99])[0] == 4

    t = K.PrefixTree()                                    # statistics :254-271
    assert t.stats()[:2] == (0, 1)
    t.insert([1, 2, 3], [10, 20, 30])
    assert t.stats()[:3] == (3, 2, 3)


def test_reference_page_pool_alloc_free():
    """tests/test_page_pool.c: an allocated page has one reference, a
    released one returns to the free list, and ids come from the free list's
    head in order."""
    p = K.Pool(8)
    a = p.alloc()
    assert a == 0 and p.refs[0] == 1 and len(p.free) == 7
    p.inc(a)
    assert p.refs[a] == 2
    p.dec(a)
    assert p.refs[a] == 1 and len(p.free) == 7
    p.dec(a)
    assert p.refs[a] == 0 and len(p.free) == 8 and p.free[-1] == a
    assert [p.alloc() for _ in range(8)] == [1, 2, 3, 4, 5, 6, 7, 0]
    assert p.alloc() == -2


# ------------------------------------------------ against the reference's compiled code
@needs_ref_pool
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_pool_matches_reference_pool(seed):
    rng = random.Random(seed)
    n = 24
    ours, ref = K.Pool(n), K.RefPool(n)
    try:
        held = []
        for _ in range(600):
            op = rng.random()
            if op < 0.4 or not held:
                a, b = ours.alloc(), ref.alloc()
                assert (a if a >= 0 else -1) == b
                if a >= 0:
                    held.append(a)
            elif op < 0.6:
                x = rng.choice(held)
                ours.inc(x)
                ref.inc(x)
                held.append(x)
            else:
                x = held.pop(rng.randrange(len(held)))
                ours.dec(x)
                ref.dec(x)
            assert len(ours.free) == ref.free_count()
            for b in range(n):
                assert ours.refs[b] == ref.refs(b)
    finally:
        ref.close()


def _rand_tokens(rng, stems, max_len=24):
    """A token string that often shares a prefix with an earlier one."""
    if stems and rng.random() < 0.7:
        base = rng.choice(stems)
        cut = rng.randint(0, len(base))
        out = list(base[:cut])
    else:
        out = []
    out += [rng.randint(0, 5) for _ in range(rng.randint(0 if out else 1, max_len))]
    return out


@needs_ref_tree
@pytest.mark.parametrize("seed", [11, 12, 13, 14])
def test_tree_matches_reference_tree(seed):
    """Same operations on the restatement and on prefix_sharing.c: same match
    lengths and page lists, insert results, eviction results and statistics.
    The reference's microsecond clock is, in the test build, a counter that
    advances by one at every reading (oracle/ref_prefix_sharing_wrap.c), so its
    timestamps order the nodes the way the logical clock does."""
    rng = random.Random(seed)
    ours, ref = K.PrefixTree(), K.RefPrefixTree()
    try:
        stems, handles, next_slot = [], [], 1000
        for step in range(260):
            op = rng.random()
            if op < 0.4:
                tok = _rand_tokens(rng, stems)
                slots = list(range(next_slot, next_slot + len(tok)))
                next_slot += len(tok)
                assert ours.insert(tok, slots) == ref.insert(tok, slots), step
                stems.append(tok)
            elif op < 0.75:
                tok = _rand_tokens(rng, stems)
                m, slots, last = ours.match(tok)
                rm, rpages, rlast = ref.match(tok)
                assert (m, slots) == (rm, rpages), step
                assert (last is ours.root) == (rlast == 0)
                if m:
                    handles.append([last.nid, rlast, 0])
            elif op < 0.85 and handles:
                h = rng.choice(handles)
                if h[0] in ours.nodes:
                    if h[2] > 0 and rng.random() < 0.5:
                        ours.unlock(h[0])
                        ref.unlock(h[1])
                        h[2] -= 1
                    else:
                        ours.lock(h[0])
                        ref.lock(h[1])
                        h[2] += 1
            else:
                n = rng.randint(1, 12)
                assert ours.evict(n) == ref.evict(n), step
            assert ours.stats() == ref.stats(), step
    finally:
        ref.close()


@needs_ref_tree
def test_match_cap_keeps_the_reference_pages_before_the_first_skip():
    """At NXT_PREFIX_MAX_MATCH_PAGES the reference skips a node it cannot
    append but keeps counting (prefix_sharing.c:241-257); the restatement ends
    the match there, with exactly the pages the reference listed before the
    skip."""
    a = list(range(2000))
    b = a + [7] * 100
    c = b + [9] * 10
    ours, ref = K.PrefixTree(), K.RefPrefixTree()
    try:
        for tok in (a, b, c):
            slots = list(range(len(tok)))
            ours.insert(tok, slots)
            ref.insert(tok, slots)
        m, slots, _ = ours.match(c)
        rm, rpages, _ = ref.match(c)
        assert rm == 2110 and len(rpages) == 2010       # the reference's gap
        assert m == 2000 and slots == rpages[:2000]
        one = list(range(100, 3100))                     # a single node past the cap
        ours.insert(one, list(range(3000)))
        ref.insert(one, list(range(3000)))
        assert ours.match(one)[0] == 0 and ref.match(one)[1] == []
    finally:
        ref.close()


# ------------------------------------------------ brute force
@pytest.mark.parametrize("seed", [21, 22, 23])
def test_match_and_insert_against_brute_force(seed):
    rng = random.Random(seed)
    t = K.PrefixTree()
    cached: list[tuple[list, list]] = []
    next_slot = 0

    def lcp(a, b):
        i = 0
        while i < min(len(a), len(b)) and a[i] == b[i]:
            i += 1
        return i

    for _ in range(300):
        tok = _rand_tokens(rng, [c[0] for c in cached], max_len=30)
        if rng.random() < 0.5:
            slots = list(range(next_slot, next_slot + len(tok)))
            next_slot += len(tok)
            want = max((lcp(tok, c) for c, _ in cached), default=0)
            assert t.insert(tok, slots) == want
            cached.append((tok, slots))
        else:
            m, slots, _ = t.match(tok)
            assert m == max((lcp(tok, c) for c, _ in cached), default=0)
            for pos in range(m):
                first = next(s for c, s in cached if lcp(tok, c) > pos)
                assert slots[pos] == first[pos]


# ------------------------------------------------ sequence rules: integrity and counts
def prefix_value(tokens, t):
    """The K/V of token t depends on tokens[0..t]: a hash of that prefix."""
    return hash(tuple(tokens[:t + 1])) & 0x7FFFFFFF


class SimCache:
    """A cache of one int per slot, written the way the GPU path writes K/V."""

    def __init__(self, num_blocks, bs):
        self.v = np.full(num_blocks * bs, -1, dtype=np.int64)

    def admit(self, tokens, mapping, src, dst):
        if len(src):
            assert not set(dst) & set(src)
            self.v[np.asarray(dst)] = self.v[np.asarray(src)]   # copies before writes
        for t, s in enumerate(mapping):
            if s >= 0:
                self.v[s] = prefix_value(tokens, t)

    def append(self, tokens, slots, start):
        for i, s in enumerate(slots):
            self.v[s] = prefix_value(tokens, start + i)


def check_integrity(ix, cache, live):
    bs = ix.bs
    for h, tokens in live.items():
        s = ix.seqs[h]
        assert s.tokens == tokens
        for t in range(len(tokens)):
            slot = s.blocks[t // bs] * bs + t % bs
            assert cache.v[slot] == prefix_value(tokens, t), (h, t)


def check_counts(ix):
    holders = [0] * len(ix.pool.refs)
    for s in ix.seqs:
        if s is not None:
            for b in s.blocks:
                holders[b] += 1
    for n in ix.tree.nodes.values():
        for b in {x // ix.bs for x in n.slots}:
            holders[b] += 1
    assert holders == ix.pool.refs
    assert sorted(ix.pool.free) == [b for b in range(len(holders)) if holders[b] == 0]


def run_sequence_ops(ix, rng, steps, cache, on_step=None):
    """Random admissions (often sharing prompts), decode steps, caching,
    releases and evictions on `ix` (oracle or product with the same API)."""
    live: dict[int, list] = {}
    prompts: list[list] = []
    for step in range(steps):
        op = rng.random()
        if op < 0.3 or not live:
            tok = _rand_tokens(rng, prompts, max_len=70)
            st, info, mapping, src, dst = ix.admit(tok)
            if st == 0:
                cache.admit(tok, mapping, src, dst)
                live[info["seq"]] = list(tok)
                prompts.append(tok)
            else:
                assert st in (-2, -3)
        elif op < 0.65:
            hs = rng.sample(sorted(live), rng.randint(1, len(live)))
            toks = [rng.randint(0, 5) for _ in hs]
            st, slots = ix.batch_append(hs, toks)
            if st == 0:
                for h, tk, sl in zip(hs, toks, slots):
                    live[h].append(tk)
                    cache.append(live[h], [sl], len(live[h]) - 1)
            else:
                assert st in (-2, -3)
        elif op < 0.75:
            h = rng.choice(sorted(live))
            ix.cache(h)
        elif op < 0.9:
            h = rng.choice(sorted(live))
            ix.release(h, rng.random() < 0.7)
            del live[h]
        else:
            ix.tree.evict(rng.randint(1, 40))
        if on_step:
            on_step(step, live)
    return live


@pytest.mark.parametrize("seed,num_blocks", [(31, 400), (32, 60), (33, 24)])
def test_sequence_rules_keep_data_and_counts(seed, num_blocks):
    rng = random.Random(seed)
    ix = K.KvIndex(num_blocks, 16, 8)
    cache = SimCache(num_blocks, 16)

    def on_step(step, live):
        check_integrity(ix, cache, live)
        check_counts(ix)
        hs = sorted(live)
        if hs:
            bt, lens = ix.tables(hs, ix.max_blocks)
            for i, h in enumerate(hs):
                assert lens[i] == len(live[h])
                nb = -(-lens[i] // 16)
                assert (bt[i, :nb] >= 0).all() and (bt[i, nb:] == -1).all()

    run_sequence_ops(ix, rng, 400, cache, on_step)


def test_shared_prompt_shares_full_pages_and_copies_the_rest():
    ix = K.KvIndex(64, 16, 16)
    prompt = list(range(100, 140))                       # 40 tokens: 2 full pages + 8
    st, a, m1, _, _ = ix.admit(prompt)
    assert st == 0 and a["cached_tokens"] == 0 and (np.asarray(m1) >= 0).all()
    ix.cache(a["seq"])
    st, b, m2, src, dst = ix.admit(prompt + [7, 8])
    assert st == 0
    assert b["cached_tokens"] == 40 and b["shared_blocks"] == 2 and b["copy_count"] == 8
    sa, sb = ix.seqs[a["seq"]], ix.seqs[b["seq"]]
    assert sb.blocks[:2] == sa.blocks[:2] and sb.blocks[2] != sa.blocks[2]
    assert src == [sa.blocks[2] * 16 + i for i in range(8)]
    assert dst == [sb.blocks[2] * 16 + i for i in range(8)]
    assert m2[:40] == [-1] * 40 and m2[40:] == [sb.blocks[2] * 16 + 8, sb.blocks[2] * 16 + 9]
    bt, lens = ix.tables([a["seq"], b["seq"]], 4)
    group, blocks = detect_prefix_groups(bt, lens, 16)
    assert list(group) == [0, 0] and list(blocks) == [2]
