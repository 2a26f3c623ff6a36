"""The product KV-cache index (libxllm_hip_backend.so host code, through
include/xllm_hip_kv_index.h) against its restatement (oracle/kv_index_oracle.py),
CPU only: the same seeded operations on both give identical results (page
ids, slots, copy lists, eviction counts, statistics, block tables, groups),
and the product keeps the integrity and reference-count properties that pin
the restatement."""
from __future__ import annotations

import random

import numpy as np
import pytest

from oracle import kv_index_oracle as K
from tests.cascade_cases import detect_prefix_groups
from tests.test_kv_index_oracle import SimCache, _rand_tokens, prefix_value
from xllms_amd.kv_index import KvIndex, KvIndexError


def product_admit(ix, tok):
    try:
        info, mapping, src, dst = ix.seq_admit(tok)
    except KvIndexError as e:
        return e.status, None, None, None, None
    return 0, info, list(mapping), list(src), list(dst)


def product_batch_append(ix, hs, toks):
    try:
        return 0, list(ix.batch_append(hs, toks))
    except KvIndexError as e:
        return e.status, None


def check_product(px, ox, cache, live, nb):
    hs = sorted(live)
    if hs:
        bt, lens = px.batch_tables(hs)
        obt, olens = ox.tables(hs, ox.max_blocks)
        assert np.array_equal(bt, obt) and np.array_equal(lens, olens)
        bs = px.block_size
        for i, h in enumerate(hs):
            toks = live[h]
            assert lens[i] == len(toks)
            for t in range(len(toks)):
                assert cache.v[bt[i, t // bs] * bs + t % bs] == prefix_value(toks, t)
        group, blocks = px.batch_prefix_groups(hs)
        og, ob = detect_prefix_groups(obt, olens, bs)
        assert np.array_equal(group, og) and np.array_equal(blocks, ob)
    assert px.blocks_free() == len(ox.pool.free)
    for b in range(nb):
        assert px.block_refs(b) == ox.pool.refs[b]
    assert px.prefix_stats() == ox.tree.stats()


@pytest.mark.parametrize("seed,num_blocks,max_blocks", [(41, 500, 8), (42, 70, 8),
                                                         (43, 20, 6), (44, 2000, 40)])
def test_product_matches_oracle(seed, num_blocks, max_blocks):
    rng = random.Random(seed)
    bs = 16
    px, ox = KvIndex(num_blocks, bs, max_blocks), K.KvIndex(num_blocks, bs, max_blocks)
    cache = SimCache(num_blocks, bs)
    live: dict[int, list] = {}
    prompts: list[list] = []
    for step in range(500):
        op = rng.random()
        if op < 0.3 or not live:
            tok = _rand_tokens(rng, prompts, max_len=90)
            got, want = product_admit(px, tok), ox.admit(tok)
            assert got[0] == want[0], step
            if want[0] == 0:
                assert got[1] == want[1] and got[2:] == want[2:], step
                cache.admit(tok, got[2], got[3], got[4])
                live[want[1]["seq"]] = list(tok)
                prompts.append(tok)
        elif op < 0.6:
            hs = rng.sample(sorted(live), rng.randint(1, len(live)))
            toks = [rng.randint(0, 5) for _ in hs]
            got, want = product_batch_append(px, hs, toks), ox.batch_append(hs, toks)
            assert got == want, step
            if want[0] == 0:
                for h, tk, sl in zip(hs, toks, want[1]):
                    live[h].append(tk)
                    cache.append(live[h], [sl], len(live[h]) - 1)
        elif op < 0.65:
            h = rng.choice(sorted(live))
            n = rng.randint(1, 20)
            toks = [rng.randint(0, 5) for _ in range(n)]
            try:
                got = (0, list(px.seq_append(h, toks)))
            except KvIndexError as e:
                got = (e.status, None)
            want = ox.append(h, toks)
            assert got == want, step
            if want[0] == 0:
                start = len(live[h])
                live[h] += toks
                cache.append(live[h], want[1], start)
        elif op < 0.73:
            h = rng.choice(sorted(live))
            assert px.seq_cache(h) == ox.cache(h), step
        elif op < 0.78:
            tok = _rand_tokens(rng, prompts, max_len=90)
            m, slots, last = px.prefix_match(tok)
            om, oslots, olast = ox.tree.match(tok)
            assert (m, list(slots)) == (om, oslots), step
            assert last == (olast.nid if om else 0)
        elif op < 0.9:
            h = rng.choice(sorted(live))
            c = rng.random() < 0.7
            assert px.seq_release(h, c) == ox.release(h, c) == 0
            del live[h]
        else:
            n = rng.randint(1, 60)
            assert px.prefix_evict(n) == ox.tree.evict(n), step
        check_product(px, ox, cache, live, num_blocks)
    px.close()


def test_lock_unlock_and_ids():
    ix = KvIndex(32, 16, 4)
    b = ix.block_alloc()
    assert ix.prefix_insert([1, 2, 3], [b * 16, b * 16 + 1, b * 16 + 2]) == 0
    m, slots, node = ix.prefix_match([1, 2, 3])
    assert m == 3 and list(slots) == [b * 16, b * 16 + 1, b * 16 + 2] and node != 0
    assert ix.block_refs(b) == 2                     # the caller's and the tree's
    assert ix.prefix_unlock(node) == -1              # never locked
    assert ix.prefix_lock(node) == 0
    assert ix.prefix_stats() == (3, 2, 0, 3)
    assert ix.prefix_evict(10) == 0
    assert ix.prefix_unlock(node) == 0
    assert ix.prefix_evict(10) == 3
    assert ix.prefix_lock(node) == -1                # evicted: the id is refused
    assert ix.block_refs(b) == 1
    assert ix.block_ref_dec(b) == 0 and ix.block_ref_dec(b) == -1
    assert ix.block_ref_inc(b) == -1                 # a free block
    assert ix.block_refs(99) == -1


def test_argument_checks():
    assert KvIndex.__init__  # the binding loads
    with pytest.raises(KvIndexError):
        KvIndex(0, 16, 4)
    with pytest.raises(KvIndexError):
        KvIndex(8, 12, 4)                            # not a power of two
    ix = KvIndex(8, 16, 2)
    with pytest.raises(KvIndexError) as e:
        ix.seq_admit(list(range(33)))                # 3 pages > 2
    assert e.value.status == -3
    with pytest.raises(KvIndexError):
        ix.seq_admit([])
    assert ix.prefix_insert([1, 2], [0, 1]) == -1    # block 0 not held
    info, _, _, _ = ix.seq_admit(list(range(32)))
    with pytest.raises(KvIndexError) as e:
        ix.batch_append([info["seq"]], [5])          # would need a third page
    assert e.value.status == -3
    with pytest.raises(KvIndexError):
        ix.batch_append([info["seq"], info["seq"]], [5, 6])
    with pytest.raises(KvIndexError):
        ix.batch_tables([info["seq"]], 1)
    assert ix.seq_release(info["seq"]) == 0 and ix.seq_release(info["seq"]) == -1
    assert ix.blocks_free() == 8


def test_pool_exhaustion_evicts_the_tree_first():
    ix = KvIndex(4, 16, 4)
    a, _, _, _ = ix.seq_admit(list(range(64)))       # all four pages
    assert ix.blocks_free() == 0
    ix.seq_release(a["seq"], cache=True)             # pages now held by the tree
    assert ix.blocks_free() == 0
    b, mapping, _, _ = ix.seq_admit([9] * 20)        # needs 2: evicts the cached prompt
    assert b["cached_tokens"] == 0 and ix.prefix_stats()[0] == 0
    with pytest.raises(KvIndexError) as e:
        ix.seq_admit([8] * 64)                       # 4 pages, 2 free, nothing to evict
    assert e.value.status == -2
    assert ix.blocks_free() == 2 and ix.seq_len(b["seq"]) == 20
