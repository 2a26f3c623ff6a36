"""Decode driven by the KV-cache index on the GPU, end to end:

- admissions that share prompts: full pages are shared, a partly matched
  page is copied with nxt_paged_kv_copy_slots;
- prefill writes through the admission's slot mapping
  (nxt_paged_kv_write_slots);
- decode steps through nxt_kv_batch_append, the K/V write and both the plain
  (nxt_paged_attention_ex) and the prefix-aware (nxt_paged_attention_cascade)
  decode, with the index's block tables and prefix groups;
- releases that cache a sequence for later admissions, and eviction.

Every step's outputs are checked against the oracle's attention
(examples/text_gen.c:1284-1310 restated) over each sequence's logical K/V,
which the test builds on the host from the token history alone, without the
index's pages or slots, at the task's fp16 tolerance.  A token's K/V depends
only on its prefix, as in a model, so sequences that share a prefix share
its K/V.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_close
from tests.test_kv_index_oracle import prefix_value
from xllms_amd import paged_attention as PA
from xllms_amd import workloads as W
from xllms_amd.kv_index import KvIndex

pytestmark = pytest.mark.gpu


class Driver:
    def __init__(self, *, num_blocks, max_blocks, KVH=8, H=32, D=128, bs=16):
        import torch
        self.KVH, self.H, self.D, self.bs = KVH, H, D, bs
        self.scale = 1.0 / np.sqrt(D)
        self.ix = KvIndex(num_blocks, bs, max_blocks)
        shape = (num_blocks, KVH, bs, D)
        self.kc = torch.full(shape, float("nan"), dtype=torch.float16, device="cuda")
        self.vc = torch.full(shape, float("nan"), dtype=torch.float16, device="cuda")
        self.live: dict[int, list] = {}
        self._rows: dict[int, np.ndarray] = {}

    def rows(self, tokens, t):
        """fp16 bits [2][KVH][D]: K and V of token t, a function of tokens[0..t]."""
        key = prefix_value(tokens, t)
        r = self._rows.get(key)
        if r is None:
            g = np.random.default_rng(key)
            r = g.standard_normal((2, self.KVH, self.D)).astype(np.float16).view(np.uint16)
            self._rows[key] = r
        return r

    @staticmethod
    def dev(a):
        import torch
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()

    def write(self, rows, slots):
        kv = np.ascontiguousarray(np.stack(rows))                  # [n][2][KVH][D]
        PA.paged_kv_append(self.kc, self.vc, W.to_torch(kv[:, 0].copy(), W.FP16),
                           W.to_torch(kv[:, 1].copy(), W.FP16), slot_mapping=self.dev(slots))

    def admit(self, tokens):
        info, mapping, src, dst = self.ix.seq_admit(tokens)
        if len(src):
            PA.paged_kv_copy_slots(self.kc, self.vc, self.dev(src), self.dev(dst))
        self.write([self.rows(tokens, t) for t in range(len(tokens))], mapping)
        self.live[info["seq"]] = list(tokens)
        return info

    def release(self, h, cache):
        assert self.ix.seq_release(h, cache) == 0
        del self.live[h]

    def logical_oracle(self, hs, q_bits):
        """Oracle attention over K/V laid out from the token histories."""
        lens = np.array([len(self.live[h]) for h in hs], dtype=np.int32)
        pages = -(-lens // self.bs)
        total = int(pages.sum())
        kc = np.zeros((total, self.KVH, self.bs, self.D), dtype=np.uint16)
        vc = np.zeros_like(kc)
        bt = np.full((len(hs), int(pages.max())), -1, dtype=np.int32)
        base = 0
        for i, h in enumerate(hs):
            toks = self.live[h]
            bt[i, :pages[i]] = np.arange(base, base + pages[i])
            for t in range(len(toks)):
                r = self.rows(toks, t)
                kc[base + t // self.bs, :, t % self.bs] = r[0]
                vc[base + t // self.bs, :, t % self.bs] = r[1]
            base += int(pages[i])
        return O.paged_attention(q_bits, kc, vc, bt, lens, num_kv_heads=self.KVH,
                                 scale=self.scale, block_size=self.bs, dtype=W.FP16,
                                 precision="mt")

    def step(self, rng, what):
        """One decode step of every live sequence; returns (groups, blocks)."""
        import torch
        hs = sorted(self.live)
        toks = rng.integers(0, 6, len(hs))
        slots = self.ix.batch_append(hs, toks)
        for h, tk in zip(hs, toks):
            self.live[h].append(int(tk))
        self.write([self.rows(self.live[h], len(self.live[h]) - 1) for h in hs], slots)
        bt, lens = self.ix.batch_tables(hs)
        q_bits = rng.standard_normal((len(hs), self.H, self.D)).astype(np.float16).view(np.uint16)
        q = W.to_torch(q_bits, W.FP16)
        bt_d, lens_d = self.dev(bt), self.dev(lens)
        out = torch.empty((len(hs), self.H, self.D), dtype=torch.float16, device="cuda")
        PA.paged_attention(out, q, self.kc, self.vc, bt_d, lens_d, num_kv_heads=self.KVH,
                           scale=self.scale, kv_dtype=W.FP16)
        group, blocks = self.ix.batch_prefix_groups(hs)
        out2 = torch.empty_like(out)
        pb = blocks if len(blocks) else np.zeros(1, np.int32)
        PA.paged_attention_cascade(out2, q, self.kc, self.vc, bt_d, lens_d, self.dev(group),
                                   self.dev(pb), num_kv_heads=self.KVH, scale=self.scale,
                                   max_groups=len(blocks), kv_dtype=W.FP16)
        torch.cuda.synchronize()
        want = self.logical_oracle(hs, q_bits)
        assert_close(out.float().cpu().numpy(), want, W.FP16, f"{what} plain")
        assert_close(out2.float().cpu().numpy(), want, W.FP16, f"{what} cascade")
        return group, blocks


def test_decode_through_the_index(cuda):
    rng = np.random.default_rng(2026)
    d = Driver(num_blocks=256, max_blocks=48)
    system = list(rng.integers(0, 50, 40))                 # 2.5 pages
    a = d.admit(system + list(rng.integers(0, 50, 60)))
    d.ix.seq_cache(a["seq"])                               # A's prompt becomes shareable
    b = d.admit(system + list(rng.integers(50, 99, 50)))
    assert (b["cached_tokens"], b["shared_blocks"], b["copy_count"]) == (40, 2, 8)
    c = d.admit(d.live[a["seq"]] + list(rng.integers(0, 50, 35)))
    assert (c["cached_tokens"], c["shared_blocks"], c["copy_count"]) == (100, 6, 4)
    d.admit(list(rng.integers(100, 150, 50)))              # shares nothing
    for i in range(6):
        print(f"step {i}", flush=True)
        group, blocks = d.step(rng, f"step {i}")
        assert sorted(group[group >= 0].tolist()) == [0, 0, 0]     # A, B and C
    d.release(a["seq"], cache=True)                        # A's history stays cached
    e = d.admit(d.live[c["seq"]][:100] + list(rng.integers(0, 50, 20)))
    assert e["cached_tokens"] == 100
    for i in range(6, 12):
        print(f"step {i}", flush=True)
        d.step(rng, f"step {i}")
    for h in list(d.live):
        d.release(h, cache=False)
    assert d.ix.prefix_evict(1 << 30) > 0
    assert d.ix.blocks_free() == 256


def test_decode_under_page_pressure(cuda):
    """A pool too small for everything: admissions and appends evict cached
    sequences' pages (never a live sequence's), and results stay exact."""
    rng = np.random.default_rng(7)
    d = Driver(num_blocks=26, max_blocks=12, KVH=2, H=8, D=64)
    prompts = [list(rng.integers(0, 5, n)) for n in (70, 50, 90)]
    for step in range(24):
        if len(d.live) < 3:
            base = prompts[int(rng.integers(0, 3))]
            cut = int(rng.integers(1, len(base)))
            try:
                d.admit(base[:cut] + list(rng.integers(0, 5, int(rng.integers(1, 30)))))
            except Exception as e:                          # pool exhausted: skip
                assert getattr(e, "status", None) == -2
        print(f"pressure step {step} live={len(d.live)} free={d.ix.blocks_free()} "
              f"cached={d.ix.prefix_stats()[0]}", flush=True)
        d.step(rng, f"pressure {step}")
        if step % 5 == 4:
            h = sorted(d.live)[0]
            d.release(h, cache=True)
