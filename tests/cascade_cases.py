"""Batches with shared prefixes for the cascade tests, and the restatement of
the shared-prefix detection rule (nxt_paged_prefix_groups) in plain Python."""
from __future__ import annotations

import dataclasses

import numpy as np

from xllms_amd import workloads as W


def detect_prefix_groups(block_tables: np.ndarray, seq_lens: np.ndarray, block_size: int):
    """Sequences whose first page is the same physical page form a group (>= 2
    members); its prefix is the longest run of leading pages every member
    shares with the lowest-numbered member, counting pages full in both.
    Groups are numbered by lowest member.  Returns (prefix_group [B],
    prefix_blocks [num_groups])."""
    B, mb = block_tables.shape
    L = np.clip(seq_lens.astype(np.int64), 0, mb * block_size)
    by_key: dict[int, list[int]] = {}
    for s in range(B):
        if L[s] >= block_size and block_tables[s, 0] >= 0:
            by_key.setdefault(int(block_tables[s, 0]), []).append(s)
    found = []
    for members in by_key.values():
        if len(members) < 2:
            continue
        lead = members[0]
        P = None
        for s in members:
            n = min(L[s], L[lead]) // block_size
            k = 0
            while k < n and block_tables[s, k] == block_tables[lead, k]:
                k += 1
            P = k if P is None else min(P, k)
        if P >= 1:
            found.append((lead, members, P))
    found.sort()
    group = np.full(B, -1, dtype=np.int32)
    blocks = np.zeros(len(found), dtype=np.int32)
    for gid, (_, members, P) in enumerate(found):
        group[members] = gid
        blocks[gid] = P
    return group, blocks


def shared_case(groups, *, singles=(), H=32, KVH=8, D=128, bs=16, kv_dtype=W.FP16, seed=0):
    """groups: list of (prefix_blocks, [suffix tokens of each member]); every
    member of a group reads the group's first member's pages for its first
    prefix_blocks pages.  singles: lengths of unshared sequences.  Returns the
    workload and the caller-side grouping (prefix_group, prefix_blocks)."""
    lens, owner = [], []
    for g, (P, suffixes) in enumerate(groups):
        for sfx in suffixes:
            lens.append(P * bs + sfx)
            owner.append(g)
    for L in singles:
        lens.append(L)
        owner.append(-1)
    wl = W.small_case(num_seqs=len(lens), H=H, KVH=KVH, D=D, bs=bs, kv_dtype=kv_dtype, seed=seed,
                      lens=lens)
    bt = wl.block_tables.copy()
    owner = np.asarray(owner)
    for g, (P, _) in enumerate(groups):
        members = np.nonzero(owner == g)[0]
        for s in members[1:]:
            bt[s, :P] = bt[members[0], :P]
    wl = dataclasses.replace(wl, block_tables=bt)
    prefix_group = owner.astype(np.int32)
    prefix_blocks = np.array([P for P, _ in groups], dtype=np.int32)
    return wl, prefix_group, prefix_blocks
