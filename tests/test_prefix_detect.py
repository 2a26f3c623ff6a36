"""Pins the restatement of the shared-prefix detection rule (CPU only) on
batches whose sharing is known by construction."""
from __future__ import annotations

import numpy as np

from tests.cascade_cases import detect_prefix_groups, shared_case
from xllms_amd import workloads as W


def test_config5_groups_are_the_generators():
    """Config 5 builds 16 groups whose members share floor(P/16) pages; the L=1
    sequences share nothing."""
    wl = W.config5()
    group, blocks = detect_prefix_groups(wl.block_tables, wl.seq_lens, wl.block_size)
    assert len(blocks) == 16
    n_fresh = 25
    assert (group[:n_fresh] == -1).all()
    # generator: sequence n_fresh + i belongs to group i % 16 (round robin)
    gen = (np.arange(wl.num_seqs - n_fresh) % 16)
    # detected ids are numbered by lowest member, which is the round-robin order
    assert np.array_equal(group[n_fresh:], gen)
    for g in range(16):
        members = np.nonzero(group == g)[0]
        lead = members[0]
        P = blocks[g]
        for s in members:
            assert np.array_equal(wl.block_tables[s, :P], wl.block_tables[lead, :P])
        # the page after the prefix is private
        assert len({int(wl.block_tables[s, P]) for s in members}) == len(members)


def test_constructed_groups_and_edge_cases():
    wl, pg, pb = shared_case([(3, [5, 0, 17]), (1, [2, 9]), (4, [1])], singles=[1, 40, 16],
                             H=8, KVH=2, D=64, seed=3)
    group, blocks = detect_prefix_groups(wl.block_tables, wl.seq_lens, wl.block_size)
    # a one-member "group" is not a group; sizes and prefixes as built
    assert list(blocks) == [3, 1]
    assert list(group) == [0, 0, 0, 1, 1, -1, -1, -1, -1]


def test_prefix_is_limited_by_the_shorter_member():
    """Full pages only: a member whose length ends inside the shared run
    limits the group's prefix."""
    wl, pg, pb = shared_case([(4, [3, 3])], H=8, KVH=2, D=64, seed=4)
    lens = wl.seq_lens.copy()
    lens[1] = 2 * 16 + 5          # only 2 full pages
    group, blocks = detect_prefix_groups(wl.block_tables, lens, 16)
    assert list(blocks) == [2] and list(group) == [0, 0]
