"""GPU parity of the prefix-aware (cascade) decode and of the shared-prefix
detection.  The cascade computes the same attention as nxt_paged_attention
(the oracle's, examples/text_gen.c:1284-1310 over the paged layout) with
shared prefix pages read once per prefix-batch sequence of 16 or 32 query
rows per kv head; results are checked against the
oracle at the task's tolerances.  Detection is checked against its
restatement (tests/cascade_cases.py), itself pinned on config 5's known
sharing in test_prefix_detect.py."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from tests.cascade_cases import detect_prefix_groups, shared_case
from tests.helpers import assert_close
from xllms_amd import paged_attention as PA
from xllms_amd import workloads as W

pytestmark = pytest.mark.gpu

DT = {"fp16": W.FP16, "bf16": W.BF16, "fp32": W.FP32}


def dev_i32(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


def run_cascade(wl, prefix_group, prefix_blocks, max_groups=None, dw=None):
    import torch
    dw = dw or W.upload(wl)
    pg = dev_i32(prefix_group)
    pb = dev_i32(prefix_blocks if len(prefix_blocks) else np.zeros(1))
    PA.paged_attention_cascade(dw.out, dw.query, dw.key_cache, dw.value_cache, dw.block_tables,
                               dw.seq_lens, pg, pb, num_kv_heads=wl.num_kv_heads, scale=wl.scale,
                               max_groups=len(prefix_blocks) if max_groups is None else max_groups,
                               kv_dtype=wl.kv_dtype)
    torch.cuda.synchronize()
    return dw.out.float().cpu().numpy()


def test_detection_matches_restatement_on_config5(cuda):
    import torch
    wl = W.config5()
    dw = W.upload(wl)
    group, blocks, count = PA.prefix_groups(dw.block_tables, dw.seq_lens, block_size=16)
    torch.cuda.synchronize()
    want_group, want_blocks = detect_prefix_groups(wl.block_tables, wl.seq_lens, 16)
    n = int(count.cpu()[0])
    assert n == len(want_blocks) == 16
    assert np.array_equal(group.cpu().numpy(), want_group)
    assert np.array_equal(blocks.cpu().numpy()[:n], want_blocks)


def test_detection_matches_restatement_on_constructed_batches(cuda):
    import torch
    for seed, spec, singles in [(5, [(3, [5, 0, 17]), (1, [2, 9]), (4, [1])], [1, 40, 16]),
                                (6, [(2, [1] * 30), (7, [0, 0])], [16] * 5),
                                (7, [], [1, 2, 3])]:
        wl, _, _ = shared_case(spec, singles=singles, H=8, KVH=2, D=64, seed=seed)
        dw = W.upload(wl)
        group, blocks, count = PA.prefix_groups(dw.block_tables, dw.seq_lens, block_size=16)
        torch.cuda.synchronize()
        want_group, want_blocks = detect_prefix_groups(wl.block_tables, wl.seq_lens, 16)
        n = int(count.cpu()[0])
        print(f"case seed={seed} groups={n}", flush=True)
        assert n == len(want_blocks)
        assert np.array_equal(group.cpu().numpy(), want_group)
        assert np.array_equal(blocks.cpu().numpy()[:n], want_blocks)


def test_cascade_config5_matches_oracle(cuda):
    import torch
    wl = W.config5()
    dw = W.upload(wl)
    group, blocks, count = PA.prefix_groups(dw.block_tables, dw.seq_lens, block_size=16)
    torch.cuda.synchronize()
    PA.paged_attention_cascade(dw.out, dw.query, dw.key_cache, dw.value_cache, dw.block_tables,
                               dw.seq_lens, group, blocks, num_kv_heads=8, scale=wl.scale,
                               max_groups=blocks.shape[0])
    torch.cuda.synchronize()
    assert_close(dw.out.float().cpu().numpy(), O.run_workload(wl, precision="mt"), wl.kv_dtype,
                 "config5 cascade")


@pytest.mark.parametrize("dtype,D,H,KVH", [("fp16", 128, 32, 8), ("bf16", 128, 64, 8),
                                          ("fp16", 64, 8, 8), ("bf16", 256, 16, 1),
                                          ("fp16", 80, 16, 4), ("fp32", 64, 12, 12),
                                          ("fp32", 128, 32, 8), ("fp16", 96, 64, 2),
                                          ("bf16", 32, 48, 1), ("fp16", 128, 64, 1),
                                          ("bf16", 64, 48, 2), ("bf16", 128, 64, 4),
                                          ("fp16", 32, 16, 4)])
def test_cascade_groups_match_oracle(cuda, dtype, D, H, KVH):
    """Groups of 1..21 members (prefix rows spanning several 16- or 32-row
    prefix sequences), members with an empty suffix, unshared sequences
    (L = 1, L = 0, long), on the MFMA (one and two 16-head row blocks per
    wavefront) and VALU tile paths.  On the MFMA path with head_size <= 128
    the two batches run in one launch with paired prefix head tiles: group 64
    fills a 64-row prefix sequence with one member, group 24 splits some
    members' rows between two prefix sequences."""
    spec = [(5, [3, 0, 40, 16, 1]), (1, [7] * 21), (12, [100]), (2, [0, 0])]
    wl, pg, pb = shared_case(spec, singles=[1, 0, 333], H=H, KVH=KVH, D=D, kv_dtype=DT[dtype],
                             seed=D + H)
    print(f"case {dtype} D={D} H={H} KVH={KVH}", flush=True)
    assert_close(run_cascade(wl, pg, pb), O.run_workload(wl, precision="mt"), wl.kv_dtype,
                 f"cascade {dtype} D={D}")


def test_cascade_ignores_entries_that_do_not_fit(cuda):
    """A group id out of range, or a prefix longer than a member's length or
    table: those sequences are decoded without sharing (same results)."""
    wl, pg, pb = shared_case([(3, [4, 4, 4]), (2, [1, 1])], singles=[50], H=32, KVH=8,
                             D=128, seed=9)
    pg = pg.copy()
    pg[-1] = 7                    # out of range
    pb = pb.copy()
    pb[1] = 40                    # longer than the members' lengths
    assert_close(run_cascade(wl, pg, pb), O.run_workload(wl, precision="mt"), wl.kv_dtype,
                 "cascade with unusable entries")


def test_cascade_without_groups_is_the_plain_decode(cuda):
    wl = W.small_case(num_seqs=5, H=32, KVH=8, D=128, seed=10, max_len=600)
    got = run_cascade(wl, np.full(wl.num_seqs, -1, np.int32), np.zeros(0, np.int32),
                      max_groups=0)
    assert_close(got, O.run_workload(wl, precision="mt"), wl.kv_dtype, "no groups")


def test_cascade_plan_beyond_the_lds_limits(cuda):
    """More than 1024 groups: the plan runs its global-memory kernel instead
    of the LDS one (same results); with fewer, the LDS kernel."""
    rng = np.random.default_rng(14)
    spec = [(1 + int(rng.integers(0, 3)), [int(x) for x in rng.integers(0, 40, size=2)])
            for _ in range(1100)]
    wl, pg, pb = shared_case(spec, singles=[7, 0, 90], H=8, KVH=2, D=64, seed=14)
    print(f"case seqs={wl.num_seqs} groups={len(pb)}", flush=True)
    ref = O.run_workload(wl, precision="mt")
    assert_close(run_cascade(wl, pg, pb), ref, wl.kv_dtype, "cascade, 1100 groups")
    # the same batch with only the first 1000 groups shared (LDS plan)
    pg2 = np.where(pg < 1000, pg, -1).astype(np.int32)
    assert_close(run_cascade(wl, pg2, pb[:1000]), ref, wl.kv_dtype, "cascade, 1000 groups")


def test_cascade_repeated_calls_reuse_the_plan_workspace(cuda):
    """Back-to-back cascade calls of different shapes on one stream."""
    cases = [shared_case([(4, [9, 2, 30])], singles=[5], seed=11),
             shared_case([(1, [3] * 40), (6, [0, 12])], singles=[], seed=12),
             shared_case([(2, [5, 5])], singles=[300, 1], H=64, KVH=8, seed=13)]
    refs = [O.run_workload(wl, precision="mt") for wl, _, _ in cases]
    for rep in range(2):
        for i, ((wl, pg, pb), ref) in enumerate(zip(cases, refs)):
            print(f"case rep={rep} shape={i}", flush=True)
            assert_close(run_cascade(wl, pg, pb), ref, wl.kv_dtype, f"rep {rep} case {i}")


@pytest.mark.parametrize("dtype,D,H,KVH", [("fp16", 128, 32, 8), ("bf16", 64, 48, 2),
                                          ("fp16", 128, 64, 1), ("bf16", 128, 16, 8)])
def test_cascade_inkernel_plan_matches_plan_kernels(cuda, dtype, D, H, KVH):
    """Up to 256 groups the partition launch plans both batches itself (in
    LDS, from the caller's arrays); with more groups the plan kernels build
    them first.  The same batch both ways (the group table padded to 300
    entries, the padding unused; a table holds at most one group per
    sequence), with every group's rows in one 64-row prefix-batch sequence:
    members then differ at most in their order within that sequence's rows,
    which no row's result depends on, and the split is the same, so the
    outputs are bit-identical.  Larger groups (several prefix-batch
    sequences) match the oracle both ways, and the in-kernel plan, whose
    member order is the sequence order, gives bit-identical repeats."""
    import dataclasses
    G = H // KVH
    k = max(1, 64 // G)  # members per prefix-batch sequence
    small = [(5, [3, 0, 40, 16, 1][:k]), (1, [7] * min(21, k)), (12, [100]), (2, [0, 0][:k]),
             (3, [9] * min(40, k))]
    large = [(5, [3, 0, 40, 16, 1]), (1, [7] * 21), (12, [100]), (2, [0, 0]), (3, [9] * 40)]
    for name, spec in (("one prefix sequence per group", small), ("larger groups", large)):
        members = sum(len(sfx) for _, sfx in spec)
        singles = [1, 0, 333, 64] + [20 + 7 * (i % 40) for i in range(max(0, 300 - members - 4))]
        wl, pg, pb = shared_case(spec, singles=singles, H=H, KVH=KVH, D=D, kv_dtype=DT[dtype],
                                 seed=3 * D + H)
        # members of the groups interleaved, as a scheduler's batch has them
        perm = np.random.default_rng(D + H).permutation(wl.num_seqs)
        wl = dataclasses.replace(wl, seq_lens=wl.seq_lens[perm],
                                 block_tables=wl.block_tables[perm], query=wl.query[perm])
        pg = pg[perm]
        print(f"case {dtype} D={D} H={H} KVH={KVH} {name} seqs={wl.num_seqs}", flush=True)
        ref = O.run_workload(wl, precision="mt")
        dw = W.upload(wl)
        got = run_cascade(wl, pg, pb, dw=dw).copy()
        dw.out.zero_()
        again = run_cascade(wl, pg, pb, dw=dw).copy()
        assert np.array_equal(got, again)
        padded = np.concatenate([pb, np.zeros(300 - len(pb), np.int32)]).astype(np.int32)
        dw.out.zero_()
        want = run_cascade(wl, pg, padded, max_groups=300, dw=dw)
        if spec is small:
            assert np.array_equal(got, want)
        assert_close(got, ref, wl.kv_dtype, f"cascade {dtype} D={D}, in-kernel plan")
        assert_close(want, ref, wl.kv_dtype, f"cascade {dtype} D={D}, plan kernels")


def test_cascade_inkernel_plan_with_many_groups(cuda):
    """150 groups (the in-kernel plan lays them out 64 at a time) of one to
    three members: the oracle's results, and bit-identical to the plan
    kernels' (the group table padded to 300 entries)."""
    rng = np.random.default_rng(21)
    spec = [(1 + int(rng.integers(0, 4)), [int(x) for x in rng.integers(0, 60, size=1 + i % 3)])
            for i in range(150)]
    members = sum(len(sfx) for _, sfx in spec)
    wl, pg, pb = shared_case(spec, singles=[1, 0, 45] + [17] * max(0, 300 - members - 3), H=32,
                             KVH=8, D=128, seed=21)
    print(f"case seqs={wl.num_seqs} groups={len(pb)}", flush=True)
    dw = W.upload(wl)
    got = run_cascade(wl, pg, pb, dw=dw).copy()
    padded = np.concatenate([pb, np.zeros(300 - len(pb), np.int32)]).astype(np.int32)
    dw.out.zero_()
    want = run_cascade(wl, pg, padded, max_groups=300, dw=dw)
    assert np.array_equal(got, want)
    assert_close(got, O.run_workload(wl, precision="mt"), wl.kv_dtype, "cascade, 150 groups")


def test_cascade_every_suffix_empty(cuda):
    """Every sequence is a member whose whole context is its group's prefix:
    the suffix batch has no split units, so the launch's workgroups all run
    the prefix batch, and the merge writes the prefix rows."""
    wl, pg, pb = shared_case([(5, [0, 0, 0]), (2, [0, 0]), (9, [0] * 17)], H=32, KVH=8, D=128,
                             seed=23)
    print(f"case seqs={wl.num_seqs}", flush=True)
    assert_close(run_cascade(wl, pg, pb), O.run_workload(wl, precision="mt"), wl.kv_dtype,
                 "cascade, empty suffixes")


@pytest.mark.parametrize("bs,dtype", [(32, "fp16"), (64, "bf16"), (8, "fp16")])
def test_cascade_block_sizes(cuda, bs, dtype):
    """Pages of 32 and 64 tokens (two and four 16-token tiles a page, on the
    MFMA path with the in-kernel plan) and of 8 (the VALU tile path, two
    passes with the prefix fold)."""
    spec = [(3, [5, 0, 40]), (1, [bs] * 9), (6, [1, 2])]
    wl, pg, pb = shared_case(spec, singles=[1, 0, 3 * bs + 5], H=32, KVH=8, D=128, bs=bs,
                             kv_dtype=DT[dtype], seed=50 + bs)
    print(f"case block_size {bs} {dtype}", flush=True)
    assert_close(run_cascade(wl, pg, pb), O.run_workload(wl, precision="mt"), wl.kv_dtype,
                 f"cascade bs={bs}")
