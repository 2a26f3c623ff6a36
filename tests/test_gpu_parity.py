"""GPU parity of the gfx950 paged-decode attention against the CPU oracle.

Every case runs the HIP kernels through the C-ABI (libxllm_hip_backend.so)
and compares with oracle/ (the C restatement of the reference CPU attention,
examples/text_gen.c:1284-1310 over include/operator_api.h paged addressing)
on identical seeded host buffers.  Tolerances are the task's: rel 1e-5 per
(seq, head) for fp32, atol 2e-3 + rtol 1e-2 elementwise for fp16/bf16.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_close
from xllms_amd import paged_attention as PA
from xllms_amd import workloads as W

pytestmark = pytest.mark.gpu

DT = {"fp16": W.FP16, "bf16": W.BF16, "fp32": W.FP32}


def run_gpu(wl, dev=None, *, partition_tokens=0, entry=None, tensors=None, **over):
    import torch
    dw = tensors or W.upload(wl)
    kw = dict(num_kv_heads=wl.num_kv_heads, scale=wl.scale, block_size=wl.block_size,
              partition_tokens=partition_tokens, kv_dtype=wl.kv_dtype, entry=entry)
    kw.update(over)
    PA.paged_attention(dw.out, dw.query, dw.key_cache, dw.value_cache, dw.block_tables,
                       dw.seq_lens, **kw)
    torch.cuda.synchronize()
    return dw.out.float().cpu().numpy()


def oracle(wl, seqs=None):
    return O.run_workload(wl, precision="mt", seqs=seqs)


# ---------------------------------------------------------------- shapes
@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("head_size", [32, 64, 80, 96, 112, 128, 192, 256])
def test_head_sizes(cuda, dtype, head_size):
    wl = W.small_case(num_seqs=3, H=4, KVH=2, D=head_size, kv_dtype=DT[dtype],
                      seed=100 + head_size, max_len=150)
    print(f"case head_size={head_size} {dtype} lens={wl.seq_lens.tolist()}", flush=True)
    assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, f"d={head_size} {dtype}")


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("heads", [(8, 8), (8, 4), (6, 2), (8, 2), (12, 4), (16, 2), (40, 8),
                                   (32, 2), (64, 4), (64, 2), (17, 1), (20, 1), (48, 2)])
def test_gqa_groups(cuda, dtype, heads):
    H, KVH = heads
    wl = W.small_case(num_seqs=3, H=H, KVH=KVH, D=128, kv_dtype=DT[dtype], seed=H * 7 + KVH,
                      max_len=180)
    print(f"case H={H} KVH={KVH} {dtype} lens={wl.seq_lens.tolist()}", flush=True)
    assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, f"H={H} KVH={KVH} {dtype}")


@pytest.mark.parametrize("block_size", [1, 2, 4, 8, 16, 32, 64, 256])
@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
def test_block_sizes(cuda, block_size, dtype):
    wl = W.small_case(num_seqs=3, H=8, KVH=2, D=64, bs=block_size, kv_dtype=DT[dtype],
                      seed=block_size, max_len=300)
    print(f"case block_size={block_size} {dtype} lens={wl.seq_lens.tolist()}", flush=True)
    assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, f"bs={block_size}")


@pytest.mark.parametrize("part", [16, 64, 512, 4096])
def test_split_k_partition_independent(cuda, part):
    """Output does not depend on the split-K partition length (vs the oracle
    and vs one-partition-per-sequence)."""
    wl = W.small_case(num_seqs=4, H=32, KVH=8, D=128, kv_dtype=W.FP16, seed=11,
                      lens=[1, 17, 1500, 3000])
    print(f"case partition={part}", flush=True)
    got = run_gpu(wl, partition_tokens=part)
    assert_close(got, oracle(wl), wl.kv_dtype, f"part={part}")
    whole = run_gpu(wl, partition_tokens=4096)
    assert np.abs(got - whole).max() <= 2e-3


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("head_size", [32, 64, 80, 256])
def test_split_k_every_tile_path(cuda, dtype, head_size):
    """Sequences cut into many pieces (small per-wavefront ranges) on every
    tile path and tile length: the merge must use the same range
    arithmetic as the partition kernel."""
    wl = W.small_case(num_seqs=5, H=8, KVH=2, D=head_size, kv_dtype=DT[dtype], seed=head_size,
                      lens=[0, 1, 63, 700, 1500])
    ref = oracle(wl)
    for part in (64, 128, 1024):
        print(f"case d={head_size} {dtype} partition={part}", flush=True)
        assert_close(run_gpu(wl, partition_tokens=part), ref, wl.kv_dtype, f"part={part}")


@pytest.mark.parametrize("shape", [
    # (H, KVH, D, dtype, num_seqs): >= 512 segments, so the merge runs one
    # workgroup per segment; float4 columns per segment 128 (two threads per
    # column split the partials), 512 and 1024 (threads own 2 / 4 columns),
    # the VALU head tiles of 8 query heads (one and four per kv head), and
    # the MFMA tiles of 32 query heads (384 and 1024 columns).
    (32, 8, 128, "fp16", 64),
    (64, 4, 128, "bf16", 128),
    (32, 2, 256, "fp16", 256),
    (64, 8, 64, "fp32", 64),
    (64, 2, 64, "fp32", 64),
    (48, 2, 64, "bf16", 256),
    (64, 2, 128, "fp16", 256),
    # 64 and 16 columns (64-thread workgroups; four threads per column), and
    # groups whose last head tile is partly filled (40 heads in tiles of
    # 32 + 8, 24 in 16 + 8, 12 in 8 + 4): those segments have at most half
    # the workgroup's columns, and threads split their partials.
    (16, 8, 128, "fp16", 64),
    (8, 8, 64, "bf16", 128),
    (80, 2, 128, "fp16", 128),
    (48, 2, 256, "fp16", 128),
    (12, 1, 128, "fp32", 256),
    # VALU groups of 17-24 heads: three head tiles of 8, the last partly
    # filled (fp32 at 128 and 64 dims; bf16 at head_size 80, which the MFMA
    # path does not take)
    (48, 2, 128, "fp32", 64),
    (40, 2, 64, "fp32", 128),
    (17, 1, 80, "bf16", 256),
])
def test_merge_per_segment_paths(cuda, shape):
    """Batches with enough segments merge with one workgroup per segment:
    every column layout of that merge, with empty sequences and segments cut
    into many partials."""
    H, KVH, D, dtype, nseq = shape
    rng = np.random.default_rng(H * D + KVH)
    lens = rng.integers(1, 700, size=nseq)
    lens[::17] = 0
    lens[5] = 1
    wl = W.small_case(num_seqs=nseq, H=H, KVH=KVH, D=D, kv_dtype=DT[dtype], seed=H + D,
                      lens=lens.tolist())
    ref = oracle(wl)
    for part in (0, 64):
        print(f"case H={H} KVH={KVH} d={D} {dtype} seqs={nseq} partition={part}", flush=True)
        assert_close(run_gpu(wl, partition_tokens=part), ref, wl.kv_dtype,
                     f"H={H} KVH={KVH} d={D} part={part}")


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("head_size", [32, 64, 96, 128, 256])
@pytest.mark.parametrize("heads", [(34, 2), (24, 1), (64, 2), (64, 1), (80, 2)])
def test_mfma_groups_of_17_to_64(cuda, dtype, head_size, heads):
    """Groups of 17-64 query heads on the MFMA path: one wavefront carries two
    16-head row blocks over every K/V tile (head_size <= 128; one block per
    wavefront above), with a partly filled last block for 17, 24 and 40
    heads, and two or more head tiles for 40 and 64; automatic plans and
    explicit partitions (partials of 32 heads merged)."""
    H, KVH = heads
    wl = W.small_case(num_seqs=5, H=H, KVH=KVH, D=head_size, kv_dtype=DT[dtype],
                      seed=H * head_size + KVH, lens=[0, 1, 40, 700, 1500])
    ref = oracle(wl)
    for part in (0, 64):
        print(f"case H={H} KVH={KVH} d={head_size} {dtype} partition={part}", flush=True)
        assert_close(run_gpu(wl, partition_tokens=part), ref, wl.kv_dtype,
                     f"H={H} KVH={KVH} d={head_size} part={part}")


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_auto_split_many_short_segments(cuda, dtype):
    """Automatic plans charge every segment a start-up cost on top of its
    tiles: runs of one-tile sequences between long ones put wavefront range
    boundaries inside segments' start-up units, at their first tile and in
    their middle, and the merge must find the same pieces."""
    rng = np.random.default_rng(7)
    lens = rng.integers(1, 24, size=160)
    lens[::9] = rng.integers(1200, 2600, size=lens[::9].size)
    lens[3] = 0
    lens[4] = 16
    wl = W.small_case(num_seqs=lens.size, H=32, KVH=8, D=128, kv_dtype=DT[dtype], seed=77,
                      lens=lens.tolist())
    print(f"case {dtype} seqs={lens.size} tokens={int(lens.sum())}", flush=True)
    assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, f"auto split {dtype}")


@pytest.mark.parametrize("case", [
    # (H, KVH, D, dtype, tile tokens): fp32 at 64 / 128 / 256 dims (16, 8
    # and 4 tokens per tile), bf16 at head_size 80 (16); groups of 1 and 2
    ("mha64", 12, 12, 64, "fp32", 16),
    ("gqa2-128", 8, 4, 128, "fp32", 8),
    ("mha256", 2, 2, 256, "fp32", 4),
    ("gqa2-80", 4, 2, 80, "bf16", 16),
])
def test_segment_launch_limits(cuda, case):
    """Small VALU batches (at most one segment per CU) run one round of
    16-wavefront workgroups, S = 1, 2 or 4 per segment by the width of the
    block table (S > 1: each workgroup leaves a partial of its share of the
    tiles and a merge combines them), each workgroup taking at most 128
    tiles.  Lengths 0, 1, a tile and one token either side, and tables of
    128 and 256 tiles filled to their last token and one token beyond (the
    wider table: a larger split, or the stream-K plan); then the same
    lengths over batches of 252-256 segments (S = 1, one workgroup per CU
    of the MI355X's 256) and of 264-272 (stream-K)."""
    name, H, KVH, D, dtype, tt = case
    base = [0, 1, tt - 1, tt, tt + 1, 3, 64 * tt]
    for top in (128 * tt, 128 * tt + 1, 256 * tt, 256 * tt + 1):
        lens = base + [top - 1, top]
        wl = W.small_case(num_seqs=len(lens), H=H, KVH=KVH, D=D, kv_dtype=DT[dtype],
                          seed=D + H + top, lens=lens)
        print(f"case {name} lens={lens}", flush=True)
        assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, f"{name} lens {lens}")
    for segs in (256, 272):
        nseq = segs // KVH
        lens = (base * (nseq // len(base) + 1))[:nseq]
        lens[-1] = 128 * tt
        wl = W.small_case(num_seqs=nseq, H=H, KVH=KVH, D=D, kv_dtype=DT[dtype],
                          seed=D + segs, lens=lens)
        print(f"case {name} segments={segs}", flush=True)
        assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, f"{name} segments {segs}")


@pytest.mark.parametrize("case", [
    # (H, KVH, D, dtype, block_size): pages of 4 and 8 tokens under tiles of
    # 16 (fp32 d=64; a load's 4 rows within a page), bf16 at head_size 112
    ("fp32-bs4", 12, 12, 64, "fp32", 4),
    ("fp32-bs8", 8, 4, 64, "fp32", 8),
    ("bf16-112", 4, 2, 112, "bf16", 16),
])
def test_segment_split_small_pages_and_heads(cuda, case):
    """The split segment launch (2 or 4 workgroups per segment, each taking
    every S-th tile) over pages smaller than a tile and at head_size 112,
    with empty, one-token and page-boundary lengths."""
    name, H, KVH, D, dtype, bs = case
    lens = [0, 1, bs - 1, bs, bs + 1, 700, 1500, 2047]
    wl = W.small_case(num_seqs=len(lens), H=H, KVH=KVH, D=D, bs=bs, kv_dtype=DT[dtype],
                      seed=D + bs, lens=lens)
    print(f"case {name} lens={lens}", flush=True)
    assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, f"{name}")


@pytest.mark.parametrize("case", [
    # (name, H, KVH, D, dtype, lengths)
    ("one-long", 12, 12, 64, "fp32", [1024] + [16] * 7),
    ("all-long", 12, 12, 64, "fp32", [2040, 2047, 2048, 1999]),
    ("mostly-empty", 12, 12, 64, "fp32", [0, 0, 1, 0, 0, 0, 0, 1300, 0, 0]),
    ("ragged-128-segs", 4, 4, 64, "fp32", [0, 1, 15, 16, 17, 700, 2000, 4000] * 4),
    ("single-seq-wide", 2, 1, 128, "fp32", [8000]),
    ("gqa2-bf16-80", 8, 4, 80, "bf16", [3000, 5, 1, 0, 2048, 2049]),
])
def test_segment_length_profiles(cuda, case):
    """Small VALU batches (the segment launch, split or not, or stream-K)
    over length profiles: one long sequence among short ones, only long
    ones, mostly empty sequences, a ragged batch of 128 segments, one
    sequence over a wide table, GQA-2 bf16 at head_size 80; each twice in a
    row on one stream and its workspace."""
    name, H, KVH, D, dtype, lens = case
    wl = W.small_case(num_seqs=len(lens), H=H, KVH=KVH, D=D, kv_dtype=DT[dtype],
                      seed=len(lens) + D, lens=lens)
    ref = oracle(wl)
    dw = W.upload(wl)
    for rep in range(2):
        print(f"case {name} rep={rep} lens={lens}", flush=True)
        assert_close(run_gpu(wl, tensors=dw), ref, wl.kv_dtype, f"{name} rep {rep}")


def test_back_to_back_launches_share_a_workspace(cuda):
    """Launches of different shapes on one stream share one split-K
    workspace (grown when a shape needs more): each launch's partials and
    unit prefix are its own, so every result is checked, with repeats of the
    same shape in between."""
    cases = [W.small_case(num_seqs=6, H=32, KVH=8, D=128, kv_dtype=W.FP16, seed=90 + i,
                          max_len=2500) for i in range(3)]
    cases.append(W.small_case(num_seqs=3, H=16, KVH=1, D=64, kv_dtype=W.BF16, seed=99,
                              max_len=3000))
    refs = [oracle(wl) for wl in cases]
    for rep in range(3):
        for i, (wl, ref) in enumerate(zip(cases, refs)):
            for part in (0, 64):
                print(f"case rep={rep} shape={i} partition={part}", flush=True)
                assert_close(run_gpu(wl, partition_tokens=part), ref, wl.kv_dtype,
                             f"rep {rep} case {i} part {part}")


# --------------------------------------------------------- entry points
def test_entry_points_identical(cuda):
    """nxt_paged_attention, _v2 and _flash (operator_api.h:63-115) are one
    implementation: bit-identical outputs."""
    wl = W.small_case(num_seqs=5, H=32, KVH=8, D=128, kv_dtype=W.FP16, seed=3, max_len=900)
    dw = W.upload(wl)
    outs = [run_gpu(wl, entry=e, tensors=dw, kv_dtype=None).copy() for e in PA.ENTRY_POINTS]
    assert_close(outs[0], oracle(wl), wl.kv_dtype, "nxt_paged_attention")
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])


def test_fp32_entry_point(cuda):
    wl = W.config1()
    got = run_gpu(wl, entry="nxt_paged_attention", kv_dtype=None)
    assert_close(got, oracle(wl), W.FP32, "config1 via nxt_paged_attention")


# ------------------------------------------------------- invariants
def test_single_token_returns_v_exactly(cuda):
    """L = 1: softmax weight 1, output = V row bit-for-bit."""
    for dt in (W.FP16, W.BF16, W.FP32):
        wl = W.small_case(num_seqs=4, H=8, KVH=2, D=128, kv_dtype=dt, seed=5, lens=[1, 1, 1, 1])
        got = run_gpu(wl)
        v = O.widen(wl.value_cache, dt)
        G = wl.group
        for s in range(wl.num_seqs):
            blk = wl.block_tables[s, 0]
            for h in range(wl.num_heads):
                assert np.array_equal(got[s, h], v[blk, h // G, 0]), (dt, s, h)


def test_constant_keys_give_mean_of_v(cuda):
    wl = W.small_case(num_seqs=2, H=8, KVH=2, D=64, kv_dtype=W.FP32, seed=9, lens=[37, 300],
                      poison=False)
    wl.key_cache[...] = 0.5
    got = run_gpu(wl)
    v = wl.value_cache
    G = wl.group
    for s, L in enumerate(wl.seq_lens):
        rows = np.stack([v[wl.block_tables[s, t // 16], :, t % 16, :] for t in range(L)])
        mean = rows.astype(np.float64).mean(axis=0)  # [KVH][D]
        for h in range(wl.num_heads):
            np.testing.assert_allclose(got[s, h], mean[h // G], rtol=1e-5, atol=2e-5)


def test_page_permutation_invariance(cuda):
    """Relabelling physical pages together with the table: identical bits."""
    wl = W.small_case(num_seqs=4, H=16, KVH=4, D=128, kv_dtype=W.BF16, seed=21, max_len=700)
    a = run_gpu(wl).copy()
    perm = np.random.default_rng(1).permutation(wl.num_blocks).astype(np.int32)
    wl.key_cache = np.ascontiguousarray(wl.key_cache[np.argsort(perm)])
    wl.value_cache = np.ascontiguousarray(wl.value_cache[np.argsort(perm)])
    bt = wl.block_tables.copy()
    bt[bt >= 0] = perm[bt[bt >= 0]]
    wl.block_tables = bt
    b = run_gpu(wl)
    assert np.array_equal(a, b)


def test_garbage_isolation(cuda):
    """NaN/Inf in unused pages and in tail slots never reach the output."""
    clean = W.small_case(num_seqs=6, H=32, KVH=8, D=128, kv_dtype=W.FP16, seed=33,
                         max_len=400, poison=False)
    dirty = W.small_case(num_seqs=6, H=32, KVH=8, D=128, kv_dtype=W.FP16, seed=33,
                         max_len=400, poison=True)
    a, b = run_gpu(clean), run_gpu(dirty)
    assert np.isfinite(b).all()
    assert np.array_equal(a, b)


def test_identical_heads_in_group(cuda):
    """Query heads h of one group share kv head h/G (not h % KVH): equal Q rows
    in a group give equal outputs, and each group follows its own kv head."""
    wl = W.small_case(num_seqs=2, H=8, KVH=2, D=128, kv_dtype=W.FP16, seed=44, max_len=200)
    G = wl.group
    for s in range(wl.num_seqs):
        for h in range(wl.num_heads):
            wl.query[s, h] = wl.query[s, (h // G) * G]
    got = run_gpu(wl)
    for h in range(wl.num_heads):
        assert np.array_equal(got[:, h], got[:, (h // G) * G])
    assert not np.array_equal(got[:, 0], got[:, G])
    assert_close(got, oracle(wl), wl.kv_dtype, "grouped heads")


def test_empty_and_negative_entries(cuda):
    """seq_len 0 -> zero row; a negative table entry inside the context is
    skipped (never dereferenced), as in the oracle."""
    wl = W.small_case(num_seqs=4, H=8, KVH=2, D=128, kv_dtype=W.FP16, seed=55,
                      lens=[0, 40, 100, 64])
    wl.block_tables[2, 2] = -1
    got = run_gpu(wl)
    assert (got[0] == 0).all()
    assert_close(got, oracle(wl), wl.kv_dtype, "negative entries")


def test_padded_strides(cuda):
    """Non-default kv_block_stride / kv_head_stride are honoured."""
    import torch
    wl = W.small_case(num_seqs=3, H=8, KVH=2, D=64, kv_dtype=W.FP16, seed=66, max_len=250)
    pad_head, pad_block = 8 * 64, 3 * 64
    nb, KVH, bs, D = wl.key_cache.shape
    hs = bs * D + pad_head
    bsd = KVH * hs + pad_block
    def padded(a):
        buf = np.full(nb * bsd, 0x7E00, dtype=np.uint16)  # NaN filler
        for h in range(KVH):
            for b in range(nb):
                buf[b * bsd + h * hs:b * bsd + h * hs + bs * D] = a[b, h].reshape(-1)
        return buf
    dw = W.upload(wl)
    dw.key_cache = W.to_torch(padded(wl.key_cache), wl.kv_dtype)
    dw.value_cache = W.to_torch(padded(wl.value_cache), wl.kv_dtype)
    got = run_gpu(wl, tensors=dw, kv_block_stride=bsd, kv_head_stride=hs,
                  max_num_blocks_per_seq=wl.max_num_blocks_per_seq)
    assert_close(got, oracle(wl), wl.kv_dtype, "padded strides")
    del torch


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
def test_context_bound_splits_launches(cuda, dtype):
    """A block table bounding 2^28 tokens per sequence (32 kv heads x 2^24
    tiles = 2^29 tiles per sequence) exceeds the 2^30 tiles one launch may
    index: the batch goes in launches of two sequences each, with the same
    results."""
    import dataclasses
    wl = W.small_case(num_seqs=5, H=32, KVH=32, D=64, kv_dtype=DT[dtype], seed=77,
                      lens=[0, 1, 50, 200, 700])
    max_blocks = 1 << 24
    bt = np.full((wl.num_seqs, max_blocks), -1, dtype=np.int32)
    bt[:, :wl.max_num_blocks_per_seq] = wl.block_tables
    wl = dataclasses.replace(wl, block_tables=bt)
    print(f"case {dtype} max_blocks={max_blocks}", flush=True)
    assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, f"context bound {dtype}")


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
def test_many_sequences_split_launches(cuda, dtype):
    """More sequences than one launch takes (8192: each workgroup scans the
    batch's split units in LDS): 8192 + 301 short sequences go in two
    launches, the second of 301 sequences, with empty ones on both sides of
    the cut."""
    rng = np.random.default_rng(8493)
    lens = rng.integers(0, 40, size=8192 + 301)
    lens[8190:8195] = [0, 33, 0, 1, 17]
    lens[0] = 39
    wl = W.small_case(num_seqs=lens.size, H=8, KVH=2, D=64, kv_dtype=DT[dtype], seed=8493,
                      lens=lens.tolist())
    print(f"case {dtype} seqs={lens.size}", flush=True)
    assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, f"{lens.size} sequences {dtype}")


# ---------------------------------------------------- benchmark configs
def test_config1_full(cuda):
    wl = W.config1()
    assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, "config1")


def test_config2_full(cuda):
    wl = W.config2()
    stats = assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, "config2")
    print("config2", stats)


def test_config3_long_context(cuda):
    wl = W.config3()
    stats = assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, "config3")
    print("config3", stats)


@pytest.mark.parametrize("kvh", [8, 4])
def test_config4_bf16(cuda, kvh):
    """Config 4 at its full batch of 128 sequences, GQA 8 and GQA 16."""
    wl = W.config4(num_kv_heads=kvh)
    assert wl.num_seqs == 128
    stats = assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, f"config4 kvh={kvh}")
    print("config4", kvh, stats)


def test_config5_shared_prefix(cuda):
    wl = W.config5()
    stats = assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, "config5")
    print("config5", stats)


@pytest.mark.parametrize("shape", [
    # the reference bench's defaults, then its flags at other values
    dict(),
    dict(batch=4, ctx=3000, heads=64, kv_heads=8, kv_dtype=W.BF16),
    dict(batch=32, ctx=77, heads=12, kv_heads=12, head_size=64, kv_dtype=W.FP32),
])
def test_reference_bench_shape(cuda, shape):
    """The reference bench's workload (tests/test_attention_bench.c:34-41,
    every sequence at the full context) with seeded data and a permuted
    table, at its defaults and at other --batch/--ctx/--heads values."""
    wl = W.ref_bench_shape(**shape)
    print(f"case {wl.name}", flush=True)
    assert_close(run_gpu(wl), oracle(wl), wl.kv_dtype, wl.name)


# ------------------------------------------------------ error handling
def test_unsupported_shapes_leave_output_untouched(cuda):
    import torch
    wl = W.small_case(num_seqs=2, H=8, KVH=2, D=128, kv_dtype=W.FP16, seed=77, max_len=64)
    dw = W.upload(wl)
    sentinel = dw.out.clone()
    lib = PA._lib.backend()
    import ctypes
    base = [dw.out.data_ptr(), dw.query.data_ptr(), dw.key_cache.data_ptr(),
            dw.value_cache.data_ptr(), dw.block_tables.data_ptr(), dw.seq_lens.data_ptr()]
    def call(**kw):
        a = dict(num_seqs=2, num_heads=8, head_size=128, num_kv_heads=2, scale=0.1,
                 maxb=wl.max_num_blocks_per_seq, bs=16, dtype_size=2, kbs=wl.kv_block_stride,
                 khs=wl.kv_head_stride)
        a.update(kw)
        lib.nxt_paged_attention(*base, a["num_seqs"], a["num_heads"], a["head_size"],
                                a["num_kv_heads"], ctypes.c_float(a["scale"]), a["maxb"], a["bs"],
                                a["dtype_size"], a["kbs"], a["khs"],
                                torch.cuda.current_stream().cuda_stream)
        return lib.nxt_attn_last_status()
    assert call(head_size=100) == PA.NXT_ATTN_E_UNSUPPORTED
    assert call(dtype_size=3) == PA.NXT_ATTN_E_UNSUPPORTED
    assert call(num_heads=7) == PA.NXT_ATTN_E_INVALID
    assert call(bs=12) == PA.NXT_ATTN_E_UNSUPPORTED
    assert call(kbs=wl.kv_block_stride + 3) == PA.NXT_ATTN_E_UNSUPPORTED
    assert call(num_seqs=-1) == PA.NXT_ATTN_E_INVALID
    assert call(num_heads=256, num_kv_heads=2) == PA.NXT_ATTN_E_UNSUPPORTED  # group 128 > 64
    assert call(num_heads=128, num_kv_heads=2, dtype_size=4) == PA.NXT_ATTN_E_UNSUPPORTED  # fp32: > 32
    torch.cuda.synchronize()
    assert torch.equal(dw.out.view(torch.int16), sentinel.view(torch.int16))
    assert call() == PA.NXT_ATTN_OK
    assert call(num_seqs=0) == PA.NXT_ATTN_OK
