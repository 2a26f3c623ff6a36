"""The seeded input generator and the benchmark workload definitions (CPU)."""
from __future__ import annotations

import math

import numpy as np
import pytest

from xllms_amd import _lib
from xllms_amd import workloads as W


def test_float_to_half_matches_numpy_rne():
    lib = _lib.workload()
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32),
        (rng.standard_normal(5000) * 1e-5).astype(np.float32),      # subnormal range
        (rng.standard_normal(5000) * 3e4).astype(np.float32),       # near overflow
        np.array([0.0, -0.0, 65504.0, 65519.9, 65520.0, 1e6, -1e6, 2**-24, 2**-25,
                  3 * 2**-26, 2**-14, 2**-14 - 2**-25, np.inf, -np.inf], dtype=np.float32),
    ])
    # exact ties of the binary16 grid: x.5 ulp with even and odd kept mantissa
    ties = (np.arange(1024, 1100, dtype=np.float32) + 0.5) * np.float32(2**-10)
    vals = np.concatenate([vals, ties, -ties])
    got = np.array([lib.xw_float_to_half(float(v)) for v in vals], dtype=np.uint16)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    assert (lib.xw_float_to_half(float("nan")) & 0x7C00) == 0x7C00


def test_float_to_bf16_matches_torch_rne():
    import torch
    lib = _lib.workload()
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.standard_normal(20000).astype(np.float32),
                           (rng.standard_normal(2000) * 1e-39).astype(np.float32),
                           np.array([1.00390625, 1.01171875, 3e38, -3e38], dtype=np.float32)])
    got = np.array([lib.xw_float_to_bf16(float(v)) for v in vals], dtype=np.uint16)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


def test_normal_stream_is_deterministic_and_thread_independent():
    a = np.empty(100003, dtype=np.float32)
    b = np.empty(100003, dtype=np.float32)
    W.fill_normal(a, W.FP32, 1234, threads=1)
    W.fill_normal(b, W.FP32, 1234, threads=7)
    assert np.array_equal(a, b)
    c = np.empty(1000, dtype=np.float32)
    W.fill_normal(c, W.FP32, 1234, offset=500)
    assert np.array_equal(c, a[500:1500])
    lib = _lib.workload()
    assert all(lib.xw_normal(1234, i) == a[i] for i in (0, 1, 77, 100002))


def test_normal_stream_statistics():
    x = W.normal_values(2_000_000, 99).astype(np.float64)
    assert abs(x.mean()) < 3e-3
    assert abs(x.std() - 1.0) < 3e-3
    assert abs((np.abs(x) < 1).mean() - 0.6827) < 2e-3
    # 16-bit streams are the fp32 stream rounded once
    h = W.normal_values(1000, 99, kv_dtype=W.FP16)
    assert np.array_equal(h, x[:1000].astype(np.float32).astype(np.float16).view(np.uint16))


def _check_tables(wl, exact_pool: bool):
    bs = wl.block_size
    used = []
    for s, L in enumerate(wl.seq_lens):
        n = -(-int(L) // bs)
        row = wl.block_tables[s]
        assert (row[:n] >= 0).all() and (row[:n] < wl.num_blocks).all()
        assert (row[n:] == -1).all()
        used.extend(row[:n].tolist())
    if exact_pool:
        assert sorted(used) == list(range(wl.num_blocks))
    return used


def test_config1_shape():
    wl = W.config1()
    assert (wl.num_seqs, wl.num_heads, wl.num_kv_heads, wl.head_size, wl.block_size) == (8, 12, 12, 64, 16)
    assert wl.kv_dtype == W.FP32 and math.isclose(wl.scale, 0.125)
    assert wl.seq_lens.min() >= 16 and wl.seq_lens.max() <= 1024
    _check_tables(wl, exact_pool=True)
    assert np.isfinite(wl.key_cache).all()
    assert wl.algorithmic_bytes() == wl.logical_bytes()


def test_ref_bench_shape_defaults():
    """The reference bench's defaults (tests/test_attention_bench.c:34-41):
    16 sequences at the full 1024-token context, 32 q / 8 kv heads, d 128,
    fp16, pages of 16; every page of the pool used exactly once, through a
    permuted (not identity) table."""
    wl = W.ref_bench_shape()
    assert (wl.num_seqs, wl.num_heads, wl.num_kv_heads, wl.head_size, wl.block_size) == (16, 32, 8, 128, 16)
    assert wl.kv_dtype == W.FP16 and math.isclose(wl.scale, 1 / math.sqrt(128), rel_tol=1e-6)
    assert (wl.seq_lens == 1024).all()
    used = _check_tables(wl, exact_pool=True)
    assert wl.num_blocks == 16 * 64
    assert used != list(range(wl.num_blocks))  # not the reference's identity table
    assert wl.name == "refbench-b16-ctx1024-32x8-d128-fp16"
    assert wl.algorithmic_bytes() == wl.logical_bytes()


def test_ref_bench_shape_flags_and_refusals():
    wl = W.ref_bench_shape(batch=3, ctx=100, heads=8, kv_heads=2, head_size=64, kv_dtype=W.BF16)
    assert (wl.num_seqs, wl.num_heads, wl.num_kv_heads, wl.head_size) == (3, 8, 2, 64)
    assert (wl.seq_lens == 100).all() and wl.kv_dtype == W.BF16
    _check_tables(wl, exact_pool=True)
    for bad in (dict(batch=0), dict(ctx=0), dict(heads=12, kv_heads=8), dict(head_size=-1)):
        with pytest.raises(ValueError):
            W.ref_bench_shape(**bad)


def _finite16(bits):
    return (bits & 0x7C00) != 0x7C00


def test_config2_shape_and_garbage():
    wl = W.config2(num_seqs=12)
    assert (wl.num_heads, wl.num_kv_heads, wl.head_size, wl.kv_dtype) == (32, 8, 128, W.FP16)
    assert wl.seq_lens.min() >= 512 and wl.seq_lens.max() <= 4096
    used = set(_check_tables(wl, exact_pool=False))
    assert len(used) * 2 == wl.num_blocks
    unused = sorted(set(range(wl.num_blocks)) - used)
    assert not _finite16(wl.key_cache[unused]).all()        # sentinels present
    bs = wl.block_size
    for s, L in enumerate(wl.seq_lens):
        for j in range(-(-int(L) // bs)):
            blk = wl.block_tables[s, j]
            n = min(bs, int(L) - j * bs)
            assert _finite16(wl.key_cache[blk, :, :n]).all()
            assert _finite16(wl.value_cache[blk, :, :n]).all()
            if n < bs:
                assert not _finite16(wl.key_cache[blk, :, n:]).any()


def test_config2_full_size_description():
    rng = np.random.default_rng(20260002)
    L = rng.integers(512, 4096, size=64, endpoint=True)
    # expectation from the benchmark definition: B=64, E[L]=2304
    assert 64 * 512 <= L.sum() <= 64 * 4096


def test_config3_spikes():
    wl = W.config3(lens=(512, 1024))
    assert list(wl.seq_lens) == [512, 1024]
    k = wl.key_cache.view(np.float16).astype(np.float32)
    ref = np.empty(wl.key_cache.size, dtype=np.float32)
    W.fill_normal(ref, W.FP32, wl.seed * 16 + W.TAG_K)
    ref = ref.reshape(k.shape)
    bs, KVH = wl.block_size, wl.num_kv_heads
    spiked = 0
    for s, Ls in enumerate(wl.seq_lens):
        for t in range(int(Ls)):
            blk = wl.block_tables[s, t // bs]
            for h in range(KVH):
                row, base = k[blk, h, t % bs], ref[blk, h, t % bs]
                if np.array_equal(row, (base * 8).astype(np.float16).astype(np.float32)) and \
                        not np.array_equal(row, base.astype(np.float16).astype(np.float32)):
                    spiked += 1
    assert spiked == round(0.01 * 512 * KVH) + round(0.01 * 1024 * KVH)


@pytest.mark.parametrize("kvh", [8, 4])
def test_config4_shape(kvh):
    wl = W.config4(num_kv_heads=kvh, num_seqs=128)
    assert wl.num_heads == 64 and wl.num_kv_heads == kvh and wl.kv_dtype == W.BF16
    assert wl.seq_lens.min() >= 1 and wl.seq_lens.max() <= 8192
    assert 900 < np.median(wl.seq_lens) < 1200        # log-normal, median exp(mu) = 1024
    _check_tables(wl, exact_pool=False)


def test_config5_prefix_sharing():
    wl = W.config5()
    bs = wl.block_size
    assert wl.num_seqs == 256
    assert (wl.seq_lens == 1).sum() >= 25
    fresh = np.nonzero(wl.seq_lens == 1)[0]
    assert list(fresh[:25]) == list(range(25))
    rest = np.arange(25, 256)
    groups = (rest - 25) % 16
    for g in range(16):
        members = rest[groups == g]
        first = wl.block_tables[members[0]]
        shared = 0
        while all(wl.block_tables[m, shared] == first[shared] for m in members) and first[shared] >= 0:
            shared += 1
        assert shared >= 256 // bs
        # the copied remainder rows of the prefix are identical across members
        blocks = [wl.block_tables[m, shared] for m in members]
        assert len(set(blocks)) == len(members)
    assert wl.algorithmic_bytes() < 0.6 * wl.logical_bytes()
