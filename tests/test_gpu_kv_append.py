"""GPU parity of the KV append (nxt_paged_kv_append / nxt_paged_kv_write_slots)
against the CPU oracle (oracle_paged_kv_append, the restatement of
examples/text_gen.c:1274-1278 over the paged layout).  Bit-exact: the append
is a byte copy, so the whole K and V caches must match the oracle's, which
also shows that nothing outside the target slots was written.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_close
from xllms_amd import paged_attention as PA
from xllms_amd import workloads as W

pytestmark = pytest.mark.gpu

DT = {"fp16": W.FP16, "bf16": W.BF16, "fp32": W.FP32}


def rows(rng, n, kvh, d, kv_dtype):
    """New K/V rows as host element bits in the cache dtype."""
    x = rng.standard_normal((n, kvh, d)).astype(np.float32)
    if kv_dtype == W.FP16:
        return x.astype(np.float16).view(np.uint16)
    if kv_dtype == W.BF16:
        return (x.view(np.uint32) >> 16).astype(np.uint16)
    return x


def host_bits(t, kv_dtype):
    """Raw element bits (the pools hold NaN garbage, so compare bits)."""
    import torch
    if kv_dtype == W.FP32:
        return t.view(torch.int32).cpu().numpy().view(np.uint32)
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def bits(a):
    return a.view(np.uint32) if a.dtype == np.float32 else a


def device_int(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("head_size", [64, 128, 256])
@pytest.mark.parametrize("block_size", [1, 16, 64])
def test_decode_append_bit_exact(cuda, dtype, head_size, block_size):
    kv_dtype = DT[dtype]
    wl = W.small_case(num_seqs=7, H=8, KVH=2, D=head_size, bs=block_size, kv_dtype=kv_dtype,
                      seed=head_size + block_size, lens=[1, 5, 16, 17, 63, 200, 90])
    rng = np.random.default_rng(head_size * 3 + block_size)
    key = rows(rng, wl.num_seqs, wl.num_kv_heads, head_size, kv_dtype)
    value = rows(rng, wl.num_seqs, wl.num_kv_heads, head_size, kv_dtype)
    positions = (wl.seq_lens - 1).astype(np.int32)   # rewrite each sequence's last token
    positions[3] = -1                                # skipped
    positions[4] = wl.max_num_blocks_per_seq * block_size   # past the table: skipped
    want_k, want_v = O.paged_kv_append(wl.key_cache, wl.value_cache, key, value,
                                       block_size=block_size, kv_block_stride=wl.kv_block_stride,
                                       kv_head_stride=wl.kv_head_stride,
                                       block_tables=wl.block_tables, positions=positions)
    dw = W.upload(wl)
    print(f"case {dtype} d={head_size} bs={block_size}", flush=True)
    PA.paged_kv_append(dw.key_cache, dw.value_cache, W.to_torch(key, kv_dtype),
                       W.to_torch(value, kv_dtype), block_tables=dw.block_tables,
                       positions=device_int(positions))
    import torch
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(dw.key_cache, kv_dtype), bits(want_k))
    assert np.array_equal(host_bits(dw.value_cache, kv_dtype), bits(want_v))


@pytest.mark.parametrize("dtype", ["fp16", "fp32"])
def test_slot_mapping_bit_exact(cuda, dtype):
    kv_dtype = DT[dtype]
    wl = W.small_case(num_seqs=4, H=8, KVH=4, D=128, bs=16, kv_dtype=kv_dtype, seed=21,
                      lens=[300, 40, 1, 77])
    rng = np.random.default_rng(22)
    n = 150
    key = rows(rng, n, wl.num_kv_heads, 128, kv_dtype)
    value = rows(rng, n, wl.num_kv_heads, 128, kv_dtype)
    slots = rng.permutation(wl.num_blocks * 16)[:n].astype(np.int32)
    slots[::9] = -1
    want_k, want_v = O.paged_kv_append(wl.key_cache, wl.value_cache, key, value, block_size=16,
                                       kv_block_stride=wl.kv_block_stride,
                                       kv_head_stride=wl.kv_head_stride, slots=slots)
    dw = W.upload(wl)
    PA.paged_kv_append(dw.key_cache, dw.value_cache, W.to_torch(key, kv_dtype),
                       W.to_torch(value, kv_dtype), slot_mapping=device_int(slots))
    import torch
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(dw.key_cache, kv_dtype), bits(want_k))
    assert np.array_equal(host_bits(dw.value_cache, kv_dtype), bits(want_v))


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("head_size", [64, 128])
def test_copy_slots_bit_exact(cuda, dtype, head_size):
    """nxt_paged_kv_copy_slots: rows move slot to slot inside the caches,
    skipped pairs and every other byte unchanged."""
    kv_dtype = DT[dtype]
    wl = W.small_case(num_seqs=4, H=8, KVH=4, D=head_size, bs=16, kv_dtype=kv_dtype,
                      seed=41 + head_size, lens=[300, 40, 1, 77])
    rng = np.random.default_rng(42)
    slots = rng.permutation(wl.num_blocks * 16).astype(np.int32)
    n = 90
    src, dst = slots[:n].copy(), slots[n:2 * n].copy()
    src[::11] = -1
    dst[5::13] = -1
    want_k, want_v = O.paged_kv_copy_slots(wl.key_cache, wl.value_cache, src, dst,
                                           num_kv_heads=4, head_size=head_size, block_size=16,
                                           kv_block_stride=wl.kv_block_stride,
                                           kv_head_stride=wl.kv_head_stride)
    dw = W.upload(wl)
    print(f"case {dtype} d={head_size}", flush=True)
    PA.paged_kv_copy_slots(dw.key_cache, dw.value_cache, device_int(src), device_int(dst))
    import torch
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(dw.key_cache, kv_dtype), bits(want_k))
    assert np.array_equal(host_bits(dw.value_cache, kv_dtype), bits(want_v))


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_decode_step_append_then_attend(cuda, dtype):
    """One decode step as text_gen.c:1274-1281 does it: store the new token at
    position L, then attend over L + 1 tokens; against the oracle doing the
    same two steps on the host."""
    import torch
    kv_dtype = DT[dtype]
    full = W.small_case(num_seqs=6, H=32, KVH=8, D=128, kv_dtype=kv_dtype, seed=31,
                        lens=[16, 1, 400, 33, 1024, 2])      # tables sized for L + 1 tokens
    before = (full.seq_lens - 1).astype(np.int32)
    rng = np.random.default_rng(32)
    key = rows(rng, full.num_seqs, 8, 128, kv_dtype)
    value = rows(rng, full.num_seqs, 8, 128, kv_dtype)
    kc, vc = O.paged_kv_append(full.key_cache, full.value_cache, key, value, block_size=16,
                               kv_block_stride=full.kv_block_stride,
                               kv_head_stride=full.kv_head_stride,
                               block_tables=full.block_tables, positions=before)
    want = O.run_workload(dataclasses.replace(full, key_cache=kc, value_cache=vc),
                          precision="mt")
    dw = W.upload(full)
    PA.paged_kv_append(dw.key_cache, dw.value_cache, W.to_torch(key, kv_dtype),
                       W.to_torch(value, kv_dtype), block_tables=dw.block_tables,
                       positions=device_int(before))
    PA.paged_attention(dw.out, dw.query, dw.key_cache, dw.value_cache, dw.block_tables,
                       dw.seq_lens, num_kv_heads=8, scale=full.scale, kv_dtype=kv_dtype)
    torch.cuda.synchronize()
    assert_close(dw.out.float().cpu().numpy(), want, kv_dtype, f"append+attend {dtype}")


def test_append_rejects_bad_arguments(cuda):
    import torch
    kc = torch.zeros((4, 2, 16, 128), dtype=torch.float16, device="cuda")
    k = torch.zeros((2, 2, 128), dtype=torch.float16, device="cuda")
    bt = device_int(np.zeros((2, 4)))
    pos = device_int([0, 1])
    with pytest.raises(PA.PagedAttentionError) as e:
        PA.paged_kv_append(kc, kc, k, k, block_tables=bt, positions=pos, block_size=12)
    assert e.value.status == PA.NXT_ATTN_E_UNSUPPORTED
    with pytest.raises(PA.PagedAttentionError) as e:
        PA.paged_kv_append(kc, kc, k, k, block_tables=bt, positions=pos, kv_dtype=9)
    assert e.value.status == PA.NXT_ATTN_E_INVALID
