"""Seeded random shapes against the oracle: every draw picks a dtype, head
size, kv heads and GQA group, block size, batch, lengths (empty ones
included), softmax scale, split-K partition and entry point at random, so
that the plans (stream-K, the small-batch segment launch with its split,
automatic and explicit partitions) meet combinations the hand-written cases
do not list.  The cascade draws random groups (sizes, prefix lengths, empty
suffixes, unshared sequences) the same way, and the plugin ABI (run_ex)
takes draws like the decode's.  Same tolerances as the parity tests: fp32
rel 1e-5 per (sequence, head), fp16/bf16 atol 2e-3 + rtol 1e-2."""
from __future__ import annotations

import ctypes
import dataclasses

import numpy as np
import pytest

from oracle import oracle as O
from tests.cascade_cases import shared_case
from tests.helpers import assert_close
from xllms_amd import _lib
from xllms_amd import paged_attention as PA
from xllms_amd import workloads as W

pytestmark = pytest.mark.gpu

DT = {"fp16": W.FP16, "bf16": W.BF16, "fp32": W.FP32}
HEAD_SIZES = [32, 64, 80, 96, 112, 128, 192, 256]


def _draw(rng):
    dtype = str(rng.choice(["fp16", "bf16", "fp32"]))
    D = int(rng.choice(HEAD_SIZES))
    bs = int(rng.choice([1, 2, 4, 8, 16, 16, 16, 32, 64]))
    mfma = dtype != "fp32" and D % 32 == 0 and bs >= 16
    groups = [1, 2, 3, 4, 5, 8, 12, 16, 24, 32] + ([48, 64] if mfma else [])
    G = int(rng.choice(groups))
    KVH = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 41))
    top = int(rng.choice([16, 300, 3000]))
    lens = rng.integers(0, top + 1, size=B)
    lens[rng.random(B) < 0.1] = 0
    if lens.max() == 0:
        lens[0] = 1
    part = int(rng.choice([0, 0, 0, 64, 256]))
    entry = str(rng.choice(["nxt_paged_attention_ex", "nxt_paged_attention_noalloc"]))
    return dtype, D, bs, G, KVH, lens.tolist(), part, entry


def _oracle(wl):
    """fp32 draws against the oracle's double-precision form: at 4-16 times
    the reference's scale (scores of tens) the fp32 restatement itself is
    1-2e-5 (relative, per row) off the exact result, the kernels 2-6e-6
    (measured on MI355X over such draws).  fp16/bf16 draws against the fp32
    restatement."""
    return O.run_workload(wl, precision="f64" if wl.kv_dtype == W.FP32 else "mt")


def _rescale(wl, rng):
    """The draw's softmax scale: 1/sqrt(d) times 0.1, 1, 4 or 16 (flat to
    nearly one-hot score rows)."""
    return dataclasses.replace(wl, scale=wl.scale * float(rng.choice([0.1, 1.0, 4.0, 16.0])))


@pytest.mark.parametrize("seed", range(200))
def test_random_decode_matches_oracle(cuda, seed):
    import torch
    rng = np.random.default_rng(1000 + seed)
    dtype, D, bs, G, KVH, lens, part, entry = _draw(rng)
    H = G * KVH
    wl = _rescale(W.small_case(num_seqs=len(lens), H=H, KVH=KVH, D=D, bs=bs,
                               kv_dtype=DT[dtype], seed=seed, lens=lens), rng)
    print(f"case seed={seed} {dtype} d={D} bs={bs} H={H} KVH={KVH} seqs={len(lens)} "
          f"max_len={max(lens)} scale={wl.scale:.4f} partition={part} {entry}", flush=True)
    dw = W.upload(wl)
    fn = getattr(_lib.backend(), entry)
    rc = fn(dw.out.data_ptr(), dw.query.data_ptr(), dw.key_cache.data_ptr(),
            dw.value_cache.data_ptr(), dw.block_tables.data_ptr(), dw.seq_lens.data_ptr(),
            wl.num_seqs, H, D, KVH, ctypes.c_float(wl.scale), wl.max_num_blocks_per_seq, bs,
            dw.key_cache.element_size(), dw.key_cache.stride(0), dw.key_cache.stride(1),
            torch.cuda.current_stream().cuda_stream, wl.kv_dtype, part)
    assert rc == PA.NXT_ATTN_OK, PA.last_status()
    torch.cuda.synchronize()
    assert_close(dw.out.float().cpu().numpy(), _oracle(wl), wl.kv_dtype, f"seed {seed}")


@pytest.mark.parametrize("seed", range(60))
def test_random_cascade_matches_oracle(cuda, seed):
    import torch
    rng = np.random.default_rng(2000 + seed)
    dtype = str(rng.choice(["fp16", "bf16"]))
    D = int(rng.choice([64, 128]))
    KVH = int(rng.choice([1, 2, 8]))
    G = int(rng.choice([1, 4, 8, 16]))
    spec = []
    for _ in range(int(rng.integers(1, 7))):
        members = int(rng.integers(1, 20))
        spec.append((int(rng.integers(1, 40)),
                     [int(x) for x in rng.integers(0, 200, size=members)]))
    singles = [int(x) for x in rng.integers(0, 500, size=int(rng.integers(0, 6)))]
    wl, pg, pb = shared_case(spec, singles=singles, H=G * KVH, KVH=KVH, D=D,
                             kv_dtype=DT[dtype], seed=seed)
    wl = _rescale(wl, rng)
    print(f"case seed={seed} {dtype} d={D} H={G * KVH} KVH={KVH} groups={len(pb)} "
          f"seqs={wl.num_seqs} scale={wl.scale:.4f}", flush=True)
    dw = W.upload(wl)
    d_pg = torch.from_numpy(pg.astype(np.int32)).cuda()
    d_pb = torch.from_numpy(pb.astype(np.int32)).cuda()
    PA.paged_attention_cascade(dw.out, dw.query, dw.key_cache, dw.value_cache, dw.block_tables,
                               dw.seq_lens, d_pg, d_pb, num_kv_heads=KVH, scale=wl.scale,
                               max_groups=len(pb), kv_dtype=wl.kv_dtype)
    torch.cuda.synchronize()
    assert_close(dw.out.float().cpu().numpy(), _oracle(wl), wl.kv_dtype, f"cascade seed {seed}")


@pytest.mark.parametrize("seed", range(40))
def test_random_plugin_run_ex_matches_oracle(cuda, seed):
    """The same draws through the plugin ABI (nxt_backend_init -> run_ex ->
    fini on the reference's descriptor, dlopen'ed like the backend manager)."""
    import torch
    from xllms_amd import backend as B
    rng = np.random.default_rng(3000 + seed)
    dtype, D, bs, G, KVH, lens, part, _ = _draw(rng)
    H = G * KVH
    wl = W.small_case(num_seqs=len(lens), H=H, KVH=KVH, D=D, bs=bs, kv_dtype=DT[dtype],
                      seed=seed, lens=lens)
    print(f"case seed={seed} {dtype} d={D} bs={bs} H={H} KVH={KVH} seqs={len(lens)} "
          f"max_len={max(lens)} partition={part} plugin run_ex", flush=True)
    dw = W.upload(wl)
    plugin = B.LoadedBackend()
    assert plugin.init() == 0
    try:
        ex = B.NxtPagedAttentionInputEx()
        ex.struct_size = ctypes.sizeof(B.NxtPagedAttentionInputEx)
        ex.base = B.make_input(dw.query, dw.key_cache, dw.value_cache, dw.block_tables,
                               dw.seq_lens, num_kv_heads=KVH, scale=wl.scale,
                               stream=torch.cuda.current_stream().cuda_stream)
        ex.kv_dtype = wl.kv_dtype
        ex.partition_tokens = part
        assert plugin.run_ex(ex, dw.out.data_ptr()) == 0
        torch.cuda.synchronize()
    finally:
        assert plugin.fini() == 0
    assert_close(dw.out.float().cpu().numpy(), _oracle(wl), wl.kv_dtype, f"plugin seed {seed}")
