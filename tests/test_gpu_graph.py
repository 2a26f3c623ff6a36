"""The decode entry points inside a HIP graph.  A call is captured once on a
stream (torch.cuda.graph) and replayed with new inputs written in place
between replays: new queries, and new lengths (shorter, or empty) over the
same block tables.  Every launch reads the lengths, tables and queries from
device memory when it runs, so a replay computes what an eager call computes
on the same inputs, bit for bit; each replay is checked against an eager call
made after it, with the program's own eager work and synchronizations
between replays.  The allocating entry points get their stream's workspace
from a warm-up call before the capture; nxt_paged_attention_noalloc needs
none."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from tests.cascade_cases import shared_case
from xllms_amd import _lib
from xllms_amd import paged_attention as PA
from xllms_amd import workloads as W

pytestmark = pytest.mark.gpu


def _replays(call, dw, mutate, reps=4):
    import torch
    s = torch.cuda.Stream()
    out_g = torch.zeros_like(dw.out)
    out_e = torch.zeros_like(dw.out)
    with torch.cuda.stream(s):
        call(out_g, s)  # warm-up: the stream's workspace exists before the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
        call(out_g, s)
    torch.cuda.synchronize()
    rng = np.random.default_rng(5)
    for rep in range(reps):
        mutate(rng, rep)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        out_e.zero_()
        call(out_e, torch.cuda.current_stream())
        torch.cuda.synchronize()
        print(f"case replay {rep}", flush=True)
        assert torch.equal(out_g, out_e), f"replay {rep} differs from the eager call"
        assert bool(torch.isfinite(out_g.float()).all())
    del g


def _new_queries_and_lengths(wl, dw, floor=None):
    """In-place mutation: fresh queries, and lengths drawn in [floor, L]
    (floor: per-sequence lower bound, default 0) of the original lengths L."""
    import torch
    lens0 = wl.seq_lens.astype(np.int64)
    lo = np.zeros_like(lens0) if floor is None else floor.astype(np.int64)
    qshape = tuple(dw.query.shape)

    def mutate(rng, rep):
        q = torch.from_numpy(rng.standard_normal(qshape).astype(np.float32))
        dw.query.copy_(q.to(dw.query.dtype))
        lens = lens0 if rep == 0 else rng.integers(lo, lens0, endpoint=True)
        dw.seq_lens.copy_(torch.from_numpy(lens.astype(np.int32)))
    return mutate


def _decode_call(wl, dw, entry):
    lib = _lib.backend()
    fn = getattr(lib, entry)

    def call(out, stream):
        rc = fn(out.data_ptr(), dw.query.data_ptr(), dw.key_cache.data_ptr(),
                dw.value_cache.data_ptr(), dw.block_tables.data_ptr(), dw.seq_lens.data_ptr(),
                wl.num_seqs, wl.num_heads, wl.head_size, wl.num_kv_heads,
                ctypes.c_float(wl.scale), wl.max_num_blocks_per_seq, wl.block_size,
                dw.key_cache.element_size(), dw.key_cache.stride(0), dw.key_cache.stride(1),
                stream.cuda_stream, wl.kv_dtype, 0)
        assert rc == PA.NXT_ATTN_OK, PA.last_status()
    return call


@pytest.mark.parametrize("entry", ["nxt_paged_attention_ex", "nxt_paged_attention_noalloc"])
@pytest.mark.parametrize("dtype,H,KVH,D,B", [("fp16", 32, 8, 128, 24), ("bf16", 64, 4, 128, 24),
                                            ("fp32", 12, 12, 64, 24), ("fp32", 12, 12, 64, 8)])
def test_decode_replays_in_a_graph(cuda, entry, dtype, H, KVH, D, B):
    """(The fp32 batch of 8 sequences, 96 segments, runs one workgroup per
    segment and no merge; the others the stream-K plan and a merge.)"""
    kv = {"fp16": W.FP16, "bf16": W.BF16, "fp32": W.FP32}[dtype]
    wl = W.small_case(num_seqs=B, H=H, KVH=KVH, D=D, kv_dtype=kv, seed=41 + H, max_len=900)
    print(f"case {entry} {dtype} H={H} KVH={KVH} D={D} seqs={B}", flush=True)
    dw = W.upload(wl)
    _replays(_decode_call(wl, dw, entry), dw, _new_queries_and_lengths(wl, dw))


@pytest.mark.parametrize("groups", [4, 300])
def test_cascade_replays_in_a_graph(cuda, groups):
    """The cascade, with the partition launch planning both batches (4
    groups) or the plan kernels first (a group table of 300): members keep
    their shared prefix, their suffixes change length."""
    import torch
    spec = [(5, [3, 0, 40, 16, 1]), (1, [7] * 21), (12, [100]), (2, [0, 0])]
    singles = [1, 0, 333] + [20 + 7 * (i % 40) for i in range(max(0, groups - 32))]
    wl, pg, pb = shared_case(spec, singles=singles, H=32, KVH=8, D=128, seed=43)
    table = np.zeros(groups, np.int32)
    table[:len(pb)] = pb
    print(f"case cascade seqs={wl.num_seqs} group table {groups}", flush=True)
    dw = W.upload(wl)
    d_pg = torch.from_numpy(pg.astype(np.int32)).cuda()
    d_pb = torch.from_numpy(table).cuda()
    floor = np.where(pg >= 0, table[np.maximum(pg, 0)] * wl.block_size, 0)

    def call(out, stream):
        PA.paged_attention_cascade(out, dw.query, dw.key_cache, dw.value_cache, dw.block_tables,
                                   dw.seq_lens, d_pg, d_pb, num_kv_heads=wl.num_kv_heads,
                                   scale=wl.scale, max_groups=groups, stream=stream)
    _replays(call, dw, _new_queries_and_lengths(wl, dw, floor))


def test_captured_workspace_outlives_growth(cuda):
    """A graph captured over nxt_paged_attention_ex holds its stream's
    workspace: a larger eager call on that stream afterwards gets a new
    buffer beside it (the old one is kept for the graph), and every replay
    still computes what an eager call computes."""
    import torch
    small = W.small_case(num_seqs=8, H=32, KVH=8, D=128, kv_dtype=W.FP16, seed=61, max_len=600)
    big = W.small_case(num_seqs=64, H=64, KVH=2, D=128, kv_dtype=W.FP16, seed=62,
                       lens=[2000] * 64)
    dws, dwb = W.upload(small), W.upload(big)
    call_small, call_big = _decode_call(small, dws, "nxt_paged_attention_ex"), \
        _decode_call(big, dwb, "nxt_paged_attention_ex")
    s = torch.cuda.Stream()
    out_g = torch.zeros_like(dws.out)
    out_e = torch.zeros_like(dws.out)
    with torch.cuda.stream(s):
        call_small(out_g, s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
        call_small(out_g, s)
    torch.cuda.synchronize()
    # grows s's workspace from the small plan's to the 32-head plan's (~65 MiB)
    out_b = torch.zeros_like(dwb.out)
    with torch.cuda.stream(s):
        call_big(out_b, s)
    torch.cuda.synchronize()
    from oracle import oracle as O
    from tests.helpers import assert_close
    print("case big call after the capture", flush=True)
    assert_close(out_b.float().cpu().numpy(), O.run_workload(big, precision="mt"), W.FP16,
                 "big eager call")
    mutate = _new_queries_and_lengths(small, dws)
    rng = np.random.default_rng(9)
    for rep in range(3):
        mutate(rng, rep)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        out_e.zero_()
        call_small(out_e, torch.cuda.current_stream())
        torch.cuda.synchronize()
        print(f"case replay after growth {rep}", flush=True)
        assert torch.equal(out_g, out_e), f"replay {rep} after growth differs from the eager call"
    del g


def test_capture_that_needs_a_new_workspace_is_refused(cuda):
    """A call captured on a stream that has no workspace of the size it
    needs returns NXT_ATTN_E_UNSUPPORTED and enqueues nothing (growing would
    need a queue wait and an allocation inside the capture)."""
    import torch
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    raw = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(raw)) == 0
    try:
        wl = W.small_case(num_seqs=6, H=32, KVH=8, D=128, kv_dtype=W.FP16, seed=63,
                          max_len=900)
        dw = W.upload(wl)
        dw.out.fill_(3.0)
        sentinel = dw.out.clone()
        s = torch.cuda.ExternalStream(raw.value)
        torch.cuda.synchronize()
        call = _decode_call(wl, dw, "nxt_paged_attention_ex")
        lib = _lib.backend()
        fn = lib.nxt_paged_attention_ex
        g = torch.cuda.CUDAGraph()
        print("case capture without a warm-up call", flush=True)
        with torch.cuda.graph(g, stream=s, capture_error_mode="relaxed"):
            dw.out.add_(0)
            rc = fn(dw.out.data_ptr(), dw.query.data_ptr(), dw.key_cache.data_ptr(),
                    dw.value_cache.data_ptr(), dw.block_tables.data_ptr(), dw.seq_lens.data_ptr(),
                    wl.num_seqs, wl.num_heads, wl.head_size, wl.num_kv_heads,
                    ctypes.c_float(wl.scale), wl.max_num_blocks_per_seq, wl.block_size,
                    dw.key_cache.element_size(), dw.key_cache.stride(0), dw.key_cache.stride(1),
                    s.cuda_stream, wl.kv_dtype, 0)
        st, msg = PA.last_status()
        assert rc == PA.NXT_ATTN_E_UNSUPPORTED and "capturing" in msg, (rc, msg)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(dw.out, sentinel)
        del g
        # outside the capture the same call works on that stream
        with torch.cuda.stream(s):
            call(dw.out, s)
        torch.cuda.synchronize()
        from oracle import oracle as O
        from tests.helpers import assert_close
        assert_close(dw.out.float().cpu().numpy(), O.run_workload(wl, precision="mt"), W.FP16,
                     "eager call after the refused capture")
    finally:
        torch.cuda.synchronize()
        assert hip.hipStreamDestroy(raw) == 0
