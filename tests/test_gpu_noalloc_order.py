"""Eager nxt_paged_attention_noalloc calls on several queues of one device.
The fixed scratch is shared by every such call on a device, so the library
orders them on the GPU (each call's stream waits for the device's previous
no-alloc call unless it went to the same queue): calls enqueued back to back
on two streams, or from two host threads on hipStreamPerThread, with no host
wait in between, each match the oracle.  Without the ordering the second
call's partition kernel would overwrite partials the first call's merge has
not read yet."""
from __future__ import annotations

import ctypes
import threading

import pytest

from oracle import oracle as O
from tests.helpers import assert_close
from xllms_amd import _lib
from xllms_amd import paged_attention as PA
from xllms_amd import workloads as W

pytestmark = pytest.mark.gpu

HIP_STREAM_PER_THREAD = 2  # hipStreamPerThread's handle value


def _cases():
    return [W.small_case(num_seqs=24, H=32, KVH=8, D=128, kv_dtype=W.FP16, seed=201,
                         max_len=3000),
            W.small_case(num_seqs=40, H=64, KVH=4, D=128, kv_dtype=W.BF16, seed=202,
                         max_len=2500),
            W.small_case(num_seqs=16, H=32, KVH=8, D=128, kv_dtype=W.FP16, seed=203,
                         max_len=4000)]


def _noalloc(wl, dw, stream_handle):
    lib = _lib.backend()
    return lib.nxt_paged_attention_noalloc(
        dw.out.data_ptr(), dw.query.data_ptr(), dw.key_cache.data_ptr(),
        dw.value_cache.data_ptr(), dw.block_tables.data_ptr(), dw.seq_lens.data_ptr(),
        wl.num_seqs, wl.num_heads, wl.head_size, wl.num_kv_heads, ctypes.c_float(wl.scale),
        wl.max_num_blocks_per_seq, wl.block_size, dw.key_cache.element_size(),
        dw.key_cache.stride(0), dw.key_cache.stride(1), stream_handle, wl.kv_dtype, 0)


def test_calls_on_two_streams_are_ordered(cuda):
    import torch
    cases = _cases()
    refs = [O.run_workload(wl, precision="mt") for wl in cases]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    # each call its own output; inputs shared per case (read only)
    uploads = [W.upload(wl) for wl in cases]
    torch.cuda.synchronize()
    outs = []
    for i in range(9):
        k = i % 3
        wl, dw = cases[k], uploads[k]
        out = torch.full_like(dw.out, float("nan"))
        call_dw = W.DeviceWorkload(dw.query, dw.key_cache, dw.value_cache, dw.block_tables,
                                   dw.seq_lens, out)
        print(f"case call {i}: shape {k} on stream {i % 2}", flush=True)
        assert _noalloc(wl, call_dw, streams[i % 2].cuda_stream) == PA.NXT_ATTN_OK, \
            PA.last_status()
        outs.append((k, out))
    torch.cuda.synchronize()
    for i, (k, out) in enumerate(outs):
        assert_close(out.float().cpu().numpy(), refs[k], cases[k].kv_dtype, f"call {i}")


def test_calls_from_two_threads_on_the_per_thread_stream(cuda):
    import torch
    cases = _cases()[:2]
    refs = [O.run_workload(wl, precision="mt") for wl in cases]
    uploads = [W.upload(wl) for wl in cases]
    # every output allocated and filled before the threads start
    all_outs = [[torch.full_like(uploads[t].out, float("nan")) for _ in range(4)]
                for t in range(2)]
    torch.cuda.synchronize()
    results = {}
    errors = []

    def worker(t):
        try:
            wl, dw = cases[t], uploads[t]
            outs = all_outs[t]
            for i, out in enumerate(outs):
                call_dw = W.DeviceWorkload(dw.query, dw.key_cache, dw.value_cache,
                                           dw.block_tables, dw.seq_lens, out)
                rc = _noalloc(wl, call_dw, HIP_STREAM_PER_THREAD)
                if rc != PA.NXT_ATTN_OK:
                    errors.append((t, i, PA.last_status()))
                    return
            hip = ctypes.CDLL("libamdhip64.so.7")
            hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
            assert hip.hipStreamSynchronize(ctypes.c_void_p(HIP_STREAM_PER_THREAD)) == 0
            results[t] = outs
        except Exception as e:  # reported on the main thread
            errors.append((t, repr(e)))

    print("case two threads x 4 calls on hipStreamPerThread", flush=True)
    threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for t in range(2):
        for i, out in enumerate(results[t]):
            assert_close(out.float().cpu().numpy(), refs[t], cases[t].kv_dtype,
                         f"thread {t} call {i}")
