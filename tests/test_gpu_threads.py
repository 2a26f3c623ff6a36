"""Re-entrancy of the operator across host threads and streams.

The reference's backend manager takes no locks (src/core/backend_manager.c:
32-46) and its operators hold no state, so callers may enqueue from several
threads at once.  Here the split-K workspace is library state, kept per
(device, stream queue): these tests enqueue from two host threads at once,
interleaving a shape that fits the current workspace with one that forces it
to grow, on
  - two streams (one workspace each),
  - one shared stream handle (one workspace, taken in turn),
  - hipStreamPerThread (one handle, a different queue per thread: one
    workspace per thread),
and check every output against the oracle.
"""
from __future__ import annotations

import ctypes
import threading

import pytest

from oracle import oracle as O
from tests.helpers import assert_close
from xllms_amd import paged_attention as PA
from xllms_amd import workloads as W

pytestmark = pytest.mark.gpu

HIP_STREAM_PER_THREAD = 2  # hipStreamPerThread, include/hip/hip_runtime_api.h
ITERS = 6


@pytest.fixture(scope="module")
def cases(cuda):
    import numpy as np
    rng = np.random.default_rng(31)
    small = W.small_case(num_seqs=8, H=32, KVH=8, D=128, kv_dtype=W.FP16, seed=41,
                         max_len=2000)
    big = W.small_case(num_seqs=64, H=32, KVH=8, D=128, kv_dtype=W.FP16, seed=42,
                       lens=rng.integers(512, 4096, size=64, endpoint=True).tolist())
    # (workload, partition_tokens): the explicit plan over the big batch
    # needs a workspace several times the automatic plan's
    return [(small, 0, O.run_workload(small, precision="mt")),
            (big, 256, O.run_workload(big, precision="mt")),
            (small, 64, None),
            (big, 0, None)]


def _hip():
    # the runtime torch already loaded (same soname), not a second copy
    lib = ctypes.CDLL("libamdhip64.so.7")
    lib.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    return lib


def _run_threads(cases, streams):
    """Thread t enqueues ITERS calls on streams[t] (a torch stream or a raw
    handle), cycling through the cases, each into its own output buffer."""
    import torch
    refs = {id(wl): ref for wl, _, ref in cases if ref is not None}
    inputs = {id(wl): W.upload(wl) for wl, _, _ in cases}
    outs = [[torch.empty_like(inputs[id(cases[(t + i) % len(cases)][0])].out)
             for i in range(ITERS)] for t in range(len(streams))]
    torch.cuda.synchronize()
    errors = []
    barrier = threading.Barrier(len(streams))

    def work(t):
        try:
            barrier.wait()
            for i in range(ITERS):
                wl, part, _ = cases[(t + i) % len(cases)]
                dw = inputs[id(wl)]
                PA.paged_attention(outs[t][i], dw.query, dw.key_cache, dw.value_cache,
                                   dw.block_tables, dw.seq_lens, num_kv_heads=wl.num_kv_heads,
                                   scale=wl.scale, partition_tokens=part, stream=streams[t])
            if isinstance(streams[t], int):  # hipStreamPerThread
                assert _hip().hipStreamSynchronize(HIP_STREAM_PER_THREAD) == 0
        except Exception as e:  # noqa: BLE001 - re-raised in the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(t,)) for t in range(len(streams))]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
        assert not th.is_alive(), "a host thread did not finish"
    torch.cuda.synchronize()
    assert not errors, errors
    for t in range(len(streams)):
        for i in range(ITERS):
            wl, part, _ = cases[(t + i) % len(cases)]
            assert_close(outs[t][i].float().cpu().numpy(), refs[id(wl)], wl.kv_dtype,
                         f"thread {t} call {i} partition {part}")


def test_two_threads_two_streams(cases):
    import torch
    PA.release_workspaces()  # the first calls allocate, the big ones grow
    print("case two threads, two streams", flush=True)
    _run_threads(cases, [torch.cuda.Stream(), torch.cuda.Stream()])


def test_two_threads_one_stream(cases):
    import torch
    PA.release_workspaces()
    print("case two threads, one stream handle", flush=True)
    s = torch.cuda.Stream()
    _run_threads(cases, [s, s])


def test_two_threads_per_thread_stream(cases):
    PA.release_workspaces()
    print("case two threads, hipStreamPerThread", flush=True)
    _run_threads(cases, [HIP_STREAM_PER_THREAD, HIP_STREAM_PER_THREAD])
