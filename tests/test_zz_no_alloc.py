"""nxt_paged_attention_noalloc: the allocation-free variant of
nxt_paged_attention_ex (split-K partials in a fixed per-device scratch array).

Through the C-ABI, two calls in a row (the second with a smaller input) must
give what nxt_paged_attention_ex gives on the same inputs, bit for bit (the
same plan runs on the scratch), and match the oracle at the task tolerance.
The big call must not lower the device's free memory (no hipMalloc), and an
explicit plan that needs more scratch is refused without touching the
output.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_close
from xllms_amd import _lib
from xllms_amd import paged_attention as PA
from xllms_amd import workloads as W

pytestmark = pytest.mark.gpu


def _call(entry, wl, dw, part=0):
    import torch
    lib = _lib.backend()
    fn = getattr(lib, entry)
    rc = fn(dw.out.data_ptr(), dw.query.data_ptr(), dw.key_cache.data_ptr(),
            dw.value_cache.data_ptr(), dw.block_tables.data_ptr(), dw.seq_lens.data_ptr(),
            wl.num_seqs, wl.num_heads, wl.head_size, wl.num_kv_heads, ctypes.c_float(wl.scale),
            wl.max_num_blocks_per_seq, wl.block_size, dw.key_cache.element_size(),
            dw.key_cache.stride(0), dw.key_cache.stride(1),
            torch.cuda.current_stream().cuda_stream, wl.kv_dtype, part)
    return rc


def _both(wl, part=0):
    """(noalloc output, _ex output) on the same uploaded inputs."""
    import torch
    dw = W.upload(wl)
    dw.out.zero_()
    assert _call("nxt_paged_attention_noalloc", wl, dw, part) == PA.NXT_ATTN_OK, PA.last_status()
    torch.cuda.synchronize()
    a = dw.out.float().cpu().numpy().copy()
    dw.out.zero_()
    assert _call("nxt_paged_attention_ex", wl, dw, part) == PA.NXT_ATTN_OK, PA.last_status()
    torch.cuda.synchronize()
    return a, dw.out.float().cpu().numpy()


def _free_bytes():
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch loaded
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_two_calls_match_the_allocating_entry_point(cuda):
    """Config 2 (64 sequences), then a smaller batch of another shape: the
    same plan as _ex on the scratch, so bit-identical outputs."""
    big = W.config2()
    print("case noalloc config2", flush=True)
    a, b = _both(big)
    assert np.array_equal(a, b)
    assert_close(a, O.run_workload(big, precision="mt"), big.kv_dtype, "noalloc config2")
    small = W.small_case(num_seqs=5, H=64, KVH=2, D=128, kv_dtype=W.BF16, seed=12,
                         lens=[0, 1, 40, 700, 1500])
    print("case noalloc small bf16 group 32", flush=True)
    a, b = _both(small)
    assert np.array_equal(a, b)
    assert_close(a, O.run_workload(small, precision="mt"), small.kv_dtype, "noalloc small")


@pytest.mark.parametrize("shape", [
    # (H, KVH, D, dtype): the largest automatic plans, 2048 wavefronts with
    # 32-head tiles at head_size 128 (65 MiB of scratch) and VALU tiles of
    # 8 heads at head_size 256
    (64, 2, 128, "fp16"),
    (64, 8, 256, "fp32"),
])
def test_largest_automatic_plans_fit(cuda, shape):
    """The largest automatic plans run on the scratch unchanged: identical to
    _ex bit for bit; then a smaller call of another shape."""
    H, KVH, D, dt = shape
    kv = {"fp16": W.FP16, "fp32": W.FP32}[dt]
    rng = np.random.default_rng(H + D)
    wl = W.small_case(num_seqs=64, H=H, KVH=KVH, D=D, kv_dtype=kv, seed=13,
                      lens=rng.integers(800, 3000, size=64).tolist())
    waves = PA.auto_waves(wl.num_seqs, H, D, KVH, wl.max_num_blocks_per_seq, 16, kv)
    print(f"case noalloc H={H} KVH={KVH} d={D} {dt} waves={waves}", flush=True)
    a, b = _both(wl)
    assert np.array_equal(a, b)
    assert_close(a, O.run_workload(wl, precision="mt"), kv, f"noalloc {shape}")
    small = W.small_case(num_seqs=3, H=12, KVH=12, D=64, kv_dtype=W.FP32, seed=14, max_len=300)
    print("case noalloc fp32 small", flush=True)
    a, b = _both(small)
    assert np.array_equal(a, b)
    assert_close(a, O.run_workload(small, precision="mt"), W.FP32, "noalloc fp32 small")


def test_no_device_allocation(cuda):
    """With the workspace cache emptied, a config-2 call through _ex would
    allocate ~33 MB; the no-alloc call leaves the free memory unchanged."""
    import torch
    wl = W.config2()
    dw = W.upload(wl)
    assert _call("nxt_paged_attention_noalloc", wl, dw) == PA.NXT_ATTN_OK  # scratch looked up
    torch.cuda.synchronize()
    assert PA.release_workspaces() == PA.NXT_ATTN_OK
    before = _free_bytes()
    for _ in range(3):
        assert _call("nxt_paged_attention_noalloc", wl, dw) == PA.NXT_ATTN_OK
    torch.cuda.synchronize()
    after = _free_bytes()
    print(f"free before {before} after {after}", flush=True)
    assert before - after < (4 << 20), (before, after)


def test_oversized_explicit_plan_is_refused(cuda):
    import torch
    wl = W.config2()
    dw = W.upload(wl)
    dw.out.fill_(3.0)
    sentinel = dw.out.clone()
    torch.cuda.synchronize()
    # 16-token ranges over config 2 need ~150 k wavefronts' partials
    assert _call("nxt_paged_attention_noalloc", wl, dw, part=16) == PA.NXT_ATTN_E_UNSUPPORTED
    st, msg = PA.last_status()
    assert st == PA.NXT_ATTN_E_UNSUPPORTED and "scratch" in msg
    torch.cuda.synchronize()
    assert torch.equal(dw.out, sentinel)
