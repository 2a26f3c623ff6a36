"""The plugin ABI on the GPU: nxt_backend_init -> run / run_ex -> fini.

libxllm_hip_backend.so is loaded the way the reference backend manager loads
a plugin (src/core/backend_manager.c:274-285: dlopen RTLD_NOW|RTLD_LOCAL,
dlsym of the three entry points) and driven with the reference's
NxtPagedAttentionInput descriptor (backends/cuda_backend.h:29-46) on device
buffers, as backends/cuda_backend.c:71-104 unpacks it.  Outputs are checked
against the oracle at the task tolerance; the conventions are those of the
reference's tests/test_backend_load.c:83-163 and tests/test_backend.c:271-307.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_close
from xllms_amd import _lib
from xllms_amd import backend as B
from xllms_amd import paged_attention as PA
from xllms_amd import workloads as W

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def oracle(wl):
    return O.run_workload(wl, precision="mt")


@pytest.fixture
def plugin(cuda):
    b = B.LoadedBackend()
    assert b.init() == 0
    assert b.state == B.STATE_READY and b.handle.backend_state
    yield b
    assert b.fini() == 0
    assert b.handle.backend_state is None
    assert b.handle.state == B.STATE_UNINITIALIZED


def _desc(dw, wl, stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    return B.make_input(dw.query, dw.key_cache, dw.value_cache, dw.block_tables, dw.seq_lens,
                        num_kv_heads=wl.num_kv_heads, scale=wl.scale, stream=s)


def _run(plugin, wl, dw=None):
    import torch
    dw = dw or W.upload(wl)
    dw.out.zero_()
    rc = plugin.run(_desc(dw, wl), dw.out.data_ptr())
    torch.cuda.synchronize()
    return rc, dw.out.float().cpu().numpy()


def test_c_harness_gpu(cuda, tmp_path):
    """tests/c/plugin_contract.c with --gpu: a C program that loads the
    plugin like backend_manager.c, checks every NULL convention, refuses a
    4-byte garbage descriptor, and runs a real fp16 decode."""
    exe = str(tmp_path / "plugin_contract")
    subprocess.run(["gcc", "-std=c11", "-O1", "-Wall", "-D__HIP_PLATFORM_AMD__",
                    "-I/opt/rocm/include", f"-I{os.path.join(ROOT, 'include')}", "-o", exe,
                    os.path.join(ROOT, "tests", "c", "plugin_contract.c"), "-ldl", "-lm",
                    "-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib", "-lamdhip64"], check=True)
    print("case plugin_contract --gpu", flush=True)
    r = subprocess.run([exe, _lib.BACKEND_SO, "--gpu"], capture_output=True, text=True,
                       timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout
    assert "PASSED" in r.stdout


def test_run_config1_fp32(plugin):
    """dtype_size 4 through the reference descriptor: config 1 (fp32 MHA)."""
    wl = W.config1()
    print("case plugin run config1", flush=True)
    rc, got = _run(plugin, wl)
    assert rc == 0
    assert_close(got, oracle(wl), W.FP32, "plugin run config1")


def test_run_config2_fp16(plugin):
    """dtype_size 2 through the reference descriptor: config 2, the headline."""
    wl = W.config2()
    print("case plugin run config2", flush=True)
    rc, got = _run(plugin, wl)
    assert rc == 0
    assert_close(got, oracle(wl), W.FP16, "plugin run config2")


@pytest.mark.parametrize("part", [0, 64])
def test_run_ex_bf16_config4a(plugin, part):
    """nxt_backend_run_ex with kv_dtype BF16 (which dtype_size cannot name)
    on config 4a's full batch, automatic and explicit split-K."""
    import torch
    wl = W.config4(num_kv_heads=8)
    dw = W.upload(wl)
    ex = B.NxtPagedAttentionInputEx()
    ex.struct_size = ctypes.sizeof(B.NxtPagedAttentionInputEx)
    ex.base = _desc(dw, wl)
    ex.kv_dtype = PA.NXT_KV_BF16
    ex.partition_tokens = part
    print(f"case plugin run_ex config4a partition={part}", flush=True)
    assert plugin.run_ex(ex, dw.out.data_ptr()) == 0
    torch.cuda.synchronize()
    assert_close(dw.out.float().cpu().numpy(), oracle(wl), W.BF16, f"run_ex part={part}")


def test_refusals_leave_output_untouched(plugin):
    """Descriptors the plugin must refuse with -1 before launching: a 4-byte
    garbage input (test_backend_load.c:116-118), NULL output, dtype_size 3,
    host pointers, unsupported head size, a short run_ex struct, bf16 via
    run_ex with a mismatched dtype_size."""
    import torch
    wl = W.small_case(num_seqs=3, H=8, KVH=2, D=128, kv_dtype=W.FP16, seed=5, max_len=100)
    dw = W.upload(wl)
    dw.out.fill_(7.0)
    sentinel = dw.out.clone()
    out = dw.out.data_ptr()
    garbage = ctypes.c_int(0xDEAD)
    assert plugin.run_fn(ctypes.byref(plugin.handle), ctypes.addressof(garbage), out) == -1
    good = _desc(dw, wl)
    assert plugin.run(good, 0) == -1
    bad = _desc(dw, wl)
    bad.dtype_size = 3
    assert plugin.run(bad, out) == -1
    host_q = np.zeros(wl.query.shape, dtype=np.float16)
    bad = _desc(dw, wl)
    bad.query = host_q.ctypes.data
    assert plugin.run(bad, out) == -1
    bad = _desc(dw, wl)
    bad.head_size = 100
    assert plugin.run(bad, out) == -1
    ex = B.NxtPagedAttentionInputEx()
    ex.struct_size = 8
    ex.base = good
    ex.kv_dtype = PA.NXT_KV_FP16
    assert plugin.run_ex(ex, out) == -1
    ex.struct_size = ctypes.sizeof(B.NxtPagedAttentionInputEx)
    ex.kv_dtype = PA.NXT_KV_FP32  # dtype_size 2 does not match fp32
    assert plugin.run_ex(ex, out) == -1
    torch.cuda.synchronize()
    assert torch.equal(dw.out, sentinel)
    # and the same descriptor, corrected, runs
    rc, got = _run(plugin, wl, dw)
    assert rc == 0
    assert_close(got, oracle(wl), W.FP16, "after refusals")


def test_fini_twice_and_run_after_fini(cuda):
    b = B.LoadedBackend()
    assert b.init() == 0
    assert b.fini() == 0
    assert b.fini() == 0  # double fini (test_backend_load.c:150-160)
    wl = W.small_case(num_seqs=2, H=8, KVH=2, D=128, kv_dtype=W.FP16, seed=6, max_len=64)
    dw = W.upload(wl)
    # the manager refuses a backend that is not READY; the plugin itself
    # refuses a handle whose state was released
    assert b.run(_desc(dw, wl), dw.out.data_ptr()) == -1
    assert b.run_fn(ctypes.byref(b.handle), ctypes.cast(ctypes.byref(_desc(dw, wl)),
                                                         ctypes.c_void_p),
                    dw.out.data_ptr()) == -1


def test_fini_releases_only_its_own_workspaces(cuda):
    """Two backends and a direct operator caller on three streams: one
    backend's fini frees the workspaces its runs allocated, and the other
    backend's and the direct caller's next launches (which reuse theirs)
    still compute the right thing."""
    import torch
    wl = W.small_case(num_seqs=24, H=32, KVH=8, D=128, kv_dtype=W.FP16, seed=8, max_len=3000)
    ref = oracle(wl)
    s1, s2, s3 = torch.cuda.Stream(), torch.cuda.Stream(), torch.cuda.Stream()
    b1, b2 = B.LoadedBackend(), B.LoadedBackend()
    assert b1.init() == 0 and b2.init() == 0
    dws = [W.upload(wl) for _ in range(3)]
    torch.cuda.synchronize()

    def check(i, what):
        torch.cuda.synchronize()
        assert_close(dws[i].out.float().cpu().numpy(), ref, W.FP16, what)
        dws[i].out.zero_()
        torch.cuda.synchronize()

    for rep in range(2):
        print(f"case fini scoping rep={rep}", flush=True)
        assert b1.run(_desc(dws[0], wl, s1.cuda_stream), dws[0].out.data_ptr()) == 0
        assert b2.run(_desc(dws[1], wl, s2.cuda_stream), dws[1].out.data_ptr()) == 0
        PA.paged_attention(dws[2].out, dws[2].query, dws[2].key_cache, dws[2].value_cache,
                           dws[2].block_tables, dws[2].seq_lens, num_kv_heads=wl.num_kv_heads,
                           scale=wl.scale, stream=s3)
        for i in range(3):
            check(i, f"rep {rep} caller {i}")
    assert b1.fini() == 0
    assert b2.run(_desc(dws[1], wl, s2.cuda_stream), dws[1].out.data_ptr()) == 0
    PA.paged_attention(dws[2].out, dws[2].query, dws[2].key_cache, dws[2].value_cache,
                       dws[2].block_tables, dws[2].seq_lens, num_kv_heads=wl.num_kv_heads,
                       scale=wl.scale, stream=s3)
    check(1, "second backend after the first one's fini")
    check(2, "direct caller after a backend's fini")
    assert b2.fini() == 0
