"""The drop-in boundary, checked on the CPU (no GPU calls that compute).

- libxllm_hip_backend.so loads and exports exactly the functions that
  include/*.h declares (operator API of the reference's include/operator_api.h
  plus the plugin ABI of backends/cuda_backend.h, plus the additive ones);
- the plugin ABI structs have the reference's layouts (compile-time asserts
  in tests/c/layout_check.c, and the ctypes mirrors of xllms_amd.backend);
- the plugin conventions of the reference's tests/test_backend_load.c:83-163
  hold (tests/c/plugin_contract.c, driven like backend_manager.c loads it);
- argument validation rejects unsupported shapes without launching.
"""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from xllms_amd import _lib
from xllms_amd import backend as B
from xllms_amd import paged_attention as PA

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_functions() -> set[str]:
    names = set()
    for fn in os.listdir(INCLUDE):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w ]*?[\s\*]+(nxt_\w+)\s*\(", text, re.M):
            names.add(m.group(1))
    return names


def exported_functions(path: str) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True,
                         text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_headers_declare_the_reference_entry_points():
    names = declared_functions()
    for ref in ("nxt_paged_attention", "nxt_paged_attention_v2", "nxt_paged_attention_flash",
                "nxt_backend_init", "nxt_backend_run", "nxt_backend_fini"):
        assert ref in names


def test_library_exports_exactly_the_declared_symbols():
    exported = exported_functions(_lib.BACKEND_SO)
    declared = declared_functions()
    assert exported == declared, (sorted(exported - declared), sorted(declared - exported))
    assert (set(_lib.OPERATOR_SYMBOLS) | set(_lib.PLUGIN_SYMBOLS) |
            set(_lib.KV_INDEX_SYMBOLS)) == declared


def test_library_loads_and_resolves_every_symbol():
    lib = _lib.backend()
    for name in declared_functions():
        assert getattr(lib, name) is not None
    assert PA.version().startswith("xllm-hip-attn")


def test_discovery_name_links_to_the_plugin():
    """The reference manager discovers libxllm_cuda_backend.so by default
    (cmake/xllm_config.h.in:18); the build provides that name too."""
    alias = os.path.join(_lib.LIB_DIR, "libxllm_cuda_backend.so")
    assert os.path.realpath(alias) == os.path.realpath(_lib.BACKEND_SO)


def test_struct_layouts_compile_time():
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{INCLUDE}", "-fsyntax-only",
                    os.path.join(ROOT, "tests", "c", "layout_check.c")], check=True)


def test_struct_layouts_ctypes_mirror():
    assert ctypes.sizeof(B.NxtBackendAPI) == 64
    assert ctypes.sizeof(B.NxtBackend) == 120
    offs = {f[0]: getattr(B.NxtBackend, f[0]).offset for f in B.NxtBackend._fields_}
    assert offs == {"name": 0, "so_path": 8, "dl_handle": 16, "api": 24, "state": 88,
                    "priority": 92, "model_count": 96, "models": 104, "backend_state": 112}
    assert ctypes.sizeof(B.NxtPagedAttentionInput) == 88
    assert B.NxtPagedAttentionInput.scale.offset == 56
    assert B.NxtPagedAttentionInput.stream.offset == 80
    assert ctypes.sizeof(B.NxtPagedAttentionInputEx) == 104


@pytest.fixture(scope="module")
def contract_binary(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("c") / "plugin_contract")
    subprocess.run(["gcc", "-std=c11", "-O1", "-Wall", "-D__HIP_PLATFORM_AMD__",
                    "-I/opt/rocm/include", f"-I{INCLUDE}", "-o", exe,
                    os.path.join(ROOT, "tests", "c", "plugin_contract.c"), "-ldl", "-lm",
                    "-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib", "-lamdhip64"], check=True)
    return exe


def test_plugin_contract_c_harness(contract_binary):
    r = subprocess.run([contract_binary, _lib.BACKEND_SO], capture_output=True, text=True,
                       timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout


@pytest.mark.parametrize("sanitize", [[], ["-fsanitize=thread", "-g"]],
                         ids=["plain", "tsan"])
def test_workspace_cache_threads(tmp_path, sanitize):
    """The per-(device, stream) workspace cache under host threads, on a mock
    device that models queues of in-flight work (tests/c/workspace_cache_test.cpp):
    no device use-after-free on growth or release, no workspace shared across
    the per-thread stream's queues, no interleaved enqueues on one handle;
    then graph-capture pinning, a reused stream handle, the entry bound and
    the per-thread entries freed at thread exit."""
    exe = str(tmp_path / "workspace_cache_test")
    subprocess.run(["g++", "-std=c++17", "-O1", "-pthread", "-Wall", *sanitize,
                    f"-I{os.path.join(ROOT, 'xllms_amd', 'csrc')}", "-o", exe,
                    os.path.join(ROOT, "tests", "c", "workspace_cache_test.cpp")], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and "PASSED" in r.stdout
    assert "WARNING: ThreadSanitizer" not in r.stderr


@pytest.mark.parametrize("variant", [[], ["-fsanitize=address,undefined", "-g"],
                                     ["-DPLANT_DROP_UPDATES"], ["-DPLANT_NO_FORGET"]],
                         ids=["plain", "asan-ubsan", "planted-drop-updates", "planted-no-forget"])
def test_resident_batch_tables(tmp_path, variant):
    """The model instance's block tables kept on the device between execs
    (xllms_amd/csrc/batch_tables.h), on a host model of the KV index and of the
    device rows (tests/c/batch_tables_test.cpp): 400 random sessions of
    same-order batches growing by 1-40 tokens, requests growing outside the
    batch, reorders, subsets, failed execs, releases and admissions that reuse
    handles; after every exec each row holds its sequence's pages, then -1.
    With the in-place updates or the release / admission notices planted out
    of the model, the checker must report stale rows."""
    exe = str(tmp_path / "batch_tables_test")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", *variant,
                    f"-I{os.path.join(ROOT, 'xllms_amd', 'csrc')}", "-o", exe,
                    os.path.join(ROOT, "tests", "c", "batch_tables_test.cpp")], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr[-2000:])
    if any(v.startswith("-DPLANT") for v in variant):
        assert r.returncode != 0 and "stale rows" in r.stderr
        return
    assert r.returncode == 0 and "PASSED" in r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr


@pytest.mark.parametrize("variant", [[], ["-fsanitize=thread", "-g"], ["-DPLANT_NO_WAIT"]],
                         ids=["plain", "tsan", "planted-no-wait"])
def test_noalloc_gate_threads(tmp_path, variant):
    """The ordering of nxt_paged_attention_noalloc calls on one device
    (xllms_amd/csrc/noalloc_gate.h) under host threads, on a mock device whose
    queues and events carry vector clocks (tests/c/noalloc_gate_test.cpp):
    every call's use of the shared scratch runs after the last one on every
    other queue (shared, own, per-thread and null stream handles), captured
    calls neither wait nor record, one event per device.  With the waits
    planted out of the mock, the checker must report overlapping calls."""
    exe = str(tmp_path / "noalloc_gate_test")
    subprocess.run(["g++", "-std=c++17", "-O1", "-pthread", "-Wall", *variant,
                    f"-I{os.path.join(ROOT, 'xllms_amd', 'csrc')}", "-o", exe,
                    os.path.join(ROOT, "tests", "c", "noalloc_gate_test.cpp")], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr[-2000:])
    if "-DPLANT_NO_WAIT" in variant:
        assert r.returncode != 0 and "may overlap" in r.stderr
        return
    assert r.returncode == 0 and "PASSED" in r.stdout
    assert "WARNING: ThreadSanitizer" not in r.stderr


def test_plugin_null_conventions_python_loader():
    b = B.LoadedBackend()
    assert b.init_fn(None) == -1
    assert b.run_fn(None, None, None) == -1
    assert b.fini_fn(None) == -1
    fresh = B.NxtBackend()
    assert b.fini_fn(ctypes.byref(fresh)) == 0
    assert fresh.state == B.STATE_UNINITIALIZED
    assert b.fini_fn(ctypes.byref(fresh)) == 0


def _call_ex(**kw):
    lib = _lib.backend()
    a = dict(num_seqs=2, num_heads=8, head_size=128, num_kv_heads=2, scale=0.1, maxb=4, bs=16,
             dtype_size=2, kbs=2 * 16 * 128, khs=16 * 128, kv_dtype=PA.NXT_KV_FP16, part=0)
    a.update(kw)
    p = 256  # any 16-byte aligned non-null address: validation fails before any use
    return lib.nxt_paged_attention_ex(p, p, p, p, p, p, a["num_seqs"], a["num_heads"],
                                      a["head_size"], a["num_kv_heads"],
                                      ctypes.c_float(a["scale"]), a["maxb"], a["bs"],
                                      a["dtype_size"], a["kbs"], a["khs"], None, a["kv_dtype"],
                                      a["part"])


@pytest.mark.parametrize("kw,status", [
    (dict(head_size=100), PA.NXT_ATTN_E_UNSUPPORTED),
    (dict(head_size=0), PA.NXT_ATTN_E_UNSUPPORTED),
    (dict(num_heads=7), PA.NXT_ATTN_E_INVALID),
    (dict(num_kv_heads=0), PA.NXT_ATTN_E_INVALID),
    (dict(num_seqs=-1), PA.NXT_ATTN_E_INVALID),
    (dict(dtype_size=4), PA.NXT_ATTN_E_INVALID),
    (dict(kv_dtype=9), PA.NXT_ATTN_E_UNSUPPORTED),
    (dict(bs=12), PA.NXT_ATTN_E_UNSUPPORTED),
    (dict(bs=0), PA.NXT_ATTN_E_INVALID),
    (dict(maxb=0), PA.NXT_ATTN_E_INVALID),
    (dict(kbs=2 * 16 * 128 + 1), PA.NXT_ATTN_E_UNSUPPORTED),
    (dict(khs=-16), PA.NXT_ATTN_E_INVALID),
    (dict(scale=float("inf")), PA.NXT_ATTN_E_INVALID),
    (dict(num_heads=66, num_kv_heads=1), PA.NXT_ATTN_E_UNSUPPORTED),
    (dict(part=24), PA.NXT_ATTN_E_UNSUPPORTED),
    (dict(part=8), PA.NXT_ATTN_E_UNSUPPORTED),
    (dict(num_seqs=0), PA.NXT_ATTN_OK),
])
def test_validation_without_launch(kw, status):
    assert _call_ex(**kw) == status
    st, msg = PA.last_status()
    assert st == status and msg


def test_void_entry_points_record_status():
    lib = _lib.backend()
    p = 256
    lib.nxt_paged_attention(p, p, p, p, p, p, 1, 8, 100, 2, ctypes.c_float(0.1), 4, 16, 2, 4096,
                            2048, None)
    assert lib.nxt_attn_last_status() == PA.NXT_ATTN_E_UNSUPPORTED
    lib.nxt_paged_attention_v2(p, p, p, p, p, p, 1, 8, 128, 2, ctypes.c_float(0.1), 4, 16, 3,
                               4096, 2048, None)
    assert lib.nxt_attn_last_status() == PA.NXT_ATTN_E_UNSUPPORTED
    lib.nxt_paged_attention_flash(p, p, p, p, p, p, 0, 8, 128, 2, ctypes.c_float(0.1), 4, 16, 2,
                                  4096, 2048, None)
    assert lib.nxt_attn_last_status() == PA.NXT_ATTN_OK


def test_cascade_validation_without_launch():
    """nxt_paged_attention_cascade refuses NULL or misaligned tensors before
    its plan kernels (which read the tables) are launched: these calls
    return without touching a GPU."""
    lib = _lib.backend()
    p = 256

    def call(out=p, q=p, k=p, v=p, bt=p, sl=p, pg=p, pb=p, max_groups=2, num_seqs=4):
        return lib.nxt_paged_attention_cascade(out, q, k, v, bt, sl, pg, pb, max_groups,
                                               num_seqs, 32, 128, 8, ctypes.c_float(0.1), 8, 16,
                                               8 * 16 * 128, 16 * 128, PA.NXT_KV_FP16, None)

    for name in ("out", "q", "k", "v", "bt", "sl", "pg", "pb"):
        assert call(**{name: None}) == PA.NXT_ATTN_E_INVALID, name
        assert PA.last_status()[0] == PA.NXT_ATTN_E_INVALID
    assert call(q=p + 8) == PA.NXT_ATTN_E_UNSUPPORTED
    assert call(k=p + 2) == PA.NXT_ATTN_E_UNSUPPORTED
    assert call(bt=p + 2) == PA.NXT_ATTN_E_INVALID
    assert call(pg=p + 1) == PA.NXT_ATTN_E_INVALID
    assert call(max_groups=-1) == PA.NXT_ATTN_E_INVALID
    # an empty batch needs no tensors, as for the ordinary entry points
    assert call(out=None, q=None, k=None, v=None, bt=None, sl=None, pg=None, pb=None,
                num_seqs=0) == PA.NXT_ATTN_OK


def test_kv_append_validation_without_launch():
    """The KV-append entry points check their arguments before any device
    call (these return without touching a GPU)."""
    lib = _lib.backend()
    p = 256
    # decode form: kv_dtype, block_size, head_size, sizes
    assert lib.nxt_paged_kv_append(p, p, p, p, p, p, 4, 2, 128, 8, 16, 4096, 2048, 9, None) == \
        PA.NXT_ATTN_E_INVALID
    assert lib.nxt_paged_kv_append(p, p, p, p, p, p, 4, 2, 128, 8, 12, 4096, 2048, 1, None) == \
        PA.NXT_ATTN_E_UNSUPPORTED
    assert lib.nxt_paged_kv_append(p, p, p, p, p, p, 4, 2, 100, 8, 16, 4096, 2048, 1, None) == \
        PA.NXT_ATTN_E_UNSUPPORTED
    assert lib.nxt_paged_kv_append(p, p, p, p, p, p, -1, 2, 128, 8, 16, 4096, 2048, 1, None) == \
        PA.NXT_ATTN_E_INVALID
    assert lib.nxt_paged_kv_append(p, p, p, p, None, p, 4, 2, 128, 8, 16, 4096, 2048, 1,
                                   None) == PA.NXT_ATTN_E_INVALID
    # misaligned cache pointer
    assert lib.nxt_paged_kv_append(p + 2, p, p, p, p, p, 4, 2, 128, 8, 16, 4096, 2048, 1,
                                   None) == PA.NXT_ATTN_E_UNSUPPORTED
    # nothing to do: OK without a device
    assert lib.nxt_paged_kv_append(None, None, None, None, None, None, 0, 2, 128, 8, 16, 4096,
                                   2048, 1, None) == PA.NXT_ATTN_OK
    # slot form
    assert lib.nxt_paged_kv_write_slots(p, p, p, p, None, 4, 2, 128, 16, 4096, 2048, 1,
                                        None) == PA.NXT_ATTN_E_INVALID
    assert lib.nxt_paged_kv_write_slots(p, p, p, p, p, 4, 2, 128, 24, 4096, 2048, 1,
                                        None) == PA.NXT_ATTN_E_UNSUPPORTED
    assert PA.last_status()[0] == PA.NXT_ATTN_E_UNSUPPORTED


def test_activation_validation_without_launch():
    """The activation entry points check their arguments before any device
    call (these return without touching a GPU)."""
    lib = _lib.backend()
    p = 256
    assert lib.nxt_activation_ex(0, p, p, 4, 16, PA.NXT_KV_FP16, None) == PA.NXT_ATTN_E_INVALID
    assert lib.nxt_activation_ex(7, p, p, 4, 16, PA.NXT_KV_FP16, None) == PA.NXT_ATTN_E_INVALID
    assert lib.nxt_activation_ex(1, p, p, 4, 16, 9, None) == PA.NXT_ATTN_E_UNSUPPORTED
    assert lib.nxt_activation_ex(1, p, p, -1, 16, PA.NXT_KV_FP16, None) == PA.NXT_ATTN_E_INVALID
    assert lib.nxt_activation_ex(1, p, p, 4, -16, PA.NXT_KV_FP16, None) == PA.NXT_ATTN_E_INVALID
    assert lib.nxt_activation_ex(1, None, p, 4, 16, PA.NXT_KV_FP16, None) == PA.NXT_ATTN_E_INVALID
    assert lib.nxt_activation_ex(1, p + 1, p, 4, 16, PA.NXT_KV_FP16, None) == PA.NXT_ATTN_E_INVALID
    # nothing to do: OK without a device
    assert lib.nxt_activation_ex(1, None, None, 0, 16, PA.NXT_KV_FP16, None) == PA.NXT_ATTN_OK
    assert lib.nxt_activation_ex(6, None, None, 4, 0, PA.NXT_KV_FP32, None) == PA.NXT_ATTN_OK
    # the reference's void entry points record their status; dtype_size other
    # than 2 / 4 is refused (the reference would run it as fp32)
    for name in _lib.ACTIVATION_ENTRY_POINTS:
        getattr(lib, name)(p, p, 4, 16, 8, None)
        assert lib.nxt_attn_last_status() == PA.NXT_ATTN_E_UNSUPPORTED, name
        getattr(lib, name)(p, p, 0, 16, 2, None)
        assert lib.nxt_attn_last_status() == PA.NXT_ATTN_OK, name


def test_product_never_imports_the_oracle():
    """The product path (package + native sources) has no route to oracle/."""
    pkg = os.path.join(ROOT, "xllms_amd")
    for dirpath, _, files in os.walk(pkg):
        for fn in files:
            if fn.endswith((".py", ".c", ".cpp", ".h", ".hip", "Makefile")):
                text = open(os.path.join(dirpath, fn)).read()
                assert not re.search(r"\boracle\b", text.replace("no route to oracle", "")), fn
