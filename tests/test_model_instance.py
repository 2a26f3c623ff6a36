"""The model / model-instance entry points of the plugin (include/xllm_hip_backend.h),
checked on the CPU: ctypes mirrors of the reference structures have the
reference header's layouts, and nxt_model_init refuses a configuration
without the decode geometry before touching a device."""
from __future__ import annotations

import ctypes

from xllms_amd import backend as B


def test_mirrors_have_the_reference_layouts():
    """Sizes and offsets as include/backend.h compiles (NxtModel.instances at
    144 is what the scheduler's poll dereferences, scheduler.c:483-486)."""
    assert ctypes.sizeof(B.NxtTensor) == 48
    assert ctypes.sizeof(B.NxtModelConfig) == 120
    assert B.NxtModelConfig.inputs.offset == 32
    assert B.NxtModelConfig.dynamic_batching.offset == 96
    assert ctypes.sizeof(B.NxtModel) == 168
    assert B.NxtModel.config.offset == 16
    assert B.NxtModel.instances.offset == 144
    assert B.NxtModel.instance_count.offset == 152
    assert B.NxtModel.backend_state.offset == 160
    assert ctypes.sizeof(B.NxtModelInstance) == 48
    assert B.NxtModelInstance.instance_state.offset == 24
    assert ctypes.sizeof(B.NxtInferRequest) == 56
    assert ctypes.sizeof(B.NxtDecodeIo) == 56


def test_model_init_refuses_a_config_without_geometry():
    m = B.DecodeModel.__new__(B.DecodeModel)
    dl = ctypes.CDLL(B._lib.BACKEND_SO)
    dl.nxt_model_init.argtypes = [ctypes.POINTER(B.NxtModel)]
    dl.nxt_model_init.restype = ctypes.c_int
    model = B.NxtModel()
    model.name = b"default"
    assert dl.nxt_model_init(ctypes.byref(model)) == -1      # no inputs at all
    assert not model.instances and model.instance_count == 0
    assert dl.nxt_model_init(None) == -1
    del m


def test_model_init_refuses_unsupported_geometry():
    # head_size 100 fp16 rows are not a multiple of 16 bytes; checked before any device call
    m = B.DecodeModel(num_blocks=16, num_kv_heads=2, block_size=16, head_size=100, num_heads=4)
    assert m.status == -1 and not m.model.instances
    m = B.DecodeModel(num_blocks=16, num_kv_heads=3, block_size=16, head_size=64, num_heads=4)
    assert m.status == -1
    m = B.DecodeModel(num_blocks=16, num_kv_heads=2, block_size=12, head_size=64, num_heads=4)
    assert m.status == -1
    m = B.DecodeModel(num_blocks=16, num_kv_heads=2, block_size=16, head_size=64, num_heads=4,
                      dtype=B.NXT_TYPE_INT32)
    assert m.status == -1


def test_instance_calls_refuse_missing_state():
    dl = ctypes.CDLL(B._lib.BACKEND_SO)
    inst = B.NxtModelInstance()
    dl.nxt_model_instance_exec.argtypes = [ctypes.POINTER(B.NxtModelInstance), ctypes.c_void_p,
                                           ctypes.c_uint32]
    dl.nxt_model_instance_exec.restype = ctypes.c_int
    assert dl.nxt_model_instance_exec(ctypes.byref(inst), None, 0) == -1
    assert dl.nxt_model_instance_exec(None, None, 0) == -1
    dl.nxt_model_instance_fini.argtypes = [ctypes.POINTER(B.NxtModelInstance)]
    assert dl.nxt_model_instance_fini(ctypes.byref(inst)) == 0
    dl.nxt_model_instance_bind.argtypes = [ctypes.POINTER(B.NxtModelInstance), ctypes.c_char_p,
                                           ctypes.c_void_p]
    assert dl.nxt_model_instance_bind(ctypes.byref(inst), b"r", None) == -1
