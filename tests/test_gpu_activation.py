"""GPU parity of the activation operators (libxllm_hip_backend.so, C-ABI).

HIP output against the oracle (oracle/activation_oracle.c, the restatement of
operators/activation_kernels.cu:24-134) on the same seeded inputs.  Both sides
evaluate the reference's fp32 formula with different exp / erf / tanh
implementations (the GPU's device library, the host's libm), so the bar is:
- every element within the error two such evaluations can make, carried
  through the roundings to the element type (tests/activation_cases.py);
- where the formula has no cancellation (|x| <= 1.5): fp32 within rel 1e-5,
  fp16 / bf16 within 1 ulp (2 for a gated product: one ulp of the rounded
  activation is up to two of the product) and at least 99.5% bit-identical;
- fp16 / bf16 everywhere within the path's atol 2e-3 + rtol 1e-2 as well;
- NaN exactly where the oracle has NaN.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from activation_cases import (DTYPES, OPS, excess, from_bits, inputs, is_gated, operands,
                              to_bits, ulp_distance)
from oracle import oracle as O
from xllms_amd import activation as A
from xllms_amd import paged_attention as PA

pytestmark = pytest.mark.gpu

TORCH = {O.FP16: torch.float16, O.BF16: torch.bfloat16, O.FP32: torch.float32}
NP = {O.FP16: np.uint16, O.BF16: np.uint16, O.FP32: np.float32}
VIEW = {O.FP16: torch.int16, O.BF16: torch.int16, O.FP32: torch.float32}


def upload(bits: np.ndarray, dt: int, dev) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16 if dt != O.FP32 else np.float32))
    return t.to(dev).view(TORCH[dt])


def download(t: torch.Tensor, dt: int) -> np.ndarray:
    return t.view(VIEW[dt]).cpu().numpy().view(NP[dt])


def check(op: int, xb: np.ndarray, got: np.ndarray, dt: int, what: str) -> None:
    ref = O.activation(op, xb, dt)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    g, r = from_bits(got, dt), from_bits(ref, dt)
    nan_g, nan_r = np.isnan(g), np.isnan(r)
    assert (nan_g == nan_r).all(), f"{what}: NaN pattern differs"
    ok = ~nan_r
    ex = excess(op, xb, got, ref, dt, evaluations=2)
    assert (ex[ok] <= 1.0).all(), f"{what}: excess {float(ex[ok].max())}"
    if dt != O.FP32:
        bound = 2e-3 + 1e-2 * np.abs(r[ok])
        assert (np.abs(g[ok] - r[ok]) <= bound).all(), f"{what}: outside atol/rtol"
    arg, _ = operands(op, xb, dt)
    calm = ok & (np.abs(arg) <= 1.5)
    if dt == O.FP32:
        rel = np.abs(g[calm] - r[calm]) / np.maximum(np.abs(r[calm]), 1e-30)
        assert (rel <= 1e-5).all(), f"{what}: fp32 rel {float(rel.max())}"
    else:
        dist = ulp_distance(got[calm], ref[calm], dt)
        assert dist.max(initial=0) <= (2 if is_gated(op) else 1), f"{what}: {int(dist.max())} ulp"
        assert (dist == 0).mean() >= 0.995, f"{what}: {(dist == 0).mean():.4f} identical"


def run(op: int, xb: np.ndarray, dt: int, dev, entry=None, offset: int = 0) -> np.ndarray:
    n = xb.shape[0]
    d = xb.shape[1] // 2 if is_gated(op) else xb.shape[1]
    flat = upload(xb.reshape(-1), dt, dev)
    if offset:
        # an input that starts `offset` elements into its allocation
        buf = torch.empty(flat.numel() + offset, dtype=TORCH[dt], device=dev)
        buf[offset:] = flat
        flat = buf[offset:]
    out = torch.full((n, d), float("nan"), dtype=TORCH[dt], device=dev)
    A.activation(op, out, flat, num_tokens=n, d=d, dtype=dt, entry=entry)
    torch.cuda.synchronize()
    return download(out, dt)


SHAPES = [(1, 8), (5, 1000), (64, 14336), (3, 11008), (17, 4096), (7, 1001), (2, 5), (9, 12)]


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{n}x{d}" for n, d in SHAPES])
@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("op", OPS)
def test_parity(cuda, op, dt, shape):
    n, d = shape
    xb = inputs(n, 2 * d if is_gated(op) else d, dt, seed=1000 * op + 10 * dt + n)
    got = run(op, xb, dt, cuda)
    check(op, xb, got, dt, f"op {op} dt {dt} {shape}")


@pytest.mark.parametrize("dt", (O.FP16, O.FP32))
@pytest.mark.parametrize("entry", sorted(A.ENTRY_POINTS))
def test_reference_entry_points(cuda, entry, dt):
    """The reference's void entry points, dtype_size 2 (fp16) / 4 (fp32)."""
    op = A.ENTRY_POINTS[entry]
    d = 4096
    xb = inputs(6, 2 * d if is_gated(op) else d, dt, seed=op + 7 * dt)
    got = run(op, xb, dt, cuda, entry=entry)
    check(op, xb, got, dt, entry)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("op", (O.ACT_SILU_AND_MUL, O.ACT_GELU))
def test_unaligned_input(cuda, op, dt):
    """An input not 16-byte aligned takes the element kernel."""
    d = 1024
    xb = inputs(5, 2 * d if is_gated(op) else d, dt, seed=3 * op + dt)
    got = run(op, xb, dt, cuda, offset=1)
    check(op, xb, got, dt, "unaligned")


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("op", OPS)
def test_vector_and_element_kernels_agree(cuda, op, dt):
    """The same rows through the 16-byte chunk kernel (aligned input) and the
    element kernel (input one element off alignment) give identical bits."""
    d = 2048
    xb = inputs(6, 2 * d if is_gated(op) else d, dt, seed=11 * op + dt, scale=30.0)
    a = run(op, xb, dt, cuda)
    b = run(op, xb, dt, cuda, offset=1)
    assert (a.view(np.uint32 if dt == O.FP32 else np.uint16) ==
            b.view(np.uint32 if dt == O.FP32 else np.uint16)).all()


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("op", OPS)
def test_special_values(cuda, op, dt):
    # -87.5 / -88: silu's fast form underflows there, bf16 takes the reference formula
    vals = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -100.0, 100.0, 1e-6, -1e-6, 6e4, -6e4,
                     -5.0, -9.0, 3.0, 2.0 ** -20, -(2.0 ** -20), -87.5, -88.0])
    x = np.stack([np.roll(vals, k) for k in range(vals.size)])  # every value meets every other
    xb = to_bits(x, dt)
    if is_gated(op):
        xb = np.concatenate([xb, xb[::-1]], axis=1)
    got = run(op, xb, dt, cuda)
    ref = O.activation(op, xb, dt)
    g, r = from_bits(got, dt), from_bits(ref, dt)
    assert (np.isnan(g) == np.isnan(r)).all()
    fin = np.isfinite(r)
    assert (np.isinf(g) == np.isinf(r)).all() and (g[~fin & ~np.isnan(r)] == r[~fin & ~np.isnan(r)]).all()
    ex = excess(op, xb, got, ref, dt, evaluations=2)
    assert (ex[fin] <= 1.0).all(), float(ex[fin].max())


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("op", (O.ACT_SILU, O.ACT_GELU))
def test_elementwise_in_place(cuda, op, dt):
    d = 2048
    xb = inputs(9, d, dt, seed=op + dt)
    t = upload(xb, dt, cuda)
    A.activation(op, t, t, dtype=dt)
    torch.cuda.synchronize()
    check(op, xb, download(t, dt), dt, "in place")


def test_empty_and_invalid_leave_output_untouched(cuda):
    out = torch.full((4, 16), 7.0, dtype=torch.float16, device=cuda)
    inp = torch.randn(4, 32, dtype=torch.float16, device=cuda)
    for n, d in ((0, 16), (4, 0)):
        assert A.silu_and_mul(out, inp, num_tokens=n, d=d) == PA.NXT_ATTN_OK
    assert A.silu_and_mul(out, inp, num_tokens=-1, d=16, check=False) == PA.NXT_ATTN_E_INVALID
    assert A.activation(9, out, inp, check=False) == PA.NXT_ATTN_E_INVALID
    lib = A._lib.backend()
    lib.nxt_silu_and_mul(out.data_ptr(), inp.data_ptr(), 4, 16, 3, None)  # dtype_size 3
    assert lib.nxt_attn_last_status() == PA.NXT_ATTN_E_UNSUPPORTED
    torch.cuda.synchronize()
    assert (out == 7.0).all()


def test_launch_split_beyond_2g_chunks(cuda):
    """A gated op over more than 2^31 sixteen-byte output chunks runs as two
    launches (the vector kernel's indices are 32-bit): 1,048,640 rows of
    d = 16384 fp16, rows cycling through 64 seeded patterns so the second
    launch, which starts inside a cycle, must read and write the right rows.
    Every row must carry the bits of the same pattern row computed in a small
    call, itself checked against the oracle.  34 GB out, 69 GB in."""
    free, _ = torch.cuda.mem_get_info()
    rows, d, period = 1_048_640, 16384, 64
    need = rows * d * 2 * 3
    if free < need + (8 << 30):
        pytest.skip(f"needs {need >> 30} GiB of free device memory")
    xb = inputs(period, 2 * d, O.FP16, seed=77)
    small = run(O.ACT_SILU_AND_MUL, xb, O.FP16, cuda)
    check(O.ACT_SILU_AND_MUL, xb, small, O.FP16, "pattern rows")
    expect = torch.from_numpy(small.view(np.int16)).to(cuda)
    pattern = upload(xb, O.FP16, cuda)
    inp = torch.empty((rows, 2 * d), dtype=torch.float16, device=cuda)
    inp.view(rows // period, period, 2 * d).copy_(pattern.expand(rows // period, period, 2 * d))
    out = torch.empty((rows, d), dtype=torch.float16, device=cuda)
    A.silu_and_mul(out, inp)
    torch.cuda.synchronize()
    del inp
    ov = out.view(torch.int16).view(rows // period, period, d)
    step = 4096
    for i in range(0, rows // period, step):
        blk = ov[i:i + step]
        assert torch.equal(blk, expect.expand_as(blk)), f"rows {i * period}.."
