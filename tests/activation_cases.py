"""Closed forms and error bounds shared by the activation tests (CPU and GPU).

The activations are evaluated in double precision (numpy, scipy.special.erf)
and rounded to the element type the way the reference rounds them
(operators/activation_kernels.cu:24-69): activation rounded to T, gated
product rounded to T.  `excess` measures an fp32 evaluation of the
reference's formula against that exact value, in units of the error such an
evaluation can make: a few ulps of the activation, plus, for the erf / tanh
forms, a few ulps of the 1 + erf (1 + tanh) term scaled by |x| (its
cancellation for negative x), carried through the roundings to T.
"""
from __future__ import annotations

import numpy as np
import scipy.special
import torch

from oracle import oracle as O

OPS = (O.ACT_SILU_AND_MUL, O.ACT_MUL_AND_SILU, O.ACT_GELU_AND_MUL, O.ACT_GELU_TANH_AND_MUL,
       O.ACT_GELU, O.ACT_SILU)
DTYPES = (O.FP16, O.BF16, O.FP32)


def is_gated(op: int) -> bool:
    return op <= O.ACT_GELU_TANH_AND_MUL


def silu64(x):
    return x * scipy.special.expit(x)


def gelu64(x):
    return 0.5 * x * (1.0 + scipy.special.erf(x / np.sqrt(2.0)))


def gelu_tanh64(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


ACT64 = {O.ACT_SILU_AND_MUL: silu64, O.ACT_MUL_AND_SILU: silu64, O.ACT_GELU_AND_MUL: gelu64,
         O.ACT_GELU_TANH_AND_MUL: gelu_tanh64, O.ACT_GELU: gelu64, O.ACT_SILU: silu64}


def to_bits(x64: np.ndarray, dt: int) -> np.ndarray:
    """float64 -> element bits, round to nearest even."""
    if dt == O.FP16:
        return x64.astype(np.float16).view(np.uint16)
    if dt == O.BF16:
        return torch.from_numpy(np.ascontiguousarray(x64)).to(torch.bfloat16).view(
            torch.int16).numpy().view(np.uint16)
    return x64.astype(np.float32)


def from_bits(b: np.ndarray, dt: int) -> np.ndarray:
    return O.widen(b, dt).astype(np.float64)


def closed_form(op: int, xb: np.ndarray, dt: int) -> np.ndarray:
    """The op in double precision on the element values, with the reference's
    roundings: activation rounded to T, product rounded to T."""
    x = from_bits(xb, dt)
    act = ACT64[op]
    if op in (O.ACT_GELU, O.ACT_SILU):
        return to_bits(act(x), dt)
    d = x.shape[1] // 2
    g, u = x[:, :d], x[:, d:]
    if op == O.ACT_MUL_AND_SILU:
        return to_bits(g * from_bits(to_bits(act(u), dt), dt), dt)
    return to_bits(from_bits(to_bits(act(g), dt), dt) * u, dt)


def ulp_distance(a: np.ndarray, b: np.ndarray, dt: int) -> np.ndarray:
    """Distance in units of the last place between element bit patterns of
    the same sign convention (monotone integer map of the values)."""
    if dt == O.FP32:
        ia = a.view(np.int32).astype(np.int64)
        ib = b.view(np.int32).astype(np.int64)
        sign = np.int64(1 << 31)
    else:
        ia = a.astype(np.int64)
        ib = b.astype(np.int64)
        sign = np.int64(1 << 15)
        ia = np.where(ia & sign, -(ia & (sign - 1)), ia)
        ib = np.where(ib & sign, -(ib & (sign - 1)), ib)
        return np.abs(ia - ib)
    ia = np.where(ia < 0, -(ia & (sign - 1)), ia)
    ib = np.where(ib < 0, -(ib & (sign - 1)), ib)
    return np.abs(ia - ib)


def inputs(n: int, cols: int, dt: int, seed: int, scale: float = 3.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, cols)) * scale
    return to_bits(x, dt)


def ulp_of(v: np.ndarray, dt: int) -> np.ndarray:
    """Spacing of the element type at |v| (float64 result)."""
    a = np.abs(v)
    if dt == O.FP16:
        return np.spacing(a.astype(np.float16)).astype(np.float64)
    if dt == O.BF16:
        e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
        return 2.0 ** (e - 7)
    return np.spacing(a.astype(np.float32)).astype(np.float64)



def operands(op: int, xb: np.ndarray, dt: int):
    """(activation argument, other operand) values of every output element."""
    xv = from_bits(xb, dt)
    if not is_gated(op):
        return xv, np.ones_like(xv)
    d = xv.shape[1] // 2
    if op == O.ACT_MUL_AND_SILU:
        return xv[:, d:], xv[:, :d]
    return xv[:, :d], xv[:, d:]


def excess(op: int, xb: np.ndarray, got: np.ndarray, ref: np.ndarray, dt: int,
           evaluations: int = 1) -> np.ndarray:
    """|got - ref| over the error bound of `evaluations` independent fp32
    evaluations of the formula (1: got vs the exact closed form; 2: two fp32
    evaluations against each other).  <= 1 everywhere passes."""
    arg, other = operands(op, xb, dt)
    a64 = ACT64[op](arg)
    e32 = 8 * np.spacing(np.abs(a64).astype(np.float32)).astype(np.float64)
    if op not in (O.ACT_SILU, O.ACT_SILU_AND_MUL, O.ACT_MUL_AND_SILU):
        e32 += 4 * np.abs(arg) * 2.0 ** -24
    e32 *= evaluations
    g, r = from_bits(got, dt), from_bits(ref, dt)
    if is_gated(op):
        bound = (e32 + evaluations * ulp_of(a64, dt)) * np.abs(other) + ulp_of(r, dt)
    else:
        bound = e32 + ulp_of(r, dt)
    return np.abs(g - r) / bound
