"""The activation oracle (oracle/activation_oracle.c), pinned on the CPU.

The reference has no CPU activation and no test of its activation kernels
(operators/activation_kernels.cu is exercised by nothing in its tests/), so
the restatement is pinned by what the mathematics fixes:
- the fp32 -> fp16 / bf16 roundings against numpy and torch;
- every op against its closed form evaluated in double precision (numpy,
  scipy.special.erf), with the same roundings to the element type;
- special values, and the identity act(x) - act(-x) = x that silu, gelu and
  gelu_tanh share (x*s(x) with s(x) + s(-x) = 1), which catches a wrong sign
  or a dropped factor without any library;
- which half of a gated row is the gate (operator_api.h:122-130).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from activation_cases import (DTYPES, OPS, closed_form, excess, from_bits, inputs, operands,
                              to_bits, ulp_distance)
from oracle import oracle as O


# ------------------------------------------------------------ conversions
def test_float_to_half_matches_numpy():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, size=20000, dtype=np.uint64).astype(np.uint32)
    vals = list(bits.view(np.float32))
    # ties between neighbouring halves, subnormals, the overflow edge
    h = np.arange(0, 0x7C00, 37, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (h[:-1] + (np.nextafter(h[:-1].astype(np.float16), np.float16(np.inf)).astype(np.float64)
                      - h[:-1]) / 2)
    vals += list(mids.astype(np.float32)) + [65504.0, 65519.99, 65520.0, 1e-8, 2.0 ** -25,
                                              3 * 2.0 ** -26, -0.0, np.inf, -np.inf]
    for v in vals:
        v = np.float32(v)
        got = O.float_to_half_bits(float(v))
        ref = int(np.array([v], dtype=np.float32).astype(np.float16).view(np.uint16)[0])
        if np.isnan(v):
            assert (got & 0x7C00) == 0x7C00 and (got & 0x3FF), hex(got)
        else:
            assert got == ref, (float(v), hex(got), hex(ref))


def test_float_to_bf16_matches_torch():
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2 ** 32, size=20000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = vals[~np.isnan(vals)]
    ref = torch.from_numpy(vals.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([O.float_to_bf16_bits(float(v)) for v in vals], dtype=np.uint16)
    assert (got == ref).all()


# ------------------------------------------------------------ closed forms
@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("op", OPS)
def test_oracle_matches_closed_form(op, dt):
    """Every element within the error the reference's fp32 formula can make,
    propagated through its roundings; and, where the formula has no
    cancellation (|x| <= 1.5), the same element-type value as the exact
    closed form but for the rare fp32 value next to a rounding boundary."""
    d = 777
    gated = op <= O.ACT_GELU_TANH_AND_MUL
    x = inputs(40, 2 * d if gated else d, dt, seed=op * 10 + dt)
    got = O.activation(op, x, dt)
    ref = closed_form(op, x, dt)
    assert got.shape == ref.shape == (40, d)
    ex = excess(op, x, got, ref, dt)
    assert (ex <= 1.0).all(), float(ex.max())
    arg, _ = operands(op, x, dt)
    calm = np.abs(arg) <= 1.5
    dist = ulp_distance(got, ref, dt)[calm]
    if dt == O.FP32:
        assert dist.max() <= 8, int(dist.max())
    else:
        # one ulp of the rounded activation is up to two ulps of its product
        assert dist.max() <= (2 if gated else 1), int(dist.max())
        assert (dist == 0).mean() >= 0.995, float((dist == 0).mean())


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("op", (O.ACT_SILU, O.ACT_GELU))
def test_odd_part_identity(op, dt):
    """act(x) - act(-x) = x for silu and gelu (and gelu_tanh below)."""
    x = np.linspace(-8, 8, 4001)
    xb = to_bits(x, O.FP32)[None, :]
    a = O.activation(op, xb, O.FP32)[0].astype(np.float64)
    b = O.activation(op, -xb, O.FP32)[0].astype(np.float64)
    xv = xb[0].astype(np.float64)
    assert np.abs(a - b - xv).max() <= 4e-7 * max(1.0, np.abs(xv).max())


def test_gelu_tanh_odd_part_and_approximation():
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    g = np.concatenate([x[None, :], np.ones((1, x.size), np.float32)], axis=1)
    gn = np.concatenate([-x[None, :], np.ones((1, x.size), np.float32)], axis=1)
    a = O.activation(O.ACT_GELU_TANH_AND_MUL, g, O.FP32)[0].astype(np.float64)
    b = O.activation(O.ACT_GELU_TANH_AND_MUL, gn, O.FP32)[0].astype(np.float64)
    assert np.abs(a - b - x).max() <= 4e-6
    # the tanh form approximates the erf form to about 5e-4 (Hendrycks &
    # Gimpel's published approximation)
    e = O.activation(O.ACT_GELU, x[None, :], O.FP32)[0].astype(np.float64)
    assert np.abs(a - e).max() < 1e-3
    assert np.abs(a - e).max() > 1e-5  # and is a different function


@pytest.mark.parametrize("dt", DTYPES)
def test_gate_is_the_first_half(dt):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 64)) * 2
    ones = np.ones_like(x)
    twos = 2 * ones
    silu = O.activation(O.ACT_SILU, to_bits(x, dt), dt)
    gelu = O.activation(O.ACT_GELU, to_bits(x, dt), dt)
    # silu(gate) * 1 == silu(gate); 1 * silu(up) == silu(up)
    assert (O.activation(O.ACT_SILU_AND_MUL, to_bits(np.hstack([x, ones]), dt), dt) == silu).all()
    assert (O.activation(O.ACT_MUL_AND_SILU, to_bits(np.hstack([ones, x]), dt), dt) == silu).all()
    assert (O.activation(O.ACT_GELU_AND_MUL, to_bits(np.hstack([x, ones]), dt), dt) == gelu).all()
    # a power-of-two up half scales exactly
    two = O.activation(O.ACT_SILU_AND_MUL, to_bits(np.hstack([x, twos]), dt), dt)
    assert (from_bits(two, dt) == 2 * from_bits(silu, dt)).all()
    # the other half is ignored by the activation
    swapped = O.activation(O.ACT_SILU_AND_MUL, to_bits(np.hstack([ones, x]), dt), dt)
    assert not (swapped == silu).all()


def test_special_values():
    x = np.array([[0.0, -0.0, np.inf, -np.inf, np.nan, -100.0, 100.0, 1e-30]], np.float32)
    silu = O.activation(O.ACT_SILU, x, O.FP32)[0]
    gelu = O.activation(O.ACT_GELU, x, O.FP32)[0]
    # 0 / 2 = 0; inf / 1 = inf; -inf / inf = NaN; -100 / (1 + e^100) = -0
    assert silu[0] == 0 and silu[2] == np.inf and np.isnan(silu[3]) and np.isnan(silu[4])
    assert silu[5] == 0 and np.signbit(silu[5]) and silu[6] == 100.0
    assert silu[7] == np.float32(5e-31)
    # (inf * 0.5) * 2 = inf; (-inf * 0.5) * (1 + -1) = NaN
    assert gelu[0] == 0 and gelu[2] == np.inf and np.isnan(gelu[3]) and np.isnan(gelu[4])
    assert gelu[5] == 0 and gelu[6] == 100.0


def test_multithreaded_is_bit_identical():
    x = inputs(64, 2 * 300, O.FP16, seed=9)
    a = O.activation(O.ACT_GELU_TANH_AND_MUL, x, O.FP16)
    b = O.activation(O.ACT_GELU_TANH_AND_MUL, x, O.FP16, threads=4)
    assert (a == b).all()


def test_rejects_bad_arguments():
    with pytest.raises(ValueError):
        O.activation(7, np.zeros((1, 4), np.float32), O.FP32)
    with pytest.raises(ValueError):
        O.activation(O.ACT_SILU, np.zeros((1, 4), np.float32), 4)
