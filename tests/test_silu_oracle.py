"""The SiLU / SwiGLU oracles pinned against FP64 mathematics (CPU).

* ``oracle.swiglu`` restates the native runtime's SwiGLU
  (/root/reference/src/venturi/ops/csrc/blocks.cu:56-70): fp16((x * sigmoid(x)) * y)
  with fp32 intermediates and a two-branch logistic.
* ``oracle.moe.silu_fp16`` restates ``F.silu(gate)`` on an fp16 tensor
  (/root/reference/src/venturi/models/flash_next/flash_next_q4.py:222): one fp32
  evaluation of g / (1 + e^-g), rounded to fp16.

Mathematics fixes both: x * y / (1 + e^-x) evaluated in FP64 and rounded once to
fp16. The oracles take a handful of fp32 roundings (and numpy's fp32 exp) on
the way, each within 2^-24 relative (a few ulps for exp), so their fp16 result
must equal the FP64 value's fp16 rounding exactly wherever that value is more
than 2^-20 (relative) away from a rounding midpoint, and be within one fp16 ulp
everywhere. The grids cover every finite fp16 input (both logistic branches,
+-0, +-65504, -30..-12, subnormals), the overflow edge of the product and
seeded random pairs; known values (silu(1) = 0.7310585786...) are checked
directly. The last test plants plausible mistakes in copies of the formulas
and checks that the same comparison rejects each of them.
"""

import numpy as np
import pytest

import oracle
from oracle import moe as omoe

GUARD = 2.0**-20  # relative band around fp16 rounding midpoints where one ulp may flip


def all_finite_fp16():
    v = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    return v[np.isfinite(v)]


def silu_f64(x):
    """x / (1 + e^-x) in FP64, through the branch that does not overflow."""
    x = np.asarray(x, np.float64)
    out = np.empty_like(x)
    pos = x >= 0
    out[pos] = x[pos] / (1.0 + np.exp(-x[pos]))
    e = np.exp(x[~pos])
    out[~pos] = x[~pos] * e / (1.0 + e)
    return out


def fp16_neighbours(v):
    """(nearest fp16 by RNE, the other fp16 value bracketing v) for finite FP64 v."""
    h = v.astype(np.float16)
    toward = np.where(h.astype(np.float64) < v, np.float16(np.inf), np.float16(-np.inf)).astype(np.float16)
    with np.errstate(over="ignore"):  # past +-65504 the other neighbour is inf
        other = np.nextafter(h, toward)
    return h, other


def compare(got16, exact64):
    """Counts of (outputs off by more than one ulp, exact-equality failures outside the guard band)."""
    got = np.asarray(got16, np.float16).astype(np.float64)
    exact = np.asarray(exact64, np.float64)
    big = np.abs(exact) >= 65520.0 * (1 + GUARD)  # beyond the last midpoint: fp16 inf
    edge = (np.abs(exact) > 65520.0 * (1 - GUARD)) & ~big
    clipped = np.clip(exact, -65504.0, 65504.0)
    h, other = fp16_neighbours(clipped)
    h64, o64 = h.astype(np.float64), other.astype(np.float64)
    midpoint = np.where(np.isfinite(o64), 0.5 * (h64 + o64), np.inf)
    near_tie = np.abs(exact - midpoint) <= GUARD * np.abs(exact)
    want = np.where(big, np.copysign(np.inf, exact), h64)
    exact_ok = (got == want) | (np.isnan(got) & np.isnan(want))
    one_ulp_ok = exact_ok | (got == o64) | (edge & (np.abs(got) >= 65504.0))
    loose = int((~one_ulp_ok).sum())
    strict = int((~exact_ok & ~near_tie & ~edge).sum())
    return loose, strict


def swiglu_inputs():
    xs = all_finite_fp16()
    ys = np.array([1.0, -1.0, 0.5, 0.99951171875, 3.140625, -7.5, 1.5e-5, 2.0**-24, 65504.0, -2.0], np.float16)
    grid_x = np.tile(xs, ys.size)
    grid_y = np.repeat(ys, xs.size)
    rng = np.random.default_rng(0)
    rx = (rng.standard_normal(200_000) * 6).astype(np.float16)
    ry = (rng.standard_normal(200_000) * 3).astype(np.float16)
    tails = np.concatenate([np.linspace(-30, -12, 4001), [0.0, -0.0, 65504.0, -65504.0, 88.5, 89.0, -88.5, -89.0,
                                                          2.0**-24, -(2.0**-24), 2.0**-14, 6.0e-5]]).astype(np.float16)
    x = np.concatenate([grid_x, rx, tails, tails])
    y = np.concatenate([grid_y, ry, np.ones_like(tails), np.full_like(tails, -3.5)])
    return x, y


def swiglu_f64(x, y):
    return silu_f64(np.asarray(x, np.float16).astype(np.float64)) * np.asarray(y, np.float16).astype(np.float64)


def test_swiglu_oracle_matches_fp64():
    x, y = swiglu_inputs()
    got = oracle.swiglu(x, y)
    loose, strict = compare(got, swiglu_f64(x, y))
    assert loose == 0, f"{loose} outputs more than one fp16 ulp from FP64"
    assert strict == 0, f"{strict} outputs differ from the FP64 rounding away from any midpoint"


def test_moe_silu_oracle_matches_fp64():
    g = np.concatenate([all_finite_fp16(), np.linspace(-30, -12, 4001).astype(np.float16)])
    got = omoe.silu_fp16(g)
    loose, strict = compare(got, silu_f64(g.astype(np.float64)))
    assert loose == 0 and strict == 0, (loose, strict)
    # The MoE's h = fp16(fp16(silu(gate)) * up): the product of two fp16 values is exact in fp32,
    # so it is the single rounding of the FP64 product of the already-rounded silu.
    up = np.random.default_rng(1).standard_normal(g.size).astype(np.float16)
    with np.errstate(over="ignore"):
        h = omoe.fp16_mul(got, up)
        want = (got.astype(np.float64) * up.astype(np.float64)).astype(np.float16)
    assert np.array_equal(h.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("x, y, value", [
    (1.0, 1.0, 0.7310585786300049),
    (-1.0, 1.0, -0.2689414213699951),
    (2.0, 1.0, 1.7615941559557649),
    (-2.0, -1.0, 0.2384058440442351),
    (0.0, 5.0, 0.0),
    (-0.0, 5.0, 0.0),
    (10.0, 0.5, 4.999773010656488),
    (-20.0, 1.0, -4.122307244877116e-08),
    (65504.0, 1.0, 65504.0),
    (-65504.0, 1.0, 0.0),
])
def test_known_values(x, y, value):
    want = np.float16(value)
    got = oracle.swiglu(np.array([x], np.float16), np.array([y], np.float16))[0]
    assert got == want, (x, y, got, want)
    if y == 1.0:
        assert omoe.silu_fp16(np.array([x], np.float16))[0] == want


def _planted_swiglu(kind):
    """Copies of the SwiGLU formula with one plausible mistake each (checker self-test)."""
    def run(a, b):
        x = np.asarray(a, np.float16).astype(np.float32)
        y = np.asarray(b, np.float16).astype(np.float32)
        with np.errstate(over="ignore", invalid="ignore"):
            pos = np.float32(1) / (np.float32(1) + np.exp(-x))
            neg = np.exp(x) / (np.float32(1) + np.exp(x))
            if kind == "branches swapped":
                sig = np.where(x >= 0, neg, pos)
            elif kind == "sign slip":
                sig = np.where(x >= 0, np.float32(1) / (np.float32(1) + np.exp(x)), neg)
            else:
                sig = np.where(x >= 0, pos, neg)
            sig = sig.astype(np.float32)
            if kind == "fp16 intermediate":
                return ((x * sig).astype(np.float16).astype(np.float32) * y).astype(np.float16)
            if kind == "y dropped":
                return (x * sig).astype(np.float16)
            return ((x * sig).astype(np.float32) * y).astype(np.float16)
    return run


@pytest.mark.parametrize("kind", ["branches swapped", "sign slip", "fp16 intermediate", "y dropped"])
def test_checker_rejects_planted_mistakes(kind):
    x, y = swiglu_inputs()
    loose, strict = compare(_planted_swiglu(kind)(x, y), swiglu_f64(x, y))
    assert loose + strict > 0, kind
    # The unmodified copy passes the same comparison.
    assert compare(_planted_swiglu("none")(x, y), swiglu_f64(x, y)) == (0, 0)
