"""Shared test helpers: seeded inputs and fp16 bit comparisons."""

import numpy as np
import torch


def bits(tensor):
    """uint16 view of a CPU/GPU fp16 or bf16 tensor."""
    return tensor.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def random_q8(n, k, seed, scale=0.004, zero_first_group=True):
    """Random Q8 planes as the reference's tiling test draws them (test_q8_tiling.py:34-38)."""
    padded = (k + 127) // 128 * 128
    gen = torch.Generator().manual_seed(seed)
    codes = torch.randint(-127, 128, (n, padded), dtype=torch.int8, generator=gen)
    scales = (torch.rand(n, padded // 32, generator=gen) * scale).half()
    if zero_first_group and k > 32:
        scales[:, 0] = 0
    return codes, scales


def guarded_out(tokens, n, dtype, device, fill=47):
    """Output view with one sentinel element on each side."""
    guard = torch.full((tokens * n + 2,), fill, dtype=dtype, device=device)
    return guard, guard[1:-1].view(tokens, n)


def ulp16(v):
    """fp16 ulp at |v| (subnormal spacing below 2^-14)."""
    v = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(v, 2.0**-14)))
    return 2.0 ** (e - 10)


def agreement(got, ref):
    """Raw agreement of fp16 outputs with reference-order fp16 values.

    ``got`` and ``ref`` are float arrays (or fp16 bit patterns as uint16) of one
    shape. Returns max-abs, the largest difference in fp16 ulps of the reference
    value, the number of outputs that differ at all, the number above 2e-3, and
    the relative L2 error.
    """
    def f64(a):
        a = np.asarray(a)
        return (a.view(np.float16) if a.dtype == np.uint16 else a).astype(np.float64)

    g, r = f64(got), f64(ref)
    diff = np.abs(g - r)
    return {
        "max_abs": float(diff.max(initial=0.0)),
        "max_ulp": float((diff / ulp16(r)).max(initial=0.0)),
        "max_over_tolerance": float((diff / np.maximum(2e-3, ulp16(r))).max(initial=0.0)),
        "flips": int((diff > 0).sum()),
        "over_2e-3": int((diff > 2e-3).sum()),
        "rel_l2": float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30)),
        "count": int(r.size),
    }


def assert_free_order(stats, flip_fraction=0.02, over_fraction=0.01):
    """The tolerance of free-order (matrix-core) routes against the reference order.

    Every output is within max(2e-3, one fp16 ulp of the reference value): the
    2e-3 gate wherever |y| < 4, where an fp16 ulp is at most 1.95e-3; above 4
    a single rounding flip is 3.9e-3, the one stated deviation from that gate.
    rel-L2 <= 1e-3; at most `flip_fraction` of the outputs differ at all and
    at most `over_fraction` by more than 2e-3.
    """
    assert stats["max_over_tolerance"] <= 1.0, stats
    assert stats["rel_l2"] <= 1e-3, stats
    assert stats["flips"] <= max(2, flip_fraction * stats["count"]), stats
    assert stats["over_2e-3"] <= max(2, over_fraction * stats["count"]), stats


def near_tie_matrix(levels, group, rows, groups, seed):
    """fp32 [rows, groups * group] whose quotients x / scale sit on or within
    three fp32 ulps of half-integers, for the RTN rule scale = fp16(max|x| /
    levels), code = rint(fl32(x / scale)).

    Each group holds max|x| = fl32(levels * d) for an fp16 scale d (normal or
    subnormal, non-power-of-two mantissas), so the stored scale is d; the other
    values are (t + 1/2) d moved by -3..3 ulps (one in seven an exact tie), so
    nearly all of them lie inside the packers' guard band around half-integers
    and take the IEEE division. (With an fp16
    scale and |t| < 128, t d is exact in fp32 and any other fp32 x has |x / d -
    t| >= ulp(x) / d > ulp(t) / 2, so fl32(x / d) is a half-integer only when
    x / d is one.)
    """
    rng = np.random.default_rng(seed)
    out = np.zeros((rows, groups * group), np.float32)
    for r in range(rows):
        for g in range(groups):
            while True:
                tiny = rng.random() < 0.15
                d = np.float16(rng.integers(1, 1024) * 2.0**-24) if tiny else np.float16(rng.uniform(2.0**-12, 4.0))
                amax = np.float32(levels * float(d))
                if d > 0 and np.float16(amax / np.float32(levels)) == d:
                    break
            vals = [amax * (1 if rng.random() < 0.5 else -1)]
            for _ in range(group - 1):
                t = rng.integers(-levels, levels) + 0.5
                x = np.float32(t * float(d))
                for _ in range(abs(step := int(rng.integers(-3, 4)))):
                    x = np.nextafter(x, np.float32(np.sign(step) * np.inf))
                vals.append(x)
            out[r, g * group:(g + 1) * group] = np.array(vals, np.float32)[rng.permutation(group)]
    return out
