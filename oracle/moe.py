"""CPU oracle of the routed-expert Q4 MoE. TEST INFRASTRUCTURE ONLY.

Loaded by tests/ and bench.py's cpu_baseline leg as a checker; never by the
product package. Restates flash_next_moe.py:139-161 / flash_next_q4.py:204-224
(fp16 boundaries) in numpy:

* per expert in ascending id order, its (position, token) pairs in
  position-major order (``torch.where((ids == e).T)``);
* gate/up and down GEMMs of fp16 activations with the fp16 decoded weights
  fp16(q * scale), accumulated in FP64 and rounded once to fp16 (the
  reference's F.linear is pinned by tolerance only, so its association is
  not restated);
* ``h = fp16(fp16(silu(gate)) * up)`` with silu in fp32;
* ``v = fp16(y * score)``; ``out[token] = fp16(out[token] + v)`` from +0.

fp16 x fp16 products and fp16 + fp16 sums are formed in fp32 and rounded to
fp16 once: the product is exact in fp32, and for the sum fp32 carries more than
2 * 11 + 2 bits, so the double rounding equals one rounding of the exact sum.
"""

import numpy as np


def silu_fp16(gate):
    """F.silu on fp16 (flash_next_q4.py:222): fp16(g / (1 + e^-g)) evaluated in fp32.

    Pinned against FP64 over every finite fp16 input (tests/test_silu_oracle.py).
    """
    g = np.asarray(gate, dtype=np.float16).astype(np.float32)
    with np.errstate(over="ignore"):  # e^-g overflows to inf for g < -88.7: g / inf = -0, as in fp32
        return (g / (np.float32(1.0) + np.exp(-g))).astype(np.float16)


def fp16_mul(a, b):
    return (np.asarray(a, np.float16).astype(np.float32) * np.asarray(b, np.float16).astype(np.float32)).astype(
        np.float16
    )


def fp16_add(a, b):
    return (np.asarray(a, np.float16).astype(np.float32) + np.asarray(b, np.float16).astype(np.float32)).astype(
        np.float16
    )


def linear_fp16(x, w):
    """fp16(x @ w^T) from FP64 accumulation of fp16 operands."""
    return (np.asarray(x, np.float16).astype(np.float64) @ np.asarray(w, np.float16).astype(np.float64).T).astype(
        np.float16
    )


def expert_pairs(ids, expert):
    """(positions, tokens) of ``torch.where((ids == expert).T)``: position-major."""
    positions, tokens = np.nonzero((np.asarray(ids) == expert).T)
    return positions, tokens


def swiglu(gate_up):
    """h = fp16(fp16(silu(gate)) * up) for gate_up fp16 [rows, 2I] (gate columns first)."""
    inter = gate_up.shape[1] // 2
    return fp16_mul(silu_fp16(gate_up[:, :inter]), gate_up[:, inter:])


def routed_experts(x, ids, scores, gate_up, down):
    """x fp16 [T, H]; ids int [T, K]; scores fp16 [T, K]; gate_up fp16 [E][2I, H]; down fp16 [E][H, I]."""
    x = np.asarray(x, np.float16)
    scores = np.asarray(scores, np.float16)
    out = np.zeros_like(x)
    for expert in np.unique(ids):
        positions, tokens = expert_pairs(ids, expert)
        h = swiglu(linear_fp16(x[tokens], gate_up[expert]))
        v = fp16_mul(linear_fp16(h, down[expert]), scores[tokens, positions][:, None])
        for i, t in enumerate(tokens):  # sequential: a token may repeat an expert
            out[t] = fp16_add(out[t], v[i])
    return out


def tokenwise(x, ids, scores, gate_up, down):
    """Per-token restatement (tests/test_flash_next_moe.py:49-72 shape): experts ascending."""
    x = np.asarray(x, np.float16)
    out = np.zeros_like(x)
    for t in range(x.shape[0]):
        order = sorted(range(ids.shape[1]), key=lambda p: (int(ids[t, p]), p))
        acc = np.zeros(x.shape[1], np.float16)
        for p in order:
            e = int(ids[t, p])
            h = swiglu(linear_fp16(x[t : t + 1], gate_up[e]))
            v = fp16_mul(linear_fp16(h, down[e]), scores[t, p])
            acc = fp16_add(acc, v[0])
        out[t] = acc
    return out


def combine(ids, pair_slot, values):
    """Ascending-expert fp16 accumulation of ``values[pair_slot[t, p]]`` per token (slot < 0 skipped)."""
    ids = np.asarray(ids)
    tokens, top_k = ids.shape
    order = np.lexsort((np.broadcast_to(np.arange(top_k), ids.shape), ids), axis=1)
    out = np.zeros((tokens, values.shape[1]), np.float16)
    rows = np.arange(tokens)
    for j in range(top_k):
        slot = pair_slot[rows, order[:, j]]
        live = slot >= 0
        out[live] = fp16_add(out[live], values[slot[live]])
    return out
