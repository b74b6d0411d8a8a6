"""Pins of the CPU oracle's Q4 and MoE functions (no GPU).

Each check is a known answer from the reference's own tests, a closed form,
or an input built so that a plausible mistake (wrong nibble, wrong scale
index, wrong lane assignment or accumulation order) changes the answer.
"""

import numpy as np
import pytest
import torch

import oracle
import oracle.moe as omoe
from venturi_amd import Q4RowSplitWeight, decode_q4_fp16, quantize_q4_rtn


def f16(values):
    return np.asarray(values, dtype=np.float16)


def q4(codes, scales):
    return Q4RowSplitWeight.from_codes(torch.tensor(codes, dtype=torch.int8), torch.tensor(scales, dtype=torch.float16))


def test_known_bytes_decode():
    """tests/test_q4_weights.py:30-44: low nibble first, no offset-zero convention."""
    codes = np.zeros((1, 64), dtype=np.uint8)
    codes[0, :3] = [0x10, 0xF8, 0x97]
    scales = f16([[0.5, -2]])
    want = [0, 0.5, -4, -0.5, 3.5, -3.5]
    assert oracle.q4_decode_fp16(codes, scales, 128)[0, :6].tolist() == want
    assert oracle.q4_decode(codes, scales, 128).view(np.float16)[0, :6].tolist() == want


def test_minus8_and_rtn_ties():
    """tests/test_flash_next_q4.py:35-48,119-121."""
    w = q4([[-8, 7, -1, 0]], [[0.5]])
    assert oracle.q4_decode(w.codes.numpy(), w.scales.numpy(), 4).view(np.float16).tolist() == [[-4.0, 3.5, -0.5, 0.0]]
    x = np.zeros((2, 128), dtype=np.float32)
    x[0, :6] = [7.0, 0.5, 1.5, 2.5, -0.5, -1.5]
    x[1, 0] = 1e-10
    codes, scales = oracle.q4_rtn(x)
    packed, plane = oracle.q4_pack_codes(codes, scales)
    y = oracle.q4_decode_fp16(packed, plane, 128)
    assert y[0, :6].tolist() == [7.0, 0.0, 2.0, 2.0, 0.0, -2.0]
    assert not y[1].any() and scales[0, 0] == 1
    # The package encoder (reference semantics, torch) gives the same planes.
    q = quantize_q4_rtn(torch.from_numpy(x))
    assert np.array_equal(q.codes.numpy(), packed) and np.array_equal(q.scales.numpy(), plane)


@pytest.mark.parametrize("k", [1, 63, 64, 65, 129, 4097])
def test_decode_c_equals_numpy_and_package(k):
    gen = torch.Generator().manual_seed(k)
    codes = torch.randint(-8, 8, (5, k), dtype=torch.int8, generator=gen)
    scales = (torch.rand(5, (k + 63) // 64, generator=gen) * 2.0**-13).half()  # includes subnormal products
    w = Q4RowSplitWeight.from_codes(codes, scales)
    a = oracle.q4_decode(w.codes.numpy(), w.scales.numpy(), k)
    b = oracle.q4_decode_fp16(w.codes.numpy(), w.scales.numpy(), k).view(np.uint16)
    c = decode_q4_fp16(w).numpy().view(np.uint16)
    assert np.array_equal(a, b) and np.array_equal(a, c)
    exact = codes.double().numpy() * np.repeat(scales.double().numpy(), 64, axis=1)[:, :k]
    assert np.array_equal(a.view(np.float16), exact.astype(np.float16))


def impulse_case(order, dtype=0):
    """x = e_j gives exactly fp16(q_j * s_j) in every order (one nonzero term)."""
    gen = torch.Generator().manual_seed(3)
    k = 200
    codes = torch.randint(-8, 8, (7, k), dtype=torch.int8, generator=gen)
    scales = (torch.rand(7, 4, generator=gen) * 0.3).half()
    w = Q4RowSplitWeight.from_codes(codes, scales)
    x = np.eye(k, dtype=np.float16).view(np.uint16)
    if dtype == 1:
        x = (np.eye(k, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)
    if order == "generic":
        y = oracle.q4_generic(x, w.codes.numpy(), w.scales.numpy(), k, dtype)
    elif order == "fused":
        y = oracle.q4_fused(x, w.codes.numpy(), w.scales.numpy(), k)
    else:
        y = oracle.q4_linear(x, w.codes.numpy(), w.scales.numpy(), k)
    want = oracle.q4_decode_fp16(w.codes.numpy(), w.scales.numpy(), k).T
    if dtype == 1:
        exact = (codes.double() * scales.double().repeat_interleave(64, 1)[:, :k]).T.float()
        want_bits = torch.from_numpy(exact.numpy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(y, want_bits)
    else:
        assert np.array_equal(y, want.view(np.uint16))


@pytest.mark.parametrize("order", ["expert", "generic", "fused"])
def test_impulse_picks_each_weight(order):
    impulse_case(order)


def test_impulse_generic_bf16():
    impulse_case("generic", dtype=1)


def cancellation(cols_big, col_small, k=192):
    """Weights 1.0 everywhere; x = +B, small, -B at the given columns (B = 2048, small = 2^-14)."""
    w = q4(np.ones((1, k), dtype=np.int8).tolist(), [[1.0] * ((k + 63) // 64)])
    x = np.zeros((1, k), dtype=np.float16)
    x[0, cols_big[0]] = 2048
    x[0, cols_big[1]] = -2048
    x[0, col_small] = 2.0**-14
    return w, x


def test_lane_assignment_and_order_expert():
    # flash_next_q4.cu:28-29: lane l owns columns l, l+32, l+64 in order.
    w, x = cancellation((0, 64), 32)  # all in lane 0: (B + small) - B = 0 in fp32
    assert oracle.q4_linear(x.view(np.uint16), w.codes.numpy(), w.scales.numpy(), 192).view(np.float16)[0, 0] == 0
    w, x = cancellation((0, 64), 1)  # small in lane 1 survives the tree
    assert oracle.q4_linear(x.view(np.uint16), w.codes.numpy(), w.scales.numpy(), 192).view(np.float16)[0, 0] == 2.0**-14


@pytest.mark.parametrize("order", ["generic", "fused"])
def test_lane_assignment_and_order_plugin(order):
    # q4_linear.cu:33-45 / q4_fused.cuh: lane l owns columns 64g+2l, 64g+2l+1.
    run = (lambda x, w: oracle.q4_generic(x, w.codes.numpy(), w.scales.numpy(), 192)) if order == "generic" else (
        lambda x, w: oracle.q4_fused(x, w.codes.numpy(), w.scales.numpy(), 192)
    )
    w, x = cancellation((0, 64), 1)  # all three in lane 0
    got = run(x.view(np.uint16), w).view(np.float16)[0, 0]
    if order == "generic":
        assert got == 0
    else:  # the fused term RNE(x0 + x1) = B first absorbs small too
        assert got == 0
    w, x = cancellation((0, 64), 32)  # small in lane 16
    assert run(x.view(np.uint16), w).view(np.float16)[0, 0] == 2.0**-14


@pytest.mark.parametrize("order", ["expert", "generic", "fused"])
def test_fp64_bound(order):
    gen = torch.Generator().manual_seed(17)
    n, k, t = 9, 333, 3
    codes = torch.randint(-8, 8, (n, k), dtype=torch.int8, generator=gen)
    scales = (torch.rand(n, 6, generator=gen) * 0.05).half()
    w = Q4RowSplitWeight.from_codes(codes, scales)
    x = torch.randn(t, k, generator=gen).half()
    xs = x.numpy().view(np.uint16)
    c, s = w.codes.numpy(), w.scales.numpy()
    y = {"expert": lambda: oracle.q4_linear(xs, c, s, k), "generic": lambda: oracle.q4_generic(xs, c, s, k),
         "fused": lambda: oracle.q4_fused(xs, c, s, k)}[order]().view(np.float16).astype(np.float64)
    wd = (codes.double() * scales.double().repeat_interleave(64, 1)[:, :k]).numpy()
    if order == "expert":
        wd = wd.astype(np.float16).astype(np.float64)
    exact = x.double().numpy() @ wd.T
    mag = np.abs(x.double().numpy()) @ np.abs(wd).T
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(exact), 2.0**-14))) - 10)
    assert (np.abs(y - exact) <= 0.5 * ulp + k * 2.0**-24 * mag).all()


# ------------------------------------------------------------------ MoE


def small_moe(seed, tokens=6, experts=5, hidden=16, inter=8, top_k=3, duplicates=False):
    rng = np.random.default_rng(seed)
    gate_up = (rng.standard_normal((experts, 2 * inter, hidden)) * 0.3).astype(np.float16)
    down = (rng.standard_normal((experts, hidden, inter)) * 0.3).astype(np.float16)
    ids = np.stack([rng.permutation(experts)[:top_k] for _ in range(tokens)])
    if duplicates:
        ids[::2, -1] = ids[::2, 0]
    scores = rng.random((tokens, top_k)).astype(np.float16)
    x = rng.standard_normal((tokens, hidden)).astype(np.float16)
    return x, ids, scores, gate_up, down


@pytest.mark.parametrize("duplicates", [False, True])
def test_moe_expert_loop_equals_tokenwise(duplicates):
    """flash_next_moe.py:139-161 per-expert loop == tests/test_flash_next_moe.py:49-72 per-token form."""
    x, ids, scores, gu, dn = small_moe(1, duplicates=duplicates)
    a = omoe.routed_experts(x, ids, scores, gu, dn)
    b = omoe.tokenwise(x, ids, scores, gu, dn)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_moe_single_expert_closed_form():
    """top_k = 1 with score 1: out = fp16(down(fp16(silu(g)) * u)) exactly."""
    x, ids, scores, gu, dn = small_moe(2, top_k=1)
    scores[:] = 1
    out = omoe.routed_experts(x, ids, scores, gu, dn)
    for t in range(x.shape[0]):
        e = ids[t, 0]
        g = (x[t].astype(np.float64) @ gu[e, :8].astype(np.float64).T).astype(np.float16)
        u = (x[t].astype(np.float64) @ gu[e, 8:].astype(np.float64).T).astype(np.float16)
        s = (g.astype(np.float32) / (1 + np.exp(-g.astype(np.float32)))).astype(np.float16)
        h = (s.astype(np.float32) * u.astype(np.float32)).astype(np.float16)
        y = (h.astype(np.float64) @ dn[e].astype(np.float64).T).astype(np.float16)
        assert np.array_equal(out[t].view(np.uint16), y.view(np.uint16))


def test_moe_combine_order_is_ascending_expert():
    """Values chosen so that fp16 addition order is visible: 2048 + 1 + 1 vs 1 + 1 + 2048."""
    ids = np.array([[3, 1, 2]])
    values = np.array([[2048.0], [1.0], [1.0]], dtype=np.float16)  # slots 0, 1, 2
    pair_slot = np.array([[0, 1, 2]])  # expert 3 -> 2048, expert 1 -> 1, expert 2 -> 1
    out = omoe.combine(ids, pair_slot, values)
    assert out[0, 0] == 2050  # ascending: 1 + 1 = 2, 2 + 2048 = 2050 (exact)
    ids = np.array([[1, 3, 2]])
    pair_slot = np.array([[0, 1, 2]])  # expert 1 -> 2048 first, then +1 twice: each rounds back to 2048
    assert omoe.combine(ids, pair_slot, values)[0, 0] == 2048
    # Skipped slots.
    assert omoe.combine(np.array([[0, 1]]), np.array([[-1, 2]]), values)[0, 0] == 1


def test_moe_pairs_position_major():
    ids = np.array([[2, 0], [0, 2], [2, 1]])
    positions, tokens = omoe.expert_pairs(ids, 2)
    assert positions.tolist() == [0, 0, 1] and tokens.tolist() == [0, 2, 1]
