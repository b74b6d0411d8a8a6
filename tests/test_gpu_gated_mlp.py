"""The reference's gated-MLP call sequence through HipBackend, checked stage by stage.

``GatedMLP`` (/root/reference/src/venturi/models/gated_mlp.py:56-67, 97-120,
245-266) is the boundary's named caller. It uploads an RMSNorm vector and the
gate, up and down weights, prepares norm, gate, up and down plans plus the
backend's ``prepare_swiglu`` / ``prepare_add`` elementwise plans, and runs

    hidden = rms(x); gate = gate(hidden); up = up(hidden)
    gate = swiglu(gate, up)        (in place)
    hidden = down(gate); out = x + hidden

The sequence is restated here (the reference is not importable on the GPU box)
at the config-2 MLP shapes (hidden 5120, intermediate 17408, q8_g32_fp16),
and every stage's device output is checked against the oracle applied to the
device's own input of that stage: RMS and add bit for bit, SwiGLU within one
fp16 ulp of the oracle (the FP64-pinned restatement), the projections on the
auto route within the free-order tolerance of the canonical order.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import agreement, assert_free_order, bits, random_q8
from venturi_amd import Q8RowSplitWeight

pytestmark = pytest.mark.gpu

HIDDEN, INTER = 5120, 17408


@pytest.fixture(scope="module")
def mlp(backend, device):
    # Scales drawn so the stages keep O(1) magnitudes (gate/up ~ 1.3, down ~ 2).
    gate_codes, gate_scales = random_q8(INTER, HIDDEN, seed=101, scale=5e-4, zero_first_group=False)
    up_codes, up_scales = random_q8(INTER, HIDDEN, seed=102, scale=5e-4, zero_first_group=False)
    down_codes, down_scales = random_q8(HIDDEN, INTER, seed=103, scale=3e-4, zero_first_group=False)
    gamma = 1 + 0.1 * torch.randn(HIDDEN, generator=torch.Generator().manual_seed(104))
    weights = {
        "gate": Q8RowSplitWeight(gate_codes, gate_scales, HIDDEN),
        "up": Q8RowSplitWeight(up_codes, up_scales, HIDDEN),
        "down": Q8RowSplitWeight(down_codes, down_scales, INTER),
    }
    for operation in ("rmsnorm", "swiglu", "add"):
        backend.require(operation, dtype=torch.float16, device=device)
    for weight in weights.values():
        backend.require_linear(weight, dtype=torch.float16, device=device)
    resident = {name: backend.upload_linear(w, dtype=torch.float16, device=device) for name, w in weights.items()}
    norm = backend.upload_rmsnorm(gamma, dtype=torch.float16, device=device, epsilon=1e-6)
    return weights, resident, norm, gamma


def _close_to_oracle_swiglu(got16, gate16, up16):
    want = oracle.swiglu(gate16.view(np.float16), up16.view(np.float16)).astype(np.float64)
    stats = agreement(got16, want.astype(np.float16).view(np.uint16))
    assert stats["max_ulp"] <= 1.0, stats


@pytest.mark.parametrize("tokens", [1, 4, 16])
def test_gated_mlp_sequence(backend, device, mlp, tokens):
    print(f"case gated-mlp tokens={tokens}", flush=True)
    weights, resident, norm, gamma = mlp
    dtype = torch.float16
    swiglu = backend.prepare_swiglu(tokens=tokens, features=INTER, dtype=dtype, device=device)
    add = backend.prepare_add(tokens=tokens, features=HIDDEN, dtype=dtype, device=device)
    plans = {name: r.prepare(tokens=tokens) for name, r in resident.items()}
    norm_plan = norm.prepare(tokens=tokens)
    assert swiglu.workspace_bytes == add.workspace_bytes == norm_plan.workspace_bytes == 0
    assert all(p.workspace_bytes == 0 for p in plans.values())

    x = torch.randn(tokens, HIDDEN, generator=torch.Generator().manual_seed(200 + tokens)).half()
    xd = x.to(device)
    hidden = backend.empty([tokens, HIDDEN], dtype=dtype, device=device)
    gate = backend.empty([tokens, INTER], dtype=dtype, device=device)
    up = backend.empty([tokens, INTER], dtype=dtype, device=device)
    out = backend.empty([tokens, HIDDEN], dtype=dtype, device=device)

    # The reference's run order, with a copy of each stage's output for the checks.
    norm_plan.run(xd, out=hidden)
    normed = bits(hidden)
    plans["gate"].run(hidden, out=gate)
    plans["up"].run(hidden, out=up)
    gate_bits, up_bits = bits(gate), bits(up)
    swiglu.run(gate, up, out=gate)
    act = bits(gate)
    plans["down"].run(gate, out=hidden)
    down_bits = bits(hidden)
    add.run(xd, hidden, out=out)
    torch.cuda.synchronize()

    np.testing.assert_array_equal(normed, oracle.rms(bits(x), gamma.numpy(), 1e-6, dtype=0))
    for name, got, source in (("gate", gate_bits, normed), ("up", up_bits, normed), ("down", down_bits, act)):
        w = weights[name]
        want = oracle.q8_linear(source, w.codes.numpy(), w.scales.numpy(), w.in_features)
        stats = agreement(got, want)
        print(f"{name} tokens={tokens}: {stats}", flush=True)
        assert_free_order(stats)
    _close_to_oracle_swiglu(act, gate_bits, up_bits)
    summed = (x.numpy().astype(np.float32) + down_bits.view(np.float16).astype(np.float32)).astype(np.float16)
    np.testing.assert_array_equal(bits(out), summed.view(np.uint16))


def test_elementwise_plans_guard_operands(backend, device):
    for prepare in (backend.prepare_swiglu, backend.prepare_add):
        plan = prepare(tokens=2, features=64, dtype=torch.float16, device=device)
        buffer = torch.randn(2 * 64 + 1, device=device).half()
        a, shifted = buffer[:128].view(2, 64), buffer[1:].view(2, 64)
        b = torch.randn(2, 64, device=device).half()
        out = torch.empty_like(b)
        with pytest.raises(ValueError, match="requires shape"):
            plan.run(a[:1], b, out=out)
        with pytest.raises(ValueError, match="requires shape"):
            plan.run(a, b.float(), out=out)
        with pytest.raises(ValueError, match="alias"):
            plan.run(a, b, out=shifted)
        want = plan.run(a.clone(), b, out=torch.empty_like(b))
        assert plan.run(a, b, out=a) is a  # in place over an operand is allowed
        torch.cuda.synchronize()
        assert torch.equal(a, want)
    with pytest.raises(ValueError, match="positive int32"):
        backend.prepare_add(tokens=0, features=64, dtype=torch.float16, device=device)
