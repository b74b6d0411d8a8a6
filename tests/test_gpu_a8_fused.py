"""Fused W8A8 projections and the SwiGLU -> A8 producer.

Modelled on the reference's test_q8_fused.py: every fused output keeps the
bytes of the A8 projection of its matrix (checked against the CPU oracle),
pitched outputs leave their padding and guards untouched, graph replays follow
the inputs, and run() does no torch math or allocation. The producer's bytes
equal venturi_swiglu_run followed by the two-pass quantizer, and the oracle's
SwiGLU + quantizer.
"""

import ctypes as C

import numpy as np
import pytest
import torch

import oracle
from helpers import bits
from venturi_amd import Q8RowSplitWeight, prepare_q8_dp4a
from venturi_amd.q8_fused import OutputDescriptor, prepare_q8_fused

pytestmark = pytest.mark.gpu


def _setup(backend, device, n, k, tokens, seed=0):
    padded = (k + 127) // 128 * 128
    gen = torch.Generator().manual_seed(911 + 7 * n + k + tokens + seed)
    codes = torch.randint(-127, 128, (n, padded), dtype=torch.int8, generator=gen)
    scales = (torch.rand(n, padded // 32, generator=gen) * 0.01).half()
    scales[:, 0] = 0
    resident = backend.upload_linear(Q8RowSplitWeight(codes, scales, k), dtype=torch.float16, device=device)
    return codes, scales, resident


@pytest.mark.parametrize("passes", [1, 2])
@pytest.mark.parametrize("tokens", [1, 2, 3, 8, 23, 32, 64, 80])
@pytest.mark.parametrize("k", [67, 5120])
@pytest.mark.parametrize("ns", [(7, 33), (31, 17, 9)])
def test_fused_reference_bytes_and_pitched_guards(backend, device, passes, tokens, k, ns):
    print(f"case a8-fused ns={ns} k={k} tokens={tokens} passes={passes}", flush=True)
    data = [_setup(backend, device, n, k, tokens, i) for i, n in enumerate(ns)]
    x_cpu = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens + k)).half()
    x = x_cpu.to(device)
    strides = [n + 5 for n in ns]
    plan = prepare_q8_fused([d[2] for d in data], tokens=tokens, residual_compensation=passes == 2,
                            output_strides=strides)
    assert plan.precision_profile.endswith("-residual-a8") == (passes == 2)
    work = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    guards = [torch.full((tokens * s + 2,), 47, dtype=torch.float16, device=device) for s in strides]
    outputs = [g[1:-1].view(tokens, s) for g, s in zip(guards, strides)]
    plan.run(x, outputs=outputs, workspace=work)
    scratch = work.clone()
    q, d = oracle.a8_quantize(bits(x_cpu), passes)
    np.testing.assert_array_equal(scratch.cpu().numpy(), oracle.a8_workspace(q, d))
    for (codes, scales, resident), n, out, g in zip(data, ns, outputs, guards):
        expected = oracle.a8_linear(q, d, codes.numpy(), scales.numpy(), k)
        np.testing.assert_array_equal(bits(out[:, :n].contiguous()), expected)
        single = prepare_q8_dp4a(resident, tokens=tokens, residual_compensation=passes == 2, route="exact")
        actual = torch.empty(tokens, n, dtype=torch.float16, device=device)
        single.run(x, out=actual, workspace=work)
        assert torch.equal(out[:, :n].contiguous().view(torch.int16), actual.view(torch.int16))
        gc = g.cpu()
        assert gc[0] == gc[-1] == 47 and bool((out[:, n:] == 47).all())
        assert torch.equal(scratch, work)


@pytest.mark.parametrize("tokens", [8, 23, 32, 70])
def test_large_and_tiny_mixed_descriptors(backend, device, tokens):
    ns = (1025, 17, 33)
    data = [_setup(backend, device, n, 6145, tokens, i) for i, n in enumerate(ns)]
    x_cpu = torch.randn(tokens, 6145, generator=torch.Generator().manual_seed(tokens)).half()
    plan = prepare_q8_fused([d[2] for d in data], tokens=tokens, residual_compensation=True)
    work = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    outs = [torch.empty(tokens, n, dtype=torch.float16, device=device) for n in ns]
    plan.run(x_cpu.to(device), outputs=outs, workspace=work)
    q, d = oracle.a8_quantize(bits(x_cpu), 2)
    for (codes, scales, _), out in zip(data, outs):
        np.testing.assert_array_equal(bits(out), oracle.a8_linear(q, d, codes.numpy(), scales.numpy(), 6145))


def test_graph_nonfinite_alias_packed_and_no_torch_math(backend, device, monkeypatch):
    res = [_setup(backend, device, n, 128, 3)[2] for n in (17, 33)]
    plan = prepare_q8_fused(res, tokens=3, residual_compensation=True)
    x = torch.ones(3, 128, dtype=torch.float16, device=device)
    work = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    outs = [torch.empty(3, n, dtype=torch.float16, device=device) for n in (17, 33)]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run(x, outputs=outs, workspace=work)
    x.fill_(float("inf"))
    graph.replay()
    torch.cuda.synchronize(device)
    assert all(torch.isnan(o).all() for o in outs)
    x.zero_()
    graph.replay()
    torch.cuda.synchronize(device)
    assert all(not o.any() for o in outs)
    with pytest.raises(ValueError, match="alias"):
        plan.run(x, outputs=[work[:102].view(torch.float16).view(3, 17), outs[1]], workspace=work)
    # packed=True reuses the caller's quantized workspace: with x changed after
    # quantizing, the outputs still follow the packed activations.
    x.fill_(1.0)
    plan.run(x, outputs=outs, workspace=work)
    want = [o.clone() for o in outs]
    x.zero_()
    plan.run(x, outputs=outs, workspace=work, packed=True)
    assert all(torch.equal(a, b) for a, b in zip(outs, want))
    with pytest.raises(ValueError, match="packed"):
        plan.run(x, outputs=outs, workspace=work, packed=1)

    def forbidden(*a, **kw):
        raise AssertionError("fused execution used torch math or allocation")

    with monkeypatch.context() as m:
        for name in ("empty", "zeros", "matmul", "mm"):
            m.setattr(torch, name, forbidden)
        plan.run(x, outputs=outs, workspace=work)
    torch.cuda.synchronize(device)


def test_plan_admission(backend, device):
    a = _setup(backend, device, 7, 67, 2)[2]
    b = _setup(backend, device, 9, 67, 2)[2]
    c = _setup(backend, device, 9, 68, 2)[2]
    with pytest.raises(ValueError, match="same device, backend and K"):
        prepare_q8_fused([a, c], tokens=2, residual_compensation=True)
    with pytest.raises(ValueError, match="strides"):
        prepare_q8_fused([a, b], tokens=2, residual_compensation=True, output_strides=[6, 9])
    with pytest.raises(ValueError, match="strides"):
        prepare_q8_fused([a, b], tokens=2, residual_compensation=True, output_strides=[7])
    plan = prepare_q8_fused([a, b], tokens=2, residual_compensation=True)
    work = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    x = torch.ones(2, 67, dtype=torch.float16, device=device)
    outs = [torch.empty(2, n, dtype=torch.float16, device=device) for n in (7, 9)]
    with pytest.raises(ValueError, match="one output per fused matrix"):
        plan.run(x, outputs=outs[:1], workspace=work)


def test_raw_invalid_descriptor_geometry(backend, device):
    values = [_setup(backend, device, n, 67, 2)[2] for n in (7, 33)]
    plan = prepare_q8_fused(values, tokens=2, residual_compensation=True)
    work = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    x = torch.ones(2, 67, dtype=torch.float16, device=device)
    outs = [torch.empty(2, n, dtype=torch.float16, device=device) for n in (7, 33)]
    plan.run(x, outputs=outs, workspace=work)
    desc = plan._descriptors(outs)
    stream = torch.cuda.current_stream(device).cuda_stream
    args = [work.data_ptr(), work.numel(), C.cast(desc, C.c_void_p), 2, 2, 67, 128, 2, stream]
    assert plan._run(*args) == 0
    for idx, value in [(0, 0), (1, work.numel() - 1), (2, None), (3, 1), (3, 4), (4, 0), (5, 0), (6, 67), (7, 3),
                       (0, work.data_ptr() + 1)]:
        bad = args.copy()
        bad[idx] = value
        assert plan._run(*bad) == -1, (idx, value)
    short = (OutputDescriptor * 2)(desc[0], OutputDescriptor(desc[1].codes, desc[1].scales, desc[1].out, 33, 32))
    assert plan._run(work.data_ptr(), work.numel(), C.cast(short, C.c_void_p), 2, 2, 67, 128, 2, stream) == -1
    assert "descriptor" in backend._native.error()
    torch.cuda.synchronize(device)


@pytest.mark.parametrize("tokens", [1, 3, 32, 257])
@pytest.mark.parametrize("k", [67, 5120, 8704])
def test_swiglu_producer_bytes(backend, device, tokens, k):
    print(f"case swiglu-a8 tokens={tokens} k={k}", flush=True)
    lib = backend._native
    gen = torch.Generator().manual_seed(tokens * 7 + k)
    gate_cpu = (torch.randn(tokens, k, generator=gen) * 3).half()
    up_cpu = torch.randn(tokens, k, generator=gen).half()
    if tokens >= 3:
        gate_cpu[1, 5] = float("inf")  # one non-finite group: zero codes, NaN scales
    gate, up = gate_cpu.to(device), up_cpu.to(device)
    need = lib.venturi_q8_dp4a_bytes(tokens, k, 2)
    stream = torch.cuda.current_stream(device).cuda_stream
    fused = torch.full((need,), 3, dtype=torch.uint8, device=device)
    inter = torch.empty(tokens, k, dtype=torch.float16, device=device)
    assert lib.venturi_swiglu_q8_quantize(gate.data_ptr(), up.data_ptr(), fused.data_ptr(), need, tokens, k, 256,
                                          inter.data_ptr(), stream) == 0
    again = torch.full((need,), 9, dtype=torch.uint8, device=device)
    assert lib.venturi_swiglu_q8_quantize(gate.data_ptr(), up.data_ptr(), again.data_ptr(), need, tokens, k, 128,
                                          None, stream) == 0
    act = torch.empty(tokens, k, dtype=torch.float16, device=device)
    assert lib.venturi_swiglu_run(gate.data_ptr(), up.data_ptr(), act.data_ptr(), tokens * k, 0, stream) == 0
    plain = torch.empty(need, dtype=torch.uint8, device=device)
    assert lib.venturi_q8_dp4a_quantize(act.data_ptr(), plain.data_ptr(), need, tokens, k, 2, stream) == 0
    torch.cuda.synchronize(device)
    assert torch.equal(fused, plain) and torch.equal(again, plain)
    assert torch.equal(inter.view(torch.int16), act.view(torch.int16))
    # SwiGLU against the oracle within one fp16 ulp (exp is not bit-pinned on
    # either side); the quantizer bytes exactly, on the device's SwiGLU values.
    want = oracle.swiglu(gate_cpu.numpy(), up_cpu.numpy()).astype(np.float64)
    got = act.cpu().numpy().astype(np.float64)
    finite = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), finite)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want[finite]), 2.0**-14))) - 10)
    assert (np.abs(got[finite] - want[finite]) <= ulp).all()
    q, d = oracle.a8_quantize(bits(act), 2)
    np.testing.assert_array_equal(fused.cpu().numpy(), oracle.a8_workspace(q, d))


def test_swiglu_producer_rejects_bad_operands(backend, device):
    lib = backend._native
    tokens, k = 2, 64
    need = lib.venturi_q8_dp4a_bytes(tokens, k, 2)
    gate = torch.ones(tokens, k, dtype=torch.float16, device=device)
    up = torch.ones(tokens, k, dtype=torch.float16, device=device)
    work = torch.empty(need + 256, dtype=torch.uint8, device=device)
    s = torch.cuda.current_stream(device).cuda_stream
    call = lib.venturi_swiglu_q8_quantize
    assert call(gate.data_ptr(), up.data_ptr(), work.data_ptr(), need, tokens, k, 64, None, s) == -1
    assert call(gate.data_ptr(), up.data_ptr(), work.data_ptr(), need - 1, tokens, k, 256, None, s) == -1
    assert call(gate.data_ptr(), up.data_ptr(), work.data_ptr() + 8, need, tokens, k, 256, None, s) == -1
    assert call(gate.data_ptr(), up.data_ptr(), gate.data_ptr(), need, tokens, k, 256, None, s) == -1
    assert "invalid fused SwiGLU" in lib.error()
    assert call(gate.data_ptr(), up.data_ptr(), work.data_ptr(), need, tokens, k, 256, work.data_ptr(), s) == -1
    assert "overlap" in lib.error()
    # The debug output may alias gate or up exactly (in-place), as the reference allows.
    assert call(gate.data_ptr(), up.data_ptr(), work.data_ptr(), need, tokens, k, 256, gate.data_ptr(), s) == 0
    torch.cuda.synchronize(device)
