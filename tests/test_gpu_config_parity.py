"""Parity at the benchmarked shapes: the launches the bench times, against the oracle.

* The fused gate+up SwiGLU plan at the config-2 gate+up matrix [34816 x 5120].
* A config-5 chain (two decoder layers of the config-2 projections, the bench's
  step) at B in {1, 8, 32}, checked stage by stage: each stage's output on
  sampled rows against the oracle fed with the stage's own device input, and
  HIP-graph replays against the eager step.
* RMSNorm + A8 at the config-3 input (2048 x 5120 with 51 channels scaled by
  20), bytes against the oracle, then the A8 GEMM at the QKV shape on it.

Free-order routes are held to helpers.assert_free_order (every output within
max(2e-3, one fp16 ulp) of the reference-order value, rel-L2 <= 1e-3, few
flips). The fused SwiGLU output is checked through its two projections
(check_swiglu).
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import agreement, assert_free_order, bits
from venturi_amd import prepare_q8_dp4a, prepare_rms_q8

pytestmark = pytest.mark.gpu

HIDDEN, QKV, O_IN, INTER = 5120, 7168, 6144, 17408


def _packed(backend, device, n, k, seed):
    gen = torch.Generator(device=device).manual_seed(seed)
    w = torch.randn(n, k, generator=gen, device=device) * 0.02
    packed = backend.quantize_q8(w)
    del w
    return packed


def _planes(packed, rows):
    index = torch.as_tensor(rows, dtype=torch.int64, device=packed.codes.device)
    return packed.codes[index].cpu().numpy(), packed.scales[index].cpu().numpy()


def _swiglu16(gate16, up16):
    return oracle.swiglu(gate16.view(np.float16), up16.view(np.float16)).view(np.uint16)


def check_swiglu(backend, device, packed, resident, x, fused_out, cols):
    """The fused SwiGLU plan's output on intermediate columns `cols`.

    * The whole output has the bytes of the matrix-core projection followed by
      venturi_silu_mul_run.
    * The projection's gate and up columns agree with the oracle's
      reference-order values (assert_free_order).
    * The epilogue: every output is within one fp16 ulp of the oracle's swiglu
      of the device's own gate and up (the exp inside silu is not bit-pinned).
    * End to end against the oracle's swiglu of the reference-order gate and
      up: rel-L2 <= 1e-3 (the stats are returned).
    """
    tokens, inter = fused_out.shape
    gate_up = torch.empty(tokens, 2 * inter, dtype=torch.float16, device=device)
    resident.prepare(tokens=tokens, route="mfma").run(x, out=gate_up)
    want = torch.empty_like(fused_out)
    backend._check(backend._native.venturi_silu_mul_run(gate_up.data_ptr(), want.data_ptr(), tokens, inter, 0,
                                                        torch.cuda.current_stream(device).cuda_stream))
    assert torch.equal(fused_out.view(torch.int16), want.view(torch.int16))
    gc, gs = _planes(packed, cols)
    uc, us = _planes(packed, cols + inter)
    gate_ref = oracle.q8_linear(bits(x), gc, gs, x.shape[1])
    up_ref = oracle.q8_linear(bits(x), uc, us, x.shape[1])
    gate_dev, up_dev = bits(gate_up)[:, cols], bits(gate_up)[:, cols + inter]
    assert_free_order(agreement(gate_dev, gate_ref))
    assert_free_order(agreement(up_dev, up_ref))
    got = bits(fused_out)[:, cols]
    epilogue = agreement(got, _swiglu16(gate_dev, up_dev))
    assert epilogue["max_ulp"] <= 1.0, epilogue
    stats = agreement(got, _swiglu16(gate_ref, up_ref))
    assert stats["rel_l2"] <= 1e-3, stats
    return stats


@pytest.mark.parametrize("tokens", [1, 8, 16, 32])
def test_swiglu_gate_up_config2(backend, device, tokens):
    print(f"case swiglu-config2 tokens={tokens}", flush=True)
    n, k = 2 * INTER, HIDDEN
    packed = _packed(backend, device, n, k, 4242)
    resident = backend.upload_linear(packed, dtype=torch.float16, device=device)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens + 1)).half().to(device)
    out = torch.empty(tokens, INTER, dtype=torch.float16, device=device)
    resident.prepare_swiglu(tokens=tokens).run(x, out=out)
    cols = np.sort(np.random.default_rng(tokens).choice(INTER, 96, replace=False))
    stats = check_swiglu(backend, device, packed, resident, x, out, cols)
    print(f"swiglu tokens={tokens}: {stats}", flush=True)


@pytest.fixture(scope="module")
def two_layers(backend, device):
    shapes = ((QKV, HIDDEN), (HIDDEN, O_IN), (2 * INTER, HIDDEN), (HIDDEN, INTER))
    layers = []
    for layer in range(2):
        row = []
        for i, (n, k) in enumerate(shapes):
            packed = _packed(backend, device, n, k, 7_000_000 + 16 * layer + i)
            row.append((packed, backend.upload_linear(packed, dtype=torch.float16, device=device)))
        layers.append(row)
    return layers


@pytest.mark.parametrize("batch", [1, 8, 32])
def test_config5_chain_stagewise(backend, device, two_layers, batch):
    print(f"case config5-chain batch={batch}", flush=True)
    plans = [[r.prepare_swiglu(tokens=batch) if i == 2 else r.prepare(tokens=batch) for i, (_, r) in enumerate(row)]
             for row in two_layers]
    gen = torch.Generator(device=device).manual_seed(batch)
    h0 = torch.randn(batch, HIDDEN, generator=gen, device=device).half()
    o_in = torch.randn(batch, O_IN, generator=gen, device=device).half()
    h = [h0.clone(), torch.empty_like(h0), torch.empty_like(h0)]
    qkv = [torch.empty(batch, QKV, dtype=torch.float16, device=device) for _ in two_layers]
    o = [torch.empty(batch, HIDDEN, dtype=torch.float16, device=device) for _ in two_layers]
    act = [torch.empty(batch, INTER, dtype=torch.float16, device=device) for _ in two_layers]

    def step():
        h[0].copy_(h0)
        for layer, p in enumerate(plans):
            p[0].run(h[layer], out=qkv[layer])
            p[1].run(o_in, out=o[layer])
            p[2].run(h[layer], out=act[layer])
            p[3].run(act[layer], out=h[layer + 1])

    step()
    torch.cuda.synchronize(device)
    eager = [t.clone() for t in h + qkv + o + act]
    rng = np.random.default_rng(batch)
    for layer, row in enumerate(two_layers):
        stages = (
            (row[0][0], h[layer], qkv[layer], QKV),
            (row[1][0], o_in, o[layer], HIDDEN),
            (row[3][0], act[layer], h[layer + 1], HIDDEN),
        )
        for packed, x, y, n in stages:
            rows = np.sort(rng.choice(n, 64, replace=False))
            codes, scales = _planes(packed, rows)
            want = oracle.q8_linear(bits(x), codes, scales, x.shape[1])
            stats = agreement(bits(y)[:, rows], want)
            assert_free_order(stats)
        cols = np.sort(rng.choice(INTER, 64, replace=False))
        check_swiglu(backend, device, row[2][0], row[2][1], h[layer], act[layer], cols)
    # HIP graph of the step, replayed with eager work between replays.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for i in range(3):
        for t in h[1:] + qkv + o + act:
            t.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize(device)
        for a, b in zip(h + qkv + o + act, eager):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"replay {i}"
        step()
        torch.cuda.synchronize(device)


@pytest.mark.parametrize("passes", [1, 2])
def test_rms_a8_config3_input(backend, device, passes):
    print(f"case rms-a8-config3 passes={passes}", flush=True)
    m, k = 2048, HIDDEN
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(m, k, generator=gen)
    outliers = torch.randperm(k, generator=torch.Generator().manual_seed(3))[:51]
    x[:, outliers] *= 20
    x = x.half()
    gamma = (1 + 0.1 * torch.randn(k, generator=gen)).float()
    norm = backend.upload_rmsnorm(gamma, dtype=torch.float16, device=device, epsilon=1e-6)
    plan = prepare_rms_q8(norm, tokens=m, residual_compensation=passes == 2)
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    inter = torch.empty(m, k, dtype=torch.float16, device=device)
    plan.run(x.to(device), workspace=workspace, intermediate=inter)
    q, d, y = oracle.rms_a8(bits(x), gamma.numpy(), 1e-6, passes)
    np.testing.assert_array_equal(bits(inter), y)
    np.testing.assert_array_equal(workspace.cpu().numpy(), oracle.a8_workspace(q, d))
    # The config-3 QKV projection on this workspace (auto route: matrix cores,
    # natural group order) on sampled rows against the reference-order oracle.
    packed = _packed(backend, device, QKV, k, 33)
    resident = backend.upload_linear(packed, dtype=torch.float16, device=device)
    gemm = prepare_q8_dp4a(resident, tokens=m, residual_compensation=passes == 2)
    out = torch.empty(m, QKV, dtype=torch.float16, device=device)
    gemm.project(out=out, workspace=workspace)
    rows = np.sort(np.random.default_rng(passes).choice(QKV, 48, replace=False))
    codes, scales = _planes(packed, rows)
    want = oracle.a8_linear(q, d, codes, scales, k)
    stats = agreement(bits(out)[:, rows], want)
    assert_free_order(stats)
    print(f"a8 config3 qkv passes={passes}: {stats}", flush=True)
