"""The int8 matrix-core A8 decode kernel (venturi_q8_a8_tiled_run, the A8
"mfma" and "auto" route at 1..32 tokens) against the oracle.

* Group dots are exact: with unit scales and sparse integer activations every
  group term is an integer and their fp32 sum is exact, so the bytes must equal
  fp16 of the brute-force integer dots (a wrong lane, column, group or code
  changes them).
* Random data: within the FP64 bound over the exact group dots and the
  reference's fp32 products, and within the stated fp16 tolerance of the
  reference-order oracle (check_a8_tolerance), for one and two passes, odd
  shapes (k not a multiple of 64 or 128, n not a multiple of 16), one and
  two token blocks, and the config-2 shapes on sampled rows.
* The plan picks the kernel: auto and mfma take it up to 32 tokens; run()
  quantizes inside the projection kernel where the activations fit (up to 16
  tokens, k % 8 == 0, x 16-byte aligned, 64 KB of LDS) and equals the separate
  quantize + project steps byte for byte, fused or not.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import bits, guarded_out
from test_gpu_a8 import _setup, check_a8_tolerance
from venturi_amd import Q8RowSplitWeight, prepare_q8_dp4a

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("passes", [1, 2])
@pytest.mark.parametrize("tokens", [1, 2, 3, 8, 13, 16, 17, 31, 32])
@pytest.mark.parametrize("shape", [(7, 1), (33, 67), (129, 1000), (70, 2000), (64, 5120), (300, 520), (40, 26000)])
def test_tiled_a8_tolerance(backend, device, passes, tokens, shape):
    n, k = shape
    print(f"case a8-tiled n={n} k={k} tokens={tokens} passes={passes}", flush=True)
    codes, scales, x, resident = _setup(backend, device, n, k, tokens)
    for route in ("auto", "mfma"):
        plan = prepare_q8_dp4a(resident, tokens=tokens, residual_compensation=passes == 2, route=route)
        assert plan.kernel == "tiled" and plan.route == "venturi-q8-a8-mfma"
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    guard, out = guarded_out(tokens, n, torch.float16, device)
    plan.run(x.to(device), out=out, workspace=workspace)
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    q, d = oracle.a8_quantize(bits(x), passes)
    np.testing.assert_array_equal(workspace.cpu().numpy(), oracle.a8_workspace(q, d))
    expected = oracle.a8_linear(q, d, codes.numpy(), scales.numpy(), k)
    flips = check_a8_tolerance(bits(out), q, d, codes.numpy(), scales.numpy(), k, expected)
    print(f"flips={flips} of {tokens * n}", flush=True)
    again = torch.empty_like(out)
    plan.run(x.to(device), out=again, workspace=workspace)
    assert torch.equal(again.view(torch.int16), out.view(torch.int16))  # deterministic
    # run() quantizes inside the projection where the activations fit; the two
    # separate steps give the same workspace and output bytes.
    split_ws = torch.full_like(workspace, 0x5A)
    split = torch.empty_like(out)
    plan.quantize(x.to(device), workspace=split_ws)
    plan.project(out=split, workspace=split_ws)
    assert torch.equal(split_ws, workspace)
    assert torch.equal(split.view(torch.int16), out.view(torch.int16))


@pytest.mark.parametrize("tokens", [1, 5, 16])
def test_tiled_a8_unaligned_input(backend, device, tokens):
    # x at a 2-byte offset takes the two-launch form: same bytes as the fused one.
    n, k = 100, 1024
    codes, scales, x, resident = _setup(backend, device, n, k, tokens)
    plan = prepare_q8_dp4a(resident, tokens=tokens, residual_compensation=False)
    base = torch.empty(tokens * k + 8, dtype=torch.float16, device=device)
    shifted = base[1 : 1 + tokens * k].view(tokens, k)
    shifted.copy_(x.to(device))
    aligned = x.to(device)
    assert shifted.data_ptr() % 16 and aligned.data_ptr() % 16 == 0
    outs, spaces = [], []
    for source in (aligned, shifted):
        ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
        out = torch.empty(tokens, n, dtype=torch.float16, device=device)
        plan.run(source, out=out, workspace=ws)
        outs.append(out)
        spaces.append(ws)
    assert torch.equal(spaces[0], spaces[1])
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    q, d = oracle.a8_quantize(bits(x), 1)
    np.testing.assert_array_equal(spaces[0].cpu().numpy(), oracle.a8_workspace(q, d))
    check_a8_tolerance(bits(outs[0]), q, d, codes.numpy(), scales.numpy(), k,
                       oracle.a8_linear(q, d, codes.numpy(), scales.numpy(), k))


def test_tiled_a8_nonfinite(backend, device):
    # A group with a non-finite value: zero codes, NaN scale, NaN outputs for that token only.
    n, k, tokens = 48, 256, 3
    _, _, x, resident = _setup(backend, device, n, k, tokens)
    x[1, 40] = float("inf")
    plan = prepare_q8_dp4a(resident, tokens=tokens, residual_compensation=True)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    plan.run(x.to(device), out=out, workspace=ws)
    q, d = oracle.a8_quantize(bits(x), 2)
    np.testing.assert_array_equal(ws.cpu().numpy(), oracle.a8_workspace(q, d))
    o = out.cpu()
    assert torch.isnan(o[1]).all() and torch.isfinite(o[0]).all() and torch.isfinite(o[2]).all()


@pytest.mark.parametrize("tokens", [1, 5, 16, 32])
@pytest.mark.parametrize("k", [32, 96, 200, 1000])
def test_tiled_a8_exact_group_dots(backend, device, tokens, k):
    # Unit weight scales, weight codes in [-2, 2] (padding included), and per
    # group one activation of 127 (activation scale exactly 1) and at most one
    # more in [-2, 2]: every term is an integer below 2^9 and the fp32 sum of at
    # most 32 of them is exact.
    n = 40
    padded = (k + 127) // 128 * 128
    gen = torch.Generator().manual_seed(700 + k + tokens)
    codes = torch.randint(-2, 3, (n, padded), dtype=torch.int8, generator=gen)
    scales = torch.ones(n, padded // 32, dtype=torch.float16)
    x = torch.zeros(tokens, k)
    groups = (k + 31) // 32
    for t in range(tokens):
        for gi in range(groups):
            width = min(32, k - 32 * gi)
            x[t, 32 * gi + int(torch.randint(width, (1,), generator=gen))] = 127.0
            col = 32 * gi + int(torch.randint(width, (1,), generator=gen))
            x[t, col] += float(torch.randint(-2, 3, (1,), generator=gen)) if x[t, col] == 0 else 0.0
    x = x.half()
    resident = backend.upload_linear(Q8RowSplitWeight(codes, scales, k), dtype=torch.float16, device=device)
    plan = prepare_q8_dp4a(resident, tokens=tokens, residual_compensation=False)
    assert plan.kernel == "tiled"
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    plan.run(x.to(device), out=out, workspace=workspace)
    q, d = oracle.a8_quantize(bits(x), 1)
    assert (d == 1.0).all()
    dots = oracle.a8_group_dots(q, codes.numpy(), k).astype(np.int64).sum(-1)
    assert (np.abs(dots) < 2**14).all()
    np.testing.assert_array_equal(bits(out), dots.astype(np.float32).astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("passes", [1, 2])
@pytest.mark.parametrize("tokens", [1, 8, 32])
@pytest.mark.parametrize("n,k", [(7168, 5120), (5120, 6144), (34816, 5120), (5120, 17408)])
def test_tiled_a8_config2_sampled(backend, device, passes, tokens, n, k):
    # The bench's A8 decode shapes; the oracle checks a seeded sample of 96 rows.
    print(f"case a8-tiled-config2 n={n} k={k} tokens={tokens} passes={passes}", flush=True)
    gen = torch.Generator(device=device).manual_seed(n + k + tokens)
    packed = backend.quantize_q8(torch.randn(n, k, generator=gen, device=device) * 0.02)
    x = torch.randn(tokens, k, generator=gen, device=device).half()
    resident = backend.upload_linear(packed, dtype=torch.float16, device=device)
    plan = prepare_q8_dp4a(resident, tokens=tokens, residual_compensation=passes == 2)
    assert plan.kernel == "tiled"
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    plan.run(x, out=out, workspace=workspace)
    rows = np.sort(np.random.default_rng(n + k).choice(n, 96, replace=False))
    q, d = oracle.a8_quantize(bits(x), passes)
    wc, ws = packed.codes.cpu().numpy()[rows], packed.scales.cpu().numpy()[rows]
    expected = oracle.a8_linear(q, d, wc, ws, k)
    flips = check_a8_tolerance(bits(out)[:, rows], q, d, wc, ws, k, expected)
    print(f"flips={flips} of {expected.size}", flush=True)


def test_tiled_a8_rejections(backend, device):
    lib = backend._native
    s = torch.cuda.current_stream(device).cuda_stream
    ws = torch.empty(4096, dtype=torch.uint8, device=device)
    planes = torch.empty(4096, dtype=torch.uint8, device=device)
    out = torch.empty(64, dtype=torch.float16, device=device)
    args = (ws.data_ptr(), ws.numel(), planes.data_ptr(), planes.data_ptr(), out.data_ptr())
    no_slots = (None, 0, s)
    assert lib.venturi_q8_a8_tiled_run(*args, 33, 1, 32, 128, 1, *no_slots) == -1
    assert "1..32 tokens" in lib.error()
    assert lib.venturi_q8_a8_tiled_run(*args, 1, 16, 64, 64, 1, *no_slots) == -1
    assert "geometry" in lib.error()
    assert lib.venturi_q8_a8_tiled_run(*args, 1, 16, 64, 128, 3, *no_slots) == -1
    assert lib.venturi_q8_a8_tiled_run(ws.data_ptr() + 4, ws.numel() - 4, *args[2:], 1, 16, 64, 128, 1, *no_slots) == -1
    assert "misaligned" in lib.error()
    assert lib.venturi_q8_a8_tiled_run(ws.data_ptr(), 8, *args[2:], 1, 16, 64, 128, 1, *no_slots) == -1
    assert "workspace" in lib.error()
    # A shape whose launch splits K refuses to run without its slots.
    n, k, tokens = 5120, 17408, 8
    assert lib.venturi_q8_a8_tiled_workspace_bytes(tokens, n, k, 2) == tokens * (n // 16) * 64
    need = int(lib.venturi_q8_a8_tiled_workspace_bytes(tokens, n, k, 2))
    big_ws = torch.empty(int(lib.venturi_q8_dp4a_bytes(tokens, k, 2)), dtype=torch.uint8, device=device)
    big_planes = torch.empty(n * k + 64, dtype=torch.uint8, device=device)
    big_out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    assert lib.venturi_q8_a8_tiled_run(big_ws.data_ptr(), big_ws.numel(), big_planes.data_ptr(), big_planes.data_ptr(),
                                       big_out.data_ptr(), tokens, n, k, k, 2, None, 0, s) == -1
    assert "slot buffer" in lib.error()
    slots = torch.empty(need, dtype=torch.uint8, device=device)
    assert lib.venturi_q8_a8_tiled_run(big_ws.data_ptr(), big_ws.numel(), big_planes.data_ptr(), big_planes.data_ptr(),
                                       big_out.data_ptr(), tokens, n, k, k, 2, slots.data_ptr(), need - 8, s) == -1
    assert "slot buffer" in lib.error()
    torch.cuda.synchronize(device)
