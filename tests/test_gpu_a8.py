"""A8 path: quantizer bytes, W8A8 projection bytes, RMS and fused RMS+A8."""

import numpy as np
import pytest
import torch

import oracle
from helpers import bits, guarded_out, random_q8
from venturi_amd import Q8RowSplitWeight, prepare_q8_dp4a, prepare_rms_q8

pytestmark = pytest.mark.gpu


def _setup(backend, device, n, k, tokens):
    # Draws as the reference's A8 test (test_q8_dp4a.py:40-50).
    padded = (k + 127) // 128 * 128
    gen = torch.Generator().manual_seed(5821 + k + n + tokens)
    codes = torch.randint(-127, 128, (n, padded), dtype=torch.int8, generator=gen)
    scales = (torch.rand(n, padded // 32, generator=gen) * 0.01).half()
    scales[:, 0] = 0
    x = torch.randn(tokens, k, generator=gen).half()
    resident = backend.upload_linear(Q8RowSplitWeight(codes, scales, k), dtype=torch.float16, device=device)
    return codes, scales, x, resident


@pytest.mark.parametrize("passes", [1, 2])
@pytest.mark.parametrize("tokens", [1, 2, 3, 4, 8, 23, 32])
@pytest.mark.parametrize("shape", [(7, 1), (33, 67), (17, 128), (9, 129), (257, 5120)])
def test_quantizer_and_projection_bytes(backend, device, passes, tokens, shape):
    n, k = shape
    print(f"case a8 n={n} k={k} tokens={tokens} passes={passes}", flush=True)
    codes, scales, x, resident = _setup(backend, device, n, k, tokens)
    plan = prepare_q8_dp4a(resident, tokens=tokens, residual_compensation=passes == 2, route="exact")
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    guard, out = guarded_out(tokens, n, torch.float16, device)
    plan.run(x.to(device), out=out, workspace=workspace)
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    q, d = oracle.a8_quantize(bits(x), passes)
    np.testing.assert_array_equal(workspace.cpu().numpy(), oracle.a8_workspace(q, d))
    expected = oracle.a8_linear(q, d, codes.numpy(), scales.numpy(), k)
    np.testing.assert_array_equal(bits(out), expected)
    assert plan.precision_profile.endswith("-residual-a8") == (passes == 2)


def test_nonfinite_and_zero_propagation(backend, device):
    _, _, x, resident = _setup(backend, device, 16, 128, 1)
    plan = prepare_q8_dp4a(resident, tokens=1, residual_compensation=True)
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    x = x.to(device)
    out = torch.empty(1, 16, dtype=torch.float16, device=device)
    x.fill_(float("inf"))
    plan.run(x, out=out, workspace=workspace)
    assert not torch.isfinite(out).any()
    x.zero_()
    plan.run(x, out=out, workspace=workspace)
    assert not out.any() and not workspace.any()


def test_workspace_guards(backend, device):
    _, _, x, resident = _setup(backend, device, 16, 128, 1)
    plan = prepare_q8_dp4a(resident, tokens=1, residual_compensation=True)
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    x = x.to(device)
    out = torch.empty(1, 16, dtype=torch.float16, device=device)
    with pytest.raises((ValueError, TypeError)):
        plan.run(x, out=out, workspace=workspace[:-1])
    with pytest.raises(ValueError, match="alias"):
        plan.run(x, out=workspace[:32].view(torch.float16).view(1, 16), workspace=workspace)
    unaligned = torch.empty(plan.workspace_bytes + 16, dtype=torch.uint8, device=device)
    with pytest.raises(ValueError, match="16-byte alignment"):
        plan.run(x, out=out, workspace=unaligned[4 : 4 + plan.workspace_bytes])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("k", [1, 31, 67, 1025, 5120])
def test_rms_bytes_and_fp64(backend, device, dtype, k):
    tokens = 5
    g = torch.Generator().manual_seed(17 + k)
    x = torch.randn(tokens, k, generator=g).to(dtype)
    w = 1 + 0.03 * torch.randn(k, generator=g)
    plan = backend.upload_rmsnorm(w, dtype=dtype, device=device, epsilon=1e-6).prepare(tokens=tokens)
    out = torch.empty(tokens, k, dtype=dtype, device=device)
    plan.run(x.to(device), out=out)
    code = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}[dtype]
    if dtype == torch.float32:
        expected = oracle.rms(x.numpy(), w.numpy(), 1e-6, dtype=2)
        np.testing.assert_array_equal(out.cpu().numpy(), expected)
    else:
        expected = oracle.rms(bits(x), w.numpy(), 1e-6, dtype=code)
        np.testing.assert_array_equal(bits(out), expected)
    xd = x.double()
    ideal = (xd * torch.rsqrt(xd.square().mean(-1, keepdim=True) + 1e-6) * w.double()).to(dtype)
    rtol = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2, torch.float32: 1e-5}[dtype]
    torch.testing.assert_close(out.cpu(), ideal, rtol=rtol, atol=2e-6)


@pytest.mark.parametrize("passes", [1, 2])
@pytest.mark.parametrize("tokens", [1, 8, 23])
@pytest.mark.parametrize("k", [1, 31, 33, 67, 1025, 5120, 8704])
def test_fused_rms_a8_bytes(backend, device, passes, tokens, k):
    # Shapes of the reference's fused-producer test (test_rms_quant.py:163-176).
    print(f"case rms-a8 k={k} tokens={tokens} passes={passes}", flush=True)
    g = torch.Generator().manual_seed(17 + tokens + k)
    x = torch.randn(tokens, k, generator=g).half()
    w = 1 + 0.03 * torch.randn(k, generator=g)
    norm = backend.upload_rmsnorm(w, dtype=torch.float16, device=device, epsilon=1e-6)
    plan = prepare_rms_q8(norm, tokens=tokens, residual_compensation=passes == 2)
    storage = torch.full((plan.workspace_bytes + 32,), 71, dtype=torch.uint8, device=device)
    workspace = storage[16:-16]
    inter = torch.empty(tokens, k, dtype=torch.float16, device=device)
    plan.run(x.to(device), workspace=workspace, intermediate=inter)
    s = storage.cpu()
    assert bool((s[:16] == 71).all()) and bool((s[-16:] == 71).all())
    q, d, y = oracle.rms_a8(bits(x), w.numpy(), 1e-6, passes)
    np.testing.assert_array_equal(bits(inter), y)
    np.testing.assert_array_equal(workspace.cpu().numpy(), oracle.a8_workspace(q, d))
    # Fused == RMSNorm then the plain quantizer on the same device.
    y_dev = torch.empty(tokens, k, dtype=torch.float16, device=device)
    norm.prepare(tokens=tokens).run(x.to(device), out=y_dev)
    assert torch.equal(y_dev, inter)
    lib = backend._native
    separate = torch.empty_like(workspace)
    backend._check(lib.venturi_q8_dp4a_quantize(y_dev.data_ptr(), separate.data_ptr(), separate.numel(), tokens, k,
                                                 passes, torch.cuda.current_stream().cuda_stream))
    assert torch.equal(separate, workspace)


@pytest.mark.parametrize("passes", [1, 2])
@pytest.mark.parametrize("tokens", [64, 65, 100, 257])
@pytest.mark.parametrize("shape", [(7, 1), (33, 67), (129, 1000), (70, 2000), (64, 5120), (100, 6144), (40, 26000)])
def test_matrix_core_projection_bytes(backend, device, passes, tokens, shape):
    # Token counts that take the int8 matrix-core GEMM: bytes must still be the reference's.
    n, k = shape
    print(f"case a8-gemm n={n} k={k} tokens={tokens} passes={passes}", flush=True)
    codes, scales, x, resident = _setup(backend, device, n, k, tokens)
    plan = prepare_q8_dp4a(resident, tokens=tokens, residual_compensation=passes == 2, route="exact")
    assert plan.route == "venturi-q8-a8"
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    guard, out = guarded_out(tokens, n, torch.float16, device)
    plan.run(x.to(device), out=out, workspace=workspace)
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    q, d = oracle.a8_quantize(bits(x), passes)
    np.testing.assert_array_equal(bits(out), oracle.a8_linear(q, d, codes.numpy(), scales.numpy(), k))


@pytest.mark.parametrize("n,k", [(7168, 5120), (5120, 6144), (34816, 5120), (5120, 17408)])
def test_config3_prefill_sampled(backend, device, n, k):
    # Config-3 shapes at 2048 tokens; the oracle checks a seeded sample
    # of 64 tokens x 128 rows (every output's order is independent of the others).
    tokens = 2048
    gen = torch.Generator(device=device).manual_seed(n ^ k)
    packed = backend.quantize_q8(torch.randn(n, k, generator=gen, device=device) * 0.02)
    x = torch.randn(tokens, k, generator=gen, device=device).half()
    resident = backend.upload_linear(packed, dtype=torch.float16, device=device)
    rng = np.random.default_rng(n + k)
    ts = np.sort(rng.choice(tokens, 64, replace=False))
    rows = np.sort(rng.choice(n, 128, replace=False))
    q, d = oracle.a8_quantize(bits(x[ts]), 1)
    wc, ws = packed.codes.cpu().numpy()[rows], packed.scales.cpu().numpy()[rows]
    expected = oracle.a8_linear(q, d, wc, ws, k)
    for route in ("exact", "mfma"):
        plan = prepare_q8_dp4a(resident, tokens=tokens, residual_compensation=False, route=route)
        workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
        out = torch.empty(tokens, n, dtype=torch.float16, device=device)
        plan.run(x, out=out, workspace=workspace)
        got = bits(out)[ts][:, rows]
        if route == "exact":
            np.testing.assert_array_equal(got, expected)
        else:
            flips = check_a8_tolerance(got, q, d, wc, ws, k, expected)
            print(f"config3 n={n} k={k} mfma: {flips} of {got.size} differ from the reference order", flush=True)


def ulp16(v):
    v = np.abs(v)
    return 2.0 ** (np.floor(np.log2(np.maximum(v, 2.0**-14))) - 10)


def check_a8_tolerance(got_bits, q, d, wcodes, wscales, k, expected_bits):
    """The mfma route against FP64 over the exact group dots and against the reference order.

    FP64: y = sum_p sum_g dot_pg * fp32(ws_g * as_pg), the reference's per-group
    terms; the fp32 natural-order sum may differ from it by at most
    G * 2^-24 * sum|terms| plus the final fp16 rounding (half an ulp).
    Reference order: every output within max(2e-3, 1 fp16 ulp) and rel-L2 <= 1e-3
    (the stated tolerance for fp16 outputs).
    """
    got = got_bits.view(np.float16).astype(np.float64)
    passes, groups = q.shape[0], q.shape[2]
    ws32 = wscales.astype(np.float32)[:, :groups]
    y = np.zeros(got.shape)
    mag = np.zeros(got.shape)
    for p in range(passes):
        dots = oracle.a8_group_dots(q[p : p + 1], wcodes, k).astype(np.float64)  # [T, N, G]
        prod = (ws32[None, :, :] * d[p][:, None, :]).astype(np.float64)  # fp32 products, as the reference
        terms = dots * prod
        y += terms.sum(-1)
        mag += np.abs(terms).sum(-1)
    bound = 0.5 * ulp16(y) + passes * groups * 2.0**-24 * mag
    assert (np.abs(got - y) <= bound).all()
    ref = expected_bits.view(np.float16).astype(np.float64)
    diff = np.abs(got - ref)
    assert (diff <= np.maximum(2e-3, ulp16(ref))).all()
    assert np.linalg.norm(got - ref) <= 1e-3 * max(np.linalg.norm(ref), 1e-12)
    return int((diff > 0).sum())


@pytest.mark.parametrize("passes", [1, 2])
@pytest.mark.parametrize("tokens", [1, 64, 65, 257])
@pytest.mark.parametrize("shape", [(7, 1), (33, 67), (129, 1000), (70, 2000), (64, 5120), (300, 520), (40, 26000)])
def test_mfma_route_tolerance(backend, device, passes, tokens, shape):
    n, k = shape
    print(f"case a8-mfma n={n} k={k} tokens={tokens} passes={passes}", flush=True)
    codes, scales, x, resident = _setup(backend, device, n, k, tokens)
    plan = prepare_q8_dp4a(resident, tokens=tokens, residual_compensation=passes == 2, route="mfma")
    assert plan.route == "venturi-q8-a8-mfma"
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


@pytest.mark.parametrize("k", [32, 96, 200])
def test_mfma_route_exact_group_dots(backend, device, k):
    # Unit scales, weight codes in [-2, 2] and two nonzero activations per group
    # (127, which makes the activation scale exactly 1, and one in [-2, 2]) keep
    # every output an integer below 2048, so fp32 sums in any order and the fp16
    # rounding are exact: any error in a group dot (a wrong lane, column or
    # code) changes the bytes.
    tokens, n = 130, 48
    padded = (k + 127) // 128 * 128
    gen = torch.Generator().manual_seed(900 + k)
    codes = torch.randint(-2, 3, (n, padded), dtype=torch.int8, generator=gen)
    scales = torch.ones(n, padded // 32, dtype=torch.float16)
    x = torch.zeros(tokens, k)
    groups = (k + 31) // 32
    for t in range(tokens):
        for gi in range(groups):
            width = min(32, k - 32 * gi)
            x[t, 32 * gi + int(torch.randint(width, (1,), generator=gen))] = 127.0  # activation scale exactly 1
            col = 32 * gi + int(torch.randint(width, (1,), generator=gen))
            x[t, col] += float(torch.randint(-2, 3, (1,), generator=gen)) if x[t, col] == 0 else 0.0
    x = x.half()
    resident = backend.upload_linear(Q8RowSplitWeight(codes, scales, k), dtype=torch.float16, device=device)
    plan = prepare_q8_dp4a(resident, tokens=tokens, residual_compensation=False, route="mfma")
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    plan.run(x.to(device), out=out, workspace=workspace)
    q, d = oracle.a8_quantize(bits(x), 1)
    assert (d == 1.0).all()
    dots = oracle.a8_group_dots(q, codes.numpy(), k).astype(np.int64).sum(-1)
    assert (np.abs(dots) < 2048).all()
    np.testing.assert_array_equal(out.cpu().float().numpy(), dots.astype(np.float32))
    np.testing.assert_array_equal(bits(out), oracle.a8_linear(q, d, codes.numpy(), scales.numpy(), k))
