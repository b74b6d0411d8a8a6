"""Q4 (q4_g64_fp16) kernels on the GPU against the CPU oracle.

Bit-exact: the fp16 decode (venturi_q4_decode, venturi_row_dequant_rows), the
expert GEMV (venturi_q4_linear, flash_next_q4.cu:23-34), the plugin GEMV
(venturi_q4_run, q4_linear.cu:21-56) and the research fused GEMV
(venturi_q4_fused_run, q4_fused.cuh:10-89), each in the reference's order.

Tolerance (matrix-core W4A16 route, whose fp32 association is its own):
  * vs FP64 of the fp16 weights fp16(q*scale): |y - exact| <= 0.5 ulp_fp16(exact)
    + 2^-19 * sum_k |x_k w_k|
  * vs the expert-order oracle: every output within max(2e-3, 1 fp16 ulp),
    rel-L2 <= 1e-3; 1-ulp flips are reported.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import bits, near_tie_matrix
from venturi_amd import Q4RowSplitWeight

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (3, 63), (5, 64), (37, 129), (64, 2048), (130, 768), (8, 4097)]


def ulp16(v):
    v = np.abs(v)
    e = np.floor(np.log2(np.maximum(v, 2.0**-14)))
    return 2.0 ** (e - 10)


def random_q4(n, k, seed, scale=0.004):
    gen = torch.Generator().manual_seed(seed)
    codes = torch.randint(-8, 8, (n, k), dtype=torch.int8, generator=gen)
    scales = (torch.rand(n, (k + 63) // 64, generator=gen) * scale).half()
    return Q4RowSplitWeight.from_codes(codes, scales)


def planes(weight):
    return weight.codes.numpy(), weight.scales.numpy()


def test_known_bytes_decode_on_device(backend, device):
    """tests/test_q4_weights.py:30-44 bytes, through the device decoders."""
    codes = torch.zeros((1, 64), dtype=torch.uint8)
    codes[0, :3] = torch.tensor([0x10, 0xF8, 0x97], dtype=torch.uint8)
    scales = torch.tensor([[0.5, -2]], dtype=torch.float16)
    lib = backend._native
    c, s = codes.to(device), scales.to(device)
    out = torch.full((1, 128), 9, dtype=torch.float16, device=device)
    assert lib.venturi_q4_decode(c.data_ptr(), s.data_ptr(), out.data_ptr(), 1, 128, 128, None) == 0
    torch.cuda.synchronize()
    assert out[0, :6].tolist() == [0, 0.5, -4, -0.5, 3.5, -3.5]
    again = torch.full((1, 128), 9, dtype=torch.float16, device=device)
    backend._check(lib.venturi_row_dequant_rows(c.data_ptr(), None, s.data_ptr(), again.data_ptr(), 0, 1, 128, 128, 4, None))
    torch.cuda.synchronize()
    assert torch.equal(out, again)


@pytest.mark.parametrize("shape", SHAPES)
def test_decode_bytes(backend, device, shape):
    n, k = shape
    print(f"case q4-decode n={n} k={k}", flush=True)
    w = random_q4(n, k, 11 + n + k)
    codes, scales = planes(w)
    expect = oracle.q4_decode_fp16(codes, scales, k).view(np.uint16)
    assert np.array_equal(expect, oracle.q4_decode(codes, scales, k))
    resident = backend.upload_linear(w, dtype=torch.float16, device=device)._payload
    out = torch.empty((n, k), dtype=torch.float16, device=device)
    resident.decode(out=out)
    assert np.array_equal(bits(out), expect)
    if n > 2:  # a row window through venturi_row_dequant_rows
        part = torch.empty((n - 2, k), dtype=torch.float16, device=device)
        resident.decode(out=part, row=1)
        assert np.array_equal(bits(part), expect[1 : n - 1])


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("tokens", [1, 2, 5, 64])
def test_exact_expert_gemv_bytes(backend, device, shape, tokens):
    n, k = shape
    print(f"case q4-exact n={n} k={k} tokens={tokens}", flush=True)
    w = random_q4(n, k, 100 + n + tokens)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens + k)).half()
    plan = backend.upload_linear(w, dtype=torch.float16, device=device).prepare(tokens=tokens, route="exact")
    guard = torch.full((tokens * n + 2,), 47, dtype=torch.float16, device=device)
    out = guard[1:-1].view(tokens, n)
    plan.run(x.to(device), out=out)
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    codes, scales = planes(w)
    assert np.array_equal(bits(out), oracle.q4_linear(bits(x), codes, scales, k))


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("tokens", [1, 4, 7])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_generic_plugin_gemv_bytes(backend, device, shape, tokens, dtype):
    from venturi_amd.ada import AdaBackend

    n, k = shape
    print(f"case q4-generic n={n} k={k} tokens={tokens} {dtype}", flush=True)
    w = random_q4(n, k, 200 + n + tokens)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(3 * tokens + k)).to(dtype)
    ada = AdaBackend()
    plan = ada.upload_linear(w, device=device).prepare(tokens=tokens, dtype=dtype)
    assert plan.route == "generic-simt"
    out = plan.empty_output()
    plan.run(x.to(device), out=out)
    codes, scales = planes(w)
    expect = oracle.q4_generic(bits(x), codes, scales, k, int(dtype == torch.bfloat16))
    assert np.array_equal(bits(out), expect)
    # The same kernel through the backend's plan.
    plan2 = backend.upload_linear(w, dtype=dtype, device=device).prepare(tokens=tokens, route="generic")
    out2 = torch.empty_like(out)
    plan2.run(x.to(device), out=out2)
    assert np.array_equal(bits(out2), expect)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("tokens", [1, 3])
def test_research_fused_gemv_bytes(backend, device, shape, tokens):
    n, k = shape
    print(f"case q4-fused n={n} k={k} tokens={tokens}", flush=True)
    w = random_q4(n, k, 300 + n + tokens)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(5 * tokens + k)).half()
    plan = backend.upload_linear(w, dtype=torch.float16, device=device).prepare(tokens=tokens, route="fused")
    out = torch.empty((tokens, n), dtype=torch.float16, device=device)
    plan.run(x.to(device), out=out)
    codes, scales = planes(w)
    assert np.array_equal(bits(out), oracle.q4_fused(bits(x), codes, scales, k))


@pytest.mark.parametrize("shape", [(1, 8), (5, 64), (37, 136), (64, 2048), (130, 768), (300, 4096), (1536, 2048)])
@pytest.mark.parametrize("tokens", [1, 3, 16, 33, 64, 65, 130])
def test_mfma_w4a16_tolerances(backend, device, shape, tokens):
    n, k = shape
    print(f"case q4-mfma n={n} k={k} tokens={tokens}", flush=True)
    w = random_q4(n, k, 400 + n + tokens, scale=0.02)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(7 * tokens + k)).half()
    plan = backend.upload_linear(w, dtype=torch.float16, device=device).prepare(tokens=tokens)
    assert plan.route == "venturi-q4-mfma"
    guard = torch.full((tokens * n + 2,), 47, dtype=torch.float16, device=device)
    out = guard[1:-1].view(tokens, n)
    plan.run(x.to(device), out=out)
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    codes, scales = planes(w)
    wd = oracle.q4_decode_fp16(codes, scales, k).astype(np.float64)
    xd = x.float().numpy().astype(np.float64)
    exact = xd @ wd.T
    got = out.cpu().float().numpy().astype(np.float64)
    bound = 0.5 * ulp16(exact) + 2.0**-19 * (np.abs(xd) @ np.abs(wd).T)
    assert (np.abs(got - exact) <= bound).all()
    if tokens <= 64:
        ref = oracle.q4_linear(bits(x), codes, scales, k).view(np.float16).astype(np.float64)
        diff = np.abs(got - ref)
        assert (diff <= np.maximum(2e-3, ulp16(ref))).all()
        assert np.linalg.norm(got - ref) <= 1e-3 * max(np.linalg.norm(ref), 1e-12)
        print(f"flips={int((diff > 0).sum())} of {tokens * n}", flush=True)


@pytest.mark.parametrize("shape", [(1, 8), (37, 136), (300, 2048), (6200, 264), (16400, 136)])
@pytest.mark.parametrize("tokens", [1, 5, 16, 24, 31])
def test_tiled_decode_equals_row_major(backend, device, shape, tokens):
    # Decode plans read the resident's tiled copy; the arithmetic and its order
    # are those of venturi_q4_gemm_run on the row-major planes, so the bits match.
    n, k = shape
    print(f"case q4-tiled n={n} k={k} tokens={tokens}", flush=True)
    w = random_q4(n, k, 900 + n + tokens, scale=0.02)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens + 3 * k)).half().to(device)
    resident = backend.upload_linear(w, dtype=torch.float16, device=device)
    plan = resident.prepare(tokens=tokens)
    assert plan.route == "venturi-q4-mfma"
    guard = torch.full((tokens * n + 2,), 47, dtype=torch.float16, device=device)
    out = guard[1:-1].view(tokens, n)
    plan.run(x, out=out)
    want = torch.empty(tokens, n, dtype=torch.float16, device=device)
    dw = resident._payload.weight
    backend._check(backend._native.venturi_q4_gemm_run(
        x.data_ptr(), dw.codes.data_ptr(), dw.scales.data_ptr(), want.data_ptr(), tokens, n, k, dw.padded_k, 0,
        torch.cuda.current_stream(device).cuda_stream))
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


def test_tiled_decode_rejects_bad_arguments(backend, device):
    lib = backend._native
    resident = backend.upload_linear(random_q4(16, 128, 5), dtype=torch.float16, device=device)
    resident.prepare(tokens=1)
    tc, ts = resident._payload.tiled
    x = torch.zeros(32, 128, dtype=torch.float16, device=device)
    o = torch.empty(32, 16, dtype=torch.float16, device=device)
    s = torch.cuda.current_stream(device).cuda_stream
    args = (x.data_ptr(), tc.data_ptr(), ts.data_ptr(), o.data_ptr())
    assert lib.venturi_q4_tiled_run(*args, 32, 16, 128, 128, 0, None, 0, s) == -1
    assert "1 to 31 tokens" in lib.error()
    assert lib.venturi_q4_tiled_run(*args, 1, 16, 128, 128, 1, None, 0, s) == -1
    assert "FP16" in lib.error()
    assert lib.venturi_q4_tiled_run(x.data_ptr(), None, ts.data_ptr(), o.data_ptr(), 1, 16, 128, 128, 0, None, 0, s) == -1
    assert lib.venturi_q4_tiled_run(*args, 1, 16, 128, 256, 0, None, 0, s) == -1
    # A shape that splits K (<= 384 row blocks, >= 64 chunks) refuses to run without its slots.
    assert lib.venturi_q4_tiled_workspace_bytes(3, 16, 8192) == 3 * 1 * 8 * 8
    assert lib.venturi_q4_tiled_workspace_bytes(3, 16, 8064) == 0  # 63 chunks: unsplit
    assert lib.venturi_q4_tiled_workspace_bytes(17, 16, 8192) == 0  # two token blocks: unsplit
    assert lib.venturi_q4_tiled_workspace_bytes(3, 6160, 8192) == 0  # 385 row blocks: unsplit
    assert lib.venturi_q4_tiled_run(*args, 1, 16, 8192, 8192, 0, None, 0, s) == -1
    assert "slot buffer" in lib.error()
    torch.cuda.synchronize(device)


@pytest.mark.parametrize("shape", [(16, 8192), (130, 8320), (37, 8200), (5120, 17408)])
@pytest.mark.parametrize("tokens", [1, 3, 16])
def test_tiled_decode_split_k(backend, device, shape, tokens):
    # Shapes that split K over two workgroups: the two halves meet in fp32 (an
    # order-free add), so outputs are deterministic and graph replays agree; the
    # W4A16 contract bound against FP64 holds, and the plan's slots end idle.
    n, k = shape
    print(f"case q4-tiled-split n={n} k={k} tokens={tokens}", flush=True)
    w = random_q4(n, k, 300 + n + tokens, scale=0.02)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(5 * tokens + k)).half()
    resident = backend.upload_linear(w, dtype=torch.float16, device=device)
    plan = resident.prepare(tokens=tokens)
    slots = plan._plan.slots if hasattr(plan, "_plan") else plan.slots
    assert slots is not None and slots.numel() == tokens * ((n + 15) // 16) * 64
    idle = slots.clone()
    xd_dev = x.to(device)
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    plan.run(xd_dev, out=out)
    again = torch.empty_like(out)
    plan.run(xd_dev, out=again)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    assert torch.equal(slots, idle)
    graph_out = torch.empty_like(out)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        plan.run(xd_dev, out=graph_out)
    for _ in range(3):
        graph_out.fill_(0)
        g.replay()
        torch.cuda.synchronize(device)
        assert torch.equal(graph_out.view(torch.int16), out.view(torch.int16))
    codes, scales = planes(w)
    wd = oracle.q4_decode_fp16(codes, scales, k).astype(np.float64)
    xd = x.float().numpy().astype(np.float64)
    exact = xd @ wd.T
    got = out.cpu().float().numpy().astype(np.float64)
    bound = 0.5 * ulp16(exact) + 2.0**-19 * (np.abs(xd) @ np.abs(wd).T)
    assert (np.abs(got - exact) <= bound).all()


def test_expert_abi_objects(device):
    """NativeQ4 (ops/flash_next_q4.py:17-89): prepare / linear / decode."""
    from venturi_amd.q4 import NativeQ4

    q4 = NativeQ4()
    w = random_q4(48, 200, 5)
    prepared = q4.prepare(w, device=device)
    x = torch.randn(3, 200, generator=torch.Generator().manual_seed(1)).half()
    y = q4.linear(x.to(device), prepared)
    codes, scales = planes(w)
    assert np.array_equal(bits(y), oracle.q4_linear(bits(x), codes, scales, 200))
    assert np.array_equal(bits(q4.decode(prepared)), oracle.q4_decode_fp16(codes, scales, 200).view(np.uint16))
    with pytest.raises(ValueError):
        q4.linear(torch.zeros(65, 200, dtype=torch.float16, device=device), prepared)


def test_status_codes_and_plugin_errors(backend, device):
    lib = backend._native
    # Expert ABI returns the HIP error code (hipErrorInvalidValue = 1).
    assert lib.venturi_q4_linear(None, None, None, None, 1, 1, 1, 128, None) == 1
    assert lib.venturi_q4_decode(None, None, None, 1, 1, 100, None) == 1
    assert lib.venturi_q4_prepare(1, 1, 1, 0, 0) == 0
    assert lib.venturi_q4_prepare(1, 1, 1, 2, 0) == -1
    assert b"invalid" in lib.venturi_ada_error()
    assert lib.venturi_q4_run(None, None, None, None, 1, 1, 128, 1, 0, 1, None) == -1
    assert lib.venturi_q4_gemm_run(None, None, None, None, 1, 1, 1, 128, 0, None) == -1
    assert "null" in backend._native.error()


@pytest.mark.parametrize("k", [1, 63, 64, 65, 129, 136, 2048, 4097])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_device_q4_pack_equals_rtn(backend, device, k, dtype):
    """venturi_q4_pack_run == quantize_q4_rtn (flash_next_q4.py:26-52) byte for byte."""
    from venturi_amd import quantize_q4_rtn

    print(f"case q4-pack k={k} {dtype}", flush=True)
    gen = torch.Generator().manual_seed(k)
    w = (torch.randn(37, k, generator=gen) * 0.02).to(dtype)
    w[0] = 0  # all-zero row: scale floor 2^-24, codes 0
    if k >= 6:
        w[1, :6] = torch.tensor([7.0, 0.5, 1.5, 2.5, -0.5, -1.5]).to(dtype)  # ties
    ref = quantize_q4_rtn(w)
    got = backend.quantize_q4(w.to(device))
    assert torch.equal(got.codes.cpu(), ref.codes)
    assert torch.equal(got.scales.cpu().view(torch.int16), ref.scales.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("trim", [0, 5])
def test_device_q4_pack_near_ties(backend, device, dtype, trim):
    # Quotients x / scale on and within three fp32 ulps of half-integers, under
    # normal and subnormal fp16 scales: the packer's reciprocal estimate leaves
    # these to the IEEE division, and the codes equal quantize_q4_rtn's.
    from venturi_amd import quantize_q4_rtn

    print(f"case q4-pack-ties {dtype} trim={trim}", flush=True)
    w = torch.from_numpy(near_tie_matrix(7, 64, 64, 4, 29 + trim))[:, : 256 - trim].contiguous().to(dtype)
    ref = quantize_q4_rtn(w)
    got = backend.quantize_q4(w.to(device))
    assert torch.equal(got.codes.cpu(), ref.codes)
    assert torch.equal(got.scales.cpu().view(torch.int16), ref.scales.view(torch.int16))
