"""The native plan table's per-matrix projection on the device: each path's
output has the bytes of the entry point it dispatches to (those entry points
are checked against the oracle in their own tests)."""

import numpy as np
import pytest
import torch

import oracle
from helpers import bits, random_q8
from venturi_amd.rowcodec import prepare_row_codec

pytestmark = pytest.mark.gpu


def _row_planes(n, k, nbits, seed):
    padded = (k + 127) // 128 * 128
    rng = np.random.default_rng(seed)
    codes = rng.integers(-(1 << (nbits - 1)), 1 << (nbits - 1), size=(n, padded))
    codes[:, k:] = 0
    scales = (rng.random((n, padded // 64)) * 0.02).astype(np.float16)
    return oracle.pack_row_codec(codes, scales, nbits)


def _dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("tokens", [1, 7, 16, 40, 300])
@pytest.mark.parametrize("k", [64, 200, 1000])
def test_q8_a16_plan(backend, device, dtype, tokens, k):
    n = 70
    codes, scales = random_q8(n, k, 5 + tokens + k)
    plan = prepare_row_codec(8, 32, dtype=dtype)
    tdt = torch.float16 if dtype == 0 else torch.bfloat16
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(k)).to(tdt).to(device)
    dc, ds = codes.to(device), scales.to(device)
    out = torch.empty(tokens, n, dtype=tdt, device=device)
    s = torch.cuda.current_stream(device).cuda_stream
    padded = codes.shape[1]
    plan.project(x.data_ptr(), dc.data_ptr(), None, ds.data_ptr(), out.data_ptr(), None, 0, tokens=tokens, n=n, k=k,
                 padded=padded, stream=s)
    want = torch.empty_like(out)
    lib = backend._native
    if tokens <= 32:
        # Direct up to 32 tokens: the reference's canonical bytes.
        expected = oracle.q8_linear(bits(x), codes.numpy(), scales.numpy(), k, dtype=dtype)
        np.testing.assert_array_equal(bits(out), expected)
    if dtype == 0 and k % 8 == 0 and tokens > 32:
        backend._check(lib.venturi_q8_prefill_run(x.data_ptr(), dc.data_ptr(), ds.data_ptr(), want.data_ptr(), tokens,
                                                  n, k, padded, dtype, s))
    else:
        backend._check(lib.venturi_q8_head_run(x.data_ptr(), dc.data_ptr(), ds.data_ptr(), want.data_ptr(), tokens, n,
                                               k, padded, dtype, s))
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("precision,passes", [("wxa8", 1), ("wxa8-residual", 2)])
@pytest.mark.parametrize("tokens", [1, 5, 70])
def test_q8_a8_plan_and_packed_reuse(backend, device, precision, passes, tokens):
    n, k = 33, 300
    codes, scales = random_q8(n, k, 9 + tokens)
    plan = prepare_row_codec(8, 32, precision=precision)
    size = plan.workspace_bytes(tokens=tokens, k=k)
    ws = torch.empty(size, dtype=torch.uint8, device=device)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens)).half().to(device)
    dc, ds = codes.to(device), scales.to(device)
    padded = codes.shape[1]
    s = torch.cuda.current_stream(device).cuda_stream
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    plan.project(x.data_ptr(), dc.data_ptr(), None, ds.data_ptr(), out.data_ptr(), ws.data_ptr(), size, tokens=tokens,
                 n=n, k=k, padded=padded, stream=s)
    lib = backend._native
    ws2 = torch.empty_like(ws)
    want = torch.empty_like(out)
    backend._check(lib.venturi_q8_dp4a_quantize(x.data_ptr(), ws2.data_ptr(), size, tokens, k, passes, s))
    backend._check(lib.venturi_q8_dp4a_run(ws2.data_ptr(), size, dc.data_ptr(), ds.data_ptr(), want.data_ptr(), tokens,
                                           n, k, padded, passes, s))
    assert torch.equal(out.view(torch.int16), want.view(torch.int16)) and torch.equal(ws, ws2)
    # packed = 1 reuses the workspace: a changed x does not change the output.
    x.zero_()
    again = torch.empty_like(out)
    plan.project(x.data_ptr(), dc.data_ptr(), None, ds.data_ptr(), again.data_ptr(), ws.data_ptr(), size,
                 tokens=tokens, n=n, k=k, padded=padded, packed=True, stream=s)
    assert torch.equal(again.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("nbits", [4, 5, 6])
@pytest.mark.parametrize("k", [128, 136, 130])
@pytest.mark.parametrize("tokens", [1, 9, 64])
def test_row_codec_a16_plans(backend, device, nbits, k, tokens):
    n = 45
    packed, high, scales = _row_planes(n, k, nbits, nbits + k + tokens)
    plan = prepare_row_codec(nbits, 64)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens)).half().to(device)
    dc, ds = _dev(packed, device), _dev(scales, device)
    dh = _dev(high if nbits > 4 else np.zeros((1, 16), np.uint8), device)
    padded = packed.shape[1] * 2
    s = torch.cuda.current_stream(device).cuda_stream
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    lib = backend._native
    if k % 8 != 0 and nbits == 6:
        with pytest.raises(RuntimeError, match="k % 8"):
            plan.project(x.data_ptr(), dc.data_ptr(), dh.data_ptr(), ds.data_ptr(), out.data_ptr(), None, 0,
                         tokens=tokens, n=n, k=k, padded=padded, stream=s)
        return
    plan.project(x.data_ptr(), dc.data_ptr(), dh.data_ptr(), ds.data_ptr(), out.data_ptr(), None, 0, tokens=tokens, n=n,
                 k=k, padded=padded, stream=s)
    want = torch.empty_like(out)
    if k % 8 == 0:
        backend._check(lib.venturi_row_gemm_run(x.data_ptr(), dc.data_ptr(), dh.data_ptr(), ds.data_ptr(),
                                                want.data_ptr(), tokens, n, k, padded, nbits, 0, s))
    elif nbits == 4:
        assert lib.venturi_q4_linear(x.data_ptr(), dc.data_ptr(), ds.data_ptr(), want.data_ptr(), tokens, n, k, padded,
                                     s) == 0
    else:
        assert lib.venturi_q5_linear(x.data_ptr(), dc.data_ptr(), dh.data_ptr(), ds.data_ptr(), want.data_ptr(), tokens,
                                     n, k, padded, s) == 0
    torch.cuda.synchronize(device)
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


def test_q4_fused_research_plan(backend, device):
    n, k, tokens = 21, 192, 3
    packed, _, scales = _row_planes(n, k, 4, 1)
    plan = prepare_row_codec(4, 64, implementation="fused-research")
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(2)).half().to(device)
    dc, ds = _dev(packed, device), _dev(scales, device)
    s = torch.cuda.current_stream(device).cuda_stream
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    plan.project(x.data_ptr(), dc.data_ptr(), None, ds.data_ptr(), out.data_ptr(), None, 0, tokens=tokens, n=n, k=k,
                 padded=256, stream=s)
    want = torch.empty_like(out)
    backend._check(backend._native.venturi_q4_fused_run(x.data_ptr(), dc.data_ptr(), ds.data_ptr(), want.data_ptr(),
                                                        tokens, n, k, 256, 0, s))
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("fmt", ["q8_g32_fp16", "q4_g64_fp16", "q5_g64_fp16"])
def test_plan_over_planes_read_from_safetensors(backend, device, tmp_path, fmt):
    # The stored schema (docs/qwen-safetensors.md:45-58) feeds the plan table as
    # read: Q8 A16 up to 32 tokens gives the canonical bytes, Q4/Q5 at k % 8 != 0
    # the exact GEMVs' bytes (flash_next_q4.cu:23-34, flash_next_q5.cu:26-38).
    from safetensors.torch import save_file
    from venturi_amd.planes import planes_of, read_planes
    from venturi_amd.weights import Q4RowSplitWeight, Q5RowSplitWeight, Q8RowSplitWeight

    n, tokens = 37, 5
    k = 300 if fmt == "q8_g32_fp16" else 130
    print(f"case planes {fmt} n={n} k={k} tokens={tokens}", flush=True)
    gen = torch.Generator().manual_seed(len(fmt) + k)
    if fmt == "q8_g32_fp16":
        weight = Q8RowSplitWeight.from_dense((torch.randn(n, k, generator=gen) * 0.02).half())
        plan, bits_ = prepare_row_codec(8, 32), 8
    else:
        lo = -8 if fmt == "q4_g64_fp16" else -16
        codes = torch.randint(lo, -lo, (n, k), generator=gen)
        scales = (torch.rand(n, -(-k // 64), generator=gen) * 0.01).half()
        cls = Q4RowSplitWeight if fmt == "q4_g64_fp16" else Q5RowSplitWeight
        weight = cls.from_codes(codes, scales)
        bits_ = 4 if fmt == "q4_g64_fp16" else 5
        plan = prepare_row_codec(bits_, 64)
    path = tmp_path / "planes.safetensors"
    save_file(planes_of("model.mlp.proj", weight), str(path))
    planes = read_planes(path, "model.mlp.proj", fmt, (n, k))
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(3)).half()
    dx = x.to(device)
    dc, ds = planes.codes.to(device), planes.scales.to(device)
    dh = planes.high.to(device) if planes.high is not None else None
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    s = torch.cuda.current_stream(device).cuda_stream
    plan.project(dx.data_ptr(), dc.data_ptr(), dh.data_ptr() if dh is not None else None, ds.data_ptr(),
                 out.data_ptr(), None, 0, tokens=tokens, n=n, k=k, padded=planes.padded_k, stream=s)
    if bits_ == 8:
        expected = oracle.q8_linear(bits(x), planes.codes.numpy(), planes.scales.numpy(), k)
    elif bits_ == 4:
        expected = oracle.q4_linear(bits(x), planes.codes.numpy(), planes.scales.numpy(), k)
    else:
        expected = oracle.q5_linear(bits(x), planes.codes.numpy(), planes.high.numpy(), planes.scales.numpy(), k)
    np.testing.assert_array_equal(bits(out), expected)
