"""Q5 operators and the Q4/Q5/Q6 row decode on the device, against the CPU oracle.

Bytes must match: the decode is one RNE rounding of an exact product, and the
W5A16 GEMV runs the reference's lane-strided fmaf order and 32-lane tree. The
reference's own execution check (a relative bound against a torch fp32
product) is kept as well.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import bits
from venturi_amd.q5 import NativeQ5, decode_q5_fp16, quantize_q5_rtn
from venturi_amd.weights import Q5RowSplitWeight

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def native():
    return NativeQ5()


@pytest.mark.parametrize("shape", [(64, 320), (33, 130), (5, 640), (1, 1), (17, 5120)])
@pytest.mark.parametrize("tokens", [1, 3, 17, 64])
def test_decode_and_linear_bytes(native, device, shape, tokens):
    n, k = shape
    print(f"case q5 n={n} k={k} tokens={tokens}", flush=True)
    torch.manual_seed(31 + n + k)
    q = quantize_q5_rtn(torch.randn(n, k))
    prepared = native.prepare(q, device=device)
    assert torch.equal(native.decode(prepared).cpu(), decode_q5_fp16(q))
    x = torch.randn(tokens, k).half()
    got = native.linear(x.to(device), prepared).cpu()
    want = oracle.q5_linear(bits(x), q.codes.numpy(), q.high.numpy(), q.scales.numpy(), k)
    np.testing.assert_array_equal(bits(got), want)
    # The reference's execution bound (tests/test_flash_next_q5.py:125-131).
    expected = (x.float() @ decode_q5_fp16(q).float().t()).half()
    peak = expected.float().abs().max().clamp_min(1e-6)
    assert float((got.float() - expected.float()).abs().max() / peak) < 1e-3


def test_linear_bounds_and_status(native, device):
    torch.manual_seed(32)
    q = quantize_q5_rtn(torch.randn(8, 128))
    prepared = native.prepare(q, device=device)
    with pytest.raises(ValueError):
        native.linear(torch.randn(65, 128, dtype=torch.float16).to(device), prepared)
    w = prepared.weight
    lib = native.lib
    s = torch.cuda.current_stream(device).cuda_stream
    out = torch.empty(1, 8, dtype=torch.float16, device=device)
    x = torch.ones(1, 128, dtype=torch.float16, device=device)
    # hipErrorInvalidValue (1) for bad geometry, as the reference's cudaErrorInvalidValue.
    assert lib.venturi_q5_linear(x.data_ptr(), w.codes.data_ptr(), w.high.data_ptr(), w.scales.data_ptr(),
                                 out.data_ptr(), 65, 8, 128, 128, s) == 1
    assert lib.venturi_q5_linear(x.data_ptr(), w.codes.data_ptr(), w.high.data_ptr(), w.scales.data_ptr(),
                                 out.data_ptr(), 1, 8, 128, 64, s) == 1
    assert lib.venturi_q5_decode(w.codes.data_ptr(), None, w.scales.data_ptr(), out.data_ptr(), 8, 128, 128, s) == 1
    torch.cuda.synchronize(device)


def _planes(n, k, nbits, seed):
    padded = (k + 127) // 128 * 128
    rng = np.random.default_rng(seed)
    codes = rng.integers(-(1 << (nbits - 1)), 1 << (nbits - 1), size=(n, padded))
    codes[:, k:] = 0
    scales = (rng.random((n, padded // 64)) * 0.02).astype(np.float16)
    return oracle.pack_row_codec(codes, scales, nbits)


@pytest.mark.parametrize("nbits", [4, 5, 6])
@pytest.mark.parametrize("k,padded_extra", [(1, 0), (63, 0), (130, 128), (2049, 0), (5120, 0)])
def test_row_dequant_rows_and_indexed(backend, device, nbits, k, padded_extra):
    print(f"case row-decode bits={nbits} k={k}", flush=True)
    n = 37
    packed, high, scales = _planes(n, k, nbits, nbits * 1000 + k)
    if padded_extra:  # a wider padded K than the minimum is accepted (blocks.cu:1079)
        packed = np.pad(packed, ((0, 0), (0, padded_extra // 2)))
        high = np.pad(high, ((0, 0), (0, padded_extra * (nbits - 4) // 8)))
        scales = np.pad(scales, ((0, 0), (0, padded_extra // 64)))
    padded = packed.shape[1] * 2
    lib = backend._native
    s = torch.cuda.current_stream(device).cuda_stream
    dc = torch.from_numpy(packed).to(device)
    dh = torch.from_numpy(high if nbits > 4 else np.zeros((n, 1), np.uint8)).to(device)
    ds = torch.from_numpy(scales).to(device)
    row0, rows = 5, 29
    guard = torch.full((rows * k + 2,), 47, dtype=torch.float16, device=device)
    out = guard[1:-1]
    backend._check(lib.venturi_row_dequant_rows(dc.data_ptr(), dh.data_ptr(), ds.data_ptr(), out.data_ptr(), row0, rows,
                                                k, padded, nbits, s))
    want = oracle.row_decode(packed, high, scales, k, nbits, np.arange(row0, row0 + rows))
    g = guard.cpu()
    assert g[0] == g[-1] == 47
    np.testing.assert_array_equal(bits(out.view(rows, k)), want)
    ids = np.array([36, 0, 5, 5, 17], dtype=np.int64)
    dids = torch.from_numpy(ids).to(device)
    out2 = torch.empty(len(ids), k, dtype=torch.float16, device=device)
    backend._check(lib.venturi_row_dequant_indexed(dc.data_ptr(), dh.data_ptr(), ds.data_ptr(), dids.data_ptr(),
                                                   out2.data_ptr(), len(ids), k, padded, nbits, s))
    np.testing.assert_array_equal(bits(out2), oracle.row_decode(packed, high, scales, k, nbits, ids))


def test_row_decode_q5_equals_native_decode(backend, native, device):
    torch.manual_seed(3)
    q = Q5RowSplitWeight.from_dense(torch.randn(12, 300))
    prepared = native.prepare(q, device=device)
    w = prepared.weight
    out = torch.empty(12, 300, dtype=torch.float16, device=device)
    backend._check(backend._native.venturi_row_dequant_rows(
        w.codes.data_ptr(), w.high.data_ptr(), w.scales.data_ptr(), out.data_ptr(), 0, 12, 300, 384, 5,
        torch.cuda.current_stream(device).cuda_stream))
    assert torch.equal(out.cpu(), native.decode(prepared).cpu())
    assert torch.equal(out.cpu(), decode_q5_fp16(q))


def test_row_decode_rejects_bad_arguments(backend, device):
    lib = backend._native
    x = torch.zeros(64, dtype=torch.uint8, device=device)
    o = torch.empty(128, dtype=torch.float16, device=device)
    s = torch.cuda.current_stream(device).cuda_stream
    assert lib.venturi_row_dequant_rows(x.data_ptr(), x.data_ptr(), x.data_ptr(), o.data_ptr(), 0, 1, 128, 128, 7, s) == -1
    assert "4, 5 or 6" in backend._native.error()
    assert lib.venturi_row_dequant_rows(x.data_ptr(), None, x.data_ptr(), o.data_ptr(), 0, 1, 128, 128, 5, s) == -1
    assert lib.venturi_row_dequant_indexed(x.data_ptr(), x.data_ptr(), x.data_ptr(), None, o.data_ptr(), 1, 128, 128,
                                           5, s) == -1
    torch.cuda.synchronize(device)


def _ulp16(v):
    v = np.abs(v)
    return 2.0 ** (np.floor(np.log2(np.maximum(v, 2.0**-14))) - 10)


@pytest.mark.parametrize("nbits", [4, 5, 6])
@pytest.mark.parametrize("shape", [(1, 8), (37, 136), (130, 768), (300, 2048), (6200, 136), (16400, 264)])
@pytest.mark.parametrize("tokens", [1, 5, 16, 24, 33, 130, 300])
def test_row_gemm_contract_tolerances(backend, device, nbits, shape, tokens):
    # The W*A16 contract: weights fp16(q * scale) (the oracle's row decode),
    # fp32 accumulation; |y - exact| <= 0.5 ulp_fp16 + 2^-19 sum|x w| against
    # FP64, and against the reference-order Q5 GEMV within 2e-3 / one ulp,
    # rel-L2 1e-3. Token counts cover the decode kernel's one and two token
    # blocks and the prefill tiles; row counts cover each decode launch shape
    # (up to 384, up to 1023 and from 1024 row blocks of 16).
    n, k = shape
    print(f"case row-gemm bits={nbits} n={n} k={k} tokens={tokens}", flush=True)
    _row_gemm_contract(backend, device, nbits, n, k, tokens)


@pytest.mark.parametrize("nbits", [4, 5, 6])
@pytest.mark.parametrize("shape,tokens", [((16400, 264), 1000), ((14336, 136), 1024)])
def test_row_prefill_large_grids(backend, device, nbits, shape, tokens):
    # Prefill grids of about a thousand workgroups (129 x 8 and 112 x 8 tiles
    # of 128 tokens x 128 rows), one of them with a ragged last token tile.
    n, k = shape
    print(f"case row-prefill bits={nbits} n={n} k={k} tokens={tokens}", flush=True)
    _row_gemm_contract(backend, device, nbits, n, k, tokens)


@pytest.mark.parametrize("nbits", [4, 5, 6])
@pytest.mark.parametrize("shape,tokens", [((5120, 136), 2085), ((6144, 264), 2048), ((7168, 72), 300)])
def test_row_prefill_wide_tiles(backend, device, nbits, shape, tokens):
    # From 256 tokens the prefill takes 256-token tiles of 160, 192 or 224
    # rows, picked per row count (these three pick each width on a 256-CU
    # part); ragged token, row and group tails.
    n, k = shape
    print(f"case row-prefill-wide bits={nbits} n={n} k={k} tokens={tokens}", flush=True)
    _row_gemm_contract(backend, device, nbits, n, k, tokens)


def _row_gemm_contract(backend, device, nbits, n, k, tokens):
    packed, high, scales = _planes(n, k, nbits, 77 * nbits + n + tokens)
    padded = packed.shape[1] * 2
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens + k)).half()
    lib = backend._native
    s = torch.cuda.current_stream(device).cuda_stream
    dc = torch.from_numpy(packed).to(device)
    dh = torch.from_numpy(high if nbits > 4 else np.zeros((1, 16), np.uint8)).to(device)
    ds = torch.from_numpy(scales).to(device)
    guard = torch.full((tokens * n + 2,), 47, dtype=torch.float16, device=device)
    out = guard[1:-1].view(tokens, n)
    backend._check(lib.venturi_row_gemm_run(x.to(device).data_ptr(), dc.data_ptr(), dh.data_ptr(), ds.data_ptr(),
                                            out.data_ptr(), tokens, n, k, padded, nbits, 0, s))
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    wd = oracle.row_decode(packed, high, scales, k, nbits).view(np.float16).astype(np.float64)
    xd = x.float().numpy().astype(np.float64)
    exact = xd @ wd.T
    got = out.cpu().float().numpy().astype(np.float64)
    bound = 0.5 * _ulp16(exact) + 2.0**-19 * (np.abs(xd) @ np.abs(wd).T)
    assert (np.abs(got - exact) <= bound).all()
    if nbits == 5 and tokens <= 64:
        ref = oracle.q5_linear(bits(x), packed, high, scales, k).view(np.float16).astype(np.float64)
        diff = np.abs(got - ref)
        assert (diff <= np.maximum(2e-3, _ulp16(ref))).all()
        assert np.linalg.norm(got - ref) <= 1e-3 * max(np.linalg.norm(ref), 1e-12)
    if nbits == 4:
        same = torch.empty_like(out)
        backend._check(lib.venturi_q4_gemm_run(x.to(device).data_ptr(), dc.data_ptr(), ds.data_ptr(), same.data_ptr(),
                                               tokens, n, k, padded, 0, s))
        assert torch.equal(same.view(torch.int16), out.view(torch.int16))


def test_row_gemm_rejects_bad_arguments(backend, device):
    lib = backend._native
    x = torch.zeros(1, 64, dtype=torch.float16, device=device)
    c = torch.zeros(1, 64, dtype=torch.uint8, device=device)
    o = torch.empty(1, 1, dtype=torch.float16, device=device)
    s = torch.cuda.current_stream(device).cuda_stream
    assert lib.venturi_row_gemm_run(x.data_ptr(), c.data_ptr(), None, c.data_ptr(), o.data_ptr(), 1, 1, 64, 128, 5, 0,
                                    s) == -1
    assert "null" in lib.error()
    assert lib.venturi_row_gemm_run(x.data_ptr(), c.data_ptr(), c.data_ptr(), c.data_ptr(), o.data_ptr(), 1, 1, 64, 128,
                                    7, 0, s) == -1
    assert "4, 5 or 6" in lib.error()
    torch.cuda.synchronize(device)


@pytest.mark.parametrize("nbits", [4, 5, 6])
@pytest.mark.parametrize("shape", [(37, 136), (300, 2048), (6200, 264)])
@pytest.mark.parametrize("tokens", [1, 5, 16, 24])
def test_row_tiled_decode_equals_row_major(backend, device, nbits, shape, tokens):
    # The tiled copies (q4.tile_q4 for 4 bits, q5.tile_row_codec for 5/6) give the
    # bits of the row-major decode GEMM for shapes that do not split K.
    from venturi_amd.q4 import tile_q4
    from venturi_amd.q5 import tile_row_codec

    n, k = shape
    print(f"case row-tiled bits={nbits} n={n} k={k} tokens={tokens}", flush=True)
    packed, high, scales = _planes(n, k, nbits, 11 * nbits + n + tokens)
    padded = packed.shape[1] * 2
    lib = backend._native
    assert lib.venturi_q4_tiled_workspace_bytes(tokens, n, k) == 0
    s = torch.cuda.current_stream(device).cuda_stream
    dc = torch.from_numpy(packed).to(device)
    dh = torch.from_numpy(high if nbits > 4 else np.zeros((1, 16), np.uint8)).to(device)
    ds = torch.from_numpy(scales).to(device)
    if nbits == 4:
        tc, ts = tile_q4(dc, ds)
        th = dh
    else:
        tc, th, ts = tile_row_codec(dc, dh, ds, nbits)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens * 3 + k)).half().to(device)
    want = torch.empty(tokens, n, dtype=torch.float16, device=device)
    backend._check(lib.venturi_row_gemm_run(x.data_ptr(), dc.data_ptr(), dh.data_ptr(), ds.data_ptr(), want.data_ptr(),
                                            tokens, n, k, padded, nbits, 0, s))
    got = torch.empty_like(want)
    backend._check(lib.venturi_row_tiled_run(x.data_ptr(), tc.data_ptr(), th.data_ptr(), ts.data_ptr(), got.data_ptr(),
                                             tokens, n, k, padded, nbits, 0, None, 0, s))
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("nbits", [5, 6])
@pytest.mark.parametrize("shape", [(16, 8192), (130, 8320), (37, 8200), (5120, 17408)])
@pytest.mark.parametrize("tokens", [1, 3, 16])
def test_row_tiled_decode_split_k(backend, device, nbits, shape, tokens):
    # Q5/Q6 tiled decode where K is split over two workgroups (the exchange
    # slots and the tiled high plane): the W*A16 contract bound against FP64,
    # the same bytes on a second run, idle slots afterwards, and HIP-graph
    # replays (eager work between them) equal to the eager result.
    from venturi_amd.q5 import tile_row_codec

    n, k = shape
    print(f"case row-tiled-split bits={nbits} n={n} k={k} tokens={tokens}", flush=True)
    packed, high, scales = _planes(n, k, nbits, 13 * nbits + n + tokens)
    padded = packed.shape[1] * 2
    lib = backend._native
    s = torch.cuda.current_stream(device).cuda_stream
    size = lib.venturi_q4_tiled_workspace_bytes(tokens, n, k)
    assert size == tokens * ((n + 15) // 16) * 64
    slots = torch.empty(size, dtype=torch.uint8, device=device)
    backend._check(lib.venturi_q4_tiled_workspace_init(slots.data_ptr(), size, s))
    idle = slots.clone()
    tc, th, ts = tile_row_codec(torch.from_numpy(packed).to(device), torch.from_numpy(high).to(device),
                                torch.from_numpy(scales).to(device), nbits)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens * 5 + k)).half()
    xd = x.to(device)

    def run(out):
        backend._check(lib.venturi_row_tiled_run(xd.data_ptr(), tc.data_ptr(), th.data_ptr(), ts.data_ptr(),
                                                 out.data_ptr(), tokens, n, k, padded, nbits, 0, slots.data_ptr(),
                                                 size, torch.cuda.current_stream(device).cuda_stream))

    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    run(out)
    again = torch.empty_like(out)
    run(again)
    torch.cuda.synchronize(device)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    assert torch.equal(slots, idle)
    replayed = torch.empty_like(out)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(replayed)
    for i in range(3):
        replayed.fill_(0)
        graph.replay()
        torch.cuda.synchronize(device)
        assert torch.equal(replayed.view(torch.int16), out.view(torch.int16)), f"replay {i}"
        run(again)
        torch.cuda.synchronize(device)
        assert torch.equal(again.view(torch.int16), out.view(torch.int16))
    assert torch.equal(slots, idle)
    wd = oracle.row_decode(packed, high, scales, k, nbits).view(np.float16).astype(np.float64)
    xf = x.float().numpy().astype(np.float64)
    exact = xf @ wd.T
    got = out.cpu().float().numpy().astype(np.float64)
    bound = 0.5 * _ulp16(exact) + 2.0**-19 * (np.abs(xf) @ np.abs(wd).T)
    assert (np.abs(got - exact) <= bound).all()
