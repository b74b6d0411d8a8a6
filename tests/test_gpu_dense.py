"""The dense W*A16 route (venturi_row_dense_run), the reference's ChunkedDense
projection (row_codec_dispatch.cuh:41-48, qwen_runtime.cuh:348-364): rows are
decoded to the contract's fp16(q*scale) weights in the workspace and multiplied
by hipBLASLt with fp32 accumulation. Outputs are checked against the FP64
product of the oracle's decoded weights (half an fp16 ulp plus 2^-19 of the
absolute product, the bound every W*A16 route here meets) and, at the
config-2 gate+up shape, against the fp32 product of the same weights within
max(2e-3, 1 fp16 ulp); chunked and whole runs, the Q4 plan's auto route and
the native plan table are covered, and every run is repeated for determinism.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import agreement, assert_free_order, ulp16
from venturi_amd.q4 import DENSE_TOKENS
from venturi_amd.rowcodec import prepare_row_codec
from venturi_amd.weights import Q4RowSplitWeight

pytestmark = pytest.mark.gpu

BLAS_BYTES = 32 * 2**20


def _planes(n, k, nbits, seed):
    padded = (k + 127) // 128 * 128
    rng = np.random.default_rng(seed)
    codes = rng.integers(-(1 << (nbits - 1)), 1 << (nbits - 1), size=(n, padded))
    codes[:, k:] = 0
    scales = (rng.random((n, padded // 64)) * 0.02).astype(np.float16)
    return oracle.pack_row_codec(codes, scales, nbits)


def _bound_check(got, x, packed, high, scales, k, nbits, rows=None, tokens=None):
    """FP64 contract bound on the (tokens x rows) sample of the output."""
    rows = np.arange(packed.shape[0]) if rows is None else rows
    tokens = np.arange(x.shape[0]) if tokens is None else tokens
    wd = oracle.row_decode(packed[rows], high[rows], scales[rows], k, nbits).view(np.float16).astype(np.float64)
    xd = x[tokens].float().numpy().astype(np.float64)
    exact = xd @ wd.T
    sample = got[np.ix_(tokens, rows)].astype(np.float64)
    bound = 0.5 * ulp16(exact) + 2.0**-19 * (np.abs(xd) @ np.abs(wd).T)
    assert (np.abs(sample - exact) <= bound).all()
    return wd, xd


def _device_planes(packed, high, scales, nbits, device):
    dc = torch.from_numpy(packed).to(device)
    dh = torch.from_numpy(high if nbits > 4 else np.zeros((1, 16), np.uint8)).to(device)
    ds = torch.from_numpy(scales).to(device)
    return dc, dh, ds


def _run(lib, backend, x, dc, dh, ds, out, tokens, n, k, padded, nbits, ws, size, s):
    backend._check(lib.venturi_row_dense_run(x.data_ptr(), dc.data_ptr(), dh.data_ptr(), ds.data_ptr(), out.data_ptr(),
                                             tokens, n, k, padded, nbits, 0, ws.data_ptr(), size, s))


@pytest.mark.parametrize("nbits", [4, 5, 6])
@pytest.mark.parametrize("shape,tokens", [((200, 264), 37), ((64, 512), 1), ((1032, 136), 300), ((256, 5120), 1024)])
@pytest.mark.parametrize("chunk", [None, 48])
def test_dense_contract(backend, device, nbits, shape, tokens, chunk):
    # chunk None: the preferred workspace (these matrices decode whole); 48: a
    # workspace of 48 shadow rows, so the rows run in 48-row chunks and the
    # last one is ragged.
    n, k = shape
    print(f"case dense bits={nbits} n={n} k={k} tokens={tokens} chunk={chunk}", flush=True)
    lib = backend._native
    s = torch.cuda.current_stream(device).cuda_stream
    packed, high, scales = _planes(n, k, nbits, 31 * nbits + n + tokens)
    padded = packed.shape[1] * 2
    dc, dh, ds = _device_planes(packed, high, scales, nbits, device)
    size = int(lib.venturi_row_dense_workspace_bytes(tokens, n, k))
    assert size == BLAS_BYTES + 2 * n * k
    if chunk is not None:
        size = BLAS_BYTES + 2 * k * chunk
    ws = torch.empty(size, dtype=torch.uint8, device=device)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens + k)).half()
    xd = x.to(device)
    guard = torch.full((tokens * n + 16,), 47, dtype=torch.float16, device=device)
    out = guard[8:-8].view(tokens, n)  # 16-byte aligned interior
    _run(lib, backend, xd, dc, dh, ds, out, tokens, n, k, padded, nbits, ws, size, s)
    again = torch.empty_like(out)
    _run(lib, backend, xd, dc, dh, ds, again, tokens, n, k, padded, nbits, ws, size, s)
    g = guard.cpu()
    assert (g[:8] == 47).all() and (g[-8:] == 47).all()
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    _bound_check(out.cpu().float().numpy(), x, packed, high, scales, k, nbits)


def test_q4_plan_auto_route_is_dense(backend, device):
    n, k, tokens = 256, 512, DENSE_TOKENS
    print(f"case dense-plan n={n} k={k} tokens={tokens}", flush=True)
    packed, high, scales = _planes(n, k, 4, 5)
    w = Q4RowSplitWeight(torch.from_numpy(packed), torch.from_numpy(scales), k)
    resident = backend.upload_linear(w, dtype=torch.float16, device=device)
    assert resident.prepare(tokens=tokens - 1).route == "venturi-q4-mfma"
    plan = resident.prepare(tokens=tokens)
    assert plan.route == "venturi-q4-dense"
    assert plan.workspace_bytes == BLAS_BYTES + 2 * n * k
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(3)).half()
    xd = x.to(device)
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    # Without a workspace (the reference's run(x, out=)) the plan runs the
    # fused matrix-core GEMM: the bytes of the mfma route.
    plain = torch.empty_like(out)
    plan.run(xd, out=plain)
    fused = torch.empty_like(out)
    resident.prepare(tokens=tokens, route="mfma").run(xd, out=fused)
    assert torch.equal(plain.view(torch.int16), fused.view(torch.int16))
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    plan.run(xd, out=out, workspace=ws)
    got = out.cpu().float().numpy()
    wd, xf = _bound_check(got, x, packed, high, scales, k, 4)
    ref = (xf.astype(np.float32) @ wd.astype(np.float32).T).astype(np.float16).astype(np.float64)
    diff = np.abs(got - ref)
    assert (diff <= np.maximum(2e-3, ulp16(ref))).all()
    # The fused matrix-core route on the same weights is the same contract.
    _bound_check(fused.cpu().float().numpy(), x, packed, high, scales, k, 4)


def test_dense_at_config2_gate_up(backend, device):
    # The timed prefill shape: 34 816 x 5120 at 2048 tokens decodes in four
    # 8192-row chunks and a 2048-row tail (the 340 MiB shadow is cut into
    # 80 MiB pieces). Sampled rows (every chunk edge among them) and tokens
    # against FP64 and fp32.
    n, k, tokens = 34816, 5120, 2048
    print(f"case dense-gate-up n={n} k={k} tokens={tokens}", flush=True)
    lib = backend._native
    assert lib.venturi_row_dense_workspace_bytes(tokens, n, k) == BLAS_BYTES + 2 * 8192 * k
    packed, high, scales = _planes(n, k, 4, 77)
    w = Q4RowSplitWeight(torch.from_numpy(packed), torch.from_numpy(scales), k)
    plan = backend.upload_linear(w, dtype=torch.float16, device=device).prepare(tokens=tokens)
    assert plan.route == "venturi-q4-dense"
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(8)).half()
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    plan.run(x.to(device), out=out, workspace=ws)
    got = out.cpu().float().numpy()
    rng = np.random.default_rng(1)
    edges = np.array([0, 8191, 8192, 16383, 16384, 24575, 24576, 32767, 32768, n - 1])
    rows = np.unique(np.concatenate([edges, rng.choice(n, 120, replace=False)]))
    toks = np.unique(np.concatenate([[0, tokens - 1], rng.choice(tokens, 62, replace=False)]))
    wd, xf = _bound_check(got, x, packed, high, scales, k, 4, rows, toks)
    ref = (xf.astype(np.float32) @ wd.astype(np.float32).T).astype(np.float16).astype(np.float64)
    stats = agreement(got[np.ix_(toks, rows)], ref)
    print(f"max_abs={stats['max_abs']:.3g} max_ulp={stats['max_ulp']:.2f} flips={stats['flips']} of {ref.size}",
          flush=True)
    assert_free_order(stats)


def test_plan_table_runs_the_dense_route(backend, device):
    # At 1024 tokens a ChunkedDense plan given its workspace runs the dense
    # route (the bits of venturi_row_dense_run with that workspace); without a
    # workspace it runs the fused matrix-core GEMM (the bits of venturi_row_gemm_run).
    n, k, tokens, nbits = 136, 384, 1024, 5
    print(f"case dense-rowcodec n={n} k={k} tokens={tokens}", flush=True)
    lib = backend._native
    s = torch.cuda.current_stream(device).cuda_stream
    packed, high, scales = _planes(n, k, nbits, 12)
    padded = packed.shape[1] * 2
    dc, dh, ds = _device_planes(packed, high, scales, nbits, device)
    plan = prepare_row_codec(nbits, 64, precision="wxa16", dtype=0, implementation="auto")
    size = plan.workspace_bytes(tokens=tokens, k=k)
    assert size == (32 + 192) * 2**20
    ws = torch.empty(size, dtype=torch.uint8, device=device)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(4)).half().to(device)
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    plan.project(x.data_ptr(), dc.data_ptr(), dh.data_ptr(), ds.data_ptr(), out.data_ptr(), ws.data_ptr(), size,
                 tokens=tokens, n=n, k=k, padded=padded, stream=s)
    want = torch.empty_like(out)
    _run(lib, backend, x, dc, dh, ds, want, tokens, n, k, padded, nbits, ws, size, s)
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    plan.project(x.data_ptr(), dc.data_ptr(), dh.data_ptr(), ds.data_ptr(), out.data_ptr(), None, 0, tokens=tokens,
                 n=n, k=k, padded=padded, stream=s)
    backend._check(lib.venturi_row_gemm_run(x.data_ptr(), dc.data_ptr(), dh.data_ptr(), ds.data_ptr(), want.data_ptr(),
                                            tokens, n, k, padded, nbits, 0, s))
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


def test_dense_rejects_bad_arguments(backend, device):
    lib = backend._native
    s = torch.cuda.current_stream(device).cuda_stream
    n, k, tokens = 16, 128, 4
    x = torch.zeros(tokens, k, dtype=torch.float16, device=device)
    c = torch.zeros(n, k // 2, dtype=torch.uint8, device=device)
    sc = torch.zeros(n, 2, dtype=torch.float16, device=device)
    o = torch.empty(tokens, n, dtype=torch.float16, device=device)
    size = int(lib.venturi_row_dense_workspace_bytes(tokens, n, k))
    ws = torch.empty(size + 256, dtype=torch.uint8, device=device)
    args = (x.data_ptr(), c.data_ptr(), None, sc.data_ptr(), o.data_ptr())
    assert lib.venturi_row_dense_run(*args, tokens, n, k, k, 4, 1, ws.data_ptr(), size, s) == -1
    assert "fp16" in lib.error()
    assert lib.venturi_row_dense_run(*args, tokens, n, 124, 128, 4, 0, ws.data_ptr(), size, s) == -1
    assert "k % 8" in lib.error()
    assert lib.venturi_row_dense_run(*args, tokens, n, k, k, 4, 0, ws.data_ptr(), BLAS_BYTES, s) == -1
    assert "16-row chunk" in lib.error()
    assert lib.venturi_row_dense_run(*args, tokens, n, k, k, 4, 0, ws.data_ptr() + 16, size, s) == -1
    assert "256-byte" in lib.error()
    assert lib.venturi_row_dense_run(*args, tokens, n, k, k, 7, 0, ws.data_ptr(), size, s) == -1
    assert lib.venturi_row_dense_run(x.data_ptr(), c.data_ptr(), None, sc.data_ptr(), None, tokens, n, k, k, 4, 0,
                                     ws.data_ptr(), size, s) == -1
    torch.cuda.synchronize(device)


# ---------------------------------------------------------------------------
# The Q8 dense route (venturi_q8_dense_run): rows decoded to the exact two-term
# fp16 form q*s = hi + lo, x doubled, one GEMM over 2k. Held to the matrix-core
# routes' contract: the FP64 bound on the exact products q*s and, against the
# canonical-order oracle, helpers.assert_free_order.

from helpers import bits, random_q8  # noqa: E402
from venturi_amd import Q8RowSplitWeight  # noqa: E402
from venturi_amd.vocabulary import DENSE_TOKENS as Q8_DENSE_TOKENS  # noqa: E402


def _q8_check(got, x, codes, scales, k):
    w = oracle.q8_unpack(codes, scales, k)  # q*s exactly, FP64
    xd = x.float().numpy().astype(np.float64)
    exact = xd @ w.T
    g = got.astype(np.float64)
    bound = 0.5 * ulp16(exact) + 2.0**-19 * (np.abs(xd) @ np.abs(w).T)
    assert (np.abs(g - exact) <= bound).all()
    stats = agreement(g, oracle.q8_linear(bits(x), codes, scales, k))
    assert_free_order(stats)
    return stats


def _q8_run(lib, backend, x, dc, ds, out, tokens, n, k, ws, size, s):
    backend._check(lib.venturi_q8_dense_run(x.data_ptr(), dc.data_ptr(), ds.data_ptr(), out.data_ptr(), tokens, n, k,
                                            dc.shape[1], 0, ws.data_ptr(), size, s))


@pytest.mark.parametrize("shape,tokens", [((200, 264), 37), ((64, 512), 1), ((1032, 136), 300), ((8200, 128), 40)])
@pytest.mark.parametrize("chunk", [None, 48])
def test_q8_dense_contract(backend, device, shape, tokens, chunk):
    # (8200, 128) runs an 8192-row chunk and an 8-row one; chunk 48 forces
    # 48-row chunks through a smaller workspace.
    n, k = shape
    print(f"case q8-dense n={n} k={k} tokens={tokens} chunk={chunk}", flush=True)
    lib = backend._native
    s = torch.cuda.current_stream(device).cuda_stream
    codes, scales = random_q8(n, k, 401 + n + tokens)
    dc, ds = codes.to(device), scales.to(device)
    size = int(lib.venturi_q8_dense_workspace_bytes(tokens, n, k))
    x2 = (4 * tokens * k + 255) // 256 * 256
    assert size == BLAS_BYTES + x2 + 4 * min(n, 8192) * k
    if chunk is not None:
        size = BLAS_BYTES + x2 + 4 * k * chunk
    ws = torch.empty(size, dtype=torch.uint8, device=device)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens + 2 * k)).half()
    xd = x.to(device)
    guard = torch.full((tokens * n + 16,), 47, dtype=torch.float16, device=device)
    out = guard[8:-8].view(tokens, n)
    _q8_run(lib, backend, xd, dc, ds, out, tokens, n, k, ws, size, s)
    again = torch.empty_like(out)
    _q8_run(lib, backend, xd, dc, ds, again, tokens, n, k, ws, size, s)
    g = guard.cpu()
    assert (g[:8] == 47).all() and (g[-8:] == 47).all()
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    stats = _q8_check(out.cpu().float().numpy(), x, codes.numpy(), scales.numpy(), k)
    print(f"flips={stats['flips']} of {stats['count']}", flush=True)


def test_q8_dense_two_term_form_is_exact_at_extreme_scales(backend, device):
    # Subnormal, tiny, ordinary and large (just below 516) scales with the
    # extreme codes: hi + lo must be q*s exactly, so a single-code row times a
    # power-of-two activation returns q*s rounded once to fp16.
    n, k, tokens = 64, 128, 8
    lib = backend._native
    s = torch.cuda.current_stream(device).cuda_stream
    picks = [2.0**-24, 3 * 2.0**-24, 2.0**-15 + 2.0**-24, 1.0009765625 * 2.0**-10, 0.0123, 1.0, 33.97, 515.5]
    scales = torch.tensor(picks * (n * 4 // len(picks)), dtype=torch.float16).view(n, 4)
    codes = torch.zeros(n, 128, dtype=torch.int8)
    rng = np.random.default_rng(3)
    codes[:, :k] = torch.from_numpy(rng.choice([-127, -126, -1, 1, 5, 77, 126, 127], size=(n, k)).astype(np.int8))
    dc, ds = codes.to(device), scales.to(device)
    size = int(lib.venturi_q8_dense_workspace_bytes(tokens, n, k))
    ws = torch.empty(size, dtype=torch.uint8, device=device)
    # Token t selects column 3t (x = 1 there, 0 elsewhere): out[t][j] = fp16(q[j][3t] * s[j][group]).
    x = torch.zeros(tokens, k, dtype=torch.float16)
    for t in range(tokens):
        x[t, 3 * t] = 1.0
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    _q8_run(lib, backend, x.to(device), dc, ds, out, tokens, n, k, ws, size, s)
    want = np.empty((tokens, n), np.float16)
    for t in range(tokens):
        c = 3 * t
        want[t] = (codes[:, c].numpy().astype(np.float64) * scales[:, c // 32].numpy().astype(np.float64)).astype(np.float16)
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint16), want.view(np.uint16))
    # A full random row mix at the same scales meets the contract bound (x is
    # scaled by 2^-10 so that the large-scale rows stay inside the fp16 range).
    codes2, _ = random_q8(n, k, 9)
    dc2 = codes2.to(device)
    xr = (torch.randn(tokens, k, generator=torch.Generator().manual_seed(1)) * 2.0**-10).half()
    _q8_run(lib, backend, xr.to(device), dc2, ds, out, tokens, n, k, ws, size, s)
    w = oracle.q8_unpack(codes2.numpy(), scales.numpy(), k)
    xd = xr.float().numpy().astype(np.float64)
    exact = xd @ w.T
    assert np.abs(exact).max() < 60000
    bound = 0.5 * ulp16(exact) + 2.0**-19 * (np.abs(xd) @ np.abs(w).T)
    assert (np.abs(out.cpu().float().numpy().astype(np.float64) - exact) <= bound).all()


def test_q8_dense_scale_limit(backend, device):
    # A scale of 516 or more puts 127 * s past the fp16 range: the route is
    # refused by the plan (auto stays on the fused GEMM), and the C entry turns
    # that row's outputs into NaN instead of a finite wrong value.
    n, k, tokens = 16, 64, Q8_DENSE_TOKENS
    lib = backend._native
    s = torch.cuda.current_stream(device).cuda_stream
    codes, scales = random_q8(n, k, 5)
    codes[3, :] = 127
    scales[3, :] = 600.0
    resident = backend.upload_linear(Q8RowSplitWeight(codes, scales, k), dtype=torch.float16, device=device)
    assert resident.prepare(tokens=tokens).route == "venturi-q8-mfma"
    with pytest.raises(ValueError, match="516"):
        resident.prepare(tokens=tokens, route="dense")
    dc, ds = codes.to(device), scales.to(device)
    size = int(lib.venturi_q8_dense_workspace_bytes(tokens, n, k))
    ws = torch.empty(size, dtype=torch.uint8, device=device)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(2)).half().to(device)
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    _q8_run(lib, backend, x, dc, ds, out, tokens, n, k, ws, size, s)
    o = out.cpu().float()
    assert torch.isnan(o[:, 3]).all()
    assert torch.isfinite(torch.cat([o[:, :3], o[:, 4:]], 1)).all()


def test_q8_plan_auto_route_is_dense(backend, device):
    n, k = 136, 256
    codes, scales = random_q8(n, k, 8)
    resident = backend.upload_linear(Q8RowSplitWeight(codes, scales, k), dtype=torch.float16, device=device)
    assert resident.prepare(tokens=Q8_DENSE_TOKENS - 1).plan.kernel == "prefill"
    plan = resident.prepare(tokens=Q8_DENSE_TOKENS)
    assert plan.route == "venturi-q8-dense" and plan.workspace_bytes > 0
    x = torch.randn(Q8_DENSE_TOKENS, k, generator=torch.Generator().manual_seed(6)).half()
    out = torch.empty(Q8_DENSE_TOKENS, n, dtype=torch.float16, device=device)
    # Without a workspace (the reference's run(x, out=)) the plan runs the
    # fused matrix-core prefill kernel: the bytes of the mfma route.
    plain = torch.empty_like(out)
    plan.run(x.to(device), out=plain)
    fused = torch.empty_like(out)
    resident.prepare(tokens=Q8_DENSE_TOKENS, route="mfma").run(x.to(device), out=fused)
    assert torch.equal(plain.view(torch.int16), fused.view(torch.int16))
    _q8_check(plain.cpu().float().numpy(), x, codes.numpy(), scales.numpy(), k)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    plan.run(x.to(device), out=out, workspace=ws)
    _q8_check(out.cpu().float().numpy(), x, codes.numpy(), scales.numpy(), k)
    bf = backend.upload_linear(Q8RowSplitWeight(codes, scales, k), dtype=torch.bfloat16, device=device)
    assert bf.prepare(tokens=Q8_DENSE_TOKENS).route == "venturi-q8-exact"


@pytest.mark.parametrize("n,k", [(34816, 5120), (5120, 17408)])
def test_q8_dense_config2_m2048_sampled_rows(backend, device, n, k):
    # The timed prefill shapes: gate+up in four 8192-row chunks and a 2048-row
    # tail, down whole. Sampled rows (chunk edges among them), every token.
    print(f"case q8-dense-config2 n={n} k={k}", flush=True)
    gen = torch.Generator(device=device).manual_seed(n + k + 3)
    w = torch.randn(n, k, generator=gen, device=device) * 0.02
    packed = backend.quantize_q8(w)
    del w
    tokens = 2048
    plan = backend.upload_linear(packed, dtype=torch.float16, device=device).prepare(tokens=tokens)
    assert plan.route == "venturi-q8-dense"
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(7)).half()
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    plan.run(x.to(device), out=out, workspace=ws)
    edges = [r for r in (0, 8191, 8192, 16383, 16384, 32767, 32768, n - 1) if r < n]
    rows = np.unique(np.concatenate([edges, np.random.default_rng(n).choice(n, 24, replace=False)]))
    codes, scales = packed.codes.cpu().numpy()[rows], packed.scales.cpu().numpy()[rows]
    stats = _q8_check(out[:, torch.from_numpy(rows).to(device)].cpu().float().numpy(), x, codes, scales, k)
    print(f"q8-dense config2 n={n} k={k}: max_abs={stats['max_abs']:.3g} flips={stats['flips']} of {stats['count']}",
          flush=True)


def test_q8_dense_rejects_bad_arguments(backend, device):
    lib = backend._native
    s = torch.cuda.current_stream(device).cuda_stream
    n, k, tokens = 16, 128, 4
    x = torch.zeros(tokens, k, dtype=torch.float16, device=device)
    c = torch.zeros(n, k, dtype=torch.int8, device=device)
    sc = torch.zeros(n, k // 32, dtype=torch.float16, device=device)
    o = torch.empty(tokens, n, dtype=torch.float16, device=device)
    size = int(lib.venturi_q8_dense_workspace_bytes(tokens, n, k))
    ws = torch.empty(size + 256, dtype=torch.uint8, device=device)
    args = (x.data_ptr(), c.data_ptr(), sc.data_ptr(), o.data_ptr())
    assert lib.venturi_q8_dense_run(*args, tokens, n, k, k, 1, ws.data_ptr(), size, s) == -1
    assert "fp16" in lib.error()
    assert lib.venturi_q8_dense_run(*args, tokens, n, k, 256, 0, ws.data_ptr(), size, s) == -1
    assert lib.venturi_q8_dense_run(*args, tokens, 12, k, k, 0, ws.data_ptr(), size, s) == -1
    assert "n % 8" in lib.error()
    assert lib.venturi_q8_dense_run(*args, tokens, n, k, k, 0, ws.data_ptr(), BLAS_BYTES, s) == -1
    assert "16-row chunk" in lib.error()
    assert lib.venturi_q8_dense_run(*args, tokens, n, k, k, 0, ws.data_ptr() + 16, size, s) == -1
    assert "256-byte" in lib.error()
    assert lib.venturi_q8_dense_workspace_bytes(70000, n, k) == 0
    torch.cuda.synchronize(device)


# ---------------------------------------------------------------------------
# The dense bridge (venturi_dense_run, blocks.cu:674-713) on hipBLASLt.

_TORCH = {0: torch.float16, 1: torch.bfloat16, 2: torch.float32}


@pytest.mark.parametrize("dtype", [0, 1, 2])
@pytest.mark.parametrize("tokens,n,k,ws_mib", [
    (1, 64, 8, 4), (37, 136, 1000, 4), (300, 64, 5120, 4), (2048, 1024, 512, 4),
    # odd K (the reference bridge takes any k > 0) and a workspace above the
    # 32 MiB share, where the heuristic may pick split-K kernels
    (37, 136, 1001, 64), (5, 24, 13, 64), (2048, 1024, 512, 64), (300, 64, 5120, 64),
])
def test_dense_bridge(backend, device, dtype, tokens, n, k, ws_mib):
    # out = x w^T in the plan's dtype with fp32 arithmetic: within half an ulp
    # of the output type plus 2^-19 (2^-17 for fp32 data) of the absolute
    # product of FP64, and the same bits on a second run.
    print(f"case dense-bridge dtype={dtype} tokens={tokens} n={n} k={k} workspace={ws_mib} MiB", flush=True)
    lib = backend._native
    s = torch.cuda.current_stream(device).cuda_stream
    t = _TORCH[dtype]
    gen = torch.Generator().manual_seed(tokens + n + k + dtype)
    x = torch.randn(tokens, k, generator=gen).to(t)
    w = (torch.randn(n, k, generator=gen) * 0.05).to(t)
    plan = lib.venturi_dense_create(dtype)
    assert plan
    try:
        ws = torch.empty(ws_mib * 2**20, dtype=torch.uint8, device=device)
        xd, wd = x.to(device), w.to(device)
        out = torch.empty(tokens, n, dtype=t, device=device)
        again = torch.empty_like(out)
        for o in (out, again):
            backend._check(lib.venturi_dense_run(plan, xd.data_ptr(), wd.data_ptr(), o.data_ptr(), tokens, n, k,
                                                 ws.data_ptr(), ws.numel(), s))
        assert torch.equal(out.view(torch.uint8), again.view(torch.uint8))
        x64, w64 = x.double().numpy(), w.double().numpy()
        exact = x64 @ w64.T
        mag = np.abs(x64) @ np.abs(w64).T
        half_ulp = {0: 0.5 * ulp16(exact), 1: 2.0 ** (np.floor(np.log2(np.maximum(np.abs(exact), 2.0**-126))) - 8),
                    2: np.abs(exact) * 2.0**-24}[dtype]
        bound = half_ulp + (2.0**-17 if dtype == 2 else 2.0**-19) * mag
        got = out.cpu().double().numpy()
        assert (np.abs(got - exact) <= bound).all()
        assert lib.venturi_dense_run(plan, xd.data_ptr(), wd.data_ptr(), out.data_ptr(), tokens, n, k, None, 0, s) == -1
        assert "null Linear operand" in lib.error()
        assert lib.venturi_dense_run(plan, xd.data_ptr(), wd.data_ptr(), out.data_ptr(), tokens, n, 0,
                                     ws.data_ptr(), ws.numel(), s) == -1
        assert lib.venturi_dense_run(plan, xd.data_ptr() + 2, wd.data_ptr(), out.data_ptr(), tokens, n, k,
                                     ws.data_ptr(), ws.numel(), s) == -1
        assert "16-byte" in lib.error()
    finally:
        lib.venturi_dense_destroy(plan)


def test_dense_chunks_under_graph_capture(backend, device):
    # A chunked run (decode, GEMM, decode, ...) captured in a HIP graph after an
    # eager run has created the hipBLASLt state: three replays give the eager bits.
    n, k, tokens, nbits = 200, 264, 37, 4
    lib = backend._native
    packed, high, scales = _planes(n, k, nbits, 17)
    padded = packed.shape[1] * 2
    dc, dh, ds = _device_planes(packed, high, scales, nbits, device)
    size = BLAS_BYTES + 2 * k * 48  # 48-row chunks: five
    ws = torch.empty(size, dtype=torch.uint8, device=device)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(5)).half().to(device)
    want = torch.empty(tokens, n, dtype=torch.float16, device=device)
    out = torch.empty_like(want)

    def run(o):
        _run(lib, backend, x, dc, dh, ds, o, tokens, n, k, padded, nbits, ws, size,
             torch.cuda.current_stream(device).cuda_stream)

    run(want)
    torch.cuda.synchronize(device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(out)
    for _ in range(3):
        out.fill_(7.0)
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
