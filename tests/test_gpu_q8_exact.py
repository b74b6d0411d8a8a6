"""Q8 A16 projection (exact route) against the oracle's canonical-order bytes."""

import numpy as np
import pytest
import torch

import oracle
from helpers import bits, guarded_out, near_tie_matrix, random_q8
from venturi_amd import Q8RowSplitWeight

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1, 1), (7, 65), (33, 129), (7, 256), (33, 512), (257, 5120)])
@pytest.mark.parametrize("tokens", [1, 2, 3, 4, 5, 7, 8, 9, 16, 26, 32])
def test_exact_bytes_tails_and_guards(backend, device, dtype, shape, tokens):
    # Shapes/tokens of the reference's byte-equality test (test_q8_tiling.py:222-248).
    n, k = shape
    print(f"case q8-exact n={n} k={k} tokens={tokens} dtype={dtype}", flush=True)
    codes, scales = random_q8(n, k, 9367 + n + tokens)
    weight = Q8RowSplitWeight(codes, scales, k)
    gen = torch.Generator().manual_seed(11 + tokens)
    x = torch.randn(tokens, k, generator=gen).to(dtype)
    resident = backend.upload_linear(weight, dtype=dtype, device=device)
    plan = resident.prepare(tokens=tokens, route="exact")
    assert "q8" in plan.route
    guard, out = guarded_out(tokens, n, dtype, device)
    plan.run(x.to(device), out=out)
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    expected = oracle.q8_linear(bits(x), codes.numpy(), scales.numpy(), k, dtype=0 if dtype == torch.float16 else 1)
    np.testing.assert_array_equal(bits(out), expected)


def test_config1_decode_bitexact(backend, device):
    # Config 1: W ~ N(0, 0.02) [4096, 4096] seed 0, x ~ N(0, 1) [1, 4096].
    w = torch.randn(4096, 4096, generator=torch.Generator().manual_seed(0)) * 0.02
    weight = Q8RowSplitWeight.from_dense(w.half())
    x = torch.randn(1, 4096, generator=torch.Generator().manual_seed(1)).half()
    resident = backend.upload_linear(weight, dtype=torch.float16, device=device)
    out = torch.empty(1, 4096, dtype=torch.float16, device=device)
    resident.prepare(tokens=1, route="exact").run(x.to(device), out=out)
    expected = oracle.q8_linear(bits(x), weight.codes.numpy(), weight.scales.numpy(), 4096)
    np.testing.assert_array_equal(bits(out), expected)
    # FP64 closed form: the fp32 result rounds within one fp16 ulp of the exact value.
    exact = x.double() @ weight.dequantize_reference().T
    err = (out.cpu().double() - exact).abs()
    ulp = torch.finfo(torch.float16).eps * exact.abs().clamp_min(2**-14)
    assert bool((err <= ulp).all())


@pytest.mark.parametrize("n,k", [(7168, 5120), (5120, 6144), (34816, 5120), (5120, 17408)])
@pytest.mark.parametrize("tokens", [1, 4, 8, 16, 32])
def test_config2_shapes_sampled_rows(backend, device, n, k, tokens):
    # Full-size launch; the oracle checks a seeded sample of 256 rows.
    print(f"case q8-config2 n={n} k={k} tokens={tokens}", flush=True)
    gen = torch.Generator(device=device).manual_seed(n + k)
    w = torch.randn(n, k, generator=gen, device=device) * 0.02
    codes, scales = oracle.q8_pack(w.cpu().numpy())
    del w
    weight = Q8RowSplitWeight(torch.from_numpy(codes), torch.from_numpy(scales), k)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens)).half()
    resident = backend.upload_linear(weight, dtype=torch.float16, device=device)
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    resident.prepare(tokens=tokens, route="exact").run(x.to(device), out=out)
    rows = np.sort(np.random.default_rng(n).choice(n, 256, replace=False))
    expected = oracle.q8_linear(bits(x), codes[rows], scales[rows], k)
    np.testing.assert_array_equal(bits(out)[:, rows], expected)


@pytest.mark.parametrize("tokens", [1, 2, 3, 17])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_exact_wide_rows(backend, device, tokens, dtype):
    # k = 45 000: the whole activation tile of one or two tokens exceeds LDS,
    # so every token count runs the slab form (K walked in staged slabs), with
    # a ragged last chunk and row count.
    n, k = 37, 45000
    print(f"case q8-exact-wide n={n} k={k} tokens={tokens} dtype={dtype}", flush=True)
    codes, scales = random_q8(n, k, 77 + tokens)
    weight = Q8RowSplitWeight(codes, scales, k)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(5 + tokens)).to(dtype)
    resident = backend.upload_linear(weight, dtype=dtype, device=device)
    guard, out = guarded_out(tokens, n, dtype, device)
    resident.prepare(tokens=tokens, route="exact").run(x.to(device), out=out)
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    expected = oracle.q8_linear(bits(x), codes.numpy(), scales.numpy(), k, dtype=0 if dtype == torch.float16 else 1)
    np.testing.assert_array_equal(bits(out), expected)


def test_impulse_last_column_and_nonfinite(backend, device):
    # Impulse at the last valid column (test_quantlinear_cuda.py:17-49 pattern).
    for k in (255, 257, 511, 512):
        n = 19
        padded = (k + 127) // 128 * 128
        codes = torch.zeros(n, padded, dtype=torch.int8)
        codes[:, k - 1] = 1
        scales = torch.ones(n, padded // 32, dtype=torch.float16)
        resident = backend.upload_linear(Q8RowSplitWeight(codes, scales, k), dtype=torch.float16, device=device)
        x = torch.zeros(4, k, dtype=torch.float16, device=device)
        x[:, -1] = 1
        out = torch.full((4, n), float("nan"), dtype=torch.float16, device=device)
        resident.prepare(tokens=4, route="exact").run(x, out=out)
        assert torch.equal(out.cpu(), torch.ones(4, n, dtype=torch.float16))
        x[0, 0] = float("inf")
        resident.prepare(tokens=4, route="exact").run(x, out=out)
        assert not torch.isfinite(out[0]).any() or bool(torch.isnan(out[0]).all())


@pytest.mark.parametrize("k", [65, 136, 5120])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("offset", [0, 1])
def test_embedding_run_rows(backend, device, k, dtype, offset):
    # venturi_q8_embedding_run through the C ABI: rows code * scale rounded once,
    # ids outside [0, vocab) give zero rows (blocks.cu:293-304); the 16-byte path
    # (k % 8 == 0, aligned output) and the element path (k = 65, or an output one
    # element past an aligned address), 8-byte aligned codes and codes one byte off.
    vocab = 37
    codes, scales = random_q8(vocab, k, 40 + k)
    planes = codes.to(device)
    padded = planes.shape[1]
    store = torch.zeros(vocab * padded + 8, dtype=torch.int8, device=device)
    store[offset:offset + vocab * padded] = planes.reshape(-1)
    dsc = scales.to(device)
    ids = torch.tensor([3, 36, 0, -1, 37, 17, 3], dtype=torch.int64, device=device)
    buf = torch.full((ids.numel() * k + 8,), 7.0, dtype=dtype, device=device)
    out = buf[offset:offset + ids.numel() * k]
    lib = backend._native
    dt = 0 if dtype == torch.float16 else 1
    s = torch.cuda.current_stream(device).cuda_stream
    backend._check(lib.venturi_q8_embedding_run(store.data_ptr() + offset, dsc.data_ptr(), ids.data_ptr(),
                                                out.data_ptr(), ids.numel(), vocab, k, padded, dt, s))
    dense = (codes.float() * scales.float().repeat_interleave(32, -1))[:, :k]
    want = torch.stack([dense[i] if 0 <= i < vocab else torch.zeros(k) for i in ids.tolist()]).to(dtype)
    assert torch.equal(out.cpu().view(ids.numel(), k), want)
    tail = buf.cpu()[offset + ids.numel() * k:]
    assert (tail == 7.0).all() and (buf.cpu()[:offset] == 7.0).all()


def test_embedding_matches_decode(backend, device):
    codes, scales = random_q8(31, 65, 18)
    weight = Q8RowSplitWeight(codes, scales, 65)
    for dtype in (torch.float16, torch.bfloat16):
        resident = backend.upload_linear(weight, dtype=dtype, device=device)
        lookup = resident.prepare_embedding([1, 30, 0])
        out = torch.empty(3, 65, dtype=dtype, device=device)
        lookup.run(out=out)
        expected = (codes.float() * scales.float().repeat_interleave(32, -1))[[1, 30, 0], :65].to(dtype)
        assert torch.equal(out.cpu(), expected)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(11, 1), (11, 31), (7, 65), (5, 129), (9, 136), (64, 4096)])
def test_device_pack_matches_from_dense(backend, device, dtype, shape):
    gen = torch.Generator().manual_seed(38 + shape[1])
    src = (torch.randn(*shape, generator=gen) * 0.01).to(dtype)
    src[0].zero_()
    if shape[1] > 40:
        src[1, 3] = 1e-30 if dtype != torch.float16 else 0  # underflowing group scale
    got = backend.quantize_q8(src.to(device))
    want = Q8RowSplitWeight.from_dense(src)
    assert torch.equal(got.codes.cpu(), want.codes)
    assert torch.equal(got.scales.cpu().view(torch.int16), want.scales.view(torch.int16))
    with pytest.raises(ValueError):
        bad = src.clone().to(device)
        bad[0, 0] = float("nan")
        backend.quantize_q8(bad)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("trim", [0, 5])
def test_device_pack_near_ties(backend, device, dtype, trim):
    # Quotients x / scale on and within three fp32 ulps of half-integers, under
    # normal and subnormal fp16 scales: the packer's reciprocal estimate leaves
    # these to the IEEE division, and the codes equal from_dense's (ties to even).
    print(f"case q8-pack-ties {dtype} trim={trim}", flush=True)
    src = torch.from_numpy(near_tie_matrix(127, 32, 64, 4, 17 + trim))[:, : 128 - trim].contiguous().to(dtype)
    got = backend.quantize_q8(src.to(device))
    want = Q8RowSplitWeight.from_dense(src)
    assert torch.equal(got.codes.cpu(), want.codes)
    assert torch.equal(got.scales.cpu().view(torch.int16), want.scales.view(torch.int16))


@pytest.mark.parametrize("offset", [1, 2, 3, 4, 5, 8, 17])
@pytest.mark.parametrize("shape,tokens", [((7, 65), 1), ((33, 300), 3), ((70, 1024), 5), ((5, 5120), 1), ((40, 2056), 17)])
def test_head_run_accepts_unaligned_codes(backend, device, offset, shape, tokens):
    # venturi_q8_head_run takes any code pointer, as the reference's does
    # (blocks.cu:935-948): a plane that starts `offset` bytes into a buffer (a
    # row-offset view) gives the canonical bytes. The plane ends exactly at the
    # end of its buffer, so no read may pass it.
    n, k = shape
    print(f"case q8-unaligned n={n} k={k} tokens={tokens} offset={offset}", flush=True)
    codes, scales = random_q8(n, k, 31 * offset + n)
    padded = codes.shape[1]
    storage = torch.zeros(offset + n * padded, dtype=torch.int8, device=device)
    plane = storage[offset:]
    plane.copy_(codes.view(-1).to(device))
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(offset)).half()
    ds = scales.to(device)
    guard, out = guarded_out(tokens, n, torch.float16, device)
    backend._check(backend._native.venturi_q8_head_run(x.to(device).data_ptr(), plane.data_ptr(), ds.data_ptr(),
                                                       out.data_ptr(), tokens, n, k, padded, 0,
                                                       torch.cuda.current_stream(device).cuda_stream))
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    np.testing.assert_array_equal(bits(out), oracle.q8_linear(bits(x), codes.numpy(), scales.numpy(), k))
