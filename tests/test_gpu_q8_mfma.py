"""Q8 A16 projection on matrix cores: agreement with the canonical order and FP64.

The MFMA route sums each 32-column group on the matrix core and applies the
group scale in fp32, so it differs from the canonical order only by fp32
association. Tolerances (written here, not relaxed silently):
  * vs FP64 exact: |y - exact| <= 0.5 ulp_fp16(exact) + 2^-19 * sum_k |x_k w_k|
  * vs the canonical-order oracle (helpers.assert_free_order): every output
    within max(2e-3, 1 fp16 ulp of the oracle value), rel-L2 <= 1e-3, at most
    2% of the outputs differing at all and at most 1% by more than 2e-3.
    Above |y| = 4 a single flip is 3.9e-3: the one stated deviation from the
    2e-3 gate.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import agreement, assert_free_order, bits, random_q8, ulp16
from venturi_amd import Q8RowSplitWeight

pytestmark = pytest.mark.gpu


def check(out, x, codes, scales, k):
    got = out.cpu().float().numpy().astype(np.float64)
    w = oracle.q8_unpack(codes, scales, k)
    xd = x.float().numpy().astype(np.float64)
    exact = xd @ w.T
    bound = 0.5 * ulp16(exact) + 2.0**-19 * (np.abs(xd) @ np.abs(w).T)
    assert (np.abs(got - exact) <= bound).all()
    stats = agreement(got, oracle.q8_linear(bits(x), codes, scales, k))
    assert_free_order(stats)
    return stats["flips"]


@pytest.mark.parametrize("shape", [(1, 64), (7, 72), (33, 136), (16, 256), (257, 5120), (100, 1000), (16400, 136), (40, 16392)])
@pytest.mark.parametrize("tokens", [1, 2, 3, 4, 8, 13, 16, 17, 32])
def test_mfma_tolerances_tails_and_guards(backend, device, shape, tokens):
    n, k = shape
    print(f"case q8-mfma n={n} k={k} tokens={tokens}", flush=True)
    codes, scales = random_q8(n, k, 77 + n + tokens)
    weight = Q8RowSplitWeight(codes, scales, k)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens)).half()
    plan = backend.upload_linear(weight, dtype=torch.float16, device=device).prepare(tokens=tokens, route="mfma")
    assert plan.route == "venturi-q8-mfma"
    guard = torch.full((tokens * n + 2,), 47, dtype=torch.float16, device=device)
    out = guard[1:-1].view(tokens, n)
    plan.run(x.to(device), out=out)
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    flips = check(out, x, codes.numpy(), scales.numpy(), k)
    print(f"flips={flips} of {tokens * n}", flush=True)


@pytest.mark.parametrize("shape", [(1, 64), (7, 72), (33, 136), (129, 1000), (257, 5120), (300, 2056)])
@pytest.mark.parametrize("tokens", [33, 64, 100, 256, 300])
def test_prefill_gemm_tolerances_tails_and_guards(backend, device, shape, tokens):
    # venturi_q8_prefill_run: the same contract as the decode kernels (exact
    # group dots on matrix cores, fp32 group scaling), at small ragged shapes.
    n, k = shape
    print(f"case q8-prefill n={n} k={k} tokens={tokens}", flush=True)
    codes, scales = random_q8(n, k, 901 + n + tokens)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens + 3)).half()
    plan = backend.upload_linear(Q8RowSplitWeight(codes, scales, k), dtype=torch.float16, device=device).prepare(
        tokens=tokens)
    assert plan.route == "venturi-q8-mfma" and plan.plan.kernel == "prefill"
    guard = torch.full((tokens * n + 2,), 47, dtype=torch.float16, device=device)
    out = guard[1:-1].view(tokens, n)
    plan.run(x.to(device), out=out)
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    flips = check(out, x, codes.numpy(), scales.numpy(), k)
    print(f"flips={flips} of {tokens * n}", flush=True)


@pytest.mark.parametrize("n,k", [(7168, 5120), (5120, 17408), (34816, 5120)])
def test_prefill_config2_m2048_sampled_rows(backend, device, n, k):
    # The three row counts take the three tilings (128 x 224, 128 x 160 and
    # 256 x 128 tiles on a 256-CU part).
    gen = torch.Generator(device=device).manual_seed(n + k + 1)
    w = torch.randn(n, k, generator=gen, device=device) * 0.02
    packed = backend.quantize_q8(w)
    del w
    tokens = 2048
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(5)).half()
    # The fused matrix-core GEMM (auto takes the dense route at this size; it is tested in test_gpu_dense.py).
    plan = backend.upload_linear(packed, dtype=torch.float16, device=device).prepare(tokens=tokens, route="mfma")
    assert plan.plan.kernel == "prefill"
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    plan.run(x.to(device), out=out)
    rows = np.sort(np.random.default_rng(n).choice(n, 32, replace=False))
    codes, scales = packed.codes.cpu().numpy()[rows], packed.scales.cpu().numpy()[rows]
    flips = check(out[:, rows], x, codes, scales, k)
    print(f"prefill config2 n={n} k={k}: flips={flips} of {tokens * 32}", flush=True)


@pytest.mark.parametrize("n,k", [(7168, 5120), (5120, 6144), (34816, 5120), (5120, 17408)])
@pytest.mark.parametrize("tokens", [1, 4, 8, 16, 32])
def test_mfma_config2_sampled_rows(backend, device, n, k, tokens):
    gen = torch.Generator(device=device).manual_seed(n + k)
    w = torch.randn(n, k, generator=gen, device=device) * 0.02
    packed = backend.quantize_q8(w)
    del w
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens)).half()
    plan = backend.upload_linear(packed, dtype=torch.float16, device=device).prepare(tokens=tokens, route="mfma")
    out = torch.empty(tokens, n, dtype=torch.float16, device=device)
    plan.run(x.to(device), out=out)
    rows = np.sort(np.random.default_rng(n).choice(n, 256, replace=False))
    codes, scales = packed.codes.cpu().numpy()[rows], packed.scales.cpu().numpy()[rows]
    flips = check(out[:, rows], x, codes, scales, k)
    print(f"config2 n={n} k={k} tokens={tokens}: flips={flips} of {tokens * 256}", flush=True)


def test_mfma_route_admission(backend, device):
    codes, scales = random_q8(8, 65, 1)
    resident = backend.upload_linear(Q8RowSplitWeight(codes, scales, 65), dtype=torch.float16, device=device)
    with pytest.raises(ValueError, match="MFMA"):
        resident.prepare(tokens=1, route="mfma")  # k % 8 != 0
    assert resident.prepare(tokens=8).route == "venturi-q8-exact"
    codes, scales = random_q8(8, 64, 1)
    resident = backend.upload_linear(Q8RowSplitWeight(codes, scales, 64), dtype=torch.float16, device=device)
    assert resident.prepare(tokens=1).route == "venturi-q8-mfma"
    assert resident.prepare(tokens=1, route="exact").route == "venturi-q8-exact"
    assert resident.prepare(tokens=2).route == "venturi-q8-mfma"
    assert resident.prepare(tokens=32).route == "venturi-q8-mfma"
    assert resident.prepare(tokens=32).plan.kernel == "mfma"
    assert resident.prepare(tokens=33).route == "venturi-q8-mfma"  # prefill GEMM above 32 tokens
    assert resident.prepare(tokens=33).plan.kernel == "prefill"
    assert resident.prepare(tokens=4096).plan.slots is None
    assert resident.prepare(tokens=4096).route == "venturi-q8-dense"  # prefill from 2048 tokens
    bf = backend.upload_linear(Q8RowSplitWeight(codes, scales, 64), dtype=torch.bfloat16, device=device)
    assert bf.prepare(tokens=8).route == "venturi-q8-exact"


@pytest.mark.parametrize("shape", [(16, 64), (34, 136), (200, 1000), (16400, 136), (18, 16392), (5000, 8200)])
@pytest.mark.parametrize("tokens", [1, 3, 4, 8, 13, 16, 32])
def test_fused_swiglu_equals_projection_then_silu_mul(backend, device, shape, tokens):
    # The fused epilogue must give the bytes of the mfma projection followed by
    # venturi_silu_mul_run (every row's dot is computed by the same MFMA sequence
    # in both tilings). Shapes cover an odd intermediate size (17), >= 1024 paired
    # blocks, K >= 16384 (the staged-activation kernels) and 313 blocks of 130
    # chunks (K split over two workgroups, at one token too).
    n, k = shape
    print(f"case q8-swiglu n={n} k={k} tokens={tokens}", flush=True)
    codes, scales = random_q8(n, k, 311 + n + tokens)
    resident = backend.upload_linear(Q8RowSplitWeight(codes, scales, k), dtype=torch.float16, device=device)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens + k)).half().to(device)
    gate_up = torch.empty(tokens, n, dtype=torch.float16, device=device)
    resident.prepare(tokens=tokens, route="mfma").run(x, out=gate_up)
    want = torch.empty(tokens, n // 2, dtype=torch.float16, device=device)
    lib = backend._native
    backend._check(lib.venturi_silu_mul_run(gate_up.data_ptr(), want.data_ptr(), tokens, n // 2, 0,
                                            torch.cuda.current_stream(device).cuda_stream))
    plan = resident.prepare_swiglu(tokens=tokens)
    assert plan.route == "venturi-q8-mfma-swiglu" and plan.out_features == n // 2
    guard = torch.full((tokens * (n // 2) + 2,), 47, dtype=torch.float16, device=device)
    out = guard[1:-1].view(tokens, n // 2)
    plan.run(x, out=out)
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))


def test_fused_swiglu_admission(backend, device):
    codes, scales = random_q8(6, 64, 3)
    bf = backend.upload_linear(Q8RowSplitWeight(codes, scales, 64), dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="SwiGLU"):
        bf.prepare_swiglu(tokens=1)
    codes, scales = random_q8(7, 64, 3)
    odd = backend.upload_linear(Q8RowSplitWeight(codes, scales, 64), dtype=torch.float16, device=device)
    with pytest.raises(ValueError, match="even row count"):
        odd.prepare_swiglu(tokens=1)


SLOT_IDLE = 0x7F8000017F800001


@pytest.mark.parametrize("n,k,tokens", [(5120, 6144, 4), (7168, 5120, 32), (200, 1000, 13), (16, 64, 2), (100, 200, 24),
                                          (5120, 17408, 1), (4200, 8192, 1), (4100, 8200, 1)])
def test_split_k_deterministic_idle_slots_and_graph_replays(backend, device, n, k, tokens):
    # Shapes whose launch splits K over two workgroups that exchange halves
    # through the plan's slots. Two runs give the same bytes, every slot is idle
    # afterwards, and HIP-graph replays (eager work and synchronisation between
    # them) match the eager result each time.
    print(f"case q8-split n={n} k={k} tokens={tokens}", flush=True)
    codes, scales = random_q8(n, k, 5 + n + tokens)
    resident = backend.upload_linear(Q8RowSplitWeight(codes, scales, k), dtype=torch.float16, device=device)
    plan = resident.prepare(tokens=tokens, route="mfma")
    slots = plan.plan.slots
    assert slots is not None and slots.numel() == tokens * ((n + 15) // 16) * 64
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(n + tokens)).half()
    xd = x.to(device)
    first = torch.empty(tokens, n, dtype=torch.float16, device=device)
    second = torch.empty_like(first)
    plan.run(xd, out=first)
    plan.run(xd, out=second)
    torch.cuda.synchronize(device)
    assert torch.equal(first.view(torch.int16), second.view(torch.int16))
    assert bool((slots.view(torch.int64) == SLOT_IDLE).all())
    if n * k <= 40_000_000:
        check(first, x, codes.numpy(), scales.numpy(), k)
    replayed = torch.full_like(first, 3.0)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run(xd, out=replayed)
    for i in range(3):
        replayed.fill_(3.0)
        graph.replay()
        torch.cuda.synchronize(device)
        assert torch.equal(replayed.view(torch.int16), first.view(torch.int16)), f"replay {i}"
        plan.run(xd, out=second)  # eager work between replays
        torch.cuda.synchronize(device)
        assert torch.equal(second.view(torch.int16), first.view(torch.int16))
    assert bool((slots.view(torch.int64) == SLOT_IDLE).all())


def test_unsplit_shapes_own_no_slots(backend, device):
    codes, scales = random_q8(7168, 128, 9)
    resident = backend.upload_linear(Q8RowSplitWeight(codes, scales, 128), dtype=torch.float16, device=device)
    assert resident.prepare(tokens=1, route="mfma").plan.slots is None
    assert resident.prepare(tokens=8, route="mfma").plan.slots is None
    assert resident.prepare(tokens=24, route="mfma").plan.slots is not None


@pytest.mark.parametrize("shape", [(16, 64), (37, 200), (100, 1000), (300, 4104), (64, 17408)])
@pytest.mark.parametrize("tokens", [1, 2, 5, 8, 11, 16])
def test_row_major_mfma_decode(backend, device, shape, tokens):
    # venturi_q8_gemm_run (the matrix-core decode over the row-major planes, an
    # exported extension): the FP64 bound and the free-order tolerance against
    # the canonical-order oracle, with k % 128 != 0 tails and output guards.
    n, k = shape
    print(f"case q8-gemm-run n={n} k={k} tokens={tokens}", flush=True)
    codes, scales = random_q8(n, k, 4000 + n + tokens)
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(tokens + 7 * k)).half()
    dc, ds = codes.to(device), scales.to(device)
    guard = torch.full((tokens * n + 2,), 47, dtype=torch.float16, device=device)
    out = guard[1:-1].view(tokens, n)
    backend._check(backend._native.venturi_q8_gemm_run(x.to(device).data_ptr(), dc.data_ptr(), ds.data_ptr(),
                                                       out.data_ptr(), tokens, n, k, codes.shape[1], 0,
                                                       torch.cuda.current_stream(device).cuda_stream))
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    flips = check(out, x, codes.numpy(), scales.numpy(), k)
    print(f"flips={flips} of {tokens * n}", flush=True)
