"""The Q8 vocabulary head and embedding at the model's shape, and the tiled residency.

The head is the largest decode projection: vocab 248 320 x hidden 5120
(tests/fixtures/qwen3_5_27b/config.json in the reference; 1.35 GB of Q8 per
token). It is held once, in the tiled layout (``residency="tiled"``), and run
on the matrix-core route at M in {1, 4}: sampled rows against the
canonical-order oracle (helpers.assert_free_order). At a smaller shape a tiled
resident's outputs equal a row-major resident's (same kernel, same bytes), and
the kernels that need row-major planes refuse it. The embedding gathers rows
of the head's planes (closed form code * scale).
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import agreement, assert_free_order, bits, random_q8
from venturi_amd import Q8RowSplitWeight

pytestmark = pytest.mark.gpu

VOCAB, HIDDEN = 248320, 5120


@pytest.fixture(scope="module")
def head(backend, device):
    gen = torch.Generator(device=device).manual_seed(248320)
    packed = backend.quantize_q8(torch.randn(VOCAB, HIDDEN, generator=gen, device=device) * 0.02)
    torch.cuda.empty_cache()
    return packed


@pytest.mark.parametrize("tokens", [1, 4])
def test_head_at_vocab_248320_tiled_residency(backend, device, head, tokens):
    print(f"case vocab-head tokens={tokens}", flush=True)
    resident = backend.upload_linear(head, dtype=torch.float16, device=device, residency="tiled")
    padded = (HIDDEN + 127) // 128 * 128
    blocks = (VOCAB + 15) // 16
    assert resident.storage_nbytes == blocks * 16 * (padded + padded // 32 * 2)  # one tiled copy, no row-major
    plan = resident.prepare(tokens=tokens)
    assert plan.route == "venturi-q8-mfma"
    x = torch.randn(tokens, HIDDEN, generator=torch.Generator().manual_seed(tokens)).half()
    out = torch.empty(tokens, VOCAB, dtype=torch.float16, device=device)
    plan.run(x.to(device), out=out)
    rows = np.sort(np.random.default_rng(tokens).choice(VOCAB, 192, replace=False))
    index = torch.as_tensor(rows, device=device)
    codes, scales = head.codes[index].cpu().numpy(), head.scales[index].cpu().numpy()
    stats = agreement(bits(out)[:, rows], oracle.q8_linear(bits(x), codes, scales, HIDDEN))
    assert_free_order(stats)
    print(f"vocab head tokens={tokens}: {stats}", flush=True)
    del resident, plan
    torch.cuda.empty_cache()


def test_tiled_residency_equals_row_major_and_refuses_other_kernels(backend, device):
    codes, scales = random_q8(1000, 1024, 5)
    weight = Q8RowSplitWeight(codes, scales, 1024)
    full = backend.upload_linear(weight, dtype=torch.float16, device=device)
    tiled = backend.upload_linear(weight, dtype=torch.float16, device=device, residency="tiled")
    assert tiled.storage_nbytes == pytest.approx(full.storage_nbytes, rel=0.01)  # one copy each, 1.06 B per weight
    for tokens in (1, 3, 16, 32):
        x = torch.randn(tokens, 1024, generator=torch.Generator().manual_seed(tokens)).half().to(device)
        a = torch.empty(tokens, 1000, dtype=torch.float16, device=device)
        b = torch.empty_like(a)
        full.prepare(tokens=tokens, route="mfma").run(x, out=a)
        tiled.prepare(tokens=tokens).run(x, out=b)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    with pytest.raises(ValueError, match="only tiled planes"):
        tiled.prepare(tokens=1, route="exact")
    with pytest.raises(ValueError, match="only tiled planes"):
        tiled.prepare(tokens=33)
    with pytest.raises(ValueError, match="only tiled planes"):
        tiled.prepare_embedding([0, 1])
    with pytest.raises(ValueError, match="only tiled planes"):
        tiled.prepare_swiglu(tokens=1)
    from venturi_amd import prepare_q8_dp4a

    with pytest.raises(ValueError, match="only tiled planes"):
        prepare_q8_dp4a(tiled, tokens=4, residual_compensation=False)
    with pytest.raises(ValueError, match="residency"):
        backend.upload_linear(weight, dtype=torch.float16, device=device, residency="columns")
    with pytest.raises(ValueError, match="matrix-core route"):
        backend.upload_linear(weight, dtype=torch.bfloat16, device=device, residency="tiled")


def test_tiled_paired_residency_runs_swiglu(backend, device):
    codes, scales = random_q8(2 * 136, 512, 6)
    weight = Q8RowSplitWeight(codes, scales, 512)
    full = backend.upload_linear(weight, dtype=torch.float16, device=device)
    paired = backend.upload_linear(weight, dtype=torch.float16, device=device, residency="tiled-paired")
    for tokens in (1, 8, 32):
        x = torch.randn(tokens, 512, generator=torch.Generator().manual_seed(tokens)).half().to(device)
        a = torch.empty(tokens, 136, dtype=torch.float16, device=device)
        b = torch.empty_like(a)
        full.prepare_swiglu(tokens=tokens).run(x, out=a)
        paired.prepare_swiglu(tokens=tokens).run(x, out=b)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    with pytest.raises(ValueError, match="only tiled planes"):
        paired.prepare(tokens=1)


def test_embedding_rows_at_vocab_248320(backend, device, head):
    resident = backend.upload_linear(head, dtype=torch.float16, device=device)
    ids = [int(i) for i in np.random.default_rng(9).choice(VOCAB, 64, replace=False)] + [VOCAB - 1, 0]
    out = torch.empty(len(ids), HIDDEN, dtype=torch.float16, device=device)
    resident.prepare_embedding(ids).run(out=out)
    index = torch.as_tensor(ids, device=device)
    want = oracle.q8_unpack(head.codes[index].cpu().numpy(), head.scales[index].cpu().numpy(), HIDDEN)
    np.testing.assert_array_equal(out.cpu().numpy(), want.astype(np.float16))
    del resident
    torch.cuda.empty_cache()
