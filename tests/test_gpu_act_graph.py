"""Elementwise SwiGLU / add (blocks.cu:56-86, 741-750) and HIP-graph replay of a
projection chain.

SwiGLU tolerance: the device exp and numpy's float32 exp are not bit-pinned
against CUDA's, so outputs must be within 1 fp16 ulp of the oracle (the count
of differing outputs is printed); add is bit-exact. Graph replays must equal
the eager result bit for bit, on every replay, with eager work in between.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import bits
from venturi_amd import Q8RowSplitWeight

pytestmark = pytest.mark.gpu


def ulp16(v):
    v = np.abs(v.astype(np.float64))
    return 2.0 ** (np.floor(np.log2(np.maximum(v, 2.0**-14))) - 10)


def test_swiglu_add_and_fused_layout(backend, device):
    gen = torch.Generator().manual_seed(5)
    a = (torch.randn(4, 3000, generator=gen) * 6).half()
    a[0, :8] = torch.tensor([-30.0, -17.0, -12.0, 0.0, -0.0, 11.0, 65504.0, -65504.0]).half()
    b = torch.randn(4, 3000, generator=gen).half()
    lib = backend._native
    da, db = a.to(device), b.to(device)
    out = torch.empty_like(da)
    stream = torch.cuda.current_stream(device).cuda_stream
    backend._check(lib.venturi_swiglu_run(da.data_ptr(), db.data_ptr(), out.data_ptr(), a.numel(), 0, stream))
    want = oracle.swiglu(a.numpy(), b.numpy()).astype(np.float64)
    got = out.cpu().numpy().astype(np.float64)
    finite = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), finite)
    assert (np.abs(got[finite] - want[finite]) <= ulp16(want[finite])).all()
    print(f"swiglu outputs differing from the oracle: {int((got[finite] != want[finite]).sum())} of {finite.sum()}")
    # The fused-layout variant reads gate and up from one [tokens][2*inter] buffer.
    gu = torch.cat((da, db), dim=1).contiguous()
    fused = torch.empty_like(da)
    backend._check(lib.venturi_silu_mul_run(gu.data_ptr(), fused.data_ptr(), 4, 3000, 0, stream))
    assert torch.equal(fused.view(torch.int16), out.view(torch.int16))
    added = torch.empty_like(da)
    backend._check(lib.venturi_add_run(da.data_ptr(), db.data_ptr(), added.data_ptr(), a.numel(), 0, stream))
    want_add = (a.float() + b.float()).half()
    assert torch.equal(added.cpu().view(torch.int16), want_add.view(torch.int16))


def test_graph_replays_equal_eager(backend, device):
    gen = torch.Generator(device=device).manual_seed(9)
    w1 = backend.quantize_q8(torch.randn(512, 256, generator=gen, device=device) * 0.05)
    w2 = backend.quantize_q8(torch.randn(256, 256, generator=gen, device=device) * 0.05)
    lib = backend._native
    for tokens in (1, 8):
        r1 = backend.upload_linear(w1, dtype=torch.float16, device=device).prepare(tokens=tokens)
        r2 = backend.upload_linear(w2, dtype=torch.float16, device=device).prepare(tokens=tokens)
        x = torch.randn(tokens, 256, generator=gen, device=device).half()
        gu = torch.empty(tokens, 512, dtype=torch.float16, device=device)
        act = torch.empty(tokens, 256, dtype=torch.float16, device=device)
        y = torch.empty(tokens, 256, dtype=torch.float16, device=device)

        def chain():
            r1.run(x, out=gu)
            backend._check(lib.venturi_silu_mul_run(gu.data_ptr(), act.data_ptr(), tokens, 256, 0,
                                                    torch.cuda.current_stream(device).cuda_stream))
            r2.run(act, out=y)

        chain()
        torch.cuda.synchronize(device)
        eager = bits(y)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            chain()
        for replay in range(4):
            y.fill_(7)
            r2.run(x, out=act)  # eager work between replays
            torch.cuda.synchronize(device)
            graph.replay()
            torch.cuda.synchronize(device)
            assert np.array_equal(bits(y), eager), (tokens, replay)
