"""venturi_q8_tiled_run_noalloc: the tiled Q8 projection with its exchange slots
in the library's static device scratch, against venturi_q8_tiled_run with a
plan-owned workspace (same kernels, so the same bytes), on two calls in a row,
the second with a smaller input, plus the scratch-size and argument guards."""

import pytest
import torch

from helpers import random_q8
from venturi_amd import native
from venturi_amd.vocabulary import tile_q8

pytestmark = pytest.mark.gpu

SLOT_IDLE = 0x7F8000017F800001


@pytest.fixture(scope="module")
def lib():
    handle = native.load()
    return handle, handle.venturi_q8_tiled_run_noalloc


def _case(handle, fn, device, n, k, tokens, seed):
    print(f"case noalloc n={n} k={k} tokens={tokens}", flush=True)
    codes, scales = random_q8(n, k, seed)
    tc, ts = tile_q8(codes.to(device), scales.to(device))
    padded = codes.shape[1]
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(seed)).half().to(device)
    stream = torch.cuda.current_stream(device).cuda_stream
    size = handle.venturi_q8_tiled_workspace_bytes(tokens, n, 0)
    assert size > 0, "the case must split K to exercise the scratch"
    slots = torch.empty(size, dtype=torch.uint8, device=device)
    handle.check(handle.venturi_q8_tiled_workspace_init(slots.data_ptr(), size, stream))
    want = torch.empty(tokens, n, dtype=torch.float16, device=device)
    handle.check(handle.venturi_q8_tiled_run(x.data_ptr(), tc.data_ptr(), ts.data_ptr(), want.data_ptr(), tokens, n,
                                             k, padded, 0, slots.data_ptr(), size, stream))
    guard = torch.full((tokens * n + 2,), 47, dtype=torch.float16, device=device)
    got = guard[1:-1].view(tokens, n)
    handle.check(fn(x.data_ptr(), tc.data_ptr(), ts.data_ptr(), got.data_ptr(), tokens, n, k, padded, 0, stream))
    torch.cuda.synchronize(device)
    g = guard.cpu()
    assert g[0] == 47 and g[-1] == 47
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert bool((slots.view(torch.int64) == SLOT_IDLE).all())


def test_first_call_on_a_side_stream_then_another_stream(lib, device):
    # Collected first in this file, so in a fresh process this is the call that
    # fills the static slots: on a side stream. The next call runs on the
    # current stream, ordered after the side stream's work by an event only
    # (no host synchronisation), and must find idle slots.
    handle, fn = lib
    n, k, tokens = 5120, 6144, 4
    codes, scales = random_q8(n, k, 73)
    tc, ts = tile_q8(codes.to(device), scales.to(device))
    x = torch.randn(tokens, k, generator=torch.Generator().manual_seed(73)).half().to(device)
    main = torch.cuda.current_stream(device)
    side = torch.cuda.Stream(device)
    side.wait_stream(main)
    first = torch.empty(tokens, n, dtype=torch.float16, device=device)
    with torch.cuda.stream(side):
        handle.check(fn(x.data_ptr(), tc.data_ptr(), ts.data_ptr(), first.data_ptr(), tokens, n, k, k, 0,
                        side.cuda_stream))
    main.wait_stream(side)
    second = torch.empty_like(first)
    handle.check(fn(x.data_ptr(), tc.data_ptr(), ts.data_ptr(), second.data_ptr(), tokens, n, k, k, 0,
                    main.cuda_stream))
    size = handle.venturi_q8_tiled_workspace_bytes(tokens, n, 0)
    slots = torch.empty(size, dtype=torch.uint8, device=device)
    handle.check(handle.venturi_q8_tiled_workspace_init(slots.data_ptr(), size, main.cuda_stream))
    want = torch.empty_like(first)
    handle.check(handle.venturi_q8_tiled_run(x.data_ptr(), tc.data_ptr(), ts.data_ptr(), want.data_ptr(), tokens, n,
                                             k, k, 0, slots.data_ptr(), size, main.cuda_stream))
    torch.cuda.synchronize(device)
    assert torch.equal(first.view(torch.int16), want.view(torch.int16))
    assert torch.equal(second.view(torch.int16), want.view(torch.int16))


def test_noalloc_equals_workspace_entry_point(lib, device):
    handle, fn = lib
    _case(handle, fn, device, 5120, 6144, 4, 71)  # split K, 320 row blocks
    _case(handle, fn, device, 200, 1000, 13, 72)  # a second, smaller split call


def test_noalloc_unsplit_and_guards(lib, device):
    handle, fn = lib
    codes, scales = random_q8(7168, 128, 9)
    tc, ts = tile_q8(codes.to(device), scales.to(device))
    x = torch.randn(1, 128, generator=torch.Generator().manual_seed(3)).half().to(device)
    stream = torch.cuda.current_stream(device).cuda_stream
    assert handle.venturi_q8_tiled_workspace_bytes(1, 7168, 0) == 0
    want = torch.empty(1, 7168, dtype=torch.float16, device=device)
    handle.check(handle.venturi_q8_tiled_run(x.data_ptr(), tc.data_ptr(), ts.data_ptr(), want.data_ptr(), 1, 7168,
                                             128, 128, 0, None, 0, stream))
    got = torch.empty_like(want)
    handle.check(fn(x.data_ptr(), tc.data_ptr(), ts.data_ptr(), got.data_ptr(), 1, 7168, 128, 128, 0, stream))
    torch.cuda.synchronize(device)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert fn(x.data_ptr(), tc.data_ptr(), ts.data_ptr(), got.data_ptr(), 33, 7168, 128, 128, 0, stream) == -1
    assert "32 tokens" in handle.error()
    assert fn(None, tc.data_ptr(), ts.data_ptr(), got.data_ptr(), 1, 7168, 128, 128, 0, stream) == -1
    assert "null" in handle.error()
    torch.cuda.synchronize(device)
