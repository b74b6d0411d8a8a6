"""Shared test helpers: seeded inputs and fp16 bit comparisons."""

import numpy as np
import torch


def bits(tensor):
    """uint16 view of a CPU/GPU fp16 or bf16 tensor."""
    return tensor.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def random_q8(n, k, seed, scale=0.004, zero_first_group=True):
    """Random Q8 planes as the reference's tiling test draws them (test_q8_tiling.py:34-38)."""
    padded = (k + 127) // 128 * 128
    gen = torch.Generator().manual_seed(seed)
    codes = torch.randint(-127, 128, (n, padded), dtype=torch.int8, generator=gen)
    scales = (torch.rand(n, padded // 32, generator=gen) * scale).half()
    if zero_first_group and k > 32:
        scales[:, 0] = 0
    return codes, scales


def guarded_out(tokens, n, dtype, device, fill=47):
    """Output view with one sentinel element on each side."""
    guard = torch.full((tokens * n + 2,), fill, dtype=dtype, device=device)
    return guard, guard[1:-1].view(tokens, n)
