"""The reference's CPU execution path, restated for the bench's cpu_baseline leg.

TEST/BASELINE INFRASTRUCTURE ONLY (never imported by venturi_amd).

Restates TorchBackend.upload_linear + _TorchQuantizedLinear.run
(ops/blocks.py:891-931, 1020-1063): Q8/Q4 weights are materialised once as
FP32 values (code * scale is exact in FP32, so this equals the reference's
FP64 decode cast to FP32), and every call is ``(x.float() @ W.T).to(dtype)``
on the host cores through torch's CPU GEMM.
"""

import os
import time

import torch


class CpuQuantizedLinear:
    def __init__(self, codes, scales, in_features, group=32):
        values = codes.to(torch.float32) * scales.to(torch.float32).repeat_interleave(group, -1)
        self.weight = values[:, :in_features].contiguous()

    def run(self, x):
        return (x.float() @ self.weight.T).to(x.dtype)


def cpu_threads():
    torch.set_num_threads(os.cpu_count() or 1)
    return torch.get_num_threads()


def time_calls(calls, seconds, min_reps=2):
    """Runs the list of zero-argument callables repeatedly for about `seconds`.

    Returns (repetitions, elapsed seconds) over whole repetitions after one
    untimed warm-up repetition.
    """
    for call in calls:
        call()
    reps, start = 0, time.perf_counter()
    while True:
        for call in calls:
            call()
        reps += 1
        elapsed = time.perf_counter() - start
        if reps >= min_reps and elapsed >= seconds:
            return reps, elapsed


def q4_fp32_weight(codes, scales, in_features):
    """fp16(q * scale) values held in FP32: the reference's staged CPU expert weights
    (flash_next_hybrid_moe.py:23-43 reads fp16 decoded weights and calls .float())."""
    lo = (codes & 15).to(torch.int16)
    hi = (codes >> 4).to(torch.int16)
    q = torch.stack((lo, hi), -1).reshape(codes.shape[0], -1)
    q = torch.where(q < 8, q, q - 16).to(torch.float32)
    values = (q.reshape(codes.shape[0], -1, 64) * scales.float().unsqueeze(-1)).reshape(codes.shape[0], -1)
    return values[:, :in_features].half().float().contiguous()


class CpuRoutedExperts:
    """cpu_expert's staged-fp32 computation (flash_next_hybrid_moe.py:23-43) over
    the routed experts in ascending order, combined as routed_experts does
    (flash_next_moe.py:154-160). Weights are materialised before timing."""

    def __init__(self, gate_up, down):
        self.gate_up, self.down = gate_up, down  # lists of FP32 [2I, H] and [H, I]

    def run(self, x, ids, scores, experts):
        out = torch.zeros_like(x)
        for e in experts:
            positions, tokens = torch.where((ids == e).T)
            if tokens.numel() == 0:
                continue
            gate, up = torch.nn.functional.linear(x[tokens].float(), self.gate_up[e]).to(torch.float16).chunk(2, -1)
            h = torch.nn.functional.silu(gate) * up
            y = torch.nn.functional.linear(h.float(), self.down[e]).to(torch.float16)
            out.index_add_(0, tokens, y * scores[tokens, positions, None])
        return out
