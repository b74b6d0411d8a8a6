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
