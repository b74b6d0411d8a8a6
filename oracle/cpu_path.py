"""The reference's CPU execution path, restated for the bench's cpu_baseline leg.

TEST AND CPU-BASELINE-LEG INFRASTRUCTURE ONLY (never imported by venturi_amd).

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


class CpuA8Linear:
    """The A8 CPU leg, labelled "oracle": the reference has no CPU int8 GEMM.

    Restates quantize_reference (tests/q8_dp4a_reference.py:6-28) in FP32 --
    per 32-column group scale = max|r| / 127, codes = RNE(r * 127 / max|r|)
    clamped to +-127, residual passes -- and projection_reference (:31-34) as
    the FP32 matmul of the represented activations with the FP32 weight values
    (materialised before timing).
    """

    def __init__(self, codes, scales, in_features, passes=1):
        values = codes.to(torch.float32) * scales.to(torch.float32).repeat_interleave(32, -1)
        self.weight = values[:, :in_features].contiguous()
        self.passes = passes

    def represented(self, x):
        tokens, k = x.shape
        groups = (k + 31) // 32
        residual = torch.zeros(tokens, groups * 32, dtype=torch.float32)
        residual[:, :k] = x.float()
        residual = residual.reshape(tokens, groups, 32)
        total = torch.zeros_like(residual)
        for _ in range(self.passes):
            maximum = residual.abs().amax(-1)
            scale = maximum / 127
            inverse = torch.where(maximum > 0, 127 / maximum, torch.zeros_like(maximum))
            q = torch.round(residual * inverse[:, :, None]).clamp(-127, 127)
            step = q * scale[:, :, None]
            total += step
            residual = residual - step
        return total.reshape(tokens, -1)[:, :k]

    def run(self, x):
        return (self.represented(x) @ self.weight.T).to(torch.float16)


def cpu_model():
    """The host CPU's model name and logical core count, from /proc/cpuinfo."""
    name, count = None, 0
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    count += 1
                    name = name or line.split(":", 1)[1].strip()
    except OSError:
        pass
    return f"{name or 'unknown CPU'} ({count or os.cpu_count()} logical cores)"
