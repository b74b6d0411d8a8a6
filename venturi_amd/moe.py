"""Routed-expert Q4 W4A16 MoE on gfx950.

Replaces the reference's per-expert host loop (flash_next_q4.py:204-224,
flash_next_moe.py:139-161) with three launches of libventuri_ops.so and no
host synchronisation: a grouped gate/up GEMM that routes its experts itself
(each workgroup ranks its expert's pairs) with SiLU*up fused in its epilogue,
a grouped down GEMM with the routing score fused in its epilogue, and a
per-token combine in ascending expert order. Above 8192 pairs routing is a
launch of its own before the GEMMs.

Semantics per token (the reference's operation graph, fp16 boundaries):
``h = fp16(fp16(silu(gate)) * up)``, ``v = fp16(fp16(h @ Wd^T) * score)``,
``out = fp16(... fp16(fp16(0 + v_e1) + v_e2) ...)`` over its experts in
ascending id order (position order for a repeated id). Expert weights are the
W4A16 contract values fp16(q * scale); GEMM association is fp32 on matrix
cores (the reference's F.linear is pinned by tolerance only).
"""

from dataclasses import dataclass

import torch

from .operands import admit, disjoint, stream_of
from .weights import Q4RowSplitWeight


@dataclass(frozen=True)
class MoEGeometry:
    """Routed-expert shape (reference flash_next_moe.py:20-32, without the shared expert)."""

    hidden_size: int
    num_experts: int
    top_k: int
    intermediate_size: int

    def __post_init__(self):
        for key in ("hidden_size", "num_experts", "top_k", "intermediate_size"):
            value = getattr(self, key)
            if type(value) is not int or value <= 0:
                raise ValueError(f"{key} must be a positive integer")
        if self.top_k > self.num_experts or self.top_k > 16 or self.num_experts > 1024:
            raise ValueError("MoE needs top_k <= min(num_experts, 16) and at most 1024 experts")
        if self.hidden_size % 8 or self.intermediate_size % 8:
            raise ValueError("hidden and intermediate sizes must be multiples of 8")


def _row_order(rows, half, swiglu, device):
    """Physical row of every tile slot (-1: padding), in tile order.

    Tiles hold 128 row slots; slot 16w + m belongs to wave w. Plain matrices
    use slot -> row tile*128 + slot. Gate/up tiles pair gate and up rows: wave
    w's slots m < 8 are gate rows tile*64 + 8w + m and slots m >= 8 the up rows
    ``half`` further on.
    """
    if not swiglu:
        tiles = (rows + 127) // 128
        order = torch.arange(tiles * 128, device=device)
        return torch.where(order < rows, order, -1)
    tiles = (half + 63) // 64
    slot = torch.arange(tiles * 128, device=device)
    tile, w, m = slot // 128, (slot % 128) // 16, slot % 16
    gate = tile * 64 + 8 * w + (m % 8)
    order = torch.where(m < 8, gate, gate + half)
    return torch.where(gate < half, order, -1)


def _tile(weights, rows, cols, swiglu, device):
    """Stacked tiled planes of the experts (layout read by the grouped GEMM kernels).

    Codes: [E][row tile][chunk][wave w][half h][lane l = 16q + m][16 bytes], the
    16-byte piece h of the 32 code bytes of slot row (w, m) for chunk columns
    [64q, 64q + 64), every nibble stored as q + 8. Scales: [E][row tile][chunk][w][l]
    fp16 of group q of the chunk. Chunks are 256 columns of the padded K; padding
    holds q = 0 and zero scales.
    """
    padded = (cols + 127) // 128 * 128
    chunks = (padded + 255) // 256
    order = _row_order(rows, rows // 2, swiglu, device)
    tiles = order.numel() // 128
    valid = order >= 0
    source = order.clamp_min(0)
    e_count = len(weights)
    codes = torch.zeros((e_count, tiles * 128, chunks * 128), dtype=torch.uint8, device=device)
    scales = torch.zeros((e_count, tiles * 128, chunks * 4), dtype=torch.float16, device=device)
    for e, w in enumerate(weights):
        if not isinstance(w, Q4RowSplitWeight) or (w.out_features, w.in_features) != (rows, cols):
            raise ValueError(f"expert {e} requires a Q4RowSplitWeight of shape [{rows}, {cols}]")
        w.validate()
        if not bool(torch.isfinite(w.scales).all()):
            raise ValueError("scales must be finite")
        codes[e, :, : padded // 2] = w.codes.to(device)[source] * valid[:, None].to(torch.uint8)
        scales[e, :, : padded // 64] = w.scales.to(device)[source] * valid[:, None].to(torch.float16)
    codes ^= 0x88  # pre-biased nibbles: q + 8 (padding becomes q = 0)
    codes = codes.view(e_count, tiles, 8, 16, chunks, 4, 2, 16).permute(0, 1, 4, 2, 6, 5, 3, 7).contiguous()
    scales = scales.view(e_count, tiles, 8, 16, chunks, 4).permute(0, 1, 4, 2, 5, 3).contiguous()
    return codes, scales


@dataclass(frozen=True)
class Q4ExpertBank:
    """All experts resident in the tiled layout of ``_tile`` (gate/up rows paired per wave)."""

    backend: object
    geometry: MoEGeometry
    gate_up_codes: torch.Tensor
    gate_up_scales: torch.Tensor
    down_codes: torch.Tensor
    down_scales: torch.Tensor

    @classmethod
    def upload(cls, backend, geometry, experts, *, device="cuda:0"):
        """``experts[e] = (gate_up, down)``: Q4RowSplitWeight [2I, H] (gate rows first) and [H, I]."""
        if len(experts) != geometry.num_experts:
            raise ValueError("one (gate_up, down) pair per expert is required")
        target = backend.resolve_device(device)
        g = geometry
        with torch.cuda.device(target):
            gu = _tile([e[0] for e in experts], 2 * g.intermediate_size, g.hidden_size, True, target)
            dn = _tile([e[1] for e in experts], g.hidden_size, g.intermediate_size, False, target)
            torch.cuda.current_stream(target).synchronize()
        return cls(backend, geometry, gu[0], gu[1], dn[0], dn[1])

    @property
    def device(self):
        return self.gate_up_codes.device

    @property
    def storage_tensors(self):
        return (self.gate_up_codes, self.gate_up_scales, self.down_codes, self.down_scales)

    @property
    def storage_nbytes(self):
        return sum(t.numel() * t.element_size() for t in self.storage_tensors)

    def prepare(self, *, tokens):
        g = self.geometry
        if type(tokens) is not int or tokens <= 0:
            raise ValueError("tokens must be a positive integer")
        lib = self.backend._native
        nbytes = lib.venturi_moe_q4_bytes(tokens, g.top_k, g.num_experts, g.hidden_size, g.intermediate_size)
        if nbytes == 0:
            raise ValueError(self.backend._native.error())
        self.backend.resolve_device(self.device)
        return RoutedExpertsPlan(self, tokens, int(nbytes))


@dataclass(frozen=True)
class RoutedExpertsPlan:
    """Fixed token count; ``run`` allocates nothing and does not synchronise.

    Workspace (256-byte aligned sections, in order): segment offsets int32
    [E+1], status int32 (count of ids outside [0, E)), pair slot int32 [T*K],
    slot token int32 [T*K], slot score fp16 [T*K], h fp16 [T*K][I], scaled
    expert outputs fp16 [T*K][H].
    """

    bank: Q4ExpertBank
    tokens: int
    workspace_bytes: int

    @property
    def route(self):
        return "venturi-moe-q4-mfma"

    def workspace_views(self, workspace):
        """Named views of a workspace after ``run`` (for inspection and tests)."""
        g, t = self.bank.geometry, self.tokens
        pairs = t * g.top_k

        def up(v):
            return (v + 255) // 256 * 256

        seg = 0
        status = up(4 * (g.num_experts + 1))
        pair_slot = status + 256
        slot_token = pair_slot + up(4 * pairs)
        slot_score = slot_token + up(4 * pairs)
        h = slot_score + up(2 * pairs)
        v = h + up(2 * pairs * g.intermediate_size)
        raw = workspace.view(torch.uint8)
        return {
            "seg": raw[seg : seg + 4 * (g.num_experts + 1)].view(torch.int32),
            "status": raw[status : status + 4].view(torch.int32),
            "pair_slot": raw[pair_slot : pair_slot + 4 * pairs].view(torch.int32).view(t, g.top_k),
            "slot_token": raw[slot_token : slot_token + 4 * pairs].view(torch.int32),
            "slot_score": raw[slot_score : slot_score + 2 * pairs].view(torch.float16),
            "h": raw[h : h + 2 * pairs * g.intermediate_size].view(torch.float16).view(pairs, g.intermediate_size),
            "v": raw[v : v + 2 * pairs * g.hidden_size].view(torch.float16).view(pairs, g.hidden_size),
        }

    def run(self, x, indices, scores, *, out, workspace):
        """Routes, projects and combines on the device; no host synchronisation.

        Expert ids outside [0, num_experts) are not checked on the host (that
        would synchronise): each pair with such an id is counted in the
        workspace's ``status`` word and skipped, and its token's output row is
        NaN, so bad routing cannot pass for a valid result.
        """
        b, g = self.bank, self.bank.geometry
        admit(x, (self.tokens, g.hidden_size), torch.float16, b.device, "x")
        admit(indices, (self.tokens, g.top_k), torch.int64, b.device, "indices")
        admit(scores, (self.tokens, g.top_k), torch.float16, b.device, "scores")
        admit(out, (self.tokens, g.hidden_size), torch.float16, b.device, "out")
        if not isinstance(workspace, torch.Tensor) or workspace.device != b.device or not workspace.is_contiguous():
            raise ValueError("workspace must be a contiguous tensor on the bank's device")
        if workspace.numel() * workspace.element_size() < self.workspace_bytes or workspace.data_ptr() % 256:
            raise ValueError(f"workspace requires {self.workspace_bytes} bytes at 256-byte alignment")
        disjoint(out, (x, indices, scores, workspace) + b.storage_tensors)
        disjoint(workspace, (x, indices, scores) + b.storage_tensors)
        with torch.cuda.device(b.device):
            b.backend._check(
                b.backend._native.venturi_moe_q4_run(
                    x.data_ptr(), indices.data_ptr(), scores.data_ptr(),
                    b.gate_up_codes.data_ptr(), b.gate_up_scales.data_ptr(),
                    b.down_codes.data_ptr(), b.down_scales.data_ptr(),
                    out.data_ptr(), workspace.data_ptr(), self.workspace_bytes,
                    self.tokens, g.top_k, g.num_experts, g.hidden_size, g.intermediate_size,
                    stream_of(b.device),
                )
            )
        return out


def routed_experts(hidden_states, indices, scores, bank):
    """The reference's ``routed_experts`` call (flash_next_moe.py:139-161) on a resident bank.

    Same argument checks, including the host range check of the expert ids
    (one synchronisation, as in the reference); allocates the output and the
    workspace. Graph-capturable code should hold a plan and call ``run``.
    """
    g = bank.geometry
    if hidden_states.ndim != 2 or hidden_states.shape[-1] != g.hidden_size or (
        indices.shape != (hidden_states.shape[0], g.top_k) or scores.shape != indices.shape
    ):
        raise ValueError("Routed expert input/selection geometry mismatch")
    if indices.dtype != torch.int64 or scores.dtype != hidden_states.dtype or any(
        t.device != hidden_states.device for t in (indices, scores)
    ):
        raise ValueError("Routed indices/scores dtype/device mismatch")
    if hidden_states.dtype != torch.float16:
        raise ValueError("Q4 W4A16 experts take FP16 hidden states")
    if indices.numel() and (indices.min().item() < 0 or indices.max().item() >= g.num_experts):
        raise ValueError("Router must select real expert ids, not padding or missing ids")
    plan = bank.prepare(tokens=hidden_states.shape[0])
    out = torch.empty_like(hidden_states)
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=hidden_states.device)
    return plan.run(hidden_states.contiguous(), indices.contiguous(), scores.contiguous(), out=out,
                    workspace=workspace)
